"""Dense render: spike/render.py:14-49 on the HIP dense kernels.

`render(model, cam, arm, k, blur_eps, near, sh_degree)` keeps the reference signature.  The
whole render is one differentiable op of the [G,14] parameter block (and w_b_raw):
geometry forward (tts_geom_fwd) -> every gaussian against every pixel (tts_render_dense);
backward: tts_render_dense_bwd -> tts_geom_bwd.  O(H*W*G) work, no O(H*W*G) memory.

With sh_degree > 0 and a model carrying color_rest [G,15,3] (spike/model.py:45) the colour is
the view-dependent SH colour in the direction means3d - camera centre (spike/render.py:23-25),
and, as in spike's autograd, its gradient also reaches the means through that direction.

Arms:
  "A"   depth-free WSR, the hot path's blend (spike/arms.py:22-31);
  "B"   A with the per-gaussian depth weight rho = sigmoid(depth_beta (depth_tau - z_cam)) on the
        opacity (:34-37); gradients to depth_beta, depth_tau and, as spike's autograd gives them,
        to the means through z_cam;
  "SZ"  soft-Z visibility prepass (:50-68), trainable model.softz_beta, z_cam a constant of the
        gradient as in the reference;
  "RV"  revealage compositing (:71-83).
The reference's arms C0, C (view-dependent opacity) and D (sorted alpha) raise.  c_b is a
constant (a registered buffer in the reference model, spike/model.py:51): its gradient is zero.
"""
import torch

from . import kernels
from .binned import background, params_of

F32 = torch.float32
ARMS = ("A", "B", "SZ", "RV")


def _check_arm(arm, sh_degree=0):
    if arm not in ARMS:
        raise NotImplementedError(f"arm {arm!r}: only the arms {ARMS} are on the HIP path")
    if not 0 <= int(sh_degree) <= 3:
        raise ValueError(f"sh_degree must be in [0, 3], got {sh_degree}")


class DenseRender(torch.autograd.Function):
    """bt: (depth_beta, depth_tau) [2] for arm B, or None; szb: softz_beta [1] for arm SZ, or
    None; rest: the SH rest coefficients in the library layout [15,3,G] (sh_degree > 0), or
    None; blend: "A", "SZ" or "RV" (arm B blends as A)."""

    @staticmethod
    def forward(ctx, P, camera, bg, bt, szb, rest, sh_degree, blend, H, W, k, blur, near):
        Pc = P.detach().contiguous()
        btc = None if bt is None else bt.detach().float().contiguous()
        szc = None if szb is None else szb.detach().float().reshape(1).contiguous()
        rc = None if rest is None else rest.detach().float().contiguous()
        deg = int(sh_degree) if rc is not None else 0
        proj, _ = kernels.geom_fwd(Pc, camera, near=near, blur=blur, depth_bt=btc, sh_rest=rc,
                                   sh_degree=deg)
        bgc = bg.detach().contiguous()
        if blend == "A":
            img, den = kernels.render_dense(proj, H, W, k, bgc)
            aux = None
        else:
            img, den, aux = kernels.render_dense_arm(proj, H, W, k, bgc, blend, szc)
        ctx.save_for_backward(Pc, camera, bg, proj, img, den, btc, szc, aux, rc)
        ctx.meta = (H, W, k, blur, near, blend, deg)
        return img

    @staticmethod
    def backward(ctx, gimg):
        Pc, camera, bg, proj, img, den, btc, szc, aux, rc = ctx.saved_tensors
        H, W, k, blur, near, blend, deg = ctx.meta
        bgc = bg.detach().contiguous()
        gi = gimg.float().contiguous()
        gszb = None
        if blend == "A":
            grad9, gwb = kernels.render_dense_bwd(proj, H, W, k, bgc, img, den, gi)
        else:
            g, gwb = kernels.render_dense_arm_bwd(proj, H, W, k, bgc, blend, img, den, aux, gi,
                                                  szc)
            grad9 = g[:, :9].contiguous()
            if blend == "SZ":
                gszb = g[:, 9].sum().reshape(1)
        gbt = grest = None
        if btc is None and deg == 0:
            gP = kernels.geom_bwd(Pc, camera, grad9, near=near, blur=blur)
        else:
            gP, grest, gdw = kernels.geom_bwd(Pc, camera, grad9, near=near, blur=blur,
                                              depth_bt=btc, depth_zgrad=btc is not None,
                                              sh_rest=rc, sh_degree=deg, sh_dirgrad=True)
            if gdw is not None:
                gbt = gdw.sum(0)
        gbg = torch.cat([gwb, torch.zeros(3, device=gwb.device, dtype=F32)])
        return gP, None, gbg, gbt, gszb, grest, None, None, None, None, None, None, None


def render(model, cam, arm, k=4.0, blur_eps=0.3, near=0.2, sh_degree=0):
    """Image [H,W,3] of `model` seen by `cam`, differentiable w.r.t. the model's parameters."""
    _check_arm(arm, sh_degree)
    P = params_of(model)
    dev = P.device
    bt = szb = None
    if arm == "B":
        bt = torch.stack([torch.as_tensor(model.depth_beta, dtype=F32, device=dev).reshape(()),
                          torch.as_tensor(model.depth_tau, dtype=F32, device=dev).reshape(())])
    if arm == "SZ":
        szb = torch.as_tensor(model.softz_beta, dtype=F32, device=dev).reshape(1)
    blend = "A" if arm == "B" else arm
    rest = None
    color_rest = getattr(model, "color_rest", None)
    if int(sh_degree) > 0 and color_rest is not None:        # spike/render.py:23-25
        rest = kernels.sh_rest_layout(color_rest.to(dev, F32))
    return DenseRender.apply(P, cam.device_block(dev), background(model, dev), bt, szb, rest,
                             int(sh_degree), blend, cam.H, cam.W, float(k), float(blur_eps),
                             float(near))
