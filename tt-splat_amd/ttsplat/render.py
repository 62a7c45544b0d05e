"""Dense render: spike/render.py:14-49 on the HIP dense kernels.

`render(model, cam, arm, k, blur_eps, near, sh_degree)` keeps the reference signature.  The
whole render is one differentiable op of the [G,14] parameter block (and w_b_raw):
geometry forward (tts_geom_fwd) -> every gaussian against every pixel (tts_render_dense);
backward: tts_render_dense_bwd -> tts_geom_bwd.  O(H*W*G) work, no O(H*W*G) memory.

Arms "A" (depth-free WSR, the hot path's blend) and "B" (A with the per-gaussian depth weight
rho = sigmoid(depth_beta (depth_tau - z_cam)) on the opacity, spike/arms.py:34-37; gradients to
depth_beta, depth_tau and, as spike's autograd gives them, to the means through z_cam) with SH
degree 0 are provided; the reference's other arms (C0, C, SZ, RV, D) raise.  c_b is a constant
(a registered buffer in the reference model, spike/model.py:51), so its gradient is zero.
"""
import torch

from . import kernels
from .binned import background, params_of

F32 = torch.float32
ARMS = ("A", "B")


def _check_arm(arm, sh_degree=0):
    if arm not in ARMS:
        raise NotImplementedError(f"arm {arm!r}: only the WSR arms 'A' and 'B' are on the HIP path")
    if sh_degree:
        raise NotImplementedError("view-dependent colour (sh_degree > 0) is not on the HIP path")


class DenseRender(torch.autograd.Function):
    """bt: (depth_beta, depth_tau) [2] for arm B, or None."""

    @staticmethod
    def forward(ctx, P, camera, bg, bt, H, W, k, blur, near):
        Pc = P.detach().contiguous()
        btc = None if bt is None else bt.detach().float().contiguous()
        proj, _ = kernels.geom_fwd(Pc, camera, near=near, blur=blur, depth_bt=btc)
        img, den = kernels.render_dense(proj, H, W, k, bg.detach().contiguous())
        ctx.save_for_backward(Pc, camera, bg, proj, img, den, btc)
        ctx.meta = (H, W, k, blur, near)
        return img

    @staticmethod
    def backward(ctx, gimg):
        Pc, camera, bg, proj, img, den, btc = ctx.saved_tensors
        H, W, k, blur, near = ctx.meta
        grad9, gwb = kernels.render_dense_bwd(proj, H, W, k, bg.detach().contiguous(), img, den,
                                              gimg.float().contiguous())
        gbt = None
        if btc is None:
            gP = kernels.geom_bwd(Pc, camera, grad9, near=near, blur=blur)
        else:
            gP, _, gdw = kernels.geom_bwd(Pc, camera, grad9, near=near, blur=blur, depth_bt=btc,
                                          depth_zgrad=True)
            gbt = gdw.sum(0)
        gbg = torch.cat([gwb, torch.zeros(3, device=gwb.device, dtype=F32)])
        return gP, None, gbg, gbt, None, None, None, None, None


def render(model, cam, arm, k=4.0, blur_eps=0.3, near=0.2, sh_degree=0):
    """Image [H,W,3] of `model` seen by `cam`, differentiable w.r.t. the model's parameters."""
    _check_arm(arm, sh_degree)
    P = params_of(model)
    dev = P.device
    bt = None
    if arm == "B":
        bt = torch.stack([torch.as_tensor(model.depth_beta, dtype=F32, device=dev).reshape(()),
                          torch.as_tensor(model.depth_tau, dtype=F32, device=dev).reshape(())])
    return DenseRender.apply(P, cam.device_block(dev), background(model, dev), bt, cam.H, cam.W,
                             float(k), float(blur_eps), float(near))
