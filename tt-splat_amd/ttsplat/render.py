"""Dense render: spike/render.py:14-49 on the HIP dense kernels.

`render(model, cam, arm, k, blur_eps, near, sh_degree)` keeps the reference signature.  The
whole render is one differentiable op of the [G,14] parameter block (and w_b_raw):
geometry forward (tts_geom_fwd) -> every gaussian against every pixel (tts_render_dense);
backward: tts_render_dense_bwd -> tts_geom_bwd.  O(H*W*G) work, no O(H*W*G) memory.

Only arm "A" (depth-free WSR, the hot path's blend) and SH degree 0 are provided; the
reference's other arms (B, C0, C, SZ, RV, D) raise.  c_b is a constant (a registered buffer in
the reference model, spike/model.py:51), so its gradient is zero.
"""
import torch

from . import kernels
from .binned import background, params_of

F32 = torch.float32
ARMS = ("A",)


def _check_arm(arm, sh_degree=0):
    if arm != "A":
        raise NotImplementedError(f"arm {arm!r}: only the WSR arm 'A' is on the HIP path")
    if sh_degree:
        raise NotImplementedError("view-dependent colour (sh_degree > 0) is not on the HIP path")


class DenseRender(torch.autograd.Function):
    @staticmethod
    def forward(ctx, P, camera, bg, H, W, k, blur, near):
        Pc = P.detach().contiguous()
        proj, _ = kernels.geom_fwd(Pc, camera, near=near, blur=blur)
        img, den = kernels.render_dense(proj, H, W, k, bg.detach().contiguous())
        ctx.save_for_backward(Pc, camera, bg, proj, img, den)
        ctx.meta = (H, W, k, blur, near)
        return img

    @staticmethod
    def backward(ctx, gimg):
        Pc, camera, bg, proj, img, den = ctx.saved_tensors
        H, W, k, blur, near = ctx.meta
        grad9, gwb = kernels.render_dense_bwd(proj, H, W, k, bg.detach().contiguous(), img, den,
                                              gimg.float().contiguous())
        gP = kernels.geom_bwd(Pc, camera, grad9, near=near, blur=blur)
        gbg = torch.cat([gwb, torch.zeros(3, device=gwb.device, dtype=F32)])
        return gP, None, gbg, None, None, None, None, None


def render(model, cam, arm, k=4.0, blur_eps=0.3, near=0.2, sh_degree=0):
    """Image [H,W,3] of `model` seen by `cam`, differentiable w.r.t. the model's parameters."""
    _check_arm(arm, sh_degree)
    P = params_of(model)
    dev = P.device
    return DenseRender.apply(P, cam.device_block(dev), background(model, dev), cam.H, cam.W,
                             float(k), float(blur_eps), float(near))
