"""WSR poly-splat over an explicit basis Phi: spike/backward.py:11-63.

`wsr_polysplat(theta_u, o, color, w_b, Phi, c_b, keep)` and `WSRPolySplatHot` run the HIP dense
kernels (tts_wsr_dense / tts_wsr_dense_bwd): C[P,3] = (w@color + w_b c_b) / (sum w + w_b) with
w = o * keep * max(Phi@theta_u^T, 0)^2, and the manual backward of spike/backward.py:41-58
(gradients for theta_u, o, color and w_b; Phi, c_b, keep are constants).

`wsr_polysplat_ref` is the reference's plain-tensor formula (autograd backward), kept under its
reference name for the same purpose it serves there: the formula the kernels are checked
against.
"""
import torch

from . import kernels

F32 = torch.float32


def wsr_polysplat_ref(theta_u, o, color, w_b, Phi, c_b, keep=None):
    """spike/backward.py:11-20."""
    u = Phi @ theta_u.t()
    w_geo = u.clamp(min=0.0) ** 2
    if keep is not None:
        w_geo = w_geo * keep[None, :]
    w = o[None, :] * w_geo
    num = w @ color + w_b * c_b[None, :]
    den = w.sum(1, keepdim=True) + w_b
    return num / den


def _bg(w_b, c_b, device):
    w = torch.as_tensor(w_b, dtype=F32, device=device).reshape(1)
    c = torch.as_tensor(c_b, dtype=F32, device=device).reshape(3)
    return torch.cat([w, c]).contiguous()


def _keep_u8(keep):
    if keep is None:
        return None
    return (keep != 0).to(torch.uint8).contiguous()


class WSRPolySplatHot(torch.autograd.Function):
    """Leaves: theta_u [G,6], o [G], color [G,3], w_b (scalar).  Phi [P,6], c_b [3], keep [G]
    are constants (spike/backward.py:23-25)."""

    @staticmethod
    def forward(ctx, theta_u, o, color, w_b, Phi, c_b, keep):
        dev = theta_u.device
        th = theta_u.detach().float().contiguous()
        oo = o.detach().float().contiguous()
        col = color.detach().float().contiguous()
        ph = Phi.detach().float().contiguous()
        bg = _bg(w_b.detach() if torch.is_tensor(w_b) else w_b, c_b.detach() if torch.is_tensor(c_b) else c_b, dev)
        k8 = _keep_u8(keep)
        C, den = kernels.wsr_dense(th, oo, col, k8, ph, bg)
        ctx.save_for_backward(th, oo, col, ph, bg, C, den)
        ctx.keep = k8
        ctx.w_b_shape = w_b.shape if torch.is_tensor(w_b) else None
        return C

    @staticmethod
    def backward(ctx, gC):
        th, oo, col, ph, bg, C, den = ctx.saved_tensors
        gth, go, gcol, gwb = kernels.wsr_dense_bwd(th, oo, col, ctx.keep, ph, bg, C, den,
                                                   gC.float().contiguous())
        gw = gwb.reshape(ctx.w_b_shape) if ctx.w_b_shape is not None else None
        return gth, go, gcol, gw, None, None, None


def wsr_polysplat(theta_u, o, color, w_b, Phi, c_b, keep=None):
    """Manual-backward entry point (spike/backward.py:61-63)."""
    return WSRPolySplatHot.apply(theta_u, o, color, w_b, Phi, c_b, keep)
