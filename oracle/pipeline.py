"""Oracle: one binned training step, composed from the other oracle modules.

Test infrastructure only (see oracle/__init__.py).

Follows the op order of the device-resident step, tools/resident_traced.py:667-744:
geometry fwd -> binning -> gather/theta -> splat fwd -> loss gradient -> splat bwd ->
theta bwd -> slot->gaussian reduce -> geometry bwd -> Adam, with the gradient of everything
after binning taken by autograd of the restated forward (the reference's manual chain,
tools/operands_manual.py:83-111, equals that autograd to 1e-3, :114-144).
w_b is held fixed, as in that trainer (tools/resident_traced.py:220).
"""
import torch

from . import adam, loss, splat


def render_and_grad(P, cam, tmap, target, R=1, K=128, k=4.0, blur_eps=0.3, near=0.2,
                    w_b_raw=-3.0, lambda_ssim=0.2, bins=None, span=2048, stable=False, rest=None,
                    sh_degree=0, depth_bt=None, c_b=None):
    """Forward + loss + autograd backward.  Returns (img, loss, dL/dP[G,14], extras); with
    SH rest coefficients (rest [G,15,3], sh_degree > 0) extras["grest"] is dL/drest, with a
    depth weight (depth_bt = (beta, tau)) extras["gdepth"] is dL/d(beta, tau).  c_b: the
    background colour (white if None; a random-background step's draw,
    tools/resident_traced.py:671-674)."""
    Pg = P.detach().clone().requires_grad_(True)
    rg = None if rest is None else rest.detach().clone().requires_grad_(True)
    bt = (None if depth_bt is None
          else torch.as_tensor(depth_bt, dtype=P.dtype).detach().clone().requires_grad_(True))
    img, ex = splat.render_binned(Pg, cam, tmap, R, K, k, blur_eps, near, w_b_raw, c_b, bins,
                                  span, stable, return_all=True, rest=rg, sh_degree=sh_degree,
                                  depth_bt=bt)
    L = loss.loss_fn(img, target, lambda_ssim)
    L.backward()
    if rg is not None:
        ex["grest"] = rg.grad.detach() if rg.grad is not None else torch.zeros_like(rg)
    if bt is not None:
        ex["gdepth"] = bt.grad.detach()
    return img.detach(), L.detach(), Pg.grad.detach(), ex


def train_step(P, m, v, t, cam, tmap, target, lr, **kw):
    """In-place Adam step on P (with moments m, v) at step number t; returns (img, loss, grad)."""
    img, L, g, _ = render_and_grad(P, cam, tmap, target, **kw)
    with torch.no_grad():
        adam.adam_step(P, m, v, g, lr, t)
    return img, L, g
