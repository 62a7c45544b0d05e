"""Per-pixel forward primitives under their reference names (spike/forward.py:13-71).

These are the small tensor formulas the reference composes its dense renderer from; they are
kept so code written against spike.forward runs unchanged.  The hot path does not call them:
the fused kernels (render, binned render, wsr_polysplat) evaluate the same quantities in
registers.  Inputs must be GPU tensors, like every other entry point of this package.
"""
import torch

C0 = 0.28209479177387814  # SH degree-0 constant (spike/sh.py:9)


def _gpu(*ts):
    for t in ts:
        if torch.is_tensor(t) and not t.is_cuda:
            raise ValueError("ttsplat works on GPU tensors; got a tensor on " + str(t.device))


def quad_form(px, py, mu2d, conic_abc):
    """Q[P,G] = a dx^2 + 2b dx dy + c dy^2, dx = px - mu_x (no /k)."""
    _gpu(px, py, mu2d, conic_abc)
    dx = px[:, None] - mu2d[None, :, 0]
    dy = py[:, None] - mu2d[None, :, 1]
    a, b, c = (conic_abc[:, i][None, :] for i in range(3))
    return a * dx * dx + 2 * b * dx * dy + c * dy * dy


def theta_from_conic(conic_abc, mu2d, k):
    """(theta_Q, theta_u) [G,6] over Phi = [px^2, py^2, px*py, px, py, 1]; u = 1 - Q/k."""
    _gpu(conic_abc, mu2d)
    a, b, c = conic_abc.unbind(-1)
    mx, my = mu2d.unbind(-1)
    theta_Q = torch.stack([a, c, 2 * b, -2 * (a * mx + b * my), -2 * (b * mx + c * my),
                           a * mx * mx + 2 * b * mx * my + c * my * my], dim=-1)
    theta_u = theta_Q * (-1.0 / k)
    theta_u[..., 5] += 1.0
    return theta_Q, theta_u


def phi(px, py):
    """Monomial basis [P,6]."""
    _gpu(px, py)
    return torch.stack([px * px, py * py, px * py, px, py, torch.ones_like(px)], dim=-1)


def quad_form_tilelocal(lx, ly, conic_abc, mu2d, tile_origin):
    """Q over one tile as Phi(lx, ly) @ theta_Q^T with the tile origin folded into the mean."""
    theta_Q, _ = theta_from_conic(conic_abc, mu2d - tile_origin, k=1.0)
    return phi(lx, ly) @ theta_Q.transpose(-1, -2)


def poly_splat_wgeo(Q, k, keep=None):
    """w_geo = max(0, 1 - Q/k)^2, gated by keep [G]."""
    _gpu(Q)
    w = (1.0 - Q / k).clamp(min=0.0) ** 2
    return w if keep is None else w * keep[None, :].to(w.dtype)


def color_from_dc(color_dc):
    """clamp(0.5 + C0*dc, min=0)."""
    _gpu(color_dc)
    return (0.5 + C0 * color_dc).clamp(min=0.0)
