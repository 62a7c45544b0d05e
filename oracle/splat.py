"""Oracle: monomial theta maps, poly-splat weight, WSR blend (dense arm A and binned).

Test infrastructure only (see oracle/__init__.py).

Restates
  spike/forward.py:13-20    quad_form (raw Mahalanobis Q, no /k)
  spike/forward.py:23-39    theta_from_conic (theta_Q, theta_u over Phi=[px^2,py^2,px*py,px,py,1])
  spike/forward.py:42-44    phi
  spike/forward.py:47-58    quad_form_tilelocal (origin folded into the mean)
  spike/forward.py:61-66    poly_splat_wgeo = max(0, 1-Q/k)^2 (* keep)
  spike/arms.py:22-31       WSR blend, arm A: C = (sum w c + w_b c_b) / (sum w + w_b), w = o*w_geo
  spike/backward.py:11-20   wsr_polysplat_ref
  spike/render.py:14-49     dense render, arms A, B, SZ, RV (spike/arms.py:34-83), SH colour
                            (spike/render.py:23-25, direction differentiable)
  tools/m4_train_binned.py:130-143  theta_u_gathered (per-tile origin fold, [T,6,K])
  tools/m4_train_binned.py:189-212  _operands (returns the 5-tuple it is meant to)
  tools/bh_views.py:65-71   binned forward: w = relu(einsum(Phi, theta))^2,
                            C = (w@col + w_b c_b)/(w@oc + w_b), img[gidx] = C
"""
import torch

from . import binning, geometry


def quad_form(px, py, mu2d, conic):
    """Q[P,G] = a dx^2 + 2b dx dy + c dy^2 with d = p - mu (spike/forward.py:13-20)."""
    dx = px[:, None] - mu2d[None, :, 0]
    dy = py[:, None] - mu2d[None, :, 1]
    a, b, c = conic[None, :, 0], conic[None, :, 1], conic[None, :, 2]
    return a * dx * dx + 2 * b * dx * dy + c * dy * dy


def theta_from_conic(conic, mu2d, k):
    """theta_Q[G,6], theta_u[G,6] with Q = Phi.theta_Q and 1 - Q/k = Phi.theta_u
    (spike/forward.py:23-39)."""
    a, b, c = conic.unbind(-1)
    mx, my = mu2d.unbind(-1)
    tq = torch.stack([a, c, 2 * b, -2 * (a * mx + b * my), -2 * (b * mx + c * my),
                      a * mx * mx + 2 * b * mx * my + c * my * my], dim=-1)
    tu = tq * (-1.0 / k)
    tu = torch.cat([tu[..., :5], tu[..., 5:] + 1.0], dim=-1)
    return tq, tu


def phi(px, py):
    """Monomial basis [P,6] (spike/forward.py:42-44)."""
    return torch.stack([px * px, py * py, px * py, px, py, torch.ones_like(px)], dim=-1)


def quad_form_tilelocal(lx, ly, conic, mu2d, origin):
    """Q over a tile as Phi(local) @ theta_Q(mu - origin)^T (spike/forward.py:47-58)."""
    tq, _ = theta_from_conic(conic, mu2d - origin, 1.0)
    return phi(lx, ly) @ tq.T


def poly_splat_wgeo(Q, k, keep=None):
    """max(0, 1 - Q/k)^2, gated by keep (spike/forward.py:61-66)."""
    w = (1.0 - Q / k).clamp(min=0.0) ** 2
    if keep is not None:
        w = w * keep[None, :].to(w.dtype)
    return w


def wsr(W, color, w_b, c_b):
    """Weighted-sum rendering with a background term (spike/arms.py:22-26)."""
    return (W @ color + w_b * c_b[None, :]) / (W.sum(dim=1, keepdim=True) + w_b)


def wsr_polysplat_ref(theta_u, o, color, w_b, Phi, c_b, keep=None):
    """Plain forward of the hot op, autograd gives the backward (spike/backward.py:11-20)."""
    u = Phi @ theta_u.T
    w_geo = u.clamp(min=0.0) ** 2
    if keep is not None:
        w_geo = w_geo * keep[None, :]
    w = o[None, :] * w_geo
    return (w @ color + w_b * c_b[None, :]) / (w.sum(1, keepdim=True) + w_b)


def blend_sz(W0, z, softz_beta, color, w_b, c_b, eps=1e-6):
    """Soft-Z visibility prepass (spike/arms.py:50-68): z* = sum W0 z / (sum W0 + eps) per pixel,
    h = sigmoid(-beta (z - z*)), WSR of W0 h; z a constant of the gradient."""
    z = z.detach()
    den0 = W0.sum(dim=1, keepdim=True) + eps
    zstar = (W0 @ z[:, None]) / den0
    h = torch.sigmoid(-softz_beta * (z[None, :] - zstar))
    return wsr(W0 * h, color, w_b, c_b)


def blend_rv(W, color, c_b, eps=1e-6):
    """Revealage compositing (spike/arms.py:71-83): C_avg (1 - R) + c_b R,
    R = exp(sum log1p(-clamp(W, 0, 1 - 1e-4)))."""
    den = W.sum(dim=1, keepdim=True) + eps
    C_avg = (W @ color) / den
    a = W.clamp(0.0, 1.0 - 1e-4)
    R = torch.exp(torch.log1p(-a).sum(dim=1, keepdim=True))
    return C_avg * (1.0 - R) + c_b[None, :] * R


def render_dense(P, cam, k=4.0, blur_eps=0.3, near=0.2, w_b_raw=-3.0, c_b=None, depth_bt=None,
                 arm="A", softz_beta=None, rest=None, sh_degree=0):
    """Dense render of the [G,14] parameter set (spike/render.py:14-49): arm "A"; with
    depth_bt = (depth_beta, depth_tau) arm B (spike/arms.py:34-37), the depth differentiable as
    in spike's autograd; arm "SZ" (softz_beta) and "RV".  With sh_degree > 0 and rest [G,15,3]
    the colour is the SH colour in the direction means3d - camera centre, that direction
    differentiable too (spike/render.py:23-25, not detached there).  O(H*W*G) memory: small
    images only."""
    from . import sh
    pr = geometry.project_params(P, cam, blur_eps, near)
    dt = P.dtype
    px, py = geometry.pixel_grid(cam["H"], cam["W"], dtype=dt)
    Q = quad_form(px, py, pr["mu2d"], pr["conic"])
    w_geo = poly_splat_wgeo(Q, k, pr["keep"])
    if sh_degree > 0 and rest is not None:
        centre = sh.camera_center(cam["R_v"].to(dt), cam["t_v"].to(dt))
        coeffs = torch.cat([P[:, 10:13][:, None, :], rest], dim=1)
        color = sh.eval_sh_color(sh_degree, coeffs, P[:, 0:3] - centre[None, :])
    else:
        color = geometry.color_from_dc(P[:, 10:13])
    o = torch.sigmoid(P[:, 13])
    if depth_bt is not None:
        o = o * torch.sigmoid(depth_bt[0] * (depth_bt[1] - pr["depth"]))
    w_b = geometry.softplus(torch.as_tensor(w_b_raw, dtype=dt))
    c_b = torch.ones(3, dtype=dt) if c_b is None else c_b.to(dt)
    if arm == "SZ":
        img = blend_sz(o[None, :] * w_geo, pr["depth"], softz_beta, color, w_b, c_b)
    elif arm == "RV":
        img = blend_rv(o[None, :] * w_geo, color, c_b)
    else:
        img = wsr(o[None, :] * w_geo, color, w_b, c_b)
    return img.reshape(cam["H"], cam["W"], 3)


def theta_u_gathered(conic_t, mu_t, origins, k):
    """conic_t[T,K,3], mu_t[T,K,2], origins[T,2] -> theta_u[T,6,K] with the tile origin folded
    into the mean (tools/m4_train_binned.py:130-143)."""
    mx = mu_t[..., 0] - origins[:, None, 0]
    my = mu_t[..., 1] - origins[:, None, 1]
    a, b, c = conic_t.unbind(-1)
    ik = 1.0 / k
    Q0 = a * mx * mx + 2.0 * b * mx * my + c * my * my
    th = torch.stack([-a * ik, -c * ik, -2.0 * b * ik,
                      2.0 * (a * mx + b * my) * ik, 2.0 * (b * mx + c * my) * ik,
                      1.0 - Q0 * ik], dim=1)
    return th.contiguous()


def operands(P, cam, tmap, R=1, K=128, k=4.0, blur_eps=0.3, near=0.2, bins=None, span=2048,
             stable=False, rest=None, sh_degree=0, depth_bt=None):
    """Geometry, binning and per-tile gather (tools/m4_train_binned.py:189-212).

    Returns (theta_u[T,6,K], color_o_t[T,K,3], o_col_t[T,K,1], proj, (idx, valid));
    differentiable w.r.t. P except through the bin indices."""
    pr = geometry.project_params(P, cam, blur_eps, near, rest, sh_degree, depth_bt)
    if bins is None:
        bins = binning.assign_bins(pr["mu2d"], pr["keep"], tmap, R, K, span=span, stable=stable)
    idx, valid = bins
    vf = valid[..., None].to(P.dtype)
    theta = theta_u_gathered(pr["conic"][idx], pr["mu2d"][idx], tmap.origins.to(P.dtype), k)
    theta = theta * valid[:, None, :].to(P.dtype)
    col = pr["color_o"][idx] * vf
    oc = pr["o_col"][idx][..., None] * vf
    return theta, col, oc, pr, (idx, valid)


def splat_tiles(theta, col, oc, Phi, w_b, c_b):
    """[T,S*S,3] tile colours and [T,S*S] denominators (tools/bh_views.py:65-71)."""
    w = torch.relu(torch.einsum("pf,tfg->tpg", Phi, theta)) ** 2
    den = w @ oc + w_b
    C = (w @ col + w_b * c_b) / den
    return C, den[..., 0]


def tiles_to_image(C, tmap):
    """Scatter per-tile pixels to the row-major image, img[gidx] = C (bh_views.py:68-70)."""
    img = torch.zeros(tmap.H * tmap.W, C.shape[-1], dtype=C.dtype)
    img = img.index_copy(0, tmap.gidx, C.reshape(-1, C.shape[-1]))
    return img.reshape(tmap.H, tmap.W, -1)


def render_binned(P, cam, tmap, R=1, K=128, k=4.0, blur_eps=0.3, near=0.2, w_b_raw=-3.0,
                  c_b=None, bins=None, span=2048, stable=False, return_all=False, rest=None,
                  sh_degree=0, depth_bt=None):
    """Binned arm-A render (tools/bh_views.py:65-71 on _operands).  Differentiable w.r.t. P
    (and the SH rest coefficients `rest` [G,15,3] when sh_degree > 0)."""
    dt = P.dtype
    theta, col, oc, pr, bins = operands(P, cam, tmap, R, K, k, blur_eps, near, bins, span, stable,
                                        rest, sh_degree, depth_bt)
    w_b = geometry.softplus(torch.as_tensor(w_b_raw, dtype=dt))
    c_b = torch.ones(3, dtype=dt) if c_b is None else c_b.to(dt)
    C, den = splat_tiles(theta, col, oc, tmap.Phi.to(dt), w_b, c_b)
    img = tiles_to_image(C, tmap)
    if return_all:
        return img, dict(theta=theta, col=col, oc=oc, proj=pr, bins=bins,
                         den=tiles_to_image(den[..., None], tmap)[..., 0])
    return img
