"""Pin the oracle against the reference's own known-answer tests and closed forms (CPU, fp64).

Each test restates a reference test (cited) or a mathematical fact chosen so that a plausible
mistake in the oracle (a dropped term, a sign, a factor of 2, a transposed operand) fails it.
"""
import math

import pytest
import torch

from oracle import adam as oadam
from oracle import binning as obin
from oracle import geometry as ogeo
from oracle import loss as oloss
from oracle import splat as osplat

DT = torch.float64


def _f(x):
    return torch.tensor(x, dtype=DT)


def _logit(p):
    return math.log(p / (1 - p))


# ---------------------------------------------------------------- theta map (spike/forward.py)
def test_theta_worked_example():
    """spike/tests/test_transform.py:15-31: conic (0.08, 0.02, 0.05), mu (3.5, 4.5), k = 4."""
    conic, mu, k = _f([[0.08, 0.02, 0.05]]), _f([[3.5, 4.5]]), 4.0
    tq, tu = osplat.theta_from_conic(conic, mu, k)
    assert torch.allclose(tq[0], _f([0.08, 0.05, 0.04, -0.74, -0.59, 2.6225]), atol=1e-12)
    px, py = _f([5.0]), _f([6.0])
    Q = osplat.quad_form(px, py, mu, conic)
    assert abs(Q.item() - 0.3825) < 1e-9
    Phi = osplat.phi(px, py)
    assert abs((Phi @ tq[0]).item() - 0.3825) < 1e-9
    assert abs((Phi @ tu[0]).item() - 0.904375) < 1e-9


def test_theta_random_spd_identity():
    """spike/tests/test_transform.py:34-49: Q = Phi.theta_Q and 1 - Q/k = Phi.theta_u."""
    g = torch.Generator().manual_seed(0)
    for _ in range(50):
        L = torch.randn(2, 2, generator=g, dtype=DT)
        M = L @ L.T + 0.1 * torch.eye(2, dtype=DT)
        conic = torch.stack([M[0, 0], M[0, 1], M[1, 1]]).reshape(1, 3)
        mu = torch.randn(1, 2, generator=g, dtype=DT) * 5
        px = torch.randn(8, generator=g, dtype=DT) * 6
        py = torch.randn(8, generator=g, dtype=DT) * 6
        Q = osplat.quad_form(px, py, mu, conic)[:, 0]
        tq, tu = osplat.theta_from_conic(conic, mu, 3.7)
        Phi = osplat.phi(px, py)
        assert torch.allclose(Phi @ tq[0], Q, atol=1e-9)
        assert torch.allclose(Phi @ tu[0], 1.0 - Q / 3.7, atol=1e-9)


def test_theta_centre_is_zero():
    conic, mu = _f([[0.13, -0.02, 0.09]]), _f([[7.0, 3.0]])
    assert abs(osplat.quad_form(mu[:, 0], mu[:, 1], mu, conic).item()) < 1e-12


def test_tile_local_equals_global():
    """spike/tests/test_tile_local.py:23-39: origin folded into the mean is exact."""
    g = torch.Generator().manual_seed(1)
    ly, lx = torch.meshgrid(torch.arange(16, dtype=DT), torch.arange(16, dtype=DT), indexing="ij")
    lx, ly = lx.reshape(-1), ly.reshape(-1)
    for _ in range(20):
        origin = torch.randint(0, 64, (2,)).to(DT) * 16.0
        L = torch.randn(5, 2, 2, generator=g, dtype=DT)
        M = L @ L.transpose(-1, -2) + 0.1 * torch.eye(2, dtype=DT)
        conic = torch.stack([M[:, 0, 0], M[:, 0, 1], M[:, 1, 1]], -1)
        mu = origin + torch.rand(5, 2, generator=g, dtype=DT) * 16.0
        Ql = osplat.quad_form_tilelocal(lx, ly, conic, mu, origin)
        Qg = osplat.quad_form(origin[0] + lx, origin[1] + ly, mu, conic)
        assert torch.allclose(Ql, Qg, atol=1e-9)


def test_tile_local_survives_bf16():
    """spike/tests/test_tile_local.py:49-75: global bf16 GEMM destroys Q, tile-local keeps it."""
    origin = _f([400.0, 400.0])
    conic = _f([[0.08, 0.02, 0.05]])
    mu = origin + _f([[7.3, 4.6]])
    ly, lx = torch.meshgrid(torch.arange(16, dtype=DT), torch.arange(16, dtype=DT), indexing="ij")
    lx, ly = lx.reshape(-1), ly.reshape(-1)
    px, py = origin[0] + lx, origin[1] + ly
    ref = osplat.quad_form(px, py, mu, conic)
    tl, _ = osplat.theta_from_conic(conic, mu - origin, 1.0)
    loc = (osplat.phi(lx, ly).bfloat16() @ tl.bfloat16().T).to(DT)
    tg, _ = osplat.theta_from_conic(conic, mu, 1.0)
    glo = (osplat.phi(px, py).bfloat16() @ tg.bfloat16().T).to(DT)
    e_loc, e_glo = (loc - ref).abs().max().item(), (glo - ref).abs().max().item()
    assert e_loc < 0.1 and e_glo > 1.0 and e_glo > 20 * e_loc


def test_theta_u_gathered_is_theta_from_conic_of_local_mean():
    """tools/m4_train_binned.py:130-143 == spike/forward.py theta_u of mu - origin, [T,6,K]."""
    g = torch.Generator().manual_seed(3)
    T, K = 4, 5
    L = torch.randn(T * K, 2, 2, generator=g, dtype=DT)
    M = L @ L.transpose(-1, -2) + 0.1 * torch.eye(2, dtype=DT)
    conic = torch.stack([M[:, 0, 0], M[:, 0, 1], M[:, 1, 1]], -1).reshape(T, K, 3)
    mu = torch.rand(T, K, 2, generator=g, dtype=DT) * 100
    origins = torch.randint(0, 6, (T, 2)).to(DT) * 16
    th = osplat.theta_u_gathered(conic, mu, origins, 4.0)
    _, tu = osplat.theta_from_conic(conic.reshape(-1, 3), (mu - origins[:, None, :]).reshape(-1, 2), 4.0)
    assert torch.allclose(th, tu.reshape(T, K, 6).transpose(1, 2), atol=1e-10)


# --------------------------------------------------------- poly splat + WSR (spike/arms.py)
def test_single_gaussian_centre_and_cutoff():
    """spike/tests/test_toy_1g.py:21-57."""
    k = 4.0
    mu, conic = _f([[8.0, 8.0]]), _f([[0.25, 0.0, 0.25]])
    color, o = _f([[0.7, 0.2, 0.1]]), torch.sigmoid(_f([_logit(0.8)]))
    w_b, c_b = _f(1e-6), _f([1.0, 1.0, 1.0])
    Q = osplat.quad_form(_f([8.0]), _f([8.0]), mu, conic)
    w = osplat.poly_splat_wgeo(Q, k)
    assert abs(w.item() - 1.0) < 1e-12
    C = osplat.wsr(o[None, :] * w, color, w_b, c_b)
    assert torch.allclose(C[0], color[0], atol=1e-3)
    Q2 = osplat.quad_form(_f([12.0]), _f([8.0]), mu, conic)
    assert abs(Q2.item() - 4.0) < 1e-9
    w2 = osplat.poly_splat_wgeo(Q2, k)
    assert w2.item() == 0.0
    assert torch.allclose(osplat.wsr(o[None, :] * w2, color, w_b, c_b)[0], c_b, atol=1e-3)
    Q3 = osplat.quad_form(_f([18.0]), _f([8.0]), mu, conic)
    assert osplat.poly_splat_wgeo(Q3, k).item() == 0.0


def test_wsr_averages_equal_weights():
    """spike/tests/test_toy_occlusion.py:42-46: depth-free WSR averages red and blue."""
    Q = osplat.quad_form(_f([0.0]), _f([0.0]), _f([[0.0, 0.0], [0.0, 0.0]]),
                         _f([[0.25, 0.0, 0.25], [0.25, 0.0, 0.25]]))
    w = osplat.poly_splat_wgeo(Q, 4.0)
    o = torch.sigmoid(_f([_logit(0.9), _logit(0.9)]))
    C = osplat.wsr(o[None, :] * w, _f([[1, 0, 0], [0, 0, 1]]), _f(1e-6), _f([1, 1, 1]))[0]
    assert torch.allclose(C, _f([0.5, 0.0, 0.5]), atol=1e-3)


def _bwd_inputs(seed, cull=True):
    g = torch.Generator().manual_seed(seed)
    P, G = 8, 5
    theta = torch.randn(G, 6, generator=g, dtype=DT, requires_grad=True)
    o = torch.rand(G, generator=g, dtype=DT, requires_grad=True)
    color = torch.rand(G, 3, generator=g, dtype=DT, requires_grad=True)
    w_b = torch.tensor(0.05, dtype=DT, requires_grad=True)
    px = torch.rand(P, generator=g, dtype=DT) * 4
    py = torch.rand(P, generator=g, dtype=DT) * 4
    keep = torch.ones(G, dtype=DT)
    if cull:
        keep[0] = 0.0
    return theta, o, color, w_b, osplat.phi(px, py), torch.ones(3, dtype=DT), keep


def test_splat_backward_gradcheck():
    """spike/tests/test_backward.py:30-33: the (autograd) backward of the hot op matches finite
    differences, keep mask included."""
    inp = _bwd_inputs(0)
    assert torch.autograd.gradcheck(osplat.wsr_polysplat_ref, inp, eps=1e-6, atol=1e-6, rtol=1e-4)


def test_splat_backward_quotient_term():
    """spike/tests/test_backward.py:51-56: the -C/den quotient term carries gradient: with
    colour == background everywhere, C is constant and every colour gradient must vanish."""
    theta, o, color, w_b, Phi, c_b, keep = _bwd_inputs(1, cull=False)
    col1 = torch.ones_like(color).requires_grad_(True)
    C = osplat.wsr_polysplat_ref(theta, o, col1, w_b, Phi, c_b)
    assert torch.allclose(C, torch.ones_like(C))
    C.sum().backward()
    assert float(theta.grad.abs().max()) < 1e-12 and float(o.grad.abs().max()) < 1e-12


def test_dense_equals_binned_when_splats_fit_their_stencil():
    """Binned render (tools/bh_views.py:65-71) == dense render (spike/render.py:14-49) when no
    tile overflows and every splat's support lies inside its 3x3 tile stencil.  Pins the tile
    origin fold, the Phi layout, the gidx scatter and the WSR."""
    from ttsplat import scenes
    P = scenes.make_params(300, seed=4, scale_range=(0.005, 0.012)).double()
    cam = ogeo.make_camera(64, 96, (0.0, 0.0, 3.0))
    tmap = obin.TileMap(64, 96, 16, dtype=DT)
    dense = osplat.render_dense(P, cam, k=4.0)
    pr = ogeo.project_params(P, cam)
    # support radius sqrt(k * lambda_max(Sigma2d)) must stay below one tile
    a, b, c = pr["conic"].unbind(-1)
    lam_min = 0.5 * ((a + c) - torch.sqrt((a - c) ** 2 + 4 * b * b))
    assert float(torch.sqrt(4.0 / lam_min[pr["keep"]]).max()) < 16.0
    binned = osplat.render_binned(P, cam, tmap, K=512, k=4.0)
    assert float((dense - binned).abs().max()) < 1e-9


def test_k_enters_as_one_over_k():
    """k = 9: w = (1 - Q/9)^2; at Q = 9 the weight vanishes, at Q = 2.25 it is 0.5625."""
    assert osplat.poly_splat_wgeo(_f([[9.0]]), 9.0).item() == 0.0
    assert abs(osplat.poly_splat_wgeo(_f([[2.25]]), 9.0).item() - 0.5625) < 1e-15


# -------------------------------------------------------------- geometry (spike/geometry.py)
def test_isotropic_projection():
    """spike/tests/test_geometry_analytic.py:12-37."""
    s, z, f, c, blur = 0.1, 4.0, 178.0, 64.0, 0.3
    cov = (s * s) * torch.eye(3, dtype=DT).unsqueeze(0)
    mu2d, conic, depth, keep = ogeo.project_ewa(_f([[0.0, 0.0, 0.0]]), cov, torch.eye(3, dtype=DT),
                                                _f([0.0, 0.0, z]), f, f, c, c, blur, 0.2)
    assert torch.allclose(mu2d[0], _f([c, c]), atol=1e-9)
    assert abs(depth.item() - z) < 1e-9 and bool(keep[0])
    pred = 1.0 / ((s * f / z) ** 2 + blur)
    assert abs(conic[0, 0].item() - pred) < 1e-6 and abs(conic[0, 2].item() - pred) < 1e-6
    assert abs(conic[0, 1].item()) < 1e-9


def test_depth_scaling_and_near_cull():
    """spike/tests/test_geometry_analytic.py:40-61."""
    def a_at(z):
        cov = 0.0025 * torch.eye(3, dtype=DT).unsqueeze(0)
        _, conic, _, _ = ogeo.project_ewa(_f([[0.0, 0.0, 0.0]]), cov, torch.eye(3, dtype=DT),
                                          _f([0.0, 0.0, z]), 178.0, 178.0, 64.0, 64.0, 0.0, 0.2)
        return conic[0, 0].item()
    assert abs(a_at(8.0) / a_at(4.0) - 4.0) < 1e-6
    cov = 0.01 * torch.eye(3, dtype=DT).unsqueeze(0)
    _, _, _, keep = ogeo.project_ewa(_f([[0.0, 0.0, 0.0]]), cov, torch.eye(3, dtype=DT),
                                     _f([0.0, 0.0, 0.05]), 100.0, 100.0, 64.0, 64.0, 0.3, 0.2)
    assert not bool(keep[0])


def test_rotation_and_covariance():
    """R(q) is orthonormal with det 1 and equals the axis-angle rotation; Sigma3 = R S^2 R^T."""
    th = 0.7
    q = _f([[math.cos(th / 2), 0.0, 0.0, math.sin(th / 2)]]) * 3.0   # unnormalised on purpose
    R = ogeo.quat_to_rotmat(q)[0]
    Rz = _f([[math.cos(th), -math.sin(th), 0], [math.sin(th), math.cos(th), 0], [0, 0, 1]])
    assert torch.allclose(R, Rz, atol=1e-12)
    cov = ogeo.cov3d(_f([[1.0, 2.0, 3.0]]), R[None])[0]
    assert torch.allclose(cov, Rz @ torch.diag(_f([1.0, 4.0, 9.0])) @ Rz.T, atol=1e-12)


def test_look_at_points_forward():
    R_v, t_v = ogeo.look_at_opencv((0.0, 0.0, 3.0))
    assert torch.allclose(R_v @ R_v.T, torch.eye(3), atol=1e-6)
    assert abs(float((R_v @ torch.zeros(3) + t_v)[2]) - 3.0) < 1e-6     # origin 3 ahead


def test_color_and_activations():
    P = torch.zeros(3, 14, dtype=DT)
    P[:, 3] = 1.0
    P[:, 10:13] = _f([[1.0, -3.0, 0.0], [0.0, 0.0, 0.0], [-10.0, 2.0, 0.5]])
    P[:, 13] = _f([0.0, 2.0, -1.0])
    P[:, 2] = _f([0.0, 0.0, 10.0])          # the third is behind the camera
    cam = ogeo.make_camera(32, 32, (0.0, 0.0, 3.0))
    pr = ogeo.project_params(P, cam)
    col = ogeo.color_from_dc(P[:, 10:13])
    assert torch.allclose(col[1], _f([0.5, 0.5, 0.5]))
    assert float(col.min()) >= 0.0                          # min-only clamp
    assert float(pr["o_col"][2]) == 0.0 and bool(pr["keep"][0]) and not bool(pr["keep"][2])
    assert torch.allclose(pr["o_col"][:2], torch.sigmoid(P[:2, 13]))


# ----------------------------------------------------------------------- loss (metrics.py)
def test_loss_identity():
    y = torch.rand(32, 40, 3, generator=torch.Generator().manual_seed(0), dtype=DT)
    L, g = oloss.loss_and_grad(y, y)
    assert abs(float(L)) < 1e-12 and float(g.abs().max()) < 1e-12


def test_ssim_constant_images_closed_form():
    a, b = 0.3, 0.7
    x = torch.full((3, 20, 24), a, dtype=DT)
    y = torch.full((3, 20, 24), b, dtype=DT)
    S = oloss.ssim_map(x, y, oloss.gauss_1d())
    pred = (2 * a * b + oloss.C1) / (a * a + b * b + oloss.C1)
    assert torch.allclose(S, torch.full_like(S, pred), atol=1e-12)


def test_ssim_filter_matches_banded_gemm():
    """The separable valid convolution == Mh x Mw^T (tools/loss_manual.py:32-47)."""
    x = torch.rand(3, 30, 26, generator=torch.Generator().manual_seed(1), dtype=DT)
    g = oloss.gauss_1d()
    Mh, Mw = oloss.band_matrix(30, g), oloss.band_matrix(26, g)
    assert torch.allclose(oloss.gaussian_filter(x, g), Mh @ x @ Mw.T, atol=1e-12)
    assert abs(float(g.sum()) - 1.0) < 1e-15 and torch.allclose(g, g.flip(0))


def test_loss_gradcheck_and_clamp():
    g = torch.Generator().manual_seed(2)
    x = (torch.rand(14, 15, 3, generator=g, dtype=DT) * 1.4 - 0.2).requires_grad_(True)
    y = torch.rand(14, 15, 3, generator=g, dtype=DT)
    assert torch.autograd.gradcheck(lambda t: oloss.loss_fn(t, y), (x,), eps=1e-7, atol=1e-6)
    # outside [0,1] only the L1 term acts: its gradient is 0.8*sign/N
    L, gr = oloss.loss_and_grad(x.detach(), y)
    out = (x.detach() < 0) | (x.detach() > 1)
    n = x.numel()
    assert torch.allclose(gr[out], 0.8 * torch.sign(x.detach() - y)[out] / n, atol=1e-15)


def test_loss_window_size_rule():
    """spike/metrics.py:14-18: min(11, H, W), made odd, at least 3."""
    assert oloss.window_size(128, 128) == 11
    assert oloss.window_size(8, 100) == 7
    assert oloss.window_size(2, 2) == 3


# ------------------------------------------------------------------------------------ adam
def adam_case(seed, n=50, steps=5, dtype=DT):
    """p0, per-step gradients whose magnitudes span 1e-9 .. 1 (so eps = 1e-8 decides the
    update of the smallest ones), and the per-column learning rates."""
    g = torch.Generator().manual_seed(seed)
    p0 = torch.randn(n, 14, generator=g, dtype=dtype)
    scale = 10.0 ** (-9.0 * torch.rand(n, 14, generator=g, dtype=dtype))
    grads = [torch.randn(n, 14, generator=g, dtype=dtype) * scale for _ in range(steps)]
    lr = torch.full((14,), 1e-3, dtype=dtype)
    lr[:3] = 1.6e-4
    return p0, grads, lr


def test_adam_matches_torch_optim():
    p0, grads, lr = adam_case(5)
    p, m, v = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    for t, gr in enumerate(grads, 1):
        oadam.adam_step(p, m, v, gr, lr, t)
    ref = oadam.torch_adam_reference(p0, grads, lr)
    # the updates, not the parameters: |update| ~ lr << |p|
    assert torch.allclose(p - p0, ref - p0, rtol=1e-9, atol=0.0)
    # the inputs are sensitive to eps: ten times eps moves the small-gradient updates
    pe, me, ve = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    for t, gr in enumerate(grads, 1):
        oadam.adam_step(pe, me, ve, gr, lr, t, eps=1e-7)
    assert not torch.allclose(pe - p0, ref - p0, rtol=1e-3, atol=0.0)
    # with unit-scale gradients the first step moves every entry by ~lr (|m/sqrt(v)| = 1)
    g1 = torch.randn(50, 14, generator=torch.Generator().manual_seed(6), dtype=DT)
    p1, m1, v1 = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    oadam.adam_step(p1, m1, v1, g1, lr, 1)
    assert torch.allclose((p0 - p1).abs(), lr.expand_as(p0), rtol=1e-4)


# --------------------------------------------------------------------------------- pipeline
def test_training_step_reduces_loss():
    from oracle import pipeline as opipe
    from ttsplat import scenes
    cfg = scenes.CONFIGS["c1_ref"]
    P = scenes.make_params(300, seed=0)
    cam = ogeo.make_camera(64, 64, (0.0, 0.0, 3.0))
    tmap = obin.TileMap(64, 64, 16)
    tgt = osplat.render_binned(scenes.make_params(300, seed=1), cam, tmap, K=cfg.K).detach()
    m, v = torch.zeros_like(P), torch.zeros_like(P)
    lr = torch.full((14,), 1e-2)
    losses = [float(opipe.train_step(P, m, v, t, cam, tmap, tgt, lr, K=128)[1]) for t in range(1, 31)]
    assert losses[-1] < 0.9 * losses[0]


def test_soft_z_and_revealage_arms_limits():
    """spike/arms.py:50-83 restated: soft-Z with beta = 0 halves every weight (h = 1/2), which the
    WSR ratio ignores except against w_b; a fully transparent set shows c_b through revealage; an
    opaque front gaussian hides one behind it in SZ for large beta."""
    from oracle import splat as osp
    D = torch.float64
    W0 = torch.rand(5, 4, dtype=D) * 0.5
    color = torch.rand(4, 3, dtype=D)
    z = torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=D)
    w_b, c_b = torch.tensor(0.05, dtype=D), torch.ones(3, dtype=D)
    a = osp.blend_sz(W0, z, torch.tensor(0.0, dtype=D), color, w_b, c_b)
    assert torch.allclose(a, osp.wsr(0.5 * W0, color, w_b, c_b))
    assert torch.allclose(osp.blend_rv(torch.zeros(3, 4, dtype=D), color, c_b),
                          torch.ones(3, 3, dtype=D))
    W = torch.tensor([[10.0, 10.0]], dtype=D)                # two equal gaussians at z = 1 and 5
    col = torch.tensor([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0]], dtype=D)
    out = osp.blend_sz(W, torch.tensor([1.0, 5.0], dtype=D), torch.tensor(50.0, dtype=D), col,
                       torch.tensor(1e-6, dtype=D), c_b)
    # z* = 3: the front one passes (h ~ 1), the back one is gated (h ~ 0)
    assert float(out[0, 0]) > 0.99 and float(out[0, 2]) < 0.01
    # revealage: an opaque pixel (W >= 1) shows the average colour, no background
    rv = osp.blend_rv(torch.tensor([[2.0, 0.0]], dtype=D), col, c_b)
    assert torch.allclose(rv, torch.tensor([[1.0, 0.0, 0.0]], dtype=D), atol=1e-3)
