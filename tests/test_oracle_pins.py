"""Pins for the oracle parts that the reference's own tests leave open (CPU, fp64).

Each check is fixed by the mathematics, computed here by a route independent of the oracle's
code (direct 2-D window sums, autograd of the pinhole map, scipy rotations, closed forms), and
chosen so that a plausible mistake fails it:
  SSIM (spike/metrics.py:15-28, pytorch_msssim's published algorithm):
      C2 = 0.03 instead of 0.03^2, a window sigma other than 1.5, a dropped or mis-signed
      structure term, and a mean taken over the wrong count all fail;
  EWA projection (spike/geometry.py:28-57): any sign or index slip in the off-axis Jacobian
      entries J02 = -fx x/z^2, J12 = -fy y/z^2 fails;
  depth weight (spike/arms.py:34-37): a flipped sign of beta (tau - z), and gradients other than
      the closed forms of tools/m8_depthweight_oracle.py:7-12, fail.
  camera and cull (spike/camera.py:51-63, spike/geometry.py:39-40, spike/synthetic.py:21): a
      frame turned 180 degrees, a non-strict near cull, another z clamp for culled gaussians, a
      vertical field of view and an ungated dense weight fail;
  operands and step: theta left unmasked in empty slots, a depth weight whose gradient reaches
      z, and an Adam step number off by one fail;
  loss: SSIM on the unclamped target fails.
"""
import math

import pytest
import torch

from oracle import adam as oadam
from oracle import geometry as ogeo
from oracle import loss as oloss
from oracle import splat as osplat

DT = torch.float64


def _f(x):
    return torch.tensor(x, dtype=DT)

# The 11-tap gaussian window of sigma 1.5, normalised (taps 0..5; the window is symmetric):
# exp(-c^2 / 4.5) / sum over c = -5..5.
WINDOW_11_15 = (0.00102838008447911, 0.007598758135239185, 0.03600077212843083,
                0.10936068950970002, 0.2130055377112537, 0.26601172486179436)
C1_LIT = 1e-4     # (0.01 * data_range)^2, data_range 1
C2_LIT = 9e-4     # (0.03 * data_range)^2


def _window_2d():
    taps = [math.exp(-(c * c) / 4.5) for c in range(-5, 6)]
    s = sum(taps)
    w = torch.tensor([t / s for t in taps], dtype=DT)
    return torch.outer(w, w)


def _window_moments(x, y):
    """Window-weighted mu_x, mu_y, E[x^2], E[y^2], E[xy] over every valid 11x11 window of
    [C,H,W] images, as direct 2-D weighted sums (no separable filtering)."""
    W2 = _window_2d()
    C, H, Wd = x.shape
    Ho, Wo = H - 10, Wd - 10
    out = [torch.empty(C, Ho, Wo, dtype=DT) for _ in range(5)]
    for i in range(Ho):
        for j in range(Wo):
            px = x[:, i:i + 11, j:j + 11]
            py = y[:, i:i + 11, j:j + 11]
            for o, t in zip(out, (px, py, px * px, py * py, px * py)):
                o[:, i, j] = (t * W2).sum((1, 2))
    return out


def test_window_taps_are_the_sigma_15_gaussian():
    for g in (oloss.gauss_1d(), oloss.gauss_1d(oloss.window_size(64, 64))):
        assert g.numel() == 11
        for c, v in enumerate(WINDOW_11_15):
            assert abs(float(g[c]) - v) < 1e-12, (c, float(g[c]), v)
            assert abs(float(g[10 - c]) - v) < 1e-12


def test_ssim_of_an_affine_pair_closed_form():
    """y = a x + b over a non-constant x: mu_y = a mu_x + b, s_y = a^2 s_x, s_xy = a s_x, so
    S = (2 mu_x mu_y + C1)(2 a s_x + C2) / ((mu_x^2 + mu_y^2 + C1)(s_x (1 + a^2) + C2))."""
    gen = torch.Generator().manual_seed(11)
    x = torch.rand(3, 19, 23, generator=gen, dtype=DT)
    for a, b in ((0.7, 0.1), (-0.4, 0.8), (1.0, 0.0)):
        y = a * x + b
        mx, _, ex2, _, _ = _window_moments(x, x)
        sx = ex2 - mx * mx
        my = a * mx + b
        pred = ((2 * mx * my + C1_LIT) * (2 * a * sx + C2_LIT)) / \
               ((mx * mx + my * my + C1_LIT) * (sx * (1 + a * a) + C2_LIT))
        got = oloss.ssim_map(x, y, oloss.gauss_1d())
        assert got.shape == pred.shape
        assert float((got - pred).abs().max()) < 1e-12, (a, b)


def test_ssim_general_pair_window_sums():
    """For unrelated x, y the map is the published formula on window moments computed here."""
    gen = torch.Generator().manual_seed(12)
    x = torch.rand(3, 16, 21, generator=gen, dtype=DT)
    y = torch.rand(3, 16, 21, generator=gen, dtype=DT) ** 2
    mx, my, ex2, ey2, exy = _window_moments(x, y)
    sx, sy, sxy = ex2 - mx * mx, ey2 - my * my, exy - mx * my
    pred = ((2 * mx * my + C1_LIT) / (mx * mx + my * my + C1_LIT)) * \
           ((2 * sxy + C2_LIT) / (sx + sy + C2_LIT))
    got = oloss.ssim_map(x, y, oloss.gauss_1d())
    assert float((got - pred).abs().max()) < 1e-12


def test_loss_mean_over_channels_and_valid_pixels_non_square():
    """loss = 0.8 mean|x - y| + 0.2 (1 - sum S / (3 Hout Wout)) on a 13 x 29 image (Hout = 3,
    Wout = 19), SSIM on the clamped images; values outside [0, 1] exercise the clamp."""
    gen = torch.Generator().manual_seed(13)
    H, W = 13, 29
    pred = torch.rand(H, W, 3, generator=gen, dtype=DT) * 1.3 - 0.15
    gt = torch.rand(H, W, 3, generator=gen, dtype=DT)
    x = pred.clamp(0, 1).permute(2, 0, 1)
    y = gt.clamp(0, 1).permute(2, 0, 1)
    mx, my, ex2, ey2, exy = _window_moments(x, y)
    sx, sy, sxy = ex2 - mx * mx, ey2 - my * my, exy - mx * my
    S = ((2 * mx * my + C1_LIT) * (2 * sxy + C2_LIT)) / \
        ((mx * mx + my * my + C1_LIT) * (sx + sy + C2_LIT))
    assert S.shape == (3, 3, 19)
    l1 = sum(abs(float(pred[i, j, c] - gt[i, j, c]))
             for i in range(H) for j in range(W) for c in range(3)) / (3 * H * W)
    expect = 0.8 * l1 + 0.2 * (1.0 - float(S.sum()) / (3 * 3 * 19))
    assert abs(float(oloss.loss_fn(pred, gt)) - expect) < 1e-12


# ------------------------------------------------------------------------ EWA projection
def _scipy_rot(q_wxyz):
    from scipy.spatial.transform import Rotation
    w, x, y, z = q_wxyz
    return torch.tensor(Rotation.from_quat([x, y, z, w]).as_matrix(), dtype=DT)


def anisotropic(cam, ratio=1.13, px=0.46, py=0.53):
    """The same pose with fx = ratio * fy and the principal point off the image centre (at
    px * W, py * H), as COLMAP's PINHOLE / OPENCV models give (spike/data.py:127-150)."""
    return {**cam, "fx": ratio * cam["fy"], "cx": px * cam["W"], "cy": py * cam["H"]}


@pytest.mark.parametrize("aniso", [False, True], ids=["fx=fy", "fx=1.13fy"])
def test_ewa_off_axis_matches_autograd_of_the_pinhole_map(aniso):
    """At points well off the optical axis: mu2d = pi(mu_cam) with pi(x, y, z) =
    (fx x / z + cx, fy y / z + cy), J = d pi / d mu_cam (autograd), Sigma2d = J Sigma_cam J^T +
    0.3 I with Sigma_cam = R_v R diag(s^2) R^T R_v^T (R from scipy), conic = Sigma2d^-1.
    With fx != fy and an off-centre principal point, fx in place of fy (or cx in place of cy)
    anywhere in the projection or its Jacobian fails."""
    gen = torch.Generator().manual_seed(21)
    cam = ogeo.make_camera(96, 160, (0.4, -0.3, 2.8))
    cam = {k: (v.to(DT) if torch.is_tensor(v) else v) for k, v in cam.items()}
    if aniso:
        cam = anisotropic(cam)
        assert abs(cam["fx"] - cam["fy"]) > 0.1 * cam["fy"] and cam["cx"] != cam["W"] / 2
    G = 12
    P = torch.zeros(G, 14, dtype=DT)
    P[:, 0:3] = torch.rand(G, 3, generator=gen, dtype=DT) * 1.6 - 0.8
    P[:, 3:7] = torch.randn(G, 4, generator=gen, dtype=DT)
    P[:, 7:10] = torch.rand(G, 3, generator=gen, dtype=DT) * 2.0 - 3.5
    pr = ogeo.project_params(P, cam)
    R_v, t_v = cam["R_v"], cam["t_v"]
    fx, fy, cx, cy = cam["fx"], cam["fy"], cam["cx"], cam["cy"]

    def pinhole(p):
        return torch.stack([fx * p[0] / p[2] + cx, fy * p[1] / p[2] + cy])

    n_off = 0
    for g in range(G):
        mc = R_v @ P[g, 0:3] + t_v
        assert float(mc[2]) > 0.2
        n_off += int(abs(float(mc[0])) > 0.2 and abs(float(mc[1])) > 0.1)
        J = torch.autograd.functional.jacobian(pinhole, mc)
        q = P[g, 3:7] / P[g, 3:7].norm()
        R = _scipy_rot(q.tolist())
        Sc = R_v @ R @ torch.diag(torch.exp(2 * P[g, 7:10])) @ R.T @ R_v.T
        S2 = J @ Sc @ J.T + 0.3 * torch.eye(2, dtype=DT)
        inv = torch.linalg.inv(S2)
        assert torch.allclose(pr["mu2d"][g], pinhole(mc), atol=1e-10)
        got = pr["conic"][g]
        assert torch.allclose(got, torch.stack([inv[0, 0], inv[0, 1], inv[1, 1]]),
                              rtol=1e-10, atol=1e-14), g
    assert n_off >= 6


# -------------------------------------------------------------------------- depth weight
def _dw_scene():
    gen = torch.Generator().manual_seed(31)
    G = 9
    P = torch.zeros(G, 14, dtype=DT)
    P[:, 0:3] = torch.rand(G, 3, generator=gen, dtype=DT) - 0.5
    P[:, 3] = 1.0
    P[:, 7:10] = -3.0
    P[:, 13] = torch.randn(G, generator=gen, dtype=DT)
    cam = ogeo.make_camera(64, 64, (0.0, 0.0, 3.0))
    cam = {k: (v.to(DT) if torch.is_tensor(v) else v) for k, v in cam.items()}
    return P, cam


def test_depth_weight_values():
    """rho = sigmoid(beta (tau - z)): 1/2 at beta = 0, at z = tau, and the closed form at a
    known (beta, tau, z); rho grows with tau for beta > 0 (nearer than tau -> weight above 1/2)."""
    P, cam = _dw_scene()
    base = ogeo.project_params(P, cam)
    o = torch.sigmoid(P[:, 13])
    z = base["depth"]
    half = ogeo.project_params(P, cam, depth_bt=torch.tensor([0.0, 2.5], dtype=DT))
    assert torch.allclose(half["o_col"], 0.5 * o, atol=1e-15)
    beta, tau = 1.7, 2.9
    dw = ogeo.project_params(P, cam, depth_bt=torch.tensor([beta, tau], dtype=DT))
    for g in range(P.shape[0]):
        rho = 1.0 / (1.0 + math.exp(-beta * (tau - float(z[g]))))
        assert abs(float(dw["o_col"][g]) - float(o[g]) * rho) < 1e-14
        if float(z[g]) < tau:
            assert float(dw["o_col"][g]) > 0.5 * float(o[g])
    at_z = ogeo.project_params(P, cam, depth_bt=torch.tensor([beta, float(z[0])], dtype=DT))
    assert abs(float(at_z["o_col"][0]) - 0.5 * float(o[0])) < 1e-14
    more = ogeo.project_params(P, cam, depth_bt=torch.tensor([beta, tau + 0.1], dtype=DT))
    assert bool((more["o_col"] > dw["o_col"]).all())


@pytest.mark.parametrize("beta,tau", [(1.3, 2.7), (4.0, 3.1), (-0.8, 2.9)])
def test_depth_weight_gradients_closed_form(beta, tau):
    """With L = sum_g c_g keo_g (keo = keep sigmoid(op) rho): dL/dbeta = sum gpre (tau - z),
    dL/dtau = sum gpre beta, gpre = c_g keep o rho (1 - rho) (tools/m8_depthweight_oracle.py:7-12)."""
    P, cam = _dw_scene()
    gen = torch.Generator().manual_seed(32)
    c = torch.randn(P.shape[0], generator=gen, dtype=DT)
    bt = torch.tensor([beta, tau], dtype=DT, requires_grad=True)
    pr = ogeo.project_params(P, cam, depth_bt=bt)
    (pr["o_col"] * c).sum().backward()
    z = pr["depth"].detach()
    o = torch.sigmoid(P[:, 13])
    rho = torch.sigmoid(beta * (tau - z))
    gpre = c * o * rho * (1 - rho)
    assert abs(float(bt.grad[0]) - float((gpre * (tau - z)).sum())) < 1e-13
    assert abs(float(bt.grad[1]) - float((gpre * beta).sum())) < 1e-13


def test_depth_weight_is_a_constant_of_the_geometry_gradient():
    """The device step holds z constant in rho = sigmoid(beta (tau - z))
    (tools/resident_traced.py:333-337): the render and the gradient of every column but the
    opacity equal those of the same scene without a depth weight whose opacity already carries
    rho (sigmoid(op') = sigmoid(op) rho).  A rho that let the gradient reach z would add a
    term to the means gradient."""
    from oracle import binning as obin
    from oracle import pipeline as opipe
    P, cam = _dw_scene()
    P[:, 7:10] = -2.2
    tmap = obin.TileMap(64, 64, 16)
    gen = torch.Generator().manual_seed(33)
    tgt = torch.rand(64, 64, 3, generator=gen, dtype=DT)
    beta, tau = 3.0, 3.0
    z = ogeo.project_params(P, cam)["depth"]
    rho = torch.sigmoid(beta * (tau - z))
    assert float(rho.min()) > 0.05 and float(rho.max()) < 0.95
    P2 = P.clone()
    o2 = torch.sigmoid(P[:, 13]) * rho
    P2[:, 13] = torch.log(o2 / (1 - o2))
    img1, L1, g1, _ = opipe.render_and_grad(P, cam, tmap, tgt, depth_bt=(beta, tau))
    img2, L2, g2, _ = opipe.render_and_grad(P2, cam, tmap, tgt)
    assert torch.allclose(img1, img2, rtol=0, atol=1e-13)
    assert float(g1[:, 0:3].abs().max()) > 1e-6
    assert torch.allclose(g1[:, :13], g2[:, :13], rtol=1e-9, atol=1e-15)


def test_empty_slots_carry_zero_operands():
    """An empty slot (valid = 0, index 0) carries theta = 0, colour 0 and opacity 0
    (tools/m4_train_binned.py:207-211 mask all three by valid)."""
    from oracle import binning as obin
    P, cam = _dw_scene()
    tmap = obin.TileMap(64, 64, 16)
    theta, col, oc, _, (idx, valid) = osplat.operands(P, cam, tmap, K=16)
    assert bool((~valid).any()) and bool(valid.any())
    assert float(theta.permute(0, 2, 1)[~valid].abs().max()) == 0.0
    assert float(col[~valid].abs().max()) == 0.0 and float(oc[~valid].abs().max()) == 0.0
    assert float(theta.permute(0, 2, 1)[valid].abs().max()) > 0.0


def test_train_step_number_is_one_based():
    """train_step(..., t) applies Adam step t counting from 1: the first call (t = 1) moves P by
    exactly what torch.optim.Adam's first step does with the same gradient."""
    from oracle import binning as obin
    from oracle import pipeline as opipe
    P, cam = _dw_scene()
    tmap = obin.TileMap(64, 64, 16)
    tgt = torch.rand(64, 64, 3, generator=torch.Generator().manual_seed(34), dtype=DT)
    lr = torch.full((14,), 1e-3, dtype=DT)
    _, _, g, _ = opipe.render_and_grad(P, cam, tmap, tgt)
    ref = oadam.torch_adam_reference(P, [g], lr)
    Pt, m, v = P.clone(), torch.zeros_like(P), torch.zeros_like(P)
    opipe.train_step(Pt, m, v, 1, cam, tmap, tgt, lr)
    assert torch.allclose(Pt - P, ref - P, rtol=1e-9, atol=1e-18)


# ------------------------------------------------------------- camera, cull, loss clamps
def test_look_at_frame_orientation():
    """look_at_opencv (spike/camera.py:51-63): z toward the target, x = normalise(up x z), and
    y = z x x, which by the triple product is the part of `up` orthogonal to z (normalised); the
    target lands on the principal point at depth |target - eye|."""
    for eye, target in (((0.3, 0.9, 2.7), (0.1, -0.2, 0.05)), ((-2.0, 0.4, -1.1), (0.0, 0.0, 0.0))):
        R_v, t_v = ogeo.look_at_opencv(eye, target, dtype=DT)
        e, t, up = _f(eye), _f(target), _f([0.0, 1.0, 0.0])
        z = (t - e) / (t - e).norm()
        y = up - z * (z @ up)
        y = y / y.norm()
        assert torch.allclose(R_v[2], z, atol=1e-14)
        assert torch.allclose(R_v[1], y, atol=1e-14)
        assert torch.allclose(R_v[0], torch.linalg.cross(y, z), atol=1e-14)
        assert abs(float(torch.det(R_v)) - 1.0) < 1e-13
        cam_t = R_v @ t + t_v
        assert torch.allclose(cam_t, torch.stack([_f(0.0), _f(0.0), (t - e).norm()]), atol=1e-14)


def test_horizontal_field_of_view():
    """make_camera's fov is horizontal (fx = fy = W / (2 tan(fov/2)), spike/synthetic.py:21):
    on a 32 x 96 image a point fov/2 off the axis horizontally lands on the right edge x = W,
    one fov/2 off vertically lands W/2 below the centre, not H/2."""
    H, W, fov = 32, 96, 60.0
    cam = ogeo.make_camera(H, W, (0.4, 0.3, 3.0), fov_deg=fov)
    R_v, t_v = cam["R_v"].to(DT), cam["t_v"].to(DT)
    tan = math.tan(math.radians(fov) / 2.0)
    pts_cam = _f([[2.0 * tan, 0.0, 2.0], [0.0, 2.0 * tan, 2.0]])
    world = (pts_cam - t_v) @ R_v                         # R_v^T (p - t_v), row-wise
    cov = torch.eye(3, dtype=DT).expand(2, 3, 3) * 1e-4
    mu2d, _, _, _ = ogeo.project_ewa(world, cov, R_v, t_v, cam["fx"], cam["fy"], cam["cx"],
                                     cam["cy"])
    assert torch.allclose(mu2d[0], _f([W, H / 2.0]), atol=1e-9)
    assert torch.allclose(mu2d[1], _f([W / 2.0, H / 2.0 + W / 2.0]), atol=1e-9)


def test_near_cull_is_strict_and_clamps_z():
    """keep = depth > near (spike/geometry.py:39): a gaussian exactly at the near plane is
    culled; a culled gaussian is projected with z clamped to near (:40), so it stays finite."""
    R_v = _f([[-1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, -1.0]])   # eye (0, 0, 2) -> origin
    t_v = _f([0.0, 0.0, 2.0])
    means = _f([[0.0, 0.0, 1.75], [0.0, 0.0, 1.7], [-0.5, -0.25, 3.0]])  # depth 0.25, 0.3, -1
    cov = torch.eye(3, dtype=DT).expand(3, 3, 3) * 0.01
    fx, fy, cx, cy = 100.0, 90.0, 32.0, 24.0
    mu2d, conic, depth, keep = ogeo.project_ewa(means, cov, R_v, t_v, fx, fy, cx, cy, 0.3, 0.25)
    assert float(depth[0]) == 0.25 and keep.tolist() == [False, True, False]
    assert torch.allclose(mu2d[2], _f([fx * 0.5 / 0.25 + cx, fy * -0.25 / 0.25 + cy]),
                          atol=1e-12)
    assert bool(torch.isfinite(conic).all())


def test_ssim_clamps_both_images():
    """SSIM sees clamp(pred, 0, 1) and clamp(gt, 0, 1) (spike/metrics.py:7), the L1 term the raw
    values: pred = 1, gt = 3 everywhere give SSIM 1 and loss (1 - lambda) * 2."""
    pred = torch.ones(16, 16, 3, dtype=DT)
    gt = torch.full((16, 16, 3), 3.0, dtype=DT)
    for a, b in ((pred, gt), (gt, pred)):
        L = float(oloss.loss_fn(a, b, 0.2))
        assert abs(L - 0.8 * 2.0) < 1e-14


def test_dense_render_ignores_culled_gaussians():
    """The poly-splat weight is gated by keep (spike/forward.py:61-66): a gaussian behind the
    camera, which the z clamp projects onto the image centre, changes nothing."""
    P, cam = _dw_scene()
    base = osplat.render_dense(P, cam)
    extra = torch.cat([P, P[:1].clone()])
    extra[-1, 0:3] = _f([0.0, 0.0, 4.0])                  # 1 behind the eye at (0, 0, 3)
    extra[-1, 13] = 3.0
    assert torch.allclose(osplat.render_dense(extra, cam), base, rtol=0, atol=1e-15)
