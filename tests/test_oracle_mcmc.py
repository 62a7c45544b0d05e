"""The oracle's MCMC pieces, pinned without the reference:

* Philox4x32-10 against the known-answer vectors of the Random123 distribution (the published
  generator the device kernels use); moments of the derived normals and uniforms;
* spike/tests/test_mcmc.py restated on the oracle's dense render: n coincident copies at o/n
  render exactly like one gaussian at o (with a negative control), a relocation with zero
  offset leaves the render nearly unchanged, SGLD noise is gated to near-dead gaussians;
* the regularisation gradient in closed form (d/dop = lambda_o/G o(1-o),
  d/dlog_s = lambda_s/(3G) s);
* the inverse-CDF target pick: empirical frequencies proportional to opacity, and exact picks
  at prefix-sum boundaries;
* hand-worked cases: the near-dead gate's midpoint and width, the SGLD noise covariance of a
  rotated anisotropic gaussian, the strict dead threshold, a relocation's split, clamp and
  copies, and the uniform grid's symmetry about 1/2.
"""
import math

import numpy as np
import pytest
import torch

from oracle import geometry, mcmc, rng, splat

D = torch.float64


def test_philox_known_answers():
    kat = [
        ([0, 0, 0, 0], [0, 0], "6627e8d5 e169c58d bc57ac4c 9b00dbd8"),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, "408f276d 41c83b0e a20bc7c6 6d5451fd"),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         "d16cfe09 94fdcceb 5001e420 24126ea1"),
    ]
    for ctr, key, want in kat:
        out = rng.philox4x32_10(np.array(ctr, dtype=np.uint64), np.array(key, dtype=np.uint64))
        assert " ".join(f"{int(x):08x}" for x in out) == want


def test_normals_and_uniforms_moments():
    z = rng.normals3(np.arange(200_000), step=7, tag=rng.TAG_SGLD, seed=1234)
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1.0) < 0.01
    assert abs(np.corrcoef(z[:, 0], z[:, 1])[0, 1]) < 0.01
    u = rng.uniform1(np.arange(200_000), step=3, tag=rng.TAG_RELOC_PICK, seed=99)
    assert 0.0 < u.min() and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.005
    # different steps and tags give different streams
    a = rng.uniform1(np.arange(10), 1, 2, 5)
    b = rng.uniform1(np.arange(10), 2, 2, 5)
    c = rng.uniform1(np.arange(10), 1, 3, 5)
    assert not np.allclose(a, b) and not np.allclose(a, c)


def _logit(p):
    return math.log(p / (1.0 - p))


def _scene(G, seed):
    g = torch.Generator().manual_seed(seed)
    P = torch.zeros(G, 14, dtype=D)
    P[:, 0:3] = (torch.rand(G, 3, generator=g, dtype=D) * 2 - 1) * 0.6
    q = torch.zeros(G, 4, dtype=D)
    q[:, 0] = 1.0
    P[:, 3:7] = q + 0.1 * torch.randn(G, 4, generator=g, dtype=D)
    P[:, 7:10] = math.log(0.08) + 0.1 * torch.randn(G, 3, generator=g, dtype=D)
    P[:, 10:13] = torch.randn(G, 3, generator=g, dtype=D) * 1.5
    P[:, 13] = _logit(0.7)
    return P


def _cam(res=24):
    return geometry.make_camera(res, res, (0.0, 0.0, 3.0))


def test_split_preserves_render_exactly():
    cam = _cam()
    o0, n = 0.6, 4
    base = _scene(1, 3)
    multi = base.repeat(n, 1)
    multi[:, 13] = _logit(o0 / n)
    single = base.clone()
    single[:, 13] = _logit(o0)
    a = splat.render_dense(single, cam)
    b = splat.render_dense(multi, cam)
    assert torch.allclose(a, b, atol=1e-10)
    multi[:, 13] = _logit(o0)                             # negative control: no split
    assert (splat.render_dense(multi, cam) - a).abs().max() > 1e-3


def test_relocate_with_zero_offset_keeps_render():
    cam = _cam()
    P = _scene(40, 5)
    P[:12, 13] = _logit(1e-4)                             # 12 dead gaussians
    before = splat.render_dense(P, cam)
    o, dead, alive = mcmc.classify(P, 0.005)
    assert dead.numel() == 12
    u = torch.tensor(rng.uniform1(np.arange(12), 1, rng.TAG_RELOC_PICK, 7))
    targets = mcmc.pick_targets(o, alive, u)
    m, v = torch.ones_like(P), torch.ones_like(P)
    touched = mcmc.relocate(P, m, v, dead, targets, torch.zeros(12, 3, dtype=D))
    after = splat.render_dense(P, cam)
    assert (before - after).abs().max() < 2e-2
    assert torch.equal(torch.sort(touched).values, torch.unique(torch.cat([dead, targets])))
    assert float(m[touched].abs().max()) == 0.0 and float(v[touched].abs().max()) == 0.0
    untouched = torch.ones(40, dtype=torch.bool)
    untouched[touched] = False
    assert float(m[untouched].min()) == 1.0
    # every opacity sum over a target and its copies is the target's old opacity
    o_new = torch.sigmoid(P[:, 13])
    for t in torch.unique(targets):
        grp = torch.cat([t[None], dead[targets == t]])
        assert abs(float(o_new[grp].sum() - o[t])) < 1e-9


def test_sgld_noise_is_opacity_gated():
    P = _scene(2, 1)
    P[0, 13] = _logit(0.99)
    P[1, 13] = _logit(1e-3)
    eps = torch.tensor(rng.normals3(np.arange(2), 1, rng.TAG_SGLD, 3), dtype=D)
    d = mcmc.sgld_noise(P, 5e-3, 100.0, eps).norm(dim=1)
    assert float(d[0]) < 1e-6
    assert float(d[1]) > float(d[0])


def test_reg_grad_closed_form():
    P = _scene(30, 2)
    lo, ls = 0.01, 0.02
    g = mcmc.reg_grad(P, lo, ls)
    o = torch.sigmoid(P[:, 13])
    assert torch.allclose(g[:, 13], lo / 30 * o * (1 - o))
    assert torch.allclose(g[:, 7:10], ls / 90 * torch.exp(P[:, 7:10]))
    assert float(g[:, :7].abs().max()) == 0.0 and float(g[:, 10:13].abs().max()) == 0.0


def test_pick_targets_frequencies_follow_opacity():
    o = torch.tensor([0.001, 0.5, 0.2, 0.0, 0.3, 0.9, 0.004], dtype=D)
    alive = torch.tensor([1, 2, 4, 5])
    u = torch.tensor(rng.uniform1(np.arange(200_000), 1, rng.TAG_RELOC_PICK, 11))
    t = mcmc.pick_targets(o, alive, u)
    freq = torch.bincount(t, minlength=7).double() / len(u)
    want = torch.zeros(7, dtype=D)
    want[alive] = o[alive] / o[alive].sum()
    assert torch.allclose(freq, want, atol=0.005)


def test_random_background_draws():
    """The random-background colour: three uniforms in (0, 1) per (view, step, seed), fp32,
    different for another view, step or seed, uniform over many steps (mean 1/2, variance
    1/12)."""
    a = rng.random_bg(0, 5, 7)
    assert a.dtype == np.float32 and a.shape == (3,)
    assert bool(((a > 0) & (a < 1)).all())
    for other in (rng.random_bg(1, 5, 7), rng.random_bg(0, 6, 7), rng.random_bg(0, 5, 8)):
        assert not np.array_equal(a, other)
    many = np.stack([rng.random_bg(0, s, 3) for s in range(20000)])
    assert abs(float(many.mean()) - 0.5) < 0.01
    assert abs(float(many.var()) - 1.0 / 12.0) < 0.005
    w = rng.draws(np.array([0]), 5, rng.TAG_BG, 7)[0]
    assert np.array_equal(a, rng.uniform(w[:3]).astype(np.float32))


def test_rgba_premult_composites_over_a_background():
    """(alpha r, alpha g, alpha b, 1 - alpha): alpha = 1 gives the colour, alpha = 0 the
    background, and pm + (1 - alpha) bg is straight compositing."""
    from ttsplat import kernels
    gen = torch.Generator().manual_seed(3)
    rgb = torch.rand(5, 7, 3, generator=gen)
    alpha = torch.rand(5, 7, 1, generator=gen)
    alpha[0, 0], alpha[0, 1] = 1.0, 0.0
    pm = kernels.rgba_premult(torch.cat([rgb, alpha], -1))
    bg = torch.tensor([0.2, 0.5, 0.9])
    out = pm[..., :3] + pm[..., 3:4] * bg
    assert torch.allclose(out, rgb * alpha + (1 - alpha) * bg, atol=1e-6)
    assert torch.equal(out[0, 0], rgb[0, 0]) and torch.allclose(out[0, 1], bg)


def test_near_dead_gate_midpoint_and_width():
    """op_sigmoid(1 - o) is 1/2 at opacity 0.005 (spike/mcmc.py:13-15: gate ~1 only for
    opacity below ~0.005) and rises from 0.1 to 0.9 over 2 ln 9 / 100 of opacity."""
    assert float(mcmc.op_sigmoid(torch.tensor(1.0 - 0.005, dtype=D))) == pytest.approx(0.5, abs=1e-12)
    lo = 0.995 - math.log(9.0) / 100.0
    hi = 0.995 + math.log(9.0) / 100.0
    assert float(mcmc.op_sigmoid(torch.tensor(lo, dtype=D))) == pytest.approx(0.1, abs=1e-12)
    assert float(mcmc.op_sigmoid(torch.tensor(hi, dtype=D))) == pytest.approx(0.9, abs=1e-12)


def test_sgld_noise_has_the_gaussian_covariance():
    """For the unit draws e_x, e_y, e_z the noise columns form w L with L L^T = Sigma, the
    gaussian's own covariance R diag(s^2) R^T (oracle/geometry.py cov3d): an anisotropic,
    rotated gaussian tells L = R diag(s) from diag(s) R."""
    P = _scene(1, 9).repeat(3, 1)
    P[:, 3:7] = torch.tensor([math.cos(0.6), 0.3, -0.5, math.sin(0.6)], dtype=D)
    P[:, 7:10] = torch.log(torch.tensor([0.05, 0.2, 0.7], dtype=D))
    P[:, 13] = _logit(1e-4)
    lr, nlr = 5e-3, 100.0
    N = mcmc.sgld_noise(P, lr, nlr, torch.eye(3, dtype=D)).T          # columns = w L e_j
    o = torch.sigmoid(P[0, 13])
    w = float(torch.sigmoid(100.0 * ((1.0 - o) - 0.995))) * nlr * lr
    R = geometry.quat_to_rotmat(P[:1, 3:7])[0]
    sigma = geometry.cov3d(torch.exp(P[:1, 7:10]), R[None])[0]
    assert torch.allclose(N @ N.T, w * w * sigma, rtol=1e-12, atol=0.0)
    assert not torch.allclose(N @ N.T, w * w * torch.diag(torch.exp(2 * P[0, 7:10])), rtol=1e-3)


def test_classify_threshold_is_strict():
    """dead = o < thr, alive = o >= thr (spike/mcmc.py:45-46): an opacity equal to the
    threshold is alive."""
    P = _scene(3, 4)
    P[:, 13] = torch.tensor([0.0, -0.1, 0.1], dtype=D)      # o = 1/2 exactly, below, above
    _, dead, alive = mcmc.classify(P, 0.5)
    assert dead.tolist() == [1] and alive.tolist() == [0, 2]


def test_pick_targets_boundaries():
    """The first live j whose inclusive prefix sum exceeds u * total: u * total on a prefix
    boundary goes to the next gaussian, u = 0 to the first, u -> 1 to the last."""
    o = torch.tensor([0.25, 0.0, 0.25, 0.5], dtype=D)
    alive = torch.tensor([0, 2, 3])
    u = torch.tensor([0.0, 0.2499, 0.25, 0.4999, 0.5, 0.75, 0.999999], dtype=D)
    assert mcmc.pick_targets(o, alive, u).tolist() == [0, 0, 2, 2, 3, 3, 3]


def test_relocate_split_clamp_and_copies():
    """Hand-worked relocation: a target at o = 0.006 with three copies splits to 0.0015 each
    (o_t / (n_t + 1), spike/mcmc.py:51-54); one at 1.5e-6 with one copy clamps to 1e-6; a copy
    takes the target's row with means + offset (spike/mcmc.py:57-65)."""
    P = _scene(7, 6)
    P[:, 13] = torch.tensor([_logit(0.006), _logit(1e-5), _logit(1e-5), _logit(1e-5),
                             _logit(1.5e-6), _logit(1e-5), _logit(0.8)], dtype=D)
    old = P.clone()
    dead = torch.tensor([1, 2, 3, 5])
    targets = torch.tensor([0, 0, 0, 4])
    offsets = torch.tensor([[0.1, 0.0, 0.0], [0.0, -0.2, 0.0], [0.0, 0.0, 0.3],
                            [0.01, 0.02, 0.03]], dtype=D)
    m, v = torch.ones_like(P), torch.ones_like(P)
    touched = mcmc.relocate(P, m, v, dead, targets, offsets)
    o_new = torch.sigmoid(P[:, 13])
    for i in (0, 1, 2, 3):
        assert float(o_new[i]) == pytest.approx(0.0015, rel=1e-12)
    for i in (4, 5):
        assert float(o_new[i]) == pytest.approx(1e-6, rel=1e-9)
    assert float(o_new[6]) == pytest.approx(0.8, rel=1e-12)
    for d, t, off in zip(dead.tolist(), targets.tolist(), offsets):
        assert torch.equal(P[d, 0:3], old[t, 0:3] + off)
        assert torch.equal(P[d, 3:13], old[t, 3:13])
    assert touched.tolist() == [0, 1, 2, 3, 4, 5]


def test_uniform_conversion_is_centred():
    """uniform(x) = ((x >> 8) + 1/2) 2^-24: the 2^24 cell midpoints, symmetric about 1/2
    (uniform(x) + uniform(~x) = 1 exactly), from 2^-25 to 1 - 2^-25."""
    x = np.concatenate([np.array([0, 255, 256, 0xFFFFFFFF], dtype=np.uint64),
                        rng.draws(np.arange(1000), 1, 2, 3).reshape(-1)])
    u = rng.uniform(x)
    assert np.array_equal(u + rng.uniform(x ^ np.uint64(0xFFFFFFFF)), np.ones_like(u))
    assert u[0] == 2.0 ** -25 and u[1] == 2.0 ** -25 and u[2] == 3 * 2.0 ** -25
    assert u[3] == 1.0 - 2.0 ** -25
