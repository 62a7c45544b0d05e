"""The oracle's view-dependent SH colour, pinned without the reference:

* the basis against scipy's complex spherical harmonics (a textbook routine): the inria/gsplat
  real basis is b_{l,m} = sqrt(2) Im Y_l^{|m|} (m < 0), Y_l^0 (m = 0), sqrt(2) Re Y_l^m (m > 0),
  Condon-Shortley phase included — a wrong constant, sign or monomial fails it;
* orthonormality over the sphere (Gauss-Legendre x uniform-azimuth quadrature, exact here);
* spike/tests/test_sh_color.py restated: zero rest == DC colour at every degree, gradcheck of
  the coefficients, colour changes with the direction when the rest is non-zero;
* the device step's gradient convention: no gradient reaches the means through the direction.
"""
import math

import numpy as np
import pytest
import torch

from oracle import geometry, sh

D = torch.float64


def _real_sh_scipy(l, m, dirs):
    from scipy.special import sph_harm_y
    d = dirs / np.linalg.norm(dirs, axis=-1, keepdims=True)
    theta = np.arccos(np.clip(d[:, 2], -1.0, 1.0))        # polar
    phi = np.arctan2(d[:, 1], d[:, 0])                     # azimuth
    if m == 0:
        return sph_harm_y(l, 0, theta, phi).real
    Y = sph_harm_y(l, abs(m), theta, phi)
    return math.sqrt(2.0) * (Y.imag if m < 0 else Y.real)


def test_basis_matches_scipy_complex_sh():
    rng = np.random.default_rng(0)
    dirs = rng.normal(size=(500, 3)) * rng.uniform(0.1, 10.0, size=(500, 1))
    b = sh.basis(3, torch.tensor(dirs, dtype=D)).numpy()
    for l in range(4):
        for m in range(-l, l + 1):
            ref = _real_sh_scipy(l, m, dirs)
            np.testing.assert_allclose(b[:, l * l + l + m], ref, atol=1e-12, rtol=0,
                                       err_msg=f"l={l} m={m}")


def test_basis_orthonormal_on_the_sphere():
    xg, wg = np.polynomial.legendre.leggauss(12)          # cos(theta) nodes
    nphi = 16
    phis = 2 * math.pi * np.arange(nphi) / nphi
    ct = np.repeat(xg, nphi)
    st = np.sqrt(1 - ct * ct)
    ph = np.tile(phis, len(xg))
    w = np.repeat(wg, nphi) * (2 * math.pi / nphi)
    dirs = torch.tensor(np.stack([st * np.cos(ph), st * np.sin(ph), ct], 1), dtype=D)
    b = sh.basis(3, dirs).numpy()
    gram = (b * w[:, None]).T @ b
    np.testing.assert_allclose(gram, np.eye(16), atol=1e-12)


def test_zero_rest_equals_dc_at_every_degree():
    torch.manual_seed(0)
    dc = torch.randn(50, 3, dtype=D)
    coeffs = torch.cat([dc[:, None, :], torch.zeros(50, 15, 3, dtype=D)], dim=1)
    dirs = torch.randn(50, 3, dtype=D)
    for deg in (0, 1, 2, 3):
        assert torch.allclose(sh.eval_sh_color(deg, coeffs, dirs), geometry.color_from_dc(dc),
                              atol=1e-12), deg


def test_eval_sh_gradcheck():
    torch.manual_seed(2)
    coeffs = torch.randn(8, 16, 3, dtype=D, requires_grad=True)
    dirs = torch.randn(8, 3, dtype=D)
    assert torch.autograd.gradcheck(lambda c: sh.eval_sh_color(3, c, dirs), (coeffs,), eps=1e-6,
                                    atol=1e-6)


def test_color_depends_on_direction_with_rest():
    torch.manual_seed(3)
    coeffs = torch.zeros(4, 16, 3, dtype=D)
    coeffs[:, 0, :] = 0.5
    coeffs[:, 1:, :] = torch.randn(4, 15, 3, dtype=D)
    c1 = sh.eval_sh_color(3, coeffs, torch.tensor([[0.0, 0.0, 1.0]] * 4, dtype=D))
    c2 = sh.eval_sh_color(3, coeffs, torch.tensor([[1.0, 0.0, 0.0]] * 4, dtype=D))
    assert (c1 - c2).abs().max() > 1e-3


def test_degree_uses_only_its_coefficients():
    torch.manual_seed(4)
    coeffs = torch.randn(6, 16, 3, dtype=D)
    dirs = torch.randn(6, 3, dtype=D)
    for deg in (0, 1, 2, 3):
        n = (deg + 1) ** 2
        c2 = coeffs.clone()
        c2[:, n:, :] = 100.0                               # unused by this degree
        assert torch.equal(sh.eval_sh_color(deg, coeffs, dirs), sh.eval_sh_color(deg, c2, dirs))


def test_view_color_has_no_gradient_through_the_direction():
    torch.manual_seed(5)
    G = 7
    R_v, t_v = geometry.look_at_opencv((0.3, -0.2, 3.0))
    means = torch.randn(G, 3, dtype=D, requires_grad=True)
    dc = torch.randn(G, 3, dtype=D, requires_grad=True)
    rest = torch.randn(G, 15, 3, dtype=D, requires_grad=True)
    col = sh.view_color(means, dc, rest, 3, R_v.to(D), t_v.to(D))
    col.sum().backward()
    assert means.grad is None
    # the coefficient gradient is the basis (through the clamp gate)
    dirs = means.detach() - sh.camera_center(R_v.to(D), t_v.to(D))[None]
    b = sh.basis(3, dirs)
    gate = (col > 0).to(D)
    assert torch.allclose(rest.grad, b[:, 1:, None] * gate[:, None, :])
    assert torch.allclose(dc.grad, sh.C0 * gate)


def test_camera_center_is_the_eye():
    eye = (0.7, -1.1, 2.5)
    R_v, t_v = geometry.look_at_opencv(eye)
    assert torch.allclose(sh.camera_center(R_v.to(D), t_v.to(D)),
                          torch.tensor(eye, dtype=D), atol=1e-6)
