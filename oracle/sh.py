"""Oracle: view-dependent colour from real spherical harmonics, degrees 0-3.

Test infrastructure only (see oracle/__init__.py).

Restates
  spike/sh.py:9-19,43-51   the SH constants C0..C3 (the normalisation constants of the real SH
                           basis in the inria/gsplat sign convention)
  spike/sh.py:54-72        eval_sh_color: colour = clamp(0.5 + sum_l b_l(dir) c_l, min=0),
                           dir normalised as dir / max(|dir|, 1e-12)
  tools/resident_traced.py:246-264,339-341
                           the device step's use: dir = means3d - camera centre, coefficients
                           [G,16,3] = [DC | color_rest[G,15,3]]
  tools/resident_traced.py:405-410
                           its backward: d colour / d coefficient = b_l through the clamp gate;
                           the view direction is a constant (no gradient reaches the means
                           through it)

Pinned by tests/test_oracle_sh.py: the basis against scipy's complex spherical harmonics
(textbook routine; catches a wrong constant, sign or monomial), orthonormality on the sphere,
and the reference's own SH checks (spike/tests/test_sh_color.py restated).
"""
import torch

C0 = 0.28209479177387814
C1 = 0.4886025119029199
C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792,
      0.5462742152960396)
C3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
      -0.4570457994644658, 1.445305721320277, -0.5900435899266435)


def n_coeffs(deg):
    """Number of SH coefficients per channel at degree deg (DC included)."""
    return (deg + 1) ** 2


def basis(deg, dirs):
    """The real SH basis b_l(dir), l < (deg+1)^2, for directions [...,3] (normalised here)
    -> [..., (deg+1)^2] (spike/sh.py:54-72 term by term)."""
    d = dirs / dirs.norm(dim=-1, keepdim=True).clamp(min=1e-12)
    x, y, z = d[..., 0], d[..., 1], d[..., 2]
    b = [torch.full_like(x, C0)]
    if deg >= 1:
        b += [-C1 * y, C1 * z, -C1 * x]
    if deg >= 2:
        xx, yy, zz, xy, yz, xz = x * x, y * y, z * z, x * y, y * z, x * z
        b += [C2[0] * xy, C2[1] * yz, C2[2] * (2.0 * zz - xx - yy), C2[3] * xz,
              C2[4] * (xx - yy)]
    if deg >= 3:
        b += [C3[0] * y * (3 * xx - yy), C3[1] * xy * z, C3[2] * y * (4 * zz - xx - yy),
              C3[3] * z * (2 * zz - 3 * xx - 3 * yy), C3[4] * x * (4 * zz - xx - yy),
              C3[5] * z * (xx - yy), C3[6] * x * (xx - 3 * yy)]
    return torch.stack(b, dim=-1)


def eval_sh_color(deg, coeffs, dirs):
    """coeffs [..., >= (deg+1)^2, 3] (coeffs[..., 0, :] = DC), dirs [..., 3]
    -> clamp(0.5 + sum_l b_l c_l, min=0) [..., 3] (spike/sh.py:54-72)."""
    nb = n_coeffs(deg)
    b = basis(deg, dirs)                                     # [..., nb]
    r = (b[..., None] * coeffs[..., :nb, :]).sum(dim=-2)
    return (r + 0.5).clamp(min=0.0)


def camera_center(R_v, t_v):
    """World position of the camera: -R_v^T t_v (spike/camera.py:46-48)."""
    return -(R_v.transpose(-1, -2) @ t_v)


def view_color(means3d, color_dc, color_rest, deg, R_v, t_v):
    """Colour of the device step: SH of degree deg in the direction means3d - centre, with the
    direction held constant for the gradient (tools/resident_traced.py:339-341,405-410).
    color_rest [G,15,3]."""
    dirs = (means3d - camera_center(R_v, t_v)[None, :]).detach()
    coeffs = torch.cat([color_dc[:, None, :], color_rest], dim=1)
    return eval_sh_color(deg, coeffs, dirs)
