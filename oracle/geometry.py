"""Oracle: per-gaussian geometry (EWA projection) and colour/opacity activations.

Test infrastructure only (see oracle/__init__.py).

Restates
  spike/geometry.py:10-19   quat_to_rotmat  (wxyz, normalised with a 1e-12 clamp)
  spike/geometry.py:22-25   cov3d           (R diag(s^2) R^T)
  spike/geometry.py:28-57   project_ewa     (mu_cam, near cull, z clamp, J, blur, 2x2 inverse)
  spike/forward.py:69-71    color_from_dc   (clamp(0.5 + C0*dc, min=0))
  tools/m4_train_binned.py:194-202  the activations keo = keep*sigmoid(op),
                                     color_o = keo*color, o_col = keo, w_b = softplus(w_b_raw)
  spike/camera.py:51-70     look_at_opencv, pixel_grid

Parameter layout of the device-resident trainer (tools/resident_traced.py:91):
  [G,14] columns mx,my,mz, qw,qx,qy,qz, lx,ly,lz, cr,cg,cb, op
"""
import math

import torch

C0 = 0.28209479177387814  # spike/sh.py:9 (SH degree-0 constant)

PN = ("mx", "my", "mz", "qw", "qx", "qy", "qz", "lx", "ly", "lz", "cr", "cg", "cb", "op")


def split_params(P):
    """[G,14] -> (means3d[G,3], quats[G,4], log_scales[G,3], color_dc[G,3], opacity_raw[G])."""
    return P[:, 0:3], P[:, 3:7], P[:, 7:10], P[:, 10:13], P[:, 13]


def look_at_opencv(eye, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0), dtype=torch.float32):
    """World->camera (R_v, t_v) for an OpenCV camera at `eye` looking at `target`
    (spike/camera.py:51-63): rows of R_v are the camera x, y, z axes in world coordinates."""
    eye = torch.as_tensor(eye, dtype=dtype)
    fwd = torch.as_tensor(target, dtype=dtype) - eye
    fwd = fwd / fwd.norm()
    right = torch.linalg.cross(torch.as_tensor(up, dtype=dtype), fwd)
    right = right / right.norm()
    down = torch.linalg.cross(fwd, right)
    R_v = torch.stack([right, down, fwd], dim=0)
    return R_v, -(R_v @ eye)


def pixel_grid(H, W, dtype=torch.float32):
    """Row-major pixel centres (spike/camera.py:66-70): px = col+0.5, py = row+0.5."""
    rows = torch.arange(H, dtype=dtype).repeat_interleave(W)
    cols = torch.arange(W, dtype=dtype).repeat(H)
    return cols + 0.5, rows + 0.5


def quat_to_rotmat(q):
    """wxyz quaternion (normalised here) -> rotation [...,3,3] (spike/geometry.py:10-19)."""
    q = q / q.norm(dim=-1, keepdim=True).clamp(min=1e-12)
    w, x, y, z = q.unbind(-1)
    rows = [
        (1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)),
        (2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)),
        (2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)),
    ]
    return torch.stack([torch.stack(r, dim=-1) for r in rows], dim=-2)


def cov3d(scales, R):
    """Sigma3 = R diag(s^2) R^T (spike/geometry.py:22-25)."""
    return (R * (scales * scales)[..., None, :]) @ R.transpose(-1, -2)


def project_ewa(means3d, cov_w, R_v, t_v, fx, fy, cx, cy, blur_eps=0.3, near=0.2):
    """EWA projection (spike/geometry.py:28-57).

    Returns mu2d[G,2], conic[G,3] = (a, b, c) of Sigma2d^-1, depth[G], keep[G] (depth > near).
    The camera-space z is clamped to `near` before use so culled gaussians stay finite."""
    mu_cam = means3d @ R_v.T + t_v
    depth = mu_cam[:, 2]
    keep = depth > near
    z = depth.clamp(min=near)
    xc, yc = mu_cam[:, 0], mu_cam[:, 1]
    mu2d = torch.stack([fx * xc / z + cx, fy * yc / z + cy], dim=-1)
    S_cam = R_v @ cov_w @ R_v.T                                       # [G,3,3]
    zero = torch.zeros_like(z)
    zz = z * z
    J = torch.stack([torch.stack([fx / z, zero, -fx * xc / zz], -1),
                     torch.stack([zero, fy / z, -fy * yc / zz], -1)], dim=-2)   # [G,2,3]
    S2 = J @ S_cam @ J.transpose(-1, -2)
    s00 = S2[:, 0, 0] + blur_eps
    s11 = S2[:, 1, 1] + blur_eps
    s01 = S2[:, 0, 1]
    det = (s00 * s11 - s01 * s01).clamp(min=1e-12)
    conic = torch.stack([s11 / det, -s01 / det, s00 / det], dim=-1)
    return mu2d, conic, depth, keep


def color_from_dc(color_dc):
    """SH degree-0 colour, min-only clamp (spike/forward.py:69-71)."""
    return (0.5 + C0 * color_dc).clamp(min=0.0)


def softplus(x):
    return torch.nn.functional.softplus(torch.as_tensor(x))


def project_params(P, cam, blur_eps=0.3, near=0.2, rest=None, sh_degree=0, depth_bt=None,
                   depth_zgrad=False):
    """Geometry + activations of the binned trainer (tools/m4_train_binned.py:194-202).

    `cam` is a dict with R_v[3,3], t_v[3], fx, fy, cx, cy.  Returns a dict with
    mu2d, conic, depth, keep, color_o[G,3], o_col[G] -- differentiable w.r.t. P (and `rest`,
    `depth_bt`).  With sh_degree > 0 and rest [G,15,3] the colour is the device step's
    view-dependent SH colour (oracle/sh.py: view_color); otherwise the DC colour.
    depth_bt = (beta, tau): the depth weight rho = sigmoid(beta (tau - depth)) multiplies the
    opacity (spike/arms.py:34-37; device step tools/resident_traced.py:333-337), with depth a
    constant of the gradient as in that step unless depth_zgrad (spike's dense autograd)."""
    means, quats, log_scales, color_dc, op = split_params(P)
    R = quat_to_rotmat(quats)
    cov = cov3d(torch.exp(log_scales), R)
    dt = P.dtype
    mu2d, conic, depth, keep = project_ewa(means, cov, cam["R_v"].to(dt), cam["t_v"].to(dt),
                                           cam["fx"], cam["fy"], cam["cx"], cam["cy"],
                                           blur_eps, near)
    if sh_degree > 0 and rest is not None:
        from . import sh
        color = sh.view_color(means, color_dc, rest, sh_degree, cam["R_v"].to(dt),
                              cam["t_v"].to(dt))
    else:
        color = color_from_dc(color_dc)
    keo = keep.to(dt) * torch.sigmoid(op)
    if depth_bt is not None:
        z = depth if depth_zgrad else depth.detach()
        keo = keo * torch.sigmoid(depth_bt[0] * (depth_bt[1] - z))
    return dict(mu2d=mu2d, conic=conic, depth=depth, keep=keep,
                color_o=keo[:, None] * color, o_col=keo)


def make_camera(H, W, eye, fov_deg=50.0, target=(0.0, 0.0, 0.0)):
    """Pinhole camera with horizontal field of view `fov_deg` (fx = fy = 0.5*W/tan(fov/2),
    as spike/synthetic.py:21), principal point at the image centre, looking at `target`."""
    R_v, t_v = look_at_opencv(eye, target)
    f = 0.5 * W / math.tan(math.radians(fov_deg) / 2.0)
    return dict(R_v=R_v, t_v=t_v, fx=f, fy=f, cx=W / 2.0, cy=H / 2.0, H=H, W=W)
