"""Gaussian geometry under the reference names (spike/geometry.py:10-57).

`project_params` is the hot path's projection: one HIP kernel (tts_geom_fwd) from the [G,14]
parameter block to the per-gaussian record (mean, conic, depth, colour x opacity, opacity).
`quat_to_rotmat`, `cov3d` and `project_ewa` are the reference's tensor formulas, kept so code
written against spike.geometry runs unchanged (GPU tensors only); the kernels compute the same
quantities in registers.
"""
import torch

from . import kernels
from .forward import _gpu


def project_params(params, cam, blur_eps=kernels.BLUR, near=kernels.NEAR):
    """[G,14] parameters -> dict(mu2d [G,2], conic [G,3], depth [G], keep [G] bool,
    color_o [G,3], o_col [G], opacity [G]) through tts_geom_fwd."""
    proj, keep = kernels.geom_fwd(params.detach().float().contiguous(),
                                  cam.device_block(params.device), near=near, blur=blur_eps)
    return dict(mu2d=proj[:, 0:2], conic=proj[:, 2:5], depth=proj[:, 5], keep=keep.bool(),
                color_o=proj[:, 6:9], o_col=proj[:, 9], opacity=proj[:, 10], proj=proj)


def quat_to_rotmat(quats):
    """[...,4] wxyz (normalised here) -> R [...,3,3]."""
    _gpu(quats)
    q = quats / quats.norm(dim=-1, keepdim=True).clamp(min=1e-12)
    w, x, y, z = q.unbind(-1)
    return torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y),
    ], dim=-1).reshape(*q.shape[:-1], 3, 3)


def cov3d(scales, R):
    """R diag(scales^2) R^T."""
    _gpu(scales, R)
    return (R * (scales * scales)[..., None, :]) @ R.transpose(-1, -2)


def project_ewa(means3d, cov3d_w, R_v, t_v, fx, fy, cx, cy, blur_eps=0.3, near=0.2):
    """EWA projection -> (mu2d [G,2], conic_abc [G,3], depth [G], keep [G])."""
    _gpu(means3d, cov3d_w)
    R_v = torch.as_tensor(R_v, dtype=means3d.dtype, device=means3d.device)
    t_v = torch.as_tensor(t_v, dtype=means3d.dtype, device=means3d.device)
    mc = means3d @ R_v.T + t_v
    depth = mc[:, 2]
    keep = depth > near
    z = depth.clamp(min=near)
    mu2d = torch.stack([fx * mc[:, 0] / z + cx, fy * mc[:, 1] / z + cy], dim=-1)
    Sc = R_v @ cov3d_w @ R_v.T
    zero = torch.zeros_like(z)
    J = torch.stack([torch.stack([fx / z, zero, -fx * mc[:, 0] / (z * z)], -1),
                     torch.stack([zero, fy / z, -fy * mc[:, 1] / (z * z)], -1)], -2)
    S2 = J @ Sc @ J.transpose(-1, -2)
    s00, s01, s11 = S2[:, 0, 0] + blur_eps, S2[:, 0, 1], S2[:, 1, 1] + blur_eps
    det = (s00 * s11 - s01 * s01).clamp(min=1e-12)
    return mu2d, torch.stack([s11 / det, -s01 / det, s00 / det], -1), depth, keep
