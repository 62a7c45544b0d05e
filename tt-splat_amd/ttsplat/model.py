"""GPU-resident gaussian set in the [G,14] layout of the device trainer.

The reference model (spike/model.py:16-95) keeps separate tensors; the device trainer keeps the
14 per-gaussian columns mx,my,mz, qw,qx,qy,qz, lx,ly,lz, cr,cg,cb, op in one block
(tools/resident_traced.py:91, :233-235).  `GaussianModel` holds that block and exposes the
reference attribute names as views, so code written against spike.model reads it unchanged.
"""
import math

import torch

C0 = 0.28209479177387814   # SH degree-0 constant (spike/sh.py:9)

PN = ("mx", "my", "mz", "qw", "qx", "qy", "qz", "lx", "ly", "lz", "cr", "cg", "cb", "op")


class GaussianModel:
    """depth_beta, depth_tau: the global depth-weight scalars of arm B; softz_beta: the gate
    sharpness of arm SZ (spike/model.py:48-50 defaults 1.0, 3.0 and 4.0).  color_rest: the SH
    rest coefficients [G,15,3] of view-dependent colour (spike/model.py:45), or None (DC colour
    only; the reference keeps a zero tensor there)."""

    def __init__(self, params, w_b_raw=-3.0, c_b=(1.0, 1.0, 1.0), depth_beta=1.0, depth_tau=3.0,
                 softz_beta=4.0, color_rest=None):
        if params.dim() != 2 or params.shape[1] != 14:
            raise ValueError(f"params must be [G,14], got {tuple(params.shape)}")
        self.params = params.float().contiguous()
        dev = self.params.device
        self.w_b_raw = torch.tensor(float(w_b_raw), device=dev)
        self.c_b = torch.as_tensor(c_b, dtype=torch.float32, device=dev)
        self.depth_beta = torch.tensor(float(depth_beta), device=dev)
        self.depth_tau = torch.tensor(float(depth_tau), device=dev)
        self.softz_beta = torch.tensor(float(softz_beta), device=dev)
        self.color_rest = None
        if color_rest is not None:
            cr = torch.as_tensor(color_rest, dtype=torch.float32, device=dev)
            if tuple(cr.shape) != (self.params.shape[0], 15, 3):
                raise ValueError(f"color_rest must be [G,15,3], got {tuple(cr.shape)}")
            self.color_rest = cr.contiguous()

    @classmethod
    def from_reference(cls, model, device="cuda"):
        """Pack a spike-style model (separate tensors) into the [G,14] block."""
        P = torch.cat([model.means3d.detach(), model.quats.detach(), model.log_scales.detach(),
                       model.color_dc.detach(), model.opacity_raw.detach().reshape(-1, 1)], 1)
        rest = getattr(model, "color_rest", None)
        return cls(P.to(device), float(model.w_b_raw), model.c_b.detach().cpu(),
                   color_rest=None if rest is None else rest.detach().to(device))

    @property
    def G(self):
        return self.params.shape[0]

    @property
    def means3d(self):
        return self.params[:, 0:3]

    @property
    def quats(self):
        return self.params[:, 3:7]

    @property
    def log_scales(self):
        return self.params[:, 7:10]

    @property
    def color_dc(self):
        return self.params[:, 10:13]

    @property
    def opacity_raw(self):
        return self.params[:, 13]


@torch.no_grad()
def init_from_points(xyz, rgb, G, seed=0, base=None):
    """[G,14] parameters initialised from a sparse point cloud (spike/model.py:53-80): G points
    drawn without replacement (or all points plus jittered copies when there are fewer), a
    common log-scale from the median nearest-neighbour distance over up to 4000 of them, and
    colour_dc the inverse DC SH of the point colours.  Quaternions and opacity come from
    `base` [G,14] when given, else the identity rotation and opacity 0.1."""
    xyz = torch.as_tensor(xyz, dtype=torch.float32)
    rgb = torch.as_tensor(rgb, dtype=torch.float32)
    g = torch.Generator().manual_seed(seed)
    n = xyz.shape[0]
    if n >= G:
        sel = torch.randperm(n, generator=g)[:G]
        pts, cols = xyz[sel], rgb[sel]
    else:
        extra = G - n
        j = torch.randint(0, n, (extra,), generator=g)
        span = (xyz.max(0).values - xyz.min(0).values).norm() * 0.01
        pts = torch.cat([xyz, xyz[j] + torch.randn(extra, 3, generator=g) * span], 0)
        cols = torch.cat([rgb, rgb[j]], 0)
    sub = pts[torch.randperm(G, generator=g)[:min(G, 4000)]]
    d = torch.cdist(sub, sub)
    d.fill_diagonal_(float("inf"))
    nn = d.min(1).values.median().clamp(min=1e-4)
    P = torch.zeros(G, 14) if base is None else torch.as_tensor(base, dtype=torch.float32).clone()
    if base is None:
        P[:, 3] = 1.0
        P[:, 13] = math.log(0.1 / 0.9)
    P[:, 0:3] = pts
    P[:, 7:10] = float(torch.log(nn))
    P[:, 10:13] = (cols - 0.5) / C0
    return P
