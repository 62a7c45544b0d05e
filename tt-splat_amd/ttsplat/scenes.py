"""Seeded synthetic workloads (the five benchmark configurations).

Draw order with torch.Generator('cpu').manual_seed(seed): means, log-scales, quaternions,
opacity, rgb.  Parameters come back as the [G,14] block (columns mx,my,mz, qw,qx,qy,qz,
lx,ly,lz, cr,cg,cb, op; tools/resident_traced.py:91) on the CPU.

  means      uniform in [-1,1]^3, or a mixture of 20 isotropic clusters (sigma 0.2) with
             centres uniform in [-2,2]^3 and uniform assignment
  scales     log-uniform in [lo, hi] per axis
  quats      normalised N(0,1)^4, [w,x,y,z]
  opacity    o ~ U[0.05, 0.95] stored as logit(o)
  colour     rgb ~ U[0,1] stored as SH-DC: (rgb - 0.5)/C0 (spike/sh.py:9)
  w_b_raw = -3, c_b = (1,1,1) (spike/model.py:47,51)
  cameras    pinhole, fov 50 deg, looking at the origin from distance 3; the single-view
             configurations sit at (0,0,3), multi-view ones on a radius-3 sphere
             (eye = 3 * normalise(N(0,1)^3), seed 2, rejecting |y| > 0.95)
"""
import math
from dataclasses import dataclass, field

import torch

from .camera import pinhole

C0 = 0.28209479177387814


def make_params(G, seed, means="uniform", scale_range=(0.01, 0.1), clusters=20,
                cluster_sigma=0.2, cluster_extent=2.0):
    g = torch.Generator("cpu").manual_seed(int(seed))
    if means == "uniform":
        m = torch.rand(G, 3, generator=g) * 2.0 - 1.0
    elif means == "clustered":
        centres = torch.rand(clusters, 3, generator=g) * (2.0 * cluster_extent) - cluster_extent
        assign = torch.randint(0, clusters, (G,), generator=g)
        m = centres[assign] + cluster_sigma * torch.randn(G, 3, generator=g)
    else:
        raise ValueError(f"unknown means distribution {means!r}")
    lo, hi = math.log(scale_range[0]), math.log(scale_range[1])
    ls = lo + torch.rand(G, 3, generator=g) * (hi - lo)
    q = torch.randn(G, 4, generator=g)
    q = q / q.norm(dim=1, keepdim=True)
    o = 0.05 + 0.9 * torch.rand(G, generator=g)
    op = torch.log(o / (1.0 - o))
    rgb = torch.rand(G, 3, generator=g)
    dc = (rgb - 0.5) / C0
    return torch.cat([m, q, ls, dc, op[:, None]], dim=1).contiguous()


def orbit_eyes(n, seed=2, radius=3.0, max_abs_y=0.95):
    """n eye positions on a sphere of `radius`, |normalised y| <= max_abs_y."""
    g = torch.Generator("cpu").manual_seed(int(seed))
    eyes = []
    while len(eyes) < n:
        v = torch.randn(3, generator=g)
        v = v / v.norm()
        if abs(float(v[1])) > max_abs_y:
            continue
        eyes.append((radius * v).tolist())
    return eyes


@dataclass
class Config:
    name: str
    G: int
    H: int
    W: int
    K: int = 128
    S: int = 16
    k: float = 4.0
    means: str = "uniform"
    scale_range: tuple = (0.01, 0.1)
    n_cams: int = 1
    dtype: str = "fp32"
    notes: str = ""
    span: int = field(default=0)

    def __post_init__(self):
        if not self.span:
            self.span = 2048 if self.S == 16 else 8192

    def params(self, seed=0):
        return make_params(self.G, seed, self.means, self.scale_range)

    def cameras(self):
        if self.n_cams == 1:
            return [pinhole(self.H, self.W, (0.0, 0.0, 3.0))]
        return [pinhole(self.H, self.W, e) for e in orbit_eyes(self.n_cams)]


CONFIGS = {
    # forward render, reference CPU path: G=2000, 128x128, fp32 (k=9 and 32x32 tiles as
    # configured; k=4 / 16x16 tiles are the reference's own constants and the parity mode)
    "c1": Config("c1", 2000, 128, 128, K=128, S=32, k=9.0),
    "c1_ref": Config("c1_ref", 2000, 128, 128, K=128, S=16, k=4.0),
    # training step, G=2000, 128x128, bf16 render operands, fp32 Adam
    "c2": Config("c2", 2000, 128, 128, K=128, S=16, k=4.0, dtype="bf16"),
    # training step, G=10k, 800x800, 8 orbit cameras
    "c3": Config("c3", 10000, 800, 800, K=128, S=16, k=4.0, n_cams=8),
    # forward + training step, G=100k clustered, 1264x832, 8 orbit cameras
    "c4": Config("c4", 100000, 832, 1264, K=128, S=16, k=4.0, means="clustered", n_cams=8),
    # stress: G=1M clustered, scales log-U[0.002,0.05], 1920x1080 cropped to 1920x1072, K=256,
    # 64 cameras per batch
    "c5": Config("c5", 1000000, 1072, 1920, K=256, S=16, k=4.0, means="clustered",
                 scale_range=(0.002, 0.05), n_cams=64, dtype="bf16",
                 notes="1080 rows cropped to 1072 (whole 16-px tiles)"),
}
