"""Write golden binning vectors with the reference's own assign_bins.

Only the reference's assign_bins (tools/m4_train_binned.py:75-127) is run: its tie order
below 32768 pairs (torch's non-stable argsort) is pinned by nothing else.  Its module imports
ttnn (:29) and spike.metrics -> pytorch_msssim (:31, spike/metrics.py:3) at top level; neither
is installed here nor used by assign_bins, so both are registered as empty modules before the
import.  Run in the build container only (the reference tree is not on the GPU machine):

    python tests/golden/make_bins_fixtures.py

Inputs are mu2d/keep from the oracle geometry on the seeded configurations (plus an
edge-case set); outputs are the reference's idx (stored int32: ids < 2^31) and valid.
Large outputs are stored as a SHA-256 digest of the reference's int64/bool bytes plus the
per-tile kept counts.
"""
import hashlib
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path[:0] = [REPO, os.path.join(REPO, "tt-splat_amd"), os.path.dirname(HERE)]

from oracle import geometry as ogeo  # noqa: E402
from ttsplat import scenes  # noqa: E402


def reference_assign_bins():
    for name in ("ttnn", "pytorch_msssim"):
        mod = types.ModuleType(name)
        if name == "pytorch_msssim":
            mod.ssim = None
        sys.modules.setdefault(name, mod)
    sys.path[:0] = [REF, os.path.join(REF, "tools")]
    import m4_train_binned as ref  # noqa: E402
    return ref


def digest(idx64, valid):
    h = hashlib.sha256()
    h.update(np.ascontiguousarray(idx64.numpy().astype("<i8")).tobytes())
    h.update(np.ascontiguousarray(valid.numpy().astype(np.uint8)).tobytes())
    return h.hexdigest()


def edge_inputs(G=3000, H=96, W=160, seed=5):
    g = torch.Generator().manual_seed(seed)
    mu = torch.empty(G, 2)
    mu[:, 0] = torch.rand(G, generator=g) * (W + 200) - 100
    mu[:, 1] = torch.rand(G, generator=g) * (H + 200) - 100
    n = G // 8
    mu[:n] = torch.tensor([37.25, 61.5])
    mu[n:2 * n, 0] = torch.randint(0, W // 16 + 1, (n,), generator=g).float() * 16
    mu[n:2 * n, 1] = torch.randint(0, H // 16 + 1, (n,), generator=g).float() * 16
    keep = torch.rand(G, generator=g) > 0.1
    return mu, keep, H, W


def main():
    ref = reference_assign_bins()
    out = {}
    cases = []
    for name in ("c1_ref", "c3", "c4"):
        cfg = scenes.CONFIGS[name]
        P = cfg.params(0)
        cam = cfg.cameras()[0]
        pr = ogeo.project_params(P, cam.as_dict())
        cases.append((name, pr["mu2d"].detach().float(), pr["keep"], cfg.H, cfg.W, cfg.K))
    mu, keep, H, W = edge_inputs()
    cases.append(("edge", mu, keep, H, W, 64))
    for name, mu2d, keep, H, W, K in cases:
        tmap = ref.TileMap(H, W)
        idx, valid = ref.assign_bins(mu2d, keep, tmap, 1, K)
        out[f"{name}_mu2d"] = mu2d.numpy().astype(np.float32)
        out[f"{name}_keep"] = keep.numpy().astype(np.bool_)
        out[f"{name}_shape"] = np.array([H, W, K], dtype=np.int32)
        out[f"{name}_count"] = valid.sum(1).numpy().astype(np.int32)
        out[f"{name}_sha256"] = np.array(digest(idx, valid))
        if name in ("c1_ref", "edge", "c3"):
            out[f"{name}_idx"] = idx.numpy().astype(np.int32)
            out[f"{name}_valid"] = valid.numpy().astype(np.bool_)
        print(f"{name}: T={tmap.T} kept={int(valid.sum())}")
    path = os.path.join(HERE, "bins_reference.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main()
