"""Write tests/golden/c2_oracle_trajectory.json: the oracle's own 3000-step training run of the
G = 2000, 128 x 128 workload (fp32 CPU restatement of the reference path, one camera at (0,0,3),
bins recomputed every step, Adam lr 1e-3 / means 1.6e-4, 0.8 L1 + 0.2 (1 - SSIM)), the target
being the oracle's render of the seed-1 gaussian set.  Records the loss every 100 steps.

Run from the repository root:  python tests/golden/make_c2_trajectory.py  (about 2 minutes)."""
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "tt-splat_amd")]

import torch  # noqa: E402

from oracle import binning as obin  # noqa: E402
from oracle import pipeline as opipe  # noqa: E402
from oracle import splat as osplat  # noqa: E402
from ttsplat import scenes  # noqa: E402

STEPS = 3000


def main():
    cfg = scenes.CONFIGS["c2"]
    cam = cfg.cameras()[0].as_dict()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    P = cfg.params(seed=0)
    with torch.no_grad():
        tgt = osplat.render_binned(cfg.params(seed=1), cam, tmap, K=cfg.K, k=cfg.k)
    m, v = torch.zeros_like(P), torch.zeros_like(P)
    lr = torch.full((14,), 1e-3)
    lr[:3] = 1.6e-4
    losses = {}
    t0 = time.time()
    for t in range(1, STEPS + 1):
        _, L, _ = opipe.train_step(P, m, v, t, cam, tmap, tgt, lr, K=cfg.K, k=cfg.k)
        if t == 1 or t % 100 == 0:
            losses[t] = float(L)
    out = dict(workload="G=2000 uniform gaussians, 128x128, K=128, S=16, k=4, camera (0,0,3), "
                        "fp32 oracle, target = oracle render of seed 1",
               steps=STEPS, loss_at=losses, final_loss=losses[STEPS],
               seconds=time.time() - t0, threads=torch.get_num_threads())
    path = os.path.join(ROOT, "tests", "golden", "c2_oracle_trajectory.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {path}: final loss {losses[STEPS]:.6f} after {STEPS} steps")


if __name__ == "__main__":
    main()
