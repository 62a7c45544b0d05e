"""Scene IO end to end on the GPU: views rendered by the HIP path are written as a NeRF-synthetic
dataset (PNG frames + OpenGL camera-to-world poses) and read back with the loader; the trained
set survives a .ply round trip render for render."""
import json
import os

import numpy as np
import pytest
import torch
from PIL import Image

from helpers import config_inputs
from ttsplat import io, kernels, scenes
from ttsplat.camera import pinhole
from ttsplat.step import TrainStep

pytestmark = pytest.mark.gpu


def _c2w_opengl(cam):
    """Inverse of camera.opengl_c2w_to_opencv_w2c."""
    flip = torch.diag(torch.tensor([1.0, -1.0, -1.0], dtype=torch.float64))
    R_v, t_v = cam.R_v.double(), cam.t_v.double()
    c2w = torch.eye(4, dtype=torch.float64)
    c2w[:3, :3] = R_v.T @ flip
    c2w[:3, 3] = -R_v.T @ t_v
    return c2w


def test_blender_round_trip_and_training(tmp_path):
    cfg, P, _ = config_inputs("c1_ref")
    H = W = 128
    cams = [pinhole(H, W, e) for e in scenes.orbit_eyes(3)]
    maker = TrainStep(cfg.params(seed=1), cams, [torch.zeros(H, W, 3)] * 3, K=cfg.K, S=16,
                      k=cfg.k)
    os.makedirs(tmp_path / "train")
    frames, rendered = [], []
    angle_x = 2 * np.arctan(0.5 * W / cams[0].fx)
    for i, c in enumerate(cams):
        img = maker.forward(i).clamp(0, 1).cpu()
        rendered.append(img)
        rgba = np.concatenate([np.round(img.numpy() * 255), np.full((H, W, 1), 255)], -1)
        Image.fromarray(rgba.astype(np.uint8), mode="RGBA").save(tmp_path / "train" / f"r_{i}.png")
        frames.append({"file_path": f"./train/r_{i}", "transform_matrix": _c2w_opengl(c).tolist()})
    with open(tmp_path / "transforms_train.json", "w") as f:
        json.dump({"camera_angle_x": float(angle_x), "frames": frames}, f)
    lcams, limgs = io.load_blender(str(tmp_path), "train", res=None)
    for c, lc, img, limg in zip(cams, lcams, rendered, limgs):
        assert torch.allclose(lc.R_v, c.R_v, atol=1e-5) and torch.allclose(lc.t_v, c.t_v, atol=1e-5)
        assert abs(lc.fx - c.fx) < 1e-3 and (lc.H, lc.W) == (H, W)
        assert float((limg - img).abs().max()) <= 0.5 / 255 + 1e-6
    ts = TrainStep(P, lcams, limgs, K=cfg.K, S=16, k=cfg.k)
    ts.capture()
    ts.step(0)
    l0 = float(ts.loss())
    for i in range(150):
        ts.step(i % 3)
    assert float(ts.loss()) < 0.8 * l0


def test_ply_round_trip_renders_identically(tmp_path):
    cfg, P, cam = config_inputs("c1_ref")
    rest = torch.randn(cfg.G, 15, 3, generator=torch.Generator().manual_seed(2)) * 0.2
    a = TrainStep(P, [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S, k=cfg.k,
                  sh_degree=3, sh_rest=rest)
    img_a = a.forward(0).clone()
    io.save_ply(tmp_path / "m.ply", a.P, color_rest=a.color_rest)
    Q, r = io.read_ply(tmp_path / "m.ply")
    b = TrainStep(Q, [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S, k=cfg.k,
                  sh_degree=3, sh_rest=r)
    img_b = b.forward(0)
    assert float((img_a - img_b).abs().max()) <= 1e-5
    assert torch.equal(a.idx, b.idx) and torch.equal(a.valid, b.valid)
