"""Shared test inputs: seeded configurations, oracle camera dicts, comparison metrics."""
import torch

from ttsplat import scenes
from ttsplat.camera import Camera


def cam_dict(cam: Camera):
    return cam.as_dict()


def rel_l2(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp(min=1e-30))


def max_abs(a, b):
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())


def config_inputs(name, seed=0, cam_index=0, G=None):
    """(config, params[G,14] CPU, camera) for a named configuration (G optionally reduced)."""
    cfg = scenes.CONFIGS[name]
    if G is not None:
        cfg = scenes.Config(**{**cfg.__dict__, "G": G, "span": cfg.span})
    P = cfg.params(seed)
    cam = cfg.cameras()[cam_index]
    return cfg, P, cam


def bins_equal_report(idx_a, valid_a, idx_b, valid_b):
    """Number of tiles whose (idx, valid) rows differ."""
    ia, va = idx_a.cpu().long(), valid_a.cpu().bool()
    ib, vb = idx_b.cpu().long(), valid_b.cpu().bool()
    diff = (ia != ib).any(1) | (va != vb).any(1)
    return int(diff.sum()), torch.nonzero(diff).flatten()
