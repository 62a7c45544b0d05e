"""Splat forward and backward on slot records (tts_splat_fwd_rec, tts_splat_fwd_mx_rec,
tts_splat_bwd_rec; the records written by tts_geom_fwd_assign_bins) against the same kernels on
proj, idx and valid in the same tile order: image, den, per-slot gradients and per-tile dL/dw_b
equal bit for bit, including slot budgets past 256 (the forwards' second staging pass) and a
tile poisoned by a NaN record."""
import pytest
import torch

from helpers import config_inputs
from ttsplat import kernels

pytestmark = pytest.mark.gpu


def binned(name, K=None):
    cfg, P, cam = config_inputs(name)
    K = cfg.K if K is None else K
    T = (cfg.H // cfg.S) * (cfg.W // cfg.S)
    order = torch.empty(T, dtype=torch.int32, device="cuda")
    rec = torch.empty(T, K, 12, device="cuda")
    pos = torch.empty(T, dtype=torch.int32, device="cuda")
    proj, keep, idx, valid, count, _ = kernels.geom_fwd_assign_bins(
        P.cuda(), cam.device_block("cuda"), cfg.H, cfg.W, cfg.S, K, cfg.span, order=order,
        slot_rec=rec, pos_count=pos)
    bg = torch.tensor([float(torch.nn.functional.softplus(torch.tensor(-3.0))), 1.0, 1.0, 1.0],
                      device="cuda")
    return cfg, K, T, proj, idx, valid, order, rec, pos, bg


def same(a, b):
    return bool(((a == b) | (a.isnan() & b.isnan())).all())


def both_ways(cfg, K, T, proj, idx, valid, order, rec, pos, bg):
    gen = torch.Generator(device="cuda").manual_seed(3)
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, order=order)
    img2, den2 = kernels.splat_fwd_rec(rec, pos, order, bg, cfg.H, cfg.W, cfg.S, cfg.k)
    gimg = torch.randn(cfg.H, cfg.W, 3, device="cuda", generator=gen)
    g1, g2 = torch.zeros(T, K, 9, device="cuda"), torch.zeros(T, K, 9, device="cuda")
    w1, w2 = torch.zeros(T, device="cuda"), torch.zeros(T, device="cuda")
    kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, img, den, gimg, g1, w1,
                      order=order)
    kernels.splat_bwd_rec(rec, pos, order, bg, cfg.H, cfg.W, cfg.S, cfg.k, img, den, gimg, g2,
                          w2)
    torch.cuda.synchronize()
    return (img, den, g1, w1), (img2, den2, g2, w2)


@pytest.mark.parametrize("name,K", [("c1_ref", 1), ("c1_ref", 128), ("c3", 128), ("c4", 128),
                                    ("c4", 300)])
def test_splat_on_records_equals_splat_on_bins(name, K):
    args = binned(name, K)
    print(f"[rec] {name} K={args[1]}", flush=True)
    (img, den, g1, w1), (img2, den2, g2, w2) = both_ways(*args)
    valid = args[5].bool()
    assert torch.equal(img, img2) and torch.equal(den, den2)
    assert torch.equal(g1[valid], g2[valid])
    assert torch.equal(w1, w2)


@pytest.mark.parametrize("name,K,bf16", [("c1_ref", 128, True), ("c3", 128, True),
                                         ("c4", 128, False), ("c4", 300, True)])
def test_matrix_core_forward_on_records(name, K, bf16):
    cfg, K, T, proj, idx, valid, order, rec, pos, bg = binned(name, K)
    print(f"[rec mx] {name} K={K} bf16={bf16}", flush=True)
    img, den = kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k,
                                    order=order, bf16=bf16)
    img2, den2 = kernels.splat_fwd_mx_rec(rec, pos, order, bg, cfg.H, cfg.W, cfg.S, cfg.k,
                                          bf16=bf16)
    torch.cuda.synchronize()
    assert torch.equal(img, img2) and torch.equal(den, den2)


def test_splat_on_records_nan_tile():
    cfg, K, T, proj, idx, valid, order, rec, pos, bg = binned("c1_ref")
    # the first kept slot of the heaviest tile: its gaussian's conic a becomes NaN in proj and in
    # the record, so both forms write that tile (and every tile holding the gaussian) as NaN
    g = int(idx[int(order[0]), 0])
    proj[g, 2] = float("nan")
    rec[0, 0, 2] = float("nan")
    ol = order.long()
    hold = (idx.long()[ol] == g) & valid.bool()[ol]      # positions whose tile keeps g
    rec[hold] = proj[g]
    (img, den, g1, w1), (img2, den2, g2, w2) = both_ways(cfg, K, T, proj, idx, valid, order,
                                                        rec, pos, bg)
    assert bool(img.isnan().any())
    assert same(img, img2) and same(den, den2)
    v = valid.bool()
    assert same(g1[v], g2[v]) and same(w1, w2)


def test_render_only_forward_equals_training_forward():
    """TrainStep.forward(grads=False) (binning without the inverse table, no den) renders the
    same image as the training step's forward and leaves den as that forward wrote it."""
    from ttsplat.step import TrainStep
    from helpers import config_inputs as ci_
    cfg, P, cam = ci_("c3")
    ts = TrainStep(P, [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S, k=cfg.k)
    img = ts.forward(0).clone()
    den = ts.den.clone()
    img2 = ts.forward(0, grads=False).clone()
    torch.cuda.synchronize()
    assert torch.equal(img, img2) and torch.equal(den, ts.den)
