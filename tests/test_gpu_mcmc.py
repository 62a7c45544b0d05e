"""Fixed-count MCMC on the GPU vs the oracle (spike/mcmc.py): the regulariser gradient, the SGLD
step (Philox draws reproduced bit for bit by the oracle's integer restatement), the fused
geometry backward + Adam with both, the device relocation (targets, copies, opacity split,
moment reset, SH rest rows) and the MCMC training step, eager and graph-replayed."""
import math

import numpy as np
import pytest
import torch

from helpers import config_inputs, rel_l2
from oracle import mcmc as omc
from oracle import rng
from ttsplat import kernels
from ttsplat.step import TrainStep, lr_vector

pytestmark = pytest.mark.gpu


def _logit(p):
    return math.log(p / (1 - p))


def step_block(t):
    s = kernels.adam_state("cuda")
    s[0] = t
    return s


def _params(G=3000, dead_frac=0.1, seed=0):
    cfg, P, cam = config_inputs("c1_ref", G=G)
    P = P.clone()
    g = torch.Generator().manual_seed(seed)
    P[:, 13] = torch.logit(torch.rand(G, generator=g) * 0.9 + 0.05)
    dead = torch.rand(G, generator=g) < dead_frac
    P[dead, 13] = _logit(1e-3)
    return cfg, P, cam


def test_reg_grad():
    _, P, _ = _params()
    g = torch.zeros(P.shape[0], 14, device="cuda")
    kernels.mcmc_reg_grad(P.cuda(), g, 0.01, 0.02)
    assert rel_l2(g, omc.reg_grad(P.double(), 0.01, 0.02)) <= 1e-5


def test_sgld_noise_matches_oracle_draws():
    _, P, _ = _params()
    G = P.shape[0]
    lr = lr_vector(device="cuda")
    Pg = P.cuda()
    kernels.sgld_noise(Pg, lr, 500.0, step_block(7), seed=12345)
    eps = torch.tensor(rng.normals3(np.arange(G), 7, rng.TAG_SGLD, 12345))
    want = omc.sgld_noise(P.double(), float(lr[0]), 500.0, eps)
    got = Pg.cpu().double()[:, 0:3] - P.double()[:, 0:3]
    assert rel_l2(got, want) <= 1e-4
    assert torch.equal(Pg.cpu()[:, 3:], P[:, 3:])
    # gated: settled gaussians barely move, near-dead ones do
    o = torch.sigmoid(P[:, 13])
    d = got.norm(dim=1)
    assert float(d[o > 0.5].max()) < 1e-6 < float(d[o < 0.002].min())


def test_fused_mcmc_backward_adam_equals_separate_kernels():
    cfg, P, cam = _params(G=2000)
    from ttsplat.step import TrainStep
    tgt = torch.rand(cfg.H, cfg.W, 3)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    ts._view_backward(0)
    camb = ts.cams[0]
    lr = ts.lr
    # separate: reduce -> geometry bwd -> + regulariser -> Adam -> SGLD
    Pa, ma, va = ts.P.clone(), torch.zeros_like(ts.P), torch.zeros_like(ts.P)
    sa = step_block(0)
    kernels.adam_advance(sa)
    grad = kernels.geom_bwd(Pa, camb, kernels.slot_reduce(ts.gslot, ts.inv))
    kernels.mcmc_reg_grad(Pa, grad, 0.01, 0.02)
    kernels.adam(Pa, ma, va, grad, lr, sa)
    kernels.sgld_noise(Pa, lr, 300.0, sa, seed=9)
    # fused
    Pb, mb, vb = ts.P.clone(), torch.zeros_like(ts.P), torch.zeros_like(ts.P)
    sb = step_block(0)
    kernels.adam_advance(sb)
    gb = torch.empty_like(Pb)
    kernels.geom_bwd_adam(Pb, camb, ts.gslot, ts.inv, mb, vb, lr, sb, gparams=gb,
                          lambda_o=0.01, lambda_s=0.02, noise_lr=300.0, seed=9)
    assert rel_l2(gb, grad) <= 1e-6
    assert rel_l2(mb, ma) <= 1e-6 and rel_l2(vb, va) <= 1e-6
    assert rel_l2(Pb - ts.P, Pa - ts.P) <= 1e-5


def _oracle_relocate(P, m, v, t, seed, thr, offset, rest=None, rest_m=None, rest_v=None):
    o, dead, alive = omc.classify(P, thr)
    nd = dead.numel()
    if nd == 0 or alive.numel() == 0:
        return 0, None
    u = torch.tensor(rng.uniform1(np.arange(nd), t, rng.TAG_RELOC_PICK, seed))
    targets = omc.pick_targets(o, alive, u)
    offs = offset * torch.tensor(rng.normals3(np.arange(nd), t, rng.TAG_RELOC_OFFSET, seed))
    touched = omc.relocate(P, m, v, dead, targets, offs, rest, rest_m, rest_v)
    return nd, touched


@pytest.mark.parametrize("G,dead_frac", [(3000, 0.1), (70_000, 0.3), (257, 0.5)])
def test_relocate_matches_oracle(G, dead_frac):
    _, P, _ = _params(G=G, dead_frac=dead_frac, seed=G)
    m = torch.rand(G, 14) + 0.5
    v = torch.rand(G, 14) + 0.5
    Pg, mg, vg = P.cuda(), m.cuda(), v.cuda()
    moved = kernels.relocate(Pg, mg, vg, step_block(5), dead_thr=0.005, offset=0.01, seed=77)
    Pr, mr, vr = P.double(), m.double(), v.double()
    nd, touched = _oracle_relocate(Pr, mr, vr, 5, 77, 0.005, 0.01)
    assert int(moved) == nd > 0
    assert torch.equal(mg.cpu() == 0, mr == 0) and torch.equal(vg.cpu() == 0, vr == 0)
    assert float((Pg.cpu().double() - Pr).abs().max()) <= 1e-5
    # the opacity of every target is shared by it and its copies: the new total is the old
    # live total (dead mass recycled)
    o0 = torch.sigmoid(P.double()[:, 13])
    o1 = torch.sigmoid(Pg.cpu().double()[:, 13])
    assert abs(float(o1.sum() - o0[o0 >= 0.005].sum())) <= 1e-4 * G


def test_relocate_with_sh_rest_rows():
    G = 5000
    _, P, _ = _params(G=G, dead_frac=0.2, seed=3)
    g = torch.Generator().manual_seed(4)
    rest = torch.randn(G, 15, 3, generator=g)
    rm = torch.rand(G, 15, 3, generator=g) + 0.5
    rv = torch.rand(G, 15, 3, generator=g) + 0.5
    m, v = torch.ones(G, 14), torch.ones(G, 14)
    Pg, mg, vg = P.cuda(), m.cuda(), v.cuda()
    sg, smg, svg = (kernels.sh_rest_layout(t.cuda()) for t in (rest, rm, rv))
    kernels.relocate(Pg, mg, vg, step_block(2), seed=5, sh_rest=sg, sh_m=smg, sh_v=svg)
    Pr, mr, vr = P.double(), m.double(), v.double()
    rr, rmr, rvr = rest.double(), rm.double(), rv.double()
    _oracle_relocate(Pr, mr, vr, 2, 5, 0.005, 0.005, rr, rmr, rvr)
    assert torch.equal(kernels.sh_rest_model(sg).cpu().double(), rr)
    assert torch.equal(kernels.sh_rest_model(smg).cpu() == 0, rmr == 0)
    assert torch.equal(kernels.sh_rest_model(svg).cpu() == 0, rvr == 0)
    assert float((Pg.cpu().double() - Pr).abs().max()) <= 1e-5


def test_relocate_nothing_to_move():
    _, P, _ = _params(G=1000, dead_frac=0.0)
    m, v = torch.ones(1000, 14, device="cuda"), torch.ones(1000, 14, device="cuda")
    Pg = P.cuda()
    moved = kernels.relocate(Pg, m, v, step_block(1))
    assert int(moved) == 0 and torch.equal(Pg.cpu(), P) and float(m.min()) == 1.0
    P[:, 13] = _logit(1e-4)                                    # everything dead: no live target
    Pg = P.cuda()
    moved = kernels.relocate(Pg, m, v, step_block(1))
    assert int(moved) == 0 and torch.equal(Pg.cpu(), P) and float(m.min()) == 1.0


MC = dict(lambda_o=0.01, lambda_s=0.01, noise_lr=50.0, relocate_every=3, seed=21)


def _target(cfg, cam):
    P1 = cfg.params(seed=1)
    ts = TrainStep(P1, [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S, k=cfg.k)
    img = ts.forward(0).clone()
    torch.cuda.synchronize()
    return img


def test_mcmc_step_graph_replay_matches_eager():
    cfg, P, cam = _params(G=2000, dead_frac=0.15)
    tgt = _target(cfg, cam)
    eager = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, mcmc=MC)
    graph = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, mcmc=MC)
    graph.capture()
    for _ in range(8):
        eager.step(0)
        graph.step(0)
        torch.cuda.synchronize()
    assert int(eager.relocations) == int(graph.relocations) > 0
    assert rel_l2(graph.P - P.cuda(), eager.P - P.cuda()) <= 1e-4
    assert abs(float(graph.loss()) - float(eager.loss())) <= 1e-5


def test_mcmc_training_reduces_loss_and_recycles_dead_slots():
    cfg, P, cam = _params(G=2000, dead_frac=0.15)
    tgt = _target(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k,
                   mcmc=dict(MC, relocate_every=30))
    ts.capture()
    ts.step(0)
    l0 = float(ts.loss())
    for _ in range(120):
        ts.step(0)
    assert float(ts.loss()) < 0.8 * l0
    assert int(ts.relocations) > 0
    o = torch.sigmoid(ts.P[:, 13])
    assert int((o < 0.005).sum()) < int((torch.sigmoid(P[:, 13]) < 0.005).sum())
