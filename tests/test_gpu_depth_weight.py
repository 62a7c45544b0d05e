"""The depth-weight occlusion lever on the GPU vs the oracle (spike/arms.py:34-37; device step
tools/resident_traced.py:333-337,418-426,503-512): geometry forward/backward with rho on the
opacity (per-gaussian dL/d(beta, tau), the depth gradient off as in the device step or on as in
spike's autograd), the device reduction + Adam of (beta, tau), the training step with the lever
(eager, batched, graph-replayed), and the dense render's arm "B" with fit()."""
import pytest
import torch

from helpers import cam_dict, config_inputs, max_abs, rel_l2
from oracle import adam as oadam
from oracle import binning as obin
from oracle import geometry as ogeo
from oracle import pipeline as opipe
from oracle import splat as osplat
from ttsplat import kernels
from ttsplat import render as trender
from ttsplat import train as ttrain
from ttsplat.model import GaussianModel
from ttsplat.step import TrainStep, lr_vector

pytestmark = pytest.mark.gpu

BT = (1.7, 2.9)


@pytest.mark.parametrize("name", ["c1_ref", "c4"])
def test_geom_fwd_depth_weight(name):
    cfg, P, cam = config_inputs(name)
    bt = torch.tensor(BT, device="cuda")
    proj, keep = kernels.geom_fwd(P.cuda(), cam.device_block("cuda"), depth_bt=bt)
    ref = ogeo.project_params(P.double(), cam_dict(cam), depth_bt=torch.tensor(BT).double())
    assert torch.equal(keep.cpu().bool(), ref["keep"])
    assert max_abs(proj[:, 9], ref["o_col"]) <= 1e-6
    assert max_abs(proj[:, 6:9], ref["color_o"]) <= 1e-6
    plain = ogeo.project_params(P.double(), cam_dict(cam))
    assert max_abs(plain["o_col"], ref["o_col"]) > 1e-2        # the lever changes the opacity


@pytest.mark.parametrize("zgrad", [False, True])
def test_geom_bwd_depth_weight(zgrad):
    cfg, P, cam = config_inputs("c1_ref")
    g = torch.Generator().manual_seed(11)
    grad9 = torch.randn(cfg.G, 9, generator=g)
    bt = torch.tensor(BT, device="cuda")
    gP, _, gdw = kernels.geom_bwd(P.cuda(), cam.device_block("cuda"), grad9.cuda(), depth_bt=bt,
                                  depth_zgrad=zgrad)
    Pr = P.double().clone().requires_grad_(True)
    btr = torch.tensor(BT, dtype=torch.float64, requires_grad=True)
    ref = ogeo.project_params(Pr, cam_dict(cam), depth_bt=btr, depth_zgrad=zgrad)
    out = torch.cat([ref["conic"], ref["mu2d"], ref["color_o"], ref["o_col"][:, None]], 1)
    (out * grad9.double()).sum().backward()
    for sl in (slice(0, 3), slice(3, 7), slice(7, 10), slice(10, 13), slice(13, 14)):
        assert rel_l2(gP.cpu()[:, sl], Pr.grad[:, sl]) <= 1e-3, sl
    assert rel_l2(gdw.sum(0), btr.grad) <= 1e-4


def test_depth_weight_adam_reduces_and_steps():
    G = 100_003
    g = torch.Generator().manual_seed(3)
    gdw = torch.randn(G, 2, generator=g)
    bt = torch.tensor([1.2, 3.4], device="cuda")
    st = torch.zeros(4, device="cuda")
    lr1 = torch.tensor([0.02], device="cuda")
    step = kernels.adam_state("cuda")
    kernels.adam_advance(step)
    kernels.depth_weight_adam(gdw.cuda(), bt, st, lr1, step)
    tot = gdw.double().sum(0)
    p, m, v = torch.tensor([1.2, 3.4], dtype=torch.float64), torch.zeros(2, dtype=torch.float64), \
        torch.zeros(2, dtype=torch.float64)
    oadam.adam_step(p, m, v, tot, torch.tensor(0.02, dtype=torch.float64), 1)
    assert max_abs(bt, p) <= 1e-6
    # fp32 (1 - b2) differs from the float64 oracle's by 1.3e-5 relative
    assert rel_l2(st[:2], m) <= 1e-5 and rel_l2(st[2:], v) <= 1e-4


def _target(cfg, cam, **kw):
    ts = TrainStep(cfg.params(seed=1), [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S,
                   k=cfg.k, **kw)
    img = ts.forward(0).clone()
    torch.cuda.synchronize()
    return img


def test_train_step_with_depth_weight_matches_oracle():
    cfg, P, cam = config_inputs("c1_ref")
    tgt = _target(cfg, cam)
    dwo = dict(beta0=BT[0], tau0=BT[1], lr_bt=0.02)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, depth_weight=dwo)
    ts.enqueue(0)
    torch.cuda.synchronize()
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    img, L, g, ex = opipe.render_and_grad(P, cam_dict(cam), tmap, tgt.cpu(), K=cfg.K, k=cfg.k,
                                          bins=bins, depth_bt=torch.tensor(BT))
    assert float((ts.image.cpu() - img).abs().max()) <= 1e-4
    assert abs(float(ts.loss()) - float(L)) <= 1e-5
    Pr, m, v = P.clone(), torch.zeros_like(P), torch.zeros_like(P)
    oadam.adam_step(Pr, m, v, g, lr_vector(device="cpu"), 1)
    assert rel_l2(ts.P.cpu() - P, Pr - P) <= 1e-2
    # (beta, tau): the first Adam moment is (1 - b1) * the summed gradient
    assert rel_l2(ts.dw_state[:2].cpu() / (1 - oadam.B1), ex["gdepth"]) <= 1e-3
    bt, mb, vb = torch.tensor(BT), torch.zeros(2), torch.zeros(2)
    oadam.adam_step(bt, mb, vb, ex["gdepth"].float(), torch.tensor(0.02), 1)
    assert max_abs(ts.dw, bt) <= 1e-5


def test_depth_weight_graph_replay_batch_and_training():
    from ttsplat import scenes
    from ttsplat.camera import pinhole
    cfg, P, _ = config_inputs("c1_ref")
    cams = [pinhole(cfg.H, cfg.W, e) for e in scenes.orbit_eyes(2)]
    tgts = [_target(cfg, c) for c in cams]
    kw = dict(K=cfg.K, S=cfg.S, k=cfg.k, depth_weight=dict(beta0=1.0))
    eager = TrainStep(P, cams, tgts, **kw)
    graph = TrainStep(P, cams, tgts, **kw)
    assert abs(float(eager.dw[1]) - float(graph.dw[1])) == 0.0   # tau0 from the depth median
    graph.capture()
    for i in range(6):
        eager.step(i % 2)
        graph.step(i % 2)
        torch.cuda.synchronize()
    assert max_abs(graph.dw, eager.dw) <= 1e-6
    assert abs(float(graph.loss()) - float(eager.loss())) <= 1e-5
    batch = TrainStep(P, cams, tgts, batch=2, **kw)
    batch.capture()
    l0 = None
    for _ in range(120):
        batch.step(0)
        if l0 is None:
            l0 = float(batch.loss())
    assert float(batch.loss()) < 0.8 * l0
    assert float(batch.gdw.abs().max()) == 0.0                   # cleared after each update
    assert max_abs(batch.dw, torch.tensor([1.0, float(eager.dw[1])])) > 1e-3   # trained


def test_dense_arm_b_forward_and_grads():
    cfg, P, cam = config_inputs("c1_ref")
    model = GaussianModel(P.cuda(), depth_beta=BT[0], depth_tau=BT[1])
    model.params.requires_grad_(True)
    model.depth_beta.requires_grad_(True)
    model.depth_tau.requires_grad_(True)
    img = trender.render(model, cam, "B")
    R = torch.randn(cam.H, cam.W, 3, generator=torch.Generator().manual_seed(5))
    (img * R.cuda()).sum().backward()
    Pr = P.double().clone().requires_grad_(True)
    btr = torch.tensor(BT, dtype=torch.float64, requires_grad=True)
    ref = osplat.render_dense(Pr, cam_dict(cam), depth_bt=btr)
    assert max_abs(img, ref) <= 1e-4
    (ref * R.double()).sum().backward()
    assert rel_l2(model.params.grad, Pr.grad) <= 1e-3
    assert rel_l2(torch.stack([model.depth_beta.grad, model.depth_tau.grad]), btr.grad) <= 1e-3


def test_fit_arm_b_trains_the_depth_scalars():
    from ttsplat import scenes
    from ttsplat.camera import pinhole
    cfg, P, _ = config_inputs("c1_ref", G=300)
    cams = [pinhole(64, 64, e) for e in scenes.orbit_eyes(2)]
    gt_model = GaussianModel(cfg.params(seed=1)[:300].cuda(), depth_beta=2.0, depth_tau=2.5)
    with torch.no_grad():
        gts = [trender.render(gt_model, c, "B") for c in cams]
    model = GaussianModel(P.cuda())
    hist = ttrain.fit(model, cams, gts, "B", iters=40)
    assert hist[-1] < 0.8 * hist[0]
    assert abs(float(model.depth_beta) - 1.0) > 1e-3 and abs(float(model.depth_tau) - 3.0) > 1e-3
