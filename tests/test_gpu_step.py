"""The graph-captured training step vs the oracle's step, and graph replay vs eager."""
import pytest
import torch

from helpers import cam_dict, config_inputs, rel_l2, update_error_ok
from oracle import adam as oadam
from oracle import binning as obin
from oracle import pipeline as opipe
from oracle import splat as osplat
from ttsplat import kernels
from ttsplat.step import TrainStep, lr_vector

pytestmark = pytest.mark.gpu

# the bf16 step's gradient contract against fp64 autograd: the bf16 render's image error (up to
# ~5e-3 here) moves dL/dimage -- the L1 term's sign flips where |x - y| is below it -- and the
# splat backward's C and den, so the gradient gets 2e-2 relative L2 per parameter group
BF16_GRAD_TOL = 2e-2
GROUPS = {"means": slice(0, 3), "quats": slice(3, 7), "scales": slice(7, 10),
          "color": slice(10, 13), "opacity": slice(13, 14)}


def target_for(cfg, cam):
    """Target image: the GPU render of the seed-1 gaussian set from the same camera."""
    P1 = cfg.params(seed=1)
    ts = TrainStep(P1, [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S, k=cfg.k)
    img = ts.forward(0).clone()
    torch.cuda.synchronize()
    return img


def test_train_step_matches_oracle():
    cfg, P, cam = config_inputs("c1_ref")
    tgt = target_for(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    ts.enqueue(0)
    torch.cuda.synchronize()
    # oracle: same bins as the GPU used (bin tables are tested bit-exact separately)
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    Pr = P.clone()
    m = torch.zeros_like(Pr)
    v = torch.zeros_like(Pr)
    lr = lr_vector(device="cpu")
    img, L, g = opipe.train_step(Pr, m, v, 1, cam_dict(cam), tmap, tgt.cpu(), lr, K=cfg.K,
                                 k=cfg.k, bins=bins)
    assert float((ts.image.cpu() - img).abs().max()) <= 1e-4
    assert abs(float(ts.loss()) - float(L)) <= 1e-5
    # Adam's first step is ~lr*sign(g): compare the parameter updates
    du_gpu = ts.P.cpu() - P
    du_ref = Pr - P
    assert rel_l2(du_gpu, du_ref) <= 1e-2
    assert int(ts.step_block[0]) == 1


def test_graph_replay_matches_eager():
    cfg, P, cam = config_inputs("c1_ref")
    tgt = target_for(cfg, cam)
    eager = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    graph = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    graph.capture()
    losses_e, losses_g = [], []
    for _ in range(5):
        eager.step(0)
        losses_e.append(float(eager.loss()))
        graph.step(0)
        losses_g.append(float(graph.loss()))   # eager work + sync between replays
    torch.cuda.synchronize()
    assert graph.steps_done == 5 and eager.steps_done == 5
    for a, b in zip(losses_e, losses_g):
        assert abs(a - b) <= 1e-5 * max(1.0, abs(a))
    assert rel_l2(graph.P - P.cuda(), eager.P - P.cuda()) <= 1e-3


def test_training_reduces_loss():
    cfg, P, cam = config_inputs("c1_ref")
    tgt = target_for(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    ts.capture()
    ts.step(0)
    l0 = float(ts.loss())
    for _ in range(200):
        ts.step(0)
    l1 = float(ts.loss())
    assert l1 < 0.8 * l0, (l0, l1)


def test_batch_step_matches_oracle_mean_gradient():
    """batch = 4: one Adam update on the mean gradient of 4 views (spike/train.py:21-33)."""
    from ttsplat import scenes
    from ttsplat.camera import pinhole
    cfg, P, _ = config_inputs("c1_ref")
    cams = [pinhole(cfg.H, cfg.W, e) for e in scenes.orbit_eyes(4)]
    tgts = [target_for(cfg, c) for c in cams]
    ts = TrainStep(P, cams, tgts, K=cfg.K, S=cfg.S, k=cfg.k, batch=4)
    assert ts.n_steps == 1
    ts.enqueue(0)
    torch.cuda.synchronize()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    grads = []
    for c, t in zip(cams, tgts):
        _, _, g, _ = opipe.render_and_grad(P, cam_dict(c), tmap, t.cpu(), K=cfg.K, k=cfg.k,
                                           stable=True)
        grads.append(g)
    g = torch.stack(grads).mean(0)
    Pr, m, v = P.clone(), torch.zeros_like(P), torch.zeros_like(P)
    oadam.adam_step(Pr, m, v, g, lr_vector(device="cpu"), 1)
    assert rel_l2(ts.P.cpu() - P, Pr - P) <= 1e-2
    assert int(ts.step_block[0]) == 1
    assert float(ts.gacc.abs().max()) == 0.0          # cleared for the next batch
    with pytest.raises(ValueError):
        TrainStep(P, cams[:3], tgts[:3], K=cfg.K, batch=2)


def test_geom_bwd_accum_adds_scaled_gradients():
    cfg, P, cam = config_inputs("c1_ref")
    tgt = target_for(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    ts._view_backward(0)
    grad9 = kernels.slot_reduce(ts.gslot, ts.inv)
    g14 = kernels.geom_bwd(ts.P, ts.cams[0], grad9)
    acc = torch.zeros_like(g14)
    kernels.geom_bwd_accum(ts.P, ts.cams[0], ts.gslot, ts.inv, acc, 0.25)
    kernels.geom_bwd_accum(ts.P, ts.cams[0], ts.gslot, ts.inv, acc, 0.5)
    assert rel_l2(acc, 0.75 * g14) <= 1e-6


def test_bf16_train_step():
    """The bf16 render variant in the training step: image within 1e-2 of the fp32 oracle, the
    graph replay equals the eager step, and training lowers the loss."""
    cfg, P, cam = config_inputs("c2")
    tgt = target_for(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, dtype="bf16")
    img = ts.forward(0).clone()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    ref = osplat.render_binned(P, cam_dict(cam), tmap, K=cfg.K, k=cfg.k, stable=True)
    assert float((img.cpu() - ref).abs().max()) <= 1e-2
    eager = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, dtype="bf16")
    ts.capture()
    for _ in range(3):
        ts.step(0)
        eager.step(0)
        assert abs(float(ts.loss()) - float(eager.loss())) <= 1e-6
    l0 = float(ts.loss())
    for _ in range(200):
        ts.step(0)
    assert float(ts.loss()) < 0.8 * l0
    with pytest.raises(ValueError):
        TrainStep(P, [cam], [tgt], K=cfg.K, S=32, k=cfg.k, dtype="bf16")


@pytest.mark.parametrize("G", [1, 257])
def test_train_step_small_and_ragged_sets(G):
    """One gaussian, and a set that leaves the last geometry workgroup ragged (257 rows): the
    step still matches the oracle's step."""
    cfg, P, cam = config_inputs("c1_ref", G=G)
    P[:, 0:3] *= 0.3                      # keep the few gaussians in view
    tgt = target_for(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    ts.enqueue(0)
    torch.cuda.synchronize()
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    assert int(ts.valid.sum()) > 0
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    Pr = P.clone()
    m = torch.zeros_like(Pr)
    v = torch.zeros_like(Pr)
    img, L, g = opipe.train_step(Pr, m, v, 1, cam_dict(cam), tmap, tgt.cpu(),
                                 lr_vector(device="cpu"), K=cfg.K, k=cfg.k, bins=bins)
    assert float((ts.image.cpu() - img).abs().max()) <= 1e-4
    assert abs(float(ts.loss()) - float(L)) <= 1e-5
    assert rel_l2(ts.P.cpu() - P, Pr - P) <= 1e-2


def test_train_step_with_everything_culled():
    """Every gaussian behind the camera: the image is the background, no gradient reaches the
    parameters (Adam leaves them unchanged), and graph replays agree with eager steps."""
    cfg, P, cam = config_inputs("c1_ref")
    P = P.clone()
    P[:, 2] = 10.0                        # the camera sits at z = 3 looking at the origin
    tgt = torch.rand(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(4))
    eager = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    graph = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    graph.capture()
    for _ in range(3):
        eager.step(0)
        graph.step(0)
    torch.cuda.synchronize()
    assert int(eager.keep.sum()) == 0 and int(eager.valid.sum()) == 0
    assert float((eager.image - 1.0).abs().max()) <= 1e-6        # w_b c_b / w_b = c_b = 1
    assert torch.equal(eager.P.cpu(), P) and torch.equal(graph.P.cpu(), P)
    assert float(eager.m.abs().max()) == 0.0
    assert abs(float(eager.loss()) - float(graph.loss())) == 0.0
    assert int(graph.step_block[0]) == 3


def test_bin_every_reuses_bins_between_rebins():
    """bin_every = 5 (tools/resident_traced.py:103,683): the bin table is rebuilt on steps 0, 5,
    10, ... only; in between the step runs on the last table.  Graph replay equals eager, and a
    reused-bin step equals the oracle's step on those (stale) bins."""
    cfg, P, cam = config_inputs("c1_ref")
    tgt = target_for(cfg, cam)
    eager = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, bin_every=5, keep_grad=True)
    graph = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, bin_every=5)
    graph.capture()
    assert set(graph.graphs) == {(0, True), (0, False)}
    rebinned = []
    for i in range(7):
        eager.count.fill_(-1)           # the binning kernels rewrite it; a reused table leaves it
        graph.count.fill_(-1)
        if i == 3:
            Pb = eager.P.cpu().clone()
        eager.step(0)
        graph.step(0)
        torch.cuda.synchronize()
        rebinned.append((int(eager.count.min()) >= 0, int(graph.count.min()) >= 0))
        assert abs(float(eager.loss()) - float(graph.loss())) <= 1e-5 * max(1.0, float(eager.loss()))
        if i == 3:      # a reused-bin step against the oracle on the same (stale) bins
            tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
            bins = (eager.idx.cpu().long(), eager.valid.cpu().bool())
            img, L, g, _ = opipe.render_and_grad(Pb, cam_dict(cam), tmap, tgt.cpu(), K=cfg.K,
                                                 k=cfg.k, bins=bins)
            assert float((eager.image.cpu() - img).abs().max()) <= 1e-4
            assert rel_l2(eager.gparams.cpu(), g) <= 1e-3
    assert [e for e, _ in rebinned] == [True, False, False, False, False, True, False]
    assert [g for _, g in rebinned] == [True, False, False, False, False, True, False]
    assert rel_l2(graph.P, eager.P) <= 1e-3
    with pytest.raises(ValueError):
        TrainStep(P, [cam, cam], [tgt, tgt], K=cfg.K, S=cfg.S, k=cfg.k, bin_every=5, batch=2)


@pytest.mark.parametrize("bin_every", [1, 2, 3])
def test_run_graphs_match_single_steps(bin_every):
    """run(i, n) (graphs of run_len consecutive steps, one per starting camera and bin-cadence
    phase, then one-step graphs for the remainder) leaves the same state, bit for bit, as n
    step() calls from step i -- also across a forward() that rebins out of cadence, after which
    both rebin on the next step."""
    from ttsplat import scenes
    cfg, P, _ = config_inputs("c1_ref")
    cams = scenes.Config(**{**cfg.__dict__, "n_cams": 3}).cameras()
    tgts = [target_for(cfg, c) for c in cams]
    runs = TrainStep(P, cams, tgts, K=cfg.K, S=cfg.S, k=cfg.k, bin_every=bin_every, seam=True)
    assert runs.seamed == (bin_every == 1)
    runs.capture(run_len=4)
    assert sorted(runs.run_graphs) == [(c, ph) for c in range(3) for ph in range(bin_every)]
    single = TrainStep(P, cams, tgts, K=cfg.K, S=cfg.S, k=cfg.k, bin_every=bin_every)
    single.capture(run_len=1)
    runs.run(1, 11)                        # two runs of 4, then 3 single steps
    for i in range(11):
        single.step((1 + i) % 3)
    for ts in (runs, single):              # a render of camera 2 rebins out of cadence
        ts.forward(2, grads=False)
    runs.run(0, 9)                         # one step() (the forced rebin), then runs of 4
    for i in range(9):
        single.step(i % 3)
    torch.cuda.synchronize()
    assert runs.steps_done == single.steps_done == 20
    for a, b in ((runs.P, single.P), (runs.m, single.m), (runs.v, single.v),
                 (runs.step_block, single.step_block)):
        assert torch.equal(a, b)
    assert float(runs.loss()) == float(single.loss())


def test_bf16_step_gradient_matches_oracle():
    """The gradient the bf16 step trains on -- the bf16 matrix-core forward, then the fp32 loss
    gradient and fp32 splat backward on that forward's image and den -- against fp64 oracle
    autograd on the same bins (G = 2000, 128 x 128): within BF16_GRAD_TOL relative L2 per
    parameter group; the image within the bf16 render's 1e-2; the loss within 1e-3; the Adam
    update applied to the gradient the kernel received, per entry."""
    cfg, P, cam = config_inputs("c2")
    tgt = target_for(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, dtype="bf16", keep_grad=True)
    ts.enqueue(0)
    torch.cuda.synchronize()
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    img, L, g, _ = opipe.render_and_grad(P.double(), cam_dict(cam), tmap, tgt.cpu().double(),
                                         K=cfg.K, k=cfg.k, bins=bins)
    err = float((ts.image.cpu().double() - img).abs().max())
    dl = abs(float(ts.loss()) - float(L))
    print(f"[c2 bf16 step] image max|err| {err:.2e}, |dloss| {dl:.2e}", flush=True)
    assert err <= 1e-2 and dl <= 1e-3
    gP = ts.gparams.cpu()
    errs = {name: rel_l2(gP[:, sl], g[:, sl]) for name, sl in GROUPS.items()}
    print("[c2 bf16 step] rel L2 " + ", ".join(f"d{n} {e:.2e}" for n, e in errs.items()),
          flush=True)
    for name, e in errs.items():
        assert e <= BF16_GRAD_TOL, name
    Pa, m, v = P.clone().double(), torch.zeros(P.shape, dtype=torch.float64), \
        torch.zeros(P.shape, dtype=torch.float64)
    oadam.adam_step(Pa, m, v, gP.double(), lr_vector(device="cpu").double(), 1)
    assert update_error_ok(ts.P, P, Pa) == 0


def test_fp32_step_gradient_matches_oracle():
    """The fp32 step's gradient (G = 2000, 128 x 128) against fp64 oracle autograd on the same
    bins: within 1e-3 relative L2 per parameter group; the fused Adam update per entry."""
    cfg, P, cam = config_inputs("c1_ref")
    tgt = target_for(cfg, cam)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, keep_grad=True)
    ts.enqueue(0)
    torch.cuda.synchronize()
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    _, _, g, _ = opipe.render_and_grad(P.double(), cam_dict(cam), tmap, tgt.cpu().double(),
                                       K=cfg.K, k=cfg.k, bins=bins)
    gP = ts.gparams.cpu()
    for name, sl in GROUPS.items():
        e = rel_l2(gP[:, sl], g[:, sl])
        print(f"[c1_ref step] d{name}: rel L2 {e:.2e}", flush=True)
        assert e <= 1e-3, name
    Pa, m, v = P.clone().double(), torch.zeros(P.shape, dtype=torch.float64), \
        torch.zeros(P.shape, dtype=torch.float64)
    oadam.adam_step(Pa, m, v, gP.double(), lr_vector(device="cpu").double(), 1)
    assert update_error_ok(ts.P, P, Pa) == 0


def test_render_between_steps_with_bin_every():
    """bin_every = 5: a step, a render of another camera that rebins without the inverse table
    (forward(grads=False)), then a step.  The render replaced the shared bins, so the second step
    rebins; its gradient matches the oracle's on the bins it used (with the render's bins and
    the first step's inverse table the slot gather would hand gaussians other slots' gradients)."""
    from ttsplat import scenes
    from ttsplat.camera import pinhole
    cfg, P, _ = config_inputs("c1_ref")
    cams = [pinhole(cfg.H, cfg.W, e) for e in scenes.orbit_eyes(2)]
    tgts = [target_for(cfg, c) for c in cams]
    ts = TrainStep(P, cams, tgts, K=cfg.K, S=cfg.S, k=cfg.k, bin_every=5, keep_grad=True)
    ts.capture()
    ts.step(0)
    ts.forward(1, grads=False)
    P1 = ts.P.cpu().clone()
    ts.step(0)
    torch.cuda.synchronize()
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    _, _, g, _ = opipe.render_and_grad(P1.double(), cam_dict(cams[0]), tmap,
                                       tgts[0].cpu().double(), K=cfg.K, k=cfg.k, bins=bins)
    gP = ts.gparams.cpu()
    for name, sl in GROUPS.items():
        e = rel_l2(gP[:, sl], g[:, sl])
        print(f"[bin_every render] d{name}: rel L2 {e:.2e}", flush=True)
        assert e <= 1e-3, name


def rgba_target(cfg, cam):
    """An RGBA target: the seed-1 render with a soft-edged disc of alpha (0 outside, 1 inside,
    partial on the rim)."""
    rgb = target_for(cfg, cam).cpu()
    yy, xx = torch.meshgrid(torch.arange(cfg.H, dtype=torch.float32),
                            torch.arange(cfg.W, dtype=torch.float32), indexing="ij")
    r = ((xx - 0.47 * cfg.W) ** 2 + (yy - 0.55 * cfg.H) ** 2).sqrt()
    alpha = (1.2 - r / (0.3 * cfg.W)).clamp(0, 1)
    return torch.cat([rgb, alpha[..., None]], -1)


def test_random_bg_step_matches_oracle():
    """random_bg: each step draws its background on the device (Philox keyed by the completed
    steps, the view and the seed; a replayed graph draws anew), composites the RGBA target over
    it and renders with it as c_b.  The draws equal the oracle's, the composited target is exact,
    and the second step's image, loss and gradient match the oracle's step on that background."""
    import numpy as np
    from oracle import rng as orng
    cfg, P, cam = config_inputs("c1_ref")
    rgba = rgba_target(cfg, cam)
    ts = TrainStep(P, [cam], [rgba], K=cfg.K, S=cfg.S, k=cfg.k, random_bg=True, bg_seed=7,
                   keep_grad=True)
    assert ts.stats_mode == "per_step"
    ts.capture()
    ts.step(0)
    torch.cuda.synchronize()
    bg1 = ts.bg.cpu().clone()
    P1 = ts.P.cpu().clone()
    ts.step(0)
    torch.cuda.synchronize()
    bg2 = ts.bg.cpu().clone()
    for step, bg in ((0, bg1), (1, bg2)):
        assert torch.equal(bg[1:], torch.from_numpy(orng.random_bg(0, step, 7))), step
    assert not torch.equal(bg1, bg2)
    pm = kernels.rgba_premult(rgba)
    target = pm[..., :3] + pm[..., 3:4] * bg2[1:]
    assert torch.equal(ts.target_buf.cpu(), target)
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    img, L, g, _ = opipe.render_and_grad(P1.double(), cam_dict(cam), tmap, target.double(),
                                         K=cfg.K, k=cfg.k, bins=bins, c_b=bg2[1:].double())
    err = float((ts.image.cpu().double() - img).abs().max())
    print(f"[random bg] bg {bg2[1:].tolist()}, image max|err| {err:.2e}", flush=True)
    assert err <= 1e-4
    assert abs(float(ts.loss()) - float(L)) <= 1e-5
    gP = ts.gparams.cpu()
    for name, sl in GROUPS.items():
        assert rel_l2(gP[:, sl], g[:, sl]) <= 1e-3, name


def test_per_step_target_stats_equal_per_view():
    """target_stats = "per_step" (one statistics buffer, recomputed at every view backward, as
    the reference's recompute_gt_stats) gives the per-view mode's state to the bit."""
    from ttsplat import scenes
    from ttsplat.camera import pinhole
    cfg, P, _ = config_inputs("c1_ref")
    cams = [pinhole(cfg.H, cfg.W, e) for e in scenes.orbit_eyes(3)]
    tgts = [target_for(cfg, c) for c in cams]
    a = TrainStep(P, cams, tgts, K=cfg.K, S=cfg.S, k=cfg.k)
    b = TrainStep(P, cams, tgts, K=cfg.K, S=cfg.S, k=cfg.k, target_stats="per_step")
    b.capture()
    for i in range(6):
        a.step(i % 3)
        b.step(i % 3)
        assert float(a.loss()) == float(b.loss())
    assert torch.equal(a.P, b.P)


def test_eval_psnr_renders_on_white():
    """eval_psnr: the binned render of each view on a white background against its image
    (RGBA composited over white), psnr on clamped images; the training state is untouched and
    the next step rebins."""
    cfg, P, cam = config_inputs("c1_ref")
    rgba = rgba_target(cfg, cam)
    ts = TrainStep(P, [cam], [rgba], K=cfg.K, S=cfg.S, k=cfg.k, random_bg=True, bg_seed=3)
    ts.capture()
    for _ in range(5):
        ts.step(0)
    torch.cuda.synchronize()
    state = [t.clone() for t in (ts.P, ts.m, ts.v, ts.step_block)]
    psnr = ts.eval_psnr([cam], [rgba])
    for t, s0 in zip((ts.P, ts.m, ts.v, ts.step_block), state):
        assert torch.equal(t, s0)
    white = rgba[..., :3] * rgba[..., 3:4] + (1 - rgba[..., 3:4])
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    ref = osplat.render_binned(ts.P.cpu().double(), cam_dict(cam), tmap, K=cfg.K, k=cfg.k,
                               stable=True)
    mse = (ref.clamp(0, 1) - white.double().clamp(0, 1)).pow(2).mean()
    want = float(-10 * torch.log10(mse))
    print(f"[eval] psnr {psnr:.4f} dB, oracle {want:.4f} dB", flush=True)
    assert abs(psnr - want) <= 1e-3
    assert ts._force_rebin
    ts.step(0)
    torch.cuda.synchronize()
    assert int(ts.step_block[0]) == 6


@pytest.mark.parametrize("mode", ["random_bg", "keep_grad", "bf16"])
def test_seamed_runs_match_single_steps(mode):
    """run() on a plain step joins consecutive steps at the seam (one launch for step i's
    geometry backward + Adam and step i+1's geometry forward + binning count; step i+1's Adam
    advance on its column scan).  With a random background (drawn between the two launches,
    before the advance, as step() draws it), with the per-step gradient kept, and with the bf16
    render, 2 runs of 5 steps and 3 single steps leave the state step() calls leave, bit for
    bit: parameters, moments, step block, background, gradient and loss."""
    from ttsplat import scenes
    cfg, P, _ = config_inputs("c2" if mode == "bf16" else "c1_ref")
    cams = scenes.Config(**{**cfg.__dict__, "n_cams": 3}).cameras()
    kw = dict(K=cfg.K, S=cfg.S, k=cfg.k, dtype=cfg.dtype, seam=True)
    if mode == "random_bg":
        tgts = [rgba_target(cfg, c) for c in cams]
        kw.update(random_bg=True, bg_seed=5)
    else:
        tgts = [target_for(cfg, c) for c in cams]
    if mode == "keep_grad":
        kw.update(keep_grad=True)
    runs = TrainStep(P, cams, tgts, **kw)
    assert runs.seamed
    runs.capture(run_len=5)
    single = TrainStep(P, cams, tgts, **kw)
    single.capture(run_len=1)
    runs.run(2, 13)
    for i in range(13):
        single.step((2 + i) % 3)
    torch.cuda.synchronize()
    for a, b in ((runs.P, single.P), (runs.m, single.m), (runs.v, single.v),
                 (runs.step_block, single.step_block), (runs.bg, single.bg),
                 (runs.image, single.image)):
        assert torch.equal(a, b)
    if mode == "keep_grad":
        assert torch.equal(runs.gparams, single.gparams)
    assert float(runs.loss()) == float(single.loss())
    assert int(runs.step_block[0]) == 13


def test_step_configurations_without_a_seam():
    """The seam is used by default from G = kernels.SEAM_MIN_G on, with seam=True for any G,
    never with seam=False; SH colour, the depth weight, MCMC terms, bin_every > 1 and batches
    keep the two launches whatever seam says, and enqueue_seamed refuses them."""
    from ttsplat import scenes
    cfg, P, cam = config_inputs("c1_ref")
    tgt = target_for(cfg, cam)
    base = dict(K=cfg.K, S=cfg.S, k=cfg.k, seam=True)
    assert TrainStep(P, [cam], [tgt], **base).seamed
    small = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k)
    assert small.seam_possible and not small.seamed          # G = 2000 < SEAM_MIN_G
    assert not TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, seam=False).seamed
    cfg_b, P_b, _ = config_inputs("c1_ref", G=kernels.SEAM_MIN_G)
    assert TrainStep(P_b, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k).seamed
    with pytest.raises(ValueError):
        TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, seam="yes")
    for kw in (dict(bin_every=2), dict(depth_weight=dict(beta0=1.0, tau0=3.0, lr_bt=0.02)),
               dict(mcmc=dict(lambda_o=0.01)),
               dict(sh_degree=1, sh_rest=torch.zeros(cfg.G, 15, 3))):
        ts = TrainStep(P, [cam], [tgt], **base, **kw)
        assert not ts.seamed and not ts.seam_possible, kw
        with pytest.raises(ValueError):
            ts.enqueue_seamed(0, 2)
    cams = scenes.Config(**{**cfg.__dict__, "n_cams": 2}).cameras()
    assert not TrainStep(P, cams, [tgt, tgt], batch=2, **base).seamed
