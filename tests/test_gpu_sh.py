"""View-dependent SH colour on the GPU vs the oracle: geometry forward and backward at every
degree, the fused backward + Adam of the rest coefficients, the batch accumulation, and a whole
training step with SH degree 3 (tools/resident_traced.py:237-264,339-341,405-410,492-501)."""
import pytest
import torch

from helpers import cam_dict, config_inputs, max_abs, rel_l2
from oracle import adam as oadam
from oracle import binning as obin
from oracle import geometry as ogeo
from oracle import pipeline as opipe
from ttsplat import _lib, kernels
from ttsplat.step import TrainStep, lr_vector

pytestmark = pytest.mark.gpu


def rest_for(G, seed=7, scale=0.3):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(G, 15, 3, generator=g) * scale            # spike's color_rest layout


@pytest.mark.parametrize("name", ["c1_ref", "c4"])
@pytest.mark.parametrize("deg", [1, 2, 3])
def test_geom_fwd_sh(name, deg):
    cfg, P, cam = config_inputs(name)
    rest = rest_for(cfg.G)
    proj, keep = kernels.geom_fwd(P.cuda(), cam.device_block("cuda"),
                                  sh_rest=kernels.sh_rest_layout(rest.cuda()), sh_degree=deg)
    proj = proj.cpu()
    ref = ogeo.project_params(P.double(), cam_dict(cam), rest=rest.double(), sh_degree=deg)
    assert torch.equal(keep.cpu().bool(), ref["keep"])
    assert max_abs(proj[:, 6:9], ref["color_o"]) <= 1e-5
    assert max_abs(proj[:, 9], ref["o_col"]) <= 1e-6
    # the direction changes the colour: degree 0 would differ
    dc = ogeo.project_params(P.double(), cam_dict(cam))
    assert max_abs(dc["color_o"], ref["color_o"]) > 1e-2


@pytest.mark.parametrize("deg", [1, 2, 3])
def test_sh_view_direction_gradient_alone(deg):
    """The SH colour's gradient through its view direction (spike/render.py:23-25: the dense
    render's direction means - centre is not detached), alone: with an upstream gradient on the
    colour only, the means receive nothing but that term, so the geometry backward with
    TTS_GRAD_SH_DIR must equal autograd of sum(gcol_o keo colour(means - centre)) through the
    direction, and without the flag give zero (the device step's detached direction)."""
    from oracle import sh as osh
    cfg, P, cam = config_inputs("c1_ref")
    rest = rest_for(cfg.G)
    G = cfg.G
    gen = torch.Generator().manual_seed(40 + deg)
    grad9 = torch.zeros(G, 9)
    grad9[:, 5:8] = torch.randn(G, 3, generator=gen)
    print(f"[sh-dir] degree {deg} G={G}", flush=True)
    Pc, camb, g9 = P.cuda(), cam.device_block("cuda"), grad9.cuda()
    rl = kernels.sh_rest_layout(rest.cuda())
    on = kernels.geom_bwd(Pc, camb, g9, sh_rest=rl, sh_degree=deg, sh_dirgrad=True)[0].cpu()
    off = kernels.geom_bwd(Pc, camb, g9, sh_rest=rl, sh_degree=deg, sh_dirgrad=False)[0].cpu()
    camd = cam_dict(cam)
    Pd = P.double()
    keo = ogeo.project_params(Pd, camd)["o_col"]
    means = Pd[:, 0:3].clone().requires_grad_(True)
    centre = osh.camera_center(camd["R_v"].double(), camd["t_v"].double())
    coeffs = torch.cat([Pd[:, 10:13][:, None, :], rest.double()], dim=1)
    colour = osh.eval_sh_color(deg, coeffs, means - centre[None, :])
    (grad9[:, 5:8].double() * keo[:, None] * colour).sum().backward()
    ref = means.grad
    assert float(ref.norm()) > 1e-3
    assert float(off[:, 0:3].abs().max()) == 0.0
    e = rel_l2(on[:, 0:3], ref)
    print(f"[sh-dir] degree {deg}: rel L2 {e:.2e}", flush=True)
    assert e <= 1e-4
    assert torch.equal(on[:, 3:], off[:, 3:])


def _lib_keep(Pc, camb):
    return kernels.geom_fwd(Pc, camb)[1]


def test_geom_fwd_sh_degree0_and_zero_rest_equal_dc():
    cfg, P, cam = config_inputs("c1_ref")
    Pc, camb = P.cuda(), cam.device_block("cuda")
    base, _ = kernels.geom_fwd(Pc, camb)
    zero = torch.zeros(15, 3, cfg.G, device="cuda")
    # degree 0 through the SH entry point is the DC kernel's result to fp32 rounding (the two
    # kernel instances may contract multiply-adds differently)
    p0 = torch.empty_like(base)
    k0 = torch.empty(cfg.G, device="cuda", dtype=torch.uint8)
    _lib.call("tts_geom_fwd_ex", _lib.ptr(Pc), _lib.ptr(zero), 0, None, cfg.G, _lib.ptr(camb),
              0.2, 0.3, _lib.ptr(p0), _lib.ptr(k0), None, 0.9, 0.999, _lib.stream())
    assert torch.equal(k0, _lib_keep(Pc, camb))
    assert float(((p0 - base).abs() / base.abs().clamp(min=1.0)).max()) <= 1e-6
    # zero rest at degree 3: the colour is the DC colour (up to the summation order)
    p3, _ = kernels.geom_fwd(Pc, camb, sh_rest=zero, sh_degree=3)
    assert float(((p3 - base).abs() / base.abs().clamp(min=1.0)).max()) <= 1e-6


@pytest.mark.parametrize("deg", [1, 3])
def test_geom_bwd_sh(deg):
    cfg, P, cam = config_inputs("c1_ref")
    rest = rest_for(cfg.G)
    g = torch.Generator().manual_seed(11)
    grad9 = torch.randn(cfg.G, 9, generator=g)
    gP, gsh, _ = kernels.geom_bwd(P.cuda(), cam.device_block("cuda"), grad9.cuda(),
                               sh_rest=kernels.sh_rest_layout(rest.cuda()), sh_degree=deg)
    Pr = P.double().clone().requires_grad_(True)
    rr = rest.double().clone().requires_grad_(True)
    ref = ogeo.project_params(Pr, cam_dict(cam), rest=rr, sh_degree=deg)
    out = torch.cat([ref["conic"], ref["mu2d"], ref["color_o"], ref["o_col"][:, None]], 1)
    (out * grad9.double()).sum().backward()
    for sl in (slice(0, 3), slice(3, 7), slice(7, 10), slice(10, 13), slice(13, 14)):
        assert rel_l2(gP.cpu()[:, sl], Pr.grad[:, sl]) <= 1e-3, sl
    n = (deg + 1) ** 2 - 1
    gm = kernels.sh_rest_model(gsh).cpu()
    assert rel_l2(gm[:, :n], rr.grad[:, :n]) <= 1e-4
    if n < 15:
        assert float(gm[:, n:].abs().max()) == 0.0


def test_bad_sh_arguments_raise():
    cfg, P, cam = config_inputs("c1_ref")
    with pytest.raises(ValueError):
        kernels.geom_fwd(P.cuda(), cam.device_block("cuda"), sh_degree=4,
                         sh_rest=torch.zeros(15, 3, cfg.G, device="cuda"))
    with pytest.raises(ValueError):
        kernels.geom_fwd(P.cuda(), cam.device_block("cuda"), sh_degree=2)
    Pc, camb = P.cuda(), cam.device_block("cuda")
    proj = torch.empty(cfg.G, 12, device="cuda")
    keep = torch.empty(cfg.G, device="cuda", dtype=torch.uint8)
    with pytest.raises(_lib.TTSError, match="SH degree"):   # the C ABI's own check
        _lib.call("tts_geom_fwd_ex", _lib.ptr(Pc), None, 2, None, cfg.G, _lib.ptr(camb), 0.2,
                  0.3, _lib.ptr(proj), _lib.ptr(keep), None, 0.9, 0.999, _lib.stream())


def target_for(cfg, cam, rest=None, deg=0):
    P1 = cfg.params(seed=1)
    ts = TrainStep(P1, [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S, k=cfg.k,
                   sh_degree=deg, sh_rest=rest)
    img = ts.forward(0).clone()
    torch.cuda.synchronize()
    return img


def test_train_step_sh3_matches_oracle():
    cfg, P, cam = config_inputs("c1_ref")
    rest = rest_for(cfg.G)
    tgt = target_for(cfg, cam, rest_for(cfg.G, seed=8), 3)
    ts = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, sh_degree=3, sh_rest=rest)
    ts.enqueue(0)
    torch.cuda.synchronize()
    bins = (ts.idx.cpu().long(), ts.valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    img, L, g, ex = opipe.render_and_grad(P, cam_dict(cam), tmap, tgt.cpu(), K=cfg.K, k=cfg.k,
                                          bins=bins, rest=rest, sh_degree=3)
    assert float((ts.image.cpu() - img).abs().max()) <= 1e-4
    assert abs(float(ts.loss()) - float(L)) <= 1e-5
    lr = lr_vector(device="cpu")
    Pr, m, v = P.clone(), torch.zeros_like(P), torch.zeros_like(P)
    oadam.adam_step(Pr, m, v, g, lr, 1)
    assert rel_l2(ts.P.cpu() - P, Pr - P) <= 1e-2
    # the rest block: Adam at the colour rate / 20
    lr_sh = float(lr[10]) / 20.0
    rr, mr, vr = rest.clone(), torch.zeros_like(rest), torch.zeros_like(rest)
    oadam.adam_step(rr, mr, vr, ex["grest"], torch.tensor(lr_sh), 1)
    assert rel_l2(ts.color_rest.cpu() - rest, rr - rest) <= 1e-2
    # the first Adam moment is (1 - b1) * gradient: the rest gradient itself, to fp32 precision
    gm = kernels.sh_rest_model(ts.sh_m).cpu() / (1 - oadam.B1)
    assert rel_l2(gm, ex["grest"]) <= 1e-3


def test_sh_graph_replay_matches_eager_and_trains():
    cfg, P, cam = config_inputs("c1_ref")
    rest = rest_for(cfg.G)
    tgt = target_for(cfg, cam, rest_for(cfg.G, seed=8), 3)
    eager = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, sh_degree=3, sh_rest=rest)
    graph = TrainStep(P, [cam], [tgt], K=cfg.K, S=cfg.S, k=cfg.k, sh_degree=3, sh_rest=rest)
    graph.capture()
    le, lg = [], []
    for _ in range(5):
        eager.step(0)
        le.append(float(eager.loss()))
        graph.step(0)
        lg.append(float(graph.loss()))
    for a, b in zip(le, lg):
        assert abs(a - b) <= 1e-5 * max(1.0, abs(a))
    assert rel_l2(graph.sh - rest_for(cfg.G).cuda().permute(1, 2, 0),
                  eager.sh - rest_for(cfg.G).cuda().permute(1, 2, 0)) <= 1e-3
    for _ in range(150):
        graph.step(0)
    assert float(graph.loss()) < 0.8 * lg[0]


def test_sh_batch_step_matches_oracle_mean_gradient():
    from ttsplat import scenes
    from ttsplat.camera import pinhole
    cfg, P, _ = config_inputs("c1_ref")
    rest = rest_for(cfg.G)
    cams = [pinhole(cfg.H, cfg.W, e) for e in scenes.orbit_eyes(2)]
    tgts = [target_for(cfg, c, rest_for(cfg.G, seed=8), 2) for c in cams]
    ts = TrainStep(P, cams, tgts, K=cfg.K, S=cfg.S, k=cfg.k, batch=2, sh_degree=2,
                   sh_rest=rest)
    ts.enqueue(0)
    torch.cuda.synchronize()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    gs, gr = [], []
    for c, t in zip(cams, tgts):
        _, _, g, ex = opipe.render_and_grad(P, cam_dict(c), tmap, t.cpu(), K=cfg.K, k=cfg.k,
                                            stable=True, rest=rest, sh_degree=2)
        gs.append(g)
        gr.append(ex["grest"])
    g = torch.stack(gs).mean(0)
    grest = torch.stack(gr).mean(0)
    lr = lr_vector(device="cpu")
    Pr, m, v = P.clone(), torch.zeros_like(P), torch.zeros_like(P)
    oadam.adam_step(Pr, m, v, g, lr, 1)
    assert rel_l2(ts.P.cpu() - P, Pr - P) <= 1e-2
    gm = kernels.sh_rest_model(ts.sh_m).cpu() / (1 - oadam.B1)
    assert rel_l2(gm[:, :8], grest[:, :8]) <= 1e-3
    assert float(gm[:, 8:].abs().max()) == 0.0                 # degree 2 uses 8 rest rows
    assert float(ts.gacc_sh.abs().max()) == 0.0                # cleared for the next batch
