"""GPU geometry forward/backward, loss gradient and Adam vs the oracle."""
import pytest
import torch

from helpers import cam_dict, config_inputs, max_abs, rel_l2, update_error_ok
from oracle import adam as oadam
from oracle import geometry as ogeo
from oracle import loss as oloss
from ttsplat import kernels

pytestmark = pytest.mark.gpu


CAMS = pytest.mark.parametrize("aniso", [False, True], ids=["fx=fy", "fx=1.13fy"])


@CAMS
@pytest.mark.parametrize("name", ["c1_ref", "c4"])
def test_geom_fwd(name, aniso):
    cfg, P, cam = config_inputs(name, aniso=aniso)
    proj, keep = kernels.geom_fwd(P.cuda(), cam.device_block("cuda"))
    proj = proj.cpu()
    ref = ogeo.project_params(P.double(), cam_dict(cam))
    k = ref["keep"]
    assert torch.equal(keep.cpu().bool(), k)
    assert rel_l2(proj[k, 0:2], ref["mu2d"][k]) <= 1e-6
    assert rel_l2(proj[k, 2:5], ref["conic"][k]) <= 1e-4
    assert rel_l2(proj[:, 5], ref["depth"]) <= 1e-6
    assert max_abs(proj[:, 6:9], ref["color_o"]) <= 1e-6
    assert max_abs(proj[:, 9], ref["o_col"]) <= 1e-6


@CAMS
@pytest.mark.parametrize("name", ["c1_ref", "c4"])
def test_geom_bwd(name, aniso):
    cfg, P, cam = config_inputs(name, aniso=aniso)
    g = torch.Generator().manual_seed(11)
    grad9 = torch.randn(cfg.G, 9, generator=g)
    gP = kernels.geom_bwd(P.cuda(), cam.device_block("cuda"), grad9.cuda()).cpu()
    Pr = P.double().clone().requires_grad_(True)
    ref = ogeo.project_params(Pr, cam_dict(cam))
    out = torch.cat([ref["conic"], ref["mu2d"], ref["color_o"], ref["o_col"][:, None]], 1)
    (out * grad9.double()).sum().backward()
    for sl in (slice(0, 3), slice(3, 7), slice(7, 10), slice(10, 13), slice(13, 14)):
        assert rel_l2(gP[:, sl], Pr.grad[:, sl]) <= 1e-3, sl


@pytest.mark.parametrize("H,W", [(128, 128), (96, 160), (11, 13)])
def test_loss_grad(H, W):
    g = torch.Generator().manual_seed(H + W)
    x = torch.rand(H, W, 3, generator=g) * 1.2 - 0.1          # some pixels outside [0,1]
    y = torch.rand(H, W, 3, generator=g)
    n, ns = kernels.loss_partials_count(H, W)
    partials = torch.empty(n, device="cuda")
    gx = kernels.loss_grad(x.cuda(), y.cuda(), 0.2, partials=partials)
    loss = kernels.loss_from_partials(partials, H, W, 0.2)
    rl, rg = oloss.loss_and_grad(x.double(), y.double(), 0.2)
    assert abs(float(loss) - float(rl)) <= 1e-5
    assert rel_l2(gx, rg) <= 1e-4


@pytest.mark.parametrize("H,W", [(11, 11), (33, 75), (96, 130), (200, 300)])
def test_loss_grad_ragged_sizes(H, W):
    """Sizes that do not divide the 40 x 64 tiles (ragged tiles, the 11 x 11 minimum), with x
    outside [0, 1] in places (the clamp gate), against the oracle; a second call into the same
    workspace gives the same result."""
    g = torch.Generator().manual_seed(H * W)
    x = (torch.rand(H, W, 3, generator=g) * 1.2 - 0.1).cuda()
    y = torch.rand(H, W, 3, generator=g).cuda()
    n, ns = kernels.loss_partials_count(H, W)
    pa = torch.empty(n, device="cuda")
    pb = torch.empty(n, device="cuda")
    ws = kernels.loss_workspace(H, W, "cuda")
    ga = kernels.loss_grad(x, y, 0.2, partials=pa, workspace=ws)
    gb = kernels.loss_grad(x, y, 0.2, partials=pb, workspace=ws)
    assert torch.equal(ga, gb) and torch.equal(pa, pb)
    rl, rg = oloss.loss_and_grad(x.cpu().double(), y.cpu().double(), 0.2)
    assert abs(float(kernels.loss_from_partials(pb, H, W, 0.2)) - float(rl)) <= 1e-5
    assert rel_l2(gb, rg) <= 1e-4


@pytest.mark.parametrize("H,W", [(11, 13), (37, 75), (200, 300)])
def test_loss_target_stats(H, W):
    """Target statistics against the oracle's window sums of the clamped target: mu_y and
    s_y = G*y^2 - mu_y^2 per channel, each channel's planes column-major [Wo][Ho]; then the
    target itself channel-planar [3][H][W], unclamped."""
    g = torch.Generator().manual_seed(3 * H + W)
    y = torch.rand(H, W, 3, generator=g) * 1.2 - 0.1          # some values outside [0,1]
    full = kernels.loss_stats(y.cuda()).cpu()
    nst = 6 * (H - 10) * (W - 10)
    assert full.numel() == nst + 3 * H * W
    assert torch.equal(full[nst:].view(3, H, W), y.permute(2, 0, 1))
    st = full[:nst].view(2, 3, W - 10, H - 10).double()
    yc = y.double().clamp(0, 1).permute(2, 0, 1)
    gw = oloss.gauss_1d()
    mu = oloss.gaussian_filter(yc, gw)
    sy = oloss.gaussian_filter(yc * yc, gw) - mu * mu
    assert max_abs(st[0].transpose(1, 2), mu) <= 1e-6
    assert max_abs(st[1].transpose(1, 2), sy) <= 1e-6


@pytest.mark.parametrize("H,W", [(11, 11), (45, 70), (832, 1264)])
def test_loss_grad_stats_equals_combined(H, W):
    """The one-kernel entry on precomputed target statistics gives exactly what the combined
    entry (statistics into its workspace, then the same kernel) gives, call after call."""
    g = torch.Generator().manual_seed(H + 7 * W)
    x = (torch.rand(H, W, 3, generator=g) * 1.2 - 0.1).cuda()
    y = torch.rand(H, W, 3, generator=g).cuda()
    n, _ = kernels.loss_partials_count(H, W)
    pa, pb = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    ga = kernels.loss_grad(x, y, 0.2, partials=pa)
    st = kernels.loss_stats(y)
    for _ in range(2):
        gb = kernels.loss_grad_stats(x, y, st, 0.2, partials=pb)
        assert torch.equal(ga, gb) and torch.equal(pa, pb)


def test_loss_identity():
    y = torch.rand(64, 64, 3, generator=torch.Generator().manual_seed(0))
    n, _ = kernels.loss_partials_count(64, 64)
    partials = torch.empty(n, device="cuda")
    gx = kernels.loss_grad(y.cuda(), y.cuda(), 0.2, partials=partials)
    assert abs(float(kernels.loss_from_partials(partials, 64, 64))) <= 1e-5
    assert float(gx.abs().max()) <= 1e-6


def test_adam_matches_torch():
    """4 steps of the device Adam against torch.optim.Adam (fp64) on gradients whose magnitudes
    span 1e-9 .. 1, so eps = 1e-8 decides the smallest updates; eps = 1e-7 fails this test."""
    G = 1000
    g = torch.Generator().manual_seed(1)
    p0 = 0.05 * torch.randn(G, 14, generator=g)
    scale = 10.0 ** (-9.0 * torch.rand(G, 14, generator=g))
    grads = [torch.randn(G, 14, generator=g) * scale for _ in range(4)]
    lr = torch.full((14,), 1e-3)
    lr[:3] = 1.6e-4
    p = p0.cuda().clone()
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    step = kernels.adam_state("cuda")
    for gr in grads:
        kernels.adam_advance(step)
        kernels.adam(p, m, v, gr.cuda(), lr.cuda(), step)
    p64, g64 = p0.double(), [gr.double() for gr in grads]
    ref = oadam.torch_adam_reference(p64, g64, lr.double())
    assert int(step[0]) == 4
    assert update_error_ok(p, p0, ref) == 0
    ref_eps = oadam.torch_adam_reference(p64, g64, lr.double(), eps=1e-7)
    assert update_error_ok(p, p0, ref_eps) > 100


def test_geom_fwd_carries_the_step_advance():
    """geom_fwd(advance=step) advances the Adam step block exactly as adam_advance does and
    renders the same projection; without it the block is untouched."""
    cfg, P, cam = config_inputs("c1_ref")
    camb = cam.device_block("cuda")
    Pc = P.cuda()
    ref_proj, ref_keep = kernels.geom_fwd(Pc, camb)
    s1 = kernels.adam_state("cuda")
    s2 = kernels.adam_state("cuda")
    for _ in range(3):
        kernels.adam_advance(s1)
        proj, keep = kernels.geom_fwd(Pc, camb, advance=s2)
        torch.cuda.synchronize()
        assert torch.equal(s1, s2)
        assert torch.equal(proj, ref_proj) and torch.equal(keep, ref_keep)
    assert int(s2[0]) == 3
    before = s2.clone()
    kernels.geom_fwd(Pc, camb)
    torch.cuda.synchronize()
    assert torch.equal(s2, before)


def test_geom_bwd_adam_fused_equals_separate():
    """slot gather-reduce + geometry bwd + Adam in one kernel == the three separate ops."""
    cfg, P, cam = config_inputs("c1_ref")
    camb = cam.device_block("cuda")
    proj, keep = kernels.geom_fwd(P.cuda(), camb)
    inv = torch.empty(cfg.G, 9, device="cuda", dtype=torch.int32)
    idx, valid, _, _ = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, cfg.K,
                                           cfg.span, inv=inv)
    T = idx.shape[0]
    gslot = torch.randn(T, cfg.K, 9, generator=torch.Generator().manual_seed(2)).cuda()
    lr = torch.full((14,), 1e-3, device="cuda")
    # separate
    p1 = P.cuda().clone(); m1 = torch.zeros_like(p1); v1 = torch.zeros_like(p1)
    s1 = kernels.adam_state("cuda")
    gP = kernels.geom_bwd(p1, camb, kernels.slot_reduce(gslot, inv))
    kernels.adam_advance(s1)
    kernels.adam(p1, m1, v1, gP, lr, s1)
    # fused
    p2 = P.cuda().clone(); m2 = torch.zeros_like(p2); v2 = torch.zeros_like(p2)
    s2 = kernels.adam_state("cuda")
    gP2 = torch.empty_like(p2)
    kernels.adam_advance(s2)
    kernels.geom_bwd_adam(p2, camb, gslot, inv, m2, v2, lr, s2, gparams=gP2)
    assert max_abs(gP, gP2) == 0.0
    assert max_abs(p1, p2) <= 1e-6
    # the reduce equals the oracle's index_add over the valid slots
    ref = torch.zeros(cfg.G, 9, dtype=torch.float64).index_add_(
        0, idx.cpu().long().reshape(-1)[valid.cpu().reshape(-1).bool()],
        gslot.cpu().double().reshape(-1, 9)[valid.cpu().reshape(-1).bool()])
    assert rel_l2(kernels.slot_reduce(gslot, inv), ref) <= 1e-6
