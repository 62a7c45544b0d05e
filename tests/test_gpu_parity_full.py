"""The kernels the training step runs, against the oracle at the headline sizes.

G = 100k clustered, 1264x832, K = 128 (k_splat_fwd_tile, the fused k_splat_bwd, the loss kernels,
the fused geometry backward + Adam, one whole training step) and G = 1M, 1920x1072, K = 256
(the bf16 matrix-core forward over the whole frame, the fused backward on sampled tiles), the
loss at 800x800, 1264x832 and 1072x1920, and slot budgets above 256 (K = 512).  The oracle
(fp64, chunked over tiles) runs on the GPU's own bins; binning is checked bit-exact
separately.  Contract: images 1e-4 max-abs (fp32) / 1e-2 (bf16), gradients 1e-3 relative L2.
"""
import pytest
import torch

from helpers import (anisotropic, cam_dict, config_inputs, max_abs, oracle_render_chunked, rel_l2,
                     update_error_ok)
from oracle import adam as oadam
from oracle import binning as obin
from oracle import loss as oloss
from oracle import splat as osplat
from ttsplat import kernels, scenes
from ttsplat.step import TrainStep, lr_vector

pytestmark = pytest.mark.gpu

GROUPS = {"means": slice(0, 3), "quats": slice(3, 7), "scales": slice(7, 10),
          "color": slice(10, 13), "opacity": slice(13, 14)}
BG = (float(torch.nn.functional.softplus(torch.tensor(-3.0))), 1.0, 1.0, 1.0)


def gpu_scene(cfg, P, cam, K=None):
    K = cfg.K if K is None else K
    camera = cam.device_block("cuda")
    proj, keep = kernels.geom_fwd(P.cuda(), camera)
    inv = torch.empty(P.shape[0], 9, device="cuda", dtype=torch.int32)
    order = torch.empty((cfg.H // cfg.S) * (cfg.W // cfg.S), device="cuda", dtype=torch.int32)
    idx, valid, count, ncand = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, K,
                                                   cfg.span, inv=inv, order=order)
    bg = torch.tensor(BG, device="cuda")
    return camera, proj, keep, idx, valid, count, inv, order, bg


@pytest.fixture(scope="module")
def c4():
    cfg, P, cam = config_inputs("c4")
    print(f"[c4] G={cfg.G} {cfg.W}x{cfg.H} K={cfg.K}", flush=True)
    return (cfg, P, cam) + gpu_scene(cfg, P, cam)


def test_c4_forward_full_frame(c4):
    cfg, P, cam, camera, proj, keep, idx, valid, count, inv, order, bg = c4
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, order=order)
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    ref, rden = oracle_render_chunked(P, cam_dict(cam), tmap, (idx, valid), cfg.k)
    err = max_abs(img, ref)
    print(f"[c4] fwd max|err| {err:.2e}, pairs {int(count.sum()) * 256}", flush=True)
    assert err <= 1e-4
    assert max_abs(den, rden) <= 1e-4 * float(rden.abs().max())


def test_c4_backward_full_frame(c4):
    """Fused splat backward -> slot gather-reduce -> geometry backward at full size."""
    cfg, P, cam, camera, proj, keep, idx, valid, count, inv, order, bg = c4
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, order=order)
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(41))
    gslot = torch.zeros(idx.shape[0], cfg.K, 9, device="cuda")
    kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, img, den, R.cuda(),
                      gslot=gslot, order=order)
    gP = kernels.geom_bwd(P.cuda(), camera, kernels.slot_reduce(gslot, inv)).cpu()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    _, _, gref = oracle_render_chunked(P, cam_dict(cam), tmap, (idx, valid), cfg.k, R=R)
    for name, sl in GROUPS.items():
        e = rel_l2(gP[:, sl], gref[:, sl])
        print(f"[c4] d{name}: rel L2 {e:.2e}", flush=True)
        assert e <= 1e-3, name


@pytest.mark.parametrize("aniso", [False, True], ids=["fx=fy", "fx=1.13fy"])
def test_c4_training_step(c4, aniso):
    """One graph-captured training step, camera 0, against the oracle's step on the GPU's bins:
    image, loss, the gradient Adam received, and the Adam update applied to it.  Also through a
    camera with fx = 1.13 fy and an off-centre principal point."""
    cfg, P, cam = c4[:3]
    if aniso:
        cam = anisotropic(cam)
    P1 = cfg.params(seed=1)
    tg = TrainStep(P1, [cam], [torch.zeros(cfg.H, cfg.W, 3)], K=cfg.K, S=cfg.S, k=cfg.k)
    target = tg.forward(0).clone()
    ts = TrainStep(P, [cam], [target], K=cfg.K, S=cfg.S, k=cfg.k, keep_grad=True)
    ts.capture()
    ts.step(0)
    torch.cuda.synchronize()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    bins = (ts.idx.cpu(), ts.valid.cpu())
    img, _ = oracle_render_chunked(P, cam_dict(cam), tmap, bins, cfg.k)
    L, gimg = oloss.loss_and_grad(img, target.cpu().double())
    _, _, gref = oracle_render_chunked(P, cam_dict(cam), tmap, bins, cfg.k, R=gimg)
    err = max_abs(ts.image, img)
    lg = float(ts.loss())
    print(f"[c4 step aniso={aniso}] image max|err| {err:.2e}, loss {lg:.6f} vs {float(L):.6f}",
          flush=True)
    assert err <= 1e-4
    assert abs(lg - float(L)) <= 1e-5
    gP = ts.gparams.cpu()
    for name, sl in GROUPS.items():
        e = rel_l2(gP[:, sl], gref[:, sl])
        print(f"[c4 step] d{name}: rel L2 {e:.2e}", flush=True)
        assert e <= 1e-3, name
    # the update: Adam's first step on the gradient the kernel received
    Pa = P.clone().double()
    m, v = torch.zeros_like(Pa), torch.zeros_like(Pa)
    oadam.adam_step(Pa, m, v, gP.double(), lr_vector(device="cpu").double(), 1)
    assert update_error_ok(ts.P, P, Pa) == 0


@pytest.fixture(scope="module")
def c5():
    cfg = scenes.CONFIGS["c5"]
    P = cfg.params(0)
    cam = cfg.cameras()[5]
    print(f"[c5] G={cfg.G} {cfg.W}x{cfg.H} K={cfg.K}", flush=True)
    return (cfg, P, cam) + gpu_scene(cfg, P, cam)


def test_c5_forward_full_frame(c5):
    """Whole frame: the bf16 render variant within 1e-2, the fp32 forwards within
    1e-4 (the oracle takes the GPU's geometry records, so only the splat is compared)."""
    cfg, P, cam, camera, proj, keep, idx, valid, count, inv, order, bg = c5
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    pc = proj.cpu()
    pr = dict(mu2d=pc[:, 0:2], conic=pc[:, 2:5], color_o=pc[:, 6:9], o_col=pc[:, 9])
    ref, rden = oracle_render_chunked(None, None, tmap, (idx, valid), cfg.k, proj=pr)
    print(f"[c5] pairs {int(count.sum()) * 256}", flush=True)
    for name, fn, tol in (
            ("mx bf16", lambda: kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S,
                                                     cfg.k, order=order, bf16=True), 1e-2),
            ("mx fp32", lambda: kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S,
                                                     cfg.k, order=order, bf16=False), 1e-4),
            ("mf", lambda: kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k,
                                             order=order), 1e-4)):
        img, den = fn()
        err = max_abs(img, ref)
        print(f"[c5] {name} max|err| {err:.2e}", flush=True)
        assert err <= tol, name
        assert max_abs(den, rden) <= tol * float(rden.abs().max()), name


@pytest.mark.parametrize("fwd", ["fp32", "bf16"])
def test_c5_fused_backward_sampled_tiles(c5, fwd):
    """The fused backward (what the step runs) on the heaviest tiles, the tiles where the
    matrix-core and VALU forwards differ most, and random tiles: per-slot gradients of
    (a, b, c, mu_x, mu_y, col_o, o_col) against oracle autograd.  fwd = "bf16": the backward is
    fed the image and den of the bf16 matrix-core forward, as the G = 1M bf16 step runs it; its
    contract is the bf16 render's, 1e-2 (image and relative L2 of the gradients)."""
    cfg, P, cam, camera, proj, keep, idx, valid, count, inv, order, bg = c5
    T = idx.shape[0]
    tol = 1e-3 if fwd == "fp32" else 1e-2
    if fwd == "fp32":
        img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k,
                                     order=order)
    else:
        img, den = kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k,
                                        order=order, bf16=True)
    g = torch.Generator().manual_seed(43)
    R = torch.randn(cfg.H, cfg.W, 3, generator=g)
    gslot = torch.zeros(T, cfg.K, 9, device="cuda")
    kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, img, den, R.cuda(),
                      gslot=gslot, order=order)
    th, col, oc = kernels.theta_gather(proj, idx, valid, cfg.H, cfg.W, cfg.S, cfg.k)
    img2, _ = kernels.splat_fwd_theta(th, col, oc, bg, cfg.H, cfg.W, cfg.S)
    dif = (img - img2).abs().amax(-1).reshape(cfg.H // cfg.S, cfg.S, cfg.W // cfg.S, cfg.S)
    worst = torch.argsort(dif.amax((1, 3)).reshape(-1), descending=True)[:8].cpu()
    heavy = torch.argsort(count.cpu(), descending=True)[:24]
    sel = torch.cat([heavy, worst, torch.randint(0, T, (40,), generator=g)]).unique()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    pc = proj.cpu().double()
    ii, vv = idx.cpu().long()[sel], valid.cpu().bool()[sel]
    vf = vv.double()
    conic = pc[:, 2:5][ii].clone().requires_grad_(True)
    mu = pc[:, 0:2][ii].clone().requires_grad_(True)
    colo = pc[:, 6:9][ii].clone().requires_grad_(True)
    ocol = pc[:, 9][ii].clone().requires_grad_(True)
    theta = osplat.theta_u_gathered(conic, mu, tmap.origins.double()[sel], cfg.k) * vf[:, None]
    C, _ = osplat.splat_tiles(theta, colo * vf[..., None], (ocol * vf)[..., None],
                              tmap.Phi.double(), torch.tensor(BG[0], dtype=torch.float64),
                              torch.ones(3, dtype=torch.float64))
    pix = tmap.gidx.reshape(T, -1)[sel]
    mine = img.reshape(-1, 3)[pix.reshape(-1).cuda()].reshape(C.shape)
    assert max_abs(mine, C) <= (1e-4 if fwd == "fp32" else 1e-2)
    (C * R.reshape(-1, 3)[pix.reshape(-1)].reshape(C.shape).double()).sum().backward()
    gs = gslot.cpu()[sel][vv]
    for name, mine_g, ref_g in (("conic", gs[:, 0:3], conic.grad[vv]),
                                ("mean2d", gs[:, 3:5], mu.grad[vv]),
                                ("col_o", gs[:, 5:8], colo.grad[vv]),
                                ("o_col", gs[:, 8], ocol.grad[vv])):
        e = rel_l2(mine_g, ref_g)
        print(f"[c5 {fwd}] {len(sel)} tiles d{name}: rel L2 {e:.2e}", flush=True)
        assert e <= tol, name


@pytest.mark.parametrize("H,W", [(800, 800), (832, 1264), (1072, 1920)])
def test_loss_at_full_size(H, W):
    g = torch.Generator().manual_seed(H + W)
    x = torch.rand(H, W, 3, generator=g) * 1.2 - 0.1          # some values outside [0, 1]
    y = torch.rand(H, W, 3, generator=g)
    print(f"[loss] {W}x{H}", flush=True)
    partials = torch.empty(kernels.loss_partials_count(H, W)[0], device="cuda")
    gx = kernels.loss_grad(x.cuda(), y.cuda(), partials=partials)
    L = float(kernels.loss_from_partials(partials, H, W))
    Lr, gr = oloss.loss_and_grad(x.double(), y.double())
    e = rel_l2(gx, gr)
    print(f"[loss] {W}x{H}: |dL| {abs(L - float(Lr)):.2e}, grad rel L2 {e:.2e}", flush=True)
    assert abs(L - float(Lr)) <= 1e-5
    assert e <= 1e-4


def test_slot_budget_512_forward_and_backward():
    """K = 512 on a crowded small scene (G = 20k clustered on 160x160, most tiles full): the
    fused 16x16 forward, the theta forward and the oracle agree; the fused backward's
    second 256-slot prologue round gives oracle parameter gradients."""
    cfg = scenes.Config("k512", 20000, 160, 160, K=512, S=16, k=4.0, means="clustered")
    P = cfg.params(0)
    cam = cfg.cameras()[0]
    camera, proj, keep, idx, valid, count, inv, order, bg = gpu_scene(cfg, P, cam)
    full = int((count == 512).sum())
    print(f"[k512] tiles {idx.shape[0]}, full {full}, max {int(count.max())}", flush=True)
    assert full >= 10 and int(count.min()) < 512
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, order=order)
    th, col, oc = kernels.theta_gather(proj, idx, valid, cfg.H, cfg.W, cfg.S, cfg.k)
    img2, den2 = kernels.splat_fwd_theta(th, col, oc, bg, cfg.H, cfg.W, cfg.S)
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(44))
    ref, rden, gref = oracle_render_chunked(P, cam_dict(cam), tmap, (idx, valid), cfg.k, R=R)
    assert max_abs(img, ref) <= 1e-4 and max_abs(img2, ref) <= 1e-4
    assert max_abs(img, img2) <= 1e-4
    gslot = torch.zeros(idx.shape[0], 512, 9, device="cuda")
    kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, img, den, R.cuda(),
                      gslot=gslot, order=order)
    gP = kernels.geom_bwd(P.cuda(), camera, kernels.slot_reduce(gslot, inv)).cpu()
    for name, sl in GROUPS.items():
        e = rel_l2(gP[:, sl], gref[:, sl])
        print(f"[k512] d{name}: rel L2 {e:.2e}", flush=True)
        assert e <= 1e-3, name


def test_nan_covariance_poisons_its_tiles():
    """A kept gaussian with a NaN covariance has NaN theta_u, so u is NaN at every pixel of each
    tile that keeps it; torch.relu propagates NaN, so those tiles are NaN in the reference.
    Every forward kernel gives exactly that NaN set; all other pixels match the oracle, and
    gaussians that touch no NaN tile keep finite, matching gradients."""
    cfg, P, cam = config_inputs("c1_ref")
    P = P.clone()
    P[17, 7] = float("nan")
    camera, proj, keep, idx, valid, count, inv, order, bg = gpu_scene(cfg, P, cam)
    assert bool(keep[17]) and bool(torch.isnan(proj[17, 2:5]).all())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(45))
    ref, rden, gref = oracle_render_chunked(P, cam_dict(cam), tmap, (idx, valid), cfg.k, R=R)
    nan_ref = torch.isnan(ref)
    assert bool(nan_ref.any()) and not bool(nan_ref.all())
    th, col, oc = kernels.theta_gather(proj, idx, valid, cfg.H, cfg.W, cfg.S, cfg.k)
    outs = {"mf": kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k),
            "theta": kernels.splat_fwd_theta(th, col, oc, bg, cfg.H, cfg.W, cfg.S),
            "mx": kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k)}
    for name, (img, den) in outs.items():
        im = img.cpu()
        assert torch.equal(torch.isnan(im), nan_ref), name
        assert torch.equal(torch.isnan(den.cpu()), torch.isnan(rden)), name
        assert max_abs(im[~nan_ref], ref[~nan_ref]) <= 1e-4, name
    img, den = outs["mf"]
    gslot = torch.zeros(idx.shape[0], cfg.K, 9, device="cuda")
    kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k, img, den, R.cuda(),
                      gslot=gslot)
    gP = kernels.geom_bwd(P.cuda(), camera, kernels.slot_reduce(gslot, inv)).cpu()
    bad_t = torch.isnan(ref.reshape(-1, 3)[tmap.gidx].reshape(tmap.T, -1)).any(1)
    invc = inv.cpu().long()
    touches = ((invc >= 0) & bad_t[(invc // cfg.K).clamp(min=0)]).any(1)
    clean = ~touches
    # the oracle (as the reference, tools/m4_train_binned.py:207-211) gathers empty slots from
    # gaussian 0 and masks them by multiplying with valid = 0, so a NaN tile's gradient reaches
    # gaussian 0 as NaN * 0; the kernels skip empty slots.  Gaussian 0 is left out here.
    clean[0] = False
    assert bool(touches[17]) and int(clean.sum()) > 1000
    assert bool(torch.isnan(gP[17]).all())
    assert bool(torch.isfinite(gP[clean]).all()) and bool(torch.isfinite(gref[clean]).all())
    assert rel_l2(gP[clean], gref[clean]) <= 1e-3


def _fma32(a, b, c):
    """fp32 fused multiply-add on the CPU: the product is exact in fp64, then rounded once to
    fp64 and once to fp32 (overflow to +-inf and inf - inf = NaN as the hardware gives them)."""
    import numpy as np
    with np.errstate(over="ignore", invalid="ignore"):
        return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(
            np.float32)


def _nan_pixels(theta, valid, S, order):
    """[T, S*S] pixels where some valid slot's u is NaN, or so large that w = u^2 overflows
    (then C = inf/inf), with u evaluated in a kernel's own order: "tile" the 16x16 kernel's
    u = (theta1 ly + P) ly + Q, P = theta2 lx + theta4, Q = (theta0 lx + theta3) lx + theta5;
    "theta" the general kernel's fmaf chain theta0 xx + (theta1 yy + (... + (theta4 ly +
    theta5)))."""
    import numpy as np
    th = theta.cpu().numpy().astype(np.float32)                 # [T,6,K]
    p = np.arange(S * S)
    lx = (p % S + 0.5).astype(np.float32)[None, :, None]
    ly = (p // S + 0.5).astype(np.float32)[None, :, None]
    t = [th[:, f, None, :] for f in range(6)]                   # [T,1,K] each
    f = _fma32
    if order == "tile":
        P = f(t[2], lx, t[4])
        Q = f(f(t[0], lx, t[3]), lx, t[5])
        u = f(f(t[1], ly, P), ly, Q)
    else:
        u = f(t[0], lx * lx, f(t[1], ly * ly, f(t[2], lx * ly, f(t[3], lx, f(t[4], ly, t[5])))))
    with np.errstate(invalid="ignore"):
        bad = (np.isnan(u) | (u > 1.8446743e19)) & valid.cpu().numpy().astype(bool)[:, None, :]
    return torch.from_numpy(bad.any(-1))


def test_overflowing_theta_terms_follow_torch_relu():
    """A gaussian with a finite theta whose terms overflow: conic a = -3e38, c = 3e38, b = 0 at
    k = 1, mean at the origin of tile (3, 2) (G = 2000, 128 x 128).  There theta0 = 3e38,
    theta1 = -3e38; in the neighbouring tiles the folded mean overflows theta3..5 to infinities.
    torch.relu keeps NaN and maps -inf to 0, so a pixel is NaN wherever u is NaN (or w = u^2
    overflows).  Where theta itself holds infinities of both signs, u is NaN at every pixel in
    any order of evaluation: those tiles are NaN whole, in every kernel.  Where only finite terms
    overflow, NaN, +inf or -inf depends on the order of the sum (torch's own on its BLAS); each
    kernel's NaN pixels are then those its own order gives, emulated on the CPU (the matrix-core
    kernel's internal order is the hardware's and is not checked there).  Tiles without a slot
    that can overflow match the fp64 oracle; the backward writes NaN gradients for every kept
    slot of a tile with a NaN pixel and the oracle's gradients elsewhere."""
    cfg, P, cam = config_inputs("c1_ref")
    k, bad = 1.0, 5
    camera = cam.device_block("cuda")
    proj, keep = kernels.geom_fwd(P.cuda(), camera)
    row = proj[bad].clone()
    row[0:5] = torch.tensor([48.0, 32.0, -3e38, 0.0, 3e38])
    proj[bad] = row
    keep[bad] = 1
    T = (cfg.H // cfg.S) * (cfg.W // cfg.S)
    inv = torch.empty(cfg.G, 9, device="cuda", dtype=torch.int32)
    order = torch.empty(T, device="cuda", dtype=torch.int32)
    idx, valid, count, ncand = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, cfg.K,
                                                   cfg.span, inv=inv, order=order)
    bg = torch.tensor(BG, device="cuda")
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    pc = proj.cpu()
    pr = dict(mu2d=pc[:, 0:2], conic=pc[:, 2:5], color_o=pc[:, 6:9], o_col=pc[:, 9])
    ref64, _ = oracle_render_chunked(None, None, tmap, (idx, valid), k, proj=pr)
    th, col, oc = kernels.theta_gather(proj, idx, valid, cfg.H, cfg.W, cfg.S, k)
    thc, vv = th.cpu(), valid.cpu().bool()
    with torch.no_grad():
        mag = thc.abs().amax(1)                                    # [T,K]
        wild_slot = (~(mag < 1e34) | torch.isnan(thc.sum(1))) & vv
        poison_slot = torch.isnan(thc.sum(1)) & vv
    wild, poison = wild_slot.any(1), poison_slot.any(1)
    print(f"[overflow] wild tiles {wild.nonzero().flatten().tolist()}, poisoned "
          f"{poison.nonzero().flatten().tolist()}", flush=True)
    assert int(poison.sum()) >= 2 and int((wild & ~poison).sum()) >= 1
    gidx = tmap.gidx.reshape(T, -1)

    def per_tile(img):
        return img.reshape(-1, 3)[gidx.reshape(-1)].reshape(T, -1, 3)

    r64 = per_tile(ref64)
    outs = {"tile": kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k, order=order),
            "theta": kernels.splat_fwd_theta(th, col, oc, bg, cfg.H, cfg.W, cfg.S),
            "mx": kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k,
                                       order=order)}
    for name, (img, den) in outs.items():
        im = per_tile(img.cpu())
        nan_gpu = torch.isnan(im).any(-1)                          # [T, 256]
        assert bool(nan_gpu[poison].all()), name                   # any order: NaN whole
        assert not bool(nan_gpu[~wild].any()), name
        assert max_abs(im[~wild], r64[~wild]) <= 1e-4, name
        if name != "mx":
            want = _nan_pixels(th, valid, cfg.S, name)
            part = want[wild & ~poison]
            assert bool(part.any()) and not bool(part.all())    # per-pixel NaN exercised
            print(f"[overflow] {name}: NaN pixels in wild tiles {int(nan_gpu[wild].sum())}, "
                  f"its order gives {int(want[wild].sum())}", flush=True)
            assert torch.equal(nan_gpu[wild], want[wild]), name
    img, den = outs["tile"]
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(46))
    gslot = torch.zeros(T, cfg.K, 9, device="cuda")
    kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k, img, den, R.cuda(),
                      gslot=gslot, order=order)
    gs = gslot.cpu()
    nan_tile = torch.isnan(per_tile(img.cpu())).any(-1).any(-1)
    assert bool(torch.isnan(gs[nan_tile][vv[nan_tile]]).all())
    clean = ~nan_tile
    assert bool(torch.isfinite(gs[clean][vv[clean]]).all())
    # the clean tiles' slot gradients against fp64 oracle autograd (no overflow there)
    ii = idx.cpu().long()[clean]
    vf = vv[clean].double()
    pd = pc.double()
    conic = pd[:, 2:5][ii].clone().requires_grad_(True)
    mu = pd[:, 0:2][ii].clone().requires_grad_(True)
    colo = pd[:, 6:9][ii].clone().requires_grad_(True)
    ocol = pd[:, 9][ii].clone().requires_grad_(True)
    theta = osplat.theta_u_gathered(conic, mu, tmap.origins.double()[clean], k) * vf[:, None]
    C, _ = osplat.splat_tiles(theta, colo * vf[..., None], (ocol * vf)[..., None],
                              tmap.Phi.double(), torch.tensor(BG[0], dtype=torch.float64),
                              torch.ones(3, dtype=torch.float64))
    pix = gidx[clean]
    (C * R.reshape(-1, 3)[pix.reshape(-1)].reshape(C.shape).double()).sum().backward()
    gc = gs[clean][vv[clean]]
    for name, mine_g, ref_g in (("conic", gc[:, 0:3], conic.grad[vv[clean]]),
                                ("mean2d", gc[:, 3:5], mu.grad[vv[clean]]),
                                ("col_o", gc[:, 5:8], colo.grad[vv[clean]]),
                                ("o_col", gc[:, 8], ocol.grad[vv[clean]])):
        assert rel_l2(mine_g, ref_g) <= 1e-3, name
