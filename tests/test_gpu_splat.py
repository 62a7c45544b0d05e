"""GPU splat forward/backward vs the oracle.

Forward: image within 1e-4 max-abs (fp32).  Backward: parameter gradients within 1e-3 relative
L2 of torch autograd through the oracle's binned render (tools/bh_views.py:65-71 on _operands,
spike/backward.py).  The oracle runs on the GPU's own bins so both sides see the same lists.
"""
import pytest
import torch

from helpers import cam_dict, config_inputs, max_abs, rel_l2
from oracle import binning as obin
from oracle import splat as osplat
from ttsplat import binned, kernels

pytestmark = pytest.mark.gpu

GROUPS = {"means": slice(0, 3), "quats": slice(3, 7), "scales": slice(7, 10),
          "color": slice(10, 13), "opacity": slice(13, 14)}
CB = (0.2, 0.5, 0.9)   # a background colour whose three channels differ


def setup(name, G=None, k=None):
    cfg, P, cam = config_inputs(name, G=G)
    k = cfg.k if k is None else k
    camera = cam.device_block("cuda")
    proj, keep = kernels.geom_fwd(P.cuda(), camera)
    setup.inv = torch.empty(cfg.G, 9, device="cuda", dtype=torch.int32)
    idx, valid, _, _ = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, cfg.K,
                                           cfg.span, inv=setup.inv)
    bg = torch.tensor([float(torch.nn.functional.softplus(torch.tensor(-3.0))), 1.0, 1.0, 1.0],
                      device="cuda")
    bins = (idx.cpu().long(), valid.cpu().bool())
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    return cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k


@pytest.mark.parametrize("name,k", [("c1_ref", 4.0), ("c1", 9.0), ("c1_ref", 9.0), ("c3", 4.0)])
def test_splat_fwd_parity(name, k):
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup(name, k=k)
    print(f"[fwd] {name} k={k}", flush=True)
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k)
    ref, ex = osplat.render_binned(P, cam_dict(cam), tmap, K=cfg.K, k=k, bins=bins,
                                   return_all=True)
    err = max_abs(img, ref)
    print(f"[fwd] {name} k={k} max|err|={err:.3e}")
    assert err <= 1e-4
    assert max_abs(den, ex["den"]) <= 1e-4 * float(ex["den"].abs().max())


@pytest.mark.parametrize("K", [1, 30, 61])
def test_splat_fwd_ragged_budgets(K):
    """Slot budgets that are not multiples of 4 (the 16x16 forward's LDS is sized from K rounded
    up to 4, the padding slots zeroed; its waves take the slots 4 apart), down to a single slot
    per tile."""
    cfg, P, cam = config_inputs("c1_ref")
    camera = cam.device_block("cuda")
    proj, keep = kernels.geom_fwd(P.cuda(), camera)
    idx, valid, count, _ = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, K,
                                               cfg.span)
    assert int(count.max()) == K
    bg = torch.tensor([float(torch.nn.functional.softplus(torch.tensor(-3.0))), 1.0, 1.0, 1.0],
                      device="cuda")
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k)
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    ref, ex = osplat.render_binned(P, cam_dict(cam), tmap, K=K, k=cfg.k,
                                   bins=(idx.cpu().long(), valid.cpu().bool()), return_all=True)
    err = max_abs(img, ref)
    print(f"[fwd] K={K} max|err|={err:.3e}", flush=True)
    assert err <= 1e-4
    assert max_abs(den, ex["den"]) <= 1e-4 * float(ex["den"].abs().max())


@pytest.mark.parametrize("K", [128, 300])
def test_splat_fwd_holes_in_valid(K):
    """Valid masks that are not a prefix of each tile's slots (user bins): the forward stages
    slot s at LDS entry s and walks to the highest valid slot, so the holes must add nothing.
    K = 300 also takes the slots past the first 256 (a second staging pass)."""
    cfg, P, cam = config_inputs("c3")
    proj, keep = kernels.geom_fwd(P.cuda(), cam.device_block("cuda"))
    idx, valid, count, _ = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, K,
                                               cfg.span)
    gen = torch.Generator().manual_seed(5)
    holes = (torch.rand(valid.shape, generator=gen) < 0.35).to(valid.device)
    valid2 = valid & ~holes.bool()
    T = valid.shape[0]
    g = int(idx[valid.bool()][0])       # a binned (kept) gaussian
    valid2[T // 2, :] = False           # one tile whose only valid slot is the last one
    valid2[T // 2, K - 1] = True
    idx[T // 2, K - 1] = g
    bg = torch.tensor([float(torch.nn.functional.softplus(torch.tensor(-3.0))), 1.0, 1.0, 1.0],
                      device="cuda")
    img, den = kernels.splat_fwd(proj, idx, valid2, bg, cfg.H, cfg.W, cfg.S, cfg.k)
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    ref, ex = osplat.render_binned(P, cam_dict(cam), tmap, K=K, k=cfg.k,
                                   bins=(idx.cpu().long(), valid2.cpu().bool()), return_all=True)
    err = max_abs(img, ref)
    print(f"[fwd holes] K={K} max|err|={err:.3e}", flush=True)
    assert err <= 1e-4
    assert max_abs(den, ex["den"]) <= 1e-4 * float(ex["den"].abs().max())


def test_theta_gather_matches_operands():
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup("c1_ref")
    th, col, oc = kernels.theta_gather(proj, idx, valid, cfg.H, cfg.W, cfg.S, k)
    rth, rcol, roc, _, _ = osplat.operands(P, cam_dict(cam), tmap, K=cfg.K, k=k, bins=bins)
    assert max_abs(col, rcol) <= 1e-6
    assert max_abs(oc, roc[..., 0]) <= 1e-6
    # theta entries scale with the tile-local offset; compare relative to their magnitude
    assert rel_l2(th, rth) <= 1e-5


@pytest.mark.parametrize("name,k,cb", [("c1_ref", 4.0, None), ("c1", 9.0, None), ("c3", 4.0, None),
                                       ("c1_ref", 4.0, CB)])
def test_splat_bwd_param_grads(name, k, cb):
    """d(sum R*img)/dparams, GPU fused backward + geometry backward vs oracle autograd (cb: a
    background colour with three different channels)."""
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup(name, k=k)
    cbt = torch.ones(3, dtype=torch.float64) if cb is None else torch.tensor(cb, dtype=torch.float64)
    if cb is not None:
        bg = torch.tensor([float(bg[0]), *cb], device="cuda")
    print(f"[bwd] {name} k={k} cb={cb}", flush=True)
    g = torch.Generator().manual_seed(7)
    R = torch.randn(cfg.H, cfg.W, 3, generator=g)
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k)
    gwb = torch.zeros(tmap.T, device="cuda")
    gslot = kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k, img, den, R.cuda(),
                              gwb=gwb)
    grad9 = kernels.slot_reduce(gslot, setup.inv)
    # the atomic scatter (bins without an inverse table) gives the same sums
    grad9_sc = kernels.slot_scatter(gslot, idx, valid, cfg.G)
    assert rel_l2(grad9_sc, grad9) <= 1e-6
    gwb = gwb.sum()
    gP = kernels.geom_bwd(P.cuda(), camera, grad9).cpu()
    Pr = P.clone().requires_grad_(True)
    ref = osplat.render_binned(Pr, cam_dict(cam), tmap, K=cfg.K, k=k, bins=bins, c_b=cbt)
    (ref * R).sum().backward()
    for gname, sl in GROUPS.items():
        e = rel_l2(gP[:, sl], Pr.grad[:, sl])
        print(f"[bwd] {name} d{gname}: rel L2 {e:.2e}")
        assert e <= 1e-3, gname
    # dL/dw_b: autograd through the oracle with w_b as a leaf
    wb = torch.tensor(float(bg[0]), dtype=torch.float64, requires_grad=True)
    th, col, oc, _, _ = osplat.operands(P.double(), cam_dict(cam), tmap, K=cfg.K, k=k, bins=bins)
    C, _ = osplat.splat_tiles(th, col, oc, tmap.Phi.double(), wb, cbt)
    (osplat.tiles_to_image(C, tmap) * R.double()).sum().backward()
    assert abs(float(gwb) - float(wb.grad)) <= 1e-3 * abs(float(wb.grad)) + 1e-4


def test_dev_render_binned_theta_api():
    """DevRenderBinned (pre-gathered operands, the _DevRenderBinned drop-in) vs oracle autograd."""
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup("c1_ref")
    th, col, oc = kernels.theta_gather(proj, idx, valid, cfg.H, cfg.W, cfg.S, k)
    th = th.clone().requires_grad_(True)
    col = col.clone().requires_grad_(True)
    oc1 = oc[..., None].clone().requires_grad_(True)
    wb = bg[0].clone().requires_grad_(True)
    img = binned.DevRenderBinned.apply(th, col, oc1, wb, tmap.Phi, tmap.gidx, bg[1:], cfg.H, cfg.W)
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(3))
    (img * R.cuda()).sum().backward()
    # oracle
    tr = th.detach().cpu().double().requires_grad_(True)
    cr = col.detach().cpu().double().requires_grad_(True)
    orr = oc1.detach().cpu().double().requires_grad_(True)
    wr = torch.tensor(float(bg[0]), dtype=torch.float64, requires_grad=True)
    C, _ = osplat.splat_tiles(tr, cr, orr, tmap.Phi.double(), wr, torch.ones(3, dtype=torch.float64))
    ref = osplat.tiles_to_image(C, tmap)
    assert max_abs(img, ref) <= 1e-4
    (ref * R.double()).sum().backward()
    assert rel_l2(th.grad, tr.grad) <= 1e-3
    assert rel_l2(col.grad, cr.grad) <= 1e-3
    assert rel_l2(oc1.grad, orr.grad) <= 1e-3
    assert abs(float(wb.grad) - float(wr.grad)) <= 1e-3 * abs(float(wr.grad)) + 1e-4


def test_render_binned_device_autograd():
    """render_binned_device (whole chain as one autograd op) vs oracle autograd."""
    from ttsplat.model import GaussianModel
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap_o, k = setup("c1_ref")
    m = GaussianModel(P.cuda())
    m.params.requires_grad_(True)
    tmap = binned.TileMap(cfg.H, cfg.W, cfg.S)
    img, gbins = binned.render_binned_device(m, cam, tmap, K=cfg.K, return_bins=True)
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(5))
    (img * R.cuda()).sum().backward()
    Pr = P.clone().requires_grad_(True)
    ref = osplat.render_binned(Pr, cam_dict(cam), tmap_o, K=cfg.K, k=k,
                               bins=(gbins[0].cpu(), gbins[1].cpu()))
    assert max_abs(img, ref) <= 1e-4
    (ref * R).sum().backward()
    assert rel_l2(m.params.grad, Pr.grad) <= 1e-3


def test_inverse_table_matches_bins():
    """inv[g][j] lists exactly the valid slots holding g (tools/m9_scatter_oracle.py:20-32)."""
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup("c4")
    inv = setup.inv.cpu().long()
    idx_c, val_c = bins
    flat = torch.nonzero(val_c.reshape(-1)).flatten()
    ent = inv[inv >= 0]
    assert torch.equal(torch.sort(ent).values, flat)                 # every valid slot once
    g_of = idx_c.reshape(-1)[ent]
    rows = torch.nonzero(inv >= 0)[:, 0]
    assert torch.equal(g_of, rows)                                   # slot holds that gaussian
    # the stencil index: tile of the slot relative to the gaussian's cell
    S = cfg.S
    mu = proj[:, 0:2].cpu()
    cx = (mu[:, 0] / S).floor().long().clamp(0, tmap.ntx - 1)
    cy = (mu[:, 1] / S).floor().long().clamp(0, tmap.nty - 1)
    gj = torch.nonzero(inv >= 0)
    t = inv[gj[:, 0], gj[:, 1]] // cfg.K
    j = ((t // tmap.ntx) - cy[gj[:, 0]] + 1) * 3 + ((t % tmap.ntx) - cx[gj[:, 0]] + 1)
    assert torch.equal(j, gj[:, 1])


def test_backward_is_deterministic():
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup("c3")
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(9)).cuda()
    img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k)
    outs = []
    for _ in range(2):
        gslot = kernels.splat_bwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k, img, den, R)
        outs.append(kernels.geom_bwd(P.cuda(), camera, kernels.slot_reduce(gslot, setup.inv)))
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("name,variant", [("c1_ref", "tile"), ("c1", "tile"), ("c1_ref", "rec"),
                                          ("c1_ref", "mx"), ("c1_ref", "mx_bf16")])
def test_splat_fwd_coloured_background(name, variant):
    """A background colour whose channels differ (a random-background training step's draw,
    tools/resident_traced.py:671-674): every forward kernel -- the 16x16 walk from proj and from
    slot records, the 32x32 kernel, the matrix-core forward in both modes -- puts w_b c_b[c]
    into channel c's numerator."""
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup(name)
    bg = torch.tensor([float(bg[0]), *CB], device="cuda")
    print(f"[fwd-bg] {name} {variant}", flush=True)
    if variant == "tile":
        img, den = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k)
    elif variant == "rec":
        order = torch.empty(tmap.T, dtype=torch.int32, device="cuda")
        slot_rec = torch.empty(tmap.T, cfg.K, 12, device="cuda")
        pos = torch.empty(tmap.T, dtype=torch.int32, device="cuda")
        inv = torch.empty(cfg.G, 9, dtype=torch.int32, device="cuda")
        kernels.geom_fwd_assign_bins(P.cuda(), camera, cfg.H, cfg.W, cfg.S, cfg.K, cfg.span,
                                     inv=inv, order=order, slot_rec=slot_rec, pos_count=pos)
        img, den = kernels.splat_fwd_rec(slot_rec, pos, order, bg, cfg.H, cfg.W, cfg.S, k)
    else:
        img, den = kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k,
                                        bf16=variant == "mx_bf16")
    ref = osplat.render_binned(P, cam_dict(cam), tmap, K=cfg.K, k=k, bins=bins,
                               c_b=torch.tensor(CB))
    tol = 1e-2 if variant == "mx_bf16" else 1e-4
    err = max_abs(img, ref)
    print(f"[fwd-bg] {name} {variant} max|err|={err:.3e}")
    assert err <= tol
    white = osplat.render_binned(P, cam_dict(cam), tmap, K=cfg.K, k=k, bins=bins)
    assert max_abs(white, ref) > 10 * tol          # the background colour shows


@pytest.mark.parametrize("name,bf16", [("c1_ref", False), ("c3", False), ("c4", False),
                                       ("c1_ref", True), ("c3", True), ("c4", True)])
def test_splat_fwd_matrix_cores(name, bf16):
    """Matrix-core forward: fp32 mode within 1e-4 of the oracle, the bf16 render variant within
    1e-2 (the contract's two image tolerances); den likewise (relative to its scale)."""
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup(name)
    print(f"[fwd-mx] {name} bf16={bf16}", flush=True)
    img, den = kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k, bf16=bf16)
    ref, ex = osplat.render_binned(P, cam_dict(cam), tmap, K=cfg.K, k=k, bins=bins,
                                   return_all=True)
    tol = 1e-2 if bf16 else 1e-4
    err = max_abs(img, ref)
    print(f"[fwd-mx] {name} bf16={bf16} max|err|={err:.3e}")
    assert err <= tol
    assert max_abs(den, ex["den"]) <= tol * float(ex["den"].abs().max())
    # same result with a tile order
    order = kernels.tile_order(torch.randint(0, cfg.K + 1, (tmap.T,), dtype=torch.int32,
                                             device="cuda"), cfg.K)
    img2, _ = kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, k, order=order,
                                   bf16=bf16)
    assert torch.equal(img, img2)


def test_splat_fwd_matrix_cores_full_slots():
    """K = 512 with every slot of many tiles valid (16 chunks of 32), ragged last chunks."""
    cfg, P, cam = config_inputs("c4")
    proj, keep = kernels.geom_fwd(P.cuda(), cam.device_block("cuda"))
    idx, valid, count, _ = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, 512,
                                               cfg.span)
    assert int(count.max()) == 512 and int((count % 32 != 0).sum()) > 0
    bg = torch.tensor([0.05, 1.0, 1.0, 1.0], device="cuda")
    a, da = kernels.splat_fwd(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k)
    b, db = kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, cfg.S, cfg.k)
    assert max_abs(a, b) <= 1e-4
    assert max_abs(da, db) <= 1e-4 * float(da.abs().max())
    with pytest.raises(Exception):
        kernels.splat_fwd_mx(proj, idx, valid, bg, cfg.H, cfg.W, 32, cfg.k)


@pytest.mark.parametrize("name", ["c1_ref", "c3"])
def test_dev_render_binned_bf16_operands(name):
    """_DevRenderBinned as the reference has it (tools/m4_train_binned.py:42-43,154-186): theta,
    col, oc uploaded as bf16.  Image and gradients equal the fp32 formulas evaluated on the
    bf16-rounded operands (1e-4 image, 1e-3 rel L2 gradients); bf16 input tensors take the same
    path with bf16 gradients back.  The rounding of theta itself costs precision (the reference
    notes it, :36): against the fp32-operand image the oracle's own bf16 render differs by
    3.6e-2 rel L2 (max 0.86) at c1_ref and 1.3e-3 (max 0.026) at c3; bounded at 5e-2 here."""
    cfg, P, cam, camera, proj, idx, valid, bg, bins, tmap, k = setup(name)
    th, col, oc = kernels.theta_gather(proj, idx, valid, cfg.H, cfg.W, cfg.S, k)
    R = torch.randn(cfg.H, cfg.W, 3, generator=torch.Generator().manual_seed(13))
    thl, coll, ocl = (t.clone().requires_grad_(True) for t in (th, col, oc[..., None]))
    wb = bg[0].clone().requires_grad_(True)
    img = binned._DevRenderBinned.apply(thl, coll, ocl, wb, tmap.Phi, tmap.gidx, bg[1:], cfg.H,
                                        cfg.W)
    ref32 = osplat.tiles_to_image(osplat.splat_tiles(
        th.cpu().double(), col.cpu().double(), oc[..., None].cpu().double(), tmap.Phi.double(),
        torch.tensor(float(bg[0]), dtype=torch.float64), torch.ones(3, dtype=torch.float64))[0],
        tmap)
    err = rel_l2(img, ref32)
    print(f"[bf16-operands] {name} rel L2 vs fp32 operands {err:.2e}", flush=True)
    assert err <= 5e-2
    (img * R.cuda()).sum().backward()
    rb = [t.to(torch.bfloat16).cpu().double().requires_grad_(True) for t in (th, col, oc[..., None])]
    wr = torch.tensor(float(bg[0]), dtype=torch.float64, requires_grad=True)
    C, _ = osplat.splat_tiles(rb[0], rb[1], rb[2], tmap.Phi.double(), wr,
                              torch.ones(3, dtype=torch.float64))
    refb = osplat.tiles_to_image(C, tmap)
    assert max_abs(img, refb) <= 1e-4
    (refb * R.double()).sum().backward()
    for mine, ref, n in ((thl.grad, rb[0].grad, "theta"), (coll.grad, rb[1].grad, "col"),
                         (ocl.grad, rb[2].grad, "oc")):
        assert mine.dtype == torch.float32
        assert rel_l2(mine, ref) <= 1e-3, n
    # bf16 input tensors: same result, bf16 gradients
    tb = th.to(torch.bfloat16).requires_grad_(True)
    img2 = binned.DevRenderBinned.apply(tb, col.to(torch.bfloat16), oc[..., None].to(torch.bfloat16),
                                        bg[0], tmap.Phi, tmap.gidx, bg[1:], cfg.H, cfg.W)
    assert torch.equal(img2, img)
    (img2 * R.cuda()).sum().backward()
    assert tb.grad.dtype == torch.bfloat16
