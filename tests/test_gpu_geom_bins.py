"""tts_geom_fwd_assign_bins (geometry forward + binning as one call; the binning's count pass
runs inside the geometry launch, in blocks of 512 gaussians up to G = 131072 and of 4096 above)
against tts_geom_fwd_ex followed by
tts_assign_bins on the same inputs: proj, keep, bins, counts and the inverse table equal bit for
bit; the tile order is a heaviest-first permutation either way (ties in no fixed order).  The
fused call also writes the slot records: slot_rec[p][s] = proj[idx[order[p]][s]] for every kept
slot and pos_count[p] = count[order[p]]."""
import dataclasses

import pytest
import torch

from helpers import config_inputs
from ttsplat import kernels

pytestmark = pytest.mark.gpu


def two_ways(cfg, P, cam, **kw):
    dev = "cuda"
    camera = cam.device_block(dev)
    T = (cfg.H // cfg.S) * (cfg.W // cfg.S)
    G = P.shape[0]
    outs = []
    for fused in (False, True):
        adv = None
        if kw.get("advance"):
            adv = torch.zeros(4, dtype=torch.int32, device=dev)
        inv = torch.full((G, 9), -7, dtype=torch.int32, device=dev)
        order = torch.empty(T, dtype=torch.int32, device=dev)
        gkw = dict(sh_rest=kw.get("sh_rest"), sh_degree=kw.get("sh_degree", 0),
                   depth_bt=kw.get("depth_bt"), advance=adv)
        rec = pos = None
        if fused:
            rec = torch.full((T, cfg.K, 12), float("nan"), device=dev)
            pos = torch.full((T,), -1, dtype=torch.int32, device=dev)
            proj, keep, idx, valid, count, ncand = kernels.geom_fwd_assign_bins(
                P, camera, cfg.H, cfg.W, cfg.S, cfg.K, cfg.span, inv=inv, order=order,
                slot_rec=rec, pos_count=pos, **gkw)
        else:
            proj, keep = kernels.geom_fwd(P, camera, **gkw)
            idx, valid, count, ncand = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W,
                                                           cfg.S, cfg.K, cfg.span, inv=inv,
                                                           order=order)
        torch.cuda.synchronize()
        outs.append(dict(proj=proj, keep=keep, idx=idx, valid=valid, count=count, ncand=ncand,
                         inv=inv, order=order, adv=adv, rec=rec, pos=pos))
    return outs


def check_equal(a, b, K):
    for k in ("proj", "keep", "idx", "valid", "count", "ncand", "inv"):
        assert torch.equal(a[k], b[k]), k
    if a["adv"] is not None:
        assert torch.equal(a["adv"], b["adv"])
    T = a["count"].numel()
    for o in (a["order"], b["order"]):
        ol = o.long()
        assert torch.equal(torch.sort(ol).values, torch.arange(T, device=ol.device))
        kept = a["count"].long()[ol]
        assert bool((kept[1:] <= kept[:-1]).all())
    check_records(b)


def check_records(o):
    """Slot records of the fused call against proj gathered through its own bins and order."""
    ol = o["order"].long()
    assert torch.equal(o["pos"], o["count"][ol])
    kept = o["valid"].bool()[ol]                       # [T, K] by dispatch position
    assert torch.equal(kept.sum(1).int(), o["pos"])   # the kept slots are a prefix
    want = o["proj"][o["idx"].long()[ol]]              # [T, K, 12]
    assert torch.equal(o["rec"][kept], want[kept])


@pytest.mark.parametrize("name,G", [("c4", None), ("c3", None), ("c1_ref", None), ("c3", 1),
                                    ("c3", 257), ("c3", 511), ("c3", 513), ("c4", 131073),
                                    ("c4", 150000), ("c4", 300017)])
def test_geom_fwd_assign_bins_equals_two_calls(name, G):
    cfg, P, cam = config_inputs(name, G=G)
    print(f"[geom+bins] {name} G={cfg.G}", flush=True)
    a, b = two_ways(cfg, P.cuda(), cam)
    check_equal(a, b, cfg.K)


@pytest.mark.parametrize("K", [256, 512])
def test_geom_fwd_assign_bins_records_large_k(K):
    # K > 128: the select places survivors by groups (heavy and light tiles)
    cfg, P, cam = config_inputs("c4", G=100000)
    cfg = dataclasses.replace(cfg, K=K)
    print(f"[geom+bins] c4 K={K}", flush=True)
    a, b = two_ways(cfg, P.cuda(), cam)
    check_equal(a, b, cfg.K)


@pytest.mark.parametrize("G", [60000, 140000])
def test_geom_fwd_assign_bins_sh_depth_weight_advance(G):
    cfg, P, cam = config_inputs("c4", G=G)
    print(f"[geom+bins] c4 SH-3 depth weight G={G}", flush=True)
    gen = torch.Generator().manual_seed(4)
    rest = torch.randn(cfg.G, 15, 3, generator=gen) * 0.1
    bt = torch.tensor([1.5, 4.0], device="cuda")
    a, b = two_ways(cfg, P.cuda(), cam, sh_rest=kernels.sh_rest_layout(rest.cuda()),
                    sh_degree=3, depth_bt=bt, advance=True)
    check_equal(a, b, cfg.K)
    assert int(a["adv"][0]) == 1


@pytest.mark.parametrize("G", [5000, 140000])
def test_geom_fwd_assign_bins_largest_grid(G):
    """The largest grid the binning takes, 38912 tiles (4096 x 2432 at S = 16): the fused
    launch's count histogram is then largest (4608 + 4 * 38912 = 160256 bytes of LDS with blocks
    of 512 gaussians, 4 * 38912 = 155648 with blocks of 4096), and the fused call equals the two
    calls."""
    from ttsplat import scenes
    cfg = scenes.Config("grid38912", G, 2432, 4096, K=128, S=16, k=4.0)
    P, cam = cfg.params(0), cfg.cameras()[0]
    assert (cfg.H // 16) * (cfg.W // 16) == 38912
    print(f"[geom+bins] {cfg.W}x{cfg.H} G={cfg.G}", flush=True)
    a, b = two_ways(cfg, P.cuda(), cam)
    check_equal(a, b, cfg.K)


@pytest.mark.parametrize("name,G", [("c4", None), ("c1_ref", 700), ("c3", 131072)])
def test_step_seam_equals_backward_then_forward_binning(name, G):
    """The step seam -- tts_geom_bwd_adam_fwd_count (step i's geometry backward + Adam, step
    i+1's geometry forward and count pass in one launch), then tts_assign_bins_counted (the
    rest of the binning, carrying step i+1's Adam step advance) -- against tts_geom_bwd_adam
    followed by tts_geom_fwd_assign_bins with the advance: params, m, v, the step block, the
    next view's proj, keep, bins, counts and inverse table bit for bit; the tile order a
    heaviest-first permutation and the slot records those of the bins in that order.  G = 700
    leaves the last block's second half empty; G = 131072 is the largest G the seam takes."""
    from helpers import anisotropic
    cfg, P, cam = config_inputs(name, G=G)
    dev = "cuda"
    G = P.shape[0]
    T = (cfg.H // cfg.S) * (cfg.W // cfg.S)
    cam_b, cam_f = cam.device_block(dev), anisotropic(cam).device_block(dev)
    print(f"[seam] {name} G={G}", flush=True)
    gen = torch.Generator().manual_seed(9)
    P0 = P.cuda()
    m0 = (0.01 * torch.randn(G, 14, generator=gen)).cuda()
    v0 = (1e-4 * torch.rand(G, 14, generator=gen)).cuda()
    lr = torch.full((14,), 1e-3, device=dev)
    lr[:3] = 1.6e-4
    inv_b = torch.empty(G, 9, dtype=torch.int32, device=dev)    # step i's bins (camera b)
    kernels.geom_fwd_assign_bins(P0, cam_b, cfg.H, cfg.W, cfg.S, cfg.K, cfg.span, inv=inv_b)
    gslot = torch.randn(T, cfg.K, 9, generator=gen).cuda() * 1e-3
    outs = []
    for seam in (False, True):
        Pw, m, v = P0.clone(), m0.clone(), v0.clone()
        step = kernels.adam_state(dev)
        kernels.adam_advance(step)                                # step i's advance
        inv = torch.full((G, 9), -7, dtype=torch.int32, device=dev)
        order = torch.empty(T, dtype=torch.int32, device=dev)
        rec = torch.full((T, cfg.K, 12), float("nan"), device=dev)
        pos = torch.full((T,), -1, dtype=torch.int32, device=dev)
        idx = torch.empty(T, cfg.K, dtype=torch.int32, device=dev)
        valid = torch.empty(T, cfg.K, dtype=torch.uint8, device=dev)
        count = torch.empty(T, dtype=torch.int32, device=dev)
        ncand = torch.empty(T, dtype=torch.int32, device=dev)
        proj = torch.empty(G, 12, device=dev)
        keep = torch.empty(G, dtype=torch.uint8, device=dev)
        if seam:
            ws = kernels.geom_bwd_adam_fwd_count(Pw, cam_b, cam_f, gslot, inv_b, m, v, lr, step,
                                                 proj, keep, cfg.H, cfg.W, cfg.S, cfg.K,
                                                 cfg.span)
            kernels.assign_bins_counted(proj, keep, cfg.H, cfg.W, cfg.S, cfg.K, cfg.span, ws,
                                        idx, valid, count, ncand, inv=inv, order=order,
                                        slot_rec=rec, pos_count=pos, advance=step)
        else:
            kernels.geom_bwd_adam(Pw, cam_b, gslot, inv_b, m, v, lr, step)
            kernels.geom_fwd_assign_bins(Pw, cam_f, cfg.H, cfg.W, cfg.S, cfg.K, cfg.span,
                                         proj=proj, keep=keep, advance=step, idx=idx,
                                         valid=valid, count=count, ncand=ncand, inv=inv,
                                         order=order, slot_rec=rec, pos_count=pos)
        torch.cuda.synchronize()
        outs.append(dict(P=Pw, m=m, v=v, step=step, proj=proj, keep=keep, idx=idx, valid=valid,
                         count=count, ncand=ncand, inv=inv, order=order, rec=rec, pos=pos))
    a, b = outs
    for k in ("P", "m", "v", "step", "proj", "keep", "idx", "valid", "count", "ncand", "inv"):
        assert torch.equal(a[k], b[k]), k
    assert int(b["step"][0]) == 2
    assert not torch.equal(b["P"], P0)
    ol = b["order"].long()
    assert torch.equal(torch.sort(ol).values, torch.arange(T, device=ol.device))
    kept = b["count"].long()[ol]
    assert bool((kept[1:] <= kept[:-1]).all())
    assert torch.equal(b["pos"].long(), kept)
    s = torch.arange(cfg.K, device=dev)
    live = s[None, :] < kept[:, None]                             # [T(p), K]
    want = b["proj"][b["idx"].long()[ol]]                         # [T(p), K, 12]
    assert torch.equal(b["rec"][live], want[live])


def test_step_seam_refuses_large_g():
    cfg, P, cam = config_inputs("c4", G=131073)
    camera = cam.device_block("cuda")
    with pytest.raises(ValueError):
        kernels.geom_bwd_adam_fwd_count(P.cuda(), camera, camera, torch.zeros(1, 1, 9, device="cuda"),
                                        torch.zeros(cfg.G, 9, dtype=torch.int32, device="cuda"),
                                        torch.zeros(cfg.G, 14, device="cuda"),
                                        torch.zeros(cfg.G, 14, device="cuda"),
                                        torch.zeros(14, device="cuda"),
                                        kernels.adam_state("cuda"),
                                        torch.empty(cfg.G, 12, device="cuda"),
                                        torch.empty(cfg.G, dtype=torch.uint8, device="cuda"),
                                        cfg.H, cfg.W)
