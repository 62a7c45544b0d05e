"""tts_assign_bins_noalloc (binning on the library's fixed device scratch, no allocation) against
tts_assign_bins on a caller workspace: every output bit-identical, on two calls in a row, the
second on a smaller scene (the scratch then holds the first call's state), plus the host-side
refusal of sizes beyond the scratch."""
import ctypes

import pytest
import torch

from helpers import config_inputs
from ttsplat import _lib, kernels

pytestmark = pytest.mark.gpu

TTS_ESCRATCH = -9


def _outputs(T, K, G, dev):
    return dict(idx=torch.full((T, K), -7, device=dev, dtype=torch.int32),
                valid=torch.full((T, K), 3, device=dev, dtype=torch.uint8),
                count=torch.full((T,), -7, device=dev, dtype=torch.int32),
                ncand=torch.full((T,), -7, device=dev, dtype=torch.int32),
                inv=torch.full((G, 9), -7, device=dev, dtype=torch.int32),
                order=torch.full((T,), -7, device=dev, dtype=torch.int32))


def _noalloc(mu, keep, cfg, out):
    P = _lib.ptr
    _lib.call("tts_assign_bins_noalloc", P(mu), mu.stride(0), P(keep), 1, mu.shape[0], cfg.H,
              cfg.W, cfg.S, 1, cfg.K, cfg.span, P(out["idx"]), P(out["valid"]), P(out["count"]),
              P(out["ncand"]), P(out["inv"]), P(out["order"]), _lib.stream())


def _check(name):
    cfg, P, cam = config_inputs(name)
    dev = torch.device("cuda:0")
    print(f"[noalloc] {name} G={cfg.G} {cfg.H}x{cfg.W} S={cfg.S} K={cfg.K}", flush=True)
    proj, keep = kernels.geom_fwd(P.to(dev), cam.device_block(dev))
    mu = proj[:, 0:2]
    T = (cfg.H // cfg.S) * (cfg.W // cfg.S)
    ref = _outputs(T, cfg.K, cfg.G, dev)
    kernels.assign_bins(mu, keep, cfg.H, cfg.W, cfg.S, cfg.K, cfg.span, idx=ref["idx"],
                        valid=ref["valid"], count=ref["count"], ncand=ref["ncand"],
                        inv=ref["inv"], order=ref["order"])
    got = _outputs(T, cfg.K, cfg.G, dev)
    _noalloc(mu, keep, cfg, got)
    torch.cuda.synchronize()
    for key in ("idx", "valid", "count", "ncand", "inv"):
        assert torch.equal(got[key], ref[key]), f"{name}: {key} differs"
    # order: tiles by kept count, heaviest first, ties in no particular order (both entry
    # points): the same permutation up to the order inside each equal-count run
    cnt = ref["count"].long()
    for o in (ref["order"], got["order"]):
        assert torch.equal(torch.sort(o.long()).values, torch.arange(T, device=dev))
        assert bool((cnt[o.long()][1:] <= cnt[o.long()][:-1]).all())
    assert torch.equal(cnt[got["order"].long()], cnt[ref["order"].long()])
    return int(ref["ncand"].sum())


def test_noalloc_matches_workspace_entry_twice():
    pairs_big = _check("c4")        # G = 100k, 1264 x 832
    pairs_small = _check("c1_ref")  # G = 2000, 128 x 128: the scratch holds c4's state
    assert pairs_big > pairs_small > 0


def test_noalloc_refuses_sizes_beyond_scratch():
    lib = _lib.load()
    dev = torch.device("cuda:0")
    G, H, W = 1 << 21, 2048, 2048
    assert lib.tts_bin_workspace_bytes(G, H, W, 16) > (40 << 20)
    mu = torch.zeros(4, 2, device=dev)
    keep = torch.zeros(4, device=dev, dtype=torch.uint8)
    idx = torch.zeros(4, device=dev, dtype=torch.int32)
    valid = torch.zeros(4, device=dev, dtype=torch.uint8)
    P = _lib.ptr
    # refused on the host before any launch (the claimed G and image never reach a kernel)
    rc = lib.tts_assign_bins_noalloc(P(mu), 2, P(keep), 1, G, H, W, 16, 1, 128, 2048, P(idx),
                                     P(valid), None, None, None, None, _lib.stream())
    assert rc == TTS_ESCRATCH
    assert b"scratch" in lib.tts_strerror(rc)
    assert ctypes.c_int(rc).value == TTS_ESCRATCH
