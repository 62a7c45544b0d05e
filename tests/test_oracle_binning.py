"""Pin the binning oracle (CPU).

  * golden vectors written by the reference's own assign_bins (tests/golden/bins_reference.npz,
    made by tests/golden/make_bins_fixtures.py): the oracle's reference-order mode must equal
    them bit for bit on every case, including c1's non-stable (introsort) order;
  * the oracle's stable mode equals them where the reference sort is the stable radix sort
    (>= 32768 pairs) and differs only in tiles with a quantised-key tie below that;
  * an independent O(T*G) brute force of the (qd2, j, g) rule on tiny inputs;
  * structural invariants.
"""
import hashlib
import math
import os

import numpy as np
import pytest
import torch

from oracle import binning as obin

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bins_reference.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def _case(z, name):
    H, W, K = (int(v) for v in z[f"{name}_shape"])
    mu = torch.from_numpy(z[f"{name}_mu2d"])
    keep = torch.from_numpy(z[f"{name}_keep"])
    return mu, keep, H, W, K


def _digest(idx, valid):
    h = hashlib.sha256()
    h.update(np.ascontiguousarray(idx.numpy().astype("<i8")).tobytes())
    h.update(np.ascontiguousarray(valid.numpy().astype(np.uint8)).tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("name", ["c1_ref", "edge", "c3", "c4"])
def test_reference_order_equals_golden(golden, name):
    mu, keep, H, W, K = _case(golden, name)
    tmap = obin.TileMap(H, W, 16)
    idx, valid = obin.assign_bins(mu, keep, tmap, 1, K, stable=False)
    assert _digest(idx, valid) == str(golden[f"{name}_sha256"])
    assert np.array_equal(valid.sum(1).numpy(), golden[f"{name}_count"])
    if f"{name}_idx" in golden:
        assert np.array_equal(idx.numpy(), golden[f"{name}_idx"].astype(np.int64))
        assert np.array_equal(valid.numpy(), golden[f"{name}_valid"])


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_stable_order_equals_golden_above_radix_threshold(golden, name):
    mu, keep, H, W, K = _case(golden, name)
    tmap = obin.TileMap(H, W, 16)
    _, _, ncand = obin.assign_bins(mu, keep, tmap, 1, K, stable=True, return_stats=True)
    assert int(ncand.sum()) >= obin.RADIX_STABLE_MIN_PAIRS
    idx, valid = obin.assign_bins(mu, keep, tmap, 1, K, stable=True)
    assert _digest(idx, valid) == str(golden[f"{name}_sha256"])


def test_stable_order_differs_only_in_tie_tiles_below_threshold(golden):
    mu, keep, H, W, K = _case(golden, "c1_ref")
    tmap = obin.TileMap(H, W, 16)
    idx, valid = obin.assign_bins(mu, keep, tmap, 1, K, stable=True)
    ref_idx = torch.from_numpy(golden["c1_ref_idx"].astype(np.int64))
    ref_valid = torch.from_numpy(golden["c1_ref_valid"])
    differ = ((idx != ref_idx).any(1) | (valid != ref_valid).any(1)).nonzero().flatten()
    ties = set(obin.tie_tiles(mu, keep, tmap).tolist())
    assert set(differ.tolist()) <= ties
    # the kept SET differs only where a tie straddles the K-th slot
    for t in differ.tolist():
        a = set(idx[t][valid[t]].tolist())
        b = set(ref_idx[t][ref_valid[t]].tolist())
        if a != b:
            tiles, gs, _ = obin.candidate_pairs(mu, keep, tmap)
            q = obin.quantised_dist2(mu, tiles, gs, tmap, 2048)
            qt = torch.sort(q[tiles == t]).values
            assert qt[K - 1] == qt[K], f"tile {t}: kept sets differ without a tie at slot K"


@pytest.mark.parametrize("S,K,seed", [(16, 4, 0), (16, 3, 1), (32, 5, 2), (16, 16, 3)])
def test_stable_equals_bruteforce(S, K, seed):
    g = torch.Generator().manual_seed(seed)
    H, W, G = 3 * S, 4 * S, 60
    mu = torch.rand(G, 2, generator=g) * torch.tensor([W + 40.0, H + 40.0]) - 20
    mu[:8] = mu[8]                                  # duplicates -> exact key ties
    mu[10:14] = (torch.randint(0, 4, (4, 2), generator=g) * S).float()   # on tile edges
    keep = torch.rand(G, generator=g) > 0.15
    tmap = obin.TileMap(H, W, S)
    span = 2048 if S == 16 else 8192
    a = obin.assign_bins(mu, keep, tmap, 1, K, span=span, stable=True)
    b = obin.assign_bins_bruteforce(mu, keep, tmap, 1, K, span=span)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_candidate_pairs_stencil_order():
    """The pair list is stencil-major (j = (dy+R)(2R+1) + dx+R ascending, dy outer, dx inner),
    gaussians ascending within one j, each pair's tile = cell + (dx, dy) inside the grid
    (tools/m4_train_binned.py:90-98), at R = 1 and R = 2."""
    g = torch.Generator().manual_seed(5)
    S, H, W, G = 16, 80, 112, 70
    mu = torch.rand(G, 2, generator=g) * torch.tensor([W + 30.0, H + 30.0]) - 15
    keep = torch.rand(G, generator=g) > 0.2
    tmap = obin.TileMap(H, W, S)
    for R in (1, 2):
        tiles, gs, js = obin.candidate_pairs(mu, keep, tmap, R)
        want = []
        for j in range((2 * R + 1) ** 2):
            dy, dx = j // (2 * R + 1) - R, j % (2 * R + 1) - R
            for gi in range(G):
                cx = min(max(int(math.floor(float(mu[gi, 0]) / S)), 0), tmap.ntx - 1)
                cy = min(max(int(math.floor(float(mu[gi, 1]) / S)), 0), tmap.nty - 1)
                tx, ty = cx + dx, cy + dy
                if bool(keep[gi]) and 0 <= tx < tmap.ntx and 0 <= ty < tmap.nty:
                    want.append((ty * tmap.ntx + tx, gi, j))
        got = list(zip(tiles.tolist(), gs.tolist(), js.tolist()))
        assert got == want


def test_invariants(golden):
    mu, keep, H, W, K = _case(golden, "c3")
    tmap = obin.TileMap(H, W, 16)
    idx, valid, ncand = obin.assign_bins(mu, keep, tmap, 1, K, stable=True, return_stats=True)
    assert torch.equal(valid.sum(1), ncand.clamp(max=K))
    assert int(idx[~valid].abs().sum()) == 0                      # empty slots hold 0
    per_g = torch.bincount(idx[valid], minlength=mu.shape[0])
    assert int(per_g.max()) <= 9                                  # R = 1: at most 9 tiles
    assert int(per_g[~keep].sum()) == 0                           # culled never binned
    # valid slots form a prefix of each tile row
    assert torch.equal(valid, torch.arange(K)[None, :] < valid.sum(1, keepdim=True))


def test_float_to_int64_semantics():
    """Non-finite and huge distances quantise through x86 truncation (INT64_MIN) then clamp:
    the GPU kernel reproduces exactly this."""
    x = torch.tensor([float("inf"), float("-inf"), float("nan"), 1e30, 3.9, -0.0])
    assert x.long().tolist()[:4] == [-2 ** 63] * 4
    assert x.long().clamp(0, 2047).tolist() == [0, 0, 0, 0, 3, 0]


def test_tilemap_layout():
    """tools/m4_train_binned.py:60-72: Phi at tile-local centres, row-major tiles and pixels."""
    tm = obin.TileMap(32, 48, 16)
    assert tm.T == 6 and tm.Phi.shape == (256, 6)
    assert torch.equal(tm.Phi[17], torch.tensor([1.5 ** 2, 1.5 ** 2, 2.25, 1.5, 1.5, 1.0]))
    assert torch.equal(tm.origins[4], torch.tensor([16.0, 16.0]))
    assert int(tm.gidx[4 * 256 + 17]) == (16 + 1) * 48 + 16 + 1
    assert torch.equal(torch.sort(tm.gidx).values, torch.arange(32 * 48))
