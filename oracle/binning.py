"""Oracle: tile map and fixed-budget spatial-hash binning.

Test infrastructure only (see oracle/__init__.py).

Restates tools/m4_train_binned.py:60-127 (TileMap, assign_bins) with the tile side S and the
quantised-distance span as parameters (the reference hard-codes S=16, span=2048; :62, :85-86,
:109-114).  With S=16, span=2048 the `stable=False` mode is the reference computation step for
step: same pair construction order, same int64 sort key, same default `torch.argsort`.

Semantics that bit-exact binning has to reproduce:
  * cell  = clamp(int64(floor(mu/S)), 0, n-1)                      (:85-86)
  * pairs = for dy in -R..R, for dx in -R..R (stencil index j = (dy+R)*(2R+1) + dx+R),
            gaussians ascending, kept if keep[g] and the tile is inside the grid  (:92-98)
  * dist2 = fl(fl((mu_x - (tx+.5)*S)^2) + fl((mu_y - (ty+.5)*S)^2)) in fp32  (:110-113)
  * key   = tile*span + clamp(int64(dist2), 0, span-1)              (:114)
            (float->int64 follows x86 truncation: NaN or |x| >= 2^63 -> INT64_MIN)
  * order = argsort(key); first K per tile are kept, slot order = sorted order  (:115-126)
  * idx[T,K] int64 with 0 in empty slots, valid[T,K] bool          (:100-101)

`stable=True` sorts with a stable sort, i.e. by (tile, qd2, j, g): the rule the reference's
own argsort follows once the pair count reaches the parallel radix-sort threshold (32768 pairs
on this torch build), and the rule the GPU kernel implements for every size.
"""
import torch

RADIX_STABLE_MIN_PAIRS = 32768


class TileMap:
    """Tile geometry (tools/m4_train_binned.py:60-72) for S x S tiles.

    Phi[S*S,6]  monomials [lx^2, ly^2, lx*ly, lx, ly, 1] at tile-local pixel centres
    origins[T,2] (tx*S, ty*S);  gidx[T*S*S] flat image index of each (tile, pixel)."""

    def __init__(self, H, W, S=16, dtype=torch.float32):
        if H % S or W % S:
            raise ValueError(f"image {H}x{W} is not a multiple of the tile side {S}")
        self.H, self.W, self.S = H, W, S
        self.nty, self.ntx = H // S, W // S
        self.T = self.nty * self.ntx
        p = torch.arange(S * S)
        lx = (p % S).to(dtype) + 0.5
        ly = (p // S).to(dtype) + 0.5
        self.Phi = torch.stack([lx * lx, ly * ly, lx * ly, lx, ly, torch.ones_like(lx)], dim=-1)
        t = torch.arange(self.T)
        ty, tx = t // self.ntx, t % self.ntx
        self.origins = torch.stack([(tx * S).to(dtype), (ty * S).to(dtype)], dim=1)
        row = ty[:, None] * S + (p // S)[None, :]
        col = tx[:, None] * S + (p % S)[None, :]
        self.gidx = (row * W + col).reshape(-1)


def candidate_pairs(mu2d, keep, tmap, R=1):
    """(tile, gaussian, j) triples in the reference's concatenation order (:90-98)."""
    S = tmap.S
    gx = (mu2d[:, 0] / S).floor().long().clamp(0, tmap.ntx - 1)
    gy = (mu2d[:, 1] / S).floor().long().clamp(0, tmap.nty - 1)
    g_all = torch.arange(mu2d.shape[0])
    tiles, gs, js = [], [], []
    j = 0
    for dy in range(-R, R + 1):
        for dx in range(-R, R + 1):
            tx, ty = gx + dx, gy + dy
            inside = keep & (tx >= 0) & (tx < tmap.ntx) & (ty >= 0) & (ty < tmap.nty)
            tiles.append((ty * tmap.ntx + tx)[inside])
            gs.append(g_all[inside])
            js.append(torch.full((int(inside.sum()),), j, dtype=torch.long))
            j += 1
    return torch.cat(tiles), torch.cat(gs), torch.cat(js)


def quantised_dist2(mu2d, tiles, gs, tmap, span):
    """clamp(int64(dist2 to the tile centre), 0, span-1) in fp32 (:110-114)."""
    S = float(tmap.S)
    cx = ((tiles % tmap.ntx).float() + 0.5) * S
    cy = ((tiles // tmap.ntx).float() + 0.5) * S
    dx = mu2d[gs, 0] - cx
    dy = mu2d[gs, 1] - cy
    return (dx * dx + dy * dy).long().clamp(0, span - 1)


@torch.no_grad()
def assign_bins(mu2d, keep, tmap, R=1, K=128, span=2048, stable=False, return_stats=False):
    """Per-tile gaussian lists (tools/m4_train_binned.py:75-127).

    mu2d[G,2] fp32, keep[G] bool -> idx[T,K] int64 (0 where empty), valid[T,K] bool.
    With return_stats, also the per-tile candidate counts ncand[T] (before the K cut)."""
    mu2d = mu2d.detach().float().cpu()
    keep = keep.detach().bool().cpu()
    idx = torch.zeros(tmap.T, K, dtype=torch.long)
    valid = torch.zeros(tmap.T, K, dtype=torch.bool)
    tiles, gs, _ = candidate_pairs(mu2d, keep, tmap, R)
    ncand = torch.bincount(tiles, minlength=tmap.T)
    if tiles.numel() == 0:
        return (idx, valid, ncand) if return_stats else (idx, valid)
    key = tiles * span + quantised_dist2(mu2d, tiles, gs, tmap, span)
    order = torch.argsort(key, stable=True) if stable else torch.argsort(key)
    tiles, gs = tiles[order], gs[order]
    starts = torch.searchsorted(tiles.contiguous(), torch.arange(tmap.T + 1))
    rank = torch.arange(tiles.numel()) - starts[tiles]
    keepm = rank < K
    flat = tiles[keepm] * K + rank[keepm]
    idx.view(-1)[flat] = gs[keepm]
    valid.view(-1)[flat] = True
    return (idx, valid, ncand) if return_stats else (idx, valid)


@torch.no_grad()
def assign_bins_bruteforce(mu2d, keep, tmap, R=1, K=128, span=2048):
    """Independent O(T*G) statement of the stable rule, for tiny inputs: for every tile, list the
    stencil candidates, sort them by (qd2, j, g) with Python's sort, keep the first K."""
    mu2d = mu2d.detach().float().cpu()
    S = tmap.S
    idx = torch.zeros(tmap.T, K, dtype=torch.long)
    valid = torch.zeros(tmap.T, K, dtype=torch.bool)
    G = mu2d.shape[0]
    cells = []
    for g in range(G):
        cx = min(max(int(torch.floor(mu2d[g, 0] / S)), 0), tmap.ntx - 1)
        cy = min(max(int(torch.floor(mu2d[g, 1] / S)), 0), tmap.nty - 1)
        cells.append((cx, cy))
    for t in range(tmap.T):
        tx, ty = t % tmap.ntx, t // tmap.ntx
        cand = []
        for g in range(G):
            if not bool(keep[g]):
                continue
            dx, dy = tx - cells[g][0], ty - cells[g][1]
            if abs(dx) > R or abs(dy) > R:
                continue
            j = (dy + R) * (2 * R + 1) + (dx + R)
            ex = mu2d[g, 0] - torch.tensor((tx + 0.5) * S, dtype=torch.float32)
            ey = mu2d[g, 1] - torch.tensor((ty + 0.5) * S, dtype=torch.float32)
            d2 = float(ex * ex + ey * ey)
            q = min(max(int(d2), 0), span - 1)
            cand.append((q, j, g))
        cand.sort()
        for s, (_, _, g) in enumerate(cand[:K]):
            idx[t, s] = g
            valid[t, s] = True
    return idx, valid


def tie_tiles(mu2d, keep, tmap, R=1, span=2048):
    """Tiles whose candidate list has two equal (tile, qd2) keys: only there may the reference's
    non-stable argsort order differ from the stable order."""
    mu2d = mu2d.detach().float().cpu()
    keep = keep.detach().bool().cpu()
    tiles, gs, _ = candidate_pairs(mu2d, keep, tmap, R)
    key = tiles * span + quantised_dist2(mu2d, tiles, gs, tmap, span)
    uk, cnt = torch.unique(key, return_counts=True)
    return torch.unique(uk[cnt > 1] // span)
