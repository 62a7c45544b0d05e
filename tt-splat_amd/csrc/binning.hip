// Fixed-budget spatial-hash binning (R = 1) in O(G + pairs), bit-exact with the reference
// order of tools/m4_train_binned.py:75-127.
//
// Every candidate (tile t, gaussian g reaching t through stencil index j) has the unique
// 64-bit key  qd2 << 36 | j << 32 | g  with qd2 = clamp(int64(fl(fl(dx*dx) + fl(dy*dy))), 0,
// span-1) measured from the tile centre.  Ascending key order IS the reference order (its int64
// sort key tile*span + qd2, ties in pair-concatenation order (j, g)); each tile keeps its K
// smallest keys.
//
// Far gaussians.  A kept gaussian whose centre lies off the image is clamped into a border cell
// (tools/m4_train_binned.py:85-86).  When its key is saturated (qd2 = span-1) for every tile its
// cell reaches, it is "far": its keys in all those tiles are (span-1, j, g), known without
// touching it.  Crowded scenes put tens of thousands of such gaussians into corner cells, so
// far gaussians are stored apart (their ids only) and tiles count them from the cell totals;
// only the selection among saturated ties ever reads them, and then only one cell's list.
//
// Passes (stream-ordered, no host round trip, no global atomics):
//   1. k_bin_count      cell and far flag of each gaussian; per-block LDS histograms written as
//                       one row per block of a count matrix [block][cell | border cell]; each
//                       regular gaussian's rank in its cell inside the block, each far
//                       gaussian's rank among its block's far gaussians of the cell, in g order.
//   2. k_bin_colscan    per column of the matrix, the exclusive scan over blocks (each block's
//                       base in the cell) and the column total; totals' prefix inside 64-cell
//                       chunks and the chunk totals.
//   3. k_bin_scatter    cell_start[T+1], far_start[T+1] from the chunk prefixes; regular
//                       gaussians -> (g, mu_x, mu_y) records, far -> g at their ranks: every
//                       cell's far ids end up ascending.  Its first blocks classify the tiles (a
//                       tile's candidates are the 3x3 box sum of the cell totals) into the heavy
//                       and light lists, and record per block how many tiles take each order
//                       key (K - kept count) and each tile's rank among them.
//   4. k_bin_select     one block per tile (below); it also writes the tile's slot of the
//                       heaviest-first order, from those per-block key counts, and (when
//                       asked) the slot records: each kept gaussian's proj record at the
//                       tile's place in that order.
// The result does not depend on the order atomics land in.

#include <mutex>

#include "bin_count.h"

namespace tts {

// Wave-aggregated LDS counter increment: the lanes that share the wave's first active bin add
// their count with one atomic (a crowded bin would otherwise serialise 64 ways); returns each
// lane's old value plus its rank among those lanes.  Other lanes add individually.
__device__ __forceinline__ int agg_inc(int* ctr, int b) {
  const int leader = first_lane(__ballot(1));
  const int b0 = read_lane(b, leader);
  const unsigned long long same = __ballot(b == b0);
  if (b == b0) {
    int base = 0;
    if (lane_id() == leader) base = atomicAdd(&ctr[b0], __popcll(same));
    return read_lane(base, leader) + __popcll(same & __lanemask_lt());
  }
  return atomicAdd(&ctr[b], 1);
}

// Wave-aggregated append position: lanes with want=true get consecutive slots of *fill.
__device__ __forceinline__ int wave_append(int* fill, bool want) {
  const unsigned long long m = __ballot(want);
  if (!m) return -1;
  const int leader = first_lane(m);
  int base = 0;
  if (lane_id() == leader) base = atomicAdd(fill, __popcll(m));
  base = read_lane(base, leader);
  return want ? base + __popcll(m & __lanemask_lt()) : -1;
}

// Histogram add with the same aggregation (no rank needed).
__device__ __forceinline__ void hist_add(unsigned* h, unsigned b) {
  const int leader = first_lane(__ballot(1));
  const unsigned b0 = static_cast<unsigned>(read_lane(static_cast<int>(b), leader));
  const unsigned long long same = __ballot(b == b0);
  if (b == b0) {
    if (lane_id() == leader) atomicAdd(&h[b0], static_cast<unsigned>(__popcll(same)));
  } else {
    atomicAdd(&h[b], 1u);
  }
}


template <int NT, int PER>
__global__ __launch_bounds__(NT) void k_bin_count(
    const float* __restrict__ mu2d, int mu_stride, const uint8_t* __restrict__ keep,
    int keep_stride, int G, int ntx, int nty, float S, int span, int NB, int Tpad,
    int* __restrict__ mat, int2* __restrict__ cell_slot) {
  using C = CountGeo<NT, PER>;
  extern __shared__ int s_lds[];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int g0 = blockIdx.x * C::kBlock + wave * C::kWaveSpan + lane;
  // loads from clamped indices, unconditionally, so that all of them are in flight at once
  // (and while the histogram is zeroed)
  float mx[PER], my[PER];
  uint8_t kv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int gc = min(g0 + 64 * i, G - 1);
    kv[i] = keep[(int64_t)gc * keep_stride];
    mx[i] = mu2d[(int64_t)gc * mu_stride];
    my[i] = mu2d[(int64_t)gc * mu_stride + 1];
  }
  count_body<NT, PER>(mx, my, kv, G, ntx, nty, S, span, NB, Tpad, s_lds, mat, cell_slot);
}

// Column scan of the count matrix, one block per chunk of 64 columns: 16 segments of rows per
// column summed in parallel, the segment sums scanned, the rows rewritten in place with their
// exclusive prefix over count blocks (a block's base in the cell).  Also the column totals
// tot[x], their exclusive prefix inside the chunk within[x], and the chunk's total.  Block 0
// also zeroes the counters the scatter pass's classification blocks accumulate into.
// adv (optional): a training step's Adam step block, advanced by block 0 (the step's advance when
// the count pass ran in the previous step's backward launch).
__global__ __launch_bounds__(1024) void k_bin_colscan(int* __restrict__ mat, int nblk, int X,
                                                      int* __restrict__ tot,
                                                      int* __restrict__ within,
                                                      int* __restrict__ chunk_tot,
                                                      int* __restrict__ cls_ctr, int n_ctr,
                                                      int32_t* adv, float b1, float b2) {
  __shared__ int s_seg[16][kChunk];
  // the scatter pass's list counters start from zero
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < n_ctr; i += 1024) cls_ctr[i] = 0;
  if (adv && blockIdx.x == 0 && threadIdx.x == 0) advance_step(adv, b1, b2);
  const int col = threadIdx.x & (kChunk - 1), seg = threadIdx.x >> 6;
  const int x = blockIdx.x * kChunk + col;
  const int rows = (nblk + 15) / 16;
  const int r0 = min(seg * rows, nblk), r1 = min(r0 + rows, nblk);
  // up to 256 count blocks a thread's rows fit in registers and are read once; more are read
  // again for the second pass
  const bool held = rows <= 16;
  int v[16];
  int sum = 0;
  if (held) {
#pragma unroll
    for (int k = 0; k < 16; ++k)
      v[k] = (x < X && r0 + k < r1) ? mat[(int64_t)(r0 + k) * X + x] : 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) sum += v[k];
  } else if (x < X) {
    for (int rb = r0; rb < r1; rb += 16) {
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = rb + k < r1 ? mat[(int64_t)(rb + k) * X + x] : 0;
#pragma unroll
      for (int k = 0; k < 16; ++k) sum += v[k];
    }
  }
  s_seg[seg][col] = sum;
  __syncthreads();
  int total = 0;
  if (seg == 0) {
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int v = s_seg[s][col];
      s_seg[s][col] = total;
      total += v;
    }
  }
  __syncthreads();
  if (x < X) {
    int base = s_seg[seg][col];
    if (held) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (r0 + k < r1) mat[(int64_t)(r0 + k) * X + x] = base;
        base += v[k];
      }
    } else {
      for (int rb = r0; rb < r1; rb += 16) {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = rb + k < r1 ? mat[(int64_t)(rb + k) * X + x] : 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          if (rb + k < r1) mat[(int64_t)(rb + k) * X + x] = base;
          base += v[k];
        }
      }
    }
  }
  if (seg == 0) {  // wave 0: the chunk's 64 columns
    const int incl = wave_incl_scan(total);
    if (x < X) {
      tot[x] = total;
      within[x] = incl - total;
    }
    if (col == kChunk - 1) chunk_tot[blockIdx.x] = incl;
  }
}

// Rank of border index b in cell order (top row, then left and right cell of each inner row,
// then the bottom row).
__device__ __forceinline__ int border_rank(int b, int ntx, int nty) {
  if (nty == 1 || ntx == 1) return b;
  if (b < ntx) return b;
  if (b < 2 * ntx) return ntx + 2 * (nty - 2) + (b - ntx);
  if (b < 2 * ntx + (nty - 2)) return ntx + 2 * (b - 2 * ntx);
  return ntx + 2 * (b - 2 * ntx - (nty - 2)) + 1;
}

struct ScatterArgs {
  const float* mu2d;
  int mu_stride, G, ntx, nty, NB, Tpad, K, cblock, ncls;
  const int2* cell_slot;
  const int* mat;
  const int* tot;
  const int* within;
  const int* chunk_tot;
  int* cell_start;
  int* far_start;
  int4* recs;
  int* far_g;
  int32_t* inv;
  int* lists;
  int* nlist;       // [2] heavy, light tiles listed (zeroed by k_bin_colscan)
  int* key_hist;    // [K+1][ncls] tiles per order key in each classification block
  int* tile_pos;    // [T] a tile's rank among its classification block's tiles of its key
};

// Classification, block cb: tiles [1024 cb, 1024 (cb + 1)).  A tile's candidates are the 3x3 box
// sum of the cell totals (regular + far).  Tiles with more than K candidates go to the front of
// lists, the others to the back (lists[T-1], lists[T-2], ...), in no particular order (one
// atomic per block and list places the block's tiles).  The order key K - min(candidates, K)
// sorts by kept count, heaviest first: the block writes its tiles' count per key (column cb of
// key_hist) and each tile's rank among them (tile_pos); k_bin_select turns these into the
// tile's slot of the order.
__device__ void classify_tiles(const ScatterArgs& a, int cb, int* s_bins, int* s_tmp) {
  const int ntx = a.ntx, nty = a.nty, T = ntx * nty, K = a.K;
  __shared__ int s_hbase, s_lbase;
  for (int c = threadIdx.x; c <= K; c += 1024) s_bins[c] = 0;
  const int t = cb * 1024 + threadIdx.x;
  int nc = -1;
  if (t < T) {
    const int tx = t % ntx, ty = t / ntx;
    nc = 0;
#pragma unroll
    for (int dy = -1; dy <= 1; ++dy) {
#pragma unroll
      for (int dx = -1; dx <= 1; ++dx) {
        const int cx = tx + dx, cy = ty + dy;
        if (cx >= 0 && cx < ntx && cy >= 0 && cy < nty) {
          nc += a.tot[cy * ntx + cx];
          if (a.NB > 0 && (cx == 0 || cx == ntx - 1 || cy == 0 || cy == nty - 1))
            nc += a.tot[a.Tpad + border_index(cx, cy, ntx, nty)];
        }
      }
    }
  }
  __syncthreads();
  const bool heavy = nc > K, light = nc >= 0 && nc <= K;
  int nh, nl;
  const int eh = block_excl_scan<1024>(heavy ? 1 : 0, s_tmp, &nh);
  const int el = block_excl_scan<1024>(light ? 1 : 0, s_tmp, &nl);
  if (threadIdx.x == 0) {
    s_hbase = nh ? atomicAdd(&a.nlist[0], nh) : 0;
    s_lbase = nl ? atomicAdd(&a.nlist[1], nl) : 0;
  }
  const int key = nc >= 0 ? K - min(nc, K) : 0;
  const int lrank = nc >= 0 ? agg_inc(s_bins, key) : 0;
  __syncthreads();
  if (heavy) a.lists[s_hbase + eh] = t;
  if (light) a.lists[T - 1 - (s_lbase + el)] = t;
  if (nc >= 0) a.tile_pos[t] = lrank;
  for (int k = threadIdx.x; k <= K; k += 1024) a.key_hist[k * a.ncls + cb] = s_bins[k];
}

// Scatter pass.  Blocks [0, ncls) classify the tiles (above).  Every other block first forms, in
// LDS, the exclusive prefix of the regular chunk totals and the far counts' prefix in cell
// order; block ncls + i then writes cell_start / far_start for cells [1024 i, 1024 (i + 1)) and
// places gaussian 1024 i + threadIdx.x: regular ones as (g, mu_x, mu_y) records at cell_start +
// its count block's base in the cell + its rank, far ones as ids at far_start + its count
// block's base + its rank, so every cell's far ids end up ascending.
__global__ __launch_bounds__(1024) void k_bin_scatter(ScatterArgs a) {
  __shared__ int s_cpre[kMaxLdsInts / kChunk];
  __shared__ int s_fp[kMaxBorder + 1];
  __shared__ int s_tmp[32];
  __shared__ int s_bins[kMaxK + 2];
  if (static_cast<int>(blockIdx.x) < a.ncls) {
    classify_tiles(a, blockIdx.x, s_bins, s_tmp);
    return;
  }
  const int ntx = a.ntx, nty = a.nty, T = ntx * nty, NB = a.NB;
  const int tid = threadIdx.x;
  const int i0 = (blockIdx.x - a.ncls) * 1024 + tid;
  // this thread's gaussian, loaded before the prologue's scans
  const int g = i0;
  const int gl = min(g, max(a.G - 1, 0));
  int2 cs = make_int2(-1, 0);
  float mx = 0.f, my = 0.f;
  if (a.G > 0) {
    cs = a.cell_slot[gl];
    mx = a.mu2d[(int64_t)gl * a.mu_stride];
    my = a.mu2d[(int64_t)gl * a.mu_stride + 1];
  }
  const int nch = a.Tpad / kChunk;
  int regtot;
  const int cex = block_excl_scan<1024>(tid < nch ? a.chunk_tot[tid] : 0, s_tmp, &regtot);
  if (tid < nch) s_cpre[tid] = cex;
  if (tid < NB) s_fp[border_rank(tid, ntx, nty)] = a.tot[a.Tpad + tid];
  __syncthreads();
  int ftot;
  const int fex = block_excl_scan<1024>(tid < NB ? s_fp[tid] : 0, s_tmp, &ftot);
  if (tid < NB) s_fp[tid] = fex;
  __syncthreads();
  if (i0 <= T) {
    const int c = i0;
    int fs = ftot;
    if (c < T && NB > 0) {
      const int cx = c % ntx, cy = c / ntx;
      const bool border = cx == 0 || cx == ntx - 1 || cy == 0 || cy == nty - 1;
      // an inner cell follows its row's left border cell: the prefix up to its right one
      fs = s_fp[border ? border_rank(border_index(cx, cy, ntx, nty), ntx, nty)
                       : ntx + 2 * (cy - 1) + 1];
    } else if (c < T) {
      fs = 0;
    }
    a.cell_start[c] = c < T ? s_cpre[c / kChunk] + a.within[c] : regtot;
    a.far_start[c] = fs;
  }
  if (g >= a.G) return;
  if (a.inv) {  // no slot yet: k_bin_select fills the kept (g, j) entries
#pragma unroll
    for (int j = 0; j < 9; ++j) a.inv[(int64_t)g * 9 + j] = -1;
  }
  if (cs.x < 0) return;
  const int X = a.Tpad + NB;
  const int* row = a.mat + (int64_t)(g / a.cblock) * X;
  if (cs.x >> kFarBit) {
    const int c = cs.x & ~(1 << kFarBit);
    const int b = border_index(c % ntx, c / ntx, ntx, nty);
    a.far_g[s_fp[border_rank(b, ntx, nty)] + row[a.Tpad + b] + cs.y] = g;
  } else {
    const int c = cs.x;
    a.recs[s_cpre[c / kChunk] + a.within[c] + row[c] + cs.y] =
        make_int4(g, __float_as_int(mx), __float_as_int(my), 0);
  }
}

struct TileCells {
  int start[9];   // first regular record of the cell reaching the tile via stencil index j
  int pre[10];    // prefix of the cells' regular counts over j (pre[9] = regular candidates)
  int fstart[9];  // first far id of the cell
  int fpre[10];   // prefix of the far counts (fpre[9] = far candidates)
};

__device__ __forceinline__ unsigned long long make_key(int q, int j, int g) {
  return (static_cast<unsigned long long>(q) << kQShift) |
         (static_cast<unsigned long long>(j) << kJShift) | static_cast<unsigned int>(g);
}

__device__ __forceinline__ unsigned long long record_key(int4 r, int j, int tx, int ty, float S,
                                                         int span) {
  return make_key(quant_dist2(__int_as_float(r.y), __int_as_float(r.z), tx, ty, S, span), j, r.x);
}

__device__ __forceinline__ int stencil_of(const TileCells& tc, int i) {
  int j = 0;
#pragma unroll
  for (int k = 1; k < 9; ++k) j += (i >= tc.pre[k]) ? 1 : 0;
  return j;
}

__device__ __forceinline__ int4 load_candidate(const TileCells& tc, const int4* __restrict__ recs,
                                               int i, int j) {
  return recs[tc.start[j] + (i - tc.pre[j])];
}

// f(key) for every regular candidate of the tile, flattened over the nine cells so that all
// loads of a light tile are issued in one round, four independent loads in flight per thread.
template <int NT, typename F>
__device__ __forceinline__ void for_each_candidate_at(const TileCells& tc,
                                                      const int4* __restrict__ recs, int tx,
                                                      int ty, float S, int span, int tid, F&& f) {
  const int n = tc.pre[9];
  int i = tid;
  for (; i + 3 * NT < n; i += 4 * NT) {
    const int j0 = stencil_of(tc, i), j1 = stencil_of(tc, i + NT);
    const int j2 = stencil_of(tc, i + 2 * NT), j3 = stencil_of(tc, i + 3 * NT);
    const int4 r0 = load_candidate(tc, recs, i, j0);
    const int4 r1 = load_candidate(tc, recs, i + NT, j1);
    const int4 r2 = load_candidate(tc, recs, i + 2 * NT, j2);
    const int4 r3 = load_candidate(tc, recs, i + 3 * NT, j3);
    f(i, record_key(r0, j0, tx, ty, S, span));
    f(i + NT, record_key(r1, j1, tx, ty, S, span));
    f(i + 2 * NT, record_key(r2, j2, tx, ty, S, span));
    f(i + 3 * NT, record_key(r3, j3, tx, ty, S, span));
  }
  for (; i < n; i += NT) {
    const int j = stencil_of(tc, i);
    f(i, record_key(load_candidate(tc, recs, i, j), j, tx, ty, S, span));
  }
}
// The same walk, f(key) only.
template <int NT, typename F>
__device__ __forceinline__ void for_each_candidate(const TileCells& tc,
                                                   const int4* __restrict__ recs, int tx, int ty,
                                                   float S, int span, int tid, F&& f) {
  for_each_candidate_at<NT>(tc, recs, tx, ty, S, span, tid,
                            [&](int, unsigned long long key) { f(key); });
}

// f(key) for the regular candidates of one cell (stencil index j) only.
template <int NT, typename F>
__device__ __forceinline__ void for_each_in_cell(const TileCells& tc,
                                                 const int4* __restrict__ recs, int j, int tx,
                                                 int ty, float S, int span, F&& f) {
  const int n = tc.pre[j + 1] - tc.pre[j];
  const int4* r = recs + tc.start[j];
  for (int i = threadIdx.x; i < n; i += NT) f(record_key(r[i], j, tx, ty, S, span));
}

// The nine neighbour cells of tile (tx, ty), loaded by lanes 0..8 of the calling wave (every
// lane of the wave must call).
__device__ __forceinline__ void load_tile_cells(TileCells& tc, int tx, int ty, int ntx, int nty,
                                                const int* __restrict__ cell_start,
                                                const int* __restrict__ far_start) {
  const int j = lane_id();
  int n = 0, st = 0, fn = 0, fst = 0;
  if (j < 9) {
    const int dy = j / 3 - 1, dx = j % 3 - 1;
    const int cx = tx - dx, cy = ty - dy;  // the cell whose gaussians reach the tile via offset j
    if (cx >= 0 && cx < ntx && cy >= 0 && cy < nty) {
      const int c = cy * ntx + cx;
      st = cell_start[c];
      n = cell_start[c + 1] - st;
      fst = far_start[c];
      fn = far_start[c + 1] - fst;
    }
  }
  const int in = wave_incl_scan(n), ifn = wave_incl_scan(fn);
  if (j < 9) {
    tc.start[j] = st;
    tc.pre[j] = in - n;
    tc.fstart[j] = fst;
    tc.fpre[j] = ifn - fn;
  }
  if (j == 8) {
    tc.pre[9] = in;
    tc.fpre[9] = ifn;
  }
}

// Find the bin holding rank r in hist[0..nbins): s_out = {bin, elements before it, its count}.
// Each thread sums a contiguous chunk, then one block scan.  Barriers inside.
template <int NT>
__device__ __forceinline__ void find_rank_bin(const unsigned* hist, int nbins, int r, int* s_tmp,
                                              int* s_out) {
  const int chunk = (nbins + NT - 1) / NT;
  const int lo = threadIdx.x * chunk, hi = min(lo + chunk, nbins);
  int sum = 0;
  for (int b = lo; b < hi; ++b) sum += hist[b];
  int total;
  int before = block_excl_scan<NT>(sum, s_tmp, &total);
  if (r >= before && r < before + sum) {
    for (int b = lo; b < hi; ++b) {
      const int c = hist[b];
      if (r < before + c) {
        s_out[0] = b;
        s_out[1] = before;
        s_out[2] = c;
        break;
      }
      before += c;
    }
  }
  __syncthreads();
}

// Inside one qd2 bin the key order is the order of sub = (j << gbits) | g.
__device__ __forceinline__ unsigned sub_key(unsigned long long key, int gbits) {
  return (static_cast<unsigned>(key >> kJShift) & 15u) << gbits |
         (static_cast<unsigned>(key) & ((1u << gbits) - 1u));
}

// Radix select of the rank-r value among the `bits`-bit values visited by `visit(g)` (g(v) is
// called for each element; the values are distinct).  Returns (prefix, stop): an element
// survives iff (v >> stop) <= (prefix >> stop); exactly r+1 elements do.  Barriers inside.
template <int NT, typename V>
__device__ __forceinline__ void radix_select(V&& visit, int r, int bits, unsigned* s_hist,
                                             int* s_tmp, int* s_out, unsigned* prefix_out,
                                             int* stop_out) {
  unsigned prefix = 0;
  int hi = bits, stop = hi;
  while (hi > 0) {
    const int w = hi < kDigitBits ? hi : kDigitBits;
    const int lo = hi - w;
    const int nb = 1 << w;
    for (int b = threadIdx.x; b < nb; b += NT) s_hist[b] = 0;
    __syncthreads();
    visit([&](unsigned s) {
      if (hi >= 32 || (s >> hi) == (prefix >> hi)) hist_add(s_hist, (s >> lo) & (nb - 1));
    });
    __syncthreads();
    find_rank_bin<NT>(s_hist, nb, r, s_tmp, s_out);
    const int b = s_out[0], bef = s_out[1], c = s_out[2];
    prefix |= static_cast<unsigned>(b) << lo;
    r -= bef;
    stop = lo;
    hi = lo;
    if (r == c - 1) break;  // the wanted element is the largest of this bin: take the bin
  }
  *prefix_out = prefix;
  *stop_out = stop;
}

// Number of the n values get(0..n-1) below v, read 8 at a time (n small: a few tie keys).
template <typename G>
__device__ __forceinline__ int count_below(unsigned v, int n, G&& get) {
  int c = 0;
  for (int f = 0; f < n; f += 8) {
    unsigned w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = f + i < n ? get(f + i) : ~0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) c += w[i] < v ? 1 : 0;
  }
  return c;
}

constexpr int kSelThreads = 256;
constexpr int kTieCap = 1024;   // tie-bin candidates kept in LDS for the sub-key select

struct SelectArgs {
  const int4* recs;
  const int* far_g;
  const int* cell_start;
  const int* far_start;
  int ntx, nty;
  float S;
  int span, K, kpow2, gbits;
  int32_t* idx;
  uint8_t* valid;
  int32_t* count;
  int32_t* ncand;
  int32_t* inv;
  int32_t* order;          // heaviest-first tile order (may be null)
  const int* key_hist;     // [K+1][ncls] per classification block tiles per order key
  const int* tile_pos;     // [T] rank among its classification block's tiles of its key
  int ncls;
  const float* proj;       // [G][12] projection records (read when rec is set)
  float* rec;              // [T][K][12] slot records by dispatch position (may be null)
  int32_t* pos_count;      // [T] kept count by dispatch position (with rec)
};

// Slot records: the kept gaussian's 12-float projection record, copied to its slot at the
// tile's place in the dispatch order (rec[position][slot]), so a splat block reads its slots as
// one contiguous run instead of order -> idx -> proj.
struct SlotRec {
  float4 r0, r1, r2;
};
__device__ __forceinline__ SlotRec rec_load(const float* __restrict__ proj, int g) {
  const float4* src = reinterpret_cast<const float4*>(proj + (int64_t)g * 12);
  return SlotRec{src[0], src[1], src[2]};
}
__device__ __forceinline__ void rec_store(float* __restrict__ rb, int slot, SlotRec r) {
  float4* dst = reinterpret_cast<float4*>(rb + (int64_t)slot * 12);
  dst[0] = r.r0;
  dst[1] = r.r1;
  dst[2] = r.r2;
}

// What a kept survivor writes at its slot `rank` of the tile whose slots start at `base`: its
// gaussian in idx, valid = 1, its inverse-table entry inv[g][j] (a gaussian reaches a tile through
// exactly one stencil index j) and, with records (rb), its slot record.  An unused slot s gets
// idx 0, valid 0.
__device__ __forceinline__ void put_slot(const SelectArgs& a, int64_t base, float* rb, int rank,
                                         unsigned long long key, const SlotRec& rec) {
  const int g = static_cast<int32_t>(key & 0xffffffffull);
  a.idx[base + rank] = g;
  if (a.inv) a.inv[(int64_t)g * 9 + ((key >> kJShift) & 15ull)] = static_cast<int32_t>(base + rank);
  a.valid[base + rank] = 1;
  if (rb) rec_store(rb, rank, rec);
}
__device__ __forceinline__ void clear_slot(const SelectArgs& a, int64_t base, int s) {
  a.idx[base + s] = 0;
  a.valid[base + s] = 0;
}

// Slot of tile t (n candidates) in the heaviest-first order: tiles of smaller keys (more kept
// slots), then this key's tiles of earlier classification blocks, then its rank in its block.
// A lane sums whole keys (key-major table, no division); full tiles (key 0) need only their
// own key's earlier blocks.  Every lane of the wave calls; the slot comes back in every lane.
__device__ __forceinline__ int order_slot(const SelectArgs& a, int t, int n) {
  const int key = a.K - min(n, a.K), cb = t >> 10, nc = a.ncls;
  int s = 0;
  for (int k = lane_id(); k <= key; k += 64) {
    const int* h = a.key_hist + k * nc;
    const int nb = k < key ? nc : cb;
    for (int b = 0; b < nb; ++b) s += h[b];
  }
  return read_lane(wave_incl_scan(s), 63) + a.tile_pos[t];
}
// The same slot in two halves: the key-major table's entries before (key, cb) form one
// contiguous prefix [0, key * ncls + cb); begin() requests up to 64 * kOsPre of them (and the
// tile's rank) into registers, end() waits for them, adds any further entries and reduces.
constexpr int kOsPre = 8;
struct OrderSlot {
  int v[kOsPre];
  int pos, len;
  __device__ __forceinline__ void begin(const SelectArgs& a, int t, int n) {
    const int key = a.K - min(n, a.K);
    len = key * a.ncls + (t >> 10);
    const int lane = lane_id();
#pragma unroll
    for (int i = 0; i < kOsPre; ++i) {
      const int e = lane + 64 * i;
      v[i] = e < len ? a.key_hist[e] : 0;
    }
    pos = a.tile_pos[t];
  }
  __device__ __forceinline__ int end(const SelectArgs& a) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < kOsPre; ++i) s += v[i];
    for (int e = lane_id() + 64 * kOsPre; e < len; e += 64) s += a.key_hist[e];
    return read_lane(wave_incl_scan(s), 63) + pos;
  }
};

// Survivors are placed by groups in key order: 55 runs of 2^shift qd2 bins below the saturated
// bin span-1 (group_shift picks the run length that puts bin qtop, the highest unsaturated bin
// that holds survivors, in run 54 or below), then the saturated bin split by stencil index j
// (groups 55..63).  Keys order by q, then j, then g, so every key of a group is below every key
// of a later group, and a survivor's slot is the number of survivors in lower groups plus its
// rank inside its group.
constexpr int kGroups = 64;
__device__ __forceinline__ int group_shift(int qtop) {
  int shift = 0;
  while ((qtop >> shift) > 54) ++shift;
  return shift;
}
__device__ __forceinline__ int key_group(unsigned long long key, int satq, int shift) {
  const int q = static_cast<int>(key >> kQShift);
  return q < satq ? (q >> shift) : 55 + static_cast<int>((key >> kJShift) & 15ull);
}
// start + the number of the c keys buf[start, start + c) below key.  The 7 entries past the
// group's end must hold larger keys (later groups, or padding): the reads go 8 at a time.
__device__ __forceinline__ int rank_in_group(unsigned long long key, const unsigned long long* buf,
                                             int start, int c) {
  int rank = start;
  if (c > 1) {
    for (int f = 0; f < c; f += 8) {
      unsigned long long w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = buf[start + f + i];
#pragma unroll
      for (int i = 0; i < 8; ++i) rank += w[i] < key ? 1 : 0;
    }
  }
  return rank;
}

// Light tile (n <= K candidates: all survive), one wave: collect the keys in LDS, then place
// them by groups.  keys holds 2 * kpow2 + 8 entries (the keys, then the keys gathered by group)
// and grp kGroups words.
__device__ __forceinline__ void select_light(int t, const SelectArgs& a, TileCells& tc,
                                             unsigned long long* keys, unsigned* grp, int* fill) {
  const int lane = lane_id();
  const int tx = t % a.ntx, ty = t / a.ntx;
  load_tile_cells(tc, tx, ty, a.ntx, a.nty, a.cell_start, a.far_start);
  if (lane == 0) *fill = 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int nfar = tc.fpre[9];
  const int satq = a.span - 1;
  // a light tile keeps all its candidates: its order slot is known now, its loads overlap the walk
  OrderSlot os;
  if (a.order) os.begin(a, t, tc.pre[9] + nfar);
  for_each_candidate<64>(tc, a.recs, tx, ty, a.S, a.span, lane, [&](unsigned long long key) {
    keys[wave_append(fill, true)] = key;
  });
  for (int i = lane; i < nfar; i += 64) {
    int j = 0;
#pragma unroll
    for (int k = 1; k < 9; ++k) j += (i >= tc.fpre[k]) ? 1 : 0;
    keys[wave_append(fill, true)] = make_key(satq, j, a.far_g[tc.fstart[j] + i - tc.fpre[j]]);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int m = *fill;
  const int64_t base = static_cast<int64_t>(t) * a.K;
  // the tile's place in the dispatch order (its key-table loads were issued before the walk)
  const int slot = a.order ? os.end(a) : 0;
  float* rb = a.rec ? a.rec + (int64_t)slot * a.K * 12 : nullptr;
  if (a.K <= 128) {
    // all pairs (cheaper than the groups' extra passes at this size)
    // the keys padded to a multiple of 16 with the largest key (never below a survivor), so the
    // rank counts read them 8 at a time with no tail
    const int m16 = (m + 15) & ~15;  // <= kpow2, a power of two >= 16
    if (lane < m16 - m) keys[m + lane] = ~0ull;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const ulonglong2* kp = reinterpret_cast<const ulonglong2*>(keys);
    for (int s0 = 0; s0 < a.K; s0 += 128) {
      // slots s0 + lane and s0 + 64 + lane share each key read
      const int sa = s0 + lane, sb = sa + 64;
      const unsigned long long ka = sa < m ? keys[sa] : 0ull, kb = sb < m ? keys[sb] : 0ull;
      // the slot records are requested before the rank counts, which hide their round trip
      SlotRec reca{}, recb{};
      if (rb && sa < m) reca = rec_load(a.proj, static_cast<int32_t>(ka & 0xffffffffull));
      if (rb && sb < m) recb = rec_load(a.proj, static_cast<int32_t>(kb & 0xffffffffull));
      int ra = 0, rnb = 0;
      if (s0 < m) {
        for (int e = 0; e < m16 / 2; e += 4) {
          const ulonglong2 k0 = kp[e], k1 = kp[e + 1], k2 = kp[e + 2], k3 = kp[e + 3];
          ra += (k0.x < ka) + (k0.y < ka) + (k1.x < ka) + (k1.y < ka) + (k2.x < ka) + (k2.y < ka) +
                (k3.x < ka) + (k3.y < ka);
          rnb += (k0.x < kb) + (k0.y < kb) + (k1.x < kb) + (k1.y < kb) + (k2.x < kb) +
                 (k2.y < kb) + (k3.x < kb) + (k3.y < kb);
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int s = h ? sb : sa;
        const unsigned long long key = h ? kb : ka;
        const int rank = h ? rnb : ra;
        if (s < m) put_slot(a, base, rb, rank, key, h ? recb : reca);
        else if (s < a.K) clear_slot(a, base, s);
      }
    }
  } else {
    // Group counts (LDS atomics), one scan, then the keys gathered by group behind the key list.
    // A group's word packs start << 20 | count << 10 | cursor (each <= K <= 512); the gathering
    // atomics advance the cursor.
    const int shift = group_shift(satq - 1);
    unsigned long long* gat = keys + a.kpow2;
    grp[lane] = 0;
    if (lane < 8) gat[m + lane] = ~0ull;  // above every key
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int s = lane; s < m; s += 64) atomicAdd(&grp[key_group(keys[s], satq, shift)], 1u);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    {
      const int v = static_cast<int>(grp[lane]);
      const int inc = wave_incl_scan(v);
      grp[lane] = static_cast<unsigned>((inc - v) << 20 | v << 10);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int s = lane; s < m; s += 64) {
      const unsigned long long key = keys[s];
      const unsigned w = atomicAdd(&grp[key_group(key, satq, shift)], 1u);
      gat[(w >> 20) + (w & 1023u)] = key;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int s = lane; s < a.K; s += 64) {
      if (s < m) {
        const unsigned long long key = keys[s];
        SlotRec rec{};
        if (rb) rec = rec_load(a.proj, static_cast<int32_t>(key & 0xffffffffull));
        const unsigned w = grp[key_group(key, satq, shift)];
        put_slot(a, base, rb,
                 rank_in_group(key, gat, static_cast<int>(w >> 20),
                               static_cast<int>((w >> 10) & 1023u)),
                 key, rec);
      } else {
        clear_slot(a, base, s);
      }
    }
  }
  if (lane == 0) {
    if (a.order) a.order[slot] = t;
    if (rb) a.pos_count[slot] = m;
    if (a.count) a.count[t] = m;
    if (a.ncand) a.ncand[t] = m;
  }
}

// One block of NT threads per heavy tile, then one wave per light tile (NT/64 per block).
//   heavy (n > K)   a walk over the regular candidates builds the LDS histogram of qd2 (far
//                   candidates add their count to bin span-1), which locates the bin qb of the
//                   K-th key; a second walk collects every key below qb.
//     qb < span-1   the tie bin holds regular candidates only: they go to an LDS tie buffer
//                   where a radix select over (j, g) picks the needed smallest ones (a bin
//                   larger than the buffer runs the same select over further walks).
//     qb = span-1   the tie set is the saturated regular candidates plus every far one.  The
//                   per-j tie counts locate the stencil index j* holding the K-th key: ties with
//                   j < j* all survive (far ones read from their lists), and inside cell j* the
//                   rest are the smallest g among its saturated regular candidates and the head
//                   of its far list (ascending in g), selected in LDS.
//   light (n <= K)  every candidate survives.
// The survivors are placed by rank (keys are unique: slot = number of smaller survivors).  A
// gaussian reaches a tile through exactly one stencil index j, so the inverse table entry
// inv[g][j] = t*K + slot has a single writer.
// 8 waves per SIMD (at most 64 registers): a heavy tile's block waits on LDS most of its time,
// and at K=256 the LDS use (~18 KB) still lets 8 blocks share a CU.
template <int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(8))) void k_bin_select(
    SelectArgs a, const int* __restrict__ lists, const int* __restrict__ nlist) {
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
  __shared__ TileCells tcs[NT / 64];
  __shared__ int s_wfill[NT / 64];
  const int T = a.ntx * a.nty;
  const int t_heavy = lists[blockIdx.x];  // this block's tile if it is a heavy one (read ahead)
  const int nh = nlist[0], nl = nlist[1];
  if (static_cast<int>(blockIdx.x) >= nh) {
    const int g0 = (static_cast<int>(blockIdx.x) - nh) * (NT / 64);
    if (g0 >= nl) return;
    const int w = threadIdx.x >> 6;
    if (g0 + w < nl) {
      unsigned long long* keys =
          reinterpret_cast<unsigned long long*>(s_dyn) + w * (2 * a.kpow2 + 8 + kGroups / 2);
      select_light(lists[T - 1 - (g0 + w)], a, tcs[w], keys,
                   reinterpret_cast<unsigned*>(keys + 2 * a.kpow2 + 8), &s_wfill[w]);
    }
    return;
  }
  const int4* __restrict__ recs = a.recs;
  const int* __restrict__ far_g = a.far_g;
  const float S = a.S;
  const int span = a.span, K = a.K, kpow2 = a.kpow2, gbits = a.gbits;
  unsigned long long* s_keys = reinterpret_cast<unsigned long long*>(s_dyn);  // [kpow2]
  unsigned long long* s_tie = s_keys + kpow2;                                 // [kTieCap]
  unsigned* s_hist = reinterpret_cast<unsigned*>(s_tie + kTieCap);  // [max(span, 2^digit)]
  TileCells& tc = tcs[0];
  __shared__ int s_tmp[NT / 64];
  __shared__ int s_out[3];
  __shared__ int s_fill, s_tfill;
  __shared__ int s_sat[9];      // saturated regular candidates per stencil index
  __shared__ int s_jstar[2];    // j*, rank inside cell j*'s tie set
  __shared__ unsigned s_grp[kGroups];  // survivors per group, then packed prefixes
  __shared__ int s_oslot;              // the tile's place in the dispatch order

  const int t = t_heavy;
  const int tx = t % a.ntx, ty = t / a.ntx;
  if (threadIdx.x < 64) load_tile_cells(tc, tx, ty, a.ntx, a.nty, a.cell_start, a.far_start);
  if (threadIdx.x == 0) {
    s_fill = 0;
    s_tfill = 0;
  }
  if (threadIdx.x < 9) s_sat[threadIdx.x] = 0;
  if (threadIdx.x < kGroups) s_grp[threadIdx.x] = 0;
  // heavy tiles (every block of this range) histogram qd2: zeroed while the cells load
  for (int b = threadIdx.x; b < span; b += NT) s_hist[b] = 0;
  __syncthreads();
  const int nreg = tc.pre[9], nfar = tc.fpre[9];
  const int n = nreg + nfar;
  const int satq = span - 1;
  // wave 0 takes the tile's order slot now; its loads overlap the candidate walks
  const int oslot = (a.order && threadIdx.x < 64) ? order_slot(a, t, n) : 0;
  if (threadIdx.x == 0) s_oslot = oslot;  // read after the barriers below

  int qlim = span;  // above every survivor's qd2 bin
  if (n <= K) {
    for_each_candidate<NT>(tc, recs, tx, ty, S, span, threadIdx.x, [&](unsigned long long key) {
      s_keys[wave_append(&s_fill, true)] = key;
    });
    for (int i = threadIdx.x; i < nfar; i += NT) {
      int j = 0;
#pragma unroll
      for (int k = 1; k < 9; ++k) j += (i >= tc.fpre[k]) ? 1 : 0;
      s_keys[wave_append(&s_fill, true)] = make_key(satq, j, far_g[tc.fstart[j] + i - tc.fpre[j]]);
    }
  } else {
    // the regular candidates' keys stay in the tie buffer when they fit, so the collecting walk
    // below reads them from LDS (its own tie entries are written only after every key is read)
    const bool cached = nreg <= kTieCap;
    for_each_candidate_at<NT>(tc, recs, tx, ty, S, span, threadIdx.x,
                              [&](int i, unsigned long long key) {
      const unsigned q = static_cast<unsigned>(key >> kQShift);
      hist_add(s_hist, q);
      if (static_cast<int>(q) == satq)
        agg_inc(s_sat, static_cast<int>((key >> kJShift) & 15ull));
      if (cached) s_tie[i] = key;
    });
    // f(key) over the regular candidates: from the cached keys (a barrier between the reads and
    // f, which may write the tie buffer) or by a walk over the records
    auto collect = [&](auto&& f) {
      if (cached) {
        unsigned long long ck[kTieCap / NT];
#pragma unroll
        for (int k = 0; k < kTieCap / NT; ++k) {
          const int i = static_cast<int>(threadIdx.x) + k * NT;
          ck[k] = i < nreg ? s_tie[i] : 0ull;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kTieCap / NT; ++k)
          if (static_cast<int>(threadIdx.x) + k * NT < nreg) f(ck[k]);
      } else {
        for_each_candidate<NT>(tc, recs, tx, ty, S, span, threadIdx.x, f);
      }
    };
    __syncthreads();
    if (threadIdx.x == 0) s_hist[satq] += nfar;
    __syncthreads();
    find_rank_bin<NT>(s_hist, span, K - 1, s_tmp, s_out);
    const int qb = s_out[0], before = s_out[1], cnt = s_out[2];
    const int r = K - 1 - before;  // rank of the K-th key inside bin qb
    qlim = qb + 1;
    if (qb < satq) {
      // ---------------- tie bin of regular candidates only ----------------
      const bool in_lds = cnt <= kTieCap;
      collect([&](unsigned long long key) {
        const int q = static_cast<int>(key >> kQShift);
        const int p = wave_append(&s_fill, q < qb);
        if (p >= 0) s_keys[p] = key;
        const int pt = wave_append(&s_tfill, q == qb && in_lds);
        if (pt >= 0) s_tie[pt] = key;
      });
      __syncthreads();
      unsigned prefix;
      int stop;
      if (r == cnt - 1) {  // the whole bin survives
        prefix = ~0u;
        stop = 0;
      } else if (cnt <= 32) {
        // a few ties (the usual case): each thread ranks one of them by its (j, g) sub-key
        if (static_cast<int>(threadIdx.x) < cnt) {
          const unsigned long long key = s_tie[threadIdx.x];
          const int below = count_below(sub_key(key, gbits), cnt,
                                        [&](int f) { return sub_key(s_tie[f], gbits); });
          const int p = wave_append(&s_fill, below <= r);
          if (p >= 0) s_keys[p] = key;
        } else {
          wave_append(&s_fill, false);
        }
        prefix = 0;
        stop = -1;
      } else if (in_lds) {
        radix_select<NT>([&](auto&& g) {
          for (int e = threadIdx.x; e < cnt; e += NT) g(sub_key(s_tie[e], gbits));
        }, r, 4 + gbits, s_hist, s_tmp, s_out, &prefix, &stop);
      } else {
        radix_select<NT>([&](auto&& g) {
          for_each_candidate<NT>(tc, recs, tx, ty, S, span, threadIdx.x, [&](unsigned long long key) {
            if (static_cast<int>(key >> kQShift) == qb) g(sub_key(key, gbits));
          });
        }, r, 4 + gbits, s_hist, s_tmp, s_out, &prefix, &stop);
      }
      const unsigned thr = stop >= 32 ? 0u : (prefix >> (stop < 0 ? 0 : stop));
      if (stop < 0) {
        // taken above
      } else if (in_lds) {
        for (int e = threadIdx.x; e < cnt; e += NT) {
          const unsigned long long key = s_tie[e];
          const bool take = (sub_key(key, gbits) >> stop) <= thr;
          const int p = wave_append(&s_fill, take);
          if (p >= 0) s_keys[p] = key;
        }
      } else {
        for_each_candidate<NT>(tc, recs, tx, ty, S, span, threadIdx.x, [&](unsigned long long key) {
          const bool take = static_cast<int>(key >> kQShift) == qb &&
                            (sub_key(key, gbits) >> stop) <= thr;
          const int p = wave_append(&s_fill, take);
          if (p >= 0 && p < kpow2) s_keys[p] = key;
        });
      }
    } else {
      // ---------------- saturated tie bin: regular saturated + far ----------------
      if (threadIdx.x == 0) {
        int cum = 0, js = 8, rr = 0;
        for (int j = 0; j < 9; ++j) {
          const int tj = s_sat[j] + (tc.fpre[j + 1] - tc.fpre[j]);
          if (r < cum + tj) {
            js = j;
            rr = r - cum;
            break;
          }
          cum += tj;
        }
        s_jstar[0] = js;
        s_jstar[1] = rr;
      }
      __syncthreads();
      const int js = s_jstar[0], rr = s_jstar[1];
      const int satj = s_sat[js];
      const int fn = tc.fpre[js + 1] - tc.fpre[js];
      const int* fl = far_g + tc.fstart[js];
      // Cell j*'s far ids ascend in g, so only its first rr+1 can be among the rr+1 smallest of
      // the cell's ties: they and the cell's saturated regular candidates fit the LDS buffer.
      const int fb = min(fn, rr + 1);
      const bool in_lds = satj + fb <= kTieCap;
      // regular keys below the bin, saturated ones with j < j*, and cell j*'s saturated ones
      collect([&](unsigned long long key) {
        const int q = static_cast<int>(key >> kQShift);
        const int j = static_cast<int>((key >> kJShift) & 15ull);
        const int p = wave_append(&s_fill, q < satq || j < js);
        if (p >= 0) s_keys[p] = key;
        const int pt = wave_append(&s_tfill, q == satq && j == js && in_lds);
        if (pt >= 0) s_tie[pt] = key;
      });
      // far keys with j < j* all survive
      const int fbefore = tc.fpre[js];
      for (int i = threadIdx.x; i < fbefore; i += NT) {
        int j = 0;
#pragma unroll
        for (int k = 1; k < 9; ++k) j += (i >= tc.fpre[k]) ? 1 : 0;
        s_keys[wave_append(&s_fill, true)] = make_key(satq, j, far_g[tc.fstart[j] + i - tc.fpre[j]]);
      }
      if (in_lds)
        for (int e = threadIdx.x; e < fb; e += NT) s_tie[satj + e] = make_key(satq, js, fl[e]);
      __syncthreads();
      const unsigned gmask = (gbits >= 32) ? ~0u : ((1u << gbits) - 1u);
      unsigned prefix;
      int stop;
      if (in_lds && satj + fb <= 32 && rr < satj + fb - 1) {
        // a few ties: each thread ranks one of them by g
        const int nt = satj + fb;
        if (static_cast<int>(threadIdx.x) < nt) {
          const unsigned long long key = s_tie[threadIdx.x];
          const int below = count_below(static_cast<unsigned>(key) & gmask, nt, [&](int f) {
            return static_cast<unsigned>(s_tie[f]) & gmask;
          });
          const int p = wave_append(&s_fill, below <= rr);
          if (p >= 0) s_keys[p] = key;
        } else {
          wave_append(&s_fill, false);
        }
      } else if (in_lds) {
        const int nt = satj + fb;
        if (rr == nt - 1) {  // all of them survive
          prefix = ~0u;
          stop = 0;
        } else {
          radix_select<NT>([&](auto&& g) {
            for (int e = threadIdx.x; e < nt; e += NT) g(static_cast<unsigned>(s_tie[e]) & gmask);
          }, rr, gbits, s_hist, s_tmp, s_out, &prefix, &stop);
        }
        const unsigned thr = stop >= 32 ? 0u : (prefix >> stop);
        for (int e = threadIdx.x; e < nt; e += NT) {
          const unsigned long long key = s_tie[e];
          const int p = wave_append(&s_fill, ((static_cast<unsigned>(key) & gmask) >> stop) <= thr);
          if (p >= 0) s_keys[p] = key;
        }
      } else {
        // more saturated regular candidates in cell j* than the buffer holds: select over the
        // cell's records and its far list directly
        if (rr == satj + fn - 1) {
          prefix = ~0u;
          stop = 0;
        } else {
          radix_select<NT>([&](auto&& g) {
            for_each_in_cell<NT>(tc, recs, js, tx, ty, S, span, [&](unsigned long long key) {
              if (static_cast<int>(key >> kQShift) == satq) g(static_cast<unsigned>(key) & gmask);
            });
            for (int e = threadIdx.x; e < fn; e += NT) g(static_cast<unsigned>(fl[e]));
          }, rr, gbits, s_hist, s_tmp, s_out, &prefix, &stop);
        }
        const unsigned thr = stop >= 32 ? 0u : (prefix >> stop);
        for_each_in_cell<NT>(tc, recs, js, tx, ty, S, span, [&](unsigned long long key) {
          const bool take = static_cast<int>(key >> kQShift) == satq &&
                            ((static_cast<unsigned>(key) & gmask) >> stop) <= thr;
          const int p = wave_append(&s_fill, take);
          if (p >= 0 && p < kpow2) s_keys[p] = key;
        });
        for (int e = threadIdx.x; e < fn; e += NT) {
          const unsigned g = static_cast<unsigned>(fl[e]);
          const int p = wave_append(&s_fill, (g >> stop) <= thr);
          if (p >= 0 && p < kpow2) s_keys[p] = make_key(satq, js, static_cast<int>(g));
        }
      }
    }
  }
  __syncthreads();
  // Place the m survivors by rank (unique keys: rank = number of smaller survivors).
  const int m = min(s_fill, K);
  const int64_t base = static_cast<int64_t>(t) * K;
  float* rb = a.rec ? a.rec + (int64_t)s_oslot * K * 12 : nullptr;
  auto put = [&](int rank, unsigned long long key, const SlotRec& rec) {
    put_slot(a, base, rb, rank, key, rec);
  };
  auto clear = [&](int s) { clear_slot(a, base, s); };
  if (K <= 128) {
    // All pairs: two adjacent lanes share a survivor, each counting over half of them; the keys
    // are padded to a multiple of 16 with the largest key (never below a survivor) and read 8 at
    // a time.
    const int m16 = (m + 15) & ~15;  // <= kpow2, a power of two >= 16
    if (static_cast<int>(threadIdx.x) < m16 - m) s_keys[m + threadIdx.x] = ~0ull;
    __syncthreads();
    const int half = threadIdx.x & 1;
    const ulonglong2* kp = reinterpret_cast<const ulonglong2*>(s_keys + half * (m16 / 2));
    for (int s0 = 0; s0 < K; s0 += NT / 2) {
      const int s = s0 + (static_cast<int>(threadIdx.x) >> 1);
      const unsigned long long key = s < m ? s_keys[s] : 0ull;
      // the slot record is requested before the rank count, which hides its round trip
      SlotRec rec{};
      if (rb && half == 0 && s < m)
        rec = rec_load(a.proj, static_cast<int32_t>(key & 0xffffffffull));
      int rank = 0;
      if (s0 < m) {
#pragma unroll 2  // 8 reads in flight; a deeper unroll spills at 64 registers
        for (int e = 0; e < m16 / 4; e += 4) {
          const ulonglong2 k0 = kp[e], k1 = kp[e + 1], k2 = kp[e + 2], k3 = kp[e + 3];
          rank += (k0.x < key) + (k0.y < key) + (k1.x < key) + (k1.y < key) + (k2.x < key) +
                  (k2.y < key) + (k3.x < key) + (k3.y < key);
        }
      }
      rank += __shfl_xor(rank, 1);
      if (half == 0 && s < K) {
        if (s < m) put(rank, key, rec);
        else clear(s);
      }
    }
  } else {
    // Larger K (the all-pairs count grows as K^2): placement by groups (key_group; every
    // survivor's bin is below qlim).  Survivor counts per group (with each survivor's arrival
    // index from the atomic), one wave's exclusive scan packed with the counts, the keys
    // gathered by group in the tie buffer, then each survivor counts the smaller keys of its
    // own group.
    const int shift = group_shift(min(qlim - 1, satq - 1));
    auto group = [&](unsigned long long key) { return key_group(key, satq, shift); };
    constexpr int kPer = kMaxK / NT;
    int pa[kPer];  // arrival index in the group (the keys are read again from s_keys)
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = static_cast<int>(threadIdx.x) + k * NT;
      pa[k] = s < m ? static_cast<int>(atomicAdd(&s_grp[group(s_keys[s])], 1u)) : 0;
    }
    if (static_cast<int>(threadIdx.x) < 8) s_tie[m + threadIdx.x] = ~0ull;  // above every key
    __syncthreads();
    if (threadIdx.x < 64) {
      const int v = static_cast<int>(s_grp[threadIdx.x]);
      const int inc = wave_incl_scan(v);
      s_grp[threadIdx.x] = static_cast<unsigned>((inc - v) << 16 | v);  // start, count (<= K)
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = static_cast<int>(threadIdx.x) + k * NT;
      if (s < m) {
        const unsigned long long key = s_keys[s];
        s_tie[(s_grp[group(key)] >> 16) + pa[k]] = key;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = static_cast<int>(threadIdx.x) + k * NT;
      if (s < m) {
        const unsigned long long key = s_keys[s];
        SlotRec rec{};
        if (rb) rec = rec_load(a.proj, static_cast<int32_t>(key & 0xffffffffull));
        const unsigned v = s_grp[group(key)];
        put(rank_in_group(key, s_tie, static_cast<int>(v >> 16), static_cast<int>(v & 0xffffu)),
            key, rec);
      } else if (s < K) {
        clear(s);
      }
    }
  }
  if (threadIdx.x == 0) {
    if (a.count) a.count[t] = m;
    if (a.ncand) a.ncand[t] = n;
    if (a.order) a.order[oslot] = t;
    if (rb) a.pos_count[oslot] = m;
  }
}

// Tiles by kept count, heaviest first (counting sort; ties in no particular order).  The splat
// kernels take their blocks in this order, so the dispatcher starts the expensive tiles first
// and fills the tail with cheap ones.
__global__ __launch_bounds__(1024) void k_tile_order(const int32_t* __restrict__ count, int T,
                                                     int K, int32_t* __restrict__ order) {
  __shared__ int s_bins[kMaxK + 2];
  __shared__ int s_tmp[16];
  for (int c = threadIdx.x; c <= K + 1; c += blockDim.x) s_bins[c] = 0;
  __syncthreads();
  // many tiles share a count (every full tile has K): wave-aggregated increments
  for (int t = threadIdx.x; t < T; t += blockDim.x)
    agg_inc(s_bins, K - min(max(count[t], 0), K));
  __syncthreads();
  // K + 1 <= 513 bins: one per thread
  const int v = threadIdx.x <= K ? s_bins[threadIdx.x] : 0;
  int total;
  const int ex = block_excl_scan<1024>(v, s_tmp, &total);
  if (threadIdx.x <= K) s_bins[threadIdx.x] = ex;
  __syncthreads();
  for (int t = threadIdx.x; t < T; t += blockDim.x)
    order[agg_inc(s_bins, K - min(max(count[t], 0), K))] = t;
}

struct BinWorkspace {
  int* mat;         // [nblk][Tpad + NB] counts per (count block, column), then block bases
  int* tot;         // [Tpad + NB] column totals: regular count per cell, far count per border cell
  int* within;      // [Tpad + NB] exclusive prefix of tot inside its 64-column chunk
  int* chunk_tot;   // [(Tpad + NB) / 64 + 1] chunk totals
  int* cell_start;  // [T+1]
  int* far_start;   // [T+1]
  int2* cell_slot;  // [G]
  int4* recs;       // [G]
  int* far_g;       // [G]
  int* lists;       // [T]  heavy tiles from the front, light tiles from the back
  int* nlist;       // [2] heavy, light counts
  int* key_hist;    // [K+1][ncls] tiles per order key per classification block
  int* tile_pos;    // [T] rank of a tile among its classification block's tiles of its key
  int NB;           // border cells with far handling (0: every gaussian is regular)
  int Tpad;         // cells rounded up to whole 64-column chunks
  int cblock;       // gaussians per count block
  int nblk;         // count-pass blocks
};

// Far handling is on when the count pass's LDS holds the border's per-wave tables beside the
// cell histogram.
inline int far_border_cells(int ntx, int nty) {
  const int NB = border_count(ntx, nty);
  return (NB <= kMaxBorder && pad_cells(ntx * nty) + kMaxCountWaves * NB <= kMaxLdsInts) ? NB : 0;
}

inline size_t bin_ws_layout(int G, int ntx, int nty, char* base, BinWorkspace* ws) {
  const int T = ntx * nty;
  const int NB = far_border_cells(ntx, nty);
  const int Tpad = pad_cells(T);
  const int cblock = count_block(G);
  const int nblk = (G + cblock - 1) / cblock;
  const size_t X = (size_t)Tpad + NB;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  const size_t g1 = (size_t)(G > 0 ? G : 1);
  char* m = take(sizeof(int) * ((size_t)nblk * X + 1));
  char* t = take(sizeof(int) * X);
  char* w = take(sizeof(int) * X);
  char* ct = take(sizeof(int) * (X / kChunk + 2));
  char* b = take(sizeof(int) * ((size_t)T + 1));
  char* b2 = take(sizeof(int) * ((size_t)T + 1));
  char* c = take(sizeof(int2) * g1);
  char* d = take(sizeof(int4) * g1);
  char* e = take(sizeof(int) * g1);
  char* l = take(sizeof(int) * (size_t)T);
  char* nl = take(sizeof(int) * 2);
  char* kh = take(sizeof(int) * (size_t)((T + 1023) / 1024) * (kMaxK + 1));
  char* tp = take(sizeof(int) * (size_t)T);
  if (ws) {
    ws->mat = reinterpret_cast<int*>(m);
    ws->tot = reinterpret_cast<int*>(t);
    ws->within = reinterpret_cast<int*>(w);
    ws->chunk_tot = reinterpret_cast<int*>(ct);
    ws->cell_start = reinterpret_cast<int*>(b);
    ws->far_start = reinterpret_cast<int*>(b2);
    ws->cell_slot = reinterpret_cast<int2*>(c);
    ws->recs = reinterpret_cast<int4*>(d);
    ws->far_g = reinterpret_cast<int*>(e);
    ws->lists = reinterpret_cast<int*>(l);
    ws->nlist = reinterpret_cast<int*>(nl);
    ws->key_hist = reinterpret_cast<int*>(kh);
    ws->tile_pos = reinterpret_cast<int*>(tp);
    ws->NB = NB;
    ws->Tpad = Tpad;
    ws->cblock = cblock;
    ws->nblk = nblk;
  }
  return off;
}

}  // namespace tts

using namespace tts;

extern "C" {

size_t tts_bin_workspace_bytes(int G, int H, int W, int S) {
  if (G < 0 || S <= 0 || H <= 0 || W <= 0) return 0;
  return bin_ws_layout(G, W / S, H / S, nullptr, nullptr);
}

}  // extern "C"

namespace tts {

// Argument checks shared by both binning entry points (nothing is launched on failure).
static int bin_check(const float* mu2d, int mu_stride, const uint8_t* keep, int keep_stride,
                     int G, int H, int W, int S, int R, int K, int span, const int32_t* idx,
                     const uint8_t* valid) {
  if (G < 0 || H <= 0 || W <= 0 || !idx || !valid) return TTS_EINVAL;
  if (G > 0 && (!mu2d || !keep || mu_stride < 2 || keep_stride < 1)) return TTS_EINVAL;
  if (G > (1 << 28)) return TTS_EG;  // (j << gbits) | g must fit in 32 bits
  if (S != 16 && S != 32) return TTS_ETILE;
  if (H % S || W % S) return TTS_ETILE;
  if (pad_cells((H / S) * (W / S)) > kMaxLdsInts) return TTS_ETILE;  // the count pass's histogram
  if (R != 1) return TTS_ERADIUS;
  if (K < 1 || K > kMaxK) return TTS_EK;
  if (span < 1 || span > kMaxSpan) return TTS_ESPAN;
  return TTS_OK;
}

// The binning passes on a laid-out workspace (arguments already checked).  Every buffer the
// passes read is written earlier in the same call: nothing has to be zero on entry.  counted:
// the count pass already ran (k_geom_fwd_count wrote ws.mat and ws.cell_slot).
static int bin_run(const float* mu2d, int mu_stride, const uint8_t* keep, int keep_stride,
                   int G, int H, int W, int S, int K, int span, int32_t* idx, uint8_t* valid,
                   int32_t* count, int32_t* ncand, int32_t* inv, int32_t* order,
                   const float* proj, float* rec, int32_t* pos_count, const BinWorkspace& ws,
                   bool counted, hipStream_t stream, int32_t* adv = nullptr, float b1 = 0.f,
                   float b2 = 0.f) {
  const int ntx = W / S, nty = H / S, T = ntx * nty;
  const float Sf = static_cast<float>(S);
  const int NB = ws.NB, Tpad = ws.Tpad, nblk = ws.nblk;
  const int X = Tpad + NB;
  if (G > 0 && !counted) {
    const bool small = ws.cblock == CountSmall::kBlock;
    const size_t lds =
        sizeof(int) * (size_t)(Tpad + (small ? CountSmall::kWaves : CountLarge::kWaves) * NB);
    static LdsLimit lim[2];
    if (lds > 65536) {
      const void* fn = small ? reinterpret_cast<const void*>(&k_bin_count<256, 2>)
                             : reinterpret_cast<const void*>(&k_bin_count<1024, 4>);
      const int e = raise_lds_limit(fn, lim[small ? 0 : 1]);
      if (e) return e;
    }
    if (small)
      k_bin_count<256, 2><<<nblk, 256, lds, stream>>>(mu2d, mu_stride, keep, keep_stride, G, ntx,
                                                      nty, Sf, span, NB, Tpad, ws.mat,
                                                      ws.cell_slot);
    else
      k_bin_count<1024, 4><<<nblk, 1024, lds, stream>>>(mu2d, mu_stride, keep, keep_stride, G,
                                                        ntx, nty, Sf, span, NB, Tpad, ws.mat,
                                                        ws.cell_slot);
  }
  k_bin_colscan<<<(X + kChunk - 1) / kChunk, 1024, 0, stream>>>(ws.mat, nblk, X, ws.tot,
                                                                ws.within, ws.chunk_tot,
                                                                ws.nlist, 2, adv, b1, b2);
  const int ncls = (T + 1023) / 1024;
  ScatterArgs sc{mu2d, mu_stride, G, ntx, nty, NB, Tpad, K, ws.cblock, ncls, ws.cell_slot,
                 ws.mat, ws.tot, ws.within, ws.chunk_tot, ws.cell_start, ws.far_start, ws.recs,
                 ws.far_g, inv, ws.lists, ws.nlist, ws.key_hist, ws.tile_pos};
  k_bin_scatter<<<ncls + (max(G, T + 1) + 1023) / 1024, 1024, 0, stream>>>(sc);
  int kpow2 = 16;  // at least 16: the survivors are padded to a multiple of 16
  while (kpow2 < K) kpow2 <<= 1;
  int gbits = 1;
  while ((1ll << gbits) < (long long)(G > 1 ? G : 2)) ++gbits;
  const int hist_bins = span > (1 << kDigitBits) ? span : (1 << kDigitBits);
  const size_t heavy_lds = sizeof(unsigned long long) * ((size_t)kpow2 + kTieCap) +
                           sizeof(unsigned) * (size_t)hist_bins;
  const size_t light_lds =
      sizeof(unsigned long long) * (2 * (size_t)kpow2 + 8 + kGroups / 2) * (kSelThreads / 64);
  const size_t lds = heavy_lds > light_lds ? heavy_lds : light_lds;
  SelectArgs sa{ws.recs, ws.far_g, ws.cell_start, ws.far_start, ntx, nty, Sf, span, K, kpow2,
                gbits, idx, valid, count, ncand, inv, order, ws.key_hist, ws.tile_pos, ncls,
                proj, rec, pos_count};
  k_bin_select<kSelThreads><<<T, kSelThreads, lds, stream>>>(sa, ws.lists, ws.nlist);
  return launch_status();
}

// Fixed scratch of tts_assign_bins_noalloc: one copy per GPU, held until the process ends.
// Host code never uses the symbol's name as an address: scratch_base() looks up each device's
// copy once (hipGetSymbolAddress) and every launch takes that pointer.
constexpr size_t kScratchBytes = TTS_BIN_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices] = {};

// Device address of the current device's scratch (looked up on the first call on that device).
static int scratch_base(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return TTS_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return TTS_EINVAL;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return TTS_OK;
}

}  // namespace tts

extern "C" {

int tts_assign_bins(const float* mu2d, int mu_stride, const uint8_t* keep, int keep_stride,
                    int G, int H, int W, int S, int R, int K, int span, int32_t* idx,
                    uint8_t* valid, int32_t* count, int32_t* ncand, int32_t* inv,
                    int32_t* order, void* workspace, size_t workspace_bytes,
                    hipStream_t stream) {
  const int rc = bin_check(mu2d, mu_stride, keep, keep_stride, G, H, W, S, R, K, span, idx, valid);
  if (rc != TTS_OK) return rc;
  const int ntx = W / S, nty = H / S;
  if (!workspace || workspace_bytes < bin_ws_layout(G, ntx, nty, nullptr, nullptr))
    return TTS_EWORKSPACE;
  BinWorkspace ws;
  bin_ws_layout(G, ntx, nty, static_cast<char*>(workspace), &ws);
  return bin_run(mu2d, mu_stride, keep, keep_stride, G, H, W, S, K, span, idx, valid, count,
                 ncand, inv, order, nullptr, nullptr, nullptr, ws, false, stream);
}

int tts_assign_bins_noalloc(const float* mu2d, int mu_stride, const uint8_t* keep,
                            int keep_stride, int G, int H, int W, int S, int R, int K, int span,
                            int32_t* idx, uint8_t* valid, int32_t* count, int32_t* ncand,
                            int32_t* inv, int32_t* order, hipStream_t stream) {
  const int rc = bin_check(mu2d, mu_stride, keep, keep_stride, G, H, W, S, R, K, span, idx, valid);
  if (rc != TTS_OK) return rc;
  const int ntx = W / S, nty = H / S;
  if (bin_ws_layout(G, ntx, nty, nullptr, nullptr) > kScratchBytes) return TTS_ESCRATCH;
  void* base = nullptr;
  const int sc = scratch_base(&base);
  if (sc != TTS_OK) return sc;
  BinWorkspace ws;
  bin_ws_layout(G, ntx, nty, static_cast<char*>(base), &ws);
  return bin_run(mu2d, mu_stride, keep, keep_stride, G, H, W, S, K, span, idx, valid, count,
                 ncand, inv, order, nullptr, nullptr, nullptr, ws, false, stream);
}

int tts_tile_order(const int32_t* count, int T, int K, int32_t* order, hipStream_t stream) {
  if (T <= 0 || !count || !order) return TTS_EINVAL;
  if (K < 1 || K > kMaxK) return TTS_EK;
  k_tile_order<<<1, 1024, 0, stream>>>(count, T, K, order);
  return launch_status();
}

// Geometry forward + binning of one view (tts_geom_fwd_ex, then tts_assign_bins on proj's
// means and keep): with count blocks of 512 gaussians (G <= 131072) the count pass runs inside
// the geometry launch (k_geom_fwd_count), otherwise the two run as their own launches.  With
// slot_rec the select pass also writes the slot records and per-position counts.
int tts_geom_fwd_assign_bins(const float* params, const float* sh_rest, int sh_degree,
                             const float* depth_bt, int G, const float* camera, float near_z,
                             float blur, float* proj, uint8_t* keep, int32_t* step_adv,
                             float beta1, float beta2, int H, int W, int S, int R, int K,
                             int span, int32_t* idx, uint8_t* valid, int32_t* count,
                             int32_t* ncand, int32_t* inv, int32_t* order, float* slot_rec,
                             int32_t* pos_count, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !proj || !keep))) return TTS_EINVAL;
  if (slot_rec && (!pos_count || !order)) return TTS_EINVAL;
  if (sh_degree < 0 || sh_degree > 3 || (sh_degree > 0 && !sh_rest)) return TTS_ESH;
  if (G >= (1 << 30)) return TTS_EG;
  const int rc = bin_check(proj, 12, keep, 1, G, H, W, S, R, K, span, idx, valid);
  if (rc != TTS_OK) return rc;
  const int ntx = W / S, nty = H / S;
  if (!workspace || workspace_bytes < bin_ws_layout(G, ntx, nty, nullptr, nullptr))
    return TTS_EWORKSPACE;
  BinWorkspace ws;
  bin_ws_layout(G, ntx, nty, static_cast<char*>(workspace), &ws);
  // the count pass inside the geometry launch: blocks of 512 (small) or 4096 (large) gaussians
  const bool small = ws.cblock == CountSmall::kBlock;
  const bool fused = G > 0 && (small ? geom_fwd_count_lds(ws.NB, ws.Tpad)
                                     : geom_fwd_count_large_lds(ws.NB, ws.Tpad)) <= kMaxLdsBytes;
  const float Sf = static_cast<float>(S);
  int e;
  if (fused && small)
    e = launch_geom_fwd_count(params, sh_rest, sh_degree, depth_bt, G, camera, near_z, blur, proj,
                              keep, step_adv, beta1, beta2, ntx, nty, Sf, span, ws.NB, ws.Tpad,
                              ws.mat, ws.cell_slot, stream);
  else if (fused)
    e = launch_geom_fwd_count_large(params, sh_rest, sh_degree, depth_bt, G, camera, near_z, blur,
                                    proj, keep, step_adv, beta1, beta2, ntx, nty, Sf, span, ws.NB,
                                    ws.Tpad, ws.mat, ws.cell_slot, stream);
  else
    e = tts_geom_fwd_ex(params, sh_rest, sh_degree, depth_bt, G, camera, near_z, blur, proj, keep,
                        step_adv, beta1, beta2, stream);
  if (e != TTS_OK) return e;
  return bin_run(proj, 12, keep, 1, G, H, W, S, K, span, idx, valid, count, ncand, inv, order,
                 proj, slot_rec, pos_count, ws, fused, stream);
}

// The seam between two training steps (k_geom_bwd_adam_fwd_count): tts_geom_bwd_adam for
// camera_bwd, then tts_geom_fwd_ex for camera_fwd and the binning's count pass of that view
// into the workspace, in one launch (count blocks of 512 gaussians: G <= 131072).  The binning
// then finishes with tts_assign_bins_counted on the same workspace.
int tts_geom_bwd_adam_fwd_count(float* params, int G, const float* camera_bwd,
                                const float* camera_fwd, float near_z, float blur,
                                const float* gslot, const int32_t* inv, float* gparams, float* m,
                                float* v, const float* lr, const int32_t* step, float beta1,
                                float beta2, float eps, float* proj, uint8_t* keep, int H, int W,
                                int S, int R, int K, int span, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  if (G <= 0 || !params || !camera_bwd || !camera_fwd || !gslot || !inv || !m || !v || !lr ||
      !step || !proj || !keep)
    return TTS_EINVAL;
  if (count_block(G) != CountSmall::kBlock) return TTS_EG;
  // bin_check's table arguments are not written here: any non-null pointers pass its check
  const int rc = bin_check(proj, 12, keep, 1, G, H, W, S, R, K, span,
                           reinterpret_cast<const int32_t*>(proj), keep);
  if (rc != TTS_OK) return rc;
  const int ntx = W / S, nty = H / S;
  if (!workspace || workspace_bytes < bin_ws_layout(G, ntx, nty, nullptr, nullptr))
    return TTS_EWORKSPACE;
  BinWorkspace ws;
  bin_ws_layout(G, ntx, nty, static_cast<char*>(workspace), &ws);
  return launch_geom_seam(params, G, camera_bwd, camera_fwd, near_z, blur, gslot, inv, gparams,
                          m, v, lr, step, beta1, beta2, eps, proj, keep, ntx, nty,
                          static_cast<float>(S), span, ws.NB, ws.Tpad, ws.mat, ws.cell_slot,
                          stream);
}

// The binning passes after a count pass that already ran into the workspace (the seam launch
// above): column scan, scatter, select -- the rest of tts_geom_fwd_assign_bins, with the same
// outputs.  step_adv (optional): the training step's Adam step block, advanced by the column
// scan.
int tts_assign_bins_counted(const float* proj, const uint8_t* keep, int G, int H, int W, int S,
                            int R, int K, int span, int32_t* idx, uint8_t* valid, int32_t* count,
                            int32_t* ncand, int32_t* inv, int32_t* order, float* slot_rec,
                            int32_t* pos_count, int32_t* step_adv, float beta1, float beta2,
                            void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (G <= 0 || !proj || !keep) return TTS_EINVAL;
  if (slot_rec && (!pos_count || !order)) return TTS_EINVAL;
  if (count_block(G) != CountSmall::kBlock) return TTS_EG;
  const int rc = bin_check(proj, 12, keep, 1, G, H, W, S, R, K, span, idx, valid);
  if (rc != TTS_OK) return rc;
  const int ntx = W / S, nty = H / S;
  if (!workspace || workspace_bytes < bin_ws_layout(G, ntx, nty, nullptr, nullptr))
    return TTS_EWORKSPACE;
  BinWorkspace ws;
  bin_ws_layout(G, ntx, nty, static_cast<char*>(workspace), &ws);
  return bin_run(proj, 12, keep, 1, G, H, W, S, K, span, idx, valid, count, ncand, inv, order,
                 proj, slot_rec, pos_count, ws, true, stream, step_adv, beta1, beta2);
}

}  // extern "C"
