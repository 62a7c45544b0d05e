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
// Passes (stream-ordered, no host round trip):
//   1. k_bin_count      cell and far flag of each gaussian; per-block LDS histograms, one global
//                       atomic per non-zero cell; each regular gaussian's rank in its cell,
//                       each far gaussian's rank among its block's far gaussians of the cell,
//                       in g order.
//   2. k_far_colscan    per border cell, exclusive scan of the far counts over count blocks.
//   3. k_bin_scan       one block: copy offsets and exclusive scans -> cell_start[T+1],
//                       far_start[T+1]; resets the counters for the next call.  When the tile
//                       grid fits its LDS (T <= 8192) it also classifies the tiles (a tile's
//                       candidates are the 3x3 box sum of the cell totals, formed as row
//                       3-sums then column 3-sums) and writes the heaviest-first tile order;
//                       larger grids run k_tile_classify / k_tile_order instead.
//   4. k_bin_scatter    regular gaussians -> (g, mu_x, mu_y) records, far -> g at their ranks:
//                       every cell's far ids end up ascending.
//   5. k_bin_select     one block per tile (below).
// The result does not depend on the order atomics land in.

#include <mutex>

#include "tts_common.h"

namespace tts {

constexpr int kMaxSpan = 8192;   // LDS histogram bins (13-bit qd2 field)
constexpr int kMaxK = 512;
constexpr int kQShift = 36;
constexpr int kJShift = 32;
constexpr int kFarBit = 30;      // cell_slot.x flag: the gaussian is far
constexpr int kDigitBits = 11;   // radix-select digit width (2048-bin LDS histogram)

__device__ __forceinline__ long long cell_raw(float mu, float S) {
  return f2i64_x86(floorf(__fdiv_rn(mu, S)));
}

__device__ __forceinline__ int clamp_cell(long long c, int n) {
  // clamp(int64(floor(mu / S)), 0, n - 1)   (tools/m4_train_binned.py:85-86)
  return static_cast<int>(c < 0 ? 0 : (c > n - 1 ? n - 1 : c));
}

// Quantised squared distance of (mx, my) to the centre of tile (tx, ty).
__device__ __forceinline__ int quant_dist2(float mx, float my, int tx, int ty, float S, int span) {
#pragma clang fp contract(off)
  // dist2 = fl(fl(dx*dx) + fl(dy*dy)), no contraction (tools/m4_train_binned.py:112-114)
  const float cx = (static_cast<float>(tx) + 0.5f) * S;
  const float cy = (static_cast<float>(ty) + 0.5f) * S;
  const float dx = __fsub_rn(mx, cx);
  const float dy = __fsub_rn(my, cy);
  const float d2 = __fadd_rn(__fmul_rn(dx, dx), __fmul_rn(dy, dy));
  long long q = f2i64_x86(d2);
  return static_cast<int>(q < 0 ? 0 : (q > span - 1 ? span - 1 : q));
}

// Border cells (only they can hold far gaussians) indexed 0..NB-1, a bijection for every grid
// shape (a single row or column is all border).
__host__ __device__ __forceinline__ int border_count(int ntx, int nty) {
  if (nty == 1) return ntx;
  if (ntx == 1) return nty;
  return 2 * ntx + 2 * (nty - 2);
}
__device__ __forceinline__ int border_index(int cx, int cy, int ntx, int nty) {
  if (nty == 1) return cx;
  if (ntx == 1) return cy;
  if (cy == 0) return cx;
  if (cy == nty - 1) return ntx + cx;
  if (cx == 0) return 2 * ntx + (cy - 1);
  return 2 * ntx + (nty - 2) + (cy - 1);
}
__device__ __forceinline__ int border_cell(int b, int ntx, int nty) {
  if (nty == 1 || ntx == 1) return b;
  if (b < ntx) return b;
  if (b < 2 * ntx) return (nty - 1) * ntx + (b - ntx);
  if (b < 2 * ntx + (nty - 2)) return (b - 2 * ntx + 1) * ntx;
  return (b - 2 * ntx - (nty - 2) + 1) * ntx + ntx - 1;
}

// Cell of a kept gaussian and whether it is far (clamped, and saturated for every tile its
// cell reaches).  qd2 is monotone in |dx| and |dy| separately (each rounding step is), so over
// the reachable tiles it is smallest at the one nearest in x and in y and largest at the one
// farthest in both; the float->int64 step maps d2 >= 2^63 (and NaN) to INT64_MIN, i.e. qd2 0.
// Hence: saturated everywhere <=> the nearest tile saturates and the farthest does not overflow.
__device__ __forceinline__ int nearest_in(float m, float S, int lo, int hi) {
  // reachable tile index in [lo, hi] whose centre is nearest m (centres (t + 0.5) S ascend)
  int t = lo;
  for (int k = lo + 1; k <= hi; ++k)
    if (fabsf(m - (static_cast<float>(k) + 0.5f) * S) < fabsf(m - (static_cast<float>(t) + 0.5f) * S)) t = k;
  return t;
}

__device__ __forceinline__ int classify(float mx, float my, float S, int ntx, int nty, int span,
                                        bool* far) {
  const long long rx = cell_raw(mx, S), ry = cell_raw(my, S);
  const int cx = clamp_cell(rx, ntx), cy = clamp_cell(ry, nty);
  bool f = (rx != cx) || (ry != cy);
  if (f) {
    const int x0 = max(cx - 1, 0), x1 = min(cx + 1, ntx - 1);
    const int y0 = max(cy - 1, 0), y1 = min(cy + 1, nty - 1);
    const int nx = nearest_in(mx, S, x0, x1), ny = nearest_in(my, S, y0, y1);
    // the farthest reachable centre in x is at one end of [x0, x1], likewise in y
    const int fx = fabsf(mx - (static_cast<float>(x0) + 0.5f) * S) >=
                   fabsf(mx - (static_cast<float>(x1) + 0.5f) * S) ? x0 : x1;
    const int fy = fabsf(my - (static_cast<float>(y0) + 0.5f) * S) >=
                   fabsf(my - (static_cast<float>(y1) + 0.5f) * S) ? y0 : y1;
    f = quant_dist2(mx, my, nx, ny, S, span) == span - 1 &&
        quant_dist2(mx, my, fx, fy, S, span) == span - 1;
  }
  *far = f;
  return cy * ntx + cx;
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(__lane_id()); }
__device__ __forceinline__ int first_lane(unsigned long long m) {
  return __ffsll(static_cast<long long>(m)) - 1;
}
__device__ __forceinline__ int read_lane(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

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

// Count pass.  Each block takes kCountBlock consecutive gaussians; wave w owns the contiguous
// range [w * kWaveSpan, (w + 1) * kWaveSpan) of them, kCountPerLane rounds of 64 (so the block
// order (wave, round, lane) is g order).  Every round's loads are issued up front.
// Regular gaussians: per-cell counts in LDS (REG_LDS) or global atomics, and the gaussian's rank
// in its cell (any order); the cells the block touched are listed as they are first counted, and
// each gets one global atomic at the end.
// Far gaussians: a rank that is stable in g order inside the block: lanes in order through
// ballots, rounds in order through a running per-cell count private to the wave, waves in order
// through the waves' totals (one block barrier).  The block's per-border-cell totals go to
// far_blk[b][block]; a column scan over blocks (k_far_colscan) then makes every cell's far list
// ascending in g.
constexpr int kCountPerLane = 2;
constexpr int kWaveSpan = 64 * kCountPerLane;
constexpr int kCountBlock = 4 * kWaveSpan;
constexpr int kMaxLdsCells = 12288;
constexpr int kMaxBorder = 1024;   // far handling needs 4 * NB ints of LDS

template <bool REG_LDS>
__global__ __launch_bounds__(256) void k_bin_count(const float* __restrict__ mu2d, int mu_stride,
                                                   const uint8_t* __restrict__ keep,
                                                   int keep_stride, int G, int ntx, int nty,
                                                   float S, int span, int NB,
                                                   int* __restrict__ reg_cnt,
                                                   int* __restrict__ far_blk, int nblk,
                                                   int2* __restrict__ cell_slot) {
  extern __shared__ int s_lds[];
  __shared__ int s_touched[kCountBlock];
  __shared__ int s_ntouched;
  const int T = ntx * nty;
  int* s_wrun = s_lds;            // [4][NB] far count per wave (running, then the wave total)
  int* s_reg = s_lds + 4 * NB;    // [T] (REG_LDS)
  const int nl = 4 * NB + (REG_LDS ? T : 0);
  for (int c = threadIdx.x; c < nl; c += blockDim.x) s_lds[c] = 0;
  if (threadIdx.x == 0) s_ntouched = 0;
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int g0 = blockIdx.x * kCountBlock + wave * kWaveSpan + lane;
  // loads from clamped indices, unconditionally, so that all of them are in flight at once
  float mx[kCountPerLane], my[kCountPerLane];
  uint8_t kv[kCountPerLane];
#pragma unroll
  for (int i = 0; i < kCountPerLane; ++i) {
    const int gc = min(g0 + 64 * i, G - 1);
    kv[i] = keep[(int64_t)gc * keep_stride];
    mx[i] = mu2d[(int64_t)gc * mu_stride];
    my[i] = mu2d[(int64_t)gc * mu_stride + 1];
  }
  bool kp[kCountPerLane];
#pragma unroll
  for (int i = 0; i < kCountPerLane; ++i) kp[i] = (g0 + 64 * i < G) && kv[i] != 0;
  int cell[kCountPerLane], rank[kCountPerLane];
  bool farv[kCountPerLane];
  // classification (ALU only)
#pragma unroll
  for (int i = 0; i < kCountPerLane; ++i) {
    int c = -1;
    bool far = false;
    if (kp[i]) {
      c = classify(mx[i], my[i], S, ntx, nty, span, &far);
      far = far && NB > 0;
    }
    cell[i] = c;
    farv[i] = far;
    rank[i] = 0;
  }
  // regular ranks: plain LDS atomics, all rounds in flight
  if (REG_LDS) {
#pragma unroll
    for (int i = 0; i < kCountPerLane; ++i)
      if (cell[i] >= 0 && !farv[i]) rank[i] = atomicAdd(&s_reg[cell[i]], 1);
    // a cell counted first by this lane goes on the block's touched list
#pragma unroll
    for (int i = 0; i < kCountPerLane; ++i) {
      const int p = wave_append(&s_ntouched, cell[i] >= 0 && !farv[i] && rank[i] == 0);
      if (p >= 0) s_touched[p] = cell[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < kCountPerLane; ++i)
      if (cell[i] >= 0 && !farv[i]) rank[i] = atomicAdd(&reg_cnt[cell[i]], 1);
  }
  // REG_LDS: once the block's regular counts are final, one global atomic per touched cell
  // (at most kCountBlock of them, two per thread) takes the block's base in the cell.  They are
  // issued here and their results used only after the far ranks, which they do not touch, so
  // the round trip overlaps that work.
  static_assert(kCountBlock <= 2 * 256, "two touched cells per thread");
  int tc0 = -1, tc1 = -1, tb0, tb1;  // tbK is set and read only when tcK >= 0
  if (REG_LDS) {
    __syncthreads();
    const int nt = s_ntouched;
    if ((int)threadIdx.x < nt) tc0 = s_touched[threadIdx.x];
    if ((int)threadIdx.x + 256 < nt) tc1 = s_touched[threadIdx.x + 256];
    if (tc0 >= 0) tb0 = atomicAdd(&reg_cnt[tc0], s_reg[tc0]);
    if (tc1 >= 0) tb1 = atomicAdd(&reg_cnt[tc1], s_reg[tc1]);
  }
  // far ranks inside the wave's range: per round, lanes of one cell are grouped by ballots
  // (registers only); each group's leader then adds the group to the wave's running count of
  // the cell with one LDS atomic, and the lanes take the returned base from their leader.
  // The group of a lane is matched on the bits of its border index b: one ballot per bit, so
  // the cost does not grow with the number of distinct far cells in the round.
  if (NB > 0) {
    int* wrun = s_wrun + wave * NB;
    const int nbits = 32 - __clz(max(NB - 1, 1));  // b < NB fits in nbits bits
#pragma unroll
    for (int i = 0; i < kCountPerLane; ++i) {
      const bool far = farv[i];
      const int b = far ? border_index(cell[i] % ntx, cell[i] / ntx, ntx, nty) : -1;
      unsigned long long m = __ballot(far);  // far lanes with every bit of b equal to this lane's
      for (int k = 0; k < nbits; ++k) {
        const bool bit = (b >> k) & 1;
        const unsigned long long bk = __ballot(far && bit);
        m &= bit ? bk : ~bk;
      }
      const int rw = __popcll(m & __lanemask_lt());
      const int cnt = __popcll(m);
      const int ldr = far ? first_lane(m) : lane;
      int base = 0;
      if (far && ldr == lane) base = atomicAdd(&wrun[b], cnt);
      base = __shfl(base, ldr);
      if (far) {
        rank[i] = base + rw;
        cell[i] |= 1 << kFarBit;
      }
    }
  }
  __syncthreads();
  // waves in order: a far gaussian's block rank adds the earlier waves' totals of its cell
  if (NB > 0) {
#pragma unroll
    for (int i = 0; i < kCountPerLane; ++i) {
      if (cell[i] >= 0 && (cell[i] >> kFarBit)) {
        const int c = cell[i] & ~(1 << kFarBit);
        const int b = border_index(c % ntx, c / ntx, ntx, nty);
        for (int w = 0; w < wave; ++w) rank[i] += s_wrun[w * NB + b];
      }
    }
    for (int b = threadIdx.x; b < NB; b += blockDim.x)
      far_blk[(int64_t)b * nblk + blockIdx.x] =
          s_wrun[b] + s_wrun[NB + b] + s_wrun[2 * NB + b] + s_wrun[3 * NB + b];
  }
  if (REG_LDS) {
    // each touched cell is listed once: this thread alone rewrites its entry with the base
    if (tc0 >= 0) s_reg[tc0] = tb0;
    if (tc1 >= 0) s_reg[tc1] = tb1;
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < kCountPerLane; ++i) {
    const int g = g0 + 64 * i;
    if (g >= G) continue;
    int2 cs = make_int2(-1, 0);
    if (cell[i] >= 0) {
      const bool far = (cell[i] >> kFarBit) & 1;
      cs = make_int2(cell[i], (REG_LDS && !far) ? s_reg[cell[i]] + rank[i] : rank[i]);
    }
    cell_slot[g] = cs;
  }
}

// Exclusive scan of far_blk[b][0..nblk) for each border cell b (one block per cell); the total
// is the cell's far count.
__global__ __launch_bounds__(256) void k_far_colscan(int* __restrict__ far_blk, int nblk,
                                                     int ntx, int nty,
                                                     int* __restrict__ far_cnt) {
  __shared__ int s_tmp[4];
  int* row = far_blk + (int64_t)blockIdx.x * nblk;
  int carry = 0;
  for (int b0 = 0; b0 < nblk; b0 += 256) {
    const int i = b0 + threadIdx.x;
    const int v = i < nblk ? row[i] : 0;
    int total;
    const int ex = block_excl_scan256(v, s_tmp, &total);
    if (i < nblk) row[i] = carry + ex;
    carry += total;
  }
  if (threadIdx.x == 0) far_cnt[border_cell(blockIdx.x, ntx, nty)] = carry;
}

// Cell offsets, one block: exclusive scans of the regular and far counts -> cell_start[T+1],
// far_start[T+1]; both counters are reset to zero for the next call.  Values are staged
// through LDS so every global access is coalesced.
//
// When the whole grid fits one chunk (T <= kScanChunk) the same block also classifies the tiles
// from the starts still in LDS (what k_tile_classify does otherwise): tiles with more than K
// candidates go to lists[0..nlist[0]), the others to lists[T-1], lists[T-2], ...; and, when
// `order` is given, it writes the tiles ordered by kept count min(candidates, K), heaviest first
// (a counting sort; the splat kernels' block -> tile map), so no separate order pass runs.
constexpr int kScanChunk = 8192;

__global__ __launch_bounds__(1024) void k_bin_scan(int* __restrict__ reg_cnt,
                                                   int* __restrict__ far_cnt,
                                                   int* __restrict__ cell_start,
                                                   int* __restrict__ far_start, int ntx, int nty,
                                                   int K, int fuse, int* __restrict__ lists,
                                                   int* __restrict__ nlist,
                                                   int32_t* __restrict__ order) {
  __shared__ int s_v[2][kScanChunk];
  __shared__ int s_tmp[32];
  __shared__ int s_n[kScanChunk];     // fused: cell totals, then their row 3-sums
  __shared__ int s_bins[kMaxK + 2];   // fused: counting-sort buckets
  const int T = ntx * nty;
  if (fuse) {
    // ---- T <= kScanChunk: counts, starts and the tile classification all in LDS ----
    int* s_r = s_v[0];
    int* s_f = s_v[1];
    for (int i = threadIdx.x; i < T; i += 1024) {
      const int r = reg_cnt[i], f = far_cnt[i];
      s_r[i] = r;
      s_f[i] = f;
      s_n[i] = r + f;
      reg_cnt[i] = 0;
      far_cnt[i] = 0;
    }
    for (int c = threadIdx.x; c <= K + 1; c += 1024) s_bins[c] = 0;
    __syncthreads();
    // thread = tiles [lo, lo + per): its partial sums of both counts, and the row 3-sums of the
    // cell totals (a tile's candidates are the 3x3 box sum of the totals around its cell)
    constexpr int kPer = kScanChunk / 1024;
    const int per = (T + 1023) / 1024;
    const int lo = threadIdx.x * per;
    int sr = 0, sf = 0, hs[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int t = lo + k;
      hs[k] = 0;
      if (k < per && t < T) {
        sr += s_r[t];
        sf += s_f[t];
        const int tx = t % ntx;
        hs[k] = s_n[t] + (tx > 0 ? s_n[t - 1] : 0) + (tx + 1 < ntx ? s_n[t + 1] : 0);
      }
    }
    int tr, tf, er, ef;  // barriers inside: every LDS read above is done
    block_excl_scan2<1024>(sr, sf, s_tmp, &er, &ef, &tr, &tf);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int t = lo + k;
      if (k < per && t < T) {
        const int r = s_r[t], f = s_f[t];
        s_r[t] = er;
        s_f[t] = ef;
        er += r;
        ef += f;
        s_n[t] = hs[k];
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < T; i += 1024) {
      cell_start[i] = s_r[i];
      far_start[i] = s_f[i];
    }
    if (threadIdx.x == 0) {
      cell_start[T] = tr;
      far_start[T] = tf;
    }
    // classification: candidates <= K -> light, else heavy.  Each thread takes its contiguous
    // tiles [lo, lo + per) again, and one block scan of its packed counts (heavy << 16 | light,
    // totals <= 8192) places them: heavy tiles to lists[0, ...), light ones to lists[T-1],
    // lists[T-2], ..., both in ascending tile order.  The kept count every tile ends with,
    // min(candidates, K), keys the heaviest-first order (histogram here, placement below).
    int ncs[kPer];
    int nh = 0, nlt = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int t = lo + k;
      ncs[k] = -1;
      if (k < per && t < T) {
        const int ty = t / ntx;
        const int nc = s_n[t] + (ty > 0 ? s_n[t - ntx] : 0) + (ty + 1 < nty ? s_n[t + ntx] : 0);
        ncs[k] = nc;
        nh += nc > K;
        nlt += nc <= K;
        if (order) agg_inc(s_bins, K - min(nc, K));
      }
    }
    int tot;
    const int ex = block_excl_scan<1024>((nh << 16) | nlt, s_tmp, &tot);
    int ph = ex >> 16, pl = ex & 0xffff;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (ncs[k] >= 0) {
        const int t = lo + k;
        if (ncs[k] > K) lists[ph++] = t;
        else lists[T - 1 - pl++] = t;
      }
    }
    if (threadIdx.x == 0) {
      nlist[0] = tot >> 16;
      nlist[1] = tot & 0xffff;
    }
    if (!order) return;
    // K + 1 <= 513 buckets: one per thread
    const int v = threadIdx.x <= K ? s_bins[threadIdx.x] : 0;
    int total;
    const int bx = block_excl_scan<1024>(v, s_tmp, &total);
    if (threadIdx.x <= K) s_bins[threadIdx.x] = bx;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (ncs[k] >= 0) order[agg_inc(s_bins, K - min(ncs[k], K))] = lo + k;
    return;
  }
  // ---- larger grids: chunked scans; k_tile_classify / k_tile_order run separately ----
  int carry[2] = {0, 0};
  for (int base = 0; base < T; base += kScanChunk) {
    const int n = min(kScanChunk, T - base);
    for (int i = threadIdx.x; i < n; i += 1024) {
      s_v[0][i] = reg_cnt[base + i];
      s_v[1][i] = far_cnt[base + i];
      reg_cnt[base + i] = 0;
      far_cnt[base + i] = 0;
    }
    __syncthreads();
    const int per = (n + 1023) / 1024;
    const int lo = threadIdx.x * per;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      int sum = 0;
      for (int k = 0; k < per; ++k)
        if (lo + k < n) sum += s_v[w][lo + k];
      int total;
      int ex = block_excl_scan<1024>(sum, s_tmp + 16 * w, &total) + carry[w];
      for (int k = 0; k < per; ++k) {
        if (lo + k < n) {
          const int v = s_v[w][lo + k];
          s_v[w][lo + k] = ex;
          ex += v;
        }
      }
      carry[w] += total;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 1024) {
      cell_start[base + i] = s_v[0][i];
      far_start[base + i] = s_v[1][i];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    cell_start[T] = carry[0];
    far_start[T] = carry[1];
    nlist[0] = 0;  // tile lists of k_tile_classify
    nlist[1] = 0;
  }
}

__global__ __launch_bounds__(256) void k_bin_scatter(const float* __restrict__ mu2d, int mu_stride,
                                                     int G, int ntx, int nty,
                                                     const int2* __restrict__ cell_slot,
                                                     const int* __restrict__ cell_start,
                                                     const int* __restrict__ far_start,
                                                     const int* __restrict__ far_blk, int nblk,
                                                     int4* __restrict__ recs,
                                                     int* __restrict__ far_g,
                                                     int32_t* __restrict__ inv) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  if (inv) {  // no slot yet: k_bin_select fills the kept (g, j) entries
#pragma unroll
    for (int j = 0; j < 9; ++j) inv[(int64_t)g * 9 + j] = -1;
  }
  const int2 cs = cell_slot[g];
  const float mx = mu2d[(int64_t)g * mu_stride], my = mu2d[(int64_t)g * mu_stride + 1];
  if (cs.x < 0) return;
  if (cs.x >> kFarBit) {
    const int c = cs.x & ~(1 << kFarBit);
    const int b = border_index(c % ntx, c / ntx, ntx, nty);
    far_g[far_start[c] + far_blk[(int64_t)b * nblk + g / kCountBlock] + cs.y] = g;
  } else {
    recs[cell_start[cs.x] + cs.y] = make_int4(g, __float_as_int(mx), __float_as_int(my), 0);
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
__device__ __forceinline__ void for_each_candidate(const TileCells& tc,
                                                   const int4* __restrict__ recs, int tx, int ty,
                                                   float S, int span, int tid, F&& f) {
  const int n = tc.pre[9];
  int i = tid;
  for (; i + 3 * NT < n; i += 4 * NT) {
    const int j0 = stencil_of(tc, i), j1 = stencil_of(tc, i + NT);
    const int j2 = stencil_of(tc, i + 2 * NT), j3 = stencil_of(tc, i + 3 * NT);
    const int4 r0 = load_candidate(tc, recs, i, j0);
    const int4 r1 = load_candidate(tc, recs, i + NT, j1);
    const int4 r2 = load_candidate(tc, recs, i + 2 * NT, j2);
    const int4 r3 = load_candidate(tc, recs, i + 3 * NT, j3);
    f(record_key(r0, j0, tx, ty, S, span));
    f(record_key(r1, j1, tx, ty, S, span));
    f(record_key(r2, j2, tx, ty, S, span));
    f(record_key(r3, j3, tx, ty, S, span));
  }
  for (; i < n; i += NT) {
    const int j = stencil_of(tc, i);
    f(record_key(load_candidate(tc, recs, i, j), j, tx, ty, S, span));
  }
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
};

// Light tile (n <= K candidates: all survive), one wave: collect the keys in LDS, then place
// them by rank.
__device__ __forceinline__ void select_light(int t, const SelectArgs& a, TileCells& tc,
                                             unsigned long long* keys, int* fill) {
  const int lane = lane_id();
  const int tx = t % a.ntx, ty = t / a.ntx;
  load_tile_cells(tc, tx, ty, a.ntx, a.nty, a.cell_start, a.far_start);
  if (lane == 0) *fill = 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int nfar = tc.fpre[9];
  const int satq = a.span - 1;
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
  for (int s = lane; s < a.K; s += 64) {
    if (s < m) {
      const unsigned long long key = keys[s];
      int rank = 0;
      for (int e = 0; e < m; ++e) rank += (keys[e] < key) ? 1 : 0;
      const int g = static_cast<int32_t>(key & 0xffffffffull);
      a.idx[base + rank] = g;
      if (a.inv) a.inv[(int64_t)g * 9 + ((key >> kJShift) & 15ull)] = static_cast<int32_t>(base + rank);
      a.valid[base + rank] = 1;
    } else {
      a.idx[base + s] = 0;
      a.valid[base + s] = 0;
    }
  }
  if (lane == 0) {
    if (a.count) a.count[t] = m;
    if (a.ncand) a.ncand[t] = m;
  }
}

// Tiles with more than K candidates go to lists[0..nlist[0]), the others to
// lists[T-1], lists[T-2], ... (nlist[1] of them).  nlist is zeroed by k_bin_scan.
__global__ __launch_bounds__(256) void k_tile_classify(const int* __restrict__ cell_start,
                                                       const int* __restrict__ far_start,
                                                       int ntx, int nty, int K,
                                                       int* __restrict__ lists,
                                                       int* __restrict__ nlist) {
  const int T = ntx * nty;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  int n = 0;
  if (t < T) {
    const int tx = t % ntx, ty = t / ntx;
    for (int j = 0; j < 9; ++j) {
      const int cx = tx - (j % 3 - 1), cy = ty - (j / 3 - 1);
      if (cx >= 0 && cx < ntx && cy >= 0 && cy < nty) {
        const int c = cy * ntx + cx;
        n += cell_start[c + 1] - cell_start[c] + far_start[c + 1] - far_start[c];
      }
    }
  }
  const int ph = wave_append(&nlist[0], t < T && n > K);
  if (ph >= 0) lists[ph] = t;
  const int pl = wave_append(&nlist[1], t < T && n <= K);
  if (pl >= 0) lists[T - 1 - pl] = t;
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
template <int NT>
__global__ __launch_bounds__(NT) void k_bin_select(SelectArgs a, const int* __restrict__ lists,
                                                   const int* __restrict__ nlist) {
  extern __shared__ unsigned char s_dyn[];
  __shared__ TileCells tcs[NT / 64];
  __shared__ int s_wfill[NT / 64];
  const int T = a.ntx * a.nty;
  const int nh = nlist[0], nl = nlist[1];
  if (static_cast<int>(blockIdx.x) >= nh) {
    const int g0 = (static_cast<int>(blockIdx.x) - nh) * (NT / 64);
    if (g0 >= nl) return;
    const int w = threadIdx.x >> 6;
    if (g0 + w < nl) {
      unsigned long long* keys = reinterpret_cast<unsigned long long*>(s_dyn) + w * a.kpow2;
      select_light(lists[T - 1 - (g0 + w)], a, tcs[w], keys, &s_wfill[w]);
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

  const int t = lists[blockIdx.x];
  const int tx = t % a.ntx, ty = t / a.ntx;
  if (threadIdx.x < 64) load_tile_cells(tc, tx, ty, a.ntx, a.nty, a.cell_start, a.far_start);
  if (threadIdx.x == 0) {
    s_fill = 0;
    s_tfill = 0;
  }
  if (threadIdx.x < 9) s_sat[threadIdx.x] = 0;
  __syncthreads();
  const int nreg = tc.pre[9], nfar = tc.fpre[9];
  const int n = nreg + nfar;
  const int satq = span - 1;

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
    for (int b = threadIdx.x; b < span; b += NT) s_hist[b] = 0;
    __syncthreads();
    for_each_candidate<NT>(tc, recs, tx, ty, S, span, threadIdx.x, [&](unsigned long long key) {
      const unsigned q = static_cast<unsigned>(key >> kQShift);
      hist_add(s_hist, q);
      if (static_cast<int>(q) == satq)
        agg_inc(s_sat, static_cast<int>((key >> kJShift) & 15ull));
    });
    __syncthreads();
    if (threadIdx.x == 0) s_hist[satq] += nfar;
    __syncthreads();
    find_rank_bin<NT>(s_hist, span, K - 1, s_tmp, s_out);
    const int qb = s_out[0], before = s_out[1], cnt = s_out[2];
    const int r = K - 1 - before;  // rank of the K-th key inside bin qb
    if (qb < satq) {
      // ---------------- tie bin of regular candidates only ----------------
      const bool in_lds = cnt <= kTieCap;
      for_each_candidate<NT>(tc, recs, tx, ty, S, span, threadIdx.x, [&](unsigned long long key) {
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
      const unsigned thr = stop >= 32 ? 0u : (prefix >> stop);
      if (in_lds) {
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
      for_each_candidate<NT>(tc, recs, tx, ty, S, span, threadIdx.x, [&](unsigned long long key) {
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
      if (in_lds) {
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
  for (int s = threadIdx.x; s < K; s += NT) {
    if (s < m) {
      const unsigned long long key = s_keys[s];
      int rank = 0;
      for (int e = 0; e < m; ++e) rank += (s_keys[e] < key) ? 1 : 0;
      const int g = static_cast<int32_t>(key & 0xffffffffull);
      a.idx[base + rank] = g;
      if (a.inv) a.inv[(int64_t)g * 9 + ((key >> kJShift) & 15ull)] = static_cast<int32_t>(base + rank);
      a.valid[base + rank] = 1;
    } else {
      a.idx[base + s] = 0;
      a.valid[base + s] = 0;
    }
  }
  if (threadIdx.x == 0) {
    if (a.count) a.count[t] = m;
    if (a.ncand) a.ncand[t] = n;
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
  int* reg_cnt;     // [T]   zero between calls
  int* far_cnt;     // [T]   zero between calls
  int* cell_start;  // [T+1]
  int* far_start;   // [T+1]
  int* far_blk;     // [NB][nblk] far count per (border cell, count block), then its column scan
  int2* cell_slot;  // [G]
  int4* recs;       // [G]
  int* far_g;       // [G]
  int* lists;       // [T]  heavy tiles from the front, light tiles from the back
  int* nlist;       // [2]  heavy, light counts
  int NB;           // border cells with far handling (0: every gaussian is regular)
  int nblk;         // count-pass blocks
};

// Far handling is on when the border fits the count pass's LDS tables and the per-block table
// stays small.
inline int far_border_cells(int G, int ntx, int nty) {
  const int NB = border_count(ntx, nty);
  const long long nblk = (G + kCountBlock - 1) / kCountBlock;
  return (NB <= kMaxBorder && nblk * NB <= (1ll << 26)) ? NB : 0;
}


inline size_t bin_ws_layout(int G, int ntx, int nty, char* base, BinWorkspace* ws) {
  const int T = ntx * nty;
  const int NB = far_border_cells(G, ntx, nty);
  const int nblk = (G + kCountBlock - 1) / kCountBlock;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  const size_t g1 = (size_t)(G > 0 ? G : 1);
  char* a = take(sizeof(int) * (size_t)T);
  char* a2 = take(sizeof(int) * (size_t)T);
  char* b = take(sizeof(int) * ((size_t)T + 1));
  char* b2 = take(sizeof(int) * ((size_t)T + 1));
  char* f = take(sizeof(int) * ((size_t)NB * nblk + 1));
  char* c = take(sizeof(int2) * g1);
  char* d = take(sizeof(int4) * g1);
  char* e = take(sizeof(int) * g1);
  char* l = take(sizeof(int) * (size_t)T);
  char* nl = take(sizeof(int) * 2);
  if (ws) {
    ws->reg_cnt = reinterpret_cast<int*>(a);
    ws->far_cnt = reinterpret_cast<int*>(a2);
    ws->cell_start = reinterpret_cast<int*>(b);
    ws->far_start = reinterpret_cast<int*>(b2);
    ws->far_blk = reinterpret_cast<int*>(f);
    ws->NB = NB;
    ws->nblk = nblk;
    ws->cell_slot = reinterpret_cast<int2*>(c);
    ws->recs = reinterpret_cast<int4*>(d);
    ws->far_g = reinterpret_cast<int*>(e);
    ws->lists = reinterpret_cast<int*>(l);
    ws->nlist = reinterpret_cast<int*>(nl);
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
  if (R != 1) return TTS_ERADIUS;
  if (K < 1 || K > kMaxK) return TTS_EK;
  if (span < 1 || span > kMaxSpan) return TTS_ESPAN;
  return TTS_OK;
}

__global__ void k_zero_i32(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// The binning passes on a laid-out workspace (arguments already checked).  clear_counters: the
// per-cell counters (reg_cnt, far_cnt) are zeroed by a fill kernel first instead of being
// trusted to be zero from the previous call.
static int bin_run(const float* mu2d, int mu_stride, const uint8_t* keep, int keep_stride,
                   int G, int H, int W, int S, int K, int span, int32_t* idx, uint8_t* valid,
                   int32_t* count, int32_t* ncand, int32_t* inv, int32_t* order,
                   const BinWorkspace& ws, bool clear_counters, hipStream_t stream) {
  const int ntx = W / S, nty = H / S, T = ntx * nty;
  if (clear_counters) {
    // reg_cnt and far_cnt are the first two sub-buffers: one fill covers both
    const int n = static_cast<int>((reinterpret_cast<char*>(ws.far_cnt) -
                                    reinterpret_cast<char*>(ws.reg_cnt)) / sizeof(int)) + T;
    k_zero_i32<<<grid1d(n, 256), 256, 0, stream>>>(ws.reg_cnt, n);
  }
  const float Sf = static_cast<float>(S);
  const int NB = ws.NB;
  const int nblk = ws.nblk;
  if (G > 0) {
    const bool reg_lds = T + 4 * NB <= kMaxLdsCells;
    const size_t lds = sizeof(int) * (size_t)(4 * NB + (reg_lds ? T : 0));
    if (reg_lds)
      k_bin_count<true><<<nblk, 256, lds, stream>>>(mu2d, mu_stride, keep, keep_stride, G, ntx,
                                                    nty, Sf, span, NB, ws.reg_cnt, ws.far_blk,
                                                    nblk, ws.cell_slot);
    else
      k_bin_count<false><<<nblk, 256, lds, stream>>>(mu2d, mu_stride, keep, keep_stride, G, ntx,
                                                     nty, Sf, span, NB, ws.reg_cnt, ws.far_blk,
                                                     nblk, ws.cell_slot);
    if (NB > 0) k_far_colscan<<<NB, 256, 0, stream>>>(ws.far_blk, nblk, ntx, nty, ws.far_cnt);
  }
  const int fuse = T <= kScanChunk;
  k_bin_scan<<<1, 1024, 0, stream>>>(ws.reg_cnt, ws.far_cnt, ws.cell_start, ws.far_start, ntx,
                                     nty, K, fuse, ws.lists, ws.nlist, order);
  if (G > 0) {
    k_bin_scatter<<<grid1d(G, 256), 256, 0, stream>>>(mu2d, mu_stride, G, ntx, nty, ws.cell_slot,
                                                      ws.cell_start, ws.far_start, ws.far_blk,
                                                      nblk, ws.recs, ws.far_g, inv);
  }
  int kpow2 = 1;
  while (kpow2 < K) kpow2 <<= 1;
  int gbits = 1;
  while ((1ll << gbits) < (long long)(G > 1 ? G : 2)) ++gbits;
  const int hist_bins = span > (1 << kDigitBits) ? span : (1 << kDigitBits);
  const size_t heavy_lds = sizeof(unsigned long long) * ((size_t)kpow2 + kTieCap) +
                           sizeof(unsigned) * (size_t)hist_bins;
  const size_t light_lds = sizeof(unsigned long long) * (size_t)kpow2 * (kSelThreads / 64);
  const size_t lds = heavy_lds > light_lds ? heavy_lds : light_lds;
  if (!fuse)
    k_tile_classify<<<grid1d(T, 256), 256, 0, stream>>>(ws.cell_start, ws.far_start, ntx, nty, K,
                                                        ws.lists, ws.nlist);
  SelectArgs sa{ws.recs, ws.far_g, ws.cell_start, ws.far_start, ntx, nty, Sf, span, K, kpow2,
                gbits, idx, valid, count, ncand, inv};
  k_bin_select<kSelThreads><<<T, kSelThreads, lds, stream>>>(sa, ws.lists, ws.nlist);
  // large grids: the order pass runs on the kept counts (the fused scan wrote it otherwise)
  if (order && !fuse) k_tile_order<<<1, 1024, 0, stream>>>(count, T, K, order);
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
  if (order && ntx * nty > kScanChunk && !count) return TTS_EINVAL;
  if (!workspace || workspace_bytes < bin_ws_layout(G, ntx, nty, nullptr, nullptr))
    return TTS_EWORKSPACE;
  BinWorkspace ws;
  bin_ws_layout(G, ntx, nty, static_cast<char*>(workspace), &ws);
  return bin_run(mu2d, mu_stride, keep, keep_stride, G, H, W, S, K, span, idx, valid, count,
                 ncand, inv, order, ws, false, stream);
}

int tts_assign_bins_noalloc(const float* mu2d, int mu_stride, const uint8_t* keep,
                            int keep_stride, int G, int H, int W, int S, int R, int K, int span,
                            int32_t* idx, uint8_t* valid, int32_t* count, int32_t* ncand,
                            int32_t* inv, int32_t* order, hipStream_t stream) {
  const int rc = bin_check(mu2d, mu_stride, keep, keep_stride, G, H, W, S, R, K, span, idx, valid);
  if (rc != TTS_OK) return rc;
  const int ntx = W / S, nty = H / S;
  if (order && ntx * nty > kScanChunk && !count) return TTS_EINVAL;
  if (bin_ws_layout(G, ntx, nty, nullptr, nullptr) > kScratchBytes) return TTS_ESCRATCH;
  void* base = nullptr;
  const int sc = scratch_base(&base);
  if (sc != TTS_OK) return sc;
  BinWorkspace ws;
  bin_ws_layout(G, ntx, nty, static_cast<char*>(base), &ws);
  return bin_run(mu2d, mu_stride, keep, keep_stride, G, H, W, S, K, span, idx, valid, count,
                 ncand, inv, order, ws, true, stream);
}

int tts_tile_order(const int32_t* count, int T, int K, int32_t* order, hipStream_t stream) {
  if (T <= 0 || !count || !order) return TTS_EINVAL;
  if (K < 1 || K > kMaxK) return TTS_EK;
  k_tile_order<<<1, 1024, 0, stream>>>(count, T, K, order);
  return launch_status();
}

}  // extern "C"
