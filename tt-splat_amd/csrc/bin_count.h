// Binning's count pass as device code shared by the binning (k_bin_count, on loaded means) and
// the geometry forward that feeds it (k_geom_fwd_count, on the means it has just projected),
// with the cell / far classification it needs.  Float steps here are never contracted into
// FMAs, whatever the including file's flags: the cells must be those of
// tools/m4_train_binned.py:85-86 exactly.
#pragma once

#include <atomic>

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
  // plain operators: the pragma governs the expressions written in this scope (the bodies of
  // __fmul_rn / __fadd_rn, plain * and + in a header, keep the including file's contraction)
  const float dx = mx - cx;
  const float dy = my - cy;
  const float d2 = dx * dx + dy * dy;
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
#pragma clang fp contract(off)
  // reachable tile index in [lo, hi] whose centre is nearest m (centres (t + 0.5) S ascend)
  int t = lo;
  for (int k = lo + 1; k <= hi; ++k)
    if (fabsf(m - (static_cast<float>(k) + 0.5f) * S) < fabsf(m - (static_cast<float>(t) + 0.5f) * S)) t = k;
  return t;
}

__device__ __forceinline__ int classify(float mx, float my, float S, int ntx, int nty, int span,
                                        bool* far) {
#pragma clang fp contract(off)
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

// Count pass.  A block of NT threads takes NT/64 * 64 * PER consecutive gaussians; wave w owns
// the contiguous range [w * 64 * PER, (w + 1) * 64 * PER), PER rounds of 64 (so the block order
// (wave, round, lane) is g order).  Every round's loads are issued up front.
// Regular gaussians: per-cell counts in an LDS histogram and each gaussian's rank in its cell
// inside the block, in LDS-atomic order (any order serves: the select pass orders by key).
// Far gaussians: a rank inside the block that is stable in g order: lanes in order through
// ballots, rounds in order through a running per-cell count private to the wave, waves in order
// through the earlier waves' totals (one block barrier).
// The block writes its row of the count matrix mat[block][Tpad + NB]: the regular counts of the
// Tpad cells, then the far counts of the NB border cells.  No global atomics: k_bin_colscan
// turns the rows into per-block bases.
constexpr int kMaxLdsInts = 38912;   // count-pass LDS (Tpad + waves * NB ints, 152 KB)
constexpr int kMaxCountWaves = 16;
constexpr int kMaxBorder = 1024;     // border cells with far handling (one per scatter thread)
constexpr int kChunk = 64;           // column-scan chunk (cells)
constexpr int kMaxCountRows = 256;   // count blocks: small blocks while the matrix stays short

// Count-pass geometry: NT threads, PER rounds of 64 per wave.  Small blocks (256 x 2) spread a
// small G over many CUs; once that would make the count matrix longer than kMaxCountRows rows,
// large blocks (1024 x 4) keep it short.
template <int NT, int PER>
struct CountGeo {
  static constexpr int kWaves = NT / 64;
  static constexpr int kWaveSpan = 64 * PER;
  static constexpr int kBlock = kWaves * kWaveSpan;
};
using CountSmall = CountGeo<256, 2>;
using CountLarge = CountGeo<1024, 4>;
inline int count_block(int G) {
  return (G + CountSmall::kBlock - 1) / CountSmall::kBlock <= kMaxCountRows ? CountSmall::kBlock
                                                                            : CountLarge::kBlock;
}

__host__ __device__ __forceinline__ int pad_cells(int T) { return (T + kChunk - 1) / kChunk * kChunk; }

// The count pass of one block on its gaussians' means and keep flags, already at hand:
// mx/my/kv[i] belong to gaussian g0 + 64 i with g0 = block * kBlock + wave * kWaveSpan + lane
// (any value for g >= G).  s_lds holds Tpad + waves * NB ints; every thread must call.
template <int NT, int PER>
__device__ __forceinline__ void count_body(const float (&mx)[PER], const float (&my)[PER],
                                           const uint8_t (&kv)[PER], int G, int ntx, int nty,
                                           float S, int span, int NB, int Tpad, int* s_lds,
                                           int* __restrict__ mat, int2* __restrict__ cell_slot) {
  using C = CountGeo<NT, PER>;
  constexpr int kCountPerLane = PER;
  int* s_reg = s_lds;            // [Tpad] regular count per cell
  int* s_wrun = s_lds + Tpad;    // [waves][NB] far count per wave (running, then total)
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int g0 = blockIdx.x * C::kBlock + wave * C::kWaveSpan + lane;
  const int nl = Tpad + C::kWaves * NB;
  for (int c = threadIdx.x; c < nl; c += NT) s_lds[c] = 0;
  __syncthreads();
  int cell[kCountPerLane], rank[kCountPerLane];
  bool farv[kCountPerLane];
#pragma unroll
  for (int i = 0; i < kCountPerLane; ++i) {
    int c = -1;
    bool far = false;
    if (g0 + 64 * i < G && kv[i] != 0) {
      c = classify(mx[i], my[i], S, ntx, nty, span, &far);
      far = far && NB > 0;
    }
    cell[i] = c;
    farv[i] = far;
    rank[i] = 0;
  }
#pragma unroll
  for (int i = 0; i < kCountPerLane; ++i)
    if (cell[i] >= 0 && !farv[i]) rank[i] = atomicAdd(&s_reg[cell[i]], 1);
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
  }
  int* row = mat + (int64_t)blockIdx.x * (Tpad + NB);
  for (int c = threadIdx.x; c < Tpad; c += NT) row[c] = s_reg[c];
  for (int b = threadIdx.x; b < NB; b += NT) {
    int s = 0;
#pragma unroll
    for (int w = 0; w < C::kWaves; ++w) s += s_wrun[w * NB + b];
    row[Tpad + b] = s;
  }
#pragma unroll
  for (int i = 0; i < kCountPerLane; ++i) {
    const int g = g0 + 64 * i;
    if (g < G) cell_slot[g] = cell[i] >= 0 ? make_int2(cell[i], rank[i]) : make_int2(-1, 0);
  }
}


// Host side: the fused geometry forward + count pass (geometry.hip), for count blocks of
// CountSmall (count_block(G) == CountSmall::kBlock); proj/keep as tts_geom_fwd_ex, mat and
// cell_slot as k_bin_count.  geom_fwd_count_lds: its dynamic LDS request in bytes; callers fall
// back to the two-kernel path when that exceeds kMaxLdsBytes (one workgroup's LDS on gfx950).
constexpr size_t kMaxLdsBytes = 160 * 1024;

// A kernel's dynamic-LDS limit (per function and device) raised to kMaxLdsBytes once per device:
// the largest any call can ask for, so that callers on several host threads or streams never
// lower it under one another (setting each call's own size would race).  One LdsLimit per
// kernel instance; the first call on a device should not be under graph capture.
constexpr int kLdsDevices = 64;
struct LdsLimit {
  std::atomic<int> ready[kLdsDevices] = {};
};
inline int raise_lds_limit(const void* fn, LdsLimit& lim) {
  int dev = 0;
  const hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) return static_cast<int>(de);
  if (dev < 0 || dev >= kLdsDevices) return TTS_EINVAL;
  if (!lim.ready[dev].load()) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(kMaxLdsBytes));
    if (e != hipSuccess) return static_cast<int>(e);
    lim.ready[dev].store(1);
  }
  return 0;
}
size_t geom_fwd_count_lds(int NB, int Tpad);
int launch_geom_fwd_count(const float* params, const float* sh_rest, int sh_degree,
                          const float* depth_bt, int G, const float* camera, float near_z,
                          float blur, float* proj, uint8_t* keep, int32_t* step_adv, float b1,
                          float b2, int ntx, int nty, float S, int span, int NB, int Tpad,
                          int* mat, int2* cell_slot, hipStream_t stream);
// The same for the large count blocks (CountLarge: 1024 threads, 4096 gaussians per block).
size_t geom_fwd_count_large_lds(int NB, int Tpad);
int launch_geom_fwd_count_large(const float* params, const float* sh_rest, int sh_degree,
                                const float* depth_bt, int G, const float* camera, float near_z,
                                float blur, float* proj, uint8_t* keep, int32_t* step_adv,
                                float b1, float b2, int ntx, int nty, float S, int span, int NB,
                                int Tpad, int* mat, int2* cell_slot, hipStream_t stream);
// The step seam (geometry.hip): geometry backward + Adam of one view, then the geometry forward
// of the next view with the count pass, for count blocks of CountSmall.  Its LDS request
// (geom_seam_lds: the larger of the staged rows and the count pass's histogram) fits whenever
// bin_check accepts the grid.
size_t geom_seam_lds(int NB, int Tpad);
int launch_geom_seam(float* params, int G, const float* cam_b, const float* cam_f, float near_z,
                     float blur, const float* gslot, const int32_t* inv, float* gparams, float* m,
                     float* v, const float* lr, const int32_t* step, float b1, float b2,
                     float eps, float* proj, uint8_t* keep, int ntx, int nty, float S, int span,
                     int NB, int Tpad, int* mat, int2* cell_slot, hipStream_t stream);

}  // namespace tts
