// Photometric loss gradient: L = (1-l)*mean|x-y| + l*(1 - mean SSIM(clamp x, clamp y)).
// SSIM: 11-tap gaussian window (sigma 1.5), valid borders, C1 = 1e-4, C2 = 9e-4
// (spike/metrics.py:6-28; the manual gradient of tools/loss_manual.py:76-103).
//
// The target's statistics mu_y = G*y and s_y = G*y^2 - mu_y^2 depend on the target only:
// k_loss_target_stats computes them (with a channel-planar copy of the target) whenever the
// target changes -- the reference's resident trainer recomputes its muy/sy maps on each view
// switch (recompute_gt_stats, tools/resident_traced.py:320-325,677-678); a caller may also keep
// one set per view.  The step kernel then filters x, x^2 and xy only.
//
// k_loss_fused: a block owns a TH x 64 tile of gradient pixels of one colour channel and runs
// the whole chain on it, the SSIM map region it needs (the tile plus the 10-pixel halo above and
// left of it) recomputed rather than exchanged through memory:
//   1 vertical filter of x, x^2, xy straight from global memory (a thread = one input column,
//     a run of map rows; its loads in flight together)            -> V[3][TH+10][84]  (LDS)
//   2 horizontal filter, S and its partials dS/dmu_x, dS/dE[x^2], dS/dE[xy] (a thread = a run
//     of map columns on one map row)                              -> D[3][TH+10][74]  (LDS)
//   3 transposed horizontal filter of the partials               -> T[3][TH+10][64]  (LDS)
//   4 transposed vertical filter (a thread = one gradient column, a run of rows, so its image
//     loads and gradient stores are coalesced), combined as dmeanS/dx = (T'A + 2 x T'B +
//     y T'C) / Ns, gated by 0 <= x <= 1 (the clamp), plus the L1 term (1-l) sign(x-y) / N.
// V, D and T share one 51 KB LDS buffer (each written after a barrier that ends the reads of
// the one before; three blocks fit a CU); the loads a phase needs from global memory are issued
// a phase ahead.  Each block also sums S over the map pixels of its tile and |x - y| over its
// pixels.  Nothing is exchanged between blocks: the kernel needs no workspace.

#include "tts_common.h"

namespace tts {

constexpr int kWin = 11;
constexpr int kHalo = kWin - 1;
constexpr int kTW = 64;                 // gradient tile width
constexpr int kMC = kTW + kHalo;        // 74 map columns
constexpr int kIC = kTW + 2 * kHalo;    // 84 input columns
constexpr int kVS = kIC + 1;            // LDS row strides (odd: column walks spread over banks)
constexpr int kDS = kMC + 1;
constexpr int kHC = 15;                 // phase 2: map columns per thread (5 runs cover 74)
constexpr int kHC3 = 13;                // phase 3: gradient columns per thread (5 runs cover 64)
constexpr int kTS = kTW + 1;
constexpr float kC1 = 1e-4f;
constexpr float kC2 = 9e-4f;

struct Taps {
  float g[kWin];
};

__device__ __forceinline__ float clamp01(float v) { return fminf(fmaxf(v, 0.f), 1.f); }

// Buffer-resource addressing: one 32-bit byte offset per lane.  A resource's size is its bound:
// a load at an offset at or past it reads 0.  Images are under 2^31 bytes (the entry points
// check), so an offset computed from a row above the image (negative, taken as unsigned) or
// kOOB plus any in-image offset stays past the bound.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr unsigned kOOB = 0x80000000u;
__device__ __forceinline__ Rsrc rsrc(const float* p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float bld(Rsrc r, unsigned voff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}
__device__ __forceinline__ void bst(Rsrc r, unsigned voff, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff, 0, 0);
}

// ------------------------------------------------------------------ target statistics ------
// One block per (64 x 16 tile of the valid map, channel): mu_y and s_y of the clamped target ->
// stats[2][3][Wo][Ho], each channel's planes column-major (the step kernel reads them along map
// rows per lane).
constexpr int kSW = 64, kSH = 16, kSR = 6;   // tile, vertical run (3 runs cover 16 rows)
__global__ __launch_bounds__(256) void k_loss_target_stats(const float* __restrict__ y, int H,
                                                           int W, int tiles_x, Taps taps,
                                                           float* __restrict__ stats) {
  __shared__ float V[2][kSH][kSW + kHalo + 1];
  const int Ho = H - kHalo, Wo = W - kHalo;
  const int t = blockIdx.x / 3, ch = blockIdx.x - 3 * t;
  const int R0 = (t / tiles_x) * kSH, C0 = (t % tiles_x) * kSW;
  const int tid = threadIdx.x;
  const Rsrc ys = rsrc(y, (size_t)H * W * 12);
  if (tid < 3 * (kSW + kHalo)) {
    const int j = tid % (kSW + kHalo), m0 = (tid / (kSW + kHalo)) * kSR;
    const int gc = C0 + j;
    const unsigned base = gc < W ? (unsigned)((((R0 + m0) * W + gc) * 3 + ch) * 4) : kOOB;
    float v[kSR + kHalo];
#pragma unroll
    for (int k = 0; k < kSR + kHalo; ++k) v[k] = clamp01(bld(ys, base + (unsigned)k * W * 12u));
    float a[2][kSR];
#pragma unroll
    for (int o = 0; o < kSR; ++o) a[0][o] = a[1][o] = 0.f;
#pragma unroll
    for (int k = 0; k < kSR + kHalo; ++k) {
      const float b = v[k], bb = b * b;
#pragma unroll
      for (int o = 0; o < kSR; ++o) {
        const int tap = k - o;
        if (tap >= 0 && tap < kWin) {
          a[0][o] += taps.g[tap] * b;
          a[1][o] += taps.g[tap] * bb;
        }
      }
    }
#pragma unroll
    for (int o = 0; o < kSR; ++o) {
      if (m0 + o < kSH) {
        V[0][m0 + o][j] = a[0][o];
        V[1][m0 + o][j] = a[1][o];
      }
    }
  }
  __syncthreads();
  const int m = tid >> 4, q0 = (tid & 15) * 4;
  float f[2][4];
#pragma unroll
  for (int o = 0; o < 4; ++o) f[0][o] = f[1][o] = 0.f;
#pragma unroll
  for (int k = 0; k < 4 + kHalo; ++k) {
    const float a = V[0][m][q0 + k], b = V[1][m][q0 + k];
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      const int tap = k - o;
      if (tap >= 0 && tap < kWin) {
        f[0][o] += taps.g[tap] * a;
        f[1][o] += taps.g[tap] * b;
      }
    }
  }
  const int gm = R0 + m;
  const size_t plane = (size_t)Ho * Wo;
#pragma unroll
  for (int o = 0; o < 4; ++o) {
    const int gq = C0 + q0 + o;
    if (gm < Ho && gq < Wo) {
      const size_t i = (size_t)gq * Ho + gm;   // column-major: a column's rows are contiguous
      stats[(size_t)ch * plane + i] = f[0][o];
      stats[(size_t)(3 + ch) * plane + i] = f[1][o] - f[0][o] * f[0][o];
    }
  }
}

// The target channel-planar ([3][H][W], after the statistics planes): the step kernel's loads of
// one channel then touch contiguous floats (the interleaved image spreads a wave's 64 columns
// over six cache lines per load).
__global__ __launch_bounds__(256) void k_loss_target_planar(const float* __restrict__ y,
                                                            int64_t n, float* __restrict__ yp) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  yp[i] = y[i * 3];
  yp[n + i] = y[i * 3 + 1];
  yp[2 * n + i] = y[i * 3 + 2];
}

// Random-background compositing of a training target (the reference's --random-bg,
// tools/resident_traced.py:182-185,671-674): bg = three uniforms from Philox4x32-10, counter
// (view, step[0], kTagBg, 0), key (seed, 0) -- the step count is read on the device, so a
// replayed graph draws a new background every step; target = premult + trans * bg per channel,
// from rgba_pm [H,W,4] = (alpha r, alpha g, alpha b, 1 - alpha), each product and sum rounded
// once as torch's CPU arithmetic does; bg4[1..3] = bg, the numerator background colour the splat
// forward reads (bg4[0], w_b, is left alone).
__global__ __launch_bounds__(256) void k_composite_random_bg(const float4* __restrict__ rgba_pm,
                                                             int64_t n,
                                                             const int32_t* __restrict__ step,
                                                             uint32_t view, uint32_t seed,
                                                             float* __restrict__ bg4,
                                                             float* __restrict__ target) {
#pragma clang fp contract(off)  // pm + tr * bg rounded twice, as torch's CPU ops round it
  const Philox4 p = philox4x32_10(view, (uint32_t)step[0], kTagBg, 0u, seed, 0u);
  const float b0 = (float)u01d(p.w[0]), b1 = (float)u01d(p.w[1]), b2 = (float)u01d(p.w[2]);
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i == 0) {
    bg4[1] = b0;
    bg4[2] = b1;
    bg4[3] = b2;
  }
  if (i >= n) return;
  const float4 v = rgba_pm[i];
  target[i * 3 + 0] = v.x + v.w * b0;
  target[i * 3 + 1] = v.y + v.w * b1;
  target[i * 3 + 2] = v.z + v.w * b2;
}

// ------------------------------------------------------------------ fused step kernel ------
// Tile order.  Neighbouring tiles read the same halo lines (20 of a tile's 84 input columns,
// 20 of its TH + 20 input rows), so the order runs vertical strips kStrip tiles wide, row-major
// inside a strip, and xcd_item hands each XCD one contiguous run of that order: a tile's left
// and upper neighbours run on the same XCD a few tiles earlier, while their lines are still in
// its L2 (about 32 tiles are resident per XCD, six strip rows).  Measured at 832 x 1264: L2
// fills per launch 93 MB in row-major order, 68 MB with kStrip = 5 (2: 78 MB, 4: 70 MB).
constexpr int kStrip = 5;
__device__ __forceinline__ int strip_tile(int s, int tiles_x, int tiles_y) {
  const int per = tiles_y * kStrip;
  const int k = s / per, r = s - k * per;
  const int w = min(kStrip, tiles_x - k * kStrip);   // the last strip may be narrower
  const int row = r / w;
  return row * tiles_x + k * kStrip + (r - row * w);
}

template <int TH>
struct FGeo {
  static constexpr int MR = TH + kHalo;              // map rows of the region
  static constexpr int VR = (MR + 2) / 3;            // phase 1: map rows per thread (3 runs)
  static constexpr int TR4 = (TH + 3) / 4;           // phase 4: gradient rows per thread
  static constexpr int N2 = 5 * MR;                  // phase 2 and 3 threads
  static constexpr int TP = 4 * TR4 + kHalo;         // T rows per plane (phase 4 reads past MR)
  static constexpr int kV = 3 * MR * kVS;            // floats of V
  static_assert(3 * MR * kDS + kDS <= kV && 3 * TP * kTS <= kV, "D and T reuse V's space");
  static_assert(3 * kIC <= 256 && N2 <= 256, "one pass each");
  static_assert(5 * kHC >= kMC && 5 * kHC3 >= kTW && 3 * VR >= MR && 4 * TR4 >= TH, "cover");
  static constexpr size_t lds_bytes = sizeof(float) * (size_t)kV;
};

template <int TH>
__global__ __launch_bounds__(256) void k_loss_fused(const float* __restrict__ x,
                                                    const float* __restrict__ y,
                                                    const float* __restrict__ stats, int H,
                                                    int W, int tiles_x, int n_items, Taps taps,
                                                    float lambda, float inv_n, float inv_ns,
                                                    float* __restrict__ gout,
                                                    float* __restrict__ partials) {
  using G = FGeo<TH>;
  extern __shared__ float s_lds[];
  float* V = s_lds;
  float* D = s_lds;
  float* T = s_lds;
  __shared__ float s_fsum[8];
  // the taps in VGPRs (an opaque copy, so they are not folded back into SGPR operands): on
  // gfx950 a v_fmac_f32 reading an SGPR issues at half the rate of one reading only VGPRs and
  // constants (measured: 4.3 vs 2.7 cycles per wave64 instruction), and the filters are FMAs
  Taps vt;
#pragma unroll
  for (int i = 0; i < kWin; ++i) asm volatile("v_mov_b32 %0, %1" : "=v"(vt.g[i]) : "s"(taps.g[i]));
  // items: (tile in strip order, channel), channels innermost so a tile's three blocks share
  // cache lines
  const int item = xcd_item(blockIdx.x, n_items);
  const int ord = item / 3, ch = item - 3 * ord;
  const int tile = strip_tile(ord, tiles_x, n_items / (3 * tiles_x));
  const int R0 = (tile / tiles_x) * TH, C0 = (tile % tiles_x) * kTW;
  const int Ho = H - kHalo, Wo = W - kHalo;
  const int tid = threadIdx.x;
  const size_t ibytes = (size_t)H * W * 12;
  // y: this channel's plane of the target's planar copy, stored after the statistics
  const size_t npix = (size_t)H * W;
  const Rsrc xs = rsrc(x, ibytes), gs_out = rsrc(gout, ibytes);
  const Rsrc ys = rsrc(stats + 6 * (size_t)Ho * Wo + (size_t)ch * npix, npix * 4);
  const Rsrc ss = rsrc(stats, (size_t)Ho * Wo * 24);
  const unsigned plane4 = (unsigned)(Ho * Wo) * 4u;
  // phase-2 role: map row m2, columns [q2, q2 + 15); its target statistics loaded up front
  const int m2 = tid % G::MR, q2 = (tid / G::MR) * kHC;
  const bool act2 = tid < G::N2;
  const int gm2 = R0 - kHalo + m2;
  float smu[kHC], ssy[kHC];
  // one add per load: map pixels outside the valid map are never used (phase 2 masks them), so
  // their offsets need no clamping -- negative ones wrap past the resource's bound (reading 0),
  // the others stay inside the statistics buffer or past its bound
  auto load_stats = [&]() {
    const unsigned off0 =
        (unsigned)((C0 - kHalo + q2) * Ho + gm2) * 4u + (unsigned)ch * plane4;
    const unsigned cstep = (unsigned)Ho * 4u;
#pragma unroll
    for (int o = 0; o < kHC; ++o) {
      const unsigned off = off0 + (unsigned)o * cstep;
      smu[o] = bld(ss, off);
      ssy[o] = bld(ss, off + 3u * plane4);
    }
  };
  // ---- phase 1: vertical filter of x, x^2, xy; thread = (input column j, run of VR map rows)
  if (tid < 3 * kIC) {
    const int j = tid % kIC, m0 = (tid / kIC) * G::VR;
    const int gc = C0 - kHalo + j;
    // rows outside the image fall past the bound (negative or >= H rows); columns outside it
    // would alias a neighbouring row, so their lanes start at kOOB
    const unsigned base = (gc >= 0 && gc < W)
                              ? (unsigned)((((R0 - kHalo + m0) * W + gc) * 3 + ch) * 4)
                              : kOOB;
    const unsigned rstep = (unsigned)W * 12u;
    const unsigned ybase = (gc >= 0 && gc < W) ? (unsigned)(((R0 - kHalo + m0) * W + gc) * 4)
                                                : kOOB;
    float xv[G::VR + kHalo], yv[G::VR + kHalo];
#pragma unroll
    for (int k = 0; k < G::VR + kHalo; ++k) {
      xv[k] = bld(xs, base + (unsigned)k * rstep);
      yv[k] = bld(ys, ybase + (unsigned)k * (unsigned)W * 4u);
    }
    // the target statistics phase 2 needs, issued after the loads phase 1 waits on
    load_stats();
    float acc[3][G::VR];
#pragma unroll
    for (int o = 0; o < G::VR; ++o) acc[0][o] = acc[1][o] = acc[2][o] = 0.f;
#pragma unroll
    for (int k = 0; k < G::VR + kHalo; ++k) {
      const float a = clamp01(xv[k]), b = clamp01(yv[k]), aa = a * a, ab = a * b;
#pragma unroll
      for (int o = 0; o < G::VR; ++o) {
        const int tap = k - o;
        if (tap >= 0 && tap < kWin) {
          const float gk = vt.g[tap];
          acc[0][o] += gk * a;
          acc[1][o] += gk * aa;
          acc[2][o] += gk * ab;
        }
      }
    }
#pragma unroll
    for (int o = 0; o < G::VR; ++o) {
      const int m = m0 + o;
      if (m < G::MR) {
#pragma unroll
        for (int qn = 0; qn < 3; ++qn) V[(qn * G::MR + m) * kVS + j] = acc[qn][o];
      }
    }
  }
  else {
    load_stats();
  }
  __syncthreads();
  // ---- phase 2: horizontal filter + SSIM partials
  float ssum = 0.f, l1sum = 0.f;
  float dv[3][kHC];
  if (act2) {
#pragma unroll
    for (int o = 0; o < kHC; ++o) dv[0][o] = dv[1][o] = dv[2][o] = 0.f;
#pragma unroll
    for (int k = 0; k < kHC + kHalo; ++k) {
      const int c = q2 + k;   // <= 84 < kVS: the row padding, feeding only dropped columns
      float vv[3];
#pragma unroll
      for (int qn = 0; qn < 3; ++qn) vv[qn] = V[(qn * G::MR + m2) * kVS + c];
#pragma unroll
      for (int o = 0; o < kHC; ++o) {
        const int tap = k - o;
        if (tap >= 0 && tap < kWin) {
          const float gk = vt.g[tap];
#pragma unroll
          for (int qn = 0; qn < 3; ++qn) dv[qn][o] += gk * vv[qn];
        }
      }
    }
    const bool row_ok = gm2 >= 0 && gm2 < Ho;
#pragma unroll
    for (int o = 0; o < kHC; ++o) {
      const int gq = C0 - kHalo + q2 + o;
      float d0 = 0.f, d1 = 0.f, d2 = 0.f;
      if (row_ok && gq >= 0 && gq < Wo && q2 + o < kMC) {
        const float mx = dv[0][o], my = smu[o];
        const float A1 = 2.f * mx * my + kC1;
        const float A2 = 2.f * (dv[2][o] - mx * my) + kC2;
        const float B1 = mx * mx + my * my + kC1;
        const float B2 = (dv[1][o] - mx * mx) + ssy[o] + kC2;
        // hardware reciprocal (1 ulp): B1 >= C1 and B2 >= C2 - rounding, so B1*B2 is normal
        const float inv_d = __builtin_amdgcn_rcpf(B1 * B2);
        const float Sv = A1 * A2 * inv_d;
        d0 = 2.f * inv_d * (my * (A2 - A1) - Sv * mx * (B2 - B1));
        d1 = -Sv * B1 * inv_d;
        d2 = 2.f * A1 * inv_d;
        if (m2 >= kHalo && q2 + o >= kHalo) ssum += Sv;   // map pixels of this tile
      }
      dv[0][o] = d0;
      dv[1][o] = d1;
      dv[2][o] = d2;
    }
  }
  __syncthreads();   // every read of V done: D overwrites it
  if (act2) {
#pragma unroll
    for (int o = 0; o < kHC; ++o) {
      if (q2 + o < kMC) {
#pragma unroll
        for (int qn = 0; qn < 3; ++qn) D[(qn * G::MR + m2) * kDS + q2 + o] = dv[qn][o];
      }
    }
  }
  // phase-4 role: gradient column c4, rows [p4, p4 + TR4); its pixels loaded two phases ahead
  const int c4 = tid & 63, p4 = (tid >> 6) * G::TR4;
  const int gc4 = C0 + c4;
  const bool col4_ok = gc4 < W;
  const unsigned off4 = (unsigned)((((R0 + p4) * W + gc4) * 3 + ch) * 4);
  const unsigned rstep4 = (unsigned)W * 12u;
  float xr[G::TR4], yr[G::TR4];
#pragma unroll
  for (int o = 0; o < G::TR4; ++o) {
    xr[o] = bld(xs, col4_ok ? off4 + (unsigned)o * rstep4 : kOOB);
    yr[o] = bld(ys, col4_ok ? (unsigned)(((R0 + p4 + o) * W + gc4) * 4) : kOOB);
  }
  __syncthreads();
  // ---- phase 3: transposed horizontal, thread = (map row m3, run of kHC3 gradient columns):
  //      gradient column c receives map columns c..c+10 through tap 10 - (q - c)
  float ta[3][kHC3];
  const int m3 = tid % G::MR, c3 = (tid / G::MR) * kHC3;
  const bool act3 = tid < 5 * G::MR;
  if (act3) {
#pragma unroll
    for (int o = 0; o < kHC3; ++o) ta[0][o] = ta[1][o] = ta[2][o] = 0.f;
#pragma unroll
    for (int k = 0; k < kHC3 + kHalo; ++k) {
      const int q = c3 + k;   // <= 74 < kDS: the row padding, feeding only dropped columns
      float dd[3];
#pragma unroll
      for (int qn = 0; qn < 3; ++qn) dd[qn] = D[(qn * G::MR + m3) * kDS + q];
#pragma unroll
      for (int o = 0; o < kHC3; ++o) {
        const int tap = kHalo - (k - o);
        if (tap >= 0 && tap < kWin) {
          const float gk = vt.g[tap];
#pragma unroll
          for (int qn = 0; qn < 3; ++qn) ta[qn][o] += gk * dd[qn];
        }
      }
    }
  }
  __syncthreads();   // every read of D done: T overwrites it
  if (act3) {
#pragma unroll
    for (int o = 0; o < kHC3; ++o) {
      const int c = c3 + o;
      if (c < kTW) {
#pragma unroll
        for (int qn = 0; qn < 3; ++qn) T[(qn * G::TP + m3) * kTS + c] = ta[qn][o];
      }
    }
  }
  __syncthreads();
  // ---- phase 4: transposed vertical + gradient, thread = (gradient column c4, run of rows):
  //      gradient row p receives map rows p..p+10 through tap 10 - (m - p)
  {
    float t[3][G::TR4];
#pragma unroll
    for (int o = 0; o < G::TR4; ++o) t[0][o] = t[1][o] = t[2][o] = 0.f;
#pragma unroll
    for (int k = 0; k < G::TR4 + kHalo; ++k) {
      const int m = p4 + k;   // rows past MR feed only dropped rows; T has room for them
      float tt[3];
#pragma unroll
      for (int qn = 0; qn < 3; ++qn) tt[qn] = T[(qn * G::TP + m) * kTS + c4];
#pragma unroll
      for (int o = 0; o < G::TR4; ++o) {
        const int tap = kHalo - (k - o);
        if (tap >= 0 && tap < kWin) {
          const float gk = vt.g[tap];
#pragma unroll
          for (int qn = 0; qn < 3; ++qn) t[qn][o] += gk * tt[qn];
        }
      }
    }
#pragma unroll
    for (int o = 0; o < G::TR4; ++o) {
      const float xo = xr[o], yo = yr[o];
      const float d = xo - yo;
      const float sgn = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
      const bool pass = xo >= 0.f && xo <= 1.f;
      const float gs =
          pass ? (t[0][o] + 2.f * clamp01(xo) * t[1][o] + clamp01(yo) * t[2][o]) * inv_ns : 0.f;
      if (col4_ok && p4 + o < TH && R0 + p4 + o < H) {
        bst(gs_out, off4 + (unsigned)o * rstep4, (1.f - lambda) * sgn * inv_n - lambda * gs);
        l1sum += fabsf(d);
      }
    }
  }
  // both block sums through one barrier
  const float sw = wave_sum(ssum), lw = wave_sum(l1sum);
  if ((tid & 63) == 0) {
    s_fsum[tid >> 6] = sw;
    s_fsum[4 + (tid >> 6)] = lw;
  }
  __syncthreads();
  if (partials && tid == 0) {
    partials[blockIdx.x] = (s_fsum[0] + s_fsum[1]) + (s_fsum[2] + s_fsum[3]);
    partials[gridDim.x + blockIdx.x] = (s_fsum[4] + s_fsum[5]) + (s_fsum[6] + s_fsum[7]);
  }
}

// 40 rows: with 256 threads phase 4 takes exactly 4 runs of 10 rows, phases 2 and 3 use 250 of
// the threads (5 runs on each of the 50 map rows), and V's 51 KB still lets three blocks share
// a CU.  Measured at 1264x832: 34 rows 32.4 us, 38 rows 32.5, 40 rows 30.4, 41 rows 30.4 (42
// rows would need 260 threads in phases 2 and 3).
constexpr int kTH = 40;

inline int fused_tiles_x(int W) { return (W + kTW - 1) / kTW; }
inline int fused_items(int H, int W) { return 3 * fused_tiles_x(W) * ((H + kTH - 1) / kTH); }

inline Taps make_taps() {
  Taps taps;
  double gd[kWin], sum = 0.0;
  for (int i = 0; i < kWin; ++i) {
    const double c = (double)(i - kWin / 2);
    gd[i] = exp(-(c * c) / (2.0 * 1.5 * 1.5));
    sum += gd[i];
  }
  for (int i = 0; i < kWin; ++i) taps.g[i] = (float)(gd[i] / sum);
  return taps;
}

inline bool loss_size_ok(int H, int W) {
  // buffer offsets are 32-bit: the statistics planes (24 bytes per map pixel) and the images
  // (12 bytes per pixel) stay below 2^31 bytes, and an out-of-image offset past the image's bound
  return H >= kWin && W >= kWin && (int64_t)H * W * 24 <= (int64_t)INT32_MAX - 16;
}

}  // namespace tts

using namespace tts;

extern "C" {

size_t tts_loss_stats_bytes(int H, int W) {
  if (H < kWin || W < kWin) return 0;
  return sizeof(float) * (6 * (size_t)(H - kHalo) * (size_t)(W - kHalo) + 3 * (size_t)H * W);
}

size_t tts_loss_workspace_bytes(int H, int W) { return tts_loss_stats_bytes(H, W); }

int tts_loss_partials_count(int H, int W, int* n_ssim) {
  if (H < kWin || W < kWin) return 0;
  const int nb = fused_items(H, W);
  if (n_ssim) *n_ssim = nb;
  return 2 * nb;
}

int tts_loss_target_stats(const float* target, int H, int W, float* stats, hipStream_t stream) {
  if (!target || !stats) return TTS_EINVAL;
  if (!loss_size_ok(H, W)) return TTS_EINVAL;
  const int tx = (W - kHalo + kSW - 1) / kSW, ty = (H - kHalo + kSH - 1) / kSH;
  k_loss_target_stats<<<tx * ty * 3, 256, 0, stream>>>(target, H, W, tx, make_taps(), stats);
  const int64_t n = (int64_t)H * W;
  k_loss_target_planar<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
      target, n, stats + 6 * (size_t)(H - kHalo) * (size_t)(W - kHalo));
  return launch_status();
}

int tts_composite_random_bg(const float* rgba_pm, int H, int W, const int32_t* step, int view,
                            unsigned seed, float* bg4, float* target, hipStream_t stream) {
  if (!rgba_pm || !step || !bg4 || !target || H <= 0 || W <= 0 || view < 0) return TTS_EINVAL;
  if ((reinterpret_cast<uintptr_t>(rgba_pm) & 15) != 0) return TTS_EINVAL;  // float4 rows
  const int64_t n = (int64_t)H * W;
  k_composite_random_bg<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
      reinterpret_cast<const float4*>(rgba_pm), n, step, (uint32_t)view, (uint32_t)seed, bg4,
      target);
  return launch_status();
}

int tts_loss_grad_stats(const float* image, const float* target, const float* stats, int H,
                        int W, float lambda, float* gimage, float* partials,
                        hipStream_t stream) {
  if (!image || !target || !stats || !gimage) return TTS_EINVAL;
  if (!loss_size_ok(H, W)) return TTS_EINVAL;
  const int tx = fused_tiles_x(W), ni = fused_items(H, W);
  const float inv_n = 1.0f / (3.0f * (float)H * (float)W);
  const float inv_ns = 1.0f / (3.0f * (float)(H - kHalo) * (float)(W - kHalo));
  k_loss_fused<kTH><<<ni, 256, FGeo<kTH>::lds_bytes, stream>>>(
      image, target, stats, H, W, tx, ni, make_taps(), lambda, inv_n, inv_ns, gimage, partials);
  return launch_status();
}

int tts_loss_grad(const float* image, const float* target, int H, int W, float lambda,
                  float* gimage, float* partials, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
  if (!image || !target || !gimage) return TTS_EINVAL;
  if (!loss_size_ok(H, W)) return TTS_EINVAL;
  if (!workspace || workspace_bytes < tts_loss_workspace_bytes(H, W)) return TTS_EWORKSPACE;
  float* stats = static_cast<float*>(workspace);
  const int e = tts_loss_target_stats(target, H, W, stats, stream);
  if (e) return e;
  return tts_loss_grad_stats(image, target, stats, H, W, lambda, gimage, partials, stream);
}

}  // extern "C"
