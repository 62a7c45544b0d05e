// Photometric loss gradient: L = (1-l)*mean|x-y| + l*(1 - mean SSIM(clamp x, clamp y)).
// SSIM: 11-tap gaussian window (sigma 1.5), valid borders, C1 = 1e-4, C2 = 9e-4
// (spike/metrics.py:6-28; the manual gradient of tools/loss_manual.py:76-103).
//
// Two kernels, one colour channel per block, separable filters with register blocking (each
// value read from LDS once per pass instead of once per tap):
//   k_ssim_maps   per OUTPUT pixel of the valid SSIM map: the five filtered moments mu_x,
//                 E[x^2], E[xy], mu_y, E[y^2], S and its partials dS/dmu_x, dS/dE[x^2],
//                 dS/dE[xy] -> maps[3][3][Ho][Wo], the tile's sum of S.  The target's moments
//                 are filtered in the same passes rather than read from a precomputed buffer:
//                 in a training step the target arrives from HBM, and its two statistics planes
//                 per channel would cost twice its own bytes again.
//   k_ssim_grad   per INPUT pixel: the transposed filter (zero outside the valid map) of the
//                 three maps, combined as  dmeanS/dx = (F'(A) + 2 x F'(B) + y F'(Cxy)) / Ns,
//                 gated by 0 <= x <= 1 (the clamp), plus the L1 term (1-l) sign(x-y) / N.

#include "tts_common.h"

namespace tts {

constexpr int kWin = 11;
constexpr int kHalo = kWin - 1;
constexpr int kTW = 32;            // tile width (outputs of a pass)
constexpr int kTH = 16;            // tile height
constexpr int kRW = kTW + kHalo;   // 42: region width
constexpr int kRH = kTH + kHalo;   // 26: region height
constexpr int kVRows = 4;          // vertical pass: output rows per thread
constexpr int kHCols = 2;          // horizontal pass: outputs per thread
constexpr float kC1 = 1e-4f;
constexpr float kC2 = 9e-4f;

struct Taps {
  float g[kWin];
};

// Work item of a 1-D grid of gx * gy * 3 blocks: (tile column, tile row, channel), channels
// innermost and tiles row-major, renumbered so that each XCD sweeps one contiguous band of tiles.
struct TileItem {
  int tx, ty, ch;
};
__device__ __forceinline__ TileItem tile_item(int gx, int gy) {
  const int n = gx * gy * 3;
  const int w = xcd_item(blockIdx.x, n);
  const int t = w / 3;
  return {t % gx, t / gx, w - 3 * t};
}

__device__ __forceinline__ float clamp01(float v) { return fminf(fmaxf(v, 0.f), 1.f); }

// Buffer-resource addressing: a wave-uniform base (scalar offset: row, plane) plus a 32-bit
// per-lane byte offset (column), so no lane forms a 64-bit address.  Every buffer handed to
// these kernels is under 2^31 bytes (the entry point checks); a resource's size is its bound,
// and the indices are clamped inside it as well.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc(const float* p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float bld(Rsrc r, unsigned voff, unsigned soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void bst(Rsrc r, unsigned voff, unsigned soff, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff, soff, 0);
}
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Map kernel: per output pixel of the valid SSIM map, the moments mu_x, E[x^2], E[xy], mu_y,
// E[y^2] (five filtered images), S and its partials dS/dmu_x, dS/dE[x^2], dS/dE[xy] ->
// maps[3][3][Ho][Wo]; the tile's sum of S.
__global__ __launch_bounds__(256) void k_ssim_maps(const float* __restrict__ x,
                                                   const float* __restrict__ y, int H, int W,
                                                   Taps taps, float* __restrict__ maps,
                                                   float* __restrict__ partials) {
  const int Ho = H - kHalo, Wo = W - kHalo;
  const TileItem it = tile_item((Wo + kTW - 1) / kTW, (Ho + kTH - 1) / kTH);
  const int ox0 = it.tx * kTW, oy0 = it.ty * kTH, ch = it.ch;
  __shared__ float sx[kRH][kRW + 1], sy[kRH][kRW + 1];
  __shared__ float v[5][kTH][kRW + 1];
  __shared__ float s_ftmp[4];
  const int tid = threadIdx.x;
  const unsigned plane = (unsigned)(Ho * Wo);
  {  // region rows [oy0, oy0+26), cols [ox0, ox0+42): lane = column, wave w takes rows w, w+4, ...
    constexpr int NI = (kRH + 3) / 4;
    const Rsrc xs = rsrc(x, (size_t)H * W * 12), ys = rsrc(y, (size_t)H * W * 12);
    const int lane = tid & 63, wv = wave_id();
    const unsigned coff = ((unsigned)min(ox0 + lane, W - 1) * 3u + (unsigned)ch) * 4u;
    float a[NI], b[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int gr = min(oy0 + wv + 4 * i, H - 1);
      a[i] = bld(xs, coff, (unsigned)(gr * W) * 12u);
      b[i] = bld(ys, coff, (unsigned)(gr * W) * 12u);
    }
    const bool col_ok = lane < kRW && ox0 + lane < W;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r = wv + 4 * i;
      if (r < kRH && lane < kRW) {
        const bool in = col_ok && oy0 + r < H;
        sx[r][lane] = in ? clamp01(a[i]) : 0.f;
        sy[r][lane] = in ? clamp01(b[i]) : 0.f;
      }
    }
  }
  // this thread's output pixels in the horizontal pass
  const int r = tid / (kTW / kHCols), c0 = (tid % (kTW / kHCols)) * kHCols;
  const int orow = oy0 + r;
  __syncthreads();
  // vertical: thread = (column c, chunk of kVRows output rows)
  if (tid < kRW * (kTH / kVRows)) {
    const int c = tid % kRW, r0 = (tid / kRW) * kVRows;
    float acc[5][kVRows];
#pragma unroll
    for (int m = 0; m < 5; ++m)
#pragma unroll
      for (int o = 0; o < kVRows; ++o) acc[m][o] = 0.f;
#pragma unroll
    for (int k = 0; k < kVRows + kHalo; ++k) {
      const float xv = sx[r0 + k][c], yv = sy[r0 + k][c];
      const float xx = xv * xv, xy = xv * yv, yy = yv * yv;
#pragma unroll
      for (int o = 0; o < kVRows; ++o) {
        const int tap = k - o;
        if (tap >= 0 && tap < kWin) {
          const float gk = taps.g[tap];
          acc[0][o] += gk * xv;
          acc[1][o] += gk * xx;
          acc[2][o] += gk * xy;
          acc[3][o] += gk * yv;
          acc[4][o] += gk * yy;
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 5; ++m)
#pragma unroll
      for (int o = 0; o < kVRows; ++o) v[m][r0 + o][c] = acc[m][o];
  }
  __syncthreads();
  // horizontal: thread = (output row r, chunk of kHCols outputs)
  float f[5][kHCols];
#pragma unroll
  for (int m = 0; m < 5; ++m)
#pragma unroll
    for (int o = 0; o < kHCols; ++o) f[m][o] = 0.f;
#pragma unroll
  for (int k = 0; k < kHCols + kHalo; ++k) {
    float vv[5];
#pragma unroll
    for (int m = 0; m < 5; ++m) vv[m] = v[m][r][c0 + k];
#pragma unroll
    for (int o = 0; o < kHCols; ++o) {
      const int tap = k - o;
      if (tap >= 0 && tap < kWin) {
        const float gk = taps.g[tap];
#pragma unroll
        for (int m = 0; m < 5; ++m) f[m][o] += gk * vv[m];
      }
    }
  }
  float ssum = 0.0f;
#pragma unroll
  for (int o = 0; o < kHCols; ++o) {
    const int ocol = ox0 + c0 + o;
    if (orow < Ho && ocol < Wo) {
      const float mx = f[0][o], my = f[3][o];
      const float A1 = 2.f * mx * my + kC1;
      const float A2 = 2.f * (f[2][o] - mx * my) + kC2;
      const float B1 = mx * mx + my * my + kC1;
      const float B2 = (f[1][o] - mx * mx) + (f[4][o] - my * my) + kC2;
      // hardware reciprocal (1 ulp): B1 >= C1 and B2 >= C2 - rounding, so B1*B2 is normal
      const float inv_d = __builtin_amdgcn_rcpf(B1 * B2);
      const float Sv = A1 * A2 * inv_d;
      const unsigned oi = (unsigned)(orow * Wo + ocol) * 4u;
      const Rsrc mp = rsrc(maps, (size_t)plane * 36);
      bst(mp, oi, ch * plane * 4u, 2.f * inv_d * (my * (A2 - A1) - Sv * mx * (B2 - B1)));
      bst(mp, oi, (3 + ch) * plane * 4u, -Sv * B1 * inv_d);
      bst(mp, oi, (6 + ch) * plane * 4u, 2.f * A1 * inv_d);
      ssum += Sv;
    }
  }
  const float tot = block_sum256(ssum, s_ftmp);
  if (partials && tid == 0)
    partials[blockIdx.x] = tot;
}

__global__ __launch_bounds__(256) void k_ssim_grad(const float* __restrict__ x,
                                                   const float* __restrict__ y, int H, int W,
                                                   Taps taps, const float* __restrict__ maps,
                                                   float lambda, float inv_n, float inv_ns,
                                                   float* __restrict__ gout,
                                                   float* __restrict__ partials) {
  const int Ho = H - kHalo, Wo = W - kHalo;
  const TileItem it = tile_item((W + kTW - 1) / kTW, (H + kTH - 1) / kTH);
  const int ix0 = it.tx * kTW, iy0 = it.ty * kTH, ch = it.ch;
  __shared__ float sm[3][kRH][kRW + 1];
  __shared__ float v[3][kTH][kRW + 1];
  __shared__ float s_ftmp[4];
  const int tid = threadIdx.x;
  const unsigned plane = (unsigned)(Ho * Wo);
  const int lane = tid & 63, wv = wave_id();
  // map rows [iy0-10, iy0+16), cols [ix0-10, ix0+32); zero outside the valid map.
  // lane = column, wave w takes rows w, w+4, ...
  {
    constexpr int NI = (kRH + 3) / 4;
    const Rsrc ms = rsrc(maps, (size_t)plane * 36);
    const int mc = ix0 - kHalo + lane;
    const unsigned coff = (unsigned)min(max(mc, 0), Wo - 1) * 4u;
    float mv[3][NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {  // every load in flight before any is used
      const int mr = min(max(iy0 - kHalo + wv + 4 * i, 0), Ho - 1);
#pragma unroll
      for (int m = 0; m < 3; ++m)
        mv[m][i] = bld(ms, coff, ((unsigned)(m * 3 + ch) * plane + (unsigned)(mr * Wo)) * 4u);
    }
    const bool col_ok = lane < kRW && mc >= 0 && mc < Wo;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r = wv + 4 * i, mr = iy0 - kHalo + r;
      if (r < kRH && lane < kRW) {
        const bool ok = col_ok && mr >= 0 && mr < Ho;
#pragma unroll
        for (int m = 0; m < 3; ++m) sm[m][r][lane] = ok ? mv[m][i] : 0.f;
      }
    }
  }
  // this thread's pixels (loaded ahead of the filtering)
  const int r = tid / (kTW / kHCols), c0 = (tid % (kTW / kHCols)) * kHCols;
  const int gr = iy0 + r;
  const Rsrc xs = rsrc(x, (size_t)H * W * 12), ys = rsrc(y, (size_t)H * W * 12);
  const unsigned roff = (unsigned)(min(gr, H - 1) * W) * 12u;  // per lane: 4 rows per wave
  float xv[kHCols], yv[kHCols];
#pragma unroll
  for (int o = 0; o < kHCols; ++o) {
    const unsigned po = ((unsigned)min(ix0 + c0 + o, W - 1) * 3u + (unsigned)ch) * 4u;
    xv[o] = bld(xs, roff + po, 0);
    yv[o] = bld(ys, roff + po, 0);
  }
  __syncthreads();
  // transposed vertical: input row r receives sum_k g[k] * map[r + 10 - k]
  if (tid < kRW * (kTH / kVRows)) {
    const int c = tid % kRW, r0 = (tid / kRW) * kVRows;
    float acc[3][kVRows];
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int o = 0; o < kVRows; ++o) acc[m][o] = 0.f;
#pragma unroll
    for (int k = 0; k < kVRows + kHalo; ++k) {
      float mv[3];
#pragma unroll
      for (int m = 0; m < 3; ++m) mv[m] = sm[m][r0 + k][c];
#pragma unroll
      for (int o = 0; o < kVRows; ++o) {
        const int tap = kHalo - (k - o);  // map row r0+k feeds input row r0+o through tap 10-(k-o)
        if (tap >= 0 && tap < kWin) {
          const float gk = taps.g[tap];
#pragma unroll
          for (int m = 0; m < 3; ++m) acc[m][o] += gk * mv[m];
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int o = 0; o < kVRows; ++o) v[m][r0 + o][c] = acc[m][o];
  }
  __syncthreads();
  float t[3][kHCols];
#pragma unroll
  for (int m = 0; m < 3; ++m)
#pragma unroll
    for (int o = 0; o < kHCols; ++o) t[m][o] = 0.f;
#pragma unroll
  for (int k = 0; k < kHCols + kHalo; ++k) {
    float vv[3];
#pragma unroll
    for (int m = 0; m < 3; ++m) vv[m] = v[m][r][c0 + k];
#pragma unroll
    for (int o = 0; o < kHCols; ++o) {
      const int tap = kHalo - (k - o);
      if (tap >= 0 && tap < kWin) {
        const float gk = taps.g[tap];
#pragma unroll
        for (int m = 0; m < 3; ++m) t[m][o] += gk * vv[m];
      }
    }
  }
  const Rsrc gs_out = rsrc(gout, (size_t)H * W * 12);
  float l1sum = 0.0f;
#pragma unroll
  for (int o = 0; o < kHCols; ++o) {
    const int gc = ix0 + c0 + o;
    if (gr < H && gc < W) {
      const float xr = xv[o], yr = yv[o];
      const float d = xr - yr;
      const float sgn = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
      const bool pass = xr >= 0.f && xr <= 1.f;
      const float gs = pass ? (t[0][o] + 2.f * clamp01(xr) * t[1][o] + clamp01(yr) * t[2][o]) * inv_ns
                            : 0.f;
      bst(gs_out, roff + ((unsigned)gc * 3u + (unsigned)ch) * 4u, 0,
          (1.f - lambda) * sgn * inv_n - lambda * gs);
      l1sum += fabsf(d);
    }
  }
  const float tot = block_sum256(l1sum, s_ftmp);
  if (partials && tid == 0)
    partials[blockIdx.x] = tot;
}

// 1-D grids (see tile_item): one block per (tile, channel)
inline int maps_grid(int H, int W) {
  const int Ho = H - kHalo, Wo = W - kHalo;
  return ((Wo + kTW - 1) / kTW) * ((Ho + kTH - 1) / kTH) * 3;
}
inline int grad_grid(int H, int W) {
  return ((W + kTW - 1) / kTW) * ((H + kTH - 1) / kTH) * 3;
}

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

}  // namespace tts

using namespace tts;

extern "C" {

size_t tts_loss_workspace_bytes(int H, int W) {
  // the SSIM partial maps: [3][3] planes of (H-10) x (W-10)
  if (H < kWin || W < kWin) return 0;
  return sizeof(float) * 9 * (size_t)(H - kHalo) * (size_t)(W - kHalo);
}

int tts_loss_partials_count(int H, int W, int* n_ssim) {
  if (H < kWin || W < kWin) return 0;
  const int gm = maps_grid(H, W), gg = grad_grid(H, W);
  if (n_ssim) *n_ssim = gm;
  return gm + gg;
}

int tts_loss_grad(const float* image, const float* target, int H, int W, float lambda,
                  float* gimage, float* partials, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
  if (!image || !target || !gimage) return TTS_EINVAL;
  if (H < kWin || W < kWin) return TTS_EINVAL;
  // buffer resources take 32-bit sizes: the 9 map planes (the largest buffer) stay below 2^31 B
  if ((int64_t)H * W * 36 > INT32_MAX) return TTS_EINVAL;
  if (!workspace || workspace_bytes < tts_loss_workspace_bytes(H, W)) return TTS_EWORKSPACE;
  const Taps taps = make_taps();
  const int gm = maps_grid(H, W), gg = grad_grid(H, W);
  const float inv_n = 1.0f / (3.0f * (float)H * (float)W);
  const float inv_ns = 1.0f / (3.0f * (float)(H - kHalo) * (float)(W - kHalo));
  float* maps = static_cast<float*>(workspace);
  k_ssim_maps<<<gm, 256, 0, stream>>>(image, target, H, W, taps, maps, partials);
  k_ssim_grad<<<gg, 256, 0, stream>>>(image, target, H, W, taps, maps, lambda, inv_n, inv_ns,
                                      gimage, partials ? partials + gm : nullptr);
  return launch_status();
}

}  // extern "C"
