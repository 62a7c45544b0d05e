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
  const int64_t plane = (int64_t)Ho * Wo;
  {
    constexpr int kPer = (kRH * kRW + 255) / 256;
    float a[kPer], b[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {  // every load in flight before any is used
      const int i = min(tid + 256 * k, kRH * kRW - 1);
      const int gr = min(oy0 + i / kRW, H - 1), gc = min(ox0 + i % kRW, W - 1);
      const int64_t pi = ((int64_t)gr * W + gc) * 3 + ch;
      a[k] = x[pi];
      b[k] = y[pi];
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = tid + 256 * k;
      if (i < kRH * kRW) {
        const int r = i / kRW, c = i % kRW;
        const bool in = oy0 + r < H && ox0 + c < W;
        sx[r][c] = in ? clamp01(a[k]) : 0.f;
        sy[r][c] = in ? clamp01(b[k]) : 0.f;
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
      const float inv_d = 1.0f / (B1 * B2);  // one division; 1/B2 = B1/(B1 B2)
      const float Sv = A1 * A2 * inv_d;
      const int64_t oi = (int64_t)orow * Wo + ocol;
      maps[(0 * 3 + ch) * plane + oi] = 2.f * inv_d * (my * (A2 - A1) - Sv * mx * (B2 - B1));
      maps[(1 * 3 + ch) * plane + oi] = -Sv * B1 * inv_d;
      maps[(2 * 3 + ch) * plane + oi] = 2.f * A1 * inv_d;
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
                                                   float lambda, float* __restrict__ gout,
                                                   float* __restrict__ partials) {
  const int Ho = H - kHalo, Wo = W - kHalo;
  const TileItem it = tile_item((W + kTW - 1) / kTW, (H + kTH - 1) / kTH);
  const int ix0 = it.tx * kTW, iy0 = it.ty * kTH, ch = it.ch;
  __shared__ float sm[3][kRH][kRW + 1];
  __shared__ float v[3][kTH][kRW + 1];
  __shared__ float s_ftmp[4];
  const int tid = threadIdx.x;
  const int64_t plane = (int64_t)Ho * Wo;
  // map rows [iy0-10, iy0+16), cols [ix0-10, ix0+32); zero outside the valid map
  {
    constexpr int kPer = (kRH * kRW + 255) / 256;
    float mv[3][kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {  // every load in flight before any is used
      const int i = min(tid + 256 * k, kRH * kRW - 1);
      const int mr = min(max(iy0 - kHalo + i / kRW, 0), Ho - 1);
      const int mc = min(max(ix0 - kHalo + i % kRW, 0), Wo - 1);
      const int64_t o = (int64_t)mr * Wo + mc;
#pragma unroll
      for (int m = 0; m < 3; ++m) mv[m][k] = maps[(m * 3 + ch) * plane + o];
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = tid + 256 * k;
      if (i < kRH * kRW) {
        const int r = i / kRW, c = i % kRW;
        const int mr = iy0 - kHalo + r, mc = ix0 - kHalo + c;
        const bool ok = mr >= 0 && mr < Ho && mc >= 0 && mc < Wo;
#pragma unroll
        for (int m = 0; m < 3; ++m) sm[m][r][c] = ok ? mv[m][k] : 0.f;
      }
    }
  }
  // this thread's pixels (loaded ahead of the filtering)
  const int r = tid / (kTW / kHCols), c0 = (tid % (kTW / kHCols)) * kHCols;
  const int gr = iy0 + r;
  float xv[kHCols], yv[kHCols];
#pragma unroll
  for (int o = 0; o < kHCols; ++o) {
    const int64_t pi = ((int64_t)min(gr, H - 1) * W + min(ix0 + c0 + o, W - 1)) * 3 + ch;
    xv[o] = x[pi];
    yv[o] = y[pi];
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
  const float inv_n = 1.0f / (3.0f * (float)H * (float)W);
  const float inv_ns = 1.0f / (3.0f * (float)Ho * (float)Wo);
  float l1sum = 0.0f;
#pragma unroll
  for (int o = 0; o < kHCols; ++o) {
    const int gc = ix0 + c0 + o;
    if (gr < H && gc < W) {
      const int64_t pi = ((int64_t)gr * W + gc) * 3 + ch;
      const float xr = xv[o], yr = yv[o];
      const float d = xr - yr;
      const float sgn = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
      const bool pass = xr >= 0.f && xr <= 1.f;
      const float gs = pass ? (t[0][o] + 2.f * clamp01(xr) * t[1][o] + clamp01(yr) * t[2][o]) * inv_ns
                            : 0.f;
      gout[pi] = (1.f - lambda) * sgn * inv_n - lambda * gs;
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
  if (!workspace || workspace_bytes < tts_loss_workspace_bytes(H, W)) return TTS_EWORKSPACE;
  const Taps taps = make_taps();
  const int gm = maps_grid(H, W), gg = grad_grid(H, W);
  float* maps = static_cast<float*>(workspace);
  k_ssim_maps<<<gm, 256, 0, stream>>>(image, target, H, W, taps, maps, partials);
  k_ssim_grad<<<gg, 256, 0, stream>>>(image, target, H, W, taps, maps, lambda, gimage,
                                      partials ? partials + gm : nullptr);
  return launch_status();
}

}  // extern "C"
