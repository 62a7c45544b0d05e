// Photometric loss gradient: L = (1-l)*mean|x-y| + l*(1 - mean SSIM(clamp x, clamp y)).
// SSIM: 11-tap gaussian window (sigma 1.5), valid borders, C1 = 1e-4, C2 = 9e-4
// (spike/metrics.py:6-28; the manual gradient of tools/loss_manual.py:76-103).
//
// Two kernels over 16x16 tiles, separable filters staged through LDS:
//   k_ssim_maps   per OUTPUT pixel of the valid map: mu_x, mu_y, s_x, s_y, s_xy from five
//                 filtered images, then dS/dfx, dS/dfxx, dS/dfxy -> workspace maps [3][3][Ho][Wo],
//                 and the tile's sum of S.
//   k_ssim_grad   per INPUT pixel: the transposed filter (zero outside the valid map) of the
//                 three maps, combined as  dmeanS/dx = (F'(A) + 2 x F'(B) + y F'(Cxy)) / Ns
//                 (gated by 0 <= x <= 1, the clamp), plus the L1 term (1-l) sign(x-y) / N.

#include "tts_common.h"

namespace tts {

constexpr int kWin = 11;
constexpr int kHalo = kWin - 1;
constexpr int kTile = 16;
constexpr int kReg = kTile + kHalo;  // 26
constexpr float kC1 = 1e-4f;
constexpr float kC2 = 9e-4f;

struct Taps {
  float g[kWin];
};

__global__ __launch_bounds__(256) void k_ssim_maps(const float* __restrict__ x,
                                                   const float* __restrict__ y, int H, int W,
                                                   Taps taps, float* __restrict__ maps,
                                                   float* __restrict__ partials) {
  const int Ho = H - kHalo, Wo = W - kHalo;
  const int ox0 = blockIdx.x * kTile, oy0 = blockIdx.y * kTile;
  __shared__ float sx[kReg][kReg + 1], sy[kReg][kReg + 1];
  __shared__ float v[5][kTile][kReg + 1];
  __shared__ float s_ftmp[4];
  const int tid = threadIdx.x;
  const int lr = tid / kTile, lc = tid % kTile;
  const int64_t plane = (int64_t)Ho * Wo;
  float ssum = 0.0f;
  for (int ch = 0; ch < 3; ++ch) {
    for (int i = tid; i < kReg * kReg; i += 256) {
      const int r = i / kReg, c = i % kReg;
      const int gr = oy0 + r, gc = ox0 + c;
      float a = 0.f, b = 0.f;
      if (gr < H && gc < W) {
        a = fminf(fmaxf(x[((int64_t)gr * W + gc) * 3 + ch], 0.f), 1.f);
        b = fminf(fmaxf(y[((int64_t)gr * W + gc) * 3 + ch], 0.f), 1.f);
      }
      sx[r][c] = a;
      sy[r][c] = b;
    }
    __syncthreads();
    // vertical pass: rows of the output tile, all 26 columns
    for (int i = tid; i < kTile * kReg; i += 256) {
      const int r = i / kReg, c = i % kReg;
      float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, a4 = 0.f;
#pragma unroll
      for (int k = 0; k < kWin; ++k) {
        const float xv = sx[r + k][c], yv = sy[r + k][c], gk = taps.g[k];
        a0 += gk * xv;
        a1 += gk * yv;
        a2 += gk * xv * xv;
        a3 += gk * yv * yv;
        a4 += gk * xv * yv;
      }
      v[0][r][c] = a0; v[1][r][c] = a1; v[2][r][c] = a2; v[3][r][c] = a3; v[4][r][c] = a4;
    }
    __syncthreads();
    float mx = 0.f, my = 0.f, fxx = 0.f, fyy = 0.f, fxy = 0.f;
#pragma unroll
    for (int k = 0; k < kWin; ++k) {
      const float gk = taps.g[k];
      mx += gk * v[0][lr][lc + k];
      my += gk * v[1][lr][lc + k];
      fxx += gk * v[2][lr][lc + k];
      fyy += gk * v[3][lr][lc + k];
      fxy += gk * v[4][lr][lc + k];
    }
    const int orow = oy0 + lr, ocol = ox0 + lc;
    if (orow < Ho && ocol < Wo) {
      const float A1 = 2.f * mx * my + kC1;
      const float A2 = 2.f * (fxy - mx * my) + kC2;
      const float B1 = mx * mx + my * my + kC1;
      const float B2 = (fxx - mx * mx) + (fyy - my * my) + kC2;
      const float D = B1 * B2;
      const float Sv = (A1 * A2) / D;
      const float dfx = (2.f / D) * (my * (A2 - A1) - Sv * mx * (B2 - B1));
      const float dfxx = -Sv / B2;
      const float dfxy = 2.f * A1 / D;
      const int64_t o = (int64_t)orow * Wo + ocol;
      maps[(0 * 3 + ch) * plane + o] = dfx;
      maps[(1 * 3 + ch) * plane + o] = dfxx;
      maps[(2 * 3 + ch) * plane + o] = dfxy;
      ssum += Sv;
    }
    __syncthreads();
  }
  const float tot = block_sum256(ssum, s_ftmp);
  if (partials && tid == 0) partials[blockIdx.y * gridDim.x + blockIdx.x] = tot;
}

__global__ __launch_bounds__(256) void k_ssim_grad(const float* __restrict__ x,
                                                   const float* __restrict__ y, int H, int W,
                                                   Taps taps, const float* __restrict__ maps,
                                                   float lambda, float* __restrict__ gout,
                                                   float* __restrict__ partials) {
  const int Ho = H - kHalo, Wo = W - kHalo;
  const int ix0 = blockIdx.x * kTile, iy0 = blockIdx.y * kTile;
  __shared__ float sm[3][kReg][kReg + 1];
  __shared__ float v[3][kTile][kReg + 1];
  __shared__ float s_ftmp[4];
  const int tid = threadIdx.x;
  const int lr = tid / kTile, lc = tid % kTile;
  const int gr = iy0 + lr, gc = ix0 + lc;
  const bool inside = gr < H && gc < W;
  const int64_t plane = (int64_t)Ho * Wo;
  const float inv_n = 1.0f / (3.0f * (float)H * (float)W);
  const float inv_ns = 1.0f / (3.0f * (float)Ho * (float)Wo);
  float gres[3] = {0.f, 0.f, 0.f};
  float l1sum = 0.0f;
  for (int ch = 0; ch < 3; ++ch) {
    // map rows [iy0-10, iy0+16), cols [ix0-10, ix0+16); zero outside the valid map
    for (int i = tid; i < kReg * kReg; i += 256) {
      const int r = i / kReg, c = i % kReg;
      const int mr = iy0 - kHalo + r, mc = ix0 - kHalo + c;
      const bool ok = mr >= 0 && mr < Ho && mc >= 0 && mc < Wo;
      const int64_t o = (int64_t)mr * Wo + mc;
#pragma unroll
      for (int m = 0; m < 3; ++m) sm[m][r][c] = ok ? maps[(m * 3 + ch) * plane + o] : 0.f;
    }
    __syncthreads();
    // transposed vertical pass: input row r receives sum_k g[k] * map[r - k]
    for (int i = tid; i < kTile * kReg; i += 256) {
      const int r = i / kReg, c = i % kReg;
      float a0 = 0.f, a1 = 0.f, a2 = 0.f;
#pragma unroll
      for (int k = 0; k < kWin; ++k) {
        const float gk = taps.g[k];
        a0 += gk * sm[0][r + kHalo - k][c];
        a1 += gk * sm[1][r + kHalo - k][c];
        a2 += gk * sm[2][r + kHalo - k][c];
      }
      v[0][r][c] = a0; v[1][r][c] = a1; v[2][r][c] = a2;
    }
    __syncthreads();
    float t1 = 0.f, t2 = 0.f, t3 = 0.f;
#pragma unroll
    for (int k = 0; k < kWin; ++k) {
      const float gk = taps.g[k];
      t1 += gk * v[0][lr][lc + kHalo - k];
      t2 += gk * v[1][lr][lc + kHalo - k];
      t3 += gk * v[2][lr][lc + kHalo - k];
    }
    if (inside) {
      const int64_t pi = ((int64_t)gr * W + gc) * 3 + ch;
      const float xr = x[pi], yr = y[pi];
      const float xc = fminf(fmaxf(xr, 0.f), 1.f), yc = fminf(fmaxf(yr, 0.f), 1.f);
      const float d = xr - yr;
      const float sgn = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
      const bool pass = xr >= 0.f && xr <= 1.f;
      const float gs = pass ? (t1 + 2.f * xc * t2 + yc * t3) * inv_ns : 0.f;
      gres[ch] = (1.f - lambda) * sgn * inv_n - lambda * gs;
      l1sum += fabsf(d);
    }
    __syncthreads();
  }
  if (inside) {
    const int64_t pi = ((int64_t)gr * W + gc) * 3;
    gout[pi + 0] = gres[0];
    gout[pi + 1] = gres[1];
    gout[pi + 2] = gres[2];
  }
  const float tot = block_sum256(l1sum, s_ftmp);
  if (partials && tid == 0) partials[blockIdx.y * gridDim.x + blockIdx.x] = tot;
}

inline void loss_grids(int H, int W, dim3* gm, dim3* gg) {
  const int Ho = H - kHalo, Wo = W - kHalo;
  *gm = dim3((Wo + kTile - 1) / kTile, (Ho + kTile - 1) / kTile);
  *gg = dim3((W + kTile - 1) / kTile, (H + kTile - 1) / kTile);
}

}  // namespace tts

using namespace tts;

extern "C" {

size_t tts_loss_workspace_bytes(int H, int W) {
  if (H < kWin || W < kWin) return 0;
  return sizeof(float) * 9 * (size_t)(H - kHalo) * (size_t)(W - kHalo);
}

int tts_loss_partials_count(int H, int W, int* n_ssim) {
  if (H < kWin || W < kWin) return 0;
  dim3 gm, gg;
  loss_grids(H, W, &gm, &gg);
  if (n_ssim) *n_ssim = (int)(gm.x * gm.y);
  return (int)(gm.x * gm.y + gg.x * gg.y);
}

int tts_loss_grad(const float* image, const float* target, int H, int W, float lambda,
                  float* gimage, float* partials, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
  if (!image || !target || !gimage) return TTS_EINVAL;
  if (H < kWin || W < kWin) return TTS_EINVAL;
  if (!workspace || workspace_bytes < tts_loss_workspace_bytes(H, W)) return TTS_EWORKSPACE;
  Taps taps;
  double gd[kWin], sum = 0.0;
  for (int i = 0; i < kWin; ++i) {
    const double c = (double)(i - kWin / 2);
    gd[i] = exp(-(c * c) / (2.0 * 1.5 * 1.5));
    sum += gd[i];
  }
  for (int i = 0; i < kWin; ++i) taps.g[i] = (float)(gd[i] / sum);
  dim3 gm, gg;
  loss_grids(H, W, &gm, &gg);
  float* maps = static_cast<float*>(workspace);
  k_ssim_maps<<<gm, 256, 0, stream>>>(image, target, H, W, taps, maps, partials);
  k_ssim_grad<<<gg, 256, 0, stream>>>(image, target, H, W, taps, maps, lambda, gimage,
                                      partials ? partials + gm.x * gm.y : nullptr);
  return launch_status();
}

}  // extern "C"
