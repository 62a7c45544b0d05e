// Dense (unbinned) poly-splat + WSR: every gaussian against every pixel, O(P*G).
//
// Two forms of the reference's dense entry points:
//   quad  : spike/render.py:14-49 arm "A" -- Q = a dx^2 + 2b dx dy + c dy^2 with dx = px - mu_x
//           (spike/forward.py:13-21), w = o*keep*max(0, 1 - Q/k)^2, WSR blend
//           (spike/arms.py:22-31).  Operands are the projected records proj[G,12]; the backward
//           yields the per-gaussian (a, b, c, mu_x, mu_y, col_o rgb, o_col) gradients that the
//           geometry backward consumes.
//   theta : spike/backward.py:11-63 (wsr_polysplat) -- u = Phi[p] . theta_u[g] for an arbitrary
//           basis Phi[P,6], w = o*keep*max(u,0)^2; backward gives g_theta[G,6], g_o[G],
//           g_color[G,3], g_w_b.
//
// Forward: one thread per pixel, gaussians staged through LDS 256 at a time.
// Backward: one thread per gaussian; the pixels are cut into bands, each (gaussian chunk, band)
// block stages its band's per-pixel WSR gradients (gnum = gC/den, gden = -(gC.C)/den) in LDS and
// accumulates the gaussian's sums over the band.  Band partials go to a workspace and are summed
// in band order by a second kernel, so the result is deterministic and there are no atomics.

#include "tts_common.h"

namespace tts {

constexpr int kDenseChunk = 256;
constexpr int kQuadComp = 9;    // a, b, c, mu_x, mu_y, col_o r, g, b, o_col
constexpr int kThetaComp = 10;  // theta 0..5, o, color r, g, b
constexpr int kDenseTargetBlocks = 2048;
constexpr size_t kDenseMaxWorkspace = size_t(1) << 30;

// Pixels per band (a multiple of 256) for G gaussians over P pixels.
inline int dense_band_pixels(int G, int P) {
  const int gchunks = (G + kDenseChunk - 1) / kDenseChunk;
  int nb = kDenseTargetBlocks / (gchunks > 0 ? gchunks : 1);
  if (nb < 1) nb = 1;
  int pb = (P + nb - 1) / nb;
  pb = ((pb + 255) / 256) * 256;
  if (pb < 256) pb = 256;
  // keep the partials within the workspace cap
  while ((size_t)((P + pb - 1) / pb) * (size_t)G * kThetaComp * 4 > kDenseMaxWorkspace) pb *= 2;
  return pb;
}

// Workspace layout: [align to 256][gwb partials, nb floats, padded to 256][partials nb*G*ncomp].
inline size_t dense_ws_bytes(int G, int P, int ncomp) {
  if (G <= 0 || P <= 0) return 0;
  const int pb = dense_band_pixels(G, P);
  const size_t nb = (size_t)((P + pb - 1) / pb);
  return 256 + ((nb * 4 + 255) & ~size_t(255)) + nb * (size_t)G * ncomp * 4;
}

// ---------------------------------------------------------------- forward

__global__ __launch_bounds__(256) void k_render_dense(const float* __restrict__ proj, int G,
                                                      int W, int P, float inv_k,
                                                      const float* __restrict__ bg,
                                                      float* __restrict__ image,
                                                      float* __restrict__ den_out) {
  __shared__ float4 s_a[kDenseChunk];  // mu_x, mu_y, a, 2b
  __shared__ float4 s_b[kDenseChunk];  // c, col_o r, g, b
  __shared__ float s_o[kDenseChunk];   // o_col
  const int p = blockIdx.x * 256 + threadIdx.x;
  const float px = (float)(p % W) + 0.5f, py = (float)(p / W) + 0.5f;
  float nr = 0.f, ng = 0.f, nb = 0.f, nd = 0.f;
  for (int g0 = 0; g0 < G; g0 += kDenseChunk) {
    const int n = min(kDenseChunk, G - g0);
    __syncthreads();
    if ((int)threadIdx.x < n) {
      const float4* r = reinterpret_cast<const float4*>(proj + (int64_t)(g0 + threadIdx.x) * 12);
      const float4 r0 = r[0], r1 = r[1], r2 = r[2];
      s_a[threadIdx.x] = make_float4(r0.x, r0.y, r0.z, 2.0f * r0.w);
      s_b[threadIdx.x] = make_float4(r1.x, r1.z, r1.w, r2.x);
      s_o[threadIdx.x] = r2.y;
    }
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      const float4 A = s_a[j], B = s_b[j];
      const float dx = px - A.x, dy = py - A.y;
      const float Q = (A.z * dx + A.w * dy) * dx + (B.x * dy) * dy;
      const float r = fmaxf(1.0f - Q * inv_k, 0.0f);
      const float w = r * r;
      nr += w * B.y;
      ng += w * B.z;
      nb += w * B.w;
      nd += w * s_o[j];
    }
  }
  if (p < P) {
    const float wb = bg[0];
    const float d = nd + wb;
    image[(int64_t)p * 3 + 0] = (nr + wb * bg[1]) / d;
    image[(int64_t)p * 3 + 1] = (ng + wb * bg[2]) / d;
    image[(int64_t)p * 3 + 2] = (nb + wb * bg[3]) / d;
    if (den_out) den_out[p] = d;
  }
}

__global__ __launch_bounds__(256) void k_wsr_dense(const float* __restrict__ theta,
                                                   const float* __restrict__ o,
                                                   const float* __restrict__ color,
                                                   const uint8_t* __restrict__ keep,
                                                   const float* __restrict__ phi, int G, int P,
                                                   const float* __restrict__ bg,
                                                   float* __restrict__ C,
                                                   float* __restrict__ den_out) {
  __shared__ float4 s_a[kDenseChunk];  // theta 0..3
  __shared__ float4 s_b[kDenseChunk];  // theta 4, 5, -, -
  __shared__ float4 s_c[kDenseChunk];  // o*keep*color, o*keep
  const int p = blockIdx.x * 256 + threadIdx.x;
  float f[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (p < P) {
#pragma unroll
    for (int i = 0; i < 6; ++i) f[i] = phi[(int64_t)p * 6 + i];
  }
  float nr = 0.f, ng = 0.f, nb = 0.f, nd = 0.f;
  for (int g0 = 0; g0 < G; g0 += kDenseChunk) {
    const int n = min(kDenseChunk, G - g0);
    __syncthreads();
    if ((int)threadIdx.x < n) {
      const int g = g0 + threadIdx.x;
      const float* th = theta + (int64_t)g * 6;
      const float ok = (keep && !keep[g]) ? 0.0f : o[g];
      s_a[threadIdx.x] = make_float4(th[0], th[1], th[2], th[3]);
      s_b[threadIdx.x] = make_float4(th[4], th[5], 0.f, 0.f);
      s_c[threadIdx.x] = make_float4(ok * color[(int64_t)g * 3 + 0], ok * color[(int64_t)g * 3 + 1],
                                     ok * color[(int64_t)g * 3 + 2], ok);
    }
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      const float4 A = s_a[j], B = s_b[j], Cc = s_c[j];
      const float u = f[0] * A.x + f[1] * A.y + f[2] * A.z + f[3] * A.w + f[4] * B.x + f[5] * B.y;
      const float r = fmaxf(u, 0.0f);
      const float w = r * r;
      nr += w * Cc.x;
      ng += w * Cc.y;
      nb += w * Cc.z;
      nd += w * Cc.w;
    }
  }
  if (p < P) {
    const float wb = bg[0];
    const float d = nd + wb;
    C[(int64_t)p * 3 + 0] = (nr + wb * bg[1]) / d;
    C[(int64_t)p * 3 + 1] = (ng + wb * bg[2]) / d;
    C[(int64_t)p * 3 + 2] = (nb + wb * bg[3]) / d;
    if (den_out) den_out[p] = d;
  }
}

// ---------------------------------------------------------------- backward

// Stage pixels [p0, p0+256) of a band: (gnum r,g,b, gden); returns this thread's share of
// dL/dw_b = sum(gnum . c_b) + sum(gden).
__device__ __forceinline__ float stage_pixel_grads(const float* __restrict__ image,
                                                   const float* __restrict__ den,
                                                   const float* __restrict__ gimage, int p,
                                                   bool in, const float* __restrict__ bg,
                                                   float4* s_px) {
  float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
  if (in) {
    const float inv = 1.0f / den[p];
    const float g0 = gimage[(int64_t)p * 3 + 0], g1 = gimage[(int64_t)p * 3 + 1],
                g2 = gimage[(int64_t)p * 3 + 2];
    const float c0 = image[(int64_t)p * 3 + 0], c1 = image[(int64_t)p * 3 + 1],
                c2 = image[(int64_t)p * 3 + 2];
    q = make_float4(g0 * inv, g1 * inv, g2 * inv, -(g0 * c0 + g1 * c1 + g2 * c2) * inv);
  }
  s_px[threadIdx.x] = q;
  return q.x * bg[1] + q.y * bg[2] + q.z * bg[3] + q.w;
}

__global__ __launch_bounds__(256) void k_render_dense_bwd(
    const float* __restrict__ proj, int G, int W, int P, int PB, float inv_k,
    const float* __restrict__ bg, const float* __restrict__ image, const float* __restrict__ den,
    const float* __restrict__ gimage, float* __restrict__ part, float* __restrict__ gwb_part) {
  __shared__ float4 s_px[256];
  __shared__ float2 s_xy[256];
  __shared__ float s_ftmp[4];
  const int band = blockIdx.y;
  const int g = blockIdx.x * 256 + threadIdx.x;
  const bool act = g < G;
  float mx = 0.f, my = 0.f, a = 0.f, b = 0.f, c = 0.f, cr = 0.f, cg = 0.f, cb = 0.f, oc = 0.f;
  if (act) {
    const float4* r = reinterpret_cast<const float4*>(proj + (int64_t)g * 12);
    const float4 r0 = r[0], r1 = r[1], r2 = r[2];
    mx = r0.x; my = r0.y; a = r0.z; b = r0.w; c = r1.x;
    cr = r1.z; cg = r1.w; cb = r2.x; oc = r2.y;
  }
  const float b2 = 2.0f * b;
  float sxx = 0.f, sxy = 0.f, syy = 0.f, sx = 0.f, sy = 0.f;
  float gr = 0.f, gg = 0.f, gbl = 0.f, go = 0.f;
  float wpart = 0.f;
  const int pend = min(P, (band + 1) * PB);
  for (int p0 = band * PB; p0 < pend; p0 += 256) {
    __syncthreads();
    const int pp = p0 + threadIdx.x;
    wpart += stage_pixel_grads(image, den, gimage, pp, pp < pend, bg, s_px);
    s_xy[threadIdx.x] = make_float2((float)(pp % W) + 0.5f, (float)(pp / W) + 0.5f);
    __syncthreads();
    const int n = min(256, pend - p0);
    for (int j = 0; j < n; ++j) {
      const float4 q = s_px[j];
      const float2 xy = s_xy[j];
      const float dx = xy.x - mx, dy = xy.y - my;
      const float Q = (a * dx + b2 * dy) * dx + (c * dy) * dy;
      const float r = fmaxf(1.0f - Q * inv_k, 0.0f);
      const float w = r * r;
      gr += w * q.x;
      gg += w * q.y;
      gbl += w * q.z;
      go += w * q.w;
      const float gu = r * (q.x * cr + q.y * cg + q.z * cb + q.w * oc);  // half of dL/du
      const float tx = gu * dx, ty = gu * dy;
      sxx += tx * dx;
      sxy += tx * dy;
      syy += ty * dy;
      sx += tx;
      sy += ty;
    }
  }
  if (blockIdx.x == 0) {
    const float tot = block_sum256(wpart, s_ftmp);
    if (threadIdx.x == 0) gwb_part[band] = tot;
  }
  if (act) {
    // dL/dQ = dL/du * (-1/k) = -2 gu / k
    const float s = -2.0f * inv_k;
    const float mxx = s * sxx, mxy = s * sxy, myy = s * syy, m_x = s * sx, m_y = s * sy;
    float* dst = part + ((int64_t)band * G + g) * kQuadComp;
    dst[0] = mxx;                          // dQ/da = dx^2
    dst[1] = 2.0f * mxy;                   // dQ/db = 2 dx dy
    dst[2] = myy;                          // dQ/dc = dy^2
    dst[3] = -2.0f * (a * m_x + b * m_y);  // dQ/dmu_x = -2 (a dx + b dy)
    dst[4] = -2.0f * (b * m_x + c * m_y);  // dQ/dmu_y = -2 (b dx + c dy)
    dst[5] = gr;
    dst[6] = gg;
    dst[7] = gbl;
    dst[8] = go;
  }
}

__global__ __launch_bounds__(256) void k_wsr_dense_bwd(
    const float* __restrict__ theta, const float* __restrict__ o, const float* __restrict__ color,
    const uint8_t* __restrict__ keep, const float* __restrict__ phi, int G, int P, int PB,
    const float* __restrict__ bg, const float* __restrict__ C, const float* __restrict__ den,
    const float* __restrict__ gC, float* __restrict__ part, float* __restrict__ gwb_part) {
  __shared__ float4 s_px[256];
  __shared__ float4 s_fa[256];  // phi 0..3
  __shared__ float2 s_fb[256];  // phi 4..5
  __shared__ float s_ftmp[4];
  const int band = blockIdx.y;
  const int g = blockIdx.x * 256 + threadIdx.x;
  const bool act = g < G;
  float th[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float og = 0.f, kp = 0.f, col[3] = {0.f, 0.f, 0.f};
  if (act) {
#pragma unroll
    for (int i = 0; i < 6; ++i) th[i] = theta[(int64_t)g * 6 + i];
    og = o[g];
    kp = (keep && !keep[g]) ? 0.0f : 1.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i) col[i] = color[(int64_t)g * 3 + i];
  }
  const float ok = og * kp;
  const float cr = ok * col[0], cg = ok * col[1], cb = ok * col[2];
  float st[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float gr = 0.f, gg = 0.f, gbl = 0.f, gd = 0.f;
  float wpart = 0.f;
  const int pend = min(P, (band + 1) * PB);
  for (int p0 = band * PB; p0 < pend; p0 += 256) {
    __syncthreads();
    const int pp = p0 + threadIdx.x;
    const bool in = pp < pend;
    wpart += stage_pixel_grads(C, den, gC, pp, in, bg, s_px);
    float4 fa = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 fb = make_float2(0.f, 0.f);
    if (in) {
      const float* f = phi + (int64_t)pp * 6;
      fa = make_float4(f[0], f[1], f[2], f[3]);
      fb = make_float2(f[4], f[5]);
    }
    s_fa[threadIdx.x] = fa;
    s_fb[threadIdx.x] = fb;
    __syncthreads();
    const int n = min(256, pend - p0);
    for (int j = 0; j < n; ++j) {
      const float4 q = s_px[j];
      const float4 fa2 = s_fa[j];
      const float2 fb2 = s_fb[j];
      const float u = fa2.x * th[0] + fa2.y * th[1] + fa2.z * th[2] + fa2.w * th[3] +
                      fb2.x * th[4] + fb2.y * th[5];
      const float r = fmaxf(u, 0.0f);
      const float w = r * r;
      gr += w * q.x;
      gg += w * q.y;
      gbl += w * q.z;
      gd += w * q.w;
      const float gu = r * (q.x * cr + q.y * cg + q.z * cb + q.w * ok);  // half of dL/du
      st[0] += gu * fa2.x;
      st[1] += gu * fa2.y;
      st[2] += gu * fa2.z;
      st[3] += gu * fa2.w;
      st[4] += gu * fb2.x;
      st[5] += gu * fb2.y;
    }
  }
  if (blockIdx.x == 0) {
    const float tot = block_sum256(wpart, s_ftmp);
    if (threadIdx.x == 0) gwb_part[band] = tot;
  }
  if (act) {
    float* dst = part + ((int64_t)band * G + g) * kThetaComp;
#pragma unroll
    for (int i = 0; i < 6; ++i) dst[i] = 2.0f * st[i];
    // num = sum w_geo*o*keep*color, den = sum w_geo*o*keep + w_b
    dst[6] = kp * (col[0] * gr + col[1] * gg + col[2] * gbl + gd);  // dL/do
    dst[7] = ok * gr;                                              // dL/dcolor
    dst[8] = ok * gg;
    dst[9] = ok * gbl;
  }
}

// out[g][c] = sum over bands of part[band][g][c], in band order; gwb = sum of gwb_part.
__global__ __launch_bounds__(256) void k_dense_reduce(const float* __restrict__ part, int nb,
                                                      int G, int ncomp,
                                                      const float* __restrict__ gwb_part,
                                                      float* __restrict__ out,
                                                      float* __restrict__ gwb) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = (int64_t)G * ncomp;
  if (i < n) {
    float s = 0.f;
    for (int b = 0; b < nb; ++b) s += part[(int64_t)b * n + i];
    out[i] = s;
  }
  if (i == 0 && gwb) {
    float s = 0.f;
    for (int b = 0; b < nb; ++b) s += gwb_part[b];
    gwb[0] = s;
  }
}

// Unpacks the workspace into (partials, gwb partials); returns the band count or an error.
inline int dense_ws(void* ws, size_t ws_bytes, int G, int P, int ncomp, float** part,
                    float** gwbp, int* PB) {
  if (!ws) return TTS_EWORKSPACE;
  if (ws_bytes < dense_ws_bytes(G, P, ncomp)) return TTS_EWORKSPACE;
  *PB = dense_band_pixels(G, P);
  const int nb = (P + *PB - 1) / *PB;
  uintptr_t base = (reinterpret_cast<uintptr_t>(ws) + 255) & ~uintptr_t(255);
  *gwbp = reinterpret_cast<float*>(base);
  *part = reinterpret_cast<float*>(base + (((size_t)nb * 4 + 255) & ~size_t(255)));
  return nb;
}

}  // namespace tts

using namespace tts;

extern "C" {

size_t tts_dense_workspace_bytes(int G, int P) {
  // sized for the larger (theta form) partial record; serves both forms
  return dense_ws_bytes(G, P, kThetaComp);
}

int tts_render_dense(const float* proj, int G, int H, int W, float k, const float* bg,
                     float* image, float* den, hipStream_t stream) {
  if ((G > 0 && !proj) || !bg || !image || H <= 0 || W <= 0 || G < 0 || !(k > 0.0f))
    return TTS_EINVAL;
  if (G > (1 << 30)) return TTS_EG;
  if ((int64_t)H * W > (int64_t(1) << 30)) return TTS_EINVAL;
  const int P = H * W;
  k_render_dense<<<grid1d(P, 256), 256, 0, stream>>>(proj, G, W, P, (float)(1.0 / (double)k), bg,
                                                     image, den);
  return launch_status();
}

int tts_render_dense_bwd(const float* proj, int G, int H, int W, float k, const float* bg,
                         const float* image, const float* den, const float* gimage, float* grad9,
                         float* gwb, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  if (!proj || !bg || !image || !den || !gimage || !grad9 || H <= 0 || W <= 0 || G <= 0 ||
      !(k > 0.0f))
    return TTS_EINVAL;
  if (G > (1 << 30)) return TTS_EG;
  if ((int64_t)H * W > (int64_t(1) << 30)) return TTS_EINVAL;
  const int P = H * W;
  float *part, *gwbp;
  int PB;
  const int nb = dense_ws(workspace, workspace_bytes, G, P, kQuadComp, &part, &gwbp, &PB);
  if (nb < 0) return nb;
  dim3 grid(grid1d(G, 256), nb);
  k_render_dense_bwd<<<grid, 256, 0, stream>>>(proj, G, W, P, PB, (float)(1.0 / (double)k), bg,
                                               image, den, gimage, part, gwbp);
  k_dense_reduce<<<grid1d((int64_t)G * kQuadComp, 256), 256, 0, stream>>>(part, nb, G, kQuadComp,
                                                                         gwbp, grad9, gwb);
  return launch_status();
}

int tts_wsr_dense(const float* theta, const float* o, const float* color, const uint8_t* keep,
                  const float* phi, int G, int P, const float* bg, float* C, float* den,
                  hipStream_t stream) {
  if ((G > 0 && (!theta || !o || !color)) || !phi || !bg || !C || P <= 0 || G < 0)
    return TTS_EINVAL;
  if (G > (1 << 30) || P > (1 << 30)) return TTS_EINVAL;
  k_wsr_dense<<<grid1d(P, 256), 256, 0, stream>>>(theta, o, color, keep, phi, G, P, bg, C, den);
  return launch_status();
}

int tts_wsr_dense_bwd(const float* theta, const float* o, const float* color,
                      const uint8_t* keep, const float* phi, int G, int P, const float* bg,
                      const float* C, const float* den, const float* gC, float* gtheta10,
                      float* gwb, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!theta || !o || !color || !phi || !bg || !C || !den || !gC || !gtheta10 || P <= 0 ||
      G <= 0)
    return TTS_EINVAL;
  if (G > (1 << 30) || P > (1 << 30)) return TTS_EINVAL;
  float *part, *gwbp;
  int PB;
  const int nb = dense_ws(workspace, workspace_bytes, G, P, kThetaComp, &part, &gwbp, &PB);
  if (nb < 0) return nb;
  dim3 grid(grid1d(G, 256), nb);
  k_wsr_dense_bwd<<<grid, 256, 0, stream>>>(theta, o, color, keep, phi, G, P, PB, bg, C, den, gC,
                                            part, gwbp);
  k_dense_reduce<<<grid1d((int64_t)G * kThetaComp, 256), 256, 0, stream>>>(
      part, nb, G, kThetaComp, gwbp, gtheta10, gwb);
  return launch_status();
}

}  // extern "C"
