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
//
// The quad form also renders the two per-pixel occlusion arms of spike/arms.py (ARM template):
//   SZ (soft-Z, :50-68):  W0 = o w_geo, z* = sum W0 z / (sum W0 + 1e-6) per pixel (pass 1),
//        h = sigmoid(-beta (z - z*)), C = WSR(W0 h) (pass 2); z is a constant of the gradient,
//        z* is not: its gradient Z = sum_g dL/dh h (1 - h) beta is a pixel pre-pass of the
//        backward, and dL/dW0 += Z (z - z*) / den0.  beta (softz_beta) gets a gradient too.
//   RV (revealage, :71-83): C = C_avg (1 - R) + c_b R, C_avg = sum W color / (sum W + 1e-6),
//        R = exp(sum log(1 - min(W, 1 - 1e-4))) (no w_b); dL/dW gains -dL/dlogR / (1 - a).
// aux [P,4] carries the per-pixel forward state to the backward (SZ: z*, den0; RV: R, C_avg).

#include "tts_common.h"

namespace tts {

constexpr int kDenseChunk = 256;
constexpr int kArmA = 0, kArmSZ = 1, kArmRV = 2;   // TTS_ARM_* values
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

// Workspace layout: [align to 256][gwb partials, nb floats, padded to 256]
// [per-pixel scratch, P floats, padded to 256][partials nb*G*ncomp].
inline size_t dense_ws_bytes(int G, int P, int ncomp) {
  if (G <= 0 || P <= 0) return 0;
  const int pb = dense_band_pixels(G, P);
  const size_t nb = (size_t)((P + pb - 1) / pb);
  return 256 + ((nb * 4 + 255) & ~size_t(255)) + (((size_t)P * 4 + 255) & ~size_t(255)) +
         nb * (size_t)G * ncomp * 4;
}

// ---------------------------------------------------------------- forward

template <int ARM>
__global__ __launch_bounds__(256) void k_render_dense(const float* __restrict__ proj, int G,
                                                      int W, int P, float inv_k,
                                                      const float* __restrict__ bg,
                                                      const float* __restrict__ szb,
                                                      float* __restrict__ image,
                                                      float* __restrict__ den_out,
                                                      float4* __restrict__ aux) {
  __shared__ float4 s_a[kDenseChunk];  // mu_x, mu_y, a, 2b
  __shared__ float4 s_b[kDenseChunk];  // c, col_o r, g, b
  __shared__ float2 s_o[kDenseChunk];  // o_col, depth
  const int p = blockIdx.x * 256 + threadIdx.x;
  const float px = (float)(p % W) + 0.5f, py = (float)(p / W) + 0.5f;
  const float beta = ARM == kArmSZ ? szb[0] : 0.0f;
  float zstar = 0.0f, den0 = 0.0f;
  // SZ runs the gaussian loop twice: pass 0 finds z*, pass 1 blends
  for (int pass = (ARM == kArmSZ ? 0 : 1); pass < 2; ++pass) {
    float nr = 0.f, ng = 0.f, nb = 0.f, nd = 0.f, lr = 0.f;
    for (int g0 = 0; g0 < G; g0 += kDenseChunk) {
      const int n = min(kDenseChunk, G - g0);
      __syncthreads();
      if ((int)threadIdx.x < n) {
        const float4* r = reinterpret_cast<const float4*>(proj + (int64_t)(g0 + threadIdx.x) * 12);
        const float4 r0 = r[0], r1 = r[1], r2 = r[2];
        s_a[threadIdx.x] = make_float4(r0.x, r0.y, r0.z, 2.0f * r0.w);
        s_b[threadIdx.x] = make_float4(r1.x, r1.z, r1.w, r2.x);
        s_o[threadIdx.x] = make_float2(r2.y, r1.y);
      }
      __syncthreads();
      for (int j = 0; j < n; ++j) {
        const float4 A = s_a[j], B = s_b[j];
        const float2 O = s_o[j];
        const float dx = px - A.x, dy = py - A.y;
        const float Q = (A.z * dx + A.w * dy) * dx + (B.x * dy) * dy;
        const float r = relu_nan(1.0f - Q * inv_k);
        float w = r * r;
        if (ARM == kArmSZ && pass == 0) {
          nd += w * O.x;
          nr += w * O.x * O.y;
          continue;
        }
        if (ARM == kArmSZ) w *= sigmoidf_(-beta * (O.y - zstar));
        if (ARM == kArmRV) lr += log1pf(-fminf(w * O.x, 1.0f - 1e-4f));
        nr += w * B.y;
        ng += w * B.z;
        nb += w * B.w;
        nd += w * O.x;
      }
    }
    if (ARM == kArmSZ && pass == 0) {
      den0 = nd + 1e-6f;
      zstar = nr / den0;
      continue;
    }
    if (p < P) {
      if (ARM == kArmRV) {
        const float d = nd + 1e-6f, R = expf(lr);
        const float a0 = nr / d, a1 = ng / d, a2 = nb / d;
        image[(int64_t)p * 3 + 0] = a0 * (1.0f - R) + bg[1] * R;
        image[(int64_t)p * 3 + 1] = a1 * (1.0f - R) + bg[2] * R;
        image[(int64_t)p * 3 + 2] = a2 * (1.0f - R) + bg[3] * R;
        if (den_out) den_out[p] = d;
        aux[p] = make_float4(R, a0, a1, a2);
      } else {
        const float wb = bg[0];
        const float d = nd + wb;
        image[(int64_t)p * 3 + 0] = (nr + wb * bg[1]) / d;
        image[(int64_t)p * 3 + 1] = (ng + wb * bg[2]) / d;
        image[(int64_t)p * 3 + 2] = (nb + wb * bg[3]) / d;
        if (den_out) den_out[p] = d;
        if (ARM == kArmSZ) aux[p] = make_float4(zstar, den0, 0.0f, 0.0f);
      }
    }
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
      const float r = relu_nan(u);
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

// Per-pixel WSR gradients of the quad form, staged in LDS: (gnum r,g,b, gden) and the arm's
// pair-independent extras (SZ: z*, Z/den0; RV: dL/dlogR).  Returns this thread's share of
// dL/dw_b (zero for RV, which has no w_b).
template <int ARM>
__device__ __forceinline__ float stage_arm_grads(const float* __restrict__ image,
                                                 const float* __restrict__ den,
                                                 const float4* __restrict__ aux,
                                                 const float* __restrict__ zk,
                                                 const float* __restrict__ gimage, int p, bool in,
                                                 const float* __restrict__ bg, float4* s_px,
                                                 float2* s_ex) {
  if (ARM != kArmRV) {
    const float wpart = stage_pixel_grads(image, den, gimage, p, in, bg, s_px);
    if (ARM == kArmSZ) s_ex[threadIdx.x] = in ? make_float2(aux[p].x, zk[p]) : make_float2(0.f, 0.f);
    return wpart;
  }
  float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
  float gs = 0.0f;
  if (in) {
    const float4 x = aux[p];  // R, C_avg
    const float R = x.x, inv = 1.0f / den[p];
    const float g0 = gimage[(int64_t)p * 3 + 0], g1 = gimage[(int64_t)p * 3 + 1],
                g2 = gimage[(int64_t)p * 3 + 2];
    const float k = (1.0f - R) * inv;  // dC/dC_avg / den
    q = make_float4(g0 * k, g1 * k, g2 * k, -(g0 * x.y + g1 * x.z + g2 * x.w) * k);
    // dL/dR * R = dL/dlogR
    gs = (g0 * (bg[1] - x.y) + g1 * (bg[2] - x.z) + g2 * (bg[3] - x.w)) * R;
  }
  s_px[threadIdx.x] = q;
  s_ex[threadIdx.x] = make_float2(gs, 0.0f);
  return 0.0f;
}

// Soft-Z backward pre-pass, one thread per pixel: Z/den0 with Z = dL/dz* =
// beta sum_g w_geo (gnum . col_o + gden o_col) h (1 - h).
__global__ __launch_bounds__(256) void k_softz_pre(const float* __restrict__ proj, int G, int W,
                                                   int P, float inv_k,
                                                   const float* __restrict__ szb,
                                                   const float* __restrict__ image,
                                                   const float* __restrict__ den,
                                                   const float4* __restrict__ aux,
                                                   const float* __restrict__ gimage,
                                                   float* __restrict__ zk) {
  __shared__ float4 s_a[kDenseChunk];
  __shared__ float4 s_b[kDenseChunk];
  __shared__ float2 s_o[kDenseChunk];
  const int p = blockIdx.x * 256 + threadIdx.x;
  const bool in = p < P;
  const float px = (float)(p % W) + 0.5f, py = (float)(p / W) + 0.5f;
  const float beta = szb[0];
  float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f, zs = 0.f, d0 = 1.f;
  if (in) {
    const float inv = 1.0f / den[p];
    const float g0 = gimage[(int64_t)p * 3 + 0], g1 = gimage[(int64_t)p * 3 + 1],
                g2 = gimage[(int64_t)p * 3 + 2];
    q0 = g0 * inv; q1 = g1 * inv; q2 = g2 * inv;
    q3 = -(g0 * image[(int64_t)p * 3 + 0] + g1 * image[(int64_t)p * 3 + 1] +
           g2 * image[(int64_t)p * 3 + 2]) * inv;
    zs = aux[p].x;
    d0 = aux[p].y;
  }
  float Z = 0.0f;
  for (int g0 = 0; g0 < G; g0 += kDenseChunk) {
    const int n = min(kDenseChunk, G - g0);
    __syncthreads();
    if ((int)threadIdx.x < n) {
      const float4* r = reinterpret_cast<const float4*>(proj + (int64_t)(g0 + threadIdx.x) * 12);
      const float4 r0 = r[0], r1 = r[1], r2 = r[2];
      s_a[threadIdx.x] = make_float4(r0.x, r0.y, r0.z, 2.0f * r0.w);
      s_b[threadIdx.x] = make_float4(r1.x, r1.z, r1.w, r2.x);
      s_o[threadIdx.x] = make_float2(r2.y, r1.y);
    }
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      const float4 A = s_a[j], B = s_b[j];
      const float2 O = s_o[j];
      const float dx = px - A.x, dy = py - A.y;
      const float Q = (A.z * dx + A.w * dy) * dx + (B.x * dy) * dy;
      const float r = relu_nan(1.0f - Q * inv_k);
      const float h = sigmoidf_(-beta * (O.y - zs));
      Z += r * r * (q0 * B.y + q1 * B.z + q2 * B.w + q3 * O.x) * h * (1.0f - h);
    }
  }
  if (in) zk[p] = beta * Z / d0;
}

// ncomp = 9 (a, b, c, mu_x, mu_y, col_o rgb, o_col), 10 for SZ (+ this gaussian's dL/dbeta).
template <int ARM>
__global__ __launch_bounds__(256) void k_render_dense_bwd(
    const float* __restrict__ proj, int G, int W, int P, int PB, float inv_k,
    const float* __restrict__ bg, const float* __restrict__ szb, const float* __restrict__ image,
    const float* __restrict__ den, const float4* __restrict__ aux, const float* __restrict__ zk,
    const float* __restrict__ gimage, float* __restrict__ part, float* __restrict__ gwb_part) {
  constexpr int NC = ARM == kArmSZ ? kQuadComp + 1 : kQuadComp;
  __shared__ float4 s_px[256];
  __shared__ float2 s_xy[256];
  __shared__ float2 s_ex[256];
  __shared__ float s_ftmp[4];
  const int band = blockIdx.y;
  const int g = blockIdx.x * 256 + threadIdx.x;
  const bool act = g < G;
  float mx = 0.f, my = 0.f, a = 0.f, b = 0.f, c = 0.f, cr = 0.f, cg = 0.f, cb = 0.f, oc = 0.f;
  float zg = 0.f;
  if (act) {
    const float4* r = reinterpret_cast<const float4*>(proj + (int64_t)g * 12);
    const float4 r0 = r[0], r1 = r[1], r2 = r[2];
    mx = r0.x; my = r0.y; a = r0.z; b = r0.w; c = r1.x;
    cr = r1.z; cg = r1.w; cb = r2.x; oc = r2.y;
    zg = r1.y;
  }
  const float beta = ARM == kArmSZ ? szb[0] : 0.0f;
  const float b2 = 2.0f * b;
  float sxx = 0.f, sxy = 0.f, syy = 0.f, sx = 0.f, sy = 0.f;
  float gr = 0.f, gg = 0.f, gbl = 0.f, go = 0.f, gbeta = 0.f;
  float wpart = 0.f;
  const int pend = min(P, (band + 1) * PB);
  for (int p0 = band * PB; p0 < pend; p0 += 256) {
    __syncthreads();
    const int pp = p0 + threadIdx.x;
    wpart += stage_arm_grads<ARM>(image, den, aux, zk, gimage, pp, pp < pend, bg, s_px, s_ex);
    s_xy[threadIdx.x] = make_float2((float)(pp % W) + 0.5f, (float)(pp / W) + 0.5f);
    __syncthreads();
    const int n = min(256, pend - p0);
    for (int j = 0; j < n; ++j) {
      const float4 q = s_px[j];
      const float2 xy = s_xy[j];
      const float dx = xy.x - mx, dy = xy.y - my;
      const float Q = (a * dx + b2 * dy) * dx + (c * dy) * dy;
      const float r = relu_nan(1.0f - Q * inv_k);
      const float w = r * r;
      const float gw = q.x * cr + q.y * cg + q.z * cb + q.w * oc;  // dL/dw_geo of arm A
      float dw;                                                   // dL/dw_geo of this arm
      if (ARM == kArmSZ) {
        const float2 ex = s_ex[j];  // z*, Z/den0
        const float h = sigmoidf_(-beta * (zg - ex.x));
        const float e = ex.y * (zg - ex.x);  // dL/dW0 through z*
        gr += w * h * q.x;
        gg += w * h * q.y;
        gbl += w * h * q.z;
        go += w * (h * q.w + e);
        gbeta -= w * gw * h * (1.0f - h) * (zg - ex.x);
        dw = h * gw + oc * e;
      } else if (ARM == kArmRV) {
        const float W0 = w * oc;
        const float e = W0 <= 1.0f - 1e-4f ? -s_ex[j].x / (1.0f - W0) : 0.0f;  // clamp gate
        gr += w * q.x;
        gg += w * q.y;
        gbl += w * q.z;
        go += w * (q.w + e);
        dw = gw + oc * e;
      } else {
        gr += w * q.x;
        gg += w * q.y;
        gbl += w * q.z;
        go += w * q.w;
        dw = gw;
      }
      const float gu = r * dw;  // half of dL/du
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
    float* dst = part + ((int64_t)band * G + g) * NC;
    dst[0] = mxx;                          // dQ/da = dx^2
    dst[1] = 2.0f * mxy;                   // dQ/db = 2 dx dy
    dst[2] = myy;                          // dQ/dc = dy^2
    dst[3] = -2.0f * (a * m_x + b * m_y);  // dQ/dmu_x = -2 (a dx + b dy)
    dst[4] = -2.0f * (b * m_x + c * m_y);  // dQ/dmu_y = -2 (b dx + c dy)
    dst[5] = gr;
    dst[6] = gg;
    dst[7] = gbl;
    dst[8] = go;
    if (ARM == kArmSZ) dst[9] = gbeta;
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
      const float r = relu_nan(u);
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

// Unpacks the workspace into (partials, gwb partials, per-pixel scratch); returns the band
// count or an error.
inline int dense_ws(void* ws, size_t ws_bytes, int G, int P, int ncomp, float** part,
                    float** gwbp, int* PB, float** pix = nullptr) {
  if (!ws) return TTS_EWORKSPACE;
  if (ws_bytes < dense_ws_bytes(G, P, ncomp)) return TTS_EWORKSPACE;
  *PB = dense_band_pixels(G, P);
  const int nb = (P + *PB - 1) / *PB;
  uintptr_t base = (reinterpret_cast<uintptr_t>(ws) + 255) & ~uintptr_t(255);
  *gwbp = reinterpret_cast<float*>(base);
  base += ((size_t)nb * 4 + 255) & ~size_t(255);
  if (pix) *pix = reinterpret_cast<float*>(base);
  base += ((size_t)P * 4 + 255) & ~size_t(255);
  *part = reinterpret_cast<float*>(base);
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
  k_render_dense<kArmA><<<grid1d(P, 256), 256, 0, stream>>>(
      proj, G, W, P, (float)(1.0 / (double)k), bg, nullptr, image, den, nullptr);
  return launch_status();
}

int tts_render_dense_arm(const float* proj, int G, int H, int W, float k, const float* bg,
                         int arm, const float* softz_beta, float* image, float* den, float* aux,
                         hipStream_t stream) {
  if ((G > 0 && !proj) || !bg || !image || H <= 0 || W <= 0 || G < 0 || !(k > 0.0f))
    return TTS_EINVAL;
  if (arm != kArmA && arm != kArmSZ && arm != kArmRV) return TTS_EINVAL;
  if (arm != kArmA && !aux) return TTS_EINVAL;
  if (arm == kArmSZ && !softz_beta) return TTS_EINVAL;
  if (G > (1 << 30)) return TTS_EG;
  if ((int64_t)H * W > (int64_t(1) << 30)) return TTS_EINVAL;
  const int P = H * W;
  const float ik = (float)(1.0 / (double)k);
  float4* ax = reinterpret_cast<float4*>(aux);
  const dim3 grid = grid1d(P, 256);
  if (arm == kArmSZ)
    k_render_dense<kArmSZ><<<grid, 256, 0, stream>>>(proj, G, W, P, ik, bg, softz_beta, image,
                                                     den, ax);
  else if (arm == kArmRV)
    k_render_dense<kArmRV><<<grid, 256, 0, stream>>>(proj, G, W, P, ik, bg, nullptr, image, den,
                                                     ax);
  else
    k_render_dense<kArmA><<<grid, 256, 0, stream>>>(proj, G, W, P, ik, bg, nullptr, image, den,
                                                    nullptr);
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
  k_render_dense_bwd<kArmA><<<grid, 256, 0, stream>>>(proj, G, W, P, PB, (float)(1.0 / (double)k),
                                                      bg, nullptr, image, den, nullptr, nullptr,
                                                      gimage, part, gwbp);
  k_dense_reduce<<<grid1d((int64_t)G * kQuadComp, 256), 256, 0, stream>>>(part, nb, G, kQuadComp,
                                                                         gwbp, grad9, gwb);
  return launch_status();
}

int tts_render_dense_arm_bwd(const float* proj, int G, int H, int W, float k, const float* bg,
                             int arm, const float* softz_beta, const float* image,
                             const float* den, const float* aux, const float* gimage,
                             float* grad10, float* gwb, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  if (!proj || !bg || !image || !den || !gimage || !grad10 || H <= 0 || W <= 0 || G <= 0 ||
      !(k > 0.0f))
    return TTS_EINVAL;
  if (arm != kArmA && arm != kArmSZ && arm != kArmRV) return TTS_EINVAL;
  if (arm != kArmA && !aux) return TTS_EINVAL;
  if (arm == kArmSZ && !softz_beta) return TTS_EINVAL;
  if (G > (1 << 30)) return TTS_EG;
  if ((int64_t)H * W > (int64_t(1) << 30)) return TTS_EINVAL;
  const int P = H * W;
  const int nc = arm == kArmSZ ? kQuadComp + 1 : kQuadComp;
  float *part, *gwbp, *zk;
  int PB;
  const int nb = dense_ws(workspace, workspace_bytes, G, P, nc, &part, &gwbp, &PB, &zk);
  if (nb < 0) return nb;
  const float ik = (float)(1.0 / (double)k);
  const float4* ax = reinterpret_cast<const float4*>(aux);
  dim3 grid(grid1d(G, 256), nb);
  if (arm == kArmSZ) {
    k_softz_pre<<<grid1d(P, 256), 256, 0, stream>>>(proj, G, W, P, ik, softz_beta, image, den,
                                                    ax, gimage, zk);
    k_render_dense_bwd<kArmSZ><<<grid, 256, 0, stream>>>(proj, G, W, P, PB, ik, bg, softz_beta,
                                                         image, den, ax, zk, gimage, part, gwbp);
  } else if (arm == kArmRV) {
    k_render_dense_bwd<kArmRV><<<grid, 256, 0, stream>>>(proj, G, W, P, PB, ik, bg, nullptr, image,
                                                         den, ax, nullptr, gimage, part, gwbp);
  } else {
    k_render_dense_bwd<kArmA><<<grid, 256, 0, stream>>>(proj, G, W, P, PB, ik, bg, nullptr, image,
                                                        den, nullptr, nullptr, gimage, part, gwbp);
  }
  k_dense_reduce<<<grid1d((int64_t)G * nc, 256), 256, 0, stream>>>(part, nb, G, nc, gwbp, grad10,
                                                                  gwb);
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
