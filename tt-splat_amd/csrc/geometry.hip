// Per-gaussian kernels: EWA projection + activations, their backward, and Adam.
// One thread per gaussian; all fp32.  The math follows spike/geometry.py:10-57,
// spike/forward.py:69-71 and tools/m4_train_binned.py:194-202; the backward is the chain rule
// of that forward (derived below, checked against torch autograd of the CPU oracle).
//
// View-dependent colour (the *_sh kernels): real spherical harmonics of degree 1-3 on top of the
// DC term, evaluated in the direction means3d - camera centre (spike/sh.py:54-72, as the device
// step uses it, tools/resident_traced.py:246-264,339-341).  The rest coefficients are stored
// coefficient-major, rest[(l * 3 + c) * G + g] for l = 0..14 (SH index l + 1) and channel c, so
// every load and store of a wave is coalesced.  Their gradient is b_{l+1}(dir) * dL/dcolour
// through the clamp gate; the direction is a constant of the backward, as in
// tools/resident_traced.py:405-410 (no gradient reaches the means through it).
//
// Depth weight (the occlusion lever of spike/arms.py:34-37 on the device step,
// tools/resident_traced.py:333-337,418-426): keo = keep * sigmoid(op) * rho with
// rho = sigmoid(beta (tau - z_cam)), beta and tau two global device scalars.  The backward gives
// per-gaussian dL/dbeta = g (tau - z_cam), dL/dtau = g beta with g = dL/dkeo keep o rho (1 - rho);
// like the reference's device step, no gradient reaches the means through z_cam unless asked
// (DepthW::zgrad, the dense arm-B autograd of spike/render.py).

#include <math.h>

#include <atomic>

#include "bin_count.h"

namespace tts {

// Forward intermediates kept for the backward (all recomputed from params, never stored).
struct GeoState {
  float qn[4];       // normalised quaternion w,x,y,z
  float qnorm;       // |q| before the 1e-12 clamp
  float qdiv;        // max(|q|, 1e-12)
  float M[3][3];     // R_v * R(q)
  float s2[3];       // exp(log_scale)^2
  float SC[3][3];    // camera-space covariance M diag(s2) M^T
  float mc[3];       // camera-space mean
  float z;           // max(depth, near)
  bool zmask;        // depth >= near (gradient passes the clamp)
  bool keep;         // depth > near
  float J00, J02, J11, J12;
  float s00, s01, s11;
  float det_inv;     // 1 / max(det, 1e-12)
  bool dmask;        // det >= 1e-12
  float mux, muy, a, b, c;
  float craw[3];     // colour before the clamp: 0.5 + C0*dc (+ the SH rest terms)
  float color[3];    // max(craw, 0)
  float o;           // sigmoid(op)
  float rho;         // depth weight sigmoid(beta (tau - z_cam)), 1 without one
  float dw_beta, dw_tau;
  bool dw;
};

// Depth-weight arguments of the geometry kernels.
struct DepthW {
  const float* bt;   // device (beta, tau), or null: no depth weight
  float* grad;       // [G,2] per-gaussian dL/d(beta, tau), or null
  float scale;       // grad (+)= scale * value
  int accumulate;    // 1: grad += ..., 0: grad = ...
  int zgrad;         // TTS_GRAD_DEPTH_Z: dL/dz_cam through rho reaches the means; TTS_GRAD_SH_DIR
                     // (k_geom_bwd): the SH colour's gradient through its direction too
};
__device__ __forceinline__ void depthw_store(const DepthW& d, int g, const float* v) {
  if (!d.bt || !d.grad) return;
  float* o = d.grad + (int64_t)g * 2;
  if (d.accumulate) {
    o[0] += d.scale * v[0];
    o[1] += d.scale * v[1];
  } else {
    o[0] = d.scale * v[0];
    o[1] = d.scale * v[1];
  }
}

// SH constants (spike/sh.py:9-19,43-51): normalisation of the real SH basis, inria/gsplat signs.
constexpr float kSC1 = 0.4886025119029199f;
constexpr float kSC2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                           -1.0925484305920792f, 0.5462742152960396f};
constexpr float kSC3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                           0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                           -0.5900435899266435f};
constexpr int kShRest = 15;  // rest coefficients per channel at degree 3
__host__ __device__ __forceinline__ int sh_rest_count(int deg) { return (deg + 1) * (deg + 1) - 1; }

__device__ __forceinline__ void geo_forward(const float* __restrict__ p, const Camera& cam,
                                            float near_z, float blur, GeoState& s,
                                            const float* __restrict__ dw = nullptr) {
  const float qw = p[3], qx = p[4], qy = p[5], qz = p[6];
  s.qnorm = sqrtf(qw * qw + qx * qx + qy * qy + qz * qz);
  s.qdiv = fmaxf(s.qnorm, 1e-12f);
  const float w = qw / s.qdiv, x = qx / s.qdiv, y = qy / s.qdiv, z = qz / s.qdiv;
  s.qn[0] = w; s.qn[1] = x; s.qn[2] = y; s.qn[3] = z;
  float R[3][3];
  R[0][0] = 1.f - 2.f * (y * y + z * z); R[0][1] = 2.f * (x * y - w * z); R[0][2] = 2.f * (x * z + w * y);
  R[1][0] = 2.f * (x * y + w * z); R[1][1] = 1.f - 2.f * (x * x + z * z); R[1][2] = 2.f * (y * z - w * x);
  R[2][0] = 2.f * (x * z - w * y); R[2][1] = 2.f * (y * z + w * x); R[2][2] = 1.f - 2.f * (x * x + y * y);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float sc = expf(p[7 + i]);
    s.s2[i] = sc * sc;
  }
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int k = 0; k < 3; ++k)
      s.M[i][k] = cam.R[3 * i + 0] * R[0][k] + cam.R[3 * i + 1] * R[1][k] + cam.R[3 * i + 2] * R[2][k];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int l = 0; l < 3; ++l)
      s.SC[i][l] = s.M[i][0] * s.M[l][0] * s.s2[0] + s.M[i][1] * s.M[l][1] * s.s2[1] +
                   s.M[i][2] * s.M[l][2] * s.s2[2];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    s.mc[i] = cam.R[3 * i + 0] * p[0] + cam.R[3 * i + 1] * p[1] + cam.R[3 * i + 2] * p[2] + cam.t[i];
  const float depth = s.mc[2];
  s.keep = depth > near_z;
  s.zmask = depth >= near_z;
  s.z = fmaxf(depth, near_z);
  const float zi = 1.0f / s.z;
  s.mux = cam.fx * s.mc[0] / s.z + cam.cx;
  s.muy = cam.fy * s.mc[1] / s.z + cam.cy;
  s.J00 = cam.fx * zi;
  s.J11 = cam.fy * zi;
  s.J02 = -cam.fx * s.mc[0] / (s.z * s.z);
  s.J12 = -cam.fy * s.mc[1] / (s.z * s.z);
  s.s00 = s.J00 * s.J00 * s.SC[0][0] + 2.f * s.J00 * s.J02 * s.SC[0][2] + s.J02 * s.J02 * s.SC[2][2] + blur;
  s.s11 = s.J11 * s.J11 * s.SC[1][1] + 2.f * s.J11 * s.J12 * s.SC[1][2] + s.J12 * s.J12 * s.SC[2][2] + blur;
  s.s01 = s.J00 * s.J11 * s.SC[0][1] + s.J00 * s.J12 * s.SC[0][2] + s.J02 * s.J11 * s.SC[1][2] +
          s.J02 * s.J12 * s.SC[2][2];
  const float det = s.s00 * s.s11 - s.s01 * s.s01;
  s.dmask = det >= 1e-12f;
  s.det_inv = 1.0f / fmaxf(det, 1e-12f);
  s.a = s.s11 * s.det_inv;
  s.b = -s.s01 * s.det_inv;
  s.c = s.s00 * s.det_inv;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    s.craw[i] = 0.5f + kC0 * p[10 + i];
    s.color[i] = fmaxf(s.craw[i], 0.0f);
  }
  s.o = sigmoidf_(p[13]);
  s.dw = dw != nullptr;
  if (dw) {
    s.dw_beta = dw[0];
    s.dw_tau = dw[1];
    s.rho = sigmoidf_(s.dw_beta * (s.dw_tau - depth));
  } else {
    s.dw_beta = s.dw_tau = 0.0f;
    s.rho = 1.0f;
  }
}

// Basis b[1..15] of the rest coefficients in the direction mean - camera centre
// (spike/sh.py:54-72; dir / max(|dir|, 1e-12)).  b[0] = C0 is the DC term's.
__device__ __forceinline__ void sh_basis(const float* __restrict__ p, const Camera& cam, float* b) {
  float d[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)  // centre = -R_v^T t_v
    d[i] = p[i] + (cam.R[0 * 3 + i] * cam.t[0] + cam.R[1 * 3 + i] * cam.t[1] +
                   cam.R[2 * 3 + i] * cam.t[2]);
  const float nrm = fmaxf(sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]), 1e-12f);
  const float x = d[0] / nrm, y = d[1] / nrm, z = d[2] / nrm;
  const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
  b[0] = kC0;
  b[1] = -kSC1 * y;
  b[2] = kSC1 * z;
  b[3] = -kSC1 * x;
  b[4] = kSC2[0] * xy;
  b[5] = kSC2[1] * yz;
  b[6] = kSC2[2] * (2.0f * zz - xx - yy);
  b[7] = kSC2[3] * xz;
  b[8] = kSC2[4] * (xx - yy);
  b[9] = kSC3[0] * y * (3.0f * xx - yy);
  b[10] = kSC3[1] * xy * z;
  b[11] = kSC3[2] * y * (4.0f * zz - xx - yy);
  b[12] = kSC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
  b[13] = kSC3[4] * x * (4.0f * zz - xx - yy);
  b[14] = kSC3[5] * z * (xx - yy);
  b[15] = kSC3[6] * x * (xx - 3.0f * yy);
}

// Gradient through the view direction (spike's dense autograd, spike/render.py:23-25: the
// direction d = mean - centre is not detached there).  gcol[c] = dL/d(raw colour c) after the
// clamp gate; gd_hat = sum_l grad b_l(d_hat) * sum_c gcol[c] rest_l,c, then through
// d_hat = d / max(|d|, 1e-12): dL/dd = (gd_hat - d_hat (d_hat . gd_hat)) / |d| (or gd_hat / 1e-12
// where the clamp holds).  Added to dL/dmeans.
__device__ __forceinline__ void sh_dir_grad(const float* __restrict__ p, const Camera& cam,
                                            const float* rv, int n, const float* gcol,
                                            float* gmean) {
  float d[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    d[i] = p[i] + (cam.R[0 * 3 + i] * cam.t[0] + cam.R[1 * 3 + i] * cam.t[1] +
                   cam.R[2 * 3 + i] * cam.t[2]);
  const float raw = sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
  const float nrm = fmaxf(raw, 1e-12f);
  const float x = d[0] / nrm, y = d[1] / nrm, z = d[2] / nrm;
  const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
  float a[kShRest];  // sum_c gcol[c] rest_l,c
#pragma unroll
  for (int l = 0; l < kShRest; ++l)
    a[l] = l < n ? gcol[0] * rv[l * 3 + 0] + gcol[1] * rv[l * 3 + 1] + gcol[2] * rv[l * 3 + 2]
                 : 0.0f;
  // grad of b_{l+1} w.r.t. (x, y, z), times a[l]
  float gx = -kSC1 * a[2], gy = -kSC1 * a[0], gz = kSC1 * a[1];
  gx += kSC2[0] * y * a[3] + (-2.0f * kSC2[2] * x) * a[5] + kSC2[3] * z * a[6] +
        2.0f * kSC2[4] * x * a[7];
  gy += kSC2[0] * x * a[3] + kSC2[1] * z * a[4] + (-2.0f * kSC2[2] * y) * a[5] -
        2.0f * kSC2[4] * y * a[7];
  gz += kSC2[1] * y * a[4] + 4.0f * kSC2[2] * z * a[5] + kSC2[3] * x * a[6];
  gx += 6.0f * kSC3[0] * xy * a[8] + kSC3[1] * yz * a[9] - 2.0f * kSC3[2] * xy * a[10] -
        6.0f * kSC3[3] * xz * a[11] + kSC3[4] * (4.0f * zz - 3.0f * xx - yy) * a[12] +
        2.0f * kSC3[5] * xz * a[13] + kSC3[6] * (3.0f * xx - 3.0f * yy) * a[14];
  gy += kSC3[0] * (3.0f * xx - 3.0f * yy) * a[8] + kSC3[1] * xz * a[9] +
        kSC3[2] * (4.0f * zz - xx - 3.0f * yy) * a[10] - 6.0f * kSC3[3] * yz * a[11] -
        2.0f * kSC3[4] * xy * a[12] - 2.0f * kSC3[5] * yz * a[13] - 6.0f * kSC3[6] * xy * a[14];
  gz += kSC3[1] * xy * a[9] + 8.0f * kSC3[2] * yz * a[10] +
        kSC3[3] * (6.0f * zz - 3.0f * xx - 3.0f * yy) * a[11] + 8.0f * kSC3[4] * xz * a[12] +
        kSC3[5] * (xx - yy) * a[13];
  if (raw > 1e-12f) {
    const float dot = x * gx + y * gy + z * gz;
    gmean[0] += (gx - x * dot) / nrm;
    gmean[1] += (gy - y * dot) / nrm;
    gmean[2] += (gz - z * dot) / nrm;
  } else {
    gmean[0] += gx / nrm;
    gmean[1] += gy / nrm;
    gmean[2] += gz / nrm;
  }
}

// Loads this gaussian's first n rest coefficients of each channel (rv[l * 3 + c]).
__device__ __forceinline__ void sh_load(const float* __restrict__ rest, int64_t G, int g, int n,
                                        float* rv) {
#pragma unroll
  for (int i = 0; i < 3 * kShRest; ++i) rv[i] = i < 3 * n ? rest[(int64_t)i * G + g] : 0.0f;
}

// Colour with the rest terms: craw = (C0*dc + sum_l b[l+1] rest[l]) + 0.5, color = max(craw, 0).
__device__ __forceinline__ void sh_apply(const float* __restrict__ p, const float* b,
                                         const float* rv, int n, GeoState& s) {
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float r = kC0 * p[10 + c];
#pragma unroll
    for (int l = 0; l < kShRest; ++l)
      if (l < n) r += b[l + 1] * rv[l * 3 + c];
    s.craw[c] = r + 0.5f;
    s.color[c] = fmaxf(s.craw[c], 0.0f);
  }
}

// Chain rule of geo_forward.  gin = (ga, gb, gc, gmux, gmuy, gcol_o r,g,b, go_col);
// gout = the 14 parameter gradients in [G,14] column order.
// ---- MCMC pieces (spike/mcmc.py) -----------------------------------------------------------
// Rotation of the normalised quaternion (w, x, y, z) (spike/geometry.py:10-19).
__device__ __forceinline__ void quat_rot(const float* q, float R[3][3]) {
  const float n = fmaxf(sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]), 1e-12f);
  const float w = q[0] / n, x = q[1] / n, y = q[2] / n, z = q[3] / n;
  R[0][0] = 1.f - 2.f * (y * y + z * z); R[0][1] = 2.f * (x * y - w * z); R[0][2] = 2.f * (x * z + w * y);
  R[1][0] = 2.f * (x * y + w * z); R[1][1] = 1.f - 2.f * (x * x + z * z); R[1][2] = 2.f * (y * z - w * x);
  R[2][0] = 2.f * (x * z - w * y); R[2][1] = 2.f * (y * z + w * x); R[2][2] = 1.f - 2.f * (x * x + y * y);
}

// SGLD step on the means (spike/mcmc.py:25-34): p[0..3) += (R(q) diag(exp(ls)) eps) * w,
// w = sigmoid(100 ((1 - o) - 0.995)) * noise_scale (noise_scale = noise_lr * means lr),
// eps the gaussian's three Philox normals for (g, step).
__device__ __forceinline__ void sgld_apply(float* p, int g, uint32_t step, uint32_t seed,
                                           float noise_scale) {
  float R[3][3], z[3];
  quat_rot(p + 3, R);
  normals3(philox4x32_10((uint32_t)g, step, kTagSgld, 0u, seed, 0u), z);
  const float o = sigmoidf_(p[13]);
  const float w = sigmoidf_(100.0f * ((1.0f - o) - 0.995f)) * noise_scale;
  float se[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) se[j] = expf(p[7 + j]) * z[j];
#pragma unroll
  for (int i = 0; i < 3; ++i) p[i] += (R[i][0] * se[0] + R[i][1] * se[1] + R[i][2] * se[2]) * w;
}

// Gradient of reg_loss = lambda_o mean(sigmoid(op)) + lambda_s mean(exp(log_scales))
// (spike/mcmc.py:18-22) added to a [14] gradient row; reg_o = lambda_o / G,
// reg_s = lambda_s / (3 G) (tools/resident_traced.py:732-738).
__device__ __forceinline__ void reg_add(const float* p, float reg_o, float reg_s, float* gout) {
  const float o = sigmoidf_(p[13]);
  gout[13] += reg_o * (o * (1.0f - o));
#pragma unroll
  for (int j = 0; j < 3; ++j) gout[7 + j] += reg_s * expf(p[7 + j]);
}

// gcolor (optional): dL/dcolour through the clamp gate, the factor of every colour coefficient's
// gradient (the DC one is gcolor * C0, the SH rest ones gcolor * b_l).  gdw (optional, with a
// depth weight): this gaussian's dL/d(beta, tau); dw_zgrad adds dL/dz_cam through rho to the
// mean gradient.
__device__ __forceinline__ void geo_backward(const float* __restrict__ p, const Camera& cam,
                                             const GeoState& s, const float* gin, float* gout,
                                             float* gcolor = nullptr, float* gdw = nullptr,
                                             bool dw_zgrad = false) {
  // activations: color_o = keo * color, o_col = keo, keo = keep * sigmoid(op) * rho
  const float keo = s.keep ? s.o * s.rho : 0.0f;
  const float gkeo = gin[5] * s.color[0] + gin[6] * s.color[1] + gin[7] * s.color[2] + gin[8];
  // depth weight: g = dL/drho * drho/dpre, pre = beta (tau - z_cam)
  const float gpre = (s.dw && s.keep) ? gkeo * s.o * s.rho * (1.0f - s.rho) : 0.0f;
  if (gdw) {
    gdw[0] = gpre * (s.dw_tau - s.mc[2]);
    gdw[1] = gpre * s.dw_beta;
  }
  // conic = (s11, -s01, s00) / det
  const float di = s.det_inv;
  float gs11 = gin[0] * di, gs01 = -gin[1] * di, gs00 = gin[2] * di;
  const float gdi = gin[0] * s.s11 - gin[1] * s.s01 + gin[2] * s.s00;
  const float gdet = s.dmask ? -gdi * di * di : 0.0f;
  gs00 += gdet * s.s11;
  gs11 += gdet * s.s00;
  gs01 += -2.0f * gdet * s.s01;
  const float h = 0.5f * gs01;
  // Sigma2d = J SC J^T with J rows J0 = (J00, 0, J02), J1 = (0, J11, J12):
  //   dL/dJ = 2 Gs J SC, Gs = [[gs00, h], [h, gs11]];  dL/dSC (symmetrised) = 2 E, E = J^T Gs J.
  float JSC0[3], JSC1[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    JSC0[k] = s.J00 * s.SC[0][k] + s.J02 * s.SC[2][k];
    JSC1[k] = s.J11 * s.SC[1][k] + s.J12 * s.SC[2][k];
  }
  const float gJ00 = 2.f * (gs00 * JSC0[0] + h * JSC1[0]);
  const float gJ02 = 2.f * (gs00 * JSC0[2] + h * JSC1[2]);
  const float gJ11 = 2.f * (h * JSC0[1] + gs11 * JSC1[1]);
  const float gJ12 = 2.f * (h * JSC0[2] + gs11 * JSC1[2]);
  float E[3][3];
  E[0][0] = gs00 * s.J00 * s.J00;
  E[0][1] = h * s.J00 * s.J11;
  E[0][2] = gs00 * s.J00 * s.J02 + h * s.J00 * s.J12;
  E[1][1] = gs11 * s.J11 * s.J11;
  E[1][2] = gs11 * s.J11 * s.J12 + h * s.J11 * s.J02;
  E[2][2] = gs00 * s.J02 * s.J02 + gs11 * s.J12 * s.J12 + 2.f * h * s.J02 * s.J12;
  E[1][0] = E[0][1]; E[2][0] = E[0][2]; E[2][1] = E[1][2];
  // SC = M diag(s2) M^T:  dL/dM = 2 E M diag(s2);  dL/ds2_m = (M^T E M)_mm
  float EM[3][3];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int m = 0; m < 3; ++m) EM[a][m] = E[a][0] * s.M[0][m] + E[a][1] * s.M[1][m] + E[a][2] * s.M[2][m];
  float gM[3][3], gs2[3];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    gs2[m] = s.M[0][m] * EM[0][m] + s.M[1][m] * EM[1][m] + s.M[2][m] * EM[2][m];
#pragma unroll
    for (int a = 0; a < 3; ++a) gM[a][m] = 2.f * EM[a][m] * s.s2[m];
  }
  // M = R_v R  ->  dL/dR = R_v^T gM
  float gR[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int k = 0; k < 3; ++k)
      gR[i][k] = cam.R[0 * 3 + i] * gM[0][k] + cam.R[1 * 3 + i] * gM[1][k] + cam.R[2 * 3 + i] * gM[2][k];
  // mean path: mu2d = f * mc_xy / z + c ;  J entries depend on z and mc_xy.
  const float fx = cam.fx, fy = cam.fy, z = s.z;
  const float zi = 1.0f / z, zi2 = zi * zi, zi3 = zi2 * zi;
  const float gmx2 = gin[3], gmy2 = gin[4];
  const float gmcx = gmx2 * fx * zi - gJ02 * fx * zi2;
  const float gmcy = gmy2 * fy * zi - gJ12 * fy * zi2;
  float gz = -gJ00 * fx * zi2 - gJ11 * fy * zi2 + 2.f * gJ02 * fx * s.mc[0] * zi3 +
             2.f * gJ12 * fy * s.mc[1] * zi3 - gmx2 * fx * s.mc[0] * zi2 - gmy2 * fy * s.mc[1] * zi2;
  const float gmcz = (s.zmask ? gz : 0.0f) - (dw_zgrad ? gpre * s.dw_beta : 0.0f);
#pragma unroll
  for (int j = 0; j < 3; ++j) gout[j] = cam.R[0 * 3 + j] * gmcx + cam.R[1 * 3 + j] * gmcy + cam.R[2 * 3 + j] * gmcz;
  // rotation from the normalised quaternion
  const float w = s.qn[0], x = s.qn[1], y = s.qn[2], zq = s.qn[3];
  const float gw = 2.f * (-zq * gR[0][1] + y * gR[0][2] + zq * gR[1][0] - x * gR[1][2] - y * gR[2][0] + x * gR[2][1]);
  const float gx = 2.f * (y * gR[0][1] + zq * gR[0][2] + y * gR[1][0] - 2.f * x * gR[1][1] - w * gR[1][2] +
                          zq * gR[2][0] + w * gR[2][1] - 2.f * x * gR[2][2]);
  const float gy = 2.f * (-2.f * y * gR[0][0] + x * gR[0][1] + w * gR[0][2] + x * gR[1][0] + zq * gR[1][2] -
                          w * gR[2][0] + zq * gR[2][1] - 2.f * y * gR[2][2]);
  const float gzq = 2.f * (-2.f * zq * gR[0][0] - w * gR[0][1] + x * gR[0][2] + w * gR[1][0] -
                           2.f * zq * gR[1][1] + y * gR[1][2] + x * gR[2][0] + y * gR[2][1]);
  // q_n = q / max(|q|, 1e-12)
  const float inv = 1.0f / s.qdiv;
  const float dot = (s.qnorm >= 1e-12f) ? (w * gw + x * gx + y * gy + zq * gzq) : 0.0f;
  gout[3] = (gw - w * dot) * inv;
  gout[4] = (gx - x * dot) * inv;
  gout[5] = (gy - y * dot) * inv;
  gout[6] = (gzq - zq * dot) * inv;
  // s2 = exp(2 log_scale)
#pragma unroll
  for (int m = 0; m < 3; ++m) gout[7 + m] = gs2[m] * 2.f * s.s2[m];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float gc = s.craw[c] >= 0.0f ? gin[5 + c] * keo : 0.0f;
    gout[10 + c] = gc * kC0;
    if (gcolor) gcolor[c] = gc;
  }
  gout[13] = s.keep ? gkeo * s.o * (1.0f - s.o) * s.rho : 0.0f;
}

__device__ __forceinline__ Camera load_camera(const float* __restrict__ cam) {
  Camera c;
#pragma unroll
  for (int i = 0; i < 9; ++i) c.R[i] = cam[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) c.t[i] = cam[9 + i];
  c.fx = cam[12]; c.fy = cam[13]; c.cx = cam[14]; c.cy = cam[15];
  return c;
}

// Per-gaussian rows ([G,14] params and moments, [G,12] proj, [G,9] inv) are moved between HBM
// and the threads through LDS: a block copies its 256 contiguous rows with coalesced accesses
// (each wave instruction covers 1 KB of consecutive bytes) and each thread then reads its own
// row from LDS.  Direct row-per-thread accesses would make every wave instruction touch ~28
// cache lines 56 bytes apart, which the L1 address path, not HBM, turns into the limit.  LDS
// rows are padded to an odd stride, so the per-thread row reads are free of bank conflicts.
// The copy has a fixed trip count (W words per thread; the ragged last block clamps its loads
// and masks its writes), so all of a thread's loads are in flight before the first LDS write:
// a loop bounded by rows * W would wait out one memory round trip per word.
constexpr int kGeoBlock = 256;
constexpr int kSeamRow = 3 * 15 + 9;  // floats of one staged row of the step seam (params, m, v, inv)
// tid: the thread's index among the kGeoBlock threads that copy these rows (threadIdx.x, or
// its index in its half of a 512-thread block).
template <int W, typename T>
__device__ __forceinline__ void stage_load(const T* __restrict__ src, int g0, int rows, T (&r)[W],
                                           int tid = threadIdx.x) {
  const T* base = src + (int64_t)g0 * W;
  const int last = rows * W - 1;
#pragma unroll
  for (int k = 0; k < W; ++k) r[k] = base[min(tid + k * kGeoBlock, last)];
}
template <int W, int SW, typename T>
__device__ __forceinline__ void stage_put(const T (&r)[W], int rows, T* s, int tid = threadIdx.x) {
  const int n = rows * W;
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int i = tid + k * kGeoBlock;
    if (i < n) s[(i / W) * SW + i % W] = r[k];
  }
}
template <int W, int SW, typename T>
__device__ __forceinline__ void stage_in(const T* __restrict__ src, int g0, int rows, T* s) {
  T r[W];
  stage_load<W>(src, g0, rows, r);
  stage_put<W, SW>(r, rows, s);
}
template <int W, int SW, typename T>
__device__ __forceinline__ void stage_out(T* __restrict__ dst, int g0, int rows, const T* s,
                                          int tid = threadIdx.x) {
  T* base = dst + (int64_t)g0 * W;
  const int n = rows * W;
  T r[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int i = min(tid + k * kGeoBlock, n - 1);
    r[k] = s[(i / W) * SW + i % W];
  }
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int i = tid + k * kGeoBlock;
    if (i < n) base[i] = r[k];
  }
}

// Slot gradient sum through inverse-table entries e[9] already loaded (see gather_slot_grads):
// each 36-byte record is read as two 16-byte and one 4-byte load.  Split in two so a caller can
// put independent work between the loads (slot_loads) and their first use (slot_sum).
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));
struct SlotRecs {
  f4u a[9], b[9];
  float c[9];
};
__device__ __forceinline__ void slot_loads(const float* __restrict__ gslot, const int* e,
                                           SlotRecs& r) {
#pragma unroll
  for (int j = 0; j < 9; ++j) {
    r.a[j] = f4u{0.f, 0.f, 0.f, 0.f};
    r.b[j] = r.a[j];
    r.c[j] = 0.f;
    if (e[j] >= 0) {  // lanes without this entry issue no address
      const float* src = gslot + (int64_t)e[j] * 9;
      r.a[j] = *reinterpret_cast<const f4u*>(src);
      r.b[j] = *reinterpret_cast<const f4u*>(src + 4);
      r.c[j] = src[8];
    }
  }
}
__device__ __forceinline__ void slot_sum(const int* e, const SlotRecs& r, float* gin) {
#pragma unroll
  for (int k = 0; k < 9; ++k) gin[k] = 0.0f;
#pragma unroll
  for (int j = 0; j < 9; ++j) {
    if (e[j] >= 0) {
      gin[0] += r.a[j].x; gin[1] += r.a[j].y; gin[2] += r.a[j].z; gin[3] += r.a[j].w;
      gin[4] += r.b[j].x; gin[5] += r.b[j].y; gin[6] += r.b[j].z; gin[7] += r.b[j].w;
      gin[8] += r.c[j];
    }
  }
}
__device__ __forceinline__ void gather_slots(const float* __restrict__ gslot, const int* e,
                                             float* gin) {
  SlotRecs r;
  slot_loads(gslot, e, r);
  slot_sum(e, r, gin);
}

// adv (optional): a training step's Adam step block, advanced by block 0 after its rows (what a
// separate k_adam_advance launch would do; nothing between this kernel and the Adam update
// reads the block).
// SH = true: view-dependent colour from the first n = sh_rest_count(deg) rest coefficients.
// One gaussian's projection from its staged parameter row: the [12] proj record into orow,
// keep[g], and the mean and keep flag handed back for the count pass.
template <bool SH>
__device__ __forceinline__ void geo_fwd_row(const float* srow, int g, int G,
                                            const float* __restrict__ rest, int n_rest,
                                            const float* __restrict__ dw, const Camera& cam,
                                            float near_z, float blur, float* orow,
                                            uint8_t* __restrict__ keep, float* mux, float* muy,
                                            uint8_t* kept) {
  float p[14];
#pragma unroll
  for (int i = 0; i < 14; ++i) p[i] = srow[i];
  float rv[SH ? 3 * kShRest : 1];
  if (SH) sh_load(rest, G, g, n_rest, rv);
  GeoState s;
  geo_forward(p, cam, near_z, blur, s, dw);
  if (SH) {
    float b[16];
    sh_basis(p, cam, b);
    sh_apply(p, b, rv, n_rest, s);
  }
  const float keo = s.keep ? s.o * s.rho : 0.0f;
  const float out[12] = {s.mux, s.muy, s.a, s.b, s.c, s.mc[2], keo * s.color[0],
                         keo * s.color[1], keo * s.color[2], keo, s.o, 0.0f};
#pragma unroll
  for (int i = 0; i < 12; ++i) orow[i] = out[i];
  keep[g] = s.keep ? 1 : 0;
  *mux = s.mux;
  *muy = s.muy;
  *kept = s.keep ? 1 : 0;
}

template <bool SH>
__global__ __launch_bounds__(256) void k_geom_fwd(const float* __restrict__ params, int G,
                                                  const float* __restrict__ rest, int n_rest,
                                                  const float* __restrict__ dw,
                                                  const float* __restrict__ camera, float near_z,
                                                  float blur, float* __restrict__ proj,
                                                  uint8_t* __restrict__ keep, int32_t* adv,
                                                  float b1, float b2) {
  __shared__ float s_p[kGeoBlock * 15];
  __shared__ float s_o[kGeoBlock * 13];
  const int g0 = blockIdx.x * kGeoBlock, rows = min(kGeoBlock, G - g0);
  const int g = g0 + threadIdx.x;
  stage_in<14, 15>(params, g0, rows, s_p);
  __syncthreads();
  if ((int)threadIdx.x < rows) {
    const Camera cam = load_camera(camera);
    float mux, muy;
    uint8_t kept;
    geo_fwd_row<SH>(s_p + threadIdx.x * 15, g, G, rest, n_rest, dw, cam, near_z, blur,
                    s_o + threadIdx.x * 13, keep, &mux, &muy, &kept);
  }
  __syncthreads();
  stage_out<12, 13>(proj, g0, rows, s_o);
  if (adv && blockIdx.x == 0 && threadIdx.x == 0) advance_step(adv, b1, b2);
}

// The geometry forward of 512 gaussians, one per thread (two 256-row halves staged by the two
// halves of the block), followed by binning's count pass over the same gaussians as a block of
// 8 waves x 64 (count blocks of 512 gaussians, as CountSmall: the same count-matrix rows): the
// means and keep flags reach the count pass through LDS instead of a second kernel reading proj
// back.  proj/keep equal k_geom_fwd's; mat rows and cell_slot are k_bin_count's (in-cell ranks
// of regular gaussians in LDS-atomic order, as there).
using CountFused = CountGeo<512, 1>;
template <bool SH>
__global__ __launch_bounds__(512) void k_geom_fwd_count(
    const float* __restrict__ params, int G, const float* __restrict__ rest, int n_rest,
    const float* __restrict__ dw, const float* __restrict__ camera, float near_z, float blur,
    float* __restrict__ proj, uint8_t* __restrict__ keep, int32_t* adv, float b1, float b2,
    int ntx, int nty, float S, int span, int NB, int Tpad, int* __restrict__ mat,
    int2* __restrict__ cell_slot) {
  static_assert(CountFused::kBlock == CountSmall::kBlock && CountFused::kBlock == 2 * kGeoBlock,
                "one count block = two geometry halves");
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  float2* s_mu = reinterpret_cast<float2*>(s_dyn);                   // [512] means
  uint8_t* s_kv = reinterpret_cast<uint8_t*>(s_mu + 2 * kGeoBlock);  // [512] keep flags
  float* s_u = reinterpret_cast<float*>(s_kv + 2 * kGeoBlock);       // staging, then count
  const int half = threadIdx.x / kGeoBlock, lt = threadIdx.x % kGeoBlock;
  float* s_p = s_u + half * kGeoBlock * 15;                          // this half's [256][15]
  float* s_o = s_u + 2 * kGeoBlock * 15 + half * kGeoBlock * 13;     // this half's [256][13]
  const int g0 = blockIdx.x * 2 * kGeoBlock + half * kGeoBlock;
  const int rows = min(kGeoBlock, G - g0);  // <= 0: the block's second half lies past G
  if (rows > 0) {  // stage_in with this half's thread index
    const float* base = params + (int64_t)g0 * 14;
    const int last = rows * 14 - 1;
    float r[14];
#pragma unroll
    for (int k = 0; k < 14; ++k) r[k] = base[min(lt + k * kGeoBlock, last)];
#pragma unroll
    for (int k = 0; k < 14; ++k) {
      const int i = lt + k * kGeoBlock;
      if (i <= last) s_p[(i / 14) * 15 + i % 14] = r[k];
    }
  }
  __syncthreads();
  float mux = 0.f, muy = 0.f;
  uint8_t kept = 0;
  if (lt < rows) {
    const Camera cam = load_camera(camera);
    geo_fwd_row<SH>(s_p + lt * 15, g0 + lt, G, rest, n_rest, dw, cam, near_z, blur,
                    s_o + lt * 13, keep, &mux, &muy, &kept);
  }
  s_mu[threadIdx.x] = make_float2(mux, muy);
  s_kv[threadIdx.x] = kept;
  __syncthreads();
  if (rows > 0) {  // stage_out with this half's thread index
    float* base = proj + (int64_t)g0 * 12;
    const int n = rows * 12;
    float r[12];
#pragma unroll
    for (int k = 0; k < 12; ++k) {
      const int i = min(lt + k * kGeoBlock, n - 1);
      r[k] = s_o[(i / 12) * 13 + i % 12];
    }
#pragma unroll
    for (int k = 0; k < 12; ++k) {
      const int i = lt + k * kGeoBlock;
      if (i < n) base[i] = r[k];
    }
  }
  if (adv && blockIdx.x == 0 && threadIdx.x == 0) advance_step(adv, b1, b2);
  __syncthreads();  // every staging read is done: the count pass reuses that LDS
  // count layout: wave w owns [64 w, 64 w + 64) -- the thread's own gaussian
  const float mx[1] = {mux}, my[1] = {muy};
  const uint8_t kv[1] = {kept};
  count_body<512, 1>(mx, my, kv, G, ntx, nty, S, span, NB, Tpad, reinterpret_cast<int*>(s_u),
                     mat, cell_slot);
}

// The same for the large count blocks (CountLarge: 1024 threads, 4096 gaussians; G above the
// small blocks' 131072): wave w takes its four rounds of 64 gaussians one after another, each
// through a wave-private LDS staging area (rows in, then the projection rows out in place), and
// keeps its means and keep flags in registers for the count pass, which then reuses the LDS.
// Replaces k_geom_fwd followed by k_bin_count<1024, 4> (one launch and one strided read of
// proj's means fewer).
using CountBig = CountLarge;
template <bool SH>
__global__ __launch_bounds__(1024) void k_geom_fwd_count_large(
    const float* __restrict__ params, int G, const float* __restrict__ rest, int n_rest,
    const float* __restrict__ dw, const float* __restrict__ camera, float near_z, float blur,
    float* __restrict__ proj, uint8_t* __restrict__ keep, int32_t* adv, float b1, float b2,
    int ntx, int nty, float S, int span, int NB, int Tpad, int* __restrict__ mat,
    int2* __restrict__ cell_slot) {
  constexpr int PER = CountBig::kWaveSpan / 64;
  static_assert(CountBig::kWaves * 64 == 1024, "one wave per 64 threads");
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* s_w = s_dyn + wave * 64 * 15;   // this wave's [64][15] rows (then [64][12] out)
  const int gw = blockIdx.x * CountBig::kBlock + wave * CountBig::kWaveSpan;
  const Camera cam = load_camera(camera);
  float mx[PER], my[PER];
  uint8_t kv[PER];
  // a round's rows (64 x 14 contiguous floats, lane-strided); without SH (whose rest
  // coefficients leave no registers for it) round i + 1's are requested before round i is
  // projected, so they arrive during it
  float nr[14];
  auto load_round = [&](int i) {
    const int g0 = gw + 64 * i;
    const int rows = min(64, G - g0);
    if (rows <= 0) return;  // wave-uniform
    const float* base = params + (int64_t)g0 * 14;
    const int last = rows * 14 - 1;
#pragma unroll
    for (int k = 0; k < 14; ++k) nr[k] = base[min(lane + 64 * k, last)];
  };
  if constexpr (!SH) load_round(0);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int g0 = gw + 64 * i;
    const int rows = min(64, G - g0);
    mx[i] = my[i] = 0.f;
    kv[i] = 0;
    if (rows <= 0) continue;  // wave-uniform (and so are the later rounds)
    {
      if constexpr (SH) load_round(i);
      float r[14];
#pragma unroll
      for (int k = 0; k < 14; ++k) r[k] = nr[k];
      if (!SH && i + 1 < PER) load_round(i + 1);
      const int last = rows * 14 - 1;
#pragma unroll
      for (int k = 0; k < 14; ++k) {
        const int e = lane + 64 * k;
        if (e <= last) s_w[(e / 14) * 15 + e % 14] = r[k];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float orow[12];
    if (lane < rows)
      geo_fwd_row<SH>(s_w + lane * 15, g0 + lane, G, rest, n_rest, dw, cam, near_z, blur, orow,
                      keep, &mx[i], &my[i], &kv[i]);
    // every lane has read its row: the rows' space takes the projection rows ([64][12])
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < rows) {
#pragma unroll
      for (int k = 0; k < 12; ++k) s_w[lane * 12 + k] = orow[k];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {  // the projection rows out: 64 x 12 contiguous floats
      float* base = proj + (int64_t)g0 * 12;
      const int n = rows * 12;
#pragma unroll
      for (int k = 0; k < 12; ++k) {
        const int e = lane + 64 * k;
        if (e < n) base[e] = s_w[e];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  if (adv && blockIdx.x == 0 && threadIdx.x == 0) advance_step(adv, b1, b2);
  __syncthreads();  // every staging access is done: the count pass reuses that LDS
  count_body<1024, PER>(mx, my, kv, G, ntx, nty, S, span, NB, Tpad,
                        reinterpret_cast<int*>(s_dyn), mat, cell_slot);
}

// gsh (SH only): dL/drest in the rest layout; rows l >= n_rest are written as zero.
template <bool SH>
__global__ __launch_bounds__(256) void k_geom_bwd(const float* __restrict__ params, int G,
                                                  const float* __restrict__ rest, int n_rest,
                                                  DepthW dwa, const float* __restrict__ camera,
                                                  float near_z, float blur,
                                                  const float* __restrict__ grad9,
                                                  float* __restrict__ gparams,
                                                  float* __restrict__ gsh) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  const Camera cam = load_camera(camera);
  const float* p = params + (int64_t)g * 14;
  float rv[SH ? 3 * kShRest : 1];
  if (SH) sh_load(rest, G, g, n_rest, rv);
  GeoState s;
  geo_forward(p, cam, near_z, blur, s, dwa.bt);
  float b[16];
  if (SH) {
    sh_basis(p, cam, b);
    sh_apply(p, b, rv, n_rest, s);
  }
  float gin[9], gout[14], gcol[3], gdw[2];
#pragma unroll
  for (int i = 0; i < 9; ++i) gin[i] = grad9[(int64_t)g * 9 + i];
  geo_backward(p, cam, s, gin, gout, gcol, gdw, (dwa.zgrad & TTS_GRAD_DEPTH_Z) != 0);
  if (SH && (dwa.zgrad & TTS_GRAD_SH_DIR)) sh_dir_grad(p, cam, rv, n_rest, gcol, gout);
#pragma unroll
  for (int i = 0; i < 14; ++i) gparams[(int64_t)g * 14 + i] = gout[i];
  depthw_store(dwa, g, gdw);
  if (SH) {
#pragma unroll
    for (int l = 0; l < kShRest; ++l)
#pragma unroll
      for (int c = 0; c < 3; ++c)
        gsh[(int64_t)(l * 3 + c) * G + g] = l < n_rest ? b[l + 1] * gcol[c] : 0.0f;
  }
}

__global__ void k_adam_advance(int32_t* step, float b1, float b2) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  advance_step(step, b1, b2);
}

// torch.optim.Adam's update, p -= lr/bc1 * m / (sqrt(v)/sqrt(bc2) + eps), with the division
// as a hardware reciprocal (1 ulp; an IEEE division is ~10 VALU instructions, 14 per gaussian)
__device__ __forceinline__ void adam_update(float& p, float& m, float& v, float g, float lr,
                                            float inv_bc1, float inv_sqrt_bc2, float b1, float b2,
                                            float eps) {
  m = b1 * m + (1.0f - b1) * g;
  v = b2 * v + (1.0f - b2) * g * g;
  p -= (lr * inv_bc1) * m * __builtin_amdgcn_rcpf(sqrtf(v) * inv_sqrt_bc2 + eps);
}

__global__ __launch_bounds__(256) void k_adam(float* __restrict__ params, float* __restrict__ m,
                                              float* __restrict__ v, const float* __restrict__ grad,
                                              const float* __restrict__ lr, int64_t n,
                                              const int32_t* __restrict__ step, float b1, float b2,
                                              float eps) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float* f = reinterpret_cast<const float*>(step);
  const float inv_bc1 = f[1], inv_sqrt_bc2 = f[2];
  float pp = params[i], mm = m[i], vv = v[i];
  adam_update(pp, mm, vv, grad[i], lr[i % 14], inv_bc1, inv_sqrt_bc2, b1, b2, eps);
  params[i] = pp;
  m[i] = mm;
  v[i] = vv;
}

// Sum of one gaussian's slot gradients, gathered through the inverse bin table inv[g][0..9)
// (tile*K + slot, or -1) in stencil order: the slot->gaussian reduce of
// tools/m9_scatter_oracle.py:35-42 / tools/resident_traced.py:383-395, without atomics and in a
// fixed order (so the result is reproducible bit for bit).
// Per-gaussian sum of its slot gradients, in stencil order j (a fixed order: deterministic).
// Every load is issued before any is used (missing slots read row 0 and are masked), so the
// gather costs one dependent round trip after the inverse-table load.
__device__ __forceinline__ void gather_slot_grads(const float* __restrict__ gslot,
                                                  const int32_t* __restrict__ inv, int g,
                                                  float* gin) {
  int e[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) e[j] = inv[(int64_t)g * 9 + j];
  float v[9][9];
#pragma unroll
  for (int j = 0; j < 9; ++j) {
    const float* src = gslot + (int64_t)(e[j] >= 0 ? e[j] : 0) * 9;
#pragma unroll
    for (int c = 0; c < 9; ++c) v[j][c] = src[c];
  }
#pragma unroll
  for (int c = 0; c < 9; ++c) gin[c] = 0.0f;
#pragma unroll
  for (int j = 0; j < 9; ++j)
#pragma unroll
    for (int c = 0; c < 9; ++c) gin[c] += e[j] >= 0 ? v[j][c] : 0.0f;
}

__global__ __launch_bounds__(256) void k_slot_reduce(const float* __restrict__ gslot,
                                                     const int32_t* __restrict__ inv, int G,
                                                     float* __restrict__ grad9) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  float gin[9];
  gather_slot_grads(gslot, inv, g, gin);
#pragma unroll
  for (int c = 0; c < 9; ++c) grad9[(int64_t)g * 9 + c] = gin[c];
}

// Slot->gaussian reduce for bins that come without an inverse table (e.g. handed in by a
// caller): float atomics, order-dependent rounding.  grad9 must be zeroed first.
__global__ __launch_bounds__(256) void k_slot_scatter(const float* __restrict__ gslot,
                                                      const int32_t* __restrict__ idx,
                                                      const uint8_t* __restrict__ valid,
                                                      int64_t TK, float* __restrict__ grad9) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= TK || !valid[i]) return;
  float* dst = grad9 + (int64_t)idx[i] * 9;
#pragma unroll
  for (int c = 0; c < 9; ++c) unsafeAtomicAdd(dst + c, gslot[i * 9 + c]);
}

// SH: the rest coefficients (and their moments sh_m, sh_v, same layout) take the same Adam step
// with the scalar learning rate lr_sh[0]; rows l >= n_rest are not touched.
// MC: the MCMC regulariser gradient is added before Adam (reg_o, reg_s) and, when
// noise_lr > 0, the SGLD step is applied to the updated means (noise scale noise_lr * lr[0]).
struct McmcArgs {
  float reg_o, reg_s, noise_lr;
  uint32_t seed;
};
// One row of the geometry backward + Adam: row t of a block's staged rows (s_p, s_m, s_v at
// stride 15, s_inv at stride 9), gaussian g.  The slot gradients are gathered through the
// row's inverse-table entries, the forward recomputed, the chain rule applied (plus the MCMC
// regulariser), and the new parameters and moments written back over the row.
template <bool SH, bool MC>
__device__ __forceinline__ void bwd_adam_row(
    int t, int g, int G, float* s_p, float* s_m, float* s_v, const int* s_inv,
    float* __restrict__ rest, float* __restrict__ sh_m, float* __restrict__ sh_v, int n_rest,
    const float* __restrict__ camera, float near_z, float blur, const float* __restrict__ gslot,
    float* __restrict__ gparams, const float* __restrict__ lr, const float* __restrict__ lr_sh,
    const int32_t* __restrict__ step, float b1, float b2, float eps, const McmcArgs& mc,
    const DepthW& dwa) {
  int e[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) e[j] = s_inv[t * 9 + j];
  float gin[9], gout[14], gcol[3];
  SlotRecs recs;
  slot_loads(gslot, e, recs);  // in flight during the forward recompute below
  float pl[14], mm[14], vv[14];
#pragma unroll
  for (int i = 0; i < 14; ++i) {
    pl[i] = s_p[t * 15 + i];
    mm[i] = s_m[t * 15 + i];
    vv[i] = s_v[t * 15 + i];
  }
  float rv[SH ? 3 * kShRest : 1];
  if (SH) sh_load(rest, G, g, n_rest, rv);
  const Camera cam = load_camera(camera);
  GeoState s;
  geo_forward(pl, cam, near_z, blur, s, dwa.bt);
  float b[16];
  if (SH) {
    sh_basis(pl, cam, b);
    sh_apply(pl, b, rv, n_rest, s);
  }
  float gdw[2];
  slot_sum(e, recs, gin);
  geo_backward(pl, cam, s, gin, gout, gcol, gdw, dwa.zgrad != 0);
  depthw_store(dwa, g, gdw);
  if (MC) reg_add(pl, mc.reg_o, mc.reg_s, gout);
  const float* f = reinterpret_cast<const float*>(step);
  const float inv_bc1 = f[1], inv_sqrt_bc2 = f[2];
  float pn[14];
#pragma unroll
  for (int i = 0; i < 14; ++i) {
    pn[i] = pl[i];
    adam_update(pn[i], mm[i], vv[i], gout[i], lr[i], inv_bc1, inv_sqrt_bc2, b1, b2, eps);
  }
  if (MC && mc.noise_lr > 0.0f)
    sgld_apply(pn, g, (uint32_t)step[0], mc.seed, mc.noise_lr * lr[0]);
#pragma unroll
  for (int i = 0; i < 14; ++i) {
    s_p[t * 15 + i] = pn[i];
    s_m[t * 15 + i] = mm[i];
    s_v[t * 15 + i] = vv[i];
    if (gparams) gparams[(int64_t)g * 14 + i] = gout[i];
  }
  if (SH) {
    const float lrs = lr_sh[0];
#pragma unroll
    for (int l = 0; l < kShRest; ++l) {
      if (l < n_rest) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const int64_t o = (int64_t)(l * 3 + c) * G + g;
          float pr = rv[l * 3 + c], mr = sh_m[o], vr = sh_v[o];
          adam_update(pr, mr, vr, b[l + 1] * gcol[c], lrs, inv_bc1, inv_sqrt_bc2, b1, b2, eps);
          rest[o] = pr;
          sh_m[o] = mr;
          sh_v[o] = vr;
        }
      }
    }
  }
}

template <bool SH, bool MC>
__global__ __launch_bounds__(256) void k_geom_bwd_adam(
    float* __restrict__ params, int G, float* __restrict__ rest, float* __restrict__ sh_m,
    float* __restrict__ sh_v, int n_rest, const float* __restrict__ camera, float near_z,
    float blur, const float* __restrict__ gslot, const int32_t* __restrict__ inv,
    float* __restrict__ gparams, float* __restrict__ m, float* __restrict__ v,
    const float* __restrict__ lr, const float* __restrict__ lr_sh,
    const int32_t* __restrict__ step, float b1, float b2, float eps, McmcArgs mc, DepthW dwa) {
  __shared__ float s_p[kGeoBlock * 15], s_m[kGeoBlock * 15], s_v[kGeoBlock * 15];
  __shared__ int s_inv[kGeoBlock * 9];
  const int g0 = blockIdx.x * kGeoBlock, rows = min(kGeoBlock, G - g0);
  const int g = g0 + threadIdx.x;
  {  // all four row copies in flight at once
    int ri[9];
    float rp[14], rm[14], rv[14];
    stage_load<9>(inv, g0, rows, ri);
    stage_load<14>(params, g0, rows, rp);
    stage_load<14>(m, g0, rows, rm);
    stage_load<14>(v, g0, rows, rv);
    stage_put<9, 9>(ri, rows, s_inv);
    stage_put<14, 15>(rp, rows, s_p);
    stage_put<14, 15>(rm, rows, s_m);
    stage_put<14, 15>(rv, rows, s_v);
  }
  __syncthreads();
  if ((int)threadIdx.x < rows)
    bwd_adam_row<SH, MC>(threadIdx.x, g, G, s_p, s_m, s_v, s_inv, rest, sh_m, sh_v, n_rest, camera,
                         near_z, blur, gslot, gparams, lr, lr_sh, step, b1, b2, eps, mc, dwa);
  __syncthreads();
  stage_out<14, 15>(params, g0, rows, s_p);
  stage_out<14, 15>(m, g0, rows, s_m);
  stage_out<14, 15>(v, g0, rows, s_v);
}

// The seam between two training steps in one launch: step i's geometry backward + Adam
// (camera cam_b, its slot gradients) and step i+1's geometry forward (camera cam_f) with the
// binning's count pass.  A gaussian's forward needs nothing of step i but its own new
// parameters, and a count block's rows are its own 512 gaussians, so no block waits on another:
// each 512-thread block runs k_geom_bwd_adam's row body on its two 256-row halves, writes the
// rows back, then projects the new rows it still holds in LDS and counts them, as
// k_geom_fwd_count does (the same proj, keep, count-matrix rows and cell slots).  What this
// saves against the two launches: one kernel boundary and the parameter reload.  No SH, depth
// weight or MCMC terms (callers take the two launches for those), and no step advance: step
// i+1's advance rides on the next binning pass (tts_assign_bins_counted), after every block
// here has read step i's bias corrections.
__global__ __launch_bounds__(512) void k_geom_bwd_adam_fwd_count(
    float* __restrict__ params, int G, const float* __restrict__ cam_b,
    const float* __restrict__ cam_f, float near_z, float blur, const float* __restrict__ gslot,
    const int32_t* __restrict__ inv, float* __restrict__ gparams, float* __restrict__ m,
    float* __restrict__ v, const float* __restrict__ lr, const int32_t* __restrict__ step,
    float b1, float b2, float eps, float* __restrict__ proj, uint8_t* __restrict__ keep, int ntx,
    int nty, float S, int span, int NB, int Tpad, int* __restrict__ mat,
    int2* __restrict__ cell_slot) {
  static_assert(CountFused::kBlock == 2 * kGeoBlock, "one count block = two row halves");
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  const int half = threadIdx.x / kGeoBlock, lt = threadIdx.x % kGeoBlock;
  float* s_p = s_dyn + half * kGeoBlock * kSeamRow;   // this half's rows: params, m, v, inv
  float* s_m = s_p + kGeoBlock * 15;
  float* s_v = s_m + kGeoBlock * 15;
  int* s_inv = reinterpret_cast<int*>(s_v + kGeoBlock * 15);
  const int g0 = blockIdx.x * 2 * kGeoBlock + half * kGeoBlock;
  const int rows = min(kGeoBlock, G - g0);  // <= 0: the block's second half lies past G
  if (rows > 0) {  // all four row copies in flight at once
    int ri[9];
    float rp[14], rm[14], rv[14];
    stage_load<9>(inv, g0, rows, ri, lt);
    stage_load<14>(params, g0, rows, rp, lt);
    stage_load<14>(m, g0, rows, rm, lt);
    stage_load<14>(v, g0, rows, rv, lt);
    stage_put<9, 9>(ri, rows, s_inv, lt);
    stage_put<14, 15>(rp, rows, s_p, lt);
    stage_put<14, 15>(rm, rows, s_m, lt);
    stage_put<14, 15>(rv, rows, s_v, lt);
  }
  __syncthreads();
  if (lt < rows)
    bwd_adam_row<false, false>(lt, g0 + lt, G, s_p, s_m, s_v, s_inv, nullptr, nullptr, nullptr, 0,
                               cam_b, near_z, blur, gslot, gparams, lr, nullptr, step, b1, b2,
                               eps, McmcArgs{0.0f, 0.0f, 0.0f, 0u},
                               DepthW{nullptr, nullptr, 1.0f, 0, 0});
  __syncthreads();
  if (rows > 0) {
    stage_out<14, 15>(params, g0, rows, s_p, lt);
    stage_out<14, 15>(m, g0, rows, s_m, lt);
    stage_out<14, 15>(v, g0, rows, s_v, lt);
  }
  __syncthreads();  // every read of s_m is done: its space takes the projection rows
  float* s_o = s_m;
  float mux = 0.f, muy = 0.f;
  uint8_t kept = 0;
  if (lt < rows) {
    const Camera cam = load_camera(cam_f);
    geo_fwd_row<false>(s_p + lt * 15, g0 + lt, G, nullptr, 0, nullptr, cam, near_z, blur,
                       s_o + lt * 13, keep, &mux, &muy, &kept);
  }
  __syncthreads();
  if (rows > 0) stage_out<12, 13>(proj, g0, rows, s_o, lt);
  __syncthreads();  // every staging read is done: the count pass reuses the LDS
  const float mx[1] = {mux}, my[1] = {muy};
  const uint8_t kv[1] = {kept};
  count_body<512, 1>(mx, my, kv, G, ntx, nty, S, span, NB, Tpad, reinterpret_cast<int*>(s_dyn),
                     mat, cell_slot);
}

// Batch form: gacc[g] += scale * dL/dparams[g] for one view (one writer per gaussian); with SH
// also gacc_sh += scale * dL/drest (rows l < n_rest).
template <bool SH>
__global__ __launch_bounds__(256) void k_geom_bwd_accum(
    const float* __restrict__ params, int G, const float* __restrict__ rest, int n_rest,
    DepthW dwa, const float* __restrict__ camera, float near_z, float blur,
    const float* __restrict__ gslot, const int32_t* __restrict__ inv, float scale,
    float* __restrict__ gacc, float* __restrict__ gacc_sh) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  const Camera cam = load_camera(camera);
  const float* p = params + (int64_t)g * 14;
  float pl[14];
#pragma unroll
  for (int i = 0; i < 14; ++i) pl[i] = p[i];
  float rv[SH ? 3 * kShRest : 1];
  if (SH) sh_load(rest, G, g, n_rest, rv);
  GeoState s;
  geo_forward(pl, cam, near_z, blur, s, dwa.bt);
  float b[16];
  if (SH) {
    sh_basis(pl, cam, b);
    sh_apply(pl, b, rv, n_rest, s);
  }
  float gin[9], gout[14], gcol[3], gdw[2];
  gather_slot_grads(gslot, inv, g, gin);
  geo_backward(pl, cam, s, gin, gout, gcol, gdw, dwa.zgrad != 0);
  depthw_store(dwa, g, gdw);
  float* a = gacc + (int64_t)g * 14;
#pragma unroll
  for (int i = 0; i < 14; ++i) a[i] += scale * gout[i];
  if (SH) {
#pragma unroll
    for (int l = 0; l < kShRest; ++l) {
      if (l < n_rest) {
#pragma unroll
        for (int c = 0; c < 3; ++c)
          gacc_sh[(int64_t)(l * 3 + c) * G + g] += scale * (b[l + 1] * gcol[c]);
      }
    }
  }
}

// Adam over a flat array with one learning rate lr1[0] (the SH rest block in batch mode).
__global__ __launch_bounds__(256) void k_adam_flat(float* __restrict__ params,
                                                   float* __restrict__ m, float* __restrict__ v,
                                                   const float* __restrict__ grad,
                                                   const float* __restrict__ lr1, int64_t n,
                                                   const int32_t* __restrict__ step, float b1,
                                                   float b2, float eps) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float* f = reinterpret_cast<const float*>(step);
  float pp = params[i], mm = m[i], vv = v[i];
  adam_update(pp, mm, vv, grad[i], lr1[0], f[1], f[2], b1, b2, eps);
  params[i] = pp;
  m[i] = mm;
  v[i] = vv;
}

// Batch-mode MCMC pieces: the regulariser gradient into a [G,14] gradient block, and the SGLD
// step on the means after the Adam update.
__global__ __launch_bounds__(256) void k_mcmc_reg_grad(const float* __restrict__ params, int G,
                                                       float reg_o, float reg_s,
                                                       float* __restrict__ grad) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  float p[14], gr[14];
#pragma unroll
  for (int i = 0; i < 14; ++i) {
    p[i] = params[(int64_t)g * 14 + i];
    gr[i] = 0.0f;
  }
  reg_add(p, reg_o, reg_s, gr);
  grad[(int64_t)g * 14 + 13] += gr[13];
#pragma unroll
  for (int j = 0; j < 3; ++j) grad[(int64_t)g * 14 + 7 + j] += gr[7 + j];
}

__global__ __launch_bounds__(256) void k_sgld(float* __restrict__ params, int G,
                                              const float* __restrict__ lr, float noise_lr,
                                              uint32_t seed, const int32_t* __restrict__ step) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  float p[14];
#pragma unroll
  for (int i = 0; i < 14; ++i) p[i] = params[(int64_t)g * 14 + i];
  sgld_apply(p, g, (uint32_t)step[0], seed, noise_lr * lr[0]);
#pragma unroll
  for (int i = 0; i < 3; ++i) params[(int64_t)g * 14 + i] = p[i];
}

// Depth weight: per-gaussian dL/d(beta, tau) [G,2] -> block partial sums (fixed order) -> one
// block sums the partials and applies Adam to the two device scalars (the reference sums on the
// host and runs a host Adam, tools/resident_traced.py:503-512).
constexpr int kDwPer = 8;  // gaussians per thread in the partial pass
__global__ __launch_bounds__(256) void k_dw_partial(const float* __restrict__ gdw, int G,
                                                    float* __restrict__ part) {
  __shared__ float tmp[4];
  const int64_t base = (int64_t)blockIdx.x * 256 * kDwPer;
  float sb = 0.0f, st = 0.0f;
#pragma unroll
  for (int k = 0; k < kDwPer; ++k) {
    const int64_t g = base + k * 256 + threadIdx.x;
    if (g < G) {
      sb += gdw[g * 2 + 0];
      st += gdw[g * 2 + 1];
    }
  }
  sb = block_sum256(sb, tmp);
  st = block_sum256(st, tmp);
  if (threadIdx.x == 0) {
    part[blockIdx.x * 2 + 0] = sb;
    part[blockIdx.x * 2 + 1] = st;
  }
}

// bt = (beta, tau); state = (m_beta, m_tau, v_beta, v_tau); lr1[0] the learning rate.
__global__ __launch_bounds__(256) void k_dw_adam(const float* __restrict__ part, int nb,
                                                 float* __restrict__ bt, float* __restrict__ state,
                                                 const float* __restrict__ lr1,
                                                 const int32_t* __restrict__ step, float b1,
                                                 float b2, float eps) {
  __shared__ float tmp[4];
  float sb = 0.0f, st = 0.0f;
  for (int i = threadIdx.x; i < nb; i += 256) {
    sb += part[i * 2 + 0];
    st += part[i * 2 + 1];
  }
  sb = block_sum256(sb, tmp);
  st = block_sum256(st, tmp);
  if (threadIdx.x == 0) {
    const float* f = reinterpret_cast<const float*>(step);
    const float g[2] = {sb, st};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float p = bt[k], m = state[k], v = state[2 + k];
      adam_update(p, m, v, g[k], lr1[0], f[1], f[2], b1, b2, eps);
      bt[k] = p;
      state[k] = m;
      state[2 + k] = v;
    }
  }
}

__global__ __launch_bounds__(256) void k_zero(float* __restrict__ buf, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) buf[i] = 0.0f;
}

// means + keep flags of 512 gaussians, then the row staging or the count histogram
size_t geom_fwd_count_lds(int NB, int Tpad) {
  const size_t stage = sizeof(float) * 2 * kGeoBlock * (15 + 13);
  const size_t cnt = sizeof(int) * ((size_t)Tpad + (size_t)CountFused::kWaves * NB);
  return (sizeof(float2) + 1) * 2 * kGeoBlock + (stage > cnt ? stage : cnt);
}

int launch_geom_fwd_count(const float* params, const float* sh_rest, int sh_degree,
                          const float* depth_bt, int G, const float* camera, float near_z,
                          float blur, float* proj, uint8_t* keep, int32_t* step_adv, float b1,
                          float b2, int ntx, int nty, float S, int span, int NB, int Tpad,
                          int* mat, int2* cell_slot, hipStream_t stream) {
  const int nblk = (G + CountFused::kBlock - 1) / CountFused::kBlock;
  const size_t lds = geom_fwd_count_lds(NB, Tpad);
  if (lds > kMaxLdsBytes) return TTS_EINVAL;  // callers check first and take the two-kernel path
  const bool sh = sh_degree > 0;
  static LdsLimit lim[2];
  if (lds > 65536) {
    const void* fn = sh ? reinterpret_cast<const void*>(&k_geom_fwd_count<true>)
                        : reinterpret_cast<const void*>(&k_geom_fwd_count<false>);
    const int e = raise_lds_limit(fn, lim[sh ? 1 : 0]);
    if (e) return e;
  }
  if (sh)
    k_geom_fwd_count<true><<<nblk, 512, lds, stream>>>(
        params, G, sh_rest, sh_rest_count(sh_degree), depth_bt, camera, near_z, blur, proj, keep,
        step_adv, b1, b2, ntx, nty, S, span, NB, Tpad, mat, cell_slot);
  else
    k_geom_fwd_count<false><<<nblk, 512, lds, stream>>>(
        params, G, nullptr, 0, depth_bt, camera, near_z, blur, proj, keep, step_adv, b1, b2, ntx,
        nty, S, span, NB, Tpad, mat, cell_slot);
  return launch_status();
}

size_t geom_fwd_count_large_lds(int NB, int Tpad) {
  const size_t stage = sizeof(float) * CountBig::kWaves * 64 * 15;
  const size_t cnt = sizeof(int) * ((size_t)Tpad + (size_t)CountBig::kWaves * NB);
  return stage > cnt ? stage : cnt;
}

int launch_geom_fwd_count_large(const float* params, const float* sh_rest, int sh_degree,
                                const float* depth_bt, int G, const float* camera, float near_z,
                                float blur, float* proj, uint8_t* keep, int32_t* step_adv,
                                float b1, float b2, int ntx, int nty, float S, int span, int NB,
                                int Tpad, int* mat, int2* cell_slot, hipStream_t stream) {
  const int nblk = (G + CountBig::kBlock - 1) / CountBig::kBlock;
  const size_t lds = geom_fwd_count_large_lds(NB, Tpad);
  if (lds > kMaxLdsBytes) return TTS_EINVAL;  // callers check first and take the two-kernel path
  const bool sh = sh_degree > 0;
  static LdsLimit lim[2];
  if (lds > 65536) {
    const void* fn = sh ? reinterpret_cast<const void*>(&k_geom_fwd_count_large<true>)
                        : reinterpret_cast<const void*>(&k_geom_fwd_count_large<false>);
    const int e = raise_lds_limit(fn, lim[sh ? 1 : 0]);
    if (e) return e;
  }
  if (sh)
    k_geom_fwd_count_large<true><<<nblk, 1024, lds, stream>>>(
        params, G, sh_rest, sh_rest_count(sh_degree), depth_bt, camera, near_z, blur, proj, keep,
        step_adv, b1, b2, ntx, nty, S, span, NB, Tpad, mat, cell_slot);
  else
    k_geom_fwd_count_large<false><<<nblk, 1024, lds, stream>>>(
        params, G, nullptr, 0, depth_bt, camera, near_z, blur, proj, keep, step_adv, b1, b2, ntx,
        nty, S, span, NB, Tpad, mat, cell_slot);
  return launch_status();
}

size_t geom_seam_lds(int NB, int Tpad) {
  const size_t stage = sizeof(float) * 2 * kGeoBlock * kSeamRow;
  const size_t cnt = sizeof(int) * ((size_t)Tpad + (size_t)CountFused::kWaves * NB);
  return stage > cnt ? stage : cnt;
}

int launch_geom_seam(float* params, int G, const float* cam_b, const float* cam_f, float near_z,
                     float blur, const float* gslot, const int32_t* inv, float* gparams, float* m,
                     float* v, const float* lr, const int32_t* step, float b1, float b2,
                     float eps, float* proj, uint8_t* keep, int ntx, int nty, float S, int span,
                     int NB, int Tpad, int* mat, int2* cell_slot, hipStream_t stream) {
  const int nblk = (G + CountFused::kBlock - 1) / CountFused::kBlock;
  const size_t lds = geom_seam_lds(NB, Tpad);
  if (lds > kMaxLdsBytes) return TTS_EINVAL;
  // its staging always passes 64 KB (TrainStep makes one call before it captures)
  static LdsLimit lim;
  const int le = raise_lds_limit(reinterpret_cast<const void*>(&k_geom_bwd_adam_fwd_count), lim);
  if (le) return le;
  k_geom_bwd_adam_fwd_count<<<nblk, 512, lds, stream>>>(
      params, G, cam_b, cam_f, near_z, blur, gslot, inv, gparams, m, v, lr, step, b1, b2, eps,
      proj, keep, ntx, nty, S, span, NB, Tpad, mat, cell_slot);
  return launch_status();
}

}  // namespace tts

using namespace tts;

extern "C" {

int tts_version(void) { return (0 << 16) | 1; }

const char* tts_strerror(int code) {
  switch (code) {
    case TTS_OK: return "ok";
    case TTS_EINVAL: return "invalid argument (null pointer, non-positive size or size over the limit)";
    case TTS_ETILE: return "tile side must be 16 or 32 and divide H and W (binning: at most 38912 tiles)";
    case TTS_EK: return "K must be in [1, 512]";
    case TTS_EWORKSPACE: return "workspace missing or too small";
    case TTS_ESPAN: return "span must be in [1, 8192]";
    case TTS_EG: return "G must be below 2^30 (at most 2^28 for binning)";
    case TTS_ERADIUS: return "only stencil radius R = 1 is supported";
    case TTS_ESH: return "SH degree must be in [0, 3], with rest coefficients when above 0";
    case TTS_ESCRATCH: return "sizes exceed the fixed scratch of the allocation-free entry point";
    default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}

int tts_geom_fwd(const float* params, int G, const float* camera, float near_z, float blur,
                 float* proj, uint8_t* keep, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !proj || !keep))) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  k_geom_fwd<false><<<grid1d(G, 256), 256, 0, stream>>>(params, G, nullptr, 0, nullptr, camera,
                                                        near_z, blur, proj, keep, nullptr, 0.f,
                                                        0.f);
  return launch_status();
}

// SH degree check shared by the *_ex entry points: 0 <= deg <= 3, rest present when deg > 0.
static int sh_args(int deg, const void* rest) {
  if (deg < 0 || deg > 3) return TTS_ESH;
  if (deg > 0 && !rest) return TTS_ESH;
  return TTS_OK;
}

int tts_geom_fwd_ex(const float* params, const float* sh_rest, int sh_degree,
                    const float* depth_bt, int G, const float* camera, float near_z, float blur,
                    float* proj, uint8_t* keep, int32_t* step_adv, float beta1, float beta2,
                    hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !proj || !keep))) return TTS_EINVAL;
  if (const int e = sh_args(sh_degree, sh_rest)) return e;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) {  // no rows: the advance alone
    if (step_adv) k_adam_advance<<<1, 64, 0, stream>>>(step_adv, beta1, beta2);
    return launch_status();
  }
  const dim3 grid = grid1d(G, 256);
  if (sh_degree > 0)
    k_geom_fwd<true><<<grid, 256, 0, stream>>>(params, G, sh_rest, sh_rest_count(sh_degree),
                                               depth_bt, camera, near_z, blur, proj, keep,
                                               step_adv, beta1, beta2);
  else
    k_geom_fwd<false><<<grid, 256, 0, stream>>>(params, G, nullptr, 0, depth_bt, camera, near_z,
                                                blur, proj, keep, step_adv, beta1, beta2);
  return launch_status();
}

int tts_geom_bwd(const float* params, int G, const float* camera, float near_z, float blur,
                 const float* grad9, float* gparams, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !grad9 || !gparams))) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  k_geom_bwd<false><<<grid1d(G, 256), 256, 0, stream>>>(params, G, nullptr, 0,
                                                        DepthW{nullptr, nullptr, 1.0f, 0, 0},
                                                        camera, near_z, blur, grad9, gparams,
                                                        nullptr);
  return launch_status();
}

int tts_geom_bwd_ex(const float* params, const float* sh_rest, int sh_degree,
                    const float* depth_bt, int depth_zgrad, int G, const float* camera,
                    float near_z, float blur, const float* grad9, float* gparams,
                    float* gsh_rest, float* gdepth, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !grad9 || !gparams))) return TTS_EINVAL;
  if (const int e = sh_args(sh_degree, sh_rest)) return e;
  if (sh_degree > 0 && !gsh_rest) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  const DepthW dwa{depth_bt, gdepth, 1.0f, 0, depth_zgrad & (TTS_GRAD_DEPTH_Z | TTS_GRAD_SH_DIR)};
  const dim3 grid = grid1d(G, 256);
  if (sh_degree > 0)
    k_geom_bwd<true><<<grid, 256, 0, stream>>>(params, G, sh_rest, sh_rest_count(sh_degree), dwa,
                                               camera, near_z, blur, grad9, gparams, gsh_rest);
  else
    k_geom_bwd<false><<<grid, 256, 0, stream>>>(params, G, nullptr, 0, dwa, camera, near_z, blur,
                                                grad9, gparams, nullptr);
  return launch_status();
}

int tts_adam_flat(float* params, float* m, float* v, const float* grad, const float* lr1,
                  int64_t n, const int32_t* step, float beta1, float beta2, float eps,
                  hipStream_t stream) {
  if (n < 0 || (n > 0 && (!params || !m || !v || !grad || !lr1 || !step))) return TTS_EINVAL;
  if (n == 0) return TTS_OK;
  k_adam_flat<<<grid1d(n, 256), 256, 0, stream>>>(params, m, v, grad, lr1, n, step, beta1, beta2,
                                                  eps);
  return launch_status();
}

int tts_adam_advance(int32_t* step, float beta1, float beta2, hipStream_t stream) {
  if (!step) return TTS_EINVAL;
  k_adam_advance<<<1, 64, 0, stream>>>(step, beta1, beta2);
  return launch_status();
}

int tts_adam(float* params, float* m, float* v, const float* grad, const float* lr, int G,
             const int32_t* step, float beta1, float beta2, float eps, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !m || !v || !grad || !lr || !step))) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  const int64_t n = (int64_t)G * 14;
  k_adam<<<grid1d(n, 256), 256, 0, stream>>>(params, m, v, grad, lr, n, step, beta1, beta2, eps);
  return launch_status();
}

int tts_geom_bwd_accum(const float* params, int G, const float* camera, float near_z,
                       float blur, const float* gslot, const int32_t* inv, float scale,
                       float* gacc, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !gslot || !inv || !gacc))) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  k_geom_bwd_accum<false><<<grid1d(G, 256), 256, 0, stream>>>(
      params, G, nullptr, 0, DepthW{nullptr, nullptr, 1.0f, 0, 0}, camera, near_z, blur, gslot,
      inv, scale, gacc, nullptr);
  return launch_status();
}

int tts_geom_bwd_accum_ex(const float* params, const float* sh_rest, int sh_degree,
                          const float* depth_bt, int G, const float* camera, float near_z,
                          float blur, const float* gslot, const int32_t* inv, float scale,
                          float* gacc, float* gacc_sh, float* gacc_depth, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !gslot || !inv || !gacc))) return TTS_EINVAL;
  if (const int e = sh_args(sh_degree, sh_rest)) return e;
  if (sh_degree > 0 && !gacc_sh) return TTS_EINVAL;
  if (depth_bt && !gacc_depth) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  const DepthW dwa{depth_bt, gacc_depth, scale, 1, 0};
  const dim3 grid = grid1d(G, 256);
  if (sh_degree > 0)
    k_geom_bwd_accum<true><<<grid, 256, 0, stream>>>(params, G, sh_rest, sh_rest_count(sh_degree),
                                                     dwa, camera, near_z, blur, gslot, inv, scale,
                                                     gacc, gacc_sh);
  else
    k_geom_bwd_accum<false><<<grid, 256, 0, stream>>>(params, G, nullptr, 0, dwa, camera, near_z,
                                                      blur, gslot, inv, scale, gacc, nullptr);
  return launch_status();
}

int tts_geom_bwd_adam(float* params, int G, const float* camera, float near_z, float blur,
                      const float* gslot, const int32_t* inv, float* gparams, float* m, float* v,
                      const float* lr, const int32_t* step, float beta1, float beta2, float eps,
                      hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !gslot || !inv || !m || !v || !lr || !step)))
    return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  k_geom_bwd_adam<false, false><<<grid1d(G, 256), 256, 0, stream>>>(
      params, G, nullptr, nullptr, nullptr, 0, camera, near_z, blur, gslot, inv, gparams, m, v,
      lr, nullptr, step, beta1, beta2, eps, McmcArgs{0.0f, 0.0f, 0.0f, 0u},
      DepthW{nullptr, nullptr, 1.0f, 0, 0});
  return launch_status();
}

int tts_geom_bwd_adam_ex(float* params, float* sh_rest, float* sh_m, float* sh_v, int sh_degree,
                         const float* depth_bt, float* gdepth, int G, const float* camera,
                         float near_z, float blur, const float* gslot, const int32_t* inv,
                         float* gparams, float* m, float* v, const float* lr, const float* lr_sh,
                         const int32_t* step, float beta1, float beta2, float eps,
                         float lambda_o, float lambda_s, float noise_lr, uint32_t seed,
                         hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !camera || !gslot || !inv || !m || !v || !lr || !step)))
    return TTS_EINVAL;
  if (const int e = sh_args(sh_degree, sh_rest)) return e;
  if (sh_degree > 0 && (!sh_m || !sh_v || !lr_sh)) return TTS_EINVAL;
  if (lambda_o < 0.0f || lambda_s < 0.0f || noise_lr < 0.0f) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  const McmcArgs mc{lambda_o / (float)G, lambda_s / (3.0f * (float)G), noise_lr, seed};
  const DepthW dwa{depth_bt, gdepth, 1.0f, 0, 0};
  const bool use_mc = lambda_o > 0.0f || lambda_s > 0.0f || noise_lr > 0.0f;
  const int n_rest = sh_rest_count(sh_degree);
  const dim3 grid = grid1d(G, 256);
#define TTS_LAUNCH_BWD_ADAM(SH, MC)                                                          \
  k_geom_bwd_adam<SH, MC><<<grid, 256, 0, stream>>>(params, G, sh_rest, sh_m, sh_v, n_rest,   \
                                                    camera, near_z, blur, gslot, inv, gparams, \
                                                    m, v, lr, lr_sh, step, beta1, beta2, eps,  \
                                                    mc, dwa)
  if (sh_degree > 0) {
    if (use_mc) TTS_LAUNCH_BWD_ADAM(true, true);
    else TTS_LAUNCH_BWD_ADAM(true, false);
  } else {
    if (use_mc) TTS_LAUNCH_BWD_ADAM(false, true);
    else TTS_LAUNCH_BWD_ADAM(false, false);
  }
#undef TTS_LAUNCH_BWD_ADAM
  return launch_status();
}

size_t tts_depth_weight_workspace_bytes(int G) {
  if (G < 0) return 0;
  const int nb = (G + 256 * kDwPer - 1) / (256 * kDwPer);
  return sizeof(float) * 2 * (size_t)(nb > 0 ? nb : 1);
}

int tts_depth_weight_adam(const float* gdepth, int G, float* depth_bt, float* bt_state,
                          const float* lr1, const int32_t* step, float beta1, float beta2,
                          float eps, void* workspace, size_t workspace_bytes,
                          hipStream_t stream) {
  if (G < 0 || !depth_bt || !bt_state || !lr1 || !step || (G > 0 && !gdepth)) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (!workspace || workspace_bytes < tts_depth_weight_workspace_bytes(G)) return TTS_EWORKSPACE;
  const int nb = (G + 256 * kDwPer - 1) / (256 * kDwPer);
  float* part = static_cast<float*>(workspace);
  if (nb > 0) k_dw_partial<<<nb, 256, 0, stream>>>(gdepth, G, part);
  k_dw_adam<<<1, 256, 0, stream>>>(part, nb, depth_bt, bt_state, lr1, step, beta1, beta2, eps);
  return launch_status();
}

int tts_mcmc_reg_grad(const float* params, int G, float lambda_o, float lambda_s, float* grad,
                      hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !grad))) return TTS_EINVAL;
  if (lambda_o < 0.0f || lambda_s < 0.0f) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  k_mcmc_reg_grad<<<grid1d(G, 256), 256, 0, stream>>>(params, G, lambda_o / (float)G,
                                                      lambda_s / (3.0f * (float)G), grad);
  return launch_status();
}

int tts_sgld_noise(float* params, int G, const float* lr, float noise_lr, uint32_t seed,
                   const int32_t* step, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !lr || !step))) return TTS_EINVAL;
  if (noise_lr < 0.0f) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0 || noise_lr == 0.0f) return TTS_OK;
  k_sgld<<<grid1d(G, 256), 256, 0, stream>>>(params, G, lr, noise_lr, seed, step);
  return launch_status();
}

int tts_slot_reduce(const float* gslot, const int32_t* inv, int G, float* grad9,
                    hipStream_t stream) {
  if (G < 0 || (G > 0 && (!gslot || !inv || !grad9))) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (G == 0) return TTS_OK;
  k_slot_reduce<<<grid1d(G, 256), 256, 0, stream>>>(gslot, inv, G, grad9);
  return launch_status();
}

int tts_slot_scatter(const float* gslot, const int32_t* idx, const uint8_t* valid, int T, int K,
                     float* grad9, hipStream_t stream) {
  if (T < 0 || K < 0) return TTS_EINVAL;
  const int64_t TK = (int64_t)T * K;   // in 64 bits: a 32-bit product could wrap past the checks
  if (TK > 0 && (!gslot || !idx || !valid || !grad9)) return TTS_EINVAL;
  if (TK == 0) return TTS_OK;
  k_slot_scatter<<<grid1d(TK, 256), 256, 0, stream>>>(gslot, idx, valid, TK, grad9);
  return launch_status();
}

int tts_zero(float* buf, int64_t n, hipStream_t stream) {
  if (n < 0 || (n > 0 && !buf)) return TTS_EINVAL;
  if (n == 0) return TTS_OK;
  k_zero<<<grid1d(n, 256), 256, 0, stream>>>(buf, n);
  return launch_status();
}

}  // extern "C"
