// Binned poly-splat + WSR render, forward and backward.  One 256-thread workgroup per S x S
// tile (S = 16 or 32).  Math: tools/bh_views.py:65-71 (forward), spike/backward.py:42-58 and
// tools/resident_traced.py:60-88 (backward + theta backward), tools/m4_train_binned.py:130-143
// (tile-local theta_u).
//
// Forward: the tile's valid slots are compacted into LDS as theta_u (6) and (col_o, o_col) (4);
// each thread owns S*S/256 pixels and walks the slots:
//     u = theta . [lx^2, ly^2, lx*ly, lx, ly, 1],  w = max(u,0)^2,  num += w*col, den += w*oc
// and writes C = (num + w_b c_b) * rcp(den + w_b) straight into the [H,W,3] image.  For S = 16
// from proj or slot records (k_splat_fwd_tile) each wave walks the whole tile for a quarter of
// the slots instead, u factored per column.
//
// Backward: per-pixel gnum = gC/den, gden = -(gC.C)/den are staged in LDS (rows padded to S+1
// entries); the slots are then contracted over the tile's pixels slot-parallel (tps adjacent
// lanes share one slot and split its rows).  Along a pixel row, u = (th0*lx + c1)*lx + c0 with
// c0, c1 fixed per row, and the theta gradient is gathered as three row moments sum(gu*lx^2),
// sum(gu*lx), sum(gu), so the inner loop costs 17 VALU ops per (pixel, slot) pair (per-row terms
// included).  Each slot's 10 partial sums are combined with lane shuffles and pushed through
// the theta backward, whose conic and tile-local mean were staged in LDS beside theta; the
// slot's 9 gradients are stored to gslot[T,K,9] (no atomics: the per-gaussian sum over its <= 9
// slots is a gather through the inverse bin table, in a fixed order, done by the geometry
// backward).

#include <type_traits>

#include "tts_common.h"

namespace tts {

constexpr int kSplatMaxK = 512;

struct SlotLDS {
  float4* ta;  // theta_u 0..3
  float4* tb;  // theta_u 4..5, tile-local mu_y, -
  float4* cl;  // col_o r,g,b, o_col
  float4* ge;  // conic a, b, c, tile-local mu_x (proj mode: the theta backward's inputs)
  int* gid;    // gaussian id (proj mode) or original slot (theta mode)
  int* sid;    // original slot index of the compacted entry
};

__device__ __forceinline__ SlotLDS carve_slots(unsigned char* base, int K) {
  SlotLDS s;
  s.ta = reinterpret_cast<float4*>(base);
  s.tb = s.ta + K;
  s.cl = s.tb + K;
  s.ge = s.cl + K;
  s.gid = reinterpret_cast<int*>(s.ge + K);
  s.sid = s.gid + K;
  return s;
}

__host__ __device__ __forceinline__ size_t slot_lds_bytes(int K) { return (size_t)K * (4 * 16 + 8); }

// Tile-local theta_u for one gaussian record r0..r2 of proj (tools/m4_train_binned.py:130-143).
__device__ __forceinline__ void slot_from_rec(const float4 r0, const float4 r1, const float4 r2,
                                              float ox, float oy, float inv_k, float4& ta,
                                              float4& tb, float4& cl) {
  const float a = r0.z, b = r0.w, c = r1.x;
  const float mx = r0.x - ox, my = r0.y - oy;
  const float Q0 = a * mx * mx + 2.0f * b * mx * my + c * my * my;
  ta = make_float4(-a * inv_k, -c * inv_k, -2.0f * b * inv_k, 2.0f * (a * mx + b * my) * inv_k);
  tb = make_float4(2.0f * (b * mx + c * my) * inv_k, 1.0f - Q0 * inv_k, my, 0.0f);
  cl = make_float4(r1.z, r1.w, r2.x, r2.y);
}
// torch.relu propagates NaN: a slot whose u is NaN at every pixel (theta_u holds a NaN, or both
// infinities -- the basis monomials are positive, so u = theta . Phi is then NaN everywhere)
// makes every pixel of its tile NaN in the reference.  The forward kernels test each valid slot
// here and write NaN over such a tile (image and den), so the backward sees NaN there too.
__device__ __forceinline__ bool theta_poisons(const float4 ta, const float4 tb) {
  return __builtin_isnan(((ta.x + ta.y) + (ta.z + ta.w)) + (tb.x + tb.y));
}
// A slot whose u can be large, infinite or NaN at some pixel: the sum of its |theta| is 1e15 or
// more, infinite or NaN (a NaN or an infinity among the six makes the sum NaN or infinite).
// Below that, at pixel coordinates under 32 every product, partial sum and u stays under 1.1e18
// whatever the order of evaluation (no monomial exceeds 1024), so u is finite, relu_bits is
// exact, and so is the fast walks' 2 relu(u) = u + |u| with its square 4 w (under FLT_MAX while
// u < 9.2e18).  A tile with such a slot walks with relu_nan and w itself: where u comes out NaN
// (inf - inf, in this kernel's order of evaluation -- torch's own order is its BLAS's), the
// pixel is NaN, as torch.relu keeps it, and -inf gives 0.  (The GPU's generated NaN can carry
// the sign bit, which relu_bits would map to 0.)  The sum of absolute values is five full-rate
// adds; the largest of them, five maxes at half rate and a NaN test besides.
__device__ __forceinline__ bool theta_wild(const float4 ta, const float4 tb) {
  const float q = ((fabsf(ta.x) + fabsf(ta.y)) + (fabsf(ta.z) + fabsf(ta.w))) +
                  (fabsf(tb.x) + fabsf(tb.y));
  return !(q < 1e15f);
}

__device__ __forceinline__ void build_slot(const float* __restrict__ proj, int g, float ox,
                                           float oy, float inv_k, float4& ta, float4& tb,
                                           float4& cl) {
  const float4* r = reinterpret_cast<const float4*>(proj + (int64_t)g * 12);
  slot_from_rec(r[0], r[1], r[2], ox, oy, inv_k, ta, tb, cl);
}

// Compact the tile's valid slots into LDS in slot order.  Returns the valid count.
__device__ __forceinline__ int load_slots_proj(const float* __restrict__ proj,
                                               const int32_t* __restrict__ idx,
                                               const uint8_t* __restrict__ valid, int t, int K,
                                               float ox, float oy, float inv_k, SlotLDS sl,
                                               int* s_tmp, bool* bad) {
  // idx is read beside valid (every slot's entry is written; an invalid one is not used), and a
  // valid slot's proj record is requested before the compaction scan, whose barriers then
  // overlap that round trip
  int base = 0;
  for (int s0 = 0; s0 < K; s0 += 256) {
    const int s = s0 + threadIdx.x;
    const int64_t ts = (int64_t)t * K + min(s, K - 1);
    const uint8_t vb = valid[ts];  // both loads unconditional: in flight together
    const int g = idx[ts];
    const int v = (s < K && vb != 0) ? 1 : 0;
    float4 r0, r1, r2;
    if (v) {
      const float4* r = reinterpret_cast<const float4*>(proj + (int64_t)g * 12);
      r0 = r[0];
      r1 = r[1];
      r2 = r[2];
    }
    int total;
    const int pos = base + block_excl_scan256(v, s_tmp, &total);
    if (v) {
      float4 ta, tb, cl;
      slot_from_rec(r0, r1, r2, ox, oy, inv_k, ta, tb, cl);
      *bad = *bad || theta_wild(ta, tb);
      sl.ta[pos] = ta;
      sl.tb[pos] = tb;
      sl.cl[pos] = cl;
      sl.ge[pos] = make_float4(r0.z, r0.w, r1.x, r0.x - ox);
      sl.gid[pos] = g;
      sl.sid[pos] = s;
    }
    base += total;
  }
  return base;
}

// The same from slot records (rec = slot_rec [T][K][12] in dispatch order, block b reads its
// own K records and kept count): the kept slots are the prefix [0, pos_count[b]), so no
// compaction.  Returns the kept count.
__device__ __forceinline__ int load_slots_rec(const float* __restrict__ rec,
                                              const int32_t* __restrict__ pos_count, int K,
                                              float ox, float oy, float inv_k, SlotLDS sl,
                                              bool* bad) {
  const int nb = min(pos_count[blockIdx.x], K);
  for (int s = threadIdx.x; s < K; s += 256) {
    // read whether kept or not: the loads are in flight beside pos_count
    const float4* r = reinterpret_cast<const float4*>(rec + ((int64_t)blockIdx.x * K + s) * 12);
    const float4 r0 = r[0], r1 = r[1], r2 = r[2];
    if (s < nb) {
      float4 ta, tb, cl;
      slot_from_rec(r0, r1, r2, ox, oy, inv_k, ta, tb, cl);
      *bad = *bad || theta_wild(ta, tb);
      sl.ta[s] = ta;
      sl.tb[s] = tb;
      sl.cl[s] = cl;
      sl.ge[s] = make_float4(r0.z, r0.w, r1.x, r0.x - ox);
      sl.gid[s] = s;
      sl.sid[s] = s;
    }
  }
  return nb;
}

__device__ __forceinline__ float opf(float x) { return x; }
__device__ __forceinline__ float opf(__bf16 x) { return (float)x; }

// Load pre-gathered operands theta[T,6,K], col[T,K,3], oc[T,K] (all K slots); OT = float, or
// __bf16 for the reference's bf16 operand upload (tools/m4_train_binned.py:42-43), widened to
// fp32 here.
template <typename OT>
__device__ __forceinline__ void load_slots_theta(const OT* __restrict__ theta,
                                                 const OT* __restrict__ col,
                                                 const OT* __restrict__ oc, int t, int K,
                                                 SlotLDS sl, bool* bad) {
  const OT* th = theta + (int64_t)t * 6 * K;
  for (int s = threadIdx.x; s < K; s += blockDim.x) {
    sl.ta[s] = make_float4(opf(th[s]), opf(th[K + s]), opf(th[2 * K + s]), opf(th[3 * K + s]));
    sl.tb[s] = make_float4(opf(th[4 * K + s]), opf(th[5 * K + s]), 0.0f, 0.0f);
    *bad = *bad || theta_wild(sl.ta[s], sl.tb[s]);
    const OT* c = col + ((int64_t)t * K + s) * 3;
    sl.cl[s] = make_float4(opf(c[0]), opf(c[1]), opf(c[2]), opf(oc[(int64_t)t * K + s]));
    sl.gid[s] = s;
    sl.sid[s] = s;
  }
}

template <int S, bool FROM_PROJ, typename OT = float>
__global__ __launch_bounds__(256) void k_splat_fwd(
    const float* __restrict__ proj, const int32_t* __restrict__ idx,
    const uint8_t* __restrict__ valid, const OT* __restrict__ theta,
    const OT* __restrict__ col, const OT* __restrict__ oc,
    const int32_t* __restrict__ order, int ntx, int W, int K, float inv_k,
    const float* __restrict__ bg, float* __restrict__ image, float* __restrict__ den_out) {
  constexpr int PPT = S * S / 256;  // pixels per thread
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
  __shared__ int s_tmp[4];
  const SlotLDS sl = carve_slots(s_dyn, K);
  const int t = order ? order[blockIdx.x] : blockIdx.x;
  const int tx = t % ntx, ty = t / ntx;
  const int ox = tx * S, oy = ty * S;
  int n;
  bool bad = false;
  if constexpr (FROM_PROJ) {
    n = load_slots_proj(proj, idx, valid, t, K, (float)ox, (float)oy, inv_k, sl, s_tmp, &bad);
  } else {
    load_slots_theta(theta, col, oc, t, K, sl, &bad);
    n = K;
  }
  // a tile with a wild slot (theta_wild) walks with relu_nan; a NaN or mixed-infinity theta
  // then makes u NaN at every pixel (the monomials are positive), so its tile comes out NaN
  const bool wild = __syncthreads_or(bad);

  float lx[PPT], ly[PPT], xx[PPT], yy[PPT], xy[PPT];
  float ar[PPT], ag[PPT], ab[PPT], ad[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int p = threadIdx.x + 256 * i;
    lx[i] = (float)(p % S) + 0.5f;
    ly[i] = (float)(p / S) + 0.5f;
    xx[i] = lx[i] * lx[i];
    yy[i] = ly[i] * ly[i];
    xy[i] = lx[i] * ly[i];
    ar[i] = ag[i] = ab[i] = ad[i] = 0.0f;
  }
  auto walk = [&](auto exact) {
    for (int s = 0; s < n; ++s) {
      const float4 A = sl.ta[s], B = sl.tb[s], C = sl.cl[s];
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        // one fixed order of evaluation (it decides where overflowing terms give NaN)
        const float u = fmaf(A.x, xx[i], fmaf(A.y, yy[i], fmaf(A.z, xy[i],
                             fmaf(A.w, lx[i], fmaf(B.x, ly[i], B.y)))));
        const float r = decltype(exact)::value ? relu_nan(u) : relu_bits(u);
        const float w = r * r;
        ar[i] += w * C.x;
        ag[i] += w * C.y;
        ab[i] += w * C.z;
        ad[i] += w * C.w;
      }
    }
  };
  if (wild)
    walk(std::true_type{});
  else
    walk(std::false_type{});
  const float wb = bg[0];
  const float cbr = wb * bg[1], cbg = wb * bg[2], cbb = wb * bg[3];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int p = threadIdx.x + 256 * i;
    const int64_t pix = (int64_t)(oy + p / S) * W + ox + p % S;
    const float d = ad[i] + wb;
    // one hardware reciprocal per pixel (1 ulp; an IEEE division costs ~10 VALU instructions)
    const float inv = __builtin_amdgcn_rcpf(d);
    image[pix * 3 + 0] = (ar[i] + cbr) * inv;
    image[pix * 3 + 1] = (ag[i] + cbg) * inv;
    image[pix * 3 + 2] = (ab[i] + cbb) * inv;
    if (den_out) den_out[pix] = d;
  }
}

// Contraction of one tile's staged slots over its pixels, then the theta backward and the
// stores (the main loop of the splat backward).  Every thread of the block must call it (it
// contains barriers when slots share rows).
// WILD = false (no slot theta_wild: each sum of |theta| < 1e15): the pixel terms q were staged
// as q/4 and the slot colours are doubled here, so with r2 = u + |u| = 2 relu(u) (one full-rate
// add instead of a half-rate max) r2^2 q/4 = w q and r2 (q/4)(2 C) = relu(u) q.C exactly
// (scalings by powers of two).  WILD = true: relu_bits on unscaled q (a NaN u only occurs in tiles whose
// den the forward made NaN, so every gradient there is NaN whatever relu gives).
template <int S, bool FROM_PROJ, bool WILD>
__device__ __forceinline__ void bwd_contract(int n, const SlotLDS& sl, const float4* s_px,
                                             int t, int K, int ox, int oy,
                                             float inv_k, const float* __restrict__ proj,
                                             float* __restrict__ gslot,
                                             float* __restrict__ gtheta,
                                             float* __restrict__ gcol, float* __restrict__ goc) {
  constexpr int kRowChunks = S == 16 ? 2 : 1;  // 8-pixel chunks of a row unrolled
  // threads per slot: split rows while slots are few.  The tps threads of a slot are adjacent
  // lanes of one wave (rows h, h + tps, ...), so their partial sums combine with lane shuffles.
  int tps = 1;
  while (tps < 16 && tps * 2 * n <= 256) tps <<= 1;
  const int sg = 256 / tps;
  const int h = threadIdx.x % tps, sl_local = threadIdx.x / tps;
  for (int c0s = 0; c0s < n; c0s += sg) {
    const int s = c0s + sl_local;
    const bool active = s < n;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f), B = A, C = A;
    if (active) {
      A = sl.ta[s];
      B = sl.tb[s];
      C = sl.cl[s];
      if constexpr (!WILD) {
        C.x *= 2.f;
        C.y *= 2.f;
        C.z *= 2.f;
        C.w *= 2.f;
      }
    }
    float g0 = 0.f, g1 = 0.f, g2 = 0.f, g3 = 0.f, g4 = 0.f, g5 = 0.f;
    float gr = 0.f, gg = 0.f, gb = 0.f, go = 0.f;
    if (active) {
#pragma unroll 2
      for (int y = h; y < S; y += tps) {
        const float ly = (float)y + 0.5f;
        const float yy = ly * ly;
        const float cc0 = A.y * yy + B.x * ly + B.y;  // u = (A.x*lx + cc1)*lx + cc0
        const float cc1 = A.z * ly + A.w;
        float m0 = 0.f, m1 = 0.f, m2 = 0.f;
        const float4* row = s_px + y * (S + 1);
        // S = 16: fully unrolled along the row, so lx and lx^2 are literals (2 VALU ops per pair
        // fewer than a rolled loop over 8-pixel chunks, which recomputes them).  S = 32 keeps
        // the rolled chunks: unrolled, its 32-pixel rows spill registers.
#pragma unroll kRowChunks
        for (int xb = 0; xb < S; xb += 8) {
          const float xbf = (float)xb;
#pragma unroll
          for (int x8 = 0; x8 < 8; ++x8) {
            const float lx = xbf + ((float)x8 + 0.5f);
            const float u = (A.x * lx + cc1) * lx + cc0;
            const float r = WILD ? relu_bits(u) : u + fabsf(u);
            const float w = r * r;
            const float4 q = row[xb + x8];
            const float gw = q.x * C.x + q.y * C.y + q.z * C.z + q.w * C.w;
            const float gu = r * gw;  // half of dL/du
            gr += w * q.x;
            gg += w * q.y;
            gb += w * q.z;
            go += w * q.w;
            m0 += gu * (lx * lx);
            m1 += gu * lx;
            m2 += gu;
          }
        }
        g0 += m0;
        g2 += ly * m1;
        g3 += m1;
        g1 += yy * m2;
        g4 += ly * m2;
        g5 += m2;
      }
    }
    // combine the tps row-partials of each slot (butterfly over its adjacent lanes)
    for (int d = 1; d < tps; d <<= 1) {
      g0 += __shfl_xor(g0, d); g1 += __shfl_xor(g1, d); g2 += __shfl_xor(g2, d);
      g3 += __shfl_xor(g3, d); g4 += __shfl_xor(g4, d); g5 += __shfl_xor(g5, d);
      gr += __shfl_xor(gr, d); gg += __shfl_xor(gg, d); gb += __shfl_xor(gb, d);
      go += __shfl_xor(go, d);
    }
    if (h == 0 && active) {
      // dL/du = 2 r gw: the factor 2 was left out of the inner loop
      g0 *= 2.f; g1 *= 2.f; g2 *= 2.f; g3 *= 2.f; g4 *= 2.f; g5 *= 2.f;
      if constexpr (FROM_PROJ) {
        // theta backward (tools/resident_traced.py:72-88), gtQ = gtheta * (-1/k); the conic and
        // tile-local mean were staged beside theta, so no global re-read
        const float4 ge = sl.ge[s];
        const float a = ge.x, b = ge.y, c = ge.z;
        const float mx = ge.w, my = B.z;
        const float nk = -inv_k;
        const float q0 = g0 * nk, q1 = g1 * nk, q2 = g2 * nk, q3 = g3 * nk, q4 = g4 * nk, q5 = g5 * nk;
        const float ga = q0 - 2.f * mx * q3 + mx * mx * q5;
        const float gbv = 2.f * q2 - 2.f * my * q3 - 2.f * mx * q4 + 2.f * mx * my * q5;
        const float gc = q1 - 2.f * my * q4 + my * my * q5;
        const float gmx = -2.f * a * q3 - 2.f * b * q4 + (2.f * a * mx + 2.f * b * my) * q5;
        const float gmy = -2.f * b * q3 - 2.f * c * q4 + (2.f * b * mx + 2.f * c * my) * q5;
        float* dst = gslot + ((int64_t)t * K + sl.sid[s]) * 9;
        dst[0] = ga;
        dst[1] = gbv;
        dst[2] = gc;
        dst[3] = gmx;
        dst[4] = gmy;
        dst[5] = gr;
        dst[6] = gg;
        dst[7] = gb;
        dst[8] = go;
      } else {
        float* th = gtheta + (int64_t)t * 6 * K;
        th[s] = g0; th[K + s] = g1; th[2 * K + s] = g2;
        th[3 * K + s] = g3; th[4 * K + s] = g4; th[5 * K + s] = g5;
        float* gcp = gcol + ((int64_t)t * K + s) * 3;
        gcp[0] = gr; gcp[1] = gg; gcp[2] = gb;
        goc[(int64_t)t * K + s] = go;
      }
    }
  }
}

// REC (with FROM_PROJ): proj is slot_rec [T][K][12] in dispatch order and pos_count[b] the
// kept count of block b's tile (load_slots_rec).
template <int S, bool FROM_PROJ, typename OT = float, bool REC = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6, 8))) void k_splat_bwd(
    const float* __restrict__ proj, const int32_t* __restrict__ idx,
    const uint8_t* __restrict__ valid, const OT* __restrict__ theta,
    const OT* __restrict__ col, const OT* __restrict__ oc,
    const int32_t* __restrict__ order, const int32_t* __restrict__ pos_count, int ntx, int W,
    int K, float inv_k,
    const float* __restrict__ bg, const float* __restrict__ image,
    const float* __restrict__ den, const float* __restrict__ gimage, float* __restrict__ gslot,
    float* __restrict__ gtheta, float* __restrict__ gcol, float* __restrict__ goc,
    float* __restrict__ gwb) {
  constexpr int P = S * S;
  constexpr int PPT = P / 256;
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
  __shared__ int s_tmp[4];
  __shared__ float s_ftmp[4];
  const SlotLDS sl = carve_slots(s_dyn, K);
  // pixel rows padded to S + 1 entries: the tps rows read together fall in different banks
  float4* s_px = reinterpret_cast<float4*>(s_dyn + slot_lds_bytes(K) + (16 - slot_lds_bytes(K) % 16) % 16);

  const int t = order ? order[blockIdx.x] : blockIdx.x;
  const int tx = t % ntx, ty = t / ntx;
  const int ox = tx * S, oy = ty * S;
  // Issue this thread's pixel loads first: their latency overlaps the slot prologue.
  float pg[PPT][3], pc[PPT][3], pd[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int p = threadIdx.x + 256 * i;
    const int64_t pix = (int64_t)(oy + p / S) * W + ox + p % S;
    pd[i] = den[pix];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      pg[i][c] = gimage[pix * 3 + c];
      pc[i][c] = image[pix * 3 + c];
    }
  }
  int n;
  bool bad = false;  // a wild slot (theta_wild): the contraction keeps relu on unscaled terms
  if constexpr (REC) {
    n = load_slots_rec(proj, pos_count, K, (float)ox, (float)oy, inv_k, sl, &bad);
  } else if constexpr (FROM_PROJ) {
    n = load_slots_proj(proj, idx, valid, t, K, (float)ox, (float)oy, inv_k, sl, s_tmp, &bad);
  } else {
    load_slots_theta(theta, col, oc, t, K, sl, &bad);
    n = K;
  }
  const bool wild = __syncthreads_or(bad);
  // Per-pixel WSR backward: gnum = gC/den, gden = -(gC . C)/den (staged as a quarter unless the
  // tile is wild, see bwd_contract).
  const float bg1 = bg[1], bg2 = bg[2], bg3 = bg[3];
  const float qs = wild ? 1.0f : 0.25f;
  float wpart = 0.0f;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const float inv = __builtin_amdgcn_rcpf(pd[i]);   // hardware reciprocal, 1 ulp
    const float4 q = make_float4(pg[i][0] * inv, pg[i][1] * inv, pg[i][2] * inv,
                                 -(pg[i][0] * pc[i][0] + pg[i][1] * pc[i][1] + pg[i][2] * pc[i][2]) * inv);
    const int p = threadIdx.x + 256 * i;
    s_px[(p / S) * (S + 1) + p % S] = make_float4(q.x * qs, q.y * qs, q.z * qs, q.w * qs);
    wpart += q.x * bg1 + q.y * bg2 + q.z * bg3 + q.w;
  }
  if (gwb) {  // per-tile partial of dL/dw_b (summed by the caller)
    const float tot = block_sum256(wpart, s_ftmp);
    if (threadIdx.x == 0) gwb[t] = tot;
  }
  __syncthreads();

  if (wild)
    bwd_contract<S, FROM_PROJ, true>(n, sl, s_px, t, K, ox, oy, inv_k, proj, gslot, gtheta, gcol,
                                     goc);
  else
    bwd_contract<S, FROM_PROJ, false>(n, sl, s_px, t, K, ox, oy, inv_k, proj, gslot, gtheta,
                                      gcol, goc);
}

// ------------------------------------------------------------------ matrix-core forward --
// The same per-tile contraction on the gfx950 matrix cores (v_mfma_f32_16x16x32_bf16, S = 16).
//   GEMM1  u^T[slot][pixel] = Theta[slot][k] . Phi^T[k][pixel].  The basis has 6 monomials but
//          the instruction contracts 32: the spare depth carries split-precision terms, so with
//          theta = th_hi + th_mid + th_lo and Phi = phi_hi + phi_lo (bf16 parts; lx, ly, 1 are
//          exact in bf16) u is accumulated from
//            k 0-5 th_hi.phi_hi | 6-11 th_mid.phi_hi | 12-17 th_lo.phi_hi |
//            18-20 th_hi.phi_lo | 21-23 th_mid.phi_lo | 24-31 zero
//          i.e. to about fp32 accuracy at no extra matrix-core cost.
//   GEMM2  [num | den][pixel][n] = w[pixel][slot] . [col_o | o_col][slot][n], w = max(u,0)^2.
//          The GEMM1 result layout (lane: pixel, registers: 4 consecutive slots of each 16-slot
//          half) is exactly the A-operand layout of GEMM2 with the slot order permuted, so the
//          colour operand is stored in that permuted order and no data moves between lanes.
//          SPLIT_W (fp32 mode): w = w_hi + w_lo and colours c_hi | c_lo in columns 0-3 | 4-7,
//          num = D[:, 0:4] + D[:, 4:8] (relative error ~2^-16).  bf16 mode: w and the colours
//          rounded once to bf16 (the reference's bf16 render operands,
//          tools/resident_traced.py:265-274), fp32 accumulation.
// Wave w owns tile rows 4w..4w+3 (one 16-pixel group each); slots are processed 32 at a time.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __bf16 to_bf(float x) { return (__bf16)x; }
__device__ __forceinline__ float from_bf(__bf16 x) { return (float)x; }

// One 32-element theta row (bf16x8 x 4) in the k layout above.
__device__ __forceinline__ void theta_row(const float* th, bf16x8* dst) {
  __bf16 hi[6], mid[6], lo[6];
#pragma unroll
  for (int m = 0; m < 6; ++m) {
    hi[m] = to_bf(th[m]);
    const float r = th[m] - from_bf(hi[m]);
    mid[m] = to_bf(r);
    lo[m] = to_bf(r - from_bf(mid[m]));
  }
  __bf16 row[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) row[k] = to_bf(0.0f);
#pragma unroll
  for (int m = 0; m < 6; ++m) {
    row[m] = hi[m];
    row[6 + m] = mid[m];
    row[12 + m] = lo[m];
  }
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    row[18 + m] = hi[m];
    row[21 + m] = mid[m];
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = row[8 * v + e];
    dst[v] = x;
  }
}

// The lane's 8-element slice (q = lane / 16) of the Phi^T operand for pixel (lx, ly).
__device__ __forceinline__ bf16x8 phi_slice(float lx, float ly, int q) {
  const float f[6] = {lx * lx, ly * ly, lx * ly, lx, ly, 1.0f};
  __bf16 fh[6], fl[3];
#pragma unroll
  for (int m = 0; m < 6; ++m) fh[m] = to_bf(f[m]);
#pragma unroll
  for (int m = 0; m < 3; ++m) fl[m] = to_bf(f[m] - from_bf(fh[m]));
  __bf16 row[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) row[k] = to_bf(0.0f);
#pragma unroll
  for (int m = 0; m < 6; ++m) {
    row[m] = fh[m];
    row[6 + m] = fh[m];
    row[12 + m] = fh[m];
  }
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    row[18 + m] = fl[m];
    row[21 + m] = fl[m];
  }
  bf16x8 v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] = row[8 * j + e];
  return q == 0 ? v[0] : (q == 1 ? v[1] : (q == 2 ? v[2] : v[3]));
}

inline size_t fwd_mx_lds(int K) {
  const int kpad = (K + 31) & ~31;
  return (size_t)kpad * 64 + (size_t)(kpad / 32) * 512;
}

// REC: the slots come from slot records (src = slot_rec, block b reads src[b] and pos_count[b];
// the kept slots are the prefix, no compaction); otherwise src = proj with idx / valid.
template <bool SPLIT_W, bool REC>
__global__ __launch_bounds__(256) void k_splat_fwd_mx(
    const float* __restrict__ src, const int32_t* __restrict__ idx,
    const uint8_t* __restrict__ valid, const int32_t* __restrict__ pos_count,
    const int32_t* __restrict__ order, int ntx, int W, int K, float inv_k,
    const float* __restrict__ bg, float* __restrict__ image, float* __restrict__ den_out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
  __shared__ int s_tmp[4];
  const int kpad = (K + 31) & ~31;
  bf16x8* s_th = reinterpret_cast<bf16x8*>(s_dyn);  // [kpad][4]
  __bf16* s_col = reinterpret_cast<__bf16*>(s_th + (size_t)kpad * 4);  // [kpad/32][4][8][8]
  const int t = order ? order[blockIdx.x] : blockIdx.x;
  const int tx = t % ntx, ty = t / ntx;
  const int ox = tx * 16, oy = ty * 16;
  const float oxf = (float)ox, oyf = (float)oy;
  // compact the valid slots, build theta in fp32 and store its split row and the colours
  const int nb = REC ? min(pos_count[blockIdx.x], K) : 0;
  int n = 0;
  bool bad = false;
  for (int s0 = 0; s0 < K; s0 += 256) {
    const int s = s0 + threadIdx.x;
    int v, pos, total;
    float4 r0, r1, r2;
    if constexpr (REC) {
      // records read whether kept or not (in flight beside pos_count)
      if (s < K) {
        const float4* r = reinterpret_cast<const float4*>(src + ((int64_t)blockIdx.x * K + s) * 12);
        r0 = r[0];
        r1 = r[1];
        r2 = r[2];
      }
      v = s < nb ? 1 : 0;
      pos = s;
      total = max(min(nb - s0, 256), 0);
    } else {
      v = (s < K) ? (valid[(int64_t)t * K + s] != 0) : 0;
      pos = n + block_excl_scan256(v, s_tmp, &total);
      if (v) {
        const float4* r =
            reinterpret_cast<const float4*>(src + (int64_t)idx[(int64_t)t * K + s] * 12);
        r0 = r[0];
        r1 = r[1];
        r2 = r[2];
      }
    }
    if (v) {
      float4 ta, tb, cl;
      slot_from_rec(r0, r1, r2, oxf, oyf, inv_k, ta, tb, cl);
      bad = bad || theta_poisons(ta, tb);
      const float th[6] = {ta.x, ta.y, ta.z, ta.w, tb.x, tb.y};
      theta_row(th, s_th + (size_t)pos * 4);
      const float c4[4] = {cl.x, cl.y, cl.z, cl.w};
      const int c = pos >> 5, r = pos & 31;
      const int q = (r & 15) >> 2, e = (r & 3) + ((r >> 4) << 2);
      __bf16* dst = s_col + (((size_t)(c * 4 + q)) * 8) * 8 + e;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const __bf16 h = to_bf(c4[m]);
        dst[m * 8] = h;
        dst[(4 + m) * 8] = SPLIT_W ? to_bf(c4[m] - from_bf(h)) : to_bf(0.0f);
      }
    }
    n += total;
  }
  const int nch = (n + 31) >> 5;
  // zero the padding slots of the last chunk
  for (int pos = n + threadIdx.x; pos < nch * 32; pos += 256) {
    const bf16x8 z = {};
#pragma unroll
    for (int v = 0; v < 4; ++v) s_th[(size_t)pos * 4 + v] = z;
    const int c = pos >> 5, r = pos & 31;
    const int q = (r & 15) >> 2, e = (r & 3) + ((r >> 4) << 2);
    __bf16* dst = s_col + (((size_t)(c * 4 + q)) * 8) * 8 + e;
#pragma unroll
    for (int m = 0; m < 8; ++m) dst[m * 8] = to_bf(0.0f);
  }
  const bool poisoned = __syncthreads_or(bad);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, q = lane >> 4;
  bf16x8 bphi[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    bphi[i] = phi_slice((float)l16 + 0.5f, (float)(4 * wave + i) + 0.5f, q);
  floatx4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  const floatx4 zero4 = {0.f, 0.f, 0.f, 0.f};
  const bf16x8 zero8 = {};
  for (int c = 0; c < nch; ++c) {
    const bf16x8 a0 = s_th[(size_t)(c * 32 + l16) * 4 + q];
    const bf16x8 a1 = s_th[(size_t)(c * 32 + 16 + l16) * 4 + q];
    const bf16x8 bc = l16 < 8 ? *reinterpret_cast<const bf16x8*>(s_col + ((size_t)(c * 4 + q) * 8 + l16) * 8)
                              : zero8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const floatx4 u0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bphi[i], zero4, 0, 0, 0);
      const floatx4 u1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bphi[i], zero4, 0, 0, 0);
      float w[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // relu_nan: the matrix-core walk's relu is a small share of its VALU work
        const float r0 = relu_nan(u0[e]), r1 = relu_nan(u1[e]);
        w[e] = r0 * r0;
        w[4 + e] = r1 * r1;
      }
      bf16x8 wh;
#pragma unroll
      for (int e = 0; e < 8; ++e) wh[e] = to_bf(w[e]);
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, bc, acc[i], 0, 0, 0);
      if constexpr (SPLIT_W) {
        bf16x8 wl;
#pragma unroll
        for (int e = 0; e < 8; ++e) wl[e] = to_bf(w[e] - from_bf(wh[e]));
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wl, bc, acc[i], 0, 0, 0);
      }
    }
  }
  // lane (q, n = l16) holds column n for pixels 4q..4q+3 of each of its rows
  const float wb = bg[0];
  const float cbn = l16 < 3 ? wb * bg[1 + l16] : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * wave + i;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = acc[i][e];
      if constexpr (SPLIT_W) v += __shfl(v, (lane + 4) & 63);
      const float d = poisoned ? __builtin_nanf("") : __shfl(v, (lane & ~15) + 3) + wb;
      const int64_t pix = (int64_t)(oy + row) * W + ox + 4 * q + e;
      if (l16 < 3) image[pix * 3 + l16] = poisoned ? d : (v + cbn) / d;
      if (l16 == 3 && den_out) den_out[pix] = d;
    }
  }
}

// Forward for 16x16 tiles from proj (tts_splat_fwd) or from slot records (tts_splat_fwd_rec).
// Each wave walks the whole tile for a quarter of the slots (slot s to wave s mod 4), 4 pixels
// per lane (column j = lane % 16, rows 4m + lane / 16): per slot and column the quadratic form
// is u = (theta1 ly + P) ly + Q with P = theta2 lx + theta4 and Q = (theta0 lx + theta3) lx +
// theta5, so a pixel costs 2 FMA for u, relu^2 as an integer max and a multiply, and 4 FMA for
// the colour and density sums.  The four waves' sums are then joined through LDS in wave order.
// (u on the fp32 matrix cores -- one v_mfma_f32_16x16x4f32 for 4 rows x 4 slots x 16 pixels --
// was 0.7 us slower at 1264x832 once the slot records had shortened the prologue.)  Slot s is
// staged at LDS entry s (zero when invalid: u = 0, w = 0) and the walk runs to the highest
// valid slot, so bins whose valid slots form a prefix (tts_assign_bins) add no zero terms
// beyond it.
// REC: the slots come from slot records (src = slot_rec [T][K][12] in dispatch order, block b
// reads src[b], its kept count pos_count[b] and its tile order[b] in one round trip); otherwise
// src = proj and the slots from idx / valid of tile order[b].
// LDS: the staged slots (theta0..3, colour, theta4..5: 40 bytes each), reused afterwards for
// the join of the four waves' sums (4 waves x 4 rows x 64 lanes x float4 = 16 KB).
inline size_t fwd_tile_lds(int K) {
  const int k4 = (K + 3) & ~3;
  const size_t a = (size_t)k4 * 40, r = 16 * 64 * sizeof(float4);
  return a > r ? a : r;
}
template <bool REC>
__global__ __launch_bounds__(256) void k_splat_fwd_tile(
    const float* __restrict__ src, const int32_t* __restrict__ idx,
    const uint8_t* __restrict__ valid, const int32_t* __restrict__ pos_count,
    const int32_t* __restrict__ order, int ntx, int W, int K, float inv_k,
    const float* __restrict__ bg, float* __restrict__ image, float* __restrict__ den_out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
  __shared__ int s_hi[2][4];
  const int k4 = (K + 3) & ~3;
  float4* s_th = reinterpret_cast<float4*>(s_dyn);         // [k4]: theta0..3
  float4* s_col = s_th + k4;                               // [k4]: col_o r, g, b, o_col
  float2* s_th2 = reinterpret_cast<float2*>(s_col + k4);   // [k4]: theta4, theta5
  const int t = order ? order[blockIdx.x] : blockIdx.x;
  const int nb = REC ? min(pos_count[blockIdx.x], K) : 0;
  const int tx = t % ntx, ty = t / ntx;
  const int ox = tx * 16, oy = ty * 16;
  const float oxf = (float)ox, oyf = (float)oy;
  // the wave index is uniform: read it into a scalar register so the walk's slot loop is scalar
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  bool bad = false;
  // slot s's coefficients go to LDS entry s (zero for an invalid slot)
  auto stage = [&](int s, int v, const float4& r0, const float4& r1, const float4& r2) {
    if (s >= k4) return;
    if (v) {
      float4 ta, tb, cl;
      slot_from_rec(r0, r1, r2, oxf, oyf, inv_k, ta, tb, cl);
      bad = bad || theta_wild(ta, tb);
      s_th[s] = ta;
      s_th2[s] = make_float2(tb.x, tb.y);
      // a quarter of the colour: the fast walk's weight is (2 relu(u))^2 = 4 w
      s_col[s] = make_float4(0.25f * cl.x, 0.25f * cl.y, 0.25f * cl.z, 0.25f * cl.w);
    } else {
      s_th[s] = make_float4(0.f, 0.f, 0.f, 0.f);
      s_th2[s] = make_float2(0.f, 0.f);
      s_col[s] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  // g: the gaussian (from idx), or with REC the slot of this block's records
  auto gather = [&](int g, float4& r0, float4& r1, float4& r2) {
    const int64_t row = REC ? (int64_t)blockIdx.x * K + g : (int64_t)g;
    const float4* r = reinterpret_cast<const float4*>(src + row * 12);
    r0 = r[0];
    r1 = r[1];
    r2 = r[2];
  };
  // the first 256 slots, one per thread: valid and idx together; the highest valid slot of
  // each wave's 64 (slot order = LDS order, so the walk needs no compaction)
  const int s = threadIdx.x;
  int v, g;
  if constexpr (REC) {
    g = min(s, K - 1);
    v = s < nb ? 1 : 0;
  } else {
    const int64_t ts = (int64_t)t * K + min(s, K - 1);
    const uint8_t vb = valid[ts];
    g = idx[ts];
    v = (s < K && vb != 0) ? 1 : 0;
    const uint64_t m = __ballot(v);
    if (lane == 0) s_hi[0][wave] = m ? wave * 64 + 64 - __clzll((long long)m) : 0;
  }
  // slots 0..63 (wave 0) are staged and walked first; the records of the other slots are
  // requested only then, so the first walk's gathers are not queued behind theirs and the rest
  // arrive during that walk
  float4 r0, r1, r2;
  if (wave == 0) {
    // records are read whether kept or not (in flight beside pos_count; a slot past the count
    // is staged as zero)
    if (v || REC) gather(g, r0, r1, r2);
    stage(s, v, r0, r1, r2);
  }
  // a wild slot (theta_wild) among slots 0..63: that walk uses relu_nan (a NaN or mixed-
  // infinity theta then makes u NaN at every pixel, so the tile comes out NaN)
  const bool wild0 = __syncthreads_or(bad);
  const int n0 = REC ? min(nb, 256)
                     : max(max(s_hi[0][0], s_hi[0][1]), max(s_hi[0][2], s_hi[0][3]));
  const bool more = n0 > 64 || k4 > 256;
  if (more && wave > 0 && v) gather(g, r0, r1, r2);

  const int j = lane & 15, q = lane >> 4;
  const float lx = (float)j + 0.5f, lyq = (float)q + 0.5f;
  float acc[4][4];
#pragma unroll
  for (int m = 0; m < 4; ++m) acc[m][0] = acc[m][1] = acc[m][2] = acc[m][3] = 0.f;
  auto walk = [&](auto exact, int s0, int s1) {
#pragma unroll 2
    for (int sl = s0 + wave; sl < s1; sl += 4) {
      const float4 th = s_th[sl];
      const float2 th2 = s_th2[sl];
      float4 cl = s_col[sl];
      if constexpr (decltype(exact)::value) {  // w itself, with the staged quarter undone
        cl.x *= 4.f;
        cl.y *= 4.f;
        cl.z *= 4.f;
        cl.w *= 4.f;
      }
      const float P = fmaf(th.z, lx, th2.x);
      const float Q = fmaf(fmaf(th.x, lx, th.w), lx, th2.y);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float ly = lyq + (float)(4 * m);
        const float u = fmaf(fmaf(th.y, ly, P), ly, Q);
        // fast: 2 relu(u) = u + |u| (one full-rate add; a max issues at half rate), exact for
        // the finite u of a tile without a wild slot; wild: relu with torch's NaN rule
        const float rl = decltype(exact)::value ? relu_nan(u) : u + fabsf(u);
        const float w = rl * rl;
        acc[m][0] += w * cl.x;
        acc[m][1] += w * cl.y;
        acc[m][2] += w * cl.z;
        acc[m][3] += w * cl.w;
      }
    }
  };
  if (wild0)
    walk(std::true_type{}, 0, min(n0, 64));
  else
    walk(std::false_type{}, 0, min(n0, 64));
  if (more) {
    if (wave > 0) stage(s, v, r0, r1, r2);
    int hi = 0;
    for (int s0 = 256; s0 < k4; s0 += 256) {
      const int s2 = s0 + threadIdx.x;
      int v2, g2;
      if constexpr (REC) {
        g2 = min(s2, K - 1);
        v2 = s2 < nb ? 1 : 0;
      } else {
        const int64_t ts = (int64_t)t * K + min(s2, K - 1);
        const uint8_t vb = valid[ts];
        g2 = idx[ts];
        v2 = (s2 < K && vb != 0) ? 1 : 0;
      }
      float4 q0, q1, q2;
      if (v2) gather(g2, q0, q1, q2);
      stage(s2, v2, q0, q1, q2);
      const uint64_t m = __ballot(v2);
      if (m) hi = s0 + wave * 64 + 64 - __clzll((long long)m);
    }
    if (lane == 0) s_hi[1][wave] = hi;
    const bool wild1 = __syncthreads_or(bad);
    const int n = REC ? nb
                      : max(n0, max(max(s_hi[1][0], s_hi[1][1]), max(s_hi[1][2], s_hi[1][3])));
    if (wild1)
      walk(std::true_type{}, 64, n);
    else
      walk(std::false_type{}, 64, n);
  }
  // join the four waves' sums in wave order; the slot LDS is reused
  float4* red = reinterpret_cast<float4*>(s_dyn);
  __syncthreads();
#pragma unroll
  for (int m = 0; m < 4; ++m)
    red[(wave * 4 + m) * 64 + lane] = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
  __syncthreads();
  float4 sum = red[wave * 64 + lane];
#pragma unroll
  for (int w2 = 1; w2 < 4; ++w2) {
    const float4 o = red[(w2 * 4 + wave) * 64 + lane];
    sum.x += o.x;
    sum.y += o.y;
    sum.z += o.z;
    sum.w += o.w;
  }
  const float ar = sum.x, ag = sum.y, ab = sum.z, ad = sum.w;
  const float wb = bg[0];
  const int64_t pix = (int64_t)(oy + 4 * wave + q) * W + ox + j;
  const float d = ad + wb;
  // one hardware reciprocal per pixel (1 ulp; an IEEE division costs ~10 VALU instructions)
  const float inv = __builtin_amdgcn_rcpf(d);
  image[pix * 3 + 0] = (ar + wb * bg[1]) * inv;
  image[pix * 3 + 1] = (ag + wb * bg[2]) * inv;
  image[pix * 3 + 2] = (ab + wb * bg[3]) * inv;
  if (den_out) den_out[pix] = d;
}

__global__ __launch_bounds__(256) void k_theta_gather(const float* __restrict__ proj,
                                                      const int32_t* __restrict__ idx,
                                                      const uint8_t* __restrict__ valid, int ntx,
                                                      int S, int K, float inv_k,
                                                      float* __restrict__ theta,
                                                      float* __restrict__ col,
                                                      float* __restrict__ oc) {
  const int t = blockIdx.x;
  const int tx = t % ntx, ty = t / ntx;
  const float ox = (float)(tx * S), oy = (float)(ty * S);
  for (int s = threadIdx.x; s < K; s += blockDim.x) {
    const int64_t ts = (int64_t)t * K + s;
    float4 ta = make_float4(0.f, 0.f, 0.f, 0.f), tb = ta, cl = ta;
    if (valid[ts]) build_slot(proj, idx[ts], ox, oy, inv_k, ta, tb, cl);
    float* th = theta + (int64_t)t * 6 * K;
    th[s] = ta.x; th[K + s] = ta.y; th[2 * K + s] = ta.z; th[3 * K + s] = ta.w;
    th[4 * K + s] = tb.x; th[5 * K + s] = tb.y;
    col[ts * 3 + 0] = cl.x; col[ts * 3 + 1] = cl.y; col[ts * 3 + 2] = cl.z;
    oc[ts] = cl.w;
  }
}

inline int check_tile(int H, int W, int S, int K) {
  if (H <= 0 || W <= 0) return TTS_EINVAL;
  if (S != 16 && S != 32) return TTS_ETILE;
  if (H % S || W % S) return TTS_ETILE;
  if (K < 1 || K > kSplatMaxK) return TTS_EK;
  return TTS_OK;
}

inline size_t fwd_lds(int K) { return slot_lds_bytes(K); }
inline size_t bwd_lds(int K, int S) {
  size_t a = slot_lds_bytes(K);
  a += (16 - a % 16) % 16;
  return a + (size_t)S * (S + 1) * 16;
}

template <bool FROM_PROJ, typename OT = float>
int launch_fwd(const float* proj, const int32_t* idx, const uint8_t* valid, const OT* theta,
               const OT* col, const OT* oc, const int32_t* order, int H, int W, int S, int K,
               float k,
               const float* bg, float* image, float* den, hipStream_t stream) {
  const int ntx = W / S, T = (H / S) * ntx;
  const float inv_k = (float)(1.0 / (double)k);
  if (S == 16 && FROM_PROJ)
    k_splat_fwd_tile<false><<<T, 256, fwd_tile_lds(K), stream>>>(
        proj, idx, valid, nullptr, order, ntx, W, K, inv_k, bg, image, den);
  else if (S == 16)
    k_splat_fwd<16, FROM_PROJ, OT><<<T, 256, fwd_lds(K), stream>>>(
        proj, idx, valid, theta, col, oc, order, ntx, W, K, inv_k, bg, image, den);
  else
    k_splat_fwd<32, FROM_PROJ, OT><<<T, 256, fwd_lds(K), stream>>>(
        proj, idx, valid, theta, col, oc, order, ntx, W, K, inv_k, bg, image, den);
  return launch_status();
}

template <bool FROM_PROJ, typename OT = float>
int launch_bwd(const float* proj, const int32_t* idx, const uint8_t* valid, const OT* theta,
               const OT* col, const OT* oc, const int32_t* order, int H, int W, int S, int K,
               float k,
               const float* bg, const float* image, const float* den, const float* gimage,
               float* gslot, float* gtheta, float* gcol, float* goc, float* gwb,
               hipStream_t stream) {
  const int ntx = W / S, T = (H / S) * ntx;
  const float inv_k = (float)(1.0 / (double)k);
  if (S == 16)
    k_splat_bwd<16, FROM_PROJ, OT><<<T, 256, bwd_lds(K, 16), stream>>>(
        proj, idx, valid, theta, col, oc, order, nullptr, ntx, W, K, inv_k, bg, image, den,
        gimage, gslot, gtheta, gcol, goc, gwb);
  else
    k_splat_bwd<32, FROM_PROJ, OT><<<T, 256, bwd_lds(K, 32), stream>>>(
        proj, idx, valid, theta, col, oc, order, nullptr, ntx, W, K, inv_k, bg, image, den,
        gimage, gslot, gtheta, gcol, goc, gwb);
  return launch_status();
}

}  // namespace tts

using namespace tts;

extern "C" {

int tts_theta_u_gathered(const float* proj, const int32_t* idx, const uint8_t* valid, int H,
                         int W, int S, int K, float k, float* theta, float* col, float* oc,
                         hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (!proj || !idx || !valid || !theta || !col || !oc) return TTS_EINVAL;
  const int ntx = W / S, T = (H / S) * ntx;
  k_theta_gather<<<T, 256, 0, stream>>>(proj, idx, valid, ntx, S, K, (float)(1.0 / (double)k),
                                        theta, col, oc);
  return launch_status();
}

int tts_splat_fwd(const float* proj, const int32_t* idx, const uint8_t* valid,
                  const int32_t* order, int H, int W, int S, int K, float k, const float* bg,
                  float* image, float* den, hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (!proj || !idx || !valid || !bg || !image) return TTS_EINVAL;
  return launch_fwd<true, float>(proj, idx, valid, nullptr, nullptr, nullptr, order, H, W, S, K, k, bg,
                          image, den, stream);
}

int tts_splat_fwd_mx(const float* proj, const int32_t* idx, const uint8_t* valid,
                     const int32_t* order, int H, int W, int S, int K, float k, const float* bg,
                     float* image, float* den, int bf16, hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (S != 16) return TTS_ETILE;
  if (!proj || !idx || !valid || !bg || !image) return TTS_EINVAL;
  const int ntx = W / S, T = (H / S) * ntx;
  const float inv_k = (float)(1.0 / (double)k);
  if (bf16)
    k_splat_fwd_mx<false, false><<<T, 256, fwd_mx_lds(K), stream>>>(
        proj, idx, valid, nullptr, order, ntx, W, K, inv_k, bg, image, den);
  else
    k_splat_fwd_mx<true, false><<<T, 256, fwd_mx_lds(K), stream>>>(
        proj, idx, valid, nullptr, order, ntx, W, K, inv_k, bg, image, den);
  return launch_status();
}

int tts_splat_fwd_theta(const float* theta, const float* col, const float* oc, int H, int W,
                        int S, int K, const float* bg, float* image, float* den,
                        hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (!theta || !col || !oc || !bg || !image) return TTS_EINVAL;
  return launch_fwd<false>(nullptr, nullptr, nullptr, theta, col, oc, nullptr, H, W, S, K, 1.0f,
                           bg, image, den, stream);
}

int tts_splat_bwd(const float* proj, const int32_t* idx, const uint8_t* valid,
                  const int32_t* order, int H, int W, int S, int K, float k, const float* bg,
                  const float* image, const float* den, const float* gimage, float* gslot,
                  float* gwb, hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (!proj || !idx || !valid || !bg || !image || !den || !gimage || !gslot) return TTS_EINVAL;
  return launch_bwd<true, float>(proj, idx, valid, nullptr, nullptr, nullptr, order, H, W, S, K, k, bg,
                          image, den, gimage, gslot, nullptr, nullptr, nullptr, gwb, stream);
}

int tts_splat_fwd_rec(const float* slot_rec, const int32_t* pos_count, const int32_t* order,
                      int H, int W, int S, int K, float k, const float* bg, float* image,
                      float* den, hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (S != 16) return TTS_ETILE;
  if (!slot_rec || !pos_count || !order || !bg || !image) return TTS_EINVAL;
  const int ntx = W / S, T = (H / S) * ntx;
  k_splat_fwd_tile<true><<<T, 256, fwd_tile_lds(K), stream>>>(
      slot_rec, nullptr, nullptr, pos_count, order, ntx, W, K, (float)(1.0 / (double)k), bg,
      image, den);
  return launch_status();
}

int tts_splat_fwd_mx_rec(const float* slot_rec, const int32_t* pos_count,
                         const int32_t* order, int H, int W, int S, int K, float k,
                         const float* bg, float* image, float* den, int bf16,
                         hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (S != 16) return TTS_ETILE;
  if (!slot_rec || !pos_count || !order || !bg || !image) return TTS_EINVAL;
  const int ntx = W / S, T = (H / S) * ntx;
  const float inv_k = (float)(1.0 / (double)k);
  if (bf16)
    k_splat_fwd_mx<false, true><<<T, 256, fwd_mx_lds(K), stream>>>(
        slot_rec, nullptr, nullptr, pos_count, order, ntx, W, K, inv_k, bg, image, den);
  else
    k_splat_fwd_mx<true, true><<<T, 256, fwd_mx_lds(K), stream>>>(
        slot_rec, nullptr, nullptr, pos_count, order, ntx, W, K, inv_k, bg, image, den);
  return launch_status();
}

int tts_splat_bwd_rec(const float* slot_rec, const int32_t* pos_count, const int32_t* order,
                      int H, int W, int S, int K, float k, const float* bg, const float* image,
                      const float* den, const float* gimage, float* gslot, float* gwb,
                      hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (S != 16) return TTS_ETILE;
  if (!slot_rec || !pos_count || !order || !bg || !image || !den || !gimage || !gslot)
    return TTS_EINVAL;
  const int ntx = W / S, T = (H / S) * ntx;
  k_splat_bwd<16, true, float, true><<<T, 256, bwd_lds(K, 16), stream>>>(
      slot_rec, nullptr, nullptr, nullptr, nullptr, nullptr, order, pos_count, ntx, W, K,
      (float)(1.0 / (double)k), bg, image, den, gimage, gslot, nullptr, nullptr, nullptr, gwb);
  return launch_status();
}

int tts_splat_bwd_theta(const float* theta, const float* col, const float* oc, int H, int W,
                        int S, int K, const float* bg, const float* image, const float* den,
                        const float* gimage, float* gtheta, float* gcol, float* goc, float* gwb,
                        hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (!theta || !col || !oc || !bg || !image || !den || !gimage || !gtheta || !gcol || !goc)
    return TTS_EINVAL;
  return launch_bwd<false>(nullptr, nullptr, nullptr, theta, col, oc, nullptr, H, W, S, K, 1.0f,
                           bg, image, den, gimage, nullptr, gtheta, gcol, goc, gwb, stream);
}

int tts_splat_fwd_theta_bf16(const uint16_t* theta, const uint16_t* col, const uint16_t* oc,
                             int H, int W, int S, int K, const float* bg, float* image,
                             float* den, hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (!theta || !col || !oc || !bg || !image) return TTS_EINVAL;
  return launch_fwd<false, __bf16>(nullptr, nullptr, nullptr,
                                   reinterpret_cast<const __bf16*>(theta),
                                   reinterpret_cast<const __bf16*>(col),
                                   reinterpret_cast<const __bf16*>(oc), nullptr, H, W, S, K, 1.0f,
                                   bg, image, den, stream);
}

int tts_splat_bwd_theta_bf16(const uint16_t* theta, const uint16_t* col, const uint16_t* oc,
                             int H, int W, int S, int K, const float* bg, const float* image,
                             const float* den, const float* gimage, float* gtheta, float* gcol,
                             float* goc, float* gwb, hipStream_t stream) {
  const int e = check_tile(H, W, S, K);
  if (e) return e;
  if (!theta || !col || !oc || !bg || !image || !den || !gimage || !gtheta || !gcol || !goc)
    return TTS_EINVAL;
  return launch_bwd<false, __bf16>(nullptr, nullptr, nullptr,
                                   reinterpret_cast<const __bf16*>(theta),
                                   reinterpret_cast<const __bf16*>(col),
                                   reinterpret_cast<const __bf16*>(oc), nullptr, H, W, S, K, 1.0f,
                                   bg, image, den, gimage, nullptr, gtheta, gcol, goc, gwb,
                                   stream);
}

}  // extern "C"
