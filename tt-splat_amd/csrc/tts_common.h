// Shared device helpers for the ttsplat HIP library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ttsplat.h"

namespace tts {

constexpr float kC0 = 0.28209479177387814f;  // SH degree-0 constant
constexpr int kBlock = 256;                   // threads per block for tile kernels

// Launch-error check used by every entry point after its last launch.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TTS_OK : static_cast<int>(e);
}

inline int grid1d(int64_t n, int block) { return static_cast<int>((n + block - 1) / block); }

// Workspace sub-buffers start on 256-byte boundaries.
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// float -> int64 with x86 cvttss2si semantics: NaN and |f| >= 2^63 give INT64_MIN.
// (PyTorch-CPU's Tensor.long() behaves so; the binning keys depend on it for saturated and
// non-finite distances.)
__device__ __forceinline__ long long f2i64_x86(float f) {
  if (!(f > -9.223372036854775808e18f && f < 9.223372036854775808e18f))
    return static_cast<long long>(0x8000000000000000ull);
  return static_cast<long long>(f);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// Adam step block: step[0] int32 step number; step[1..2] fp32 1/bc1 and 1/sqrt(bc2) for that
// step (double-precision powers, as torch.optim.Adam's host-side bias corrections).  One thread.
__device__ __forceinline__ void advance_step(int32_t* step, float b1, float b2) {
  const int t = step[0] + 1;
  step[0] = t;
  const double bc1 = 1.0 - pow((double)b1, (double)t);
  const double bc2 = 1.0 - pow((double)b2, (double)t);
  float* f = reinterpret_cast<float*>(step);
  f[1] = (float)(1.0 / bc1);
  f[2] = (float)(1.0 / sqrt(bc2));
}

// relu with torch's NaN rule (torch.relu and clamp(min=0) keep a NaN):
//   relu_nan: u <= 0 -> +0, else u; a NaN of either sign fails the compare and passes through.
//   relu_bits: one integer max on the bit pattern.  Equal to relu_nan for every u except a NaN
//   with the sign bit set, which it maps to +0 -- and the NaN the GPU generates (inf - inf) can
//   carry the sign bit.  The splat kernels use it only where u is finite: the forward walks of
//   tiles without a wild slot (theta_wild), and the backward, whose tiles with a NaN u have a NaN
//   den from the forward, so every gradient of such a tile is NaN whatever relu gives.
__device__ __forceinline__ float relu_nan(float u) { return u <= 0.0f ? 0.0f : u; }
__device__ __forceinline__ float relu_bits(float u) {
  return __int_as_float(max(__float_as_int(u), 0));
}

// Wave64 inclusive prefix sum of an int, on DPP lane moves (VALU only; a shuffle would take six
// dependent LDS-crossbar round trips): Hillis-Steele inside each row of 16 lanes (row_shr 1, 2,
// 4, 8, lanes shifted in from outside the row read 0), then lane 15 of rows 0 and 2 is added
// into rows 1 and 3 (row_bcast:15) and lane 31 into rows 2 and 3 (row_bcast:31).  DPP reads
// the neighbour lanes' registers whatever their exec bit: all 64 lanes of the wave must call.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// Block-wide exclusive prefix sum for blockDim.x == NT (NT/64 waves).  `tmp` holds NT/64 ints.
// Returns the exclusive prefix of `v`; *total receives the block sum.  Contains barriers:
// every thread of the block must call it.
template <int NT>
__device__ __forceinline__ int block_excl_scan(int v, int* tmp, int* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = wave_incl_scan(v);
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    int tw = tmp[w];
    if (w < wave) base += tw;
    sum += tw;
  }
  __syncthreads();
  *total = sum;
  return base + incl - v;
}

// Two independent block-wide exclusive prefix sums under one pair of barriers.  `tmp` holds
// 2 * NT/64 ints.
template <int NT>
__device__ __forceinline__ void block_excl_scan2(int a, int b, int* tmp, int* ea, int* eb,
                                                 int* ta, int* tb) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ia = wave_incl_scan(a), ib = wave_incl_scan(b);
  if (lane == 63) {
    tmp[wave] = ia;
    tmp[NW + wave] = ib;
  }
  __syncthreads();
  int ba = 0, bb = 0, sa = 0, sb = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int xa = tmp[w], xb = tmp[NW + w];
    if (w < wave) {
      ba += xa;
      bb += xb;
    }
    sa += xa;
    sb += xb;
  }
  __syncthreads();
  *ea = ba + ia - a;
  *eb = bb + ib - b;
  *ta = sa;
  *tb = sb;
}

__device__ __forceinline__ int block_excl_scan256(int v, int* tmp, int* total) {
  return block_excl_scan<256>(v, tmp, total);
}

// MI355X dispatches the workgroups of a 1-D grid round-robin over its 8 XCDs, each with its own
// L2.  xcd_item(p, n) renumbers physical block p of n so that every XCD takes one contiguous run
// of work items (XCD x gets items [x*per + min(x, extra), ...), per = n / 8, extra = n % 8): work
// items that share input lines (neighbouring image tiles, the channels of one tile) then meet in
// the same L2.  A bijection on [0, n) for any n.
constexpr int kNumXcd = 8;
__device__ __forceinline__ int xcd_item(int p, int n) {
  const int per = n / kNumXcd, extra = n % kNumXcd;
  const int x = p % kNumXcd, k = p / kNumXcd;
  return x * per + min(x, extra) + k;
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): a counter-based generator, four 32-bit
// words per (counter, key), no state to carry between calls or graph replays.
struct Philox4 {
  uint32_t w[4];
};
__device__ __forceinline__ Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2,
                                                 uint32_t c3, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return {{c0, c1, c2, c3}};
}

// Stream tags (counter word 2) of the MCMC draws; counter = (index, step, tag, 0), key = (seed, 0).
constexpr uint32_t kTagSgld = 1, kTagRelocPick = 2, kTagRelocOffset = 3;
// Random training backgrounds: counter = (view, step, kTagBg, 0), key = (seed, 0).
constexpr uint32_t kTagBg = 4;

// Uniform in (0, 1) from the top 24 bits: ((x >> 8) + 0.5) * 2^-24 (exact in double).
__device__ __forceinline__ double u01d(uint32_t x) {
  return ((double)(x >> 8) + 0.5) * 5.9604644775390625e-08;
}

// Three standard normals (Box-Muller on words 0,1 and 2,3; the fourth value is unused).
__device__ __forceinline__ void normals3(const Philox4& p, float* z) {
  const float u0 = (float)u01d(p.w[0]), u1 = (float)u01d(p.w[1]);
  const float u2 = (float)u01d(p.w[2]), u3 = (float)u01d(p.w[3]);
  const float r0 = sqrtf(-2.0f * logf(u0)), r1 = sqrtf(-2.0f * logf(u2));
  float s0, c0, s1, c1;
  sincosf(6.283185307179586f * u1, &s0, &c0);
  sincosf(6.283185307179586f * u3, &s1, &c1);
  z[0] = r0 * c0;
  z[1] = r0 * s0;
  z[2] = r1 * c1;
}

// Wave64 float sum on the DPP pattern of wave_incl_scan (lane 63 ends with the total, a fixed
// summation order), broadcast from lane 63.  All 64 lanes of the wave must call.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false);
  return v + __builtin_bit_cast(float, o);
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0x111, 0xf>(v);  // row_shr:1
  v = dpp_add<0x112, 0xf>(v);  // row_shr:2
  v = dpp_add<0x114, 0xf>(v);  // row_shr:4
  v = dpp_add<0x118, 0xf>(v);  // row_shr:8
  v = dpp_add<0x142, 0xa>(v);  // row_bcast:15
  v = dpp_add<0x143, 0xc>(v);  // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Block-wide float sum for blockDim.x == 256; result valid in every thread.
__device__ __forceinline__ float block_sum256(float v, float* tmp) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) tmp[wave] = v;
  __syncthreads();
  float s = tmp[0] + tmp[1] + tmp[2] + tmp[3];
  __syncthreads();
  return s;
}

// Camera block as stored in device memory (16 floats).
struct Camera {
  float R[9];
  float t[3];
  float fx, fy, cx, cy;
};

}  // namespace tts
