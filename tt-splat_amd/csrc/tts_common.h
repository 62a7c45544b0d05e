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

// float -> int64 with x86 cvttss2si semantics: NaN and |f| >= 2^63 give INT64_MIN.
// (PyTorch-CPU's Tensor.long() behaves so; the binning keys depend on it for saturated and
// non-finite distances.)
__device__ __forceinline__ long long f2i64_x86(float f) {
  if (!(f > -9.223372036854775808e18f && f < 9.223372036854775808e18f))
    return static_cast<long long>(0x8000000000000000ull);
  return static_cast<long long>(f);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// Wave64 inclusive prefix sum of an int.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
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
