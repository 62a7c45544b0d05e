// Fixed-budget spatial-hash binning (R = 1) in O(G + pairs), bit-exact with the reference
// order of tools/m4_train_binned.py:75-127.
//
// Passes (all stream-ordered, no host round trip):
//   1. k_bin_count   one thread per gaussian: cell = clamp(int64(floor(mu/S))), atomically
//                    count the cell and remember the gaussian's slot in it.
//   2. k_bin_scan    one block: exclusive scan of the cell counts -> cell_start[T+1]; resets
//                    the counts to zero for the next call.
//   3. k_bin_scatter one thread per gaussian: record (g, mu_x, mu_y) at its cell position.
//   4. k_bin_select  one block per tile: the tile's candidates are the records of its 3x3
//                    neighbour cells.  Each candidate has the unique 64-bit key
//                        key = qd2 << 36 | j << 32 | g,
//                    qd2 = clamp(int64(fl(fl(dx*dx) + fl(dy*dy))), 0, span-1), j the stencil
//                    index, g the gaussian id.  Ascending key order IS the reference order
//                    (its int64 sort key tile*span + qd2, ties in pair-concatenation order
//                    (j, g)).  If more than K candidates exist, an exact radix select over
//                    the key digits (qd2 | j | g in 11-bit chunks) finds the K-th smallest key
//                    with LDS histograms; the <= K survivors are bitonic-sorted in LDS.
//   The result does not depend on the order atomics land in.

#include "tts_common.h"

namespace tts {

constexpr int kMaxSpan = 8192;   // LDS histogram bins (13-bit qd2 field)
constexpr int kMaxK = 512;
constexpr int kQShift = 36;
constexpr int kJShift = 32;

__device__ __forceinline__ int cell_coord(float mu, float S, int n) {
  // clamp(int64(floor(mu / S)), 0, n - 1)   (tools/m4_train_binned.py:85-86)
  const long long c = f2i64_x86(floorf(__fdiv_rn(mu, S)));
  return static_cast<int>(c < 0 ? 0 : (c > n - 1 ? n - 1 : c));
}

__global__ __launch_bounds__(256) void k_bin_count(const float* __restrict__ mu2d, int mu_stride,
                                                   const uint8_t* __restrict__ keep,
                                                   int keep_stride, int G, int ntx, int nty,
                                                   float S, int* __restrict__ cell_cnt,
                                                   int2* __restrict__ cell_slot) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  int2 cs = make_int2(-1, 0);
  if (keep[(int64_t)g * keep_stride]) {
    const float mx = mu2d[(int64_t)g * mu_stride], my = mu2d[(int64_t)g * mu_stride + 1];
    const int c = cell_coord(my, S, nty) * ntx + cell_coord(mx, S, ntx);
    cs = make_int2(c, atomicAdd(&cell_cnt[c], 1));
  }
  cell_slot[g] = cs;
}

__global__ __launch_bounds__(1024) void k_bin_scan(int* __restrict__ cell_cnt,
                                                   int* __restrict__ cell_start, int T) {
  __shared__ int s_wave[16];
  __shared__ int s_carry;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (int base = 0; base < T; base += 1024) {
    const int i = base + threadIdx.x;
    const int v = i < T ? cell_cnt[i] : 0;
    const int incl = wave_incl_scan(v);
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    int off = s_carry;
    for (int w = 0; w < wave; ++w) off += s_wave[w];
    if (i < T) {
      cell_start[i] = off + incl - v;
      cell_cnt[i] = 0;
    }
    __syncthreads();
    if (threadIdx.x == 1023) s_carry = off + incl;
    __syncthreads();
  }
  if (threadIdx.x == 0) cell_start[T] = s_carry;
}

__global__ __launch_bounds__(256) void k_bin_scatter(const float* __restrict__ mu2d, int mu_stride,
                                                     int G, const int2* __restrict__ cell_slot,
                                                     const int* __restrict__ cell_start,
                                                     int4* __restrict__ recs) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  const int2 cs = cell_slot[g];
  if (cs.x < 0) return;
  const float mx = mu2d[(int64_t)g * mu_stride], my = mu2d[(int64_t)g * mu_stride + 1];
  recs[cell_start[cs.x] + cs.y] = make_int4(g, __float_as_int(mx), __float_as_int(my), 0);
}

struct TileCells {
  int start[9];  // first record of neighbour cell j
  int pre[10];   // prefix of candidate counts over j
};

// Candidate i of the tile (0 <= i < pre[9]) -> its 64-bit key.
__device__ __forceinline__ unsigned long long candidate_key(const TileCells& tc,
                                                            const int4* __restrict__ recs, int i,
                                                            float cx, float cy, int span) {
#pragma clang fp contract(off)
  int j = 0;
  while (i >= tc.pre[j + 1]) ++j;
  const int4 r = recs[tc.start[j] + (i - tc.pre[j])];
  // dist2 = fl(fl(dx*dx) + fl(dy*dy)), no contraction (tools/m4_train_binned.py:112-113)
  const float dx = __fsub_rn(__int_as_float(r.y), cx);
  const float dy = __fsub_rn(__int_as_float(r.z), cy);
  const float d2 = __fadd_rn(__fmul_rn(dx, dx), __fmul_rn(dy, dy));
  long long q = f2i64_x86(d2);
  q = q < 0 ? 0 : (q > span - 1 ? span - 1 : q);
  return (static_cast<unsigned long long>(q) << kQShift) |
         (static_cast<unsigned long long>(j) << kJShift) | static_cast<unsigned int>(r.x);
}

// Find the bin holding rank r in hist[0..nbins): returns bin, elements before it, its count.
// 256 threads; each sums a contiguous chunk, then one block scan.  Barriers inside.
__device__ __forceinline__ void find_rank_bin(const unsigned* hist, int nbins, int r, int* s_tmp,
                                              int* s_out) {
  const int chunk = (nbins + 255) / 256;
  const int lo = threadIdx.x * chunk, hi = min(lo + chunk, nbins);
  int sum = 0;
  for (int b = lo; b < hi; ++b) sum += hist[b];
  int total;
  int before = block_excl_scan256(sum, s_tmp, &total);
  if (r >= before && r < before + sum) {
    for (int b = lo; b < hi; ++b) {
      const int c = hist[b];
      if (r < before + c) {
        s_out[0] = b;
        s_out[1] = before;
        s_out[2] = c;
        break;
      }
      before += c;
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(256) void k_bin_select(const int4* __restrict__ recs,
                                                    const int* __restrict__ cell_start, int ntx,
                                                    int nty, float S, int span, int K, int kpow2,
                                                    int gbits, int32_t* __restrict__ idx,
                                                    uint8_t* __restrict__ valid,
                                                    int32_t* __restrict__ count,
                                                    int32_t* __restrict__ ncand) {
  extern __shared__ unsigned char s_dyn[];
  unsigned long long* s_keys = reinterpret_cast<unsigned long long*>(s_dyn);    // [kpow2]
  unsigned* s_hist = reinterpret_cast<unsigned*>(s_keys + kpow2);                // [span]
  __shared__ TileCells tc;
  __shared__ int s_tmp[4];
  __shared__ int s_out[3];
  __shared__ int s_fill;

  const int t = blockIdx.x;
  const int tx = t % ntx, ty = t / ntx;
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int j = 0; j < 9; ++j) {
      const int dy = j / 3 - 1, dx = j % 3 - 1;
      const int cx = tx - dx, cy = ty - dy;  // the cell whose gaussians reach tile t via offset j
      int n = 0, st = 0;
      if (cx >= 0 && cx < ntx && cy >= 0 && cy < nty) {
        const int c = cy * ntx + cx;
        st = cell_start[c];
        n = cell_start[c + 1] - st;
      }
      tc.start[j] = st;
      tc.pre[j] = acc;
      acc += n;
    }
    tc.pre[9] = acc;
    s_fill = 0;
  }
  __syncthreads();
  const int n = tc.pre[9];
  const float cx = (static_cast<float>(tx) + 0.5f) * S;
  const float cy = (static_cast<float>(ty) + 0.5f) * S;

  // Selection: all keys whose bits above `stop` are <= those of `prefix` survive.
  unsigned long long prefix = ~0ull;
  int stop = 0;
  if (n > K) {
    prefix = 0;
    int r = K - 1;  // rank of the K-th smallest key inside the current prefix group
    int shifts[8], widths[8], nlev = 0;
    shifts[nlev] = kQShift; widths[nlev] = 13; ++nlev;
    shifts[nlev] = kJShift; widths[nlev] = 4; ++nlev;
    for (int sh = gbits; sh > 0;) {
      const int w = sh < 11 ? sh : 11;
      sh -= w;
      shifts[nlev] = sh; widths[nlev] = w; ++nlev;
    }
    for (int lev = 0; lev < nlev; ++lev) {
      const int sh = shifts[lev], w = widths[lev];
      const int nb = (lev == 0) ? span : (1 << w);
      const int hi = sh + w;
      for (int b = threadIdx.x; b < nb; b += blockDim.x) s_hist[b] = 0;
      __syncthreads();
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const unsigned long long key = candidate_key(tc, recs, i, cx, cy, span);
        if ((key >> hi) == (prefix >> hi))
          atomicAdd(&s_hist[(key >> sh) & ((1ull << w) - 1)], 1u);
      }
      __syncthreads();
      find_rank_bin(s_hist, nb, r, s_tmp, s_out);
      const int b = s_out[0], before = s_out[1], cnt = s_out[2];
      prefix |= static_cast<unsigned long long>(b) << sh;
      r -= before;
      stop = sh;
      if (r == cnt - 1) break;  // the K-th key is the largest of this bin: take the whole bin
    }
  }
  // Collect the survivors (exactly min(n, K) keys) in LDS.
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const unsigned long long key = candidate_key(tc, recs, i, cx, cy, span);
    if ((key >> stop) <= (prefix >> stop)) {
      const int pos = atomicAdd(&s_fill, 1);
      if (pos < kpow2) s_keys[pos] = key;
    }
  }
  __syncthreads();
  const int m = min(s_fill, K);
  for (int i = m + threadIdx.x; i < kpow2; i += blockDim.x) s_keys[i] = ~0ull;
  __syncthreads();
  // Bitonic sort of kpow2 keys, ascending.
  for (int size = 2; size <= kpow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < kpow2 / 2; i += blockDim.x) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const unsigned long long a = s_keys[lo], b = s_keys[hi];
        if ((a > b) == up) {
          s_keys[lo] = b;
          s_keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  const int64_t base = static_cast<int64_t>(t) * K;
  for (int s = threadIdx.x; s < K; s += blockDim.x) {
    const bool v = s < m;
    idx[base + s] = v ? static_cast<int32_t>(s_keys[s] & 0xffffffffull) : 0;
    valid[base + s] = v ? 1 : 0;
  }
  if (threadIdx.x == 0) {
    if (count) count[t] = m;
    if (ncand) ncand[t] = n;
  }
}

struct BinWorkspace {
  int* cell_cnt;    // [T]   zero between calls
  int* cell_start;  // [T+1]
  int2* cell_slot;  // [G]
  int4* recs;       // [G]
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline size_t bin_ws_layout(int G, int T, char* base, BinWorkspace* ws) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  char* a = take(sizeof(int) * (size_t)T);
  char* b = take(sizeof(int) * ((size_t)T + 1));
  char* c = take(sizeof(int2) * (size_t)(G > 0 ? G : 1));
  char* d = take(sizeof(int4) * (size_t)(G > 0 ? G : 1));
  if (ws) {
    ws->cell_cnt = reinterpret_cast<int*>(a);
    ws->cell_start = reinterpret_cast<int*>(b);
    ws->cell_slot = reinterpret_cast<int2*>(c);
    ws->recs = reinterpret_cast<int4*>(d);
  }
  return off;
}

}  // namespace tts

using namespace tts;

extern "C" {

size_t tts_bin_workspace_bytes(int G, int H, int W, int S) {
  if (G < 0 || S <= 0 || H <= 0 || W <= 0) return 0;
  const int T = (H / S) * (W / S);
  return bin_ws_layout(G, T, nullptr, nullptr);
}

int tts_assign_bins(const float* mu2d, int mu_stride, const uint8_t* keep, int keep_stride,
                    int G, int H, int W, int S, int R, int K, int span, int32_t* idx,
                    uint8_t* valid, int32_t* count, int32_t* ncand, void* workspace,
                    size_t workspace_bytes, hipStream_t stream) {
  if (G < 0 || H <= 0 || W <= 0 || !idx || !valid) return TTS_EINVAL;
  if (G > 0 && (!mu2d || !keep || mu_stride < 2 || keep_stride < 1)) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (S != 16 && S != 32) return TTS_ETILE;
  if (H % S || W % S) return TTS_ETILE;
  if (R != 1) return TTS_ERADIUS;
  if (K < 1 || K > kMaxK) return TTS_EK;
  if (span < 1 || span > kMaxSpan) return TTS_ESPAN;
  const int ntx = W / S, nty = H / S, T = ntx * nty;
  if (!workspace || workspace_bytes < bin_ws_layout(G, T, nullptr, nullptr)) return TTS_EWORKSPACE;
  BinWorkspace ws;
  bin_ws_layout(G, T, static_cast<char*>(workspace), &ws);
  const float Sf = static_cast<float>(S);
  if (G > 0) {
    k_bin_count<<<grid1d(G, 256), 256, 0, stream>>>(mu2d, mu_stride, keep, keep_stride, G, ntx,
                                                    nty, Sf, ws.cell_cnt, ws.cell_slot);
  }
  k_bin_scan<<<1, 1024, 0, stream>>>(ws.cell_cnt, ws.cell_start, T);
  if (G > 0) {
    k_bin_scatter<<<grid1d(G, 256), 256, 0, stream>>>(mu2d, mu_stride, G, ws.cell_slot,
                                                      ws.cell_start, ws.recs);
  }
  int kpow2 = 1;
  while (kpow2 < K) kpow2 <<= 1;
  int gbits = 1;
  while ((1ll << gbits) < (long long)(G > 1 ? G : 2)) ++gbits;
  const size_t lds = sizeof(unsigned long long) * kpow2 + sizeof(unsigned) * (size_t)span;
  k_bin_select<<<T, 256, lds, stream>>>(ws.recs, ws.cell_start, ntx, nty, Sf, span, K, kpow2,
                                        gbits, idx, valid, count, ncand);
  return launch_status();
}

}  // extern "C"
