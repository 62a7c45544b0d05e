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

// Same result as k_bin_count, with the cell histogram privatised in LDS: clustered scenes put
// thousands of gaussians in one cell, and the global atomics of k_bin_count serialise there.
// Each block counts kCountPerThread gaussians per thread into LDS, then adds each non-zero cell
// count to the global histogram once, and hands every gaussian (global base + LDS rank).
constexpr int kCountPerThread = 8;
constexpr int kMaxLdsCells = 12288;

__global__ __launch_bounds__(256) void k_bin_count_lds(const float* __restrict__ mu2d,
                                                       int mu_stride,
                                                       const uint8_t* __restrict__ keep,
                                                       int keep_stride, int G, int ntx, int nty,
                                                       float S, int* __restrict__ cell_cnt,
                                                       int2* __restrict__ cell_slot) {
  extern __shared__ int s_cells[];  // [T]
  const int T = ntx * nty;
  for (int c = threadIdx.x; c < T; c += blockDim.x) s_cells[c] = 0;
  __syncthreads();
  const int g0 = blockIdx.x * blockDim.x * kCountPerThread + threadIdx.x;
  int cell[kCountPerThread], rank[kCountPerThread];
#pragma unroll
  for (int i = 0; i < kCountPerThread; ++i) {
    const int g = g0 + i * blockDim.x;
    cell[i] = -1;
    rank[i] = 0;
    if (g < G && keep[(int64_t)g * keep_stride]) {
      const float mx = mu2d[(int64_t)g * mu_stride], my = mu2d[(int64_t)g * mu_stride + 1];
      cell[i] = cell_coord(my, S, nty) * ntx + cell_coord(mx, S, ntx);
      rank[i] = atomicAdd(&s_cells[cell[i]], 1);
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < T; c += blockDim.x) {
    const int h = s_cells[c];
    if (h) s_cells[c] = atomicAdd(&cell_cnt[c], h);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kCountPerThread; ++i) {
    const int g = g0 + i * blockDim.x;
    if (g < G) cell_slot[g] = cell[i] >= 0 ? make_int2(cell[i], s_cells[cell[i]] + rank[i])
                                           : make_int2(-1, 0);
  }
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
                                                     int4* __restrict__ recs,
                                                     int32_t* __restrict__ inv) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  if (inv) {  // no slot yet: k_bin_select fills the kept (g, j) entries
#pragma unroll
    for (int j = 0; j < 9; ++j) inv[(int64_t)g * 9 + j] = -1;
  }
  const int2 cs = cell_slot[g];
  if (cs.x < 0) return;
  const float mx = mu2d[(int64_t)g * mu_stride], my = mu2d[(int64_t)g * mu_stride + 1];
  recs[cell_start[cs.x] + cs.y] = make_int4(g, __float_as_int(mx), __float_as_int(my), 0);
}

struct TileCells {
  int start[9];  // first record of the neighbour cell reaching the tile via stencil index j
  int pre[10];   // prefix of the cells' record counts over j (pre[9] = candidates)
};

// 64-bit key of one candidate record reached via stencil index j.
__device__ __forceinline__ unsigned long long make_key(int4 r, int j, float cx, float cy,
                                                       int span) {
#pragma clang fp contract(off)
  // dist2 = fl(fl(dx*dx) + fl(dy*dy)), no contraction (tools/m4_train_binned.py:112-113)
  const float dx = __fsub_rn(__int_as_float(r.y), cx);
  const float dy = __fsub_rn(__int_as_float(r.z), cy);
  const float d2 = __fadd_rn(__fmul_rn(dx, dx), __fmul_rn(dy, dy));
  long long q = f2i64_x86(d2);
  q = q < 0 ? 0 : (q > span - 1 ? span - 1 : q);
  return (static_cast<unsigned long long>(q) << kQShift) |
         (static_cast<unsigned long long>(j) << kJShift) | static_cast<unsigned int>(r.x);
}

__device__ __forceinline__ int stencil_of(const TileCells& tc, int i) {
  int j = 0;
#pragma unroll
  for (int k = 1; k < 9; ++k) j += (i >= tc.pre[k]) ? 1 : 0;
  return j;
}

__device__ __forceinline__ int4 load_candidate(const TileCells& tc, const int4* __restrict__ recs,
                                               int i, int j) {
  return recs[tc.start[j] + (i - tc.pre[j])];
}

// f(key) for every candidate of the tile, flattened over the nine cells so that all loads of a
// light tile are issued in one round, four independent loads in flight per thread.
template <int NT, typename F>
__device__ __forceinline__ void for_each_candidate(const TileCells& tc,
                                                   const int4* __restrict__ recs, float cx,
                                                   float cy, int span, F&& f) {
  const int n = tc.pre[9];
  int i = threadIdx.x;
  for (; i + 3 * NT < n; i += 4 * NT) {
    const int j0 = stencil_of(tc, i), j1 = stencil_of(tc, i + NT);
    const int j2 = stencil_of(tc, i + 2 * NT), j3 = stencil_of(tc, i + 3 * NT);
    const int4 r0 = load_candidate(tc, recs, i, j0);
    const int4 r1 = load_candidate(tc, recs, i + NT, j1);
    const int4 r2 = load_candidate(tc, recs, i + 2 * NT, j2);
    const int4 r3 = load_candidate(tc, recs, i + 3 * NT, j3);
    f(make_key(r0, j0, cx, cy, span));
    f(make_key(r1, j1, cx, cy, span));
    f(make_key(r2, j2, cx, cy, span));
    f(make_key(r3, j3, cx, cy, span));
  }
  for (; i < n; i += NT) {
    const int j = stencil_of(tc, i);
    f(make_key(load_candidate(tc, recs, i, j), j, cx, cy, span));
  }
}

// Find the bin holding rank r in hist[0..nbins): s_out = {bin, elements before it, its count}.
// Each thread sums a contiguous chunk, then one block scan.  Barriers inside.
template <int NT>
__device__ __forceinline__ void find_rank_bin(const unsigned* hist, int nbins, int r, int* s_tmp,
                                              int* s_out) {
  const int chunk = (nbins + NT - 1) / NT;
  const int lo = threadIdx.x * chunk, hi = min(lo + chunk, nbins);
  int sum = 0;
  for (int b = lo; b < hi; ++b) sum += hist[b];
  int total;
  int before = block_excl_scan<NT>(sum, s_tmp, &total);
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

// Inside one qd2 bin the key order is the order of sub = (j << gbits) | g.
__device__ __forceinline__ unsigned sub_key(unsigned long long key, int gbits) {
  return (static_cast<unsigned>(key >> kJShift) & 15u) << gbits |
         (static_cast<unsigned>(key) & ((1u << gbits) - 1u));
}

// Radix select of the rank-r sub-key among the elements visited by `visit(g)` (g(sub) is
// called for each element of the tie bin).  Returns (prefix, stop): an element survives iff
// (sub >> stop) <= (prefix >> stop); exactly r+1 elements do.  Barriers inside.
template <int NT, typename V>
__device__ __forceinline__ void select_sub(V&& visit, int r, int gbits, unsigned* s_hist,
                                           int* s_tmp, int* s_out, unsigned* prefix_out,
                                           int* stop_out) {
  unsigned prefix = 0;
  int hi = 4 + gbits, stop = hi;
  while (hi > 0) {
    const int w = hi < 11 ? hi : 11;
    const int lo = hi - w;
    const int nb = 1 << w;
    for (int b = threadIdx.x; b < nb; b += NT) s_hist[b] = 0;
    __syncthreads();
    visit([&](unsigned s) {
      if (hi >= 32 || (s >> hi) == (prefix >> hi)) atomicAdd(&s_hist[(s >> lo) & (nb - 1)], 1u);
    });
    __syncthreads();
    find_rank_bin<NT>(s_hist, nb, r, s_tmp, s_out);
    const int b = s_out[0], bef = s_out[1], c = s_out[2];
    prefix |= static_cast<unsigned>(b) << lo;
    r -= bef;
    stop = lo;
    hi = lo;
    if (r == c - 1) break;  // the wanted element is the largest of this bin: take the bin
  }
  *prefix_out = prefix;
  *stop_out = stop;
}

constexpr int kSelThreads = 512;
constexpr int kTieCap = 2048;   // tie-bin candidates kept in LDS for the sub-key select

// One block per tile.  <= K candidates: one walk collects them.  Otherwise a walk builds the LDS
// histogram of qd2, which locates the bin qb holding the K-th key; a second walk collects every
// key with qd2 < qb, and the keys of bin qb into an LDS tie buffer, where a radix select over
// (j, g) picks the needed smallest ones (a tie bin larger than the buffer, e.g. the saturated
// span-1 bin of a crowded border tile, runs the same select over further walks).  The <= K
// survivors are then placed by rank: keys are unique, so a key's slot is the number of smaller
// survivors.  A gaussian reaches a tile through exactly one stencil index j, so the inverse
// table entry inv[g][j] = t*K + slot has a single writer.
template <int NT>
__global__ __launch_bounds__(NT) void k_bin_select(const int4* __restrict__ recs,
                                                   const int* __restrict__ cell_start, int ntx,
                                                   int nty, float S, int span, int K, int kpow2,
                                                   int gbits, int32_t* __restrict__ idx,
                                                   uint8_t* __restrict__ valid,
                                                   int32_t* __restrict__ count,
                                                   int32_t* __restrict__ ncand,
                                                   int32_t* __restrict__ inv) {
  extern __shared__ unsigned char s_dyn[];
  unsigned long long* s_keys = reinterpret_cast<unsigned long long*>(s_dyn);  // [kpow2]
  unsigned long long* s_tie = s_keys + kpow2;                                 // [kTieCap]
  unsigned* s_hist = reinterpret_cast<unsigned*>(s_tie + kTieCap);            // [max(span,2048)]
  __shared__ TileCells tc;
  __shared__ int s_tmp[NT / 64];
  __shared__ int s_out[3];
  __shared__ int s_fill, s_tfill;

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
    s_tfill = 0;
  }
  __syncthreads();
  const int n = tc.pre[9];
  const float cx = (static_cast<float>(tx) + 0.5f) * S;
  const float cy = (static_cast<float>(ty) + 0.5f) * S;

  if (n <= K) {
    for_each_candidate<NT>(tc, recs, cx, cy, span, [&](unsigned long long key) {
      s_keys[atomicAdd(&s_fill, 1)] = key;
    });
  } else {
    for (int b = threadIdx.x; b < span; b += NT) s_hist[b] = 0;
    __syncthreads();
    for_each_candidate<NT>(tc, recs, cx, cy, span, [&](unsigned long long key) {
      atomicAdd(&s_hist[key >> kQShift], 1u);
    });
    __syncthreads();
    find_rank_bin<NT>(s_hist, span, K - 1, s_tmp, s_out);
    const unsigned long long qb = static_cast<unsigned long long>(s_out[0]);
    const int before = s_out[1], cnt = s_out[2];
    const int r = K - 1 - before;  // rank of the K-th key inside bin qb
    const bool in_lds = cnt <= kTieCap;
    for_each_candidate<NT>(tc, recs, cx, cy, span, [&](unsigned long long key) {
      const unsigned long long q = key >> kQShift;
      if (q < qb) s_keys[atomicAdd(&s_fill, 1)] = key;
      else if (q == qb && in_lds) s_tie[atomicAdd(&s_tfill, 1)] = key;
    });
    __syncthreads();
    unsigned prefix;
    int stop;
    if (r == cnt - 1) {  // the whole bin survives
      prefix = ~0u;
      stop = 0;
    } else if (in_lds) {
      select_sub<NT>([&](auto&& g) {
        for (int e = threadIdx.x; e < cnt; e += NT) g(sub_key(s_tie[e], gbits));
      }, r, gbits, s_hist, s_tmp, s_out, &prefix, &stop);
    } else {
      select_sub<NT>([&](auto&& g) {
        for_each_candidate<NT>(tc, recs, cx, cy, span, [&](unsigned long long key) {
          if ((key >> kQShift) == qb) g(sub_key(key, gbits));
        });
      }, r, gbits, s_hist, s_tmp, s_out, &prefix, &stop);
    }
    const unsigned thr = stop >= 32 ? 0u : (prefix >> stop);
    if (in_lds) {
      for (int e = threadIdx.x; e < cnt; e += NT) {
        const unsigned long long key = s_tie[e];
        if ((sub_key(key, gbits) >> stop) <= thr) s_keys[atomicAdd(&s_fill, 1)] = key;
      }
    } else {
      for_each_candidate<NT>(tc, recs, cx, cy, span, [&](unsigned long long key) {
        if ((key >> kQShift) == qb && (sub_key(key, gbits) >> stop) <= thr) {
          const int pos = atomicAdd(&s_fill, 1);
          if (pos < kpow2) s_keys[pos] = key;
        }
      });
    }
  }
  __syncthreads();
  // Place the m survivors by rank (unique keys: rank = number of smaller survivors).
  const int m = min(s_fill, K);
  const int64_t base = static_cast<int64_t>(t) * K;
  for (int s = threadIdx.x; s < K; s += NT) {
    if (s < m) {
      const unsigned long long key = s_keys[s];
      int rank = 0;
      for (int e = 0; e < m; ++e) rank += (s_keys[e] < key) ? 1 : 0;
      const int g = static_cast<int32_t>(key & 0xffffffffull);
      idx[base + rank] = g;
      if (inv) inv[(int64_t)g * 9 + ((key >> kJShift) & 15ull)] = static_cast<int32_t>(base + rank);
      valid[base + rank] = 1;
    } else {
      idx[base + s] = 0;
      valid[base + s] = 0;
    }
  }
  if (threadIdx.x == 0) {
    if (count) count[t] = m;
    if (ncand) ncand[t] = n;
  }
}

// Tiles by kept count, heaviest first (counting sort; ties in no particular order).  The splat
// kernels take their blocks in this order, so the dispatcher starts the expensive tiles first
// and fills the tail with cheap ones.
__global__ __launch_bounds__(1024) void k_tile_order(const int32_t* __restrict__ count, int T,
                                                     int K, int32_t* __restrict__ order) {
  __shared__ int s_bins[kMaxK + 2];
  for (int c = threadIdx.x; c <= K + 1; c += blockDim.x) s_bins[c] = 0;
  __syncthreads();
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const int c = min(max(count[t], 0), K);
    atomicAdd(&s_bins[K - c], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int c = 0; c <= K; ++c) {
      const int h = s_bins[c];
      s_bins[c] = acc;
      acc += h;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const int c = min(max(count[t], 0), K);
    order[atomicAdd(&s_bins[K - c], 1)] = t;
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
                    uint8_t* valid, int32_t* count, int32_t* ncand, int32_t* inv,
                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (G < 0 || H <= 0 || W <= 0 || !idx || !valid) return TTS_EINVAL;
  if (G > 0 && (!mu2d || !keep || mu_stride < 2 || keep_stride < 1)) return TTS_EINVAL;
  if (G > (1 << 28)) return TTS_EG;  // (j << gbits) | g must fit in 32 bits
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
  if (G > 0 && T <= kMaxLdsCells) {
    const int per_block = 256 * kCountPerThread;
    k_bin_count_lds<<<grid1d(G, per_block), 256, sizeof(int) * (size_t)T, stream>>>(
        mu2d, mu_stride, keep, keep_stride, G, ntx, nty, Sf, ws.cell_cnt, ws.cell_slot);
  } else if (G > 0) {
    k_bin_count<<<grid1d(G, 256), 256, 0, stream>>>(mu2d, mu_stride, keep, keep_stride, G, ntx,
                                                    nty, Sf, ws.cell_cnt, ws.cell_slot);
  }
  k_bin_scan<<<1, 1024, 0, stream>>>(ws.cell_cnt, ws.cell_start, T);
  if (G > 0) {
    k_bin_scatter<<<grid1d(G, 256), 256, 0, stream>>>(mu2d, mu_stride, G, ws.cell_slot,
                                                      ws.cell_start, ws.recs, inv);
  }
  int kpow2 = 1;
  while (kpow2 < K) kpow2 <<= 1;
  int gbits = 1;
  while ((1ll << gbits) < (long long)(G > 1 ? G : 2)) ++gbits;
  const size_t lds = sizeof(unsigned long long) * ((size_t)kpow2 + kTieCap) +
                     sizeof(unsigned) * (size_t)(span > 2048 ? span : 2048);
  k_bin_select<kSelThreads><<<T, kSelThreads, lds, stream>>>(
      ws.recs, ws.cell_start, ntx, nty, Sf, span, K, kpow2, gbits, idx, valid, count, ncand,
      inv);
  return launch_status();
}

int tts_tile_order(const int32_t* count, int T, int K, int32_t* order, hipStream_t stream) {
  if (T <= 0 || !count || !order) return TTS_EINVAL;
  if (K < 1 || K > kMaxK) return TTS_EK;
  k_tile_order<<<1, 1024, 0, stream>>>(count, T, K, order);
  return launch_status();
}

}  // extern "C"
