// Fixed-count MCMC relocation on the device (spike/mcmc.py:41-93; the reference runs it on the
// host between device steps, tools/resident_traced.py:631-663): dead slots (sigmoid(op) < thr)
// copy a live gaussian drawn with probability proportional to its opacity, the target's
// opacity is split o -> o / (n + 1) over itself and its n copies (which leaves a WSR render
// unchanged), and the Adam moments of every touched slot are zeroed.
//
// Six kernels, no host synchronisation, fixed grids (graph-capturable whatever the dead count):
//   k_reloc_count   per 256-gaussian block: dead / live counts and live opacity sum; zero the
//                   per-gaussian copy counts
//   k_reloc_scan    one block: exclusive scans of the block totals (opacity sums in double)
//   k_reloc_lists   dead list and live list in ascending index order, the live opacity CDF
//   k_reloc_pick    per dead slot i: u from Philox (i, step, pick tag), target = first live j with
//                   CDF[j] > u * total (binary search); count[target] += 1
//   k_reloc_copy    per dead slot: copy the target with the split opacity, position offset by
//                   offset * N(0,1) (Philox normals), moments zeroed
//   k_reloc_split   per target: opacity o / (count + 1), moments zeroed
// Opacities are split with the target's opacity from before the relocation (copy runs before
// split).  Dead and live sets are disjoint, so no copy reads a slot another copy writes.

#include <math.h>

#include "tts_common.h"

namespace tts {

constexpr int kRelocBlock = 256;
constexpr int kRelocScanThreads = 1024;
constexpr int kShRows = 45;  // SH rest coefficients per gaussian (15 x 3), coefficient-major

struct RelocHeader {
  int n_dead, n_alive;
  double total;
};

struct RelocWs {
  RelocHeader* hdr;
  int* blk_dead;
  int* blk_alive;
  double* blk_w;
  int* dead_list;
  int* alive_list;
  double* cdf;
  int* target;
  int* count;
};

inline size_t reloc_layout(int G, char* base, RelocWs* ws) {
  const int nb = (G + kRelocBlock - 1) / kRelocBlock;
  const size_t g1 = (size_t)(G > 0 ? G : 1), nb1 = (size_t)(nb > 0 ? nb : 1);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  char* h = take(sizeof(RelocHeader));
  char* bd = take(sizeof(int) * nb1);
  char* ba = take(sizeof(int) * nb1);
  char* bw = take(sizeof(double) * nb1);
  char* dl = take(sizeof(int) * g1);
  char* al = take(sizeof(int) * g1);
  char* cd = take(sizeof(double) * g1);
  char* tg = take(sizeof(int) * g1);
  char* ct = take(sizeof(int) * g1);
  if (ws) {
    ws->hdr = reinterpret_cast<RelocHeader*>(h);
    ws->blk_dead = reinterpret_cast<int*>(bd);
    ws->blk_alive = reinterpret_cast<int*>(ba);
    ws->blk_w = reinterpret_cast<double*>(bw);
    ws->dead_list = reinterpret_cast<int*>(dl);
    ws->alive_list = reinterpret_cast<int*>(al);
    ws->cdf = reinterpret_cast<double*>(cd);
    ws->target = reinterpret_cast<int*>(tg);
    ws->count = reinterpret_cast<int*>(ct);
  }
  return off;
}

// Block-wide (256 threads) exclusive scans of two int flags and an inclusive scan of a double.
struct RelocScan {
  int dead_excl, alive_excl;
  double w_incl;
  int dead_tot, alive_tot;
  double w_tot;
};
__device__ __forceinline__ RelocScan reloc_block_scan(int dflag, int aflag, double w) {
  __shared__ int s_d[kRelocBlock], s_a[kRelocBlock];
  __shared__ double s_w[kRelocBlock];
  const int t = threadIdx.x;
  s_d[t] = dflag;
  s_a[t] = aflag;
  s_w[t] = w;
  __syncthreads();
  for (int o = 1; o < kRelocBlock; o <<= 1) {  // Hillis-Steele inclusive scans
    int d = 0, a = 0;
    double x = 0.0;
    if (t >= o) {
      d = s_d[t - o];
      a = s_a[t - o];
      x = s_w[t - o];
    }
    __syncthreads();
    s_d[t] += d;
    s_a[t] += a;
    s_w[t] += x;
    __syncthreads();
  }
  RelocScan r;
  r.dead_excl = s_d[t] - dflag;
  r.alive_excl = s_a[t] - aflag;
  r.w_incl = s_w[t];
  r.dead_tot = s_d[kRelocBlock - 1];
  r.alive_tot = s_a[kRelocBlock - 1];
  r.w_tot = s_w[kRelocBlock - 1];
  return r;
}

__device__ __forceinline__ void reloc_flags(const float* __restrict__ params, int G, int g,
                                            float thr, int& dead, int& alive, double& w) {
  dead = alive = 0;
  w = 0.0;
  if (g < G) {
    const float o = sigmoidf_(params[(int64_t)g * 14 + 13]);
    dead = o < thr;
    alive = !dead;
    w = alive ? (double)o : 0.0;
  }
}

__global__ __launch_bounds__(kRelocBlock) void k_reloc_count(const float* __restrict__ params,
                                                             int G, float thr, RelocWs ws) {
  const int g = blockIdx.x * kRelocBlock + threadIdx.x;
  int d, a;
  double w;
  reloc_flags(params, G, g, thr, d, a, w);
  if (g < G) ws.count[g] = 0;
  const RelocScan r = reloc_block_scan(d, a, w);
  if (threadIdx.x == 0) {
    ws.blk_dead[blockIdx.x] = r.dead_tot;
    ws.blk_alive[blockIdx.x] = r.alive_tot;
    ws.blk_w[blockIdx.x] = r.w_tot;
  }
}

// One block: block totals -> exclusive block offsets; header totals; moved count.
__global__ __launch_bounds__(kRelocScanThreads) void k_reloc_scan(int nb, RelocWs ws,
                                                                  int32_t* __restrict__ moved) {
  __shared__ int s_d[kRelocScanThreads], s_a[kRelocScanThreads];
  __shared__ double s_w[kRelocScanThreads];
  const int t = threadIdx.x;
  int cd = 0, ca = 0;
  double cw = 0.0;
  for (int base = 0; base < nb; base += kRelocScanThreads) {
    const int i = base + t;
    const int d = i < nb ? ws.blk_dead[i] : 0, a = i < nb ? ws.blk_alive[i] : 0;
    const double w = i < nb ? ws.blk_w[i] : 0.0;
    s_d[t] = d;
    s_a[t] = a;
    s_w[t] = w;
    __syncthreads();
    for (int o = 1; o < kRelocScanThreads; o <<= 1) {
      int xd = 0, xa = 0;
      double xw = 0.0;
      if (t >= o) {
        xd = s_d[t - o];
        xa = s_a[t - o];
        xw = s_w[t - o];
      }
      __syncthreads();
      s_d[t] += xd;
      s_a[t] += xa;
      s_w[t] += xw;
      __syncthreads();
    }
    if (i < nb) {
      ws.blk_dead[i] = cd + s_d[t] - d;
      ws.blk_alive[i] = ca + s_a[t] - a;
      ws.blk_w[i] = cw + (s_w[t] - w);
    }
    cd += s_d[kRelocScanThreads - 1];
    ca += s_a[kRelocScanThreads - 1];
    cw += s_w[kRelocScanThreads - 1];
    __syncthreads();
  }
  if (t == 0) {
    ws.hdr->n_dead = cd;
    ws.hdr->n_alive = ca;
    ws.hdr->total = cw;
    if (moved) moved[0] = ca > 0 ? cd : 0;
  }
}

__global__ __launch_bounds__(kRelocBlock) void k_reloc_lists(const float* __restrict__ params,
                                                             int G, float thr, RelocWs ws) {
  const int g = blockIdx.x * kRelocBlock + threadIdx.x;
  int d, a;
  double w;
  reloc_flags(params, G, g, thr, d, a, w);
  const RelocScan r = reloc_block_scan(d, a, w);
  if (d) ws.dead_list[ws.blk_dead[blockIdx.x] + r.dead_excl] = g;
  if (a) {
    const int j = ws.blk_alive[blockIdx.x] + r.alive_excl;
    ws.alive_list[j] = g;
    ws.cdf[j] = ws.blk_w[blockIdx.x] + r.w_incl;
  }
}

__global__ __launch_bounds__(256) void k_reloc_pick(int G, uint32_t seed,
                                                    const int32_t* __restrict__ step,
                                                    RelocWs ws) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int nd = ws.hdr->n_dead, na = ws.hdr->n_alive;
  if (i >= nd || na == 0 || i >= G) return;
  const Philox4 r = philox4x32_10((uint32_t)i, (uint32_t)step[0], kTagRelocPick, 0u, seed, 0u);
  const double x = u01d(r.w[0]) * ws.hdr->total;
  int lo = 0, hi = na - 1;  // first j with cdf[j] > x (the last one if none)
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (ws.cdf[mid] > x) hi = mid;
    else lo = mid + 1;
  }
  const int t = ws.alive_list[lo];
  ws.target[i] = t;
  atomicAdd(ws.count + t, 1);
}

__device__ __forceinline__ float split_logit(float op, int c) {
  const float o = sigmoidf_(op);
  const float n = fminf(fmaxf(o / (float)(c + 1), 1e-6f), 1.0f - 1e-6f);
  return logf(n / (1.0f - n));
}

__global__ __launch_bounds__(256) void k_reloc_copy(float* __restrict__ params,
                                                    float* __restrict__ m, float* __restrict__ v,
                                                    float* __restrict__ rest,
                                                    float* __restrict__ rest_m,
                                                    float* __restrict__ rest_v, int G,
                                                    float offset, uint32_t seed,
                                                    const int32_t* __restrict__ step,
                                                    RelocWs ws) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int nd = ws.hdr->n_dead, na = ws.hdr->n_alive;
  if (i >= nd || na == 0 || i >= G) return;
  const int d = ws.dead_list[i], t = ws.target[i];
  float src[14];
#pragma unroll
  for (int k = 0; k < 14; ++k) src[k] = params[(int64_t)t * 14 + k];
  float z[3];
  normals3(philox4x32_10((uint32_t)i, (uint32_t)step[0], kTagRelocOffset, 0u, seed, 0u), z);
#pragma unroll
  for (int k = 0; k < 3; ++k) src[k] += offset * z[k];
  src[13] = split_logit(src[13], ws.count[t]);
#pragma unroll
  for (int k = 0; k < 14; ++k) {
    params[(int64_t)d * 14 + k] = src[k];
    m[(int64_t)d * 14 + k] = 0.0f;
    v[(int64_t)d * 14 + k] = 0.0f;
  }
  if (rest) {
    for (int r = 0; r < kShRows; ++r) {
      rest[(int64_t)r * G + d] = rest[(int64_t)r * G + t];
      rest_m[(int64_t)r * G + d] = 0.0f;
      rest_v[(int64_t)r * G + d] = 0.0f;
    }
  }
}

__global__ __launch_bounds__(256) void k_reloc_split(float* __restrict__ params,
                                                     float* __restrict__ m, float* __restrict__ v,
                                                     float* __restrict__ rest_m,
                                                     float* __restrict__ rest_v, int G,
                                                     RelocWs ws) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= G) return;
  const int c = ws.count[g];
  if (c == 0) return;
  params[(int64_t)g * 14 + 13] = split_logit(params[(int64_t)g * 14 + 13], c);
#pragma unroll
  for (int k = 0; k < 14; ++k) {
    m[(int64_t)g * 14 + k] = 0.0f;
    v[(int64_t)g * 14 + k] = 0.0f;
  }
  if (rest_m) {
    for (int r = 0; r < kShRows; ++r) {
      rest_m[(int64_t)r * G + g] = 0.0f;
      rest_v[(int64_t)r * G + g] = 0.0f;
    }
  }
}

}  // namespace tts

using namespace tts;

extern "C" {

size_t tts_relocate_workspace_bytes(int G) {
  if (G < 0) return 0;
  return reloc_layout(G, nullptr, nullptr);
}

int tts_relocate(float* params, float* m, float* v, float* sh_rest, float* sh_m, float* sh_v,
                 int G, float dead_thr, float offset, uint32_t seed, const int32_t* step,
                 int32_t* moved, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (G < 0 || (G > 0 && (!params || !m || !v || !step))) return TTS_EINVAL;
  if (sh_rest && (!sh_m || !sh_v)) return TTS_EINVAL;
  if (!(dead_thr > 0.0f && dead_thr < 1.0f) || !(offset >= 0.0f)) return TTS_EINVAL;
  if (G >= (1 << 30)) return TTS_EG;
  if (!workspace || workspace_bytes < reloc_layout(G, nullptr, nullptr)) return TTS_EWORKSPACE;
  if (G == 0) return TTS_OK;
  RelocWs ws;
  reloc_layout(G, static_cast<char*>(workspace), &ws);
  const int nb = (G + kRelocBlock - 1) / kRelocBlock;
  k_reloc_count<<<nb, kRelocBlock, 0, stream>>>(params, G, dead_thr, ws);
  k_reloc_scan<<<1, kRelocScanThreads, 0, stream>>>(nb, ws, moved);
  k_reloc_lists<<<nb, kRelocBlock, 0, stream>>>(params, G, dead_thr, ws);
  const int ng = grid1d(G, 256);
  k_reloc_pick<<<ng, 256, 0, stream>>>(G, seed, step, ws);
  k_reloc_copy<<<ng, 256, 0, stream>>>(params, m, v, sh_rest, sh_m, sh_v, G, offset, seed, step,
                                       ws);
  k_reloc_split<<<ng, 256, 0, stream>>>(params, m, v, sh_rest ? sh_m : nullptr,
                                        sh_rest ? sh_v : nullptr, G, ws);
  return launch_status();
}

}  // extern "C"
