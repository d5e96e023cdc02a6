// Token-side kernels of the device-resident training loop (train.js:246-276):
//  - batch_gather: the B windows of seqLen+1 ids of one step, cut from a token
//    buffer resident in device memory at host-drawn starts (train.js:255-260);
//  - sort_*: a bitonic sort of 64-bit keys (id << 32 | position), which orders
//    the positions of equal ids by increasing position;
//  - embed_bwd_sorted: the embedding backward (tensor.js:92-98) over the
//    sorted keys, each id's row summed in increasing position onto the
//    existing gradient row — the reference's sequence of fp32 +=, with no
//    host-built plan, so a recorded graph step can replay it with new ids.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kSortThreads = 1024;
constexpr int kSortChunk = 8192;  // keys per workgroup in LDS (64 KiB)
constexpr uint64_t kNoKey = ~0ull;

// ids[b*T+i] = row[i], targets[b*T+i] = row[i+1], row[i] = data[s_b+i], or
// data[n-1] past the end (the reference's `data[s+i] ?? data[len-1]`).  A
// value outside [0,V) becomes -1 (NaN row / NaN loss downstream, as a
// reference id that indexes nothing).
__global__ void __launch_bounds__(kThreads) batch_gather_kernel(int32_t* __restrict__ ids,
                                                                int32_t* __restrict__ tgt,
                                                                const int32_t* __restrict__ data, int64_t n,
                                                                const int32_t* __restrict__ starts, int B, int T,
                                                                int V) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= (int64_t)B * T) return;
  const int b = (int)(e / T), i = (int)(e - (int64_t)b * T);
  int64_t s = starts[b];
  s = s < 0 ? 0 : (s >= n ? n - 1 : s);  // the host validates starts; never read outside data
  const int64_t k0 = s + i, k1 = s + i + 1;
  const int32_t x = data[k0 < n ? k0 : n - 1];
  const int32_t y = data[k1 < n ? k1 : n - 1];
  ids[e] = (x >= 0 && x < V) ? x : -1;
  tgt[e] = (y >= 0 && y < V) ? y : -1;
}

__device__ __forceinline__ uint64_t make_key(int32_t id, int64_t t, int V) {
  return (id >= 0 && id < V) ? (((uint64_t)(uint32_t)id) << 32) | (uint64_t)(uint32_t)t : kNoKey;
}

// Compare-exchange of the bitonic network: stage (k, j) orders the pair
// (lo, lo + j) ascending when bit k of lo is clear, descending otherwise.
__device__ __forceinline__ void cmp_swap(uint64_t& a, uint64_t& b, bool asc) {
  if ((a > b) == asc) {
    const uint64_t t = a;
    a = b;
    b = t;
  }
}

// One workgroup sorts its chunk of C keys in LDS through the stages
// k = k_lo .. k_hi (powers of two) with j < C; with init the keys are built
// from ids first (positions >= T and ids outside [0,V) get kNoKey).
__global__ void __launch_bounds__(kSortThreads) sort_lds_kernel(uint64_t* __restrict__ keys,
                                                                const int32_t* __restrict__ ids, int64_t T, int V,
                                                                int C, int64_t k_lo, int64_t k_hi, int init) {
  __shared__ uint64_t sk[kSortChunk];
  const int64_t base = (int64_t)blockIdx.x * C;
  for (int i = threadIdx.x; i < C; i += kSortThreads) {
    const int64_t g = base + i;
    sk[i] = init ? (g < T ? make_key(ids[g], g, V) : kNoKey) : keys[g];
  }
  __syncthreads();
  for (int64_t k = k_lo; k <= k_hi; k <<= 1) {
    for (int j = (int)((k < C ? k : C) >> 1); j > 0; j >>= 1) {
      for (int p = threadIdx.x; p < C / 2; p += kSortThreads) {
        const int lo = ((p & ~(j - 1)) << 1) | (p & (j - 1));
        cmp_swap(sk[lo], sk[lo + j], ((base + lo) & k) == 0);
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < C; i += kSortThreads) keys[base + i] = sk[i];
}

// One global stage (k, j) with j >= C: one thread per pair.
__global__ void __launch_bounds__(kThreads) sort_step_kernel(uint64_t* __restrict__ keys, int64_t P, int64_t k,
                                                             int64_t j) {
  const int64_t p = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (p >= P / 2) return;
  const int64_t lo = ((p & ~(j - 1)) << 1) | (p & (j - 1));
  uint64_t a = keys[lo], b = keys[lo + j];
  const uint64_t a0 = a;
  cmp_swap(a, b, (lo & k) == 0);
  if (a != a0) {
    keys[lo] = a;
    keys[lo + j] = b;
  }
}

// Workgroups stride over sorted positions; the first position of each id
// walks its run of equal ids in increasing position.  Invalid ids (kNoKey)
// sort last and end the walk.
__global__ void __launch_bounds__(kThreads) embed_bwd_sorted_kernel(float* __restrict__ gW,
                                                                    const float* __restrict__ g,
                                                                    const uint64_t* __restrict__ keys, int T,
                                                                    int V, int D, int beta) {
  for (int s = blockIdx.x; s < T; s += gridDim.x) {
    const uint64_t key = keys[s];
    if (key == kNoKey) break;
    const uint32_t id = (uint32_t)(key >> 32);
    if (id >= (uint32_t)V) break;  // keys of ids >= V (never built here) would sort after every valid one
    if (s > 0 && (uint32_t)(keys[s - 1] >> 32) == id) continue;
    float* row = gW + (int64_t)id * D;
    for (int d = threadIdx.x; d < D; d += kThreads) {
      float acc = beta ? row[d] : 0.f;
      for (int k = s; k < T; ++k) {
        const uint64_t kk = keys[k];
        if ((uint32_t)(kk >> 32) != id) break;  // kNoKey's id field is never a valid id
        acc += g[(int64_t)(uint32_t)kk * D + d];
      }
      row[d] = acc;
    }
  }
}

// The same sums for D % 4 == 0 and 16-byte aligned rows: one wave per sorted
// position, lane l holding float4 columns l, l+64, ... of the gradient row
// (every element still takes row + g[t1] + g[t2] + ... in increasing t, one
// fp32 add at a time, as above).  J float4 per lane per pass (J·64 >= the row
// width up to 1024 float4, so a row takes one pass): the row's loads and those
// of its first gradient row are issued together.  beta 0 starts each sum
// from +0 instead of reading the row (the same bits as reading a zero row).
template <int J>
__global__ void __launch_bounds__(kThreads) embed_bwd_sorted4_kernel(float* __restrict__ gW,
                                                                     const float* __restrict__ g,
                                                                     const uint64_t* __restrict__ keys, int T,
                                                                     int V, int D4, int beta) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6));
  const int nw = gridDim.x * (kThreads / 64);
  const float4* g4 = reinterpret_cast<const float4*>(g);
  for (int s = wave; s < T; s += nw) {
    const uint64_t key = keys[s];
    const uint64_t prev = s > 0 ? keys[s - 1] : kNoKey;
    if (key == kNoKey) break;
    const uint32_t id = (uint32_t)(key >> 32);
    if (id >= (uint32_t)V) break;
    if (s > 0 && (uint32_t)(prev >> 32) == id) continue;
    float4* row = reinterpret_cast<float4*>(gW) + (int64_t)id * D4;
    const float4* g0 = g4 + (int64_t)(uint32_t)key * D4;
    for (int c0 = lane; c0 < D4; c0 += 64 * J) {
      float4 acc[J], v[J];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = c0 + 64 * j < D4 ? c0 + 64 * j : c0;  // a valid column (unused past D4)
        acc[j] = beta ? row[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        v[j] = g0[c];
      }
#pragma unroll
      for (int j = 0; j < J; ++j) {
        acc[j].x += v[j].x; acc[j].y += v[j].y; acc[j].z += v[j].z; acc[j].w += v[j].w;
      }
      for (int k = s + 1; k < T; ++k) {
        const uint64_t kk = keys[k];
        if ((uint32_t)(kk >> 32) != id) break;  // kNoKey's id field is never a valid id
        const float4* gr = g4 + (int64_t)(uint32_t)kk * D4;
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const int c = c0 + 64 * j < D4 ? c0 + 64 * j : c0;
          const float4 u = gr[c];
          acc[j].x += u.x; acc[j].y += u.y; acc[j].z += u.z; acc[j].w += u.w;
        }
      }
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = c0 + 64 * j;
        if (c < D4) row[c] = acc[j];
      }
    }
  }
}

int64_t keys_len(int64_t T) {
  int64_t P = 2;
  while (P < T) P <<= 1;
  return P;
}

}  // namespace

extern "C" int fg_batch_gather(int32_t* ids, int32_t* targets, const int32_t* data, int64_t n,
                               const int32_t* starts, int B, int T, int V) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(ids && targets && data && starts && n > 0 && B > 0 && T > 0 && V > 0,
               "fg_batch_gather: bad arguments (n=%lld B=%d T=%d V=%d)", (long long)n, B, T, V);
  const int64_t total = (int64_t)B * T;
  fg::KProfScope prof("batch_gather", 0.0, 16.0 * (double)total);
  FG_LAUNCH(batch_gather_kernel, dim3((unsigned)((total + kThreads - 1) / kThreads)), dim3(kThreads), 0, ids,
            targets, data, n, starts, B, T, V);
  return FG_OK;
}

extern "C" int fg_embed_keys_len(int T, int64_t* len) {
  FG_ARG_CHECK(T > 0 && len, "fg_embed_keys_len: bad arguments");
  *len = keys_len(T);
  return FG_OK;
}

extern "C" int fg_embed_sort_keys(uint64_t* keys, int64_t len, const int32_t* ids, int T, int V) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(keys && ids && T > 0 && V > 0, "fg_embed_sort_keys: bad arguments");
  const int64_t P = keys_len(T);
  FG_ARG_CHECK(len >= P, "fg_embed_sort_keys: %lld keys given, %lld needed for T=%d", (long long)len,
               (long long)P, T);
  const int C = (int)(P < kSortChunk ? P : kSortChunk);
  const unsigned chunks = (unsigned)(P / C);
  fg::KProfScope prof("embed_sort", 0.0, 16.0 * (double)P);
  FG_LAUNCH(sort_lds_kernel, dim3(chunks), dim3(kSortThreads), 0, keys, ids, (int64_t)T, V, C, (int64_t)2,
            (int64_t)C, 1);
  for (int64_t k = 2 * (int64_t)C; k <= P; k <<= 1) {
    for (int64_t j = k >> 1; j >= C; j >>= 1)
      FG_LAUNCH(sort_step_kernel, dim3((unsigned)((P / 2 + kThreads - 1) / kThreads)), dim3(kThreads), 0, keys, P,
                k, j);
    FG_LAUNCH(sort_lds_kernel, dim3(chunks), dim3(kSortThreads), 0, keys, ids, (int64_t)T, V, C, k, k, 0);
  }
  return FG_OK;
}

extern "C" int fg_embed_bwd_sorted(float* gW, const float* g, const uint64_t* keys, int T, int V, int D,
                                   int beta) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(gW && g && keys && T > 0 && V > 0 && D > 0, "fg_embed_bwd_sorted: bad arguments");
  fg::KProfScope prof("embed_bwd", 0.0, (beta ? 12.0 : 8.0) * (double)T * D);
  if (D % 4 == 0 && (uintptr_t)gW % 16 == 0 && (uintptr_t)g % 16 == 0) {
    const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
    const int blocks = max(1, min((T + 3) / 4, 32 * cus));  // one wave per sorted position
    const int D4 = D / 4;
    if (D4 <= 64) FG_LAUNCH((embed_bwd_sorted4_kernel<1>), dim3(blocks), dim3(kThreads), 0, gW, g, keys, T, V, D4, beta);
    else if (D4 <= 256) FG_LAUNCH((embed_bwd_sorted4_kernel<4>), dim3(blocks), dim3(kThreads), 0, gW, g, keys, T, V, D4, beta);
    else if (D4 <= 512) FG_LAUNCH((embed_bwd_sorted4_kernel<8>), dim3(blocks), dim3(kThreads), 0, gW, g, keys, T, V, D4, beta);
    else FG_LAUNCH((embed_bwd_sorted4_kernel<16>), dim3(blocks), dim3(kThreads), 0, gW, g, keys, T, V, D4, beta);
    return FG_OK;
  }
  const int grid = T < 2048 ? T : 2048;
  FG_LAUNCH(embed_bwd_sorted_kernel, dim3(grid), dim3(kThreads), 0, gW, g, keys, T, V, D, beta);
  return FG_OK;
}
