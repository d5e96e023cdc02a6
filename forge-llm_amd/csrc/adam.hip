// Adam.step (autograd.js:221-243) for gfx950: global-norm clipping, L2 weight
// decay, moments and the bias-corrected update over every parameter tensor in
// three launches per step:
//   1. sqnorm: fixed-size chunks of all gradients -> fp64 partial sums
//   2. finalize: one workgroup sums the partials in a fixed order -> gnorm, scale
//   3. update: same chunks; reads scale from device memory; fp64 math, fp32 stores
// The chunk table (tensor pointers, offsets) is uploaded once and reused while
// the parameter set is unchanged.  Traffic: 4 B/param (norm) + 28 B/param
// (update: read p, g, m, v; write p, m, v).
#include "common.h"

#include <math.h>
#include <cstring>
#include <vector>

namespace {

constexpr int kThreads = 256;
constexpr int64_t kChunk = 8192;  // elements per workgroup (8 float4 per thread)

struct Chunk {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t off;  // first element of this chunk within its tensor
  int64_t len;  // elements in this chunk
};

__global__ void __launch_bounds__(kThreads) sqnorm_kernel(const Chunk* __restrict__ chunks,
                                                          double* __restrict__ part) {
  const Chunk c = chunks[blockIdx.x];
  const float* g = c.g + c.off;
  double acc = 0.0;
  const bool vec = (((uintptr_t)g) % 16 == 0);
  if (vec) {
    const int64_t n4 = c.len / 4;
    for (int64_t i = threadIdx.x; i < n4; i += kThreads) {
      const float4 v = reinterpret_cast<const float4*>(g)[i];
      acc += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    for (int64_t i = n4 * 4 + threadIdx.x; i < c.len; i += kThreads) acc += (double)g[i] * g[i];
  } else {
    for (int64_t i = threadIdx.x; i < c.len; i += kThreads) acc += (double)g[i] * g[i];
  }
  acc = fg_wave_sum_d(acc);
  __shared__ double sh[kThreads / 64];
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int i = 0; i < kThreads / 64; ++i) t += sh[i];
    part[blockIdx.x] = t;
  }
}

// stats[0] = gnorm, stats[1] = scale
__global__ void __launch_bounds__(kThreads) finalize_kernel(const double* __restrict__ part, int n, double clip,
                                                            double* __restrict__ stats) {
  // eight loads in flight, added in the same order as one at a time
  double acc = 0.0;
  int i = threadIdx.x;
  for (; i + 7 * kThreads < n; i += 8 * kThreads) {
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += v[u];
  }
  for (; i < n; i += kThreads) acc += part[i];
  acc = fg_wave_sum_d(acc);
  __shared__ double sh[kThreads / 64];
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int i = 0; i < kThreads / 64; ++i) t += sh[i];
    const double gnorm = sqrt(t);
    stats[0] = gnorm;
    stats[1] = gnorm > clip ? clip / gnorm : 1.0;
  }
}

typedef float v4f __attribute__((ext_vector_type(4)));

struct AdamHyper {
  double lr, b1, b2, eps, wd, bc1, bc2;
};

__device__ __forceinline__ void adam1(float& p, float g, float& m, float& v, double scale, const AdamHyper& h) {
#pragma clang fp contract(off)
  const double gi = (double)g * scale + h.wd * (double)p;
  m = (float)(h.b1 * (double)m + (1.0 - h.b1) * gi);
  v = (float)(h.b2 * (double)v + (1.0 - h.b2) * gi * gi);
  const double mh = (double)m / h.bc1;
  const double vh = (double)v / h.bc2;
  p = (float)((double)p - h.lr * mh / (sqrt(vh) + h.eps));
}

// sched (device, may be null) = {lr_t, bc1, bc2} replacing the by-value
// ones: the per-step values of a recorded graph step live in device memory.
__global__ void __launch_bounds__(kThreads) update_kernel(const Chunk* __restrict__ chunks,
                                                          const double* __restrict__ stats, AdamHyper h,
                                                          const double* __restrict__ sched) {
  const Chunk c = chunks[blockIdx.x];
  const double scale = stats[1];
  if (sched) {
    h.lr = sched[0];
    h.bc1 = sched[1];
    h.bc2 = sched[2];
  }
  float* p = c.p + c.off;
  const float* g = c.g + c.off;
  float* m = c.m + c.off;
  float* v = c.v + c.off;
  const bool vec = ((((uintptr_t)p) | ((uintptr_t)g) | ((uintptr_t)m) | ((uintptr_t)v)) % 16) == 0;
  int64_t done = 0;
  if (vec) {
    const int64_t n4 = c.len / 4;
    // Parameters, gradients and moments are streamed once per step and not
    // reused before the next one: nontemporal loads and stores.
    v4f* p4 = reinterpret_cast<v4f*>(p);
    const v4f* g4 = reinterpret_cast<const v4f*>(g);
    v4f* m4 = reinterpret_cast<v4f*>(m);
    v4f* v4 = reinterpret_cast<v4f*>(v);
    for (int64_t i = threadIdx.x; i < n4; i += kThreads) {
      v4f pp = __builtin_nontemporal_load(p4 + i);
      const v4f gg = __builtin_nontemporal_load(g4 + i);
      v4f mm = __builtin_nontemporal_load(m4 + i);
      v4f vv = __builtin_nontemporal_load(v4 + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pe = pp[e], me = mm[e], ve = vv[e];
        adam1(pe, gg[e], me, ve, scale, h);
        pp[e] = pe;
        mm[e] = me;
        vv[e] = ve;
      }
      __builtin_nontemporal_store(pp, p4 + i);
      __builtin_nontemporal_store(mm, m4 + i);
      __builtin_nontemporal_store(vv, v4 + i);
    }
    done = n4 * 4;
  }
  for (int64_t i = done + threadIdx.x; i < c.len; i += kThreads) {
    float pp = p[i], mm = m[i], vv = v[i];
    adam1(pp, g[i], mm, vv, scale, h);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
  }
}

// Cached device copy of the chunk table.
std::vector<Chunk> g_last;
Chunk* g_dev_chunks = nullptr;
size_t g_dev_cap = 0;
double* g_stats = nullptr;

}  // namespace

namespace {

int adam_impl(const fg_adam_tensor* tensors, int count, double lr_t, double b1, double b2, double eps, double wd,
              double clip, double bc1, double bc2, const double* sched_dev, double* stats_dev) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(count >= 0 && (count == 0 || tensors), "fg_adam_step: bad tensor list");
  FG_ARG_CHECK(sched_dev || (bc1 > 0 && bc2 > 0), "fg_adam_step: bias corrections must be positive (bc1=%g bc2=%g)",
               bc1, bc2);
  std::vector<Chunk> chunks;
  double nparams = 0;
  for (int j = 0; j < count; ++j) {
    const fg_adam_tensor& t = tensors[j];
    FG_ARG_CHECK(t.n >= 0, "fg_adam_step: tensor %d has negative size", j);
    if (t.n == 0) continue;
    FG_ARG_CHECK(t.p && t.g && t.m && t.v, "fg_adam_step: tensor %d has a null pointer", j);
    nparams += (double)t.n;
    for (int64_t off = 0; off < t.n; off += kChunk) {
      Chunk c;
      c.p = t.p; c.g = t.g; c.m = t.m; c.v = t.v;
      c.off = off;
      c.len = (t.n - off) < kChunk ? (t.n - off) : kChunk;
      chunks.push_back(c);
    }
  }
  const int nch = (int)chunks.size();
  const bool same = chunks.size() == g_last.size() &&
                    memcmp(chunks.data(), g_last.data(), chunks.size() * sizeof(Chunk)) == 0;
  // A new tensor list needs a synchronous table upload, which a graph cannot
  // record: run one step outside the capture first.
  if (nch == 0 || !same || (!stats_dev && !g_stats)) FG_NO_CAPTURE("fg_adam_step with a new tensor list");
  if (!stats_dev && !g_stats) {
    void* p = nullptr;
    FG_HIP_CHECK(hipMalloc(&p, 2 * sizeof(double)));
    g_stats = (double*)p;
  }
  double* stats = stats_dev ? stats_dev : g_stats;
  fg::KProfScope prof("adam", 0.0, 32.0 * nparams);
  if (nch == 0) {
    double z[2] = {0.0, 1.0};
    FG_HIP_CHECK(hipMemcpyAsync(stats, z, sizeof(z), hipMemcpyHostToDevice, fg::stream()));
    FG_HIP_CHECK(hipStreamSynchronize(fg::stream()));
    return FG_OK;
  }
  if (!same) {
    if ((size_t)nch > g_dev_cap) {
      FG_HIP_CHECK(hipStreamSynchronize(fg::stream()));
      if (g_dev_chunks) FG_HIP_CHECK(hipFree(g_dev_chunks));
      void* p = nullptr;
      FG_HIP_CHECK(hipMalloc(&p, sizeof(Chunk) * (size_t)nch));
      g_dev_chunks = (Chunk*)p;
      g_dev_cap = (size_t)nch;
    }
    FG_HIP_CHECK(hipMemcpyAsync(g_dev_chunks, chunks.data(), sizeof(Chunk) * (size_t)nch, hipMemcpyHostToDevice,
                                fg::stream()));
    FG_HIP_CHECK(hipStreamSynchronize(fg::stream()));
    g_last = chunks;
  }
  fg::Workspace ws;
  int rc = ws.get(sizeof(double) * (size_t)nch);
  if (rc) return rc;
  FG_LAUNCH(sqnorm_kernel, dim3(nch), dim3(kThreads), 0, g_dev_chunks, (double*)ws.ptr);
  FG_LAUNCH(finalize_kernel, dim3(1), dim3(kThreads), 0, (const double*)ws.ptr, nch, clip, stats);
  AdamHyper h;
  h.lr = lr_t; h.b1 = b1; h.b2 = b2; h.eps = eps; h.wd = wd; h.bc1 = bc1; h.bc2 = bc2;
  FG_LAUNCH(update_kernel, dim3(nch), dim3(kThreads), 0, g_dev_chunks, (const double*)stats, h, sched_dev);
  return FG_OK;
}

}  // namespace

extern "C" int fg_adam_step(const fg_adam_tensor* tensors, int count, double lr_t, double b1, double b2, double eps,
                            double wd, double clip, double bc1, double bc2, double* stats_dev) {
  return adam_impl(tensors, count, lr_t, b1, b2, eps, wd, clip, bc1, bc2, nullptr, stats_dev);
}

extern "C" int fg_adam_step_sched(const fg_adam_tensor* tensors, int count, const double* sched_dev, double b1,
                                  double b2, double eps, double wd, double clip, double* stats_dev) {
  FG_ARG_CHECK(sched_dev, "fg_adam_step_sched: null schedule pointer");
  return adam_impl(tensors, count, 0.0, b1, b2, eps, wd, clip, 0.0, 0.0, sched_dev, stats_dev);
}
