// Adam.step (autograd.js:221-243) for gfx950: global-norm clipping, L2 weight
// decay, moments and the bias-corrected update over every parameter tensor in
// three launches per step:
//   1. sqnorm: fixed-size chunks of all gradients -> fp64 partial sums
//   2. finalize: one workgroup sums the partials in a fixed order -> gnorm, scale
//   3. update: same chunks; reads scale from device memory; fp64 math, fp32 stores
// The chunk table (tensor pointers, offsets) lives in device memory in a plan:
// one per optimizer (fg_adam_plan_*, created by its owner), or one per distinct
// tensor list for the list entry points (kept for the life of the process, so
// a recorded graph's table is never rewritten).  Traffic: 4 B/param (norm) +
// 28 B/param (update: read p, g, m, v; write p, m, v).
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

// stats = {gnorm 0, scale 1}: a step with no gradients at all.
__global__ void stats_empty_kernel(double* __restrict__ stats) {
  if (threadIdx.x == 0) {
    stats[0] = 0.0;
    stats[1] = 1.0;
  }
}

typedef float v4f __attribute__((ext_vector_type(4)));

struct AdamHyper {
  double lr, b1, b2, eps, wd, bc1, bc2;
};

// a / b for b > 0 given y = RN(1/b), correctly rounded (Markstein): q = RN(a y)
// is within one ulp of a/b, so the remainder a - b q is exact in one fma and
// RN(q + r y) = RN(a/b).  For a zero, infinite or NaN a, q itself is a / b
// (the remainder step would turn -0 into +0 and inf into NaN).  About half
// the instructions of a division by a per-element divisor, and no v_rcp_f64;
// bit-identical to the division over every fp32 significand of a against
// 9774 divisors 1 - b^t and over every fp32 bit pattern of a (zeros,
// denormals, inf and NaN included) against 24 of them (a CPU sweep).
__device__ __forceinline__ double div_by_recip(double a, double b, double y) {
  const double q = a * y;
  const double r = __builtin_fma(-b, q, a);
  const double c = __builtin_fma(r, y, q);
  return (a == 0.0 || !__builtin_isfinite(a)) ? q : c;
}

// rc1 = RN(1 / bc1), rc2 = RN(1 / bc2): the bias corrections are the same for
// every element of a step.  R = false divides (the degenerate b1 or b2 = 1,
// whose zero correction has no finite reciprocal).
template <bool R>
__device__ __forceinline__ void adam1(float& p, float g, float& m, float& v, double scale, const AdamHyper& h,
                                      double rc1, double rc2) {
#pragma clang fp contract(off)
  const double gi = (double)g * scale + h.wd * (double)p;
  m = (float)(h.b1 * (double)m + (1.0 - h.b1) * gi);
  v = (float)(h.b2 * (double)v + (1.0 - h.b2) * gi * gi);
  const double mh = R ? div_by_recip((double)m, h.bc1, rc1) : (double)m / h.bc1;
  const double vh = R ? div_by_recip((double)v, h.bc2, rc2) : (double)v / h.bc2;
  p = (float)((double)p - h.lr * mh / (sqrt(vh) + h.eps));
}

template <bool R>
__device__ __forceinline__ void update_chunk(const Chunk& c, double scale, const AdamHyper& h, double rc1,
                                             double rc2) {
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
        adam1<R>(pe, gg[e], me, ve, scale, h, rc1, rc2);
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
    adam1<R>(pp, g[i], mm, vv, scale, h, rc1, rc2);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
  }
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
  const double rc1 = 1.0 / h.bc1, rc2 = 1.0 / h.bc2;
  if (__builtin_isfinite(rc1) && __builtin_isfinite(rc2))
    update_chunk<true>(c, scale, h, rc1, rc2);
  else
    update_chunk<false>(c, scale, h, rc1, rc2);
}

}  // namespace

// A chunk table in device memory for one tensor list (fg_adam_plan_*), with
// the fp64 norm partials next to it: a step over a plan allocates nothing.
struct fg_adam_plan {
  std::vector<Chunk> host;  // the table as uploaded (pointers, offsets, lengths)
  Chunk* dev = nullptr;     // nch chunks, then nch fp64 partials
  double* part = nullptr;
  int nch = 0;
  double nparams = 0;
};

namespace {

std::vector<Chunk> chunk_list(const fg_adam_tensor* tensors, int count, double* nparams) {
  std::vector<Chunk> chunks;
  double np = 0;
  for (int j = 0; j < count; ++j) {
    const fg_adam_tensor& t = tensors[j];
    if (t.n == 0) continue;
    np += (double)t.n;
    for (int64_t off = 0; off < t.n; off += kChunk) {
      Chunk c;
      c.p = t.p; c.g = t.g; c.m = t.m; c.v = t.v;
      c.off = off;
      c.len = (t.n - off) < kChunk ? (t.n - off) : kChunk;
      chunks.push_back(c);
    }
  }
  *nparams = np;
  return chunks;
}

int check_list(const char* fn, const fg_adam_tensor* tensors, int count) {
  FG_ARG_CHECK(count >= 0 && (count == 0 || tensors), "%s: bad tensor list", fn);
  for (int j = 0; j < count; ++j) {
    FG_ARG_CHECK(tensors[j].n >= 0, "%s: tensor %d has negative size", fn, j);
    FG_ARG_CHECK(tensors[j].n == 0 || (tensors[j].p && tensors[j].g && tensors[j].m && tensors[j].v),
                 "%s: tensor %d has a null pointer", fn, j);
  }
  return FG_OK;
}

// Uploads a table (synchronously: the host copy is not kept alive).
int plan_create(const fg_adam_tensor* tensors, int count, fg_adam_plan** out) {
  double np = 0;
  std::vector<Chunk> chunks = chunk_list(tensors, count, &np);
  fg_adam_plan* pl = new fg_adam_plan;
  pl->host = chunks;
  pl->nch = (int)chunks.size();
  pl->nparams = np;
  if (pl->nch > 0) {
    void* mem = nullptr;
    const size_t tb = ((sizeof(Chunk) * (size_t)pl->nch + 255) / 256) * 256;
    int rc = fg_malloc(&mem, tb + sizeof(double) * (size_t)pl->nch);
    if (rc) { delete pl; return rc; }
    pl->dev = (Chunk*)mem;
    pl->part = (double*)((char*)mem + tb);
    hipError_t e = hipMemcpyAsync(pl->dev, chunks.data(), sizeof(Chunk) * (size_t)pl->nch, hipMemcpyHostToDevice,
                                  fg::stream());
    if (e == hipSuccess) e = hipStreamSynchronize(fg::stream());
    if (e != hipSuccess) {
      fg_free(mem);
      delete pl;
      return fg::set_error(FG_ERR_HIP, "fg_adam_plan_create: table upload failed: %s", hipGetErrorString(e));
    }
  }
  *out = pl;
  return FG_OK;
}

// Tables of the tensor-list entry points (fg_adam_step / _sched), one per
// distinct list, kept for the life of the process: a recorded graph holds
// the table's device address, so a table is never rewritten or freed once a
// step has used it — a second optimizer (another list) gets its own.
std::vector<fg_adam_plan*> g_list_plans;
double* g_stats = nullptr;

int plan_for_list(const fg_adam_tensor* tensors, int count, fg_adam_plan** out) {
  double np = 0;
  std::vector<Chunk> chunks = chunk_list(tensors, count, &np);
  for (fg_adam_plan* pl : g_list_plans)
    if (pl->host.size() == chunks.size() &&
        (chunks.empty() || memcmp(pl->host.data(), chunks.data(), chunks.size() * sizeof(Chunk)) == 0)) {
      *out = pl;
      return FG_OK;
    }
  // A new tensor list needs a synchronous table upload, which a graph cannot
  // record: run one step outside the capture first.
  FG_NO_CAPTURE("fg_adam_step with a new tensor list");
  int rc = plan_create(tensors, count, out);
  if (rc) return rc;
  g_list_plans.push_back(*out);
  return FG_OK;
}

int adam_run(fg_adam_plan* pl, double lr_t, double b1, double b2, double eps, double wd, double clip, double bc1,
             double bc2, const double* sched_dev, double* stats_dev) {
  if (!stats_dev && !g_stats) {
    FG_NO_CAPTURE("fg_adam_step without a stats buffer (first call)");
    void* p = nullptr;
    FG_HIP_CHECK(hipMalloc(&p, 2 * sizeof(double)));
    g_stats = (double*)p;
  }
  double* stats = stats_dev ? stats_dev : g_stats;
  fg::KProfScope prof("adam", 0.0, 32.0 * pl->nparams);
  if (pl->nch == 0) {
    // no gradients: gnorm 0, scale 1 (a fill kernel, so a graph may hold it)
    FG_LAUNCH(stats_empty_kernel, dim3(1), dim3(64), 0, stats);
    return FG_OK;
  }
  FG_LAUNCH(sqnorm_kernel, dim3(pl->nch), dim3(kThreads), 0, pl->dev, pl->part);
  FG_LAUNCH(finalize_kernel, dim3(1), dim3(kThreads), 0, (const double*)pl->part, pl->nch, clip, stats);
  AdamHyper h;
  h.lr = lr_t; h.b1 = b1; h.b2 = b2; h.eps = eps; h.wd = wd; h.bc1 = bc1; h.bc2 = bc2;
  FG_LAUNCH(update_kernel, dim3(pl->nch), dim3(kThreads), 0, pl->dev, (const double*)stats, h, sched_dev);
  return FG_OK;
}

int adam_impl(const fg_adam_tensor* tensors, int count, double lr_t, double b1, double b2, double eps, double wd,
              double clip, double bc1, double bc2, const double* sched_dev, double* stats_dev) {
  FG_REQUIRE_INIT();
  int rc = check_list("fg_adam_step", tensors, count);
  if (rc) return rc;
  FG_ARG_CHECK(sched_dev || (bc1 > 0 && bc2 > 0), "fg_adam_step: bias corrections must be positive (bc1=%g bc2=%g)",
               bc1, bc2);
  fg_adam_plan* pl = nullptr;
  rc = plan_for_list(tensors, count, &pl);
  if (rc) return rc;
  return adam_run(pl, lr_t, b1, b2, eps, wd, clip, bc1, bc2, sched_dev, stats_dev);
}

}  // namespace

extern "C" int fg_adam_plan_create(const fg_adam_tensor* tensors, int count, fg_adam_plan** plan) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(plan, "fg_adam_plan_create: null plan pointer");
  FG_NO_CAPTURE("fg_adam_plan_create");
  int rc = check_list("fg_adam_plan_create", tensors, count);
  if (rc) return rc;
  return plan_create(tensors, count, plan);
}

extern "C" int fg_adam_plan_matches(const fg_adam_plan* plan, const fg_adam_tensor* tensors, int count, int* match) {
  FG_ARG_CHECK(plan && match, "fg_adam_plan_matches: null pointer");
  int rc = check_list("fg_adam_plan_matches", tensors, count);
  if (rc) return rc;
  double np = 0;
  std::vector<Chunk> chunks = chunk_list(tensors, count, &np);
  *match = plan->host.size() == chunks.size() &&
           (chunks.empty() || memcmp(plan->host.data(), chunks.data(), chunks.size() * sizeof(Chunk)) == 0);
  return FG_OK;
}

extern "C" int fg_adam_plan_destroy(fg_adam_plan* plan) {
  if (!plan) return FG_OK;
  if (plan->dev) {
    int rc = fg_free(plan->dev);  // stream-ordered: queued steps still see it
    if (rc) return rc;
  }
  delete plan;
  return FG_OK;
}

extern "C" int fg_adam_step_plan(fg_adam_plan* plan, double lr_t, double b1, double b2, double eps, double wd,
                                 double clip, double bc1, double bc2, double* stats_dev) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(plan, "fg_adam_step_plan: null plan");
  FG_ARG_CHECK(bc1 > 0 && bc2 > 0, "fg_adam_step_plan: bias corrections must be positive (bc1=%g bc2=%g)", bc1, bc2);
  return adam_run(plan, lr_t, b1, b2, eps, wd, clip, bc1, bc2, nullptr, stats_dev);
}

extern "C" int fg_adam_step_sched_plan(fg_adam_plan* plan, const double* sched_dev, double b1, double b2, double eps,
                                       double wd, double clip, double* stats_dev) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(plan && sched_dev, "fg_adam_step_sched_plan: null plan or schedule pointer");
  return adam_run(plan, 0.0, b1, b2, eps, wd, clip, 0.0, 0.0, sched_dev, stats_dev);
}

extern "C" int fg_adam_step(const fg_adam_tensor* tensors, int count, double lr_t, double b1, double b2, double eps,
                            double wd, double clip, double bc1, double bc2, double* stats_dev) {
  return adam_impl(tensors, count, lr_t, b1, b2, eps, wd, clip, bc1, bc2, nullptr, stats_dev);
}

extern "C" int fg_adam_step_sched(const fg_adam_tensor* tensors, int count, const double* sched_dev, double b1,
                                  double b2, double eps, double wd, double clip, double* stats_dev) {
  FG_ARG_CHECK(sched_dev, "fg_adam_step_sched: null schedule pointer");
  return adam_impl(tensors, count, 0.0, b1, b2, eps, wd, clip, 0.0, 0.0, sched_dev, stats_dev);
}
