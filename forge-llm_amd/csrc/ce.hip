// crossEntropyMean forward/backward (tensor.js:393-417) for gfx950.
//
// Forward: one workgroup per row (512 threads; 1024 for rows over 32768
// floats) streams the row once with an online (max, sum-exp) pair per
// thread, merges the pairs across the workgroup and writes lse[row] and the
// row loss lse - x[target].
// Exponentials are exp2 of log2(e)-scaled differences (one v_exp_f32 each).  A single
// workgroup then sums the row losses in fp64 in a fixed order (deterministic).
// Backward: recomputes softmax from the saved lse (the reference stores the
// T×V probability matrix instead) and writes (g/rows)·(P − onehot), one
// coalesced float4 pass: read logits, write dlogits.
#include "common.h"

#include <math.h>
#include <mutex>

namespace {

// Threads per row workgroup: 512 (16 float4 per thread for a 32000-word row
// held in registers) measured 2% faster than 256 at 8192 x 32000.
constexpr int kThreads = 512;

constexpr float kL2E = 1.4426950408889634f;  // log2(e): exp(x) = exp2(x * log2 e), one v_exp_f32

// v_exp_f32 itself (exp2f adds a range fix-up for results below 2^-126 to
// every call): such results flush to zero, which changes no sum of
// exponentials here (every row sum holds a term >= 1) and leaves gradient
// entries below (1/rows) * 2^-126 at zero instead of subnormal.  exp2(-inf)
// is 0.  Every CE kernel uses it, so the fused and separate forms still give
// the same bits.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void merge_ms(float& m, float& s, float m2, float s2) {
  float M = fmaxf(m, m2);
  if (M == -INFINITY) return;  // both empty
  s = s * fexp2((m - M) * kL2E) + s2 * fexp2((m2 - M) * kL2E);
  m = M;
}

constexpr int kFwdPer = 4;  // float4 loads in flight per thread (forward)

template <int NT>
__global__ void __launch_bounds__(NT) ce_fwd_rows_kernel(const float* __restrict__ logits,
                                                               const int32_t* __restrict__ targets,
                                                               float* __restrict__ lse_out,
                                                               double* __restrict__ row_loss, int V,
                                                               int vec4) {
  const int row = blockIdx.x;
  const float* x = logits + (size_t)row * V;
  float m = -INFINITY, s = 0.f;
  if (vec4) {
    // The row is read once and not again until the backward: nontemporal
    // loads.  The running sum is rescaled only when the running max grows.
    // kFwdPer float4 loads are issued together, then folded in order.
    const v4f* x4 = reinterpret_cast<const v4f*>(x);
    const int n4 = V >> 2;
    for (int i0 = threadIdx.x; i0 < n4; i0 += NT * kFwdPer) {
      v4f vs[kFwdPer];
#pragma unroll
      for (int u = 0; u < kFwdPer; ++u) {
        const int i = i0 + u * NT;
        vs[u] = i < n4 ? __builtin_nontemporal_load(x4 + i) : v4f{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
#pragma unroll
      for (int u = 0; u < kFwdPer; ++u) {
        const v4f v = vs[u];
        const float lm = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        if (lm > m) {
          s *= fexp2((m - lm) * kL2E);
          m = lm;
        }
        if (m != -INFINITY)
          s += fexp2((v[0] - m) * kL2E) + fexp2((v[1] - m) * kL2E) + fexp2((v[2] - m) * kL2E) +
               fexp2((v[3] - m) * kL2E);
      }
    }
  } else {
    for (int i = threadIdx.x; i < V; i += NT) {
      float v = x[i];
      float M = fmaxf(m, v);
      if (M != -INFINITY) {
        s = s * fexp2((m - M) * kL2E) + fexp2((v - M) * kL2E);
        m = M;
      }
    }
  }
  // wave merge
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge_ms(m, s, m2, s2);
  }
  __shared__ float sm[NT / 64], ss[NT / 64];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { sm[w] = m; ss[w] = s; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], S = ss[0];
    for (int i = 1; i < NT / 64; ++i) merge_ms(M, S, sm[i], ss[i]);
    double lse = (double)M + log((double)S);
    lse_out[row] = (float)lse;
    int t = targets[row];
    row_loss[row] = (t >= 0 && t < V) ? lse - (double)x[t] : (double)NAN;
  }
}

// Sums row losses in fp64 with a fixed reduction tree; writes the mean.
// With xp set it also fills the FG_XP_PARTS partial maxima of the seed-1
// gradient the fused kernels wrote with their bound xv = 1/rows
// (|softmax - onehot| <= 1), for the GEMM that reads that gradient.
__global__ void __launch_bounds__(kThreads) ce_mean_kernel(const double* __restrict__ row_loss, int rows,
                                                           float* __restrict__ loss, float* __restrict__ xp, float xv) {
  static_assert(kThreads >= FG_XP_PARTS, "one partial per thread");
  if (xp && threadIdx.x < FG_XP_PARTS) xp[threadIdx.x] = xv;
  // eight loads in flight, added in the same order as one at a time
  double acc = 0.0;
  int i = threadIdx.x;
  for (; i + 7 * kThreads < rows; i += 8 * kThreads) {
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = row_loss[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += v[u];
  }
  for (; i < rows; i += kThreads) acc += row_loss[i];
  acc = fg_wave_sum_d(acc);
  __shared__ double part[kThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int i = 0; i < kThreads / 64; ++i) t += part[i];
    *loss = (float)(t / rows);
  }
}

// grid: (rows, 1) for float4 rows (a workgroup streams its row), else
// (rows, chunks) with kPer*4 scalars per thread.
// PER float4 loads in flight per thread (float4 rows): 8, or kOnePass for
// rows of at most 8192 float4 (V <= 32768), which then take one pass with
// every load issued before the first store (5% faster at 8192 x 32000).
constexpr int kPer = 8;
constexpr int kOnePass = 8192 / kThreads;
template <int PER>
__global__ void __launch_bounds__(kThreads) ce_bwd_kernel(float* __restrict__ dl, const float* __restrict__ logits,
                                                          const float* __restrict__ lse,
                                                          const int32_t* __restrict__ targets,
                                                          const float* __restrict__ gloss, int rows, int V,
                                                          int beta, int vec4) {
  const int row = blockIdx.x;
  const float k = (float)((gloss ? (double)(*gloss) : 1.0) / (double)rows);  // null: the seed gradient 1
  const float l = lse[row];
  const int t = targets[row];
  const size_t base = (size_t)row * V;
  if (vec4) {
    // One row per workgroup (grid.y == 1): the row constants are loaded once.
    // logits are read for the last time and dlogits (rows x V) goes straight
    // to the LM-head GEMMs: nontemporal loads and stores, PER in flight.
    const v4f* x4 = reinterpret_cast<const v4f*>(logits + base);
    v4f* d4 = reinterpret_cast<v4f*>(dl + base);
    const int n4 = V >> 2;
    for (int i0 = threadIdx.x; i0 < n4; i0 += kThreads * PER) {
      v4f v[PER];
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int i = i0 + u * kThreads;
        if (i < n4) v[u] = __builtin_nontemporal_load(x4 + i);
      }
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int i = i0 + u * kThreads;
        if (i < n4) {
          v4f r;
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = k * fexp2((v[u][e] - l) * kL2E);
          const int j = i * 4;
          if (t >= j && t < j + 4) r[t - j] -= k;
          if (beta) r += d4[i];
          __builtin_nontemporal_store(r, d4 + i);
        }
      }
    }
  } else {
    const int start = blockIdx.y * (kThreads * kPer * 4) + threadIdx.x;
    for (int u = 0; u < kPer * 4; ++u) {
      int i = start + u * kThreads;
      if (i < V) {
        float r = k * fexp2((logits[base + i] - l) * kL2E);
        if (i == t) r -= k;
        if (beta) r += dl[base + i];
        dl[base + i] = r;
      }
    }
  }
}

// Forward and the backward of a seed gradient of 1 in one kernel, for a loss
// whose backward always follows (the training step): one workgroup per row
// reads the row (cached loads: the second pass finds it in L2 / Infinity
// Cache), forms (max, sum exp), lse and the row loss exactly as
// ce_fwd_rows_kernel, then writes dl = (1/rows)(softmax - onehot) exactly as
// ce_bwd_kernel does for gloss = 1 — one HBM read of the logits instead of two.
template <int NT, int PER2>
__global__ void __launch_bounds__(NT) ce_fused_rows_kernel(float* __restrict__ dl, const float* __restrict__ logits,
                                                                 const int32_t* __restrict__ targets,
                                                                 float* __restrict__ lse_out,
                                                                 double* __restrict__ row_loss, int rows, int V,
                                                                 int vec4) {
  const int row = blockIdx.x;
  const float* x = logits + (size_t)row * V;
  float m = -INFINITY, s = 0.f;
  if (vec4) {
    const v4f* x4 = reinterpret_cast<const v4f*>(x);
    const int n4 = V >> 2;
    for (int i0 = threadIdx.x; i0 < n4; i0 += NT * kFwdPer) {
      v4f vs[kFwdPer];
#pragma unroll
      for (int u = 0; u < kFwdPer; ++u) {
        const int i = i0 + u * NT;
        vs[u] = i < n4 ? x4[i] : v4f{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
#pragma unroll
      for (int u = 0; u < kFwdPer; ++u) {
        const v4f v = vs[u];
        const float lm = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        if (lm > m) {
          s *= fexp2((m - lm) * kL2E);
          m = lm;
        }
        if (m != -INFINITY)
          s += fexp2((v[0] - m) * kL2E) + fexp2((v[1] - m) * kL2E) + fexp2((v[2] - m) * kL2E) +
               fexp2((v[3] - m) * kL2E);
      }
    }
  } else {
    for (int i = threadIdx.x; i < V; i += NT) {
      float v = x[i];
      float M = fmaxf(m, v);
      if (M != -INFINITY) {
        s = s * fexp2((m - M) * kL2E) + fexp2((v - M) * kL2E);
        m = M;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge_ms(m, s, m2, s2);
  }
  __shared__ float sm[NT / 64], ss[NT / 64], lsh;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { sm[w] = m; ss[w] = s; }
  __syncthreads();
  const int t = targets[row];
  if (threadIdx.x == 0) {
    float M = sm[0], S = ss[0];
    for (int i = 1; i < NT / 64; ++i) merge_ms(M, S, sm[i], ss[i]);
    double lse = (double)M + log((double)S);
    lse_out[row] = (float)lse;
    lsh = (float)lse;
    row_loss[row] = (t >= 0 && t < V) ? lse - (double)x[t] : (double)NAN;
  }
  __syncthreads();
  const float l = lsh;
  const float k = (float)(1.0 / (double)rows);
  float* d = dl + (size_t)row * V;
  if (vec4) {
    const v4f* x4 = reinterpret_cast<const v4f*>(x);
    v4f* d4 = reinterpret_cast<v4f*>(d);
    const int n4 = V >> 2;
    for (int i0 = threadIdx.x; i0 < n4; i0 += NT * PER2) {
      v4f v[PER2];
#pragma unroll
      for (int u = 0; u < PER2; ++u) {
        const int i = i0 + u * NT;
        if (i < n4) v[u] = x4[i];
      }
#pragma unroll
      for (int u = 0; u < PER2; ++u) {
        const int i = i0 + u * NT;
        if (i < n4) {
          v4f r;
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = k * fexp2((v[u][e] - l) * kL2E);
          const int j = i * 4;
          if (t >= j && t < j + 4) r[t - j] -= k;
          __builtin_nontemporal_store(r, d4 + i);
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < V; i += NT) {
      float r = k * fexp2((x[i] - l) * kL2E);
      if (i == t) r -= k;
      d[i] = r;
    }
  }
}

// The same for float4 rows of at most kRegsRow4 float4 (V <= 32768): each
// thread holds its whole share of the row in registers (float4 i = tid +
// NT·j, j = 0..kRegsRow4/NT - 1, padded with -inf), so the row is read
// from HBM once, with every load in flight at the start.  The (max, sum-exp)
// fold visits the elements in the order ce_fwd_rows_kernel does (padding adds
// exp2(-inf) = 0, which leaves s unchanged), so lse, the row loss and dl are
// bit-identical to the unfused forward and backward.
constexpr int kRegsRow4 = 8192;  // float4 of the longest row held in registers (V <= 32768)
template <int NT>
__global__ void __launch_bounds__(NT) ce_fused_regs_kernel(float* __restrict__ dl,
                                                                 const float* __restrict__ logits,
                                                                 const int32_t* __restrict__ targets,
                                                                 float* __restrict__ lse_out,
                                                                 double* __restrict__ row_loss, int rows, int V) {
  const int row = blockIdx.x;
  const float* x = logits + (size_t)row * V;
  const v4f* x4 = reinterpret_cast<const v4f*>(x);
  const int n4 = V >> 2;
  v4f v[(kRegsRow4 / NT)];
#pragma unroll
  for (int j = 0; j < (kRegsRow4 / NT); ++j) {
    const int i = threadIdx.x + j * NT;
    v[j] = i < n4 ? __builtin_nontemporal_load(x4 + i) : v4f{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  }
  float m = -INFINITY, s = 0.f;
#pragma unroll
  for (int j = 0; j < (kRegsRow4 / NT); ++j) {
    const float lm = fmaxf(fmaxf(v[j][0], v[j][1]), fmaxf(v[j][2], v[j][3]));
    if (lm > m) {
      s *= fexp2((m - lm) * kL2E);
      m = lm;
    }
    if (m != -INFINITY)
      s += fexp2((v[j][0] - m) * kL2E) + fexp2((v[j][1] - m) * kL2E) + fexp2((v[j][2] - m) * kL2E) +
           fexp2((v[j][3] - m) * kL2E);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge_ms(m, s, m2, s2);
  }
  __shared__ float sm[NT / 64], ss[NT / 64], lsh;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { sm[w] = m; ss[w] = s; }
  __syncthreads();
  const int t = targets[row];
  if (threadIdx.x == 0) {
    float M = sm[0], S = ss[0];
    for (int i = 1; i < NT / 64; ++i) merge_ms(M, S, sm[i], ss[i]);
    double lse = (double)M + log((double)S);
    lse_out[row] = (float)lse;
    lsh = (float)lse;
    row_loss[row] = (t >= 0 && t < V) ? lse - (double)x[t] : (double)NAN;
  }
  __syncthreads();
  const float l = lsh;
  const float k = (float)(1.0 / (double)rows);
  v4f* d4 = reinterpret_cast<v4f*>(dl + (size_t)row * V);
#pragma unroll
  for (int j = 0; j < (kRegsRow4 / NT); ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < n4) {
      v4f r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = k * fexp2((v[j][e] - l) * kL2E);
      const int q = i * 4;
      if (t >= q && t < q + 4) r[t - q] -= k;
      __builtin_nontemporal_store(r, d4 + i);
    }
  }
}

// Rows longer than 32768 floats (the 128256-word vocabulary: 513 KB rows)
// use 1024-thread workgroups; the forward kernel uses the same thread count
// for such rows, so the fused and separate forms still give the same bits.
constexpr int kLongThreads = 1024;

// Float4 rows of 32768 < V <= 131072 floats, read from HBM once: each of the
// 1024 threads owns float4 i = tid + 1024 j, j = 0..31 (padded with -inf),
// the first kLongRegs of them in registers and the other kLongLds in LDS
// (144 KB: one workgroup per CU, 4 waves per SIMD within 128 VGPRs).  The LDS
// share is loaded straight into LDS (global_load_lds, 16 B per lane at the
// wave's base + 16·lane: no registers), so all 32 loads of a thread are in
// flight at once; each thread reads back only its own LDS entries.  The
// (max, sum-exp) fold visits j in increasing order, as ce_fwd_rows_kernel
// does (padding adds exp2(-inf) = 0), so lse, the row loss and dl are
// bit-identical to the separate forward and backward.  (A persistent form,
// one workgroup per CU refilling each slot with the next row as it is
// written out, measured slower: 868 against 803 us at 4096 x 128256.)
constexpr int kLongRegs = 23, kLongLds = 9;
constexpr int kLongMax4 = (kLongRegs + kLongLds) * kLongThreads;  // float4 of the longest row (131072 floats)
__global__ void __launch_bounds__(kLongThreads) ce_fused_long_kernel(float* __restrict__ dl,
                                                                     const float* __restrict__ logits,
                                                                     const int32_t* __restrict__ targets,
                                                                     float* __restrict__ lse_out,
                                                                     double* __restrict__ row_loss, int rows,
                                                                     int V) {
  constexpr int NT = kLongThreads;
  __shared__ __attribute__((aligned(16))) v4f sl[kLongLds * NT];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const float* x = logits + (size_t)row * V;
  const v4f* x4 = reinterpret_cast<const v4f*>(x);
  const int n4 = V >> 2;
  const v4f ninf = v4f{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int j = 0; j < kLongLds; ++j) {
    const int i = tid + (kLongRegs + j) * NT;
    if (i < n4)
      __builtin_amdgcn_global_load_lds((const void*)(x4 + i),
                                       (__attribute__((address_space(3))) void*)(sl + j * NT + w * 64), 16, 0, 0);
  }
  v4f v[kLongRegs];
#pragma unroll
  for (int j = 0; j < kLongRegs; ++j) {
    const int i = tid + j * NT;
    v[j] = i < n4 ? __builtin_nontemporal_load(x4 + i) : ninf;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the LDS share has landed
  __syncthreads();
  auto at = [&](int tt, int j) -> v4f { return tt + j * NT < n4 ? sl[(j - kLongRegs) * NT + tt] : ninf; };
  float m = -INFINITY, s = 0.f;
  auto fold = [&](const v4f& q) {
    const float lm = fmaxf(fmaxf(q[0], q[1]), fmaxf(q[2], q[3]));
    if (lm > m) {
      s *= fexp2((m - lm) * kL2E);
      m = lm;
    }
    if (m != -INFINITY)
      s += fexp2((q[0] - m) * kL2E) + fexp2((q[1] - m) * kL2E) + fexp2((q[2] - m) * kL2E) + fexp2((q[3] - m) * kL2E);
  };
#pragma unroll
  for (int j = 0; j < kLongRegs; ++j) fold(v[j]);
#pragma unroll
  for (int j = kLongRegs; j < kLongRegs + kLongLds; ++j) fold(at(tid, j));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge_ms(m, s, m2, s2);
  }
  __shared__ float sm[NT / 64], ss[NT / 64], lsh;
  if (lane == 0) { sm[w] = m; ss[w] = s; }
  __syncthreads();
  const int t = targets[row];
  if (tid == 0) {
    float M = sm[0], S = ss[0];
    for (int i = 1; i < NT / 64; ++i) merge_ms(M, S, sm[i], ss[i]);
    double lse = (double)M + log((double)S);
    lse_out[row] = (float)lse;
    lsh = (float)lse;
    row_loss[row] = (t >= 0 && t < V) ? lse - (double)x[t] : (double)NAN;
  }
  __syncthreads();
  const float l = lsh;
  const float k = (float)(1.0 / (double)rows);
  v4f* d4 = reinterpret_cast<v4f*>(dl + (size_t)row * V);
  // An opaque copy of the thread index: the store offsets are recomputed
  // here instead of being held (spilled) from the loads.
  int tt = tid;
  asm volatile("" : "+v"(tt));
  auto put = [&](const v4f& q, int j) {
    const int i = tt + j * NT;
    if (i < n4) {
      v4f r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = k * fexp2((q[e] - l) * kL2E);
      const int c = i * 4;
      if (t >= c && t < c + 4) r[t - c] -= k;
      __builtin_nontemporal_store(r, d4 + i);
    }
  };
#pragma unroll
  for (int j = 0; j < kLongRegs; ++j) put(v[j], j);
#pragma unroll
  for (int j = kLongRegs; j < kLongRegs + kLongLds; ++j) put(at(tt, j), j);
}

// Row-workgroup kernels of the training loss: forward + seed-1 backward.
int ce_fused_launch(float* dlogits, const float* logits, const int32_t* targets, float* lse, double* part,
                    int rows, int V) {
  const int vec4 = (V % 4 == 0) && ((uintptr_t)logits % 16 == 0) && ((uintptr_t)dlogits % 16 == 0);
  if (vec4 && V <= kRegsRow4 * 4) {  // the row in registers: one HBM read
    FG_LAUNCH((ce_fused_regs_kernel<kThreads>), dim3(rows), dim3(kThreads), 0, dlogits, logits, targets, lse, part,
              rows, V);
  } else if (V <= 32768) {  // rows of <= 128 KB: the second read of a row hits the caches
    FG_LAUNCH((ce_fused_rows_kernel<kThreads, kPer>), dim3(rows), dim3(kThreads), 0, dlogits, logits, targets, lse,
              part, rows, V, vec4);
  } else if (vec4 && V <= kLongMax4 * 4) {  // the row in registers and LDS: one HBM read
    FG_LAUNCH(ce_fused_long_kernel, dim3(rows), dim3(kLongThreads), 0, dlogits, logits, targets, lse, part, rows, V);
  } else {  // the 256 rows in flight (~131 MB) stay in the Infinity Cache for the second read

    FG_LAUNCH((ce_fused_rows_kernel<kLongThreads, 16>), dim3(rows), dim3(kLongThreads), 0, dlogits, logits, targets,
              lse, part, rows, V, vec4);
  }
  return FG_OK;
}

int ce_fwd_launch(const float* logits, const int32_t* targets, float* lse, double* part, int rows, int V) {
  const int vec4 = (V % 4 == 0) && ((uintptr_t)logits % 16 == 0);
  if (V <= 32768)
    FG_LAUNCH((ce_fwd_rows_kernel<kThreads>), dim3(rows), dim3(kThreads), 0, logits, targets, lse, part, V, vec4);
  else
    FG_LAUNCH((ce_fwd_rows_kernel<kLongThreads>), dim3(rows), dim3(kLongThreads), 0, logits, targets, lse, part, V,
              vec4);
  return FG_OK;
}

}  // namespace

extern "C" int fg_ce_fwd_bwd(float* loss, float* lse, float* dlogits, const float* logits, const int32_t* targets,
                             int rows, int V) {
  return fg_ce_fwd_bwd_p(loss, lse, dlogits, logits, targets, rows, V, nullptr);
}

extern "C" int fg_ce_fwd_bwd_p(float* loss, float* lse, float* dlogits, const float* logits, const int32_t* targets,
                               int rows, int V, float* xp_grad) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && V > 0, "fg_ce_fwd_bwd: rows=%d V=%d must be positive", rows, V);
  FG_ARG_CHECK(loss && lse && dlogits && logits && targets, "fg_ce_fwd_bwd: null pointer");
  FG_ARG_CHECK(dlogits != logits, "fg_ce_fwd_bwd: dlogits must not alias logits");
  fg::KProfScope prof("ce_fwd_bwd", 0.0, 8.0 * rows * (double)V + 12.0 * rows);
  fg::Workspace ws;
  int rc = ws.get(sizeof(double) * (size_t)rows);
  if (rc) return rc;
  rc = ce_fused_launch(dlogits, logits, targets, lse, (double*)ws.ptr, rows, V);
  if (rc) return rc;
  FG_LAUNCH(ce_mean_kernel, dim3(1), dim3(kThreads), 0, (const double*)ws.ptr, rows, loss, xp_grad,
            (float)(1.0 / rows));
  return FG_OK;
}

// ── the training loss without allocation (fg_ce_fwd_bwd_noalloc) ─────────
// The per-row losses of fg_ce_fwd_bwd live in this array instead of a
// workspace: 64 Ki rows of fp64 (512 KiB), held on every device the library
// runs on until the process ends.  Each row kernel writes the entry of every
// row before ce_mean reads them, so nothing needs clearing between calls.
constexpr int kNoAllocRows = 1 << 16;
static __device__ __align__(256) double scratch[kNoAllocRows];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
double* g_scratch_dev[kMaxDevices] = {};  // the array's address on each device

// The array's device address on the current device, looked up once per device.
int scratch_ptr(double** out) {
  int dev = 0;
  FG_HIP_CHECK(hipGetDevice(&dev));
  FG_ARG_CHECK(dev >= 0 && dev < kMaxDevices, "fg_ce_fwd_bwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    FG_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    FG_ARG_CHECK(p != nullptr, "fg_ce_fwd_bwd_noalloc: no device address for the scratch array");
    g_scratch_dev[dev] = static_cast<double*>(p);
  }
  *out = g_scratch_dev[dev];
  return FG_OK;
}
}  // namespace

extern "C" int fg_ce_fwd_bwd_noalloc(float* loss, float* lse, float* dlogits, const float* logits,
                                     const int32_t* targets, int rows, int V) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && V > 0, "fg_ce_fwd_bwd_noalloc: rows=%d V=%d must be positive", rows, V);
  FG_ARG_CHECK(rows <= kNoAllocRows, "fg_ce_fwd_bwd_noalloc: rows=%d exceeds the %d rows of its static scratch",
               rows, kNoAllocRows);
  FG_ARG_CHECK(loss && lse && dlogits && logits && targets, "fg_ce_fwd_bwd_noalloc: null pointer");
  FG_ARG_CHECK(dlogits != logits, "fg_ce_fwd_bwd_noalloc: dlogits must not alias logits");
  double* part = nullptr;
  int rc = scratch_ptr(&part);
  if (rc) return rc;
  // the kernels and launch shapes of fg_ce_fwd_bwd, with the scratch array
  // in place of the workspace
  rc = ce_fused_launch(dlogits, logits, targets, lse, part, rows, V);
  if (rc) return rc;
  FG_LAUNCH(ce_mean_kernel, dim3(1), dim3(kThreads), 0, (const double*)part, rows, loss, nullptr, 0.f);
  return FG_OK;
}

extern "C" int fg_ce_fwd(float* loss, float* lse, const float* logits, const int32_t* targets, int rows, int V) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && V > 0, "fg_ce_fwd: rows=%d V=%d must be positive", rows, V);
  FG_ARG_CHECK(loss && lse && logits && targets, "fg_ce_fwd: null pointer");
  fg::KProfScope prof("ce_fwd", 0.0, 4.0 * rows * (double)V + 12.0 * rows);
  fg::Workspace ws;
  int rc = ws.get(sizeof(double) * (size_t)rows);
  if (rc) return rc;
  rc = ce_fwd_launch(logits, targets, lse, (double*)ws.ptr, rows, V);
  if (rc) return rc;
  FG_LAUNCH(ce_mean_kernel, dim3(1), dim3(kThreads), 0, (const double*)ws.ptr, rows, loss, nullptr, 0.f);
  return FG_OK;
}

// The bound |gloss| / rows of a fresh CE gradient as FG_XP_PARTS partial maxima.
__global__ void __launch_bounds__(FG_XP_PARTS) ce_grad_bound_kernel(float* __restrict__ xp,
                                                                    const float* __restrict__ gloss, float inv_rows) {
  xp[threadIdx.x] = fabsf(gloss[0]) * inv_rows;
}

extern "C" int fg_ce_bwd(float* dlogits, const float* logits, const float* lse, const int32_t* targets,
                         const float* gloss, int rows, int V, int beta) {
  return fg_ce_bwd_p(dlogits, logits, lse, targets, gloss, rows, V, beta, nullptr);
}

extern "C" int fg_ce_bwd_p(float* dlogits, const float* logits, const float* lse, const int32_t* targets,
                           const float* gloss, int rows, int V, int beta, float* xp_grad) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && V > 0, "fg_ce_bwd: rows=%d V=%d must be positive", rows, V);
  FG_ARG_CHECK(dlogits && logits && lse && targets && gloss, "fg_ce_bwd: null pointer");
  fg::KProfScope prof("ce_bwd", 0.0, (beta ? 12.0 : 8.0) * rows * (double)V);
  int vec4 = (V % 4 == 0) && ((uintptr_t)logits % 16 == 0) && ((uintptr_t)dlogits % 16 == 0);
  int per_block = kThreads * kPer * 4;  // elements per workgroup (scalar path)
  dim3 grid(rows, vec4 ? 1 : (V + per_block - 1) / per_block);
  if (vec4 && V / 4 <= kThreads * kOnePass) {
    FG_LAUNCH((ce_bwd_kernel<kOnePass>), grid, dim3(kThreads), 0, dlogits, logits, lse, targets, gloss, rows, V,
              beta ? 1 : 0, vec4);
  } else {
    FG_LAUNCH((ce_bwd_kernel<kPer>), grid, dim3(kThreads), 0, dlogits, logits, lse, targets, gloss, rows, V,
              beta ? 1 : 0, vec4);
  }
  if (xp_grad) {
    FG_ARG_CHECK(!beta, "fg_ce_bwd_p: the gradient bound holds for a fresh gradient (beta 0) only");
    FG_LAUNCH(ce_grad_bound_kernel, dim3(1), dim3(FG_XP_PARTS), 0, xp_grad, gloss, (float)(1.0 / rows));
  }
  return FG_OK;
}
