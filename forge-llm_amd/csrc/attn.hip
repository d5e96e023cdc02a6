// causalAttn / causalAttnBatch forward and backward (tensor.js:191-268,
// 299-376) for gfx950.  Up to head size 128, flash style: the T×T probability
// matrix the reference stores is never materialised; the forward saves the
// row log-sum-exp and the backward recomputes P from it.  Above 128 the
// attention is composed from batched GEMM launches over T×T workspaces.
//
// Layout: Q[B*T, nH*dH], K/V[B*T, nKV*dH] (row-major, head h in columns
// [h*dH, (h+1)*dH)), block-diagonal causal mask (row b*T+t sees b*T..b*T+t),
// GQA map kvh = h / max(1, nH/nKV), scale 1/sqrt(dH).  lse[(b*nH+h)*T + t].
//
// Three kernel families:
//  * MFMA (dH in {32, 64, 96, 128}): 32x32 blocks on v_mfma_f32_32x32x16_f16
//    with every fp32 operand scaled by a power of two and split into fp16 hi
//    and lo pieces (f16split.h), in
//    a transposed formulation — S^T = K·Q^T and O^T = V^T·P^T — so each lane
//    owns one query (lane%32) and its softmax statistics; the 16 score values
//    a lane holds are exactly the k-values it feeds to the next MFMA, so P
//    never goes through LDS.  Backward = D = rowsum(dO∘O) (attn_d_pre), then
//    one launch holding the dQ work items (per query block) and the dK/dV work
//    items (per key block; with GQA per group member, partials summed in order
//    by attn_dkv_reduce): deterministic, no atomics.  Head sizes between 32
//    and 128 without a kernel of their own (e.g. 48, 80, 112) run the next
//    size's kernels on head-padded copies (attn_pad_kernel).
//  * scalar (dH below 32 and other sizes up to 128 on unaligned tensors, and
//    the backward when nH < nKV): one thread per query / key row holding its
//    head vector in registers (templated on the largest head size of its
//    class: 64 or 128), for the tiny shapes of the gradient checks and the
//    demo configuration.
//  * head sizes above 128 (any size): S = Q·K^T and O = P·V (and the
//    backward's five products) as batched GEMM launches over the (sample,
//    head) problems on gemm.hip's kernels, with a row kernel for the softmax
//    — the whole T×T square, the causal half of it wasted, in T×T workspaces.
#include "common.h"
#include "f16split.h"

#include <atomic>

#include <math.h>

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ═════════════════════════ scalar kernels (dH <= 128) ═════════════════════════
// kSMax: the largest head size the instance handles (64 or 128: registers per
// row and LDS tiles [kSRows][kSMax + 1]).
constexpr int kSRows = 64;  // rows per workgroup (one wave)

template <int kSMax>
__global__ void __launch_bounds__(kSRows) attn_fwd_scalar(float* __restrict__ O, float* __restrict__ lse,
                                                          const float* __restrict__ Q, const float* __restrict__ K,
                                                          const float* __restrict__ V, int T, int nH, int nKV,
                                                          int dH, float scale) {
  __shared__ float Ks[kSRows][kSMax + 1], Vs[kSRows][kSMax + 1];
  const int bh = blockIdx.y, b = bh / nH, h = bh % nH;
  const int group = nH / nKV > 1 ? nH / nKV : 1, kvh = h / group;
  const int qD = nH * dH, kvD = nKV * dH;
  const int t = blockIdx.x * kSRows + threadIdx.x;
  const bool valid = t < T;
  float q[kSMax], o[kSMax];
  const size_t qrow = ((size_t)b * T + (valid ? t : 0)) * qD + (size_t)h * dH;
#pragma unroll
  for (int d = 0; d < kSMax; ++d) {
    q[d] = (d < dH) ? Q[qrow + d] : 0.f;
    o[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int last = min(T - 1, blockIdx.x * kSRows + kSRows - 1);
  for (int j0 = 0; j0 <= last; j0 += kSRows) {
    __syncthreads();
    for (int e = threadIdx.x; e < kSRows * dH; e += kSRows) {
      const int r = e / dH, d = e % dH, j = j0 + r;
      const size_t krow = ((size_t)b * T + j) * kvD + (size_t)kvh * dH + d;
      Ks[r][d] = j < T ? K[krow] : 0.f;
      Vs[r][d] = j < T ? V[krow] : 0.f;
    }
    __syncthreads();
    if (valid) {
      const int jend = min(t, j0 + kSRows - 1);
      for (int j = j0; j <= jend; ++j) {
        const int r = j - j0;
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < kSMax; ++d)
          if (d < dH) s += q[d] * Ks[r][d];
        s *= scale;
        const float mn = fmaxf(m, s);
        const float alpha = expf(m - mn), p = expf(s - mn);
        l = l * alpha + p;
#pragma unroll
        for (int d = 0; d < kSMax; ++d)
          if (d < dH) o[d] = o[d] * alpha + p * Vs[r][d];
        m = mn;
      }
    }
  }
  if (valid) {
    const float il = 1.f / l;
#pragma unroll
    for (int d = 0; d < kSMax; ++d)
      if (d < dH) O[qrow + d] = o[d] * il;
    lse[(size_t)bh * T + t] = m + logf(l);
  }
}

// Dq[(b*nH+h)*T + t] = sum_d dO·O  (shared by both backward families)
__global__ void __launch_bounds__(256) attn_bwd_pre(float* __restrict__ Dq, const float* __restrict__ dO,
                                                    const float* __restrict__ O, int B, int T, int nH, int dH) {
  const int64_t n = (int64_t)B * T * nH;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t row = e / nH;  // b*T + t
    const int h = (int)(e - row * nH);
    const size_t base = (size_t)row * nH * dH + (size_t)h * dH;
    float acc = 0.f;
    for (int d = 0; d < dH; ++d) acc += dO[base + d] * O[base + d];
    const int64_t b = row / T, t = row - b * T;
    Dq[(b * nH + h) * T + t] = acc;
  }
}

template <int kSMax>
__global__ void __launch_bounds__(kSRows) attn_dq_scalar(float* __restrict__ dQ, int beta,
                                                         const float* __restrict__ dO, const float* __restrict__ Q,
                                                         const float* __restrict__ K, const float* __restrict__ V,
                                                         const float* __restrict__ lse, const float* __restrict__ Dq,
                                                         int T, int nH, int nKV, int dH, float scale) {
  __shared__ float Ks[kSRows][kSMax + 1], Vs[kSRows][kSMax + 1];
  const int bh = blockIdx.y, b = bh / nH, h = bh % nH;
  const int group = nH / nKV > 1 ? nH / nKV : 1, kvh = h / group;
  const int qD = nH * dH, kvD = nKV * dH;
  const int t = blockIdx.x * kSRows + threadIdx.x;
  const bool valid = t < T;
  float q[kSMax], go[kSMax], dq[kSMax];
  const size_t qrow = ((size_t)b * T + (valid ? t : 0)) * qD + (size_t)h * dH;
#pragma unroll
  for (int d = 0; d < kSMax; ++d) {
    q[d] = (d < dH) ? Q[qrow + d] : 0.f;
    go[d] = (d < dH) ? dO[qrow + d] : 0.f;
    dq[d] = 0.f;
  }
  const float L = valid ? lse[(size_t)bh * T + t] : 0.f;
  const float Dt = valid ? Dq[(size_t)bh * T + t] : 0.f;
  const int last = min(T - 1, blockIdx.x * kSRows + kSRows - 1);
  for (int j0 = 0; j0 <= last; j0 += kSRows) {
    __syncthreads();
    for (int e = threadIdx.x; e < kSRows * dH; e += kSRows) {
      const int r = e / dH, d = e % dH, j = j0 + r;
      const size_t krow = ((size_t)b * T + j) * kvD + (size_t)kvh * dH + d;
      Ks[r][d] = j < T ? K[krow] : 0.f;
      Vs[r][d] = j < T ? V[krow] : 0.f;
    }
    __syncthreads();
    if (valid) {
      const int jend = min(t, j0 + kSRows - 1);
      for (int j = j0; j <= jend; ++j) {
        const int r = j - j0;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int d = 0; d < kSMax; ++d)
          if (d < dH) {
            s += q[d] * Ks[r][d];
            dp += go[d] * Vs[r][d];
          }
        const float p = expf(s * scale - L);
        const float ds = p * (dp - Dt);
#pragma unroll
        for (int d = 0; d < kSMax; ++d)
          if (d < dH) dq[d] += ds * Ks[r][d];
      }
    }
  }
  if (valid) {
#pragma unroll
    for (int d = 0; d < kSMax; ++d)
      if (d < dH) {
        const float v = dq[d] * scale;
        dQ[qrow + d] = beta ? dQ[qrow + d] + v : v;
      }
  }
}

template <int kSMax>
__global__ void __launch_bounds__(kSRows) attn_dkv_scalar(float* __restrict__ dK, int beta_k, float* __restrict__ dV,
                                                          int beta_v, const float* __restrict__ dO,
                                                          const float* __restrict__ Q, const float* __restrict__ K,
                                                          const float* __restrict__ V, const float* __restrict__ lse,
                                                          const float* __restrict__ Dq, int T, int nH, int nKV, int dH,
                                                          float scale) {
  __shared__ float Qs[kSRows][kSMax + 1], Gs[kSRows][kSMax + 1], Ls[kSRows], Ds[kSRows];
  const int bk = blockIdx.y, b = bk / nKV, kvh = bk % nKV;
  const int group = nH / nKV > 1 ? nH / nKV : 1;
  const int qD = nH * dH, kvD = nKV * dH;
  const int j = blockIdx.x * kSRows + threadIdx.x;
  const bool valid = j < T;
  float k[kSMax], v[kSMax], dk[kSMax], dv[kSMax];
  const size_t krow = ((size_t)b * T + (valid ? j : 0)) * kvD + (size_t)kvh * dH;
#pragma unroll
  for (int d = 0; d < kSMax; ++d) {
    k[d] = (d < dH) ? K[krow + d] : 0.f;
    v[d] = (d < dH) ? V[krow + d] : 0.f;
    dk[d] = 0.f;
    dv[d] = 0.f;
  }
  const int first = blockIdx.x * kSRows;
  for (int gi = 0; gi < group; ++gi) {
    const int h = kvh * group + gi;
    if (h >= nH) break;
    const size_t bh = (size_t)b * nH + h;
    for (int t0 = first; t0 < T; t0 += kSRows) {
      __syncthreads();
      for (int e = threadIdx.x; e < kSRows * dH; e += kSRows) {
        const int r = e / dH, d = e % dH, t = t0 + r;
        const size_t qrow = ((size_t)b * T + t) * qD + (size_t)h * dH + d;
        Qs[r][d] = t < T ? Q[qrow] : 0.f;
        Gs[r][d] = t < T ? dO[qrow] : 0.f;
      }
      {
        const int t = t0 + threadIdx.x;
        Ls[threadIdx.x] = t < T ? lse[bh * T + t] : 0.f;
        Ds[threadIdx.x] = t < T ? Dq[bh * T + t] : 0.f;
      }
      __syncthreads();
      if (valid) {
        const int tbeg = max(j, t0), tend = min(T - 1, t0 + kSRows - 1);
        for (int t = tbeg; t <= tend; ++t) {
          const int r = t - t0;
          float s = 0.f, dp = 0.f;
#pragma unroll
          for (int d = 0; d < kSMax; ++d)
            if (d < dH) {
              s += Qs[r][d] * k[d];
              dp += Gs[r][d] * v[d];
            }
          const float p = expf(s * scale - Ls[r]);
          const float ds = p * (dp - Ds[r]);
#pragma unroll
          for (int d = 0; d < kSMax; ++d)
            if (d < dH) {
              dv[d] += p * Gs[r][d];
              dk[d] += ds * Qs[r][d];
            }
        }
      }
    }
  }
  if (valid) {
#pragma unroll
    for (int d = 0; d < kSMax; ++d)
      if (d < dH) {
        const float a = dk[d] * scale, c = dv[d];
        dK[krow + d] = beta_k ? dK[krow + d] + a : a;
        dV[krow + d] = beta_v ? dV[krow + d] + c : c;
      }
  }
}

// ═══════════════ head sizes above 128: attention as GEMM launches ═══════════════
// For a chunk of (sample, head) problems at once (batched GEMM launches on
// gemm.hip's split-fp16 128x128 tiles): S = Q_h·K_kvh^T over the whole T×T
// square, a row kernel for the causal softmax, O_h = P·V_kvh.  The backward
// recomputes S, takes P from the saved lse, forms dP = dO_h·V_kvh^T, then per
// row D = Σ_j P·dP (the reference's dotP) and dS = P∘(dP − D)·scale, and
// dQ_h = dS·K_kvh, dK_h = dS^T·Q_h, dV_h = P^T·dO_h, the last two summed over
// a GQA group in head order.  The T×T matrices (4·T² bytes per problem) live
// in chunk workspaces.  The GEMMs work on their causal halves only: the S and
// dP launches skip the 128×128 tiles past the diagonal (never read), the row
// kernels zero P and dS past each row's diagonal, and the products with P or
// dS sum only the k range where those can be nonzero.
constexpr int kRowThreads = 256;

__device__ __forceinline__ float row_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Row t (blockIdx.x) of problem zl (blockIdx.y): P = exp(S·scale − m) /
// Σ_{j<=t} exp(S·scale − m) for j <= t (fp32 exponentials, fp64 sum in a
// fixed order), 0 past t, over S; lse[zl*T + t] = m + ln Σ.
__global__ void __launch_bounds__(kRowThreads) attn_rows_softmax(float* __restrict__ S, float* __restrict__ lse, int T,
                                                                 float scale) {
  const int t = blockIdx.x, w = threadIdx.x >> 6;
  float* row = S + ((size_t)blockIdx.y * T + t) * T;
  __shared__ float wm[kRowThreads / 64];
  __shared__ double ws[kRowThreads / 64];
  float m = -INFINITY;
  for (int j = threadIdx.x; j <= t; j += kRowThreads) m = fmaxf(m, row[j] * scale);
  m = fg_wave_max(m);
  if ((threadIdx.x & 63) == 0) wm[w] = m;
  __syncthreads();
  m = wm[0];
  for (int i = 1; i < kRowThreads / 64; ++i) m = fmaxf(m, wm[i]);
  double sum = 0.0;
  for (int j = threadIdx.x; j <= t; j += kRowThreads) sum += (double)row_exp2((row[j] * scale - m) * kLog2e);
  sum = fg_wave_sum_d(sum);
  if ((threadIdx.x & 63) == 0) ws[w] = sum;
  __syncthreads();
  sum = 0.0;
  for (int i = 0; i < kRowThreads / 64; ++i) sum += ws[i];
  const double inv = 1.0 / sum;
  for (int j = threadIdx.x; j < T; j += kRowThreads)
    row[j] = j <= t ? (float)((double)row_exp2((row[j] * scale - m) * kLog2e) * inv) : 0.f;
  if (threadIdx.x == 0) lse[(size_t)blockIdx.y * T + t] = (float)((double)m + log(sum));
}

// Row t of problem zl in the backward: P = exp(S·scale − lse) for j <= t, 0
// past t, over S; D = Σ_j P·dP (fp64, fixed order); dS = P∘(dP − D)·scale
// over dP.
__global__ void __launch_bounds__(kRowThreads) attn_rows_softmax_bwd(float* __restrict__ S, float* __restrict__ dP,
                                                                     const float* __restrict__ lse, int T,
                                                                     float scale) {
  const int t = blockIdx.x, w = threadIdx.x >> 6;
  const size_t r = (size_t)blockIdx.y * T + t;
  float* srow = S + r * T;
  float* drow = dP + r * T;
  __shared__ double ws[kRowThreads / 64];
  const float l = lse[r];
  double d = 0.0;
  for (int j = threadIdx.x; j < T; j += kRowThreads) {
    const float p = j <= t ? row_exp2((srow[j] * scale - l) * kLog2e) : 0.f;
    srow[j] = p;
    if (j <= t) d += (double)p * drow[j];  // past t: tiles the causal GEMMs leave unwritten
  }
  d = fg_wave_sum_d(d);
  if ((threadIdx.x & 63) == 0) ws[w] = d;
  __syncthreads();
  d = 0.0;
  for (int i = 0; i < kRowThreads / 64; ++i) d += ws[i];
  for (int j = threadIdx.x; j < T; j += kRowThreads)
    drow[j] = j <= t ? (float)((double)srow[j] * ((double)drow[j] - d) * scale) : 0.f;
}

// The chunk's per-problem [T][dH] results into their column blocks of a
// [B*T][ld] tensor: problem zl (blockIdx.y) is z = z0 + zl = b * nh + h and
// lands in head h / g of sample b, the sum of the g consecutive problems of a
// group (zl = g·k .. g·k + g − 1, added in that order) when g > 1 — the
// launch then covers nz / g groups; dst (+)= the sum.  A null src writes 0
// (kv heads that no query head reaches).
__global__ void __launch_bounds__(256) attn_head_cols(float* __restrict__ dst, int ld, const float* __restrict__ src,
                                                      int T, int dH, int nh, int z0, int g, int beta) {
  const int64_t n = (int64_t)T * dH;
  const int zl = blockIdx.y * g, z = z0 + zl, b = z / nh, hh = (z - b * nh) / g;
  float* out = dst + (size_t)b * T * ld + (size_t)hh * dH;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t t = e / dH;
    float v = 0.f;
    if (src)
      for (int k = 0; k < g; ++k) v += src[(size_t)(zl + k) * n + e];
    float* y = out + t * ld + (e - t * dH);
    *y = beta ? *y + v : v;
  }
}

// ═════════════════════════ MFMA kernels (dH in {32,64,96,128}) ═════════════════════════
typedef float f32x16 __attribute__((ext_vector_type(16)));
constexpr int kBlk = 32;             // keys / queries per MFMA block
constexpr int kWaves = 4;
constexpr int kMThreads = 64 * kWaves;

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int v = 0; v < 16; ++v) z[v] = 0.f;
  return z;
}
// Row (within a 32-block) held by accumulator register v of a lane in half h.
__device__ __forceinline__ int acc_row(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

// The wave index as a scalar: branches on it (causal block ranges, diagonal
// blocks) are then uniform jumps, not per-lane selects.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Buffer resource over one block's rows (wave-uniform base, raw addressing,
// 32-bit data format): the loads below then take a 32-bit per-lane byte
// offset and an SGPR row offset, with no 64-bit address arithmetic per load.
// Used only for blocks wholly inside the tensor.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_rsrc(const float* blk) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(blk), 0, 0x7fffffff, 0x00020000);
}
// The LLVM intrinsics by name: this compiler lowers
// __builtin_amdgcn_raw_buffer_load_b128 to a single-dword load splatted over
// the four lanes of the result.
typedef float f32x4v __attribute__((ext_vector_type(4)));
__device__ f32x4v raw_buf_load_v4f32(__amdgpu_buffer_rsrc_t rs, int voff, int soff, int aux) __asm(
    "llvm.amdgcn.raw.ptr.buffer.load.v4f32");
__device__ float raw_buf_load_f32(__amdgpu_buffer_rsrc_t rs, int voff, int soff, int aux) __asm(
    "llvm.amdgcn.raw.ptr.buffer.load.f32");
__device__ __forceinline__ float4 buf_f4(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  const f32x4v w = raw_buf_load_v4f32(rs, (int)off, 0, 0);
  return make_float4(w.x, w.y, w.z, w.w);
}
__device__ __forceinline__ float buf_f1(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t soff) {
  return raw_buf_load_f32(rs, (int)off, (int)soff, 0);
}

// A 32 x DH block (rows r0.., row stride ld) held in registers, DH/32 float4
// per thread; rows >= rmax read as zero (clamped address + select).  Blocks
// wholly below rmax (all but a ragged last one) take the plain loads: the
// branch is uniform over the workgroup.
template <int DH>
struct BlockLoader {
  static constexpr int kPer = DH / 32;
  float4 r[kPer];
  __device__ __forceinline__ void load(const float* __restrict__ base, size_t ld, int r0, int rmax) {
    if (r0 + kBlk <= rmax) {
      const __amdgpu_buffer_rsrc_t rs = block_rsrc(base + (size_t)r0 * ld);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int e = threadIdx.x + kMThreads * u;
        const int row = e / (DH / 4), c4 = e % (DH / 4);
        r[u] = buf_f4(rs, (uint32_t)(row * (int)ld + c4 * 4) * 4u);
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int e = threadIdx.x + kMThreads * u;
      const int row = e / (DH / 4), c4 = e % (DH / 4);
      const int rr = r0 + row;
      const int rc = rr < rmax ? rr : rmax - 1;
      const float4 v = *reinterpret_cast<const float4*>(base + (size_t)rc * ld + c4 * 4);
      r[u] = rr < rmax ? v : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
};

// Row fragment straight from global memory (row r, bounded), times a factor.
template <int DH>
__device__ __forceinline__ void glb_rowfrag(float (&f)[DH / 2], const float* __restrict__ base, size_t ld, int r,
                                            int rmax, float mul) {
  const int lane = threadIdx.x & 63;
  const bool ok = r < rmax;
  const float4* p = reinterpret_cast<const float4*>(base + (size_t)(ok ? r : rmax - 1) * ld + (lane >> 5) * (DH / 2));
#pragma unroll
  for (int q = 0; q < DH / 8; ++q) {
    const float4 v = p[q];
    const float m = ok ? mul : 0.f;
    f[4 * q] = v.x * m; f[4 * q + 1] = v.y * m; f[4 * q + 2] = v.z * m; f[4 * q + 3] = v.w * m;
  }
}

// Writes a transposed accumulator (rows = d, cols = row index lane%32) to
// out[row][d] (+ beta), 16 d values per 32-column tile as float4.
template <int DH>
__device__ __forceinline__ void store_T(const f32x16 (&acc)[DH / 32], float* __restrict__ base, size_t ld, int r,
                                        int rmax, float mul, int beta, int esc = 0) {
  const int lane = threadIdx.x & 63, h = lane >> 5;
  if (r >= rmax) return;
  float* row = base + (size_t)r * ld;
#pragma unroll
  for (int dt = 0; dt < DH / 32; ++dt)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const int d0 = 32 * dt + 8 * v4 + 4 * h;
      float4 val = make_float4(__builtin_amdgcn_ldexpf(acc[dt][4 * v4], esc) * mul,
                               __builtin_amdgcn_ldexpf(acc[dt][4 * v4 + 1], esc) * mul,
                               __builtin_amdgcn_ldexpf(acc[dt][4 * v4 + 2], esc) * mul,
                               __builtin_amdgcn_ldexpf(acc[dt][4 * v4 + 3], esc) * mul);
      float4* p = reinterpret_cast<float4*>(row + d0);
      if (beta) {
        const float4 o = *p;
        val.x += o.x; val.y += o.y; val.z += o.z; val.w += o.w;
      }
      *p = val;
    }
}

// Row strides (floats) of the MFMA kernels' operands — Q, K/V (same layout),
// O/dO, dQ and dK/dV — and the optional RoPE^T of the dQ / dK stores.  The
// attention of a fused projection reads q, k, v as column blocks of one
// qkv[rows, (nH + 2 nKV) dH] buffer (stride (nH + 2 nKV) dH) and writes its
// gradient [R^T dQ | R^T dK | dV] into the matching qkv gradient.
struct AttnLd {
  int ldq, ldk, ldo, ldgq, ldgk;
  const double* rc;  // null: plain stores
  const double* rs;
  int pos0, posStride;
};

// store_T (beta = 0) with each (even, odd) d pair turned back by the angle of
// row grow's position: (a c + b s, -a s + b c) in fp64 from the fp32 values
// store_T would write — the ropeRows backward (tensor.js:150-166) of them.
typedef double d2v __attribute__((ext_vector_type(2)));
template <int DH>
__device__ __forceinline__ void store_T_rope(const f32x16 (&acc)[DH / 32], float* __restrict__ base, size_t ld,
                                             int r, int rmax, float mul, const AttnLd& L, int64_t grow, int esc) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, h = lane >> 5;
  if (r >= rmax) return;
  const int64_t pos = L.pos0 + (L.posStride > 0 ? grow % L.posStride : grow);
  const double* cr = L.rc + pos * (DH / 2);
  const double* sr = L.rs + pos * (DH / 2);
  float* row = base + (size_t)r * ld;
#pragma unroll
  for (int dt = 0; dt < DH / 32; ++dt)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const int d0 = 32 * dt + 8 * v4 + 4 * h;
      const float g[4] = {__builtin_amdgcn_ldexpf(acc[dt][4 * v4], esc) * mul,
                          __builtin_amdgcn_ldexpf(acc[dt][4 * v4 + 1], esc) * mul,
                          __builtin_amdgcn_ldexpf(acc[dt][4 * v4 + 2], esc) * mul,
                          __builtin_amdgcn_ldexpf(acc[dt][4 * v4 + 3], esc) * mul};
      // the two pairs' angles as one 16-byte load each (d0 / 2 is even)
      const d2v c2 = *reinterpret_cast<const d2v*>(cr + d0 / 2), s2 = *reinterpret_cast<const d2v*>(sr + d0 / 2);
      float o[4];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const double cc = c2[q], ss = s2[q];
        const double a = g[2 * q], b = g[2 * q + 1];
        o[2 * q] = (float)(a * cc + b * ss);
        o[2 * q + 1] = (float)(-a * ss + b * cc);
      }
      *reinterpret_cast<float4*>(row + d0) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

// ═════════════ split-fp16 MFMA kernels (dH in {32, 64, 96, 128}) ═════════════
// Same formulation as above on v_mfma_f32_32x32x16_f16 with every operand
// scaled by a power of two and split into its fp16 hi and lo pieces
// (f16split.h): three MFMAs per 16-wide k-chunk.  The powers of two come from
// the operands' largest magnitudes (partial maxima from absmax_parts, folded
// per wave): Q, K, V and dO each have their own; P = exp2(s - m) <= 1 is
// scaled by 2^14; dS = P (dP - D) is scaled from the bound
// |dS| <= 2 dH max|dO| max|V| (|dP| <= dH max|dO| max|V| and D is a convex
// combination of one row of dP).  Accumulators hold the product of their
// operands' powers of two, which the score code and the stores take off
// exactly.
//
// LDS tiles hold the pieces:
//  * row layout  [32 rows][hi DH | lo DH] fp16 + 16 B (4*DH + 16 bytes per
//    row, an odd number of 16-byte slots): a fragment = 8 consecutive d of
//    one row = one ds_read_b128 per piece;
//  * column layout [DH rows (d)][hi 32 | lo 32] fp16 + 16 B (144 B per row)
//    with the 32 keys (queries) of the block in "accumulator order":
//    position 16c + 8h + e holds row acc_row(8c + e, h) = 16c + 8(e/4) + 4h +
//    e%4, i.e. bits 2 and 3 of the row index swapped.  Then the 8 values a
//    lane of half h holds in accumulator registers 8c..8c+7 are the B operand
//    of chunk c, and the matching A fragment is 8 consecutive positions.
namespace x3 {

using fg::f32x16;
using fg::f16x8;
using fg::Pair;

// v_exp_f32 directly: results below 2^-126 flush to zero (probabilities that
// small add nothing to an fp32 sum), exp2(-inf) = 0 for masked scores.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
using fg::u32x2;
using fg::u32x4;

constexpr int kPExp = 14;  // P <= 1 is scaled by 2^14 before its split

// Partial maxima of the kernels' operands (FG_XP_PARTS floats each).
struct AttnXp {
  const float* q;
  const float* k;
  const float* v;
  const float* g;  // dO (backward only)
};

// Exponents of one launch, the same in every wave (see the section comment).
struct Exps {
  int q, k, v, g;  // plain operands
  int qs, ks;      // Q or K times scale * log2(e)
  int ds;          // dS
};
template <int DH>
__device__ __forceinline__ Exps attn_exps(const AttnXp& X, float scale, bool bwd) {
  const int qq = fg::bound_q(fg::fold_parts(X.q)), qk = fg::bound_q(fg::fold_parts(X.k));
  const int qv = fg::bound_q(fg::fold_parts(X.v));
  const int qg = bwd ? fg::bound_q(fg::fold_parts(X.g)) : fg::kQZero;
  const int qc = fg::bound_q(scale * kLog2e);
  constexpr int kLogDh = DH <= 32 ? 5 : DH <= 64 ? 6 : 7;  // 2^kLogDh >= DH
  Exps e;
  e.q = fg::exponent_of_bound(qq);
  e.k = fg::exponent_of_bound(qk);
  e.v = fg::exponent_of_bound(qv);
  e.g = fg::exponent_of_bound(qg);
  e.qs = fg::exponent_of_bound(qq + qc);
  e.ks = fg::exponent_of_bound(qk + qc);
  e.ds = fg::exponent_of_bound(qg + qv + 1 + kLogDh);
  return e;
}

template <int DH>
struct Tile {
  static constexpr int kRS = 4 * DH + 16;    // row-layout bytes per row
  static constexpr int kRow = kBlk * kRS;     // row-layout block bytes
  static constexpr int kCS = 144;            // column-layout bytes per d
  static constexpr int kCol = DH * kCS;       // column-layout block bytes
};

__device__ __forceinline__ int col_pos(int r) {  // row -> position in the column layout
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

// Row-layout store of a 32 x DH block from BlockLoader registers (float4 per
// (row, d-quad)), scaled by 2^e: split, two ds_write_b64.
template <int DH>
__device__ __forceinline__ void store_rows2(char* __restrict__ lds, const BlockLoader<DH>& L, int e) {
#pragma unroll
  for (int u = 0; u < BlockLoader<DH>::kPer; ++u) {
    const int el = threadIdx.x + kMThreads * u;
    const int row = el / (DH / 4), c4 = el % (DH / 4);
    u32x2 h, l;
    fg::split4h(L.r[u].x, L.r[u].y, L.r[u].z, L.r[u].w, e, h, l);
    char* p = lds + row * Tile<DH>::kRS + c4 * 8;
    *reinterpret_cast<u32x2*>(p) = h;
    *reinterpret_cast<u32x2*>(p + 2 * DH) = l;
  }
}

// Column-layout loader: unit (d, c, h) = the 8 rows 16c + 4h + {0..3, 8..11}
// of column d (positions 16c + 8h .. +7); 4*DH units over the workgroup.
template <int DH>
struct ColLoader {
  static constexpr int kUnits = 4 * DH;
  static constexpr int kPer = (kUnits + kMThreads - 1) / kMThreads;  // dH 96: 384 units, the second pass half idle
  float v[kPer][8];
  __device__ __forceinline__ void load(const float* __restrict__ base, size_t ld, int r0, int rmax) {
    if (r0 + kBlk <= rmax) {  // whole block in range (uniform branch)
      const __amdgpu_buffer_rsrc_t rs = block_rsrc(base + (size_t)r0 * ld);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int unit = threadIdx.x + kMThreads * u;
        // idle threads (DH = 32) address the block's first rows, never past it
        const int d = unit % DH, g = unit < kUnits ? unit / DH : 0, c = g >> 1, h = g & 1;
        const uint32_t off = (uint32_t)((16 * c + 4 * h) * (int)ld + d) * 4u;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[u][e] = (unit < kUnits) ? buf_f1(rs, off, (uint32_t)((e & 3) + 8 * (e >> 2)) * (uint32_t)ld * 4u) : 0.f;
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int unit = threadIdx.x + kMThreads * u;
      const int d = unit % DH, g = unit / DH, c = g >> 1, h = g & 1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int rr = r0 + 16 * c + 4 * h + (e & 3) + 8 * (e >> 2);
        const int rc = rr < rmax ? rr : rmax - 1;
        const float x = (unit < kUnits) ? base[(size_t)rc * ld + d] : 0.f;
        v[u][e] = rr < rmax ? x : 0.f;
      }
    }
  }
  // scaled by 2^ex and split
  __device__ __forceinline__ void store(char* __restrict__ lds, int ex) const {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int unit = threadIdx.x + kMThreads * u;
      if (unit >= kUnits) break;
      const int d = unit % DH, g = unit / DH, c = g >> 1, h = g & 1;
      u32x4 hp, lp;
      fg::split8h(v[u], ex, hp, lp);
      char* p = lds + d * Tile<DH>::kCS + (16 * c + 8 * h) * 2;
      *reinterpret_cast<u32x4*>(p) = hp;
      *reinterpret_cast<u32x4*>(p + 64) = lp;
    }
  }
};

// Fragment pieces of a row-layout block: row lane%32, d = 16c + 8*(lane/32) .. +7.
template <int DH>
__device__ __forceinline__ Pair row_pair(const char* lds, int c) {
  const int lane = threadIdx.x & 63;
  return fg::lds_pair(lds + (lane & 31) * Tile<DH>::kRS + (16 * c + 8 * (lane >> 5)) * 2, 2 * DH);
}
// Fragment pieces of a column-layout block: d = 32*dt + lane%32, positions 16c + 8*(lane/32) .. +7.
template <int DH>
__device__ __forceinline__ Pair col_pair(const char* lds, int dt, int c) {
  const int lane = threadIdx.x & 63;
  return fg::lds_pair(lds + (32 * dt + (lane & 31)) * Tile<DH>::kCS + (16 * c + 8 * (lane >> 5)) * 2, 64);
}
// Per-lane fragment pieces of global row r (bounded), times a factor, scaled
// by 2^e: chunk c holds d = 16c + 8*(lane/32) .. +7.
template <int DH>
__device__ __forceinline__ void glb_pairs(Pair (&f)[DH / 16], const float* __restrict__ base, size_t ld, int r,
                                          int rmax, float mul, int e) {
  const int lane = threadIdx.x & 63;
  const bool ok = r < rmax;
  const float m = ok ? mul : 0.f;
  const float* row = base + (size_t)(ok ? r : rmax - 1) * ld + 8 * (lane >> 5);
#pragma unroll
  for (int c = 0; c < DH / 16; ++c) {
    const float4 a = *reinterpret_cast<const float4*>(row + 16 * c);
    const float4 b = *reinterpret_cast<const float4*>(row + 16 * c + 4);
    const float x[8] = {a.x * m, a.y * m, a.z * m, a.w * m, b.x * m, b.y * m, b.z * m, b.w * m};
    f[c] = fg::split_pair(x, e);
  }
}
// Accumulator registers 8c..8c+7 (the B operand of chunk c) as pieces, scaled by 2^e.
__device__ __forceinline__ Pair acc_pair(const f32x16& s, int c, int e) {
  const float x[8] = {s[8 * c], s[8 * c + 1], s[8 * c + 2], s[8 * c + 3],
                      s[8 * c + 4], s[8 * c + 5], s[8 * c + 6], s[8 * c + 7]};
  return fg::split_pair(x, e);
}
// Accumulator values times 2^e (exact).
__device__ __forceinline__ void scale_acc(f32x16& s, int e) {
#pragma unroll
  for (int v = 0; v < 16; ++v) s[v] = __builtin_amdgcn_ldexpf(s[v], e);
}
// The factor 2^e that the softmax folds into its first fma (x * 2^e - m
// rounds once, as ldexp then subtract does), or 1 after scaling the
// accumulators here when 2^e is not a normal float (wave-uniform).
__device__ __forceinline__ float fold_scale(f32x16& s, int e) {
  if (e >= -126 && e <= 126) return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
  scale_acc(s, e);
  return 1.f;
}

// ───────── forward ─────────
// Three workgroups per CU at dH <= 64 (168 VGPRs, 52 KB of LDS each): 6% faster
// than two at B8 T2048 nH16 nKV4, the same at B8 T1024 nH12.
template <int DH>
__global__ void __launch_bounds__(kMThreads, DH <= 32 ? 4 : DH <= 64 ? 3 : DH <= 96 ? 2 : 1)
    attn_fwd(float* __restrict__ O, float* __restrict__ lse, const float* __restrict__ Q,
             const float* __restrict__ K, const float* __restrict__ V, int T, int nH, int nKV, float scale,
             AttnLd L, AttnXp X) {
  __shared__ __attribute__((aligned(16))) char Ks[2][Tile<DH>::kRow];
  __shared__ __attribute__((aligned(16))) char Vt[2][Tile<DH>::kCol];
  const Exps E = attn_exps<DH>(X, scale, false);
  const int nqb = (T + 127) / 128;
  const int qblk = nqb - 1 - blockIdx.y;  // longest causal prefix first, across all heads
  const int bh = blockIdx.x, b = bh / nH, h = bh % nH;
  const int group = nH / nKV > 1 ? nH / nKV : 1, kvh = h / group;
  const size_t qD = L.ldq, kvD = L.ldk, oD = L.ldo;
  const int wave = wave_id(), lane = threadIdx.x & 63, hl = lane >> 5;
  const int q0w = qblk * 128 + wave * 32;
  const int myq = q0w + (lane & 31);

  const float* Qb = Q + (size_t)b * T * qD + (size_t)h * DH;
  const float* Kb = K + (size_t)b * T * kvD + (size_t)kvh * DH;
  const float* Vb = V + (size_t)b * T * kvD + (size_t)kvh * DH;

  Pair qf[DH / 16];
  glb_pairs<DH>(qf, Qb, qD, myq, T, scale * kLog2e, E.qs);

  f32x16 oacc[DH / 32];
#pragma unroll
  for (int dt = 0; dt < DH / 32; ++dt) oacc[dt] = zero16();
  float m = -INFINITY, l = 0.f;

  const int nkb = min((T + kBlk - 1) / kBlk, qblk * 4 + 4);
  const int mylast = q0w / kBlk;
  BlockLoader<DH> lk;
  ColLoader<DH> lv;
  lk.load(Kb, kvD, 0, T);
  lv.load(Vb, kvD, 0, T);
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    store_rows2<DH>(Ks[buf], lk, E.k);
    lv.store(Vt[buf], E.v);
    __syncthreads();
    if (kb + 1 < nkb) {
      lk.load(Kb, kvD, (kb + 1) * kBlk, T);
      lv.load(Vb, kvD, (kb + 1) * kBlk, T);
    }
    if (kb <= mylast) {
      // S^T[key][query] = K · Q^T (log2 units), two accumulation chains
      f32x16 s0 = zero16(), s1 = zero16();
#pragma unroll
      for (int c = 0; c < DH / 16; c += 2) {
        s0 = fg::mfma3(row_pair<DH>(Ks[buf], c), qf[c], s0);
        s1 = fg::mfma3(row_pair<DH>(Ks[buf], c + 1), qf[c + 1], s1);
      }
      f32x16 s = s0 + s1;
      const float sc = fold_scale(s, -(E.qs + E.k));  // s * sc: log2 units
      const bool diag = (kb == mylast) || ((kb + 1) * kBlk > T);
      if (diag) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = kb * kBlk + acc_row(v, hl);
          if (key > myq || key >= T) s[v] = -INFINITY;
        }
      }
      float bm = s[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) bm = fmaxf(bm, s[v]);
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64)) * sc;
      const float mn = fmaxf(m, bm);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = fast_exp2(m - mref);
      float ls = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        s[v] = fast_exp2(__builtin_fmaf(s[v], sc, -mref));
        ls += s[v];
      }
      ls += __shfl_xor(ls, 32, 64);
      l = l * alpha + ls;
      m = mn;
      if (__any(alpha != 1.f)) {  // the running max moved for some query of the wave
#pragma unroll
        for (int dt = 0; dt < DH / 32; ++dt) oacc[dt] *= alpha;
      }
      // O^T[d][query] += V^T[d][key] · P^T[key][query]
      const Pair p0 = acc_pair(s, 0, kPExp), p1 = acc_pair(s, 1, kPExp);
#pragma unroll
      for (int dt = 0; dt < DH / 32; ++dt) {
        oacc[dt] = fg::mfma3(col_pair<DH>(Vt[buf], dt, 0), p0, oacc[dt]);
        oacc[dt] = fg::mfma3(col_pair<DH>(Vt[buf], dt, 1), p1, oacc[dt]);
      }
    }
    // No barrier here: the next store goes to the other buffer, and the one
    // after it (back to this buffer) follows the next iteration's barrier,
    // which every wave reaches only once it is done reading this one.
  }
  const float il = 1.f / l;
  store_T<DH>(oacc, O + (size_t)b * T * oD + (size_t)h * DH, oD, myq, T, il, 0, -(kPExp + E.v));
  if (hl == 0 && myq < T) lse[(size_t)bh * T + myq] = (m + log2f(l)) * kLn2;
}


// ───────── backward: dQ, and D = rowsum(dO∘O) for the dK/dV kernel ─────────
// Half of D = rowsum(dO∘O) for one query: the d values 16c + 8·half .. +7 of
// every 16-wide chunk (orow / grow point at the row's first of them).  The
// dQ body (two half-waves) and attn_d_pre (one thread) add the two halves.
template <int DH>
__device__ __forceinline__ float d_half(const float* __restrict__ orow, const float* __restrict__ grow) {
#pragma clang fp contract(off)
  float part = 0.f;
#pragma unroll
  for (int c = 0; c < DH / 16; ++c) {
    const float4 o0 = *reinterpret_cast<const float4*>(orow + 16 * c);
    const float4 o1 = *reinterpret_cast<const float4*>(orow + 16 * c + 4);
    const float4 g0 = *reinterpret_cast<const float4*>(grow + 16 * c);
    const float4 g1 = *reinterpret_cast<const float4*>(grow + 16 * c + 4);
    part += (o0.x * g0.x + o0.y * g0.y) + (o0.z * g0.z + o0.w * g0.w);
    part += (o1.x * g1.x + o1.y * g1.y) + (o1.z * g1.z + o1.w * g1.w);
  }
  return part;
}

// D for every (sample, head, query) before the merged backward launch: one
// thread per (row, head), the same sums as the dQ body forms.
template <int DH>
__global__ void __launch_bounds__(256) attn_d_pre(float* __restrict__ Dq, const float* __restrict__ dO,
                                                  const float* __restrict__ O, int B, int T, int nH, int ldo) {
  const int64_t n = (int64_t)B * T * nH;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t row = e / nH;
    const int h = (int)(e - row * nH);
    const size_t base = (size_t)row * ldo + (size_t)h * DH;
    const float d = d_half<DH>(O + base, dO + base) + d_half<DH>(O + base + 8, dO + base + 8);
    const int64_t b = row / T, t = row - b * T;
    Dq[(b * nH + h) * T + t] = d;
  }
}

// LDS bytes of the two backward bodies (they share one buffer in the merged launch).
template <int DH>
struct BwdLds {
  static constexpr int kDq = 2 * Tile<DH>::kRow + 2 * Tile<DH>::kCol + 2 * Tile<DH>::kRow;
  static constexpr int kDkv = 2 * Tile<DH>::kRow + 2 * Tile<DH>::kCol + 2 * kBlk * 4;
  static constexpr int kMax = kDq > kDkv ? kDq : kDkv;
};

// dQ of query block qblk (128 queries) of (sample, head) bh.  With compute_d
// it also forms D = rowsum(dO∘O) of its queries into Dq; otherwise it reads
// D from Dq.
template <int DH>
__device__ __forceinline__ void dq_body(char* __restrict__ lds, int qblk, int bh, bool compute_d,
                                        float* __restrict__ dQ, int beta, float* __restrict__ Dq,
                                        const float* __restrict__ dO, const float* __restrict__ O,
                                        const float* __restrict__ Q, const float* __restrict__ K,
                                        const float* __restrict__ V, const float* __restrict__ lse, int T, int nH,
                                        int nKV, float scale, const AttnLd& L, const Exps& E) {
  char (*Ks)[Tile<DH>::kRow] = reinterpret_cast<char (*)[Tile<DH>::kRow]>(lds);
  char (*Kc)[Tile<DH>::kCol] = reinterpret_cast<char (*)[Tile<DH>::kCol]>(lds + 2 * Tile<DH>::kRow);
  char (*Vs)[Tile<DH>::kRow] = reinterpret_cast<char (*)[Tile<DH>::kRow]>(lds + 2 * Tile<DH>::kRow + 2 * Tile<DH>::kCol);
  const int b = bh / nH, h = bh % nH;
  const int group = nH / nKV > 1 ? nH / nKV : 1, kvh = h / group;
  const size_t qD = L.ldq, kvD = L.ldk, oD = L.ldo;
  const int wave = wave_id(), lane = threadIdx.x & 63, hl = lane >> 5;
  const int q0w = qblk * 128 + wave * 32;
  const int myq = q0w + (lane & 31);

  const float* Qb = Q + (size_t)b * T * qD + (size_t)h * DH;
  const float* dOb = dO + (size_t)b * T * oD + (size_t)h * DH;
  const float* Kb = K + (size_t)b * T * kvD + (size_t)kvh * DH;
  const float* Vb = V + (size_t)b * T * kvD + (size_t)kvh * DH;

  Pair qf[DH / 16], gf[DH / 16];
  glb_pairs<DH>(qf, Qb, qD, myq, T, scale * kLog2e, E.qs);
  glb_pairs<DH>(gf, dOb, oD, myq, T, 1.f, E.g);
  // D = rowsum(dO∘O) of this lane's query: the two half-waves hold the two
  // halves of each 16-wide d chunk; the dK/dV kernel reads D from Dq.
  float Dt;
  if (!compute_d) {
    Dt = myq < T ? Dq[(size_t)bh * T + myq] : 0.f;
  } else {
    const float* Ob = O + (size_t)b * T * oD + (size_t)h * DH;
    const int rq = myq < T ? myq : T - 1;
    const float part = d_half<DH>(Ob + (size_t)rq * oD + 8 * hl, dOb + (size_t)rq * oD + 8 * hl);
    Dt = part + __shfl_xor(part, 32, 64);
    if (myq >= T) Dt = 0.f;
    else if (hl == 0) Dq[(size_t)bh * T + myq] = Dt;
  }
  const float L2 = myq < T ? lse[(size_t)bh * T + myq] * kLog2e : 0.f;

  f32x16 dq[DH / 32];
#pragma unroll
  for (int dt = 0; dt < DH / 32; ++dt) dq[dt] = zero16();

  const int nkb = min((T + kBlk - 1) / kBlk, qblk * 4 + 4);
  const int mylast = q0w / kBlk;
  BlockLoader<DH> lk, lv;
  ColLoader<DH> lkc;
  lk.load(Kb, kvD, 0, T);
  lkc.load(Kb, kvD, 0, T);
  lv.load(Vb, kvD, 0, T);
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    store_rows2<DH>(Ks[buf], lk, E.k);
    lkc.store(Kc[buf], E.k);
    store_rows2<DH>(Vs[buf], lv, E.v);
    __syncthreads();
    if (kb + 1 < nkb) {
      lk.load(Kb, kvD, (kb + 1) * kBlk, T);
      lkc.load(Kb, kvD, (kb + 1) * kBlk, T);
      lv.load(Vb, kvD, (kb + 1) * kBlk, T);
    }
    if (kb <= mylast) {
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int c = 0; c < DH / 16; ++c) {
        s = fg::mfma3(row_pair<DH>(Ks[buf], c), qf[c], s);   // S^T = K·Q^T
        dp = fg::mfma3(row_pair<DH>(Vs[buf], c), gf[c], dp);  // dP^T = V·dO^T
      }
      const float sc = fold_scale(s, -(E.k + E.qs)), gc = fold_scale(dp, -(E.v + E.g));
      // Masks only on the diagonal / ragged key block: below it every key
      // precedes every query of the wave and lies inside the sequence.
      if ((kb == mylast) || ((kb + 1) * kBlk > T)) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = kb * kBlk + acc_row(v, hl);
          float p = fast_exp2(__builtin_fmaf(s[v], sc, -L2));
          if (key > myq || key >= T || myq >= T) p = 0.f;
          s[v] = p * __builtin_fmaf(dp[v], gc, -Dt);  // dS^T
        }
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) s[v] = fast_exp2(__builtin_fmaf(s[v], sc, -L2)) * __builtin_fmaf(dp[v], gc, -Dt);
      }
      // dQ^T[d][query] += K^T[d][key] · dS^T[key][query]
      const Pair d0 = acc_pair(s, 0, E.ds), d1 = acc_pair(s, 1, E.ds);
#pragma unroll
      for (int dt = 0; dt < DH / 32; ++dt) {
        dq[dt] = fg::mfma3(col_pair<DH>(Kc[buf], dt, 0), d0, dq[dt]);
        dq[dt] = fg::mfma3(col_pair<DH>(Kc[buf], dt, 1), d1, dq[dt]);
      }
    }
    // double-buffered tiles: no trailing barrier (as in attn_fwd)
  }
  if (L.rc)
    store_T_rope<DH>(dq, dQ + (size_t)b * T * L.ldgq + (size_t)h * DH, L.ldgq, myq, T, scale, L,
                     (int64_t)b * T + myq, -(E.k + E.ds));
  else
    store_T<DH>(dq, dQ + (size_t)b * T * L.ldgq + (size_t)h * DH, L.ldgq, myq, T, scale, beta, -(E.k + E.ds));
}

// ───────── backward: dK, dV (per key block, the GQA group's heads in registers) ─────────
template <int DH>
__device__ __forceinline__ void dkv_body(char* __restrict__ lds, int item, int nbk, float* __restrict__ dK,
                                         int beta_k, float* __restrict__ dV, int beta_v,
                                         const float* __restrict__ dO, const float* __restrict__ Q,
                                         const float* __restrict__ K, const float* __restrict__ V,
                                         const float* __restrict__ lse, const float* __restrict__ Dq, int T, int nH,
                                         int nKV, float scale, const AttnLd& L, float* __restrict__ part,
                                         float* __restrict__ dS, int npairs, const Exps& E) {
  char* Qs = lds;
  char* Qc = lds + Tile<DH>::kRow;
  char* Gs = lds + Tile<DH>::kRow + Tile<DH>::kCol;
  char* Gc = lds + 2 * Tile<DH>::kRow + Tile<DH>::kCol;
  float* Ls = reinterpret_cast<float*>(lds + 2 * Tile<DH>::kRow + 2 * Tile<DH>::kCol);
  float* Ds = Ls + kBlk;
  // Work item (kblk, bk, z): 128 keys of kv head bk % nKV of sample bk / nKV,
  // and with `part` set the query heads of one group member z (GQA: each
  // member's partial dK/dV goes to part, summed in order by attn_dkv_reduce);
  // items in decreasing causal length (key block 0 sees the most queries).
  const int group = nH / nKV > 1 ? nH / nKV : 1;
  const int nz = part ? group : 1;
  const int z = item % nz, bk = (item / nz) % nbk, kblk = item / (nz * nbk);  // nbk = B * nKV
  const int b = bk / nKV, kvh = bk % nKV;
  const size_t qD = L.ldq, kvD = L.ldk, oD = L.ldo;
  const int wave = wave_id(), lane = threadIdx.x & 63, hl = lane >> 5;
  const int k0w = kblk * 128 + wave * 32;
  const int mykey = k0w + (lane & 31);

  const float* Kb = K + (size_t)b * T * kvD + (size_t)kvh * DH;
  const float* Vb = V + (size_t)b * T * kvD + (size_t)kvh * DH;
  Pair kf[DH / 16], vf[DH / 16];
  glb_pairs<DH>(kf, Kb, kvD, mykey, T, scale * kLog2e, E.ks);
  glb_pairs<DH>(vf, Vb, kvD, mykey, T, 1.f, E.v);

  f32x16 dk[DH / 32], dv[DH / 32];
#pragma unroll
  for (int dt = 0; dt < DH / 32; ++dt) {
    dk[dt] = zero16();
    dv[dt] = zero16();
  }
  const int qb0 = kblk * 4;  // first query block that can see these keys
  const int nqblk = (T + kBlk - 1) / kBlk;
  const int per_head = nqblk - qb0;
  const int total = per_head * (part ? 1 : group);
  const int gbase = part ? z : 0;  // the group member of iteration 0
  // Tiles are loaded, split and stored at the top of each iteration (no
  // register prefetch: it would hold 32 more VGPRs through the MFMA phase
  // and spill (measured: 10% slower at dH = 64, 60% at dH = 128); the other
  // resident workgroup hides the loads).
  for (int it = 0; it < total; ++it) {
    const int gi = gbase + it / per_head, qb = qb0 + it % per_head;
    {
      const int h = kvh * group + gi;
      const size_t bh = (size_t)b * nH + h;
      const float* Qb = Q + (size_t)b * T * qD + (size_t)h * DH;
      const float* Gb = dO + (size_t)b * T * oD + (size_t)h * DH;
      float lv = 0.f, dv_ = 0.f;
      const int t = qb * kBlk + (threadIdx.x & (kBlk - 1));
      if constexpr (DH <= 64) {
        // every load of the four tiles (and of lse / D) is issued before the
        // first of them is split and stored: one memory latency per block
        // instead of four in a row (at dH = 128 the registers this holds
        // spill: 9% slower there, so that size loads tile by tile)
        BlockLoader<DH> lq, lg;
        ColLoader<DH> lcq, lcg;
        lq.load(Qb, qD, qb * kBlk, T);
        lg.load(Gb, oD, qb * kBlk, T);
        lcq.load(Qb, qD, qb * kBlk, T);
        lcg.load(Gb, oD, qb * kBlk, T);
        if (threadIdx.x < kBlk) {
          const int tc = t < T ? t : T - 1;
          lv = lse[bh * T + tc] * kLog2e;
          dv_ = Dq[bh * T + tc];
        }
        store_rows2<DH>(Qs, lq, E.q);
        store_rows2<DH>(Gs, lg, E.g);
        lcq.store(Qc, E.q);
        lcg.store(Gc, E.g);
      } else {
        {
          BlockLoader<DH> lq;
          lq.load(Qb, qD, qb * kBlk, T);
          store_rows2<DH>(Qs, lq, E.q);
        }
        {
          BlockLoader<DH> lg;
          lg.load(Gb, oD, qb * kBlk, T);
          store_rows2<DH>(Gs, lg, E.g);
        }
        {
          ColLoader<DH> lc;
          lc.load(Qb, qD, qb * kBlk, T);
          lc.store(Qc, E.q);
        }
        {
          ColLoader<DH> lc;
          lc.load(Gb, oD, qb * kBlk, T);
          lc.store(Gc, E.g);
        }
        if (threadIdx.x < kBlk) {
          const int tc = t < T ? t : T - 1;
          lv = lse[bh * T + tc] * kLog2e;
          dv_ = Dq[bh * T + tc];
        }
      }
      if (threadIdx.x < kBlk) {
        Ls[threadIdx.x] = t < T ? lv : 0.f;
        Ds[threadIdx.x] = t < T ? dv_ : 0.f;
      }
    }
    __syncthreads();
    if (qb * kBlk + kBlk - 1 >= k0w) {  // some query of this block sees some key of this wave
      // S[query][key] = Q · K^T (log2 units); dP[query][key] = dO · V^T
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int c = 0; c < DH / 16; ++c) {
        s = fg::mfma3(row_pair<DH>(Qs, c), kf[c], s);
        dp = fg::mfma3(row_pair<DH>(Gs, c), vf[c], dp);
      }
      const float sc = fold_scale(s, -(E.q + E.ks)), gc = fold_scale(dp, -(E.g + E.v));
      // Masks only on the diagonal / ragged query block: past it every query
      // follows every key of the wave and lies inside the sequence.
      if ((qb * kBlk == k0w) || ((qb + 1) * kBlk > T)) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = acc_row(v, hl);
          const int qi = qb * kBlk + r;
          float p = fast_exp2(__builtin_fmaf(s[v], sc, -Ls[r]));
          if (mykey > qi || qi >= T || mykey >= T) p = 0.f;
          s[v] = p;                                      // P[query][key]
          dp[v] = p * __builtin_fmaf(dp[v], gc, -Ds[r]);  // dS[query][key]
        }
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = acc_row(v, hl);
          const float p = fast_exp2(__builtin_fmaf(s[v], sc, -Ls[r]));
          s[v] = p;
          dp[v] = p * __builtin_fmaf(dp[v], gc, -Ds[r]);
        }
      }
      // dV^T[d][key] += dO^T[d][query] · P[query][key];  dK^T += Q^T · dS
      const Pair p0 = acc_pair(s, 0, kPExp), p1 = acc_pair(s, 1, kPExp);
#pragma unroll
      for (int dt = 0; dt < DH / 32; ++dt) {
        dv[dt] = fg::mfma3(col_pair<DH>(Gc, dt, 0), p0, dv[dt]);
        dv[dt] = fg::mfma3(col_pair<DH>(Gc, dt, 1), p1, dv[dt]);
      }
      const Pair e0 = acc_pair(dp, 0, E.ds), e1 = acc_pair(dp, 1, E.ds);
      if (dS) {
        // dS block (query block qb, this wave's key block) for the dQ launch,
        // as the fp16 pieces the dK product splits it into (scaled by 2^E.ds):
        // [piece][32 queries][32 keys in accumulator order], 4 bytes per
        // element as the fp32 value took; each store instruction writes two
        // whole 64-byte rows
        const size_t bhs = (size_t)b * nH + kvh * group + gi;
        _Float16* blk = reinterpret_cast<_Float16*>(
                            dS + (bhs * npairs + (size_t)qb * (qb + 1) / 2 + k0w / kBlk) * (kBlk * kBlk)) +
                        col_pos(lane & 31);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          blk[acc_row(v, hl) * kBlk] = e0.h[v];
          blk[acc_row(v + 8, hl) * kBlk] = e1.h[v];
          blk[kBlk * kBlk + acc_row(v, hl) * kBlk] = e0.l[v];
          blk[kBlk * kBlk + acc_row(v + 8, hl) * kBlk] = e1.l[v];
        }
      }
#pragma unroll
      for (int dt = 0; dt < DH / 32; ++dt) {
        dk[dt] = fg::mfma3(col_pair<DH>(Qc, dt, 0), e0, dk[dt]);
        dk[dt] = fg::mfma3(col_pair<DH>(Qc, dt, 1), e1, dk[dt]);
      }
    }
    __syncthreads();
  }
  if (part) {  // raw partial sums of this group member: [item][2][128 keys][DH]
    float* pk = part + (size_t)item * 2 * 128 * DH;
    store_T<DH>(dk, pk, DH, mykey - kblk * 128, 128, 1.f, 0, -(E.q + E.ds));
    store_T<DH>(dv, pk + 128 * DH, DH, mykey - kblk * 128, 128, 1.f, 0, -(E.g + kPExp));
    return;
  }
  if (L.rc)
    store_T_rope<DH>(dk, dK + (size_t)b * T * L.ldgk + (size_t)kvh * DH, L.ldgk, mykey, T, scale, L,
                     (int64_t)b * T + mykey, -(E.q + E.ds));
  else
    store_T<DH>(dk, dK + (size_t)b * T * L.ldgk + (size_t)kvh * DH, L.ldgk, mykey, T, scale, beta_k, -(E.q + E.ds));
  store_T<DH>(dv, dV + (size_t)b * T * L.ldgk + (size_t)kvh * DH, L.ldgk, mykey, T, 1.f, beta_v, -(E.g + kPExp));
}

// Both backward kernels in one launch (D precomputed by attn_d_pre): level y
// holds the dK/dV items of key block y, then the dQ items of query block
// nqb-1-y, so the launch starts with the longest causal ranges of both and
// each one's short items fill the other's tail.  One LDS buffer for both.
template <int DH>
__global__ void __launch_bounds__(kMThreads, DH <= 64 ? 2 : 1)
    attn_bwd_merged(float* __restrict__ dQ, int beta_q, float* __restrict__ dK, int beta_k, float* __restrict__ dV,
                    int beta_v, float* __restrict__ Dq, const float* __restrict__ dO, const float* __restrict__ O,
                    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
                    const float* __restrict__ lse, int T, int nH, int nKV, float scale, AttnLd L,
                    float* __restrict__ part, int nbk, int nkv_items, int nq_items, float* __restrict__ dS,
                    int npairs, AttnXp X) {
  __shared__ __attribute__((aligned(16))) char lds[BwdLds<DH>::kMax];
  const Exps E = attn_exps<DH>(X, scale, true);
  const int per_level = nkv_items + nq_items;
  const int y = blockIdx.x / per_level, r = blockIdx.x - y * per_level;
  if (r < nkv_items) {
    dkv_body<DH>(lds, y * nkv_items + r, nbk, dK, beta_k, dV, beta_v, dO, Q, K, V, lse, Dq, T, nH, nKV, scale, L,
                 part, dS, npairs, E);
  } else {
    const int nqb = (T + 127) / 128;
    dq_body<DH>(lds, nqb - 1 - y, r - nkv_items, false, dQ, beta_q, Dq, dO, O, Q, K, V, lse, T, nH, nKV, scale, L,
                E);
  }
}

// dQ of query block qblk (128 queries, 32 per wave) of (sample, head)
// blockIdx.x from the dS blocks the dK/dV launch wrote: dQ^T[d][query] +=
// K^T[d][key] · dS^T[key][query] over the key blocks of its causal range —
// one tile product per block pair, where recomputing S and dP takes three.
// A wave's dS block is read straight into its B-operand registers as the
// fp16 pieces the dK/dV launch formed (the keys of a row are stored in
// accumulator order), so no split happens here; K^T is staged in LDS (column
// layout).
template <int DH>
__global__ void __launch_bounds__(kMThreads, 2)
    attn_dq_ds(float* __restrict__ dQ, int beta, const float* __restrict__ dS, const float* __restrict__ K, int T,
               int nH, int nKV, float scale, AttnLd L, int npairs, AttnXp X) {
  __shared__ __attribute__((aligned(16))) char Kc[2][Tile<DH>::kCol];
  const Exps E = attn_exps<DH>(X, scale, true);
  const int nqb = (T + 127) / 128;
  const int qblk = nqb - 1 - blockIdx.y;  // longest causal prefix first
  const int bh = blockIdx.x, b = bh / nH, h = bh % nH;
  const int group = nH / nKV > 1 ? nH / nKV : 1, kvh = h / group;
  const size_t kvD = L.ldk;
  const int wave = wave_id(), lane = threadIdx.x & 63, hl = lane >> 5;
  const int q0w = qblk * 128 + wave * 32;
  const int myq = q0w + (lane & 31);
  const bool live = q0w < T;  // waves past the last query read no dS block
  const int qb = q0w / kBlk;
  const float* Kb = K + (size_t)b * T * kvD + (size_t)kvh * DH;

  f32x16 dq[DH / 32];
#pragma unroll
  for (int dt = 0; dt < DH / 32; ++dt) dq[dt] = zero16();

  const int nkb = min((T + kBlk - 1) / kBlk, qblk * 4 + 4);
  const int mylast = live ? qb : -1;
  // a block's pieces: hi and lo of chunk c at positions 16c + 8h .. +7 of
  // the query's row (f[c] = hi, f[2 + c] = lo)
  auto load_ds = [&](f16x8 (&f)[4], int kb) {
    const f16x8* p = reinterpret_cast<const f16x8*>(
        reinterpret_cast<const _Float16*>(dS + ((size_t)bh * npairs + (size_t)qb * (qb + 1) / 2 + kb) * (kBlk * kBlk)) +
        (lane & 31) * kBlk + 8 * hl);
    f[0] = p[0]; f[1] = p[2]; f[2] = p[kBlk * kBlk / 8]; f[3] = p[kBlk * kBlk / 8 + 2];
  };
  // Two key blocks in flight: the K^T tile and the dS block of block kb + 2
  // are loaded while block kb's MFMAs run (one block's 24 MFMAs per wave do
  // not cover a memory latency).  Slot A holds the even blocks, slot B the
  // odd ones.
  ColLoader<DH> la, lb;
  f16x8 fa[4], fb[4];
  la.load(Kb, kvD, 0, T);
  if (nkb > 1) lb.load(Kb, kvD, kBlk, T);
  if (mylast >= 0) load_ds(fa, 0);
  if (mylast >= 1) load_ds(fb, 1);
  auto step = [&](ColLoader<DH>& l, f16x8 (&f)[4], int kb) {
    const int buf = kb & 1;
    l.store(Kc[buf], E.k);
    __syncthreads();
    if (kb + 2 < nkb) l.load(Kb, kvD, (kb + 2) * kBlk, T);
    if (kb <= mylast) {
      const Pair d0{f[0], f[2]}, d1{f[1], f[3]};
      if (kb + 2 <= mylast) load_ds(f, kb + 2);
#pragma unroll
      for (int dt = 0; dt < DH / 32; ++dt) {
        dq[dt] = fg::mfma3(col_pair<DH>(Kc[buf], dt, 0), d0, dq[dt]);
        dq[dt] = fg::mfma3(col_pair<DH>(Kc[buf], dt, 1), d1, dq[dt]);
      }
    }
    // double-buffered tiles: no trailing barrier (as in attn_fwd)
  };
  for (int kb = 0; kb < nkb; kb += 2) {
    step(la, fa, kb);
    if (kb + 1 < nkb) step(lb, fb, kb + 1);
  }
  if (L.rc)
    store_T_rope<DH>(dq, dQ + (size_t)b * T * L.ldgq + (size_t)h * DH, L.ldgq, myq, T, scale, L,
                     (int64_t)b * T + myq, -(E.k + E.ds));
  else
    store_T<DH>(dq, dQ + (size_t)b * T * L.ldgq + (size_t)h * DH, L.ldgq, myq, T, scale, beta, -(E.k + E.ds));
}

// dK = scale * sum_z part_z(dK), dV = sum_z part_z(dV) over the group members
// in order z = 0..group-1 (deterministic), written (+beta) to the outputs;
// with RoPE tables, dK's pairs turned back as store_T_rope does.  One thread
// per (kv head, key, d pair).
template <int DH>
__global__ void __launch_bounds__(256)
    attn_dkv_reduce(float* __restrict__ dK, int beta_k, float* __restrict__ dV, int beta_v,
                    const float* __restrict__ part, int B, int T, int nKV, int group, float scale, AttnLd L) {
#pragma clang fp contract(off)
  const int nkb = (T + 127) / 128;
  const int64_t pairs = (int64_t)B * nKV * T * (DH / 2);
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < pairs; e += (int64_t)gridDim.x * 256) {
    const int p = (int)(e % (DH / 2));
    const int64_t rk = e / (DH / 2);  // (bk, key)
    const int key = (int)(rk % T), bk = (int)(rk / T);
    const int kblk = key / 128, r = key % 128;
    const int b = bk / nKV, kvh = bk % nKV;
    const float* src = part + ((size_t)(kblk * (B * nKV) + bk) * group) * 2 * 128 * DH + (size_t)r * DH + 2 * p;
    float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    for (int zz = 0; zz < group; ++zz) {
      const float* q = src + (size_t)zz * 2 * 128 * DH;
      k0 += q[0];
      k1 += q[1];
      v0 += q[128 * DH];
      v1 += q[128 * DH + 1];
    }
    k0 *= scale;
    k1 *= scale;
    const size_t grow = (size_t)b * T + key;
    float* ko = dK + grow * L.ldgk + (size_t)kvh * DH + 2 * p;
    float* vo = dV + grow * L.ldgk + (size_t)kvh * DH + 2 * p;
    if (L.rc) {
      const int64_t pos = L.pos0 + (L.posStride > 0 ? (int64_t)grow % L.posStride : (int64_t)grow);
      const double cc = L.rc[pos * (DH / 2) + p], ss = L.rs[pos * (DH / 2) + p];
      const double a = k0, bb = k1;
      ko[0] = (float)(a * cc + bb * ss);
      ko[1] = (float)(-a * ss + bb * cc);
    } else {
      ko[0] = beta_k ? ko[0] + k0 : k0;
      ko[1] = beta_k ? ko[1] + k1 : k1;
    }
    vo[0] = beta_v ? vo[0] + v0 : v0;
    vo[1] = beta_v ? vo[1] + v1 : v1;
    (void)nkb;
  }
}

}  // namespace x3

// Partial maxima of the MFMA kernels' operands, one launch: Q, K, V into
// qkv_io (3 x FG_XP_PARTS floats; workspace when null) unless have_qkv says
// qkv_io already holds them, and dO (when given) into workspace.
int attn_maxima(fg::Workspace& ws, x3::AttnXp& X, const float* Q, const float* K, const float* V, const float* dO,
                int B, int T, int nH, int nKV, int DH, const AttnLd& L, float* qkv_io = nullptr,
                bool have_qkv = false) {
  have_qkv = have_qkv && qkv_io;
  int rc = ws.get(sizeof(float) * FG_XP_PARTS * 4);
  if (rc) return rc;
  float* xw = static_cast<float*>(ws.ptr);
  float* xq = qkv_io ? qkv_io : xw;
  float* xg = xw + 3 * FG_XP_PARTS;
  const int64_t rows = (int64_t)B * T;
  fg::XpSpec sp[4];
  int n = 0;
  if (!have_qkv) {
    sp[n++] = fg::XpSpec{Q, xq, rows, L.ldq, nH * DH};
    sp[n++] = fg::XpSpec{K, xq + FG_XP_PARTS, rows, L.ldk, nKV * DH};
    sp[n++] = fg::XpSpec{V, xq + 2 * FG_XP_PARTS, rows, L.ldk, nKV * DH};
  }
  if (dO) sp[n++] = fg::XpSpec{dO, xg, rows, L.ldo, nH * DH};
  if ((rc = fg::absmax_parts(sp, n, "attn_absmax"))) return rc;
  X = x3::AttnXp{xq, xq + FG_XP_PARTS, xq + 2 * FG_XP_PARTS, dO ? xg : nullptr};
  return FG_OK;
}

template <int DH>
int launch_fwd_mfma(float* O, float* lse, const float* Q, const float* K, const float* V, int B, int T, int nH, int nKV,
                    float scale, const AttnLd& L, float* xp_qkv = nullptr) {
  fg::Workspace wx;
  x3::AttnXp X;
  int rc = attn_maxima(wx, X, Q, K, V, nullptr, B, T, nH, nKV, DH, L, xp_qkv, false);
  if (rc) return rc;
  dim3 grid(B * nH, (T + 127) / 128);
  FG_LAUNCH((x3::attn_fwd<DH>), grid, dim3(kMThreads), 0, O, lse, Q, K, V, T, nH, nKV, scale, L, X);
  return FG_OK;
}

// The stored dS takes 4 bytes per causal pair and head (half of the
// reference's P matrix); above this size (8 GiB unless fg_attn_set_ds_limit
// changed it) the backward recomputes S and dP for dQ instead (the single
// launch with dQ items), so memory stays bounded at long sequences.
std::atomic<size_t> g_ds_limit{8ull << 30};

template <int DH>
int launch_bwd_mfma(float* dQ, int bq, float* dK, int bk, float* dV, int bv, const float* dO, const float* Q,
                    const float* K, const float* V, const float* O, const float* lse, float* Dq, int B, int T, int nH,
                    int nKV, float scale, const AttnLd& L, const float* xp_qkv = nullptr) {
  // D = rowsum(dO∘O) first, then the dQ and dK/dV work items in one merged
  // launch; with GQA the dK/dV items are per group member (partials summed in
  // order by attn_dkv_reduce)
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  fg::Workspace wx;
  x3::AttnXp X;
  {
    int rc = attn_maxima(wx, X, Q, K, V, dO, B, T, nH, nKV, DH, L, const_cast<float*>(xp_qkv), xp_qkv != nullptr);
    if (rc) return rc;
  }
  {
    const int64_t n = (int64_t)B * T * nH;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 16LL * cus) blocks = 16LL * cus;
    FG_LAUNCH((x3::attn_d_pre<DH>), dim3((unsigned)blocks), dim3(256), 0, Dq, dO, O, B, T, nH, L.ldo);
  }
  const int group = nH / nKV > 1 ? nH / nKV : 1;
  const int nkb = (T + 127) / 128;
  const int nbk = B * nKV;
  fg::Workspace wp;
  float* part = nullptr;
  if (group > 1) {
    int rc = wp.get(sizeof(float) * (size_t)nkb * nbk * group * 2 * 128 * DH);
    if (rc) return rc;
    part = (float*)wp.ptr;
  }
  // dQ from stored dS blocks: the dK/dV items write dS (4 bytes per causal
  // pair), and a second launch forms dQ = dS·K from them
  const int64_t nq32 = (T + kBlk - 1) / kBlk;
  const int64_t npairs64 = nq32 * (nq32 + 1) / 2;
  const int npairs = npairs64 < INT32_MAX ? (int)npairs64 : 0;
  fg::Workspace wds;
  float* dS = nullptr;
  const double ds_bytes = (double)sizeof(float) * B * nH * (double)npairs64 * kBlk * kBlk;
  if (npairs > 0 && ds_bytes <= (double)g_ds_limit.load(std::memory_order_relaxed)) {
    int rc = wds.get((size_t)ds_bytes);
    if (rc) return rc;
    dS = (float*)wds.ptr;
  }
  const int nkv_items = nbk * (group > 1 ? group : 1), nq_items = dS ? 0 : B * nH;
  FG_LAUNCH((x3::attn_bwd_merged<DH>), dim3(nkb * (nkv_items + nq_items)), dim3(kMThreads), 0, dQ, bq, dK, bk, dV,
            bv, Dq, dO, O, Q, K, V, lse, T, nH, nKV, scale, L, part, nbk, nkv_items, nq_items, dS, npairs, X);
  if (dS)
    FG_LAUNCH((x3::attn_dq_ds<DH>), dim3(B * nH, (T + 127) / 128), dim3(kMThreads), 0, dQ, bq, (const float*)dS, K, T,
              nH, nKV, scale, L, npairs, X);
  if (group > 1) {
    const int64_t pairs = (int64_t)B * nKV * T * (DH / 2);
    int64_t blocks = (pairs + 255) / 256;
    if (blocks > 16LL * cus) blocks = 16LL * cus;
    FG_LAUNCH((x3::attn_dkv_reduce<DH>), dim3((unsigned)blocks), dim3(256), 0, dK, bk, dV, bv, part, B, T, nKV, group,
              scale, L);
  }
  return FG_OK;
}

// Head sizes without an MFMA kernel of their own (32 < dH < 128, other than
// 64 and 96) run the MFMA kernels of the next size DP (64, 96 or 128) on copies whose
// heads are padded with zeros to DP columns: the zero columns add exact
// zeros to every S / dP / D sum (which are formed over 16-wide d chunks in
// order, so the first dH columns give the unpadded chunk sums), the output
// columns past dH come out zero and are dropped by the unpad pass, and the
// scale stays 1/sqrt(dH).  The copies cost a pass over Q, K, V (and O, dO,
// the three gradients in the backward); the products cost DP/dH of the
// unpadded flops.
// P[rows][nh * DP] = X[rows][nh * dH] (row stride ld), zeros at d >= dH.
__global__ void __launch_bounds__(256) attn_pad_kernel(float* __restrict__ P, const float* __restrict__ X,
                                                       int64_t rows, int nh, int dH, int DP, int64_t ld) {
  const int64_t w = (int64_t)nh * DP, n = rows * w;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / w;
    const int c = (int)(e - r * w), h = c / DP, d = c - h * DP;
    P[e] = d < dH ? X[r * ld + (int64_t)h * dH + d] : 0.f;
  }
}
// Y[rows][nh * dH] (row stride ld) = (beta ? Y + : ) P[rows][nh * DP], d < dH
// (the add of a beta store, in the same order).
__global__ void __launch_bounds__(256) attn_unpad_kernel(float* __restrict__ Y, const float* __restrict__ P,
                                                         int64_t rows, int nh, int dH, int DP, int64_t ld, int beta) {
  const int64_t w = (int64_t)nh * dH, n = rows * w;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / w;
    const int c = (int)(e - r * w), h = c / dH, d = c - h * dH;
    const float v = P[r * (int64_t)nh * DP + (int64_t)h * DP + d];
    float* y = Y + r * ld + c;
    *y = beta ? *y + v : v;
  }
}
bool pad_mfma(int dH) { return dH > 32 && dH < 128 && dH != 64 && dH != 96; }
int pad_dim(int dH) { return dH <= 64 ? 64 : dH <= 96 ? 96 : 128; }
int64_t stream_blocks(int64_t n) {
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  const int64_t b = (n + 255) / 256;
  return b < 16LL * cus ? (b > 0 ? b : 1) : 16LL * cus;
}
int pad_heads(float* P, const float* X, int64_t rows, int nh, int dH, int DP) {
  FG_LAUNCH(attn_pad_kernel, dim3((unsigned)stream_blocks(rows * nh * DP)), dim3(256), 0, P, X, rows, nh, dH, DP,
            (int64_t)nh * dH);
  return FG_OK;
}
int unpad_heads(float* Y, const float* P, int64_t rows, int nh, int dH, int DP, int beta) {
  FG_LAUNCH(attn_unpad_kernel, dim3((unsigned)stream_blocks(rows * nh * dH)), dim3(256), 0, Y, P, rows, nh, dH, DP,
            (int64_t)nh * dH, beta);
  return FG_OK;
}

AttnLd dense_ld(int nH, int nKV, int dH) {
  return AttnLd{nH * dH, nKV * dH, nH * dH, nH * dH, nKV * dH, nullptr, nullptr, 0, 0};
}

bool use_mfma(int dH, const void* a, const void* b, const void* c) {
  return (dH == 32 || dH == 64 || dH == 96 || dH == 128) && ((uintptr_t)a % 16 == 0) && ((uintptr_t)b % 16 == 0) &&
         ((uintptr_t)c % 16 == 0);
}

int check_shape(const char* name, int B, int T, int nH, int nKV, int dH) {
  FG_ARG_CHECK(B > 0 && T > 0 && nH > 0 && nKV > 0 && dH > 0, "%s: bad shape B=%d T=%d nH=%d nKV=%d dH=%d", name, B, T,
               nH, nKV, dH);
  const int group = nH / nKV > 1 ? nH / nKV : 1;
  FG_ARG_CHECK((nH - 1) / group < nKV, "%s: head %d maps to kv head %d >= nKV=%d (nH/nKV=%d)", name, nH - 1,
               (nH - 1) / group, nKV, group);
  return FG_OK;
}

// The scalar kernels for a head size: the instance of the smallest class
// (64, 128, 256) that holds it.
int launch_fwd_scalar(float* O, float* lse, const float* Q, const float* K, const float* V, int B, int T, int nH,
                      int nKV, int dH, float scale) {
  dim3 grid((T + kSRows - 1) / kSRows, B * nH);
  if (dH <= 64) FG_LAUNCH(attn_fwd_scalar<64>, grid, dim3(kSRows), 0, O, lse, Q, K, V, T, nH, nKV, dH, scale);
  else FG_LAUNCH(attn_fwd_scalar<128>, grid, dim3(kSRows), 0, O, lse, Q, K, V, T, nH, nKV, dH, scale);
  return FG_OK;
}

template <int DM>
int launch_bwd_scalar_t(float* dQ, int beta_q, float* dK, int beta_k, float* dV, int beta_v, const float* dO,
                        const float* Q, const float* K, const float* V, const float* lse, const float* Dq, int B,
                        int T, int nH, int nKV, int dH, float scale) {
  dim3 gq((T + kSRows - 1) / kSRows, B * nH);
  FG_LAUNCH(attn_dq_scalar<DM>, gq, dim3(kSRows), 0, dQ, beta_q, dO, Q, K, V, lse, Dq, T, nH, nKV, dH, scale);
  // one workgroup per (sample, kv head): a kv head that no query head maps
  // to (nH < nKV) gets zero gradients, as the reference's loop over h < nH
  // leaves them
  dim3 gk((T + kSRows - 1) / kSRows, B * nKV);
  FG_LAUNCH(attn_dkv_scalar<DM>, gk, dim3(kSRows), 0, dK, beta_k, dV, beta_v, dO, Q, K, V, lse, Dq, T, nH, nKV, dH,
            scale);
  return FG_OK;
}

int launch_bwd_scalar(float* dQ, int beta_q, float* dK, int beta_k, float* dV, int beta_v, const float* dO,
                      const float* Q, const float* K, const float* V, const float* lse, const float* Dq, int B, int T,
                      int nH, int nKV, int dH, float scale) {
  if (dH <= 64)
    return launch_bwd_scalar_t<64>(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, lse, Dq, B, T, nH, nKV, dH, scale);
  return launch_bwd_scalar_t<128>(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, lse, Dq, B, T, nH, nKV, dH, scale);
}

// Columns of ngroups groups of g problems (see attn_head_cols).
int head_cols(float* dst, int ld, const float* src, int T, int dH, int nh, int z0, int g, int ngroups, int beta) {
  const int64_t n = (int64_t)T * dH;
  int64_t bx = (n + 255) / 256;
  if (bx > 64) bx = 64;
  FG_LAUNCH(attn_head_cols, dim3((unsigned)bx, ngroups), dim3(256), 0, dst, ld, src, T, dH, nh, z0, g, beta);
  return FG_OK;
}

// Problems per chunk: the T×T workspaces at most ~2 GiB each, a whole number
// of GQA groups, at most the grid's 65535 in z.
int chunk_problems(int T, int Z, int group) {
  const double per = 4.0 * T * (double)T;
  int zc = (int)((double)(1u << 31) / per);
  if (zc > 65535) zc = 65535;
  zc -= zc % group;
  if (zc < group) zc = group;
  return zc < Z ? zc : Z;
}

// The attention as batched GEMM launches (head sizes above 128).
int fwd_gemm(float* O, float* lse, const float* Q, const float* K, const float* V, int B, int T, int nH, int nKV,
             int dH, float scale) {
  const int group = nH / nKV > 1 ? nH / nKV : 1, qD = nH * dH, kvD = nKV * dH, Z = B * nH;
  const int zc = chunk_problems(T, Z, 1);
  fg::Workspace ws_s, ws_o;
  int rc;
  if ((rc = ws_s.get(sizeof(float) * (size_t)zc * T * T))) return rc;
  if ((rc = ws_o.get(sizeof(float) * (size_t)zc * T * dH))) return rc;
  float *S = (float*)ws_s.ptr, *Ot = (float*)ws_o.ptr;
  const int64_t TT = (int64_t)T * T, TD = (int64_t)T * dH;
  for (int z0 = 0; z0 < Z; z0 += zc) {
    const int nz = Z - z0 < zc ? Z - z0 : zc;
    // S = Q_h · K_kvh^T
    fg::GemmBatch bs{nH, z0, {0, (int64_t)T * qD, dH, 1, 0}, {0, (int64_t)T * kvD, dH, group, 0}, TT, 1};
    if ((rc = fg::gemm_batched(true, true, S, Q, K, T, T, dH, qD, kvD, bs, nz))) return rc;
    FG_LAUNCH(attn_rows_softmax, dim3(T, nz), dim3(kRowThreads), 0, S, lse + (size_t)z0 * T, T, scale);
    // O_h = P · V_kvh
    fg::GemmBatch bo{nH, z0, {TT, 0, 0, 1, 1}, {0, (int64_t)T * kvD, dH, group, 0}, TD, 2};
    if ((rc = fg::gemm_batched(true, false, Ot, S, V, T, dH, T, T, kvD, bo, nz))) return rc;
    if ((rc = head_cols(O, qD, Ot, T, dH, nH, z0, 1, nz, 0))) return rc;
  }
  return FG_OK;
}

int bwd_gemm(float* dQ, int beta_q, float* dK, int beta_k, float* dV, int beta_v, const float* dO, const float* Q,
             const float* K, const float* V, const float* lse, int B, int T, int nH, int nKV, int dH, float scale) {
  const int group = nH / nKV > 1 ? nH / nKV : 1, qD = nH * dH, kvD = nKV * dH, Z = B * nH;
  FG_ARG_CHECK(nH < nKV || nH % group == 0, "fg_attn_bwd: %d query heads are not whole groups of %d", nH, group);
  const int zc = chunk_problems(T, Z, group);
  fg::Workspace ws_s, ws_d, ws_t;
  int rc;
  if ((rc = ws_s.get(sizeof(float) * (size_t)zc * T * T))) return rc;
  if ((rc = ws_d.get(sizeof(float) * (size_t)zc * T * T))) return rc;
  if ((rc = ws_t.get(sizeof(float) * (size_t)zc * T * dH))) return rc;
  float *S = (float*)ws_s.ptr, *dP = (float*)ws_d.ptr, *tmp = (float*)ws_t.ptr;
  const int64_t TT = (int64_t)T * T, TD = (int64_t)T * dH;
  // nH < nKV: kv heads past the last query head get no contribution (the
  // reference's loop over h < nH leaves them at zero)
  if (nH < nKV)
    for (int b = 0; b < B; ++b)
      for (int kvh = nH; kvh < nKV; ++kvh) {
        const int zk = b * nKV + kvh;  // problem index of this kv head with nh = nKV, g = 1
        if (!beta_k && (rc = head_cols(dK, kvD, nullptr, T, dH, nKV, zk, 1, 1, 0))) return rc;
        if (!beta_v && (rc = head_cols(dV, kvD, nullptr, T, dH, nKV, zk, 1, 1, 0))) return rc;
      }
  const fg::BatchOperand q_h{0, (int64_t)T * qD, dH, 1, 0}, kv_h{0, (int64_t)T * kvD, dH, group, 0};
  const fg::BatchOperand loc{TT, 0, 0, 1, 1};
  for (int z0 = 0; z0 < Z; z0 += zc) {
    const int nz = Z - z0 < zc ? Z - z0 : zc;
    // S = Q_h · K_kvh^T, dP = dO_h · V_kvh^T
    if ((rc = fg::gemm_batched(true, true, S, Q, K, T, T, dH, qD, kvD, fg::GemmBatch{nH, z0, q_h, kv_h, TT, 1}, nz)))
      return rc;
    if ((rc = fg::gemm_batched(true, true, dP, dO, V, T, T, dH, qD, kvD, fg::GemmBatch{nH, z0, q_h, kv_h, TT, 1}, nz)))
      return rc;
    FG_LAUNCH(attn_rows_softmax_bwd, dim3(T, nz), dim3(kRowThreads), 0, S, dP, lse + (size_t)z0 * T, T, scale);
    // dQ_h = dS · K_kvh
    if ((rc = fg::gemm_batched(true, false, tmp, dP, K, T, dH, T, T, kvD, fg::GemmBatch{nH, z0, loc, kv_h, TD, 2}, nz)))
      return rc;
    if ((rc = head_cols(dQ, qD, tmp, T, dH, nH, z0, 1, nz, beta_q))) return rc;
    // dK_kvh (+)= Σ_group dS^T · Q_h, dV_kvh (+)= Σ_group P^T · dO_h
    const int ng = nz / group;
    if ((rc = fg::gemm_batched(false, false, tmp, dP, Q, T, dH, T, T, qD, fg::GemmBatch{nH, z0, loc, q_h, TD, 3}, nz)))
      return rc;
    if ((rc = head_cols(dK, kvD, tmp, T, dH, nH, z0, group, ng, beta_k))) return rc;
    if ((rc = fg::gemm_batched(false, false, tmp, S, dO, T, dH, T, T, qD, fg::GemmBatch{nH, z0, loc, q_h, TD, 3}, nz)))
      return rc;
    if ((rc = head_cols(dV, kvD, tmp, T, dH, nH, z0, group, ng, beta_v))) return rc;
  }
  return FG_OK;
}
}  // namespace

extern "C" int fg_attn_set_ds_limit(size_t bytes) {
  g_ds_limit.store(bytes, std::memory_order_relaxed);
  return FG_OK;
}

extern "C" int fg_attn_fwd(float* O, float* lse, const float* Q, const float* K, const float* V, int B, int T, int nH,
                           int nKV, int dH) {
  FG_REQUIRE_INIT();
  int rc = check_shape("fg_attn_fwd", B, T, nH, nKV, dH);
  if (rc) return rc;
  FG_ARG_CHECK(O && lse && Q && K && V, "fg_attn_fwd: null pointer");
  const double pairs = (double)T * (T + 1) / 2.0;
  fg::KProfScope prof("attn_fwd", 4.0 * dH * pairs * B * nH,
                      4.0 * B * T * ((double)nH * dH * 2 + (double)nKV * dH * 2 + nH));
  const float scale = (float)(1.0 / sqrt((double)dH));
  if (use_mfma(dH, Q, K, V) && (uintptr_t)O % 16 == 0) {
    const AttnLd L = dense_ld(nH, nKV, dH);
    if (dH == 32) return launch_fwd_mfma<32>(O, lse, Q, K, V, B, T, nH, nKV, scale, L);
    if (dH == 64) return launch_fwd_mfma<64>(O, lse, Q, K, V, B, T, nH, nKV, scale, L);
    if (dH == 96) return launch_fwd_mfma<96>(O, lse, Q, K, V, B, T, nH, nKV, scale, L);
    return launch_fwd_mfma<128>(O, lse, Q, K, V, B, T, nH, nKV, scale, L);
  }
  if (pad_mfma(dH)) {  // heads padded with zeros to the next MFMA size
    const int DP = pad_dim(dH);
    const int64_t rows = (int64_t)B * T;
    fg::Workspace wq, wkv, wo;
    if ((rc = wq.get(sizeof(float) * (size_t)rows * nH * DP))) return rc;
    if ((rc = wkv.get(sizeof(float) * (size_t)rows * nKV * DP * 2))) return rc;
    if ((rc = wo.get(sizeof(float) * (size_t)rows * nH * DP))) return rc;
    float *Qp = (float*)wq.ptr, *Kp = (float*)wkv.ptr, *Vp = Kp + (size_t)rows * nKV * DP, *Op = (float*)wo.ptr;
    if ((rc = pad_heads(Qp, Q, rows, nH, dH, DP))) return rc;
    if ((rc = pad_heads(Kp, K, rows, nKV, dH, DP))) return rc;
    if ((rc = pad_heads(Vp, V, rows, nKV, dH, DP))) return rc;
    const AttnLd L = dense_ld(nH, nKV, DP);
    rc = DP == 64   ? launch_fwd_mfma<64>(Op, lse, Qp, Kp, Vp, B, T, nH, nKV, scale, L)
         : DP == 96 ? launch_fwd_mfma<96>(Op, lse, Qp, Kp, Vp, B, T, nH, nKV, scale, L)
                    : launch_fwd_mfma<128>(Op, lse, Qp, Kp, Vp, B, T, nH, nKV, scale, L);
    if (rc) return rc;
    return unpad_heads(O, Op, rows, nH, dH, DP, 0);
  }
  if (dH > 128) return fwd_gemm(O, lse, Q, K, V, B, T, nH, nKV, dH, scale);
  return launch_fwd_scalar(O, lse, Q, K, V, B, T, nH, nKV, dH, scale);
}

extern "C" int fg_attn_bwd(float* dQ, int beta_q, float* dK, int beta_k, float* dV, int beta_v, const float* dO,
                           const float* Q, const float* K, const float* V, const float* O, const float* lse, int B,
                           int T, int nH, int nKV, int dH) {
  FG_REQUIRE_INIT();
  int rc = check_shape("fg_attn_bwd", B, T, nH, nKV, dH);
  if (rc) return rc;
  FG_ARG_CHECK(dQ && dK && dV && dO && Q && K && V && O && lse, "fg_attn_bwd: null pointer");
  const double pairs = (double)T * (T + 1) / 2.0;
  fg::KProfScope prof("attn_bwd", 8.0 * dH * pairs * B * nH,
                      4.0 * B * T * ((double)nH * dH * 4 + (double)nKV * dH * 4 + 2.0 * nH));
  const float scale = (float)(1.0 / sqrt((double)dH));
  fg::Workspace ws;
  rc = ws.get(sizeof(float) * (size_t)B * nH * T);
  if (rc) return rc;
  float* Dq = (float*)ws.ptr;
  // nH < nKV leaves kv heads without query heads: the scalar kernels give
  // them zero gradients (the MFMA work items assume every kv head has a group)
  const bool mf = use_mfma(dH, Q, K, V) && nH >= nKV && ((uintptr_t)dO % 16 == 0) && ((uintptr_t)O % 16 == 0) &&
                  ((uintptr_t)dQ % 16 == 0) && ((uintptr_t)dK % 16 == 0) && ((uintptr_t)dV % 16 == 0);
  if (mf) {
    const AttnLd L = dense_ld(nH, nKV, dH);
    if (dH == 32) return launch_bwd_mfma<32>(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L);
    if (dH == 64) return launch_bwd_mfma<64>(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L);
    if (dH == 96) return launch_bwd_mfma<96>(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L);
    return launch_bwd_mfma<128>(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L);
  }
  if (pad_mfma(dH) && nH >= nKV) {  // heads padded with zeros to the next MFMA size
    const int DP = pad_dim(dH);
    const int64_t rows = (int64_t)B * T;
    const size_t nq = (size_t)rows * nH * DP, nk = (size_t)rows * nKV * DP;
    fg::Workspace wq, wkv;
    if ((rc = wq.get(sizeof(float) * nq * 4))) return rc;   // Q, O, dO, dQ
    if ((rc = wkv.get(sizeof(float) * nk * 4))) return rc;  // K, V, dK, dV
    float *Qp = (float*)wq.ptr, *Op = Qp + nq, *dOp = Op + nq, *dQp = dOp + nq;
    float *Kp = (float*)wkv.ptr, *Vp = Kp + nk, *dKp = Vp + nk, *dVp = dKp + nk;
    if ((rc = pad_heads(Qp, Q, rows, nH, dH, DP))) return rc;
    if ((rc = pad_heads(Op, O, rows, nH, dH, DP))) return rc;
    if ((rc = pad_heads(dOp, dO, rows, nH, dH, DP))) return rc;
    if ((rc = pad_heads(Kp, K, rows, nKV, dH, DP))) return rc;
    if ((rc = pad_heads(Vp, V, rows, nKV, dH, DP))) return rc;
    const AttnLd L = dense_ld(nH, nKV, DP);
    rc = DP == 64   ? launch_bwd_mfma<64>(dQp, 0, dKp, 0, dVp, 0, dOp, Qp, Kp, Vp, Op, lse, Dq, B, T, nH, nKV, scale, L)
         : DP == 96 ? launch_bwd_mfma<96>(dQp, 0, dKp, 0, dVp, 0, dOp, Qp, Kp, Vp, Op, lse, Dq, B, T, nH, nKV, scale, L)
                    : launch_bwd_mfma<128>(dQp, 0, dKp, 0, dVp, 0, dOp, Qp, Kp, Vp, Op, lse, Dq, B, T, nH, nKV, scale, L);
    if (rc) return rc;
    if ((rc = unpad_heads(dQ, dQp, rows, nH, dH, DP, beta_q))) return rc;
    if ((rc = unpad_heads(dK, dKp, rows, nKV, dH, DP, beta_k))) return rc;
    return unpad_heads(dV, dVp, rows, nKV, dH, DP, beta_v);
  }
  if (dH > 128) return bwd_gemm(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, lse, B, T, nH, nKV, dH, scale);
  {
    int64_t n = (int64_t)B * T * nH;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    FG_LAUNCH(attn_bwd_pre, dim3((unsigned)blocks), dim3(256), 0, Dq, dO, O, B, T, nH, dH);
  }
  return launch_bwd_scalar(dQ, beta_q, dK, beta_k, dV, beta_v, dO, Q, K, V, lse, Dq, B, T, nH, nKV, dH, scale);
}

// Attention of a fused projection qkv[B*T, (nH + 2 nKV) dH] whose q and k
// columns are already rotated: q, k, v are read as column blocks of qkv.
extern "C" int fg_attn_fwd_qkv_p(float* O, float* lse, const float* qkv, int B, int T, int nH, int nKV, int dH,
                                 float* xp_qkv) {
  FG_REQUIRE_INIT();
  int rc = check_shape("fg_attn_fwd_qkv", B, T, nH, nKV, dH);
  if (rc) return rc;
  FG_ARG_CHECK(O && lse && qkv, "fg_attn_fwd_qkv: null pointer");
  FG_ARG_CHECK((dH == 32 || dH == 64 || dH == 96 || dH == 128) && (uintptr_t)qkv % 16 == 0 && (uintptr_t)O % 16 == 0,
               "fg_attn_fwd_qkv: needs dH in {32, 64, 96, 128} and 16-byte aligned tensors (dH=%d)", dH);
  const double pairs = (double)T * (T + 1) / 2.0;
  fg::KProfScope prof("attn_fwd", 4.0 * dH * pairs * B * nH,
                      4.0 * B * T * ((double)nH * dH * 2 + (double)nKV * dH * 2 + nH));
  const float scale = (float)(1.0 / sqrt((double)dH));
  const int W = (nH + 2 * nKV) * dH;
  const AttnLd L{W, W, nH * dH, 0, 0, nullptr, nullptr, 0, 0};
  const float* Q = qkv;
  const float* K = qkv + (size_t)nH * dH;
  const float* V = K + (size_t)nKV * dH;
  if (dH == 32) return launch_fwd_mfma<32>(O, lse, Q, K, V, B, T, nH, nKV, scale, L, xp_qkv);
  if (dH == 64) return launch_fwd_mfma<64>(O, lse, Q, K, V, B, T, nH, nKV, scale, L, xp_qkv);
  if (dH == 96) return launch_fwd_mfma<96>(O, lse, Q, K, V, B, T, nH, nKV, scale, L, xp_qkv);
  return launch_fwd_mfma<128>(O, lse, Q, K, V, B, T, nH, nKV, scale, L, xp_qkv);
}

extern "C" int fg_attn_fwd_qkv(float* O, float* lse, const float* qkv, int B, int T, int nH, int nKV, int dH) {
  return fg_attn_fwd_qkv_p(O, lse, qkv, B, T, nH, nKV, dH, nullptr);
}

// Its backward: gqkv = [R^T dQ | R^T dK | dV] (written, not accumulated), the
// rotation by the RoPE table of position pos0 + (row % posStride, or row).
extern "C" int fg_attn_bwd_qkv_p(float* gqkv, const float* dO, const float* qkv, const float* O, const float* lse,
                                 int B, int T, int nH, int nKV, int dH, const double* cos_tab, const double* sin_tab,
                                 int npos, int pos0, int posStride, const float* xp_qkv) {
  FG_REQUIRE_INIT();
  int rc = check_shape("fg_attn_bwd_qkv", B, T, nH, nKV, dH);
  if (rc) return rc;
  FG_ARG_CHECK(gqkv && dO && qkv && O && lse && cos_tab && sin_tab, "fg_attn_bwd_qkv: null pointer");
  FG_ARG_CHECK(nH >= nKV, "fg_attn_bwd_qkv: nH=%d < nKV=%d (kv heads without query heads) needs fg_attn_bwd", nH, nKV);
  FG_ARG_CHECK((dH == 32 || dH == 64 || dH == 96 || dH == 128) && (uintptr_t)qkv % 16 == 0 && (uintptr_t)O % 16 == 0 &&
                   (uintptr_t)dO % 16 == 0 && (uintptr_t)gqkv % 16 == 0 && (uintptr_t)cos_tab % 16 == 0 &&
                   (uintptr_t)sin_tab % 16 == 0,
               "fg_attn_bwd_qkv: needs dH in {32, 64, 96, 128} and 16-byte aligned tensors (dH=%d)", dH);
  const int64_t rows = (int64_t)B * T;
  FG_ARG_CHECK(pos0 >= 0 && posStride >= 0, "fg_attn_bwd_qkv: bad positions");
  const int64_t maxpos = pos0 + (posStride > 0 ? (rows < posStride ? rows : posStride) : rows) - 1;
  FG_ARG_CHECK(maxpos < npos, "fg_attn_bwd_qkv: positions up to %lld exceed the %d-entry table", (long long)maxpos,
               npos);
  const double pairs = (double)T * (T + 1) / 2.0;
  fg::KProfScope prof("attn_bwd", 8.0 * dH * pairs * B * nH,
                      4.0 * B * T * ((double)nH * dH * 4 + (double)nKV * dH * 4 + 2.0 * nH));
  const float scale = (float)(1.0 / sqrt((double)dH));
  fg::Workspace ws;
  rc = ws.get(sizeof(float) * (size_t)B * nH * T);
  if (rc) return rc;
  float* Dq = (float*)ws.ptr;
  const int W = (nH + 2 * nKV) * dH;
  const AttnLd L{W, W, nH * dH, W, W, cos_tab, sin_tab, pos0, posStride};
  const float* Q = qkv;
  const float* K = qkv + (size_t)nH * dH;
  const float* V = K + (size_t)nKV * dH;
  float* gQ = gqkv;
  float* gK = gqkv + (size_t)nH * dH;
  float* gV = gK + (size_t)nKV * dH;
  if (dH == 32) return launch_bwd_mfma<32>(gQ, 0, gK, 0, gV, 0, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L, xp_qkv);
  if (dH == 64) return launch_bwd_mfma<64>(gQ, 0, gK, 0, gV, 0, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L, xp_qkv);
  if (dH == 96) return launch_bwd_mfma<96>(gQ, 0, gK, 0, gV, 0, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L, xp_qkv);
  return launch_bwd_mfma<128>(gQ, 0, gK, 0, gV, 0, dO, Q, K, V, O, lse, Dq, B, T, nH, nKV, scale, L, xp_qkv);
}

extern "C" int fg_attn_bwd_qkv(float* gqkv, const float* dO, const float* qkv, const float* O, const float* lse,
                               int B, int T, int nH, int nKV, int dH, const double* cos_tab, const double* sin_tab,
                               int npos, int pos0, int posStride) {
  return fg_attn_bwd_qkv_p(gqkv, dO, qkv, O, lse, B, T, nH, nKV, dH, cos_tab, sin_tab, npos, pos0, posStride, nullptr);
}
