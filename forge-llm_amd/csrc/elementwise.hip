// Bandwidth-bound ops of the training path for gfx950: rmsNorm, ropeRows,
// swigluRows, embedLookup, sliceCols, addTensors, weightedSum (tensor.js,
// train.js).  Each is one coalesced pass over its operands; reductions are
// two-stage with fixed reduction trees (deterministic, no atomics).
#include "common.h"
#include "swiglu_math.h"

#include <math.h>
#include <vector>

namespace {

constexpr int kThreads = 256;

inline bool al16(const void* p) { return ((uintptr_t)p % 16) == 0; }

unsigned grid_1d(int64_t work, int per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  // up to 128 workgroups per CU: streaming kernels reach ~6 TB/s with full
  // grids and ~5.2 TB/s with 16 per CU (measured on MI355X)
  int64_t cap = (int64_t)(fg::device_cu_count() > 0 ? fg::device_cu_count() : 256) * 128;
  if (g > cap) g = cap;
  return (unsigned)(g < 1 ? 1 : g);
}

// Block-wide sum of a double (256 threads).
__device__ __forceinline__ double block_sum_d(double v, double* sh) {
  v = fg_wave_sum_d(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) t += sh[i];
  return t;
}

// ───────────────────────── rmsNorm (tensor.js:103-128) ─────────────────────────
// Wave-per-row kernels for D % 4 == 0 and D <= 64*4*NJ: lane l owns float4
// columns l, l+64, ...; row reductions are wave shuffles (no barriers).
// Generic workgroup-per-row kernels cover any other D.

// Sum over the wave in fp64 of a per-lane fp32 partial.
__device__ __forceinline__ double wave_sum_f2d(float v) { return fg_wave_sum_d((double)v); }

typedef float v4f __attribute__((ext_vector_type(4)));

// One row per wave iteration; the next row's loads are issued before the
// current row's reduction and stores, so reads and writes overlap.  X and Y
// are streamed (nontemporal: each is read once more by other kernels, much
// later or from the GEMM's own tiles).
template <int NJ>
__global__ void __launch_bounds__(kThreads) rmsnorm_fwd_wave(float* __restrict__ Y, float* __restrict__ inv,
                                                             const float* __restrict__ X, const float* __restrict__ w,
                                                             int T, int D, double eps) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int nwaves = gridDim.x * (kThreads / 64);
  const int D4 = D >> 2;
  const v4f* w4 = reinterpret_cast<const v4f*>(w);
  v4f cur[NJ], nxt[NJ];
  auto load = [&](int r, v4f* dst) {
    const v4f* x4 = reinterpret_cast<const v4f*>(X + (size_t)r * D);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + 64 * j;
      dst[j] = c < D4 ? x4[c] : v4f{0.f, 0.f, 0.f, 0.f};
    }
  };
  int r = wave;
  if (r < T) load(r, cur);
  for (; r < T; r += nwaves) {
    if (r + nwaves < T) load(r + nwaves, nxt);
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      ss += (double)cur[j].x * cur[j].x + (double)cur[j].y * cur[j].y + (double)cur[j].z * cur[j].z +
            (double)cur[j].w * cur[j].w;
    ss = fg_wave_sum_d(ss);
    const float iv = (float)(1.0 / sqrt(ss / D + eps));
    if (lane == 0) inv[r] = iv;
    v4f* y4 = reinterpret_cast<v4f*>(Y + (size_t)r * D);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + 64 * j;
      if (c < D4) {
        const v4f wv = w4[c];
        v4f o;
        o.x = (float)((double)cur[j].x * iv * wv.x);
        o.y = (float)((double)cur[j].y * iv * wv.y);
        o.z = (float)((double)cur[j].z * iv * wv.z);
        o.w = (float)((double)cur[j].w * iv * wv.w);
        __builtin_nontemporal_store(o, y4 + c);
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) cur[j] = nxt[j];
  }
}

// Rows over 1024 floats: one workgroup (four waves) per row, F float4 per
// thread held in registers with the next row's loads issued before the
// current row's reduction and stores (the wave-per-row kernel holds a whole
// 4096-float row and its successor in one wave's registers: 254 VGPRs, two
// waves per SIMD).  The fp64 sum of squares is summed per thread, over the
// wave, then over the four waves in order.
template <int F>
__global__ void __launch_bounds__(kThreads) rmsnorm_fwd_rowwg(float* __restrict__ Y, float* __restrict__ inv,
                                                              const float* __restrict__ X,
                                                              const float* __restrict__ w, int T, int D,
                                                              double eps) {
  __shared__ double red[2][kThreads / 64];
  const int D4 = D >> 2;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const v4f* w4 = reinterpret_cast<const v4f*>(w);
  v4f cur[F], nxt[F];
  auto load = [&](int r, v4f* dst) {
    const v4f* x4 = reinterpret_cast<const v4f*>(X + (size_t)r * D);
#pragma unroll
    for (int j = 0; j < F; ++j) {
      const int c = threadIdx.x + kThreads * j;
      v4f v = x4[c < D4 ? c : 0];  // a clamped, always valid column (plain loads: X, just written
                                   // by the residual add, is often still in the Infinity Cache)
      if (c >= D4) v = v4f{0.f, 0.f, 0.f, 0.f};
      dst[j] = v;
    }
  };
  int r = blockIdx.x;
  if (r < T) load(r, cur);
  for (int par = 0; r < T; r += gridDim.x, par ^= 1) {
    if (r + gridDim.x < T) load(r + gridDim.x, nxt);
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < F; ++j)
      ss += (double)cur[j].x * cur[j].x + (double)cur[j].y * cur[j].y + (double)cur[j].z * cur[j].z +
            (double)cur[j].w * cur[j].w;
    ss = fg_wave_sum_d(ss);
    if (lane == 0) red[par][wv] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int k = 0; k < kThreads / 64; ++k) tot += red[par][k];
    const float iv = (float)(1.0 / sqrt(tot / D + eps));
    if (threadIdx.x == 0) inv[r] = iv;
    v4f* y4 = reinterpret_cast<v4f*>(Y + (size_t)r * D);
#pragma unroll
    for (int j = 0; j < F; ++j) {
      const int c = threadIdx.x + kThreads * j;
      if (c < D4) {
        const v4f wq = w4[c];
        v4f o;
        o.x = (float)((double)cur[j].x * iv * wq.x);
        o.y = (float)((double)cur[j].y * iv * wq.y);
        o.z = (float)((double)cur[j].z * iv * wq.z);
        o.w = (float)((double)cur[j].w * iv * wq.w);
        __builtin_nontemporal_store(o, y4 + c);
      }
    }
#pragma unroll
    for (int j = 0; j < F; ++j) cur[j] = nxt[j];
  }
}

// gX (+)= g*w*inv - c*x, c = sum(g*w*x) / (D r^3), r = 1/inv; each workgroup
// writes its partial column sums of g*x*inv (for gw) to partial[blockIdx.x].
// G2: the incoming gradient arrives as two halves (the K pieces of the GEMM
// that produced it), g = g[i] + g2[i] in fp32 — the value that GEMM's own
// reduction would have stored.
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
template <int NJ, bool G2>
__global__ void __launch_bounds__(kThreads) rmsnorm_bwd_wave(float* gX, const float* gx_old,
                                                             float* __restrict__ partial, const float* __restrict__ g,
                                                             const float* __restrict__ g2,
                                                             const float* __restrict__ X, const float* __restrict__ w,
                                                             const float* __restrict__ inv, int T, int D) {
  const bool beta_x = gx_old != nullptr;
  __shared__ float4 red[kThreads / 64][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wave = blockIdx.x * (kThreads / 64) + wv;
  const int nwaves = gridDim.x * (kThreads / 64);
  const int D4 = D >> 2;
  const float4* w4 = reinterpret_cast<const float4*>(w);
  float4 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  static_assert(NJ <= 4, "rows over 1024 floats take rmsnorm_bwd_rowwg");
  // One row per iteration; the next row's g and x are loaded before the
  // current row's reduction and stores, so the read and write streams
  // overlap (the accumulated gX row is loaded at the top of its own
  // iteration and lands during the reduction).  Rows enter acc in
  // increasing order.
  float4 gc[NJ], xc[NJ], gn[NJ], xn[NJ], oc[NJ], wr[NJ], gn2[NJ];
  // Loads read a clamped, always valid column and zero the value past D:
  // selecting between a load and a local constant makes the compiler load
  // through a pointer to a stack copy of the constant.
  auto ld = [&](const float4* p4, int c) {
    float4 v = p4[c < D4 ? c : 0];
    if (c >= D4) v = make_float4(0.f, 0.f, 0.f, 0.f);
    return v;
  };
#pragma unroll
  for (int j = 0; j < NJ; ++j) wr[j] = ld(w4, lane + 64 * j);
  int r = wave;
  float ivc = 0.f;
  if (r < T) {
    const float4* g4 = reinterpret_cast<const float4*>(g + (size_t)r * D);
    const float4* x4 = reinterpret_cast<const float4*>(X + (size_t)r * D);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      gc[j] = ld(g4, lane + 64 * j);
      xc[j] = ld(x4, lane + 64 * j);
    }
    if (G2) {
      const float4* g24 = reinterpret_cast<const float4*>(g2 + (size_t)r * D);
#pragma unroll
      for (int j = 0; j < NJ; ++j) gc[j] = add4(gc[j], ld(g24, lane + 64 * j));
    }
    ivc = inv[r];
  }
  for (; r < T; r += nwaves) {
    float4* gx4 = reinterpret_cast<float4*>(gX + (size_t)r * D);
    if (beta_x) {
      const float4* go4 = reinterpret_cast<const float4*>(gx_old + (size_t)r * D);
#pragma unroll
      for (int j = 0; j < NJ; ++j) oc[j] = ld(go4, lane + 64 * j);
    }
    const int rn = r + nwaves;
    float ivn = 0.f;
    if (rn < T) {
      const float4* g4 = reinterpret_cast<const float4*>(g + (size_t)rn * D);
      const float4* x4 = reinterpret_cast<const float4*>(X + (size_t)rn * D);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        gn[j] = ld(g4, lane + 64 * j);
        xn[j] = ld(x4, lane + 64 * j);
      }
      if (G2) {
        const float4* g24 = reinterpret_cast<const float4*>(g2 + (size_t)rn * D);
#pragma unroll
        for (int j = 0; j < NJ; ++j) gn2[j] = ld(g24, lane + 64 * j);
      }
      ivn = inv[rn];
    }
    double dot = 0.0;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      dot += (double)gc[j].x * wr[j].x * xc[j].x + (double)gc[j].y * wr[j].y * xc[j].y +
             (double)gc[j].z * wr[j].z * xc[j].z + (double)gc[j].w * wr[j].w * xc[j].w;
    dot = fg_wave_sum_d(dot);
    const float iv = ivc;
    const double rr = 1.0 / (double)iv;
    const double c = dot / ((double)D * rr * rr * rr);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int cc = lane + 64 * j;
      if (cc < D4) {
        float4 o;
        o.x = (float)((double)gc[j].x * wr[j].x * iv - c * xc[j].x);
        o.y = (float)((double)gc[j].y * wr[j].y * iv - c * xc[j].y);
        o.z = (float)((double)gc[j].z * wr[j].z * iv - c * xc[j].z);
        o.w = (float)((double)gc[j].w * wr[j].w * iv - c * xc[j].w);
        if (beta_x) {
          o.x += oc[j].x; o.y += oc[j].y; o.z += oc[j].z; o.w += oc[j].w;
        }
        gx4[cc] = o;
        acc[j].x += gc[j].x * xc[j].x * iv;
        acc[j].y += gc[j].y * xc[j].y * iv;
        acc[j].z += gc[j].z * xc[j].z * iv;
        acc[j].w += gc[j].w * xc[j].w * iv;
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      gc[j] = G2 ? add4(gn[j], gn2[j]) : gn[j];
      xc[j] = xn[j];
    }
    ivc = ivn;
  }
  if (!partial) return;
  // combine the workgroup's waves in a fixed order, one float4 column chunk at a time
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    red[wv][lane] = acc[j];
    __syncthreads();
    if (wv == 0) {
      float4 s = red[0][lane];
#pragma unroll
      for (int k = 1; k < kThreads / 64; ++k) {
        const float4 o = red[k][lane];
        s.x += o.x; s.y += o.y; s.z += o.z; s.w += o.w;
      }
      const int cc = lane + 64 * j;
      if (cc < D4) reinterpret_cast<float4*>(partial + (size_t)blockIdx.x * D)[cc] = s;
    }
    __syncthreads();
  }
}

// Wide rows (1024 < D <= 4096, D % 4 == 0): one workgroup per row, F float4
// columns per thread (c = tid + 256 j) held in registers — g, x and the next
// row's g, x, loaded before the current row's reduction — so each element is
// read once; the row's dot product is summed per thread, per wave, then over
// the four waves in order (LDS, double-buffered by row parity: one barrier
// per row).  Each thread owns its columns of the dw partial sums, so the
// workgroup's partial row needs no combine.  Same formulas as the wave
// kernel.
template <int F, bool G2>
__global__ void __launch_bounds__(kThreads) rmsnorm_bwd_rowwg(float* gX, const float* gx_old,
                                                              float* __restrict__ partial,
                                                              const float* __restrict__ g,
                                                              const float* __restrict__ g2,
                                                              const float* __restrict__ X,
                                                              const float* __restrict__ w,
                                                              const float* __restrict__ inv, int T, int D) {
  const bool beta_x = gx_old != nullptr;
  __shared__ double red[2][kThreads / 64];
  const int D4 = D >> 2;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float4* w4 = reinterpret_cast<const float4*>(w);
  // a clamped, always valid column, zeroed past D (no select on a load)
  auto ld = [&](const float4* p4, int c) {
    float4 v = p4[c < D4 ? c : 0];
    if (c >= D4) v = make_float4(0.f, 0.f, 0.f, 0.f);
    return v;
  };
  float4 wr[F], acc[F], gc[F], xc[F], gn[F], xn[F], oc[F];
#pragma unroll
  for (int j = 0; j < F; ++j) {
    wr[j] = ld(w4, threadIdx.x + kThreads * j);
    acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  auto load_row = [&](int r, float4* gg, float4* xx) {
    const float4* g4 = reinterpret_cast<const float4*>(g + (size_t)r * D);
    const float4* x4 = reinterpret_cast<const float4*>(X + (size_t)r * D);
#pragma unroll
    for (int j = 0; j < F; ++j) {
      gg[j] = ld(g4, threadIdx.x + kThreads * j);
      xx[j] = ld(x4, threadIdx.x + kThreads * j);
    }
    if (G2) {
      const float4* g24 = reinterpret_cast<const float4*>(g2 + (size_t)r * D);
#pragma unroll
      for (int j = 0; j < F; ++j) gg[j] = add4(gg[j], ld(g24, threadIdx.x + kThreads * j));
    }
  };
  int r = blockIdx.x;
  float ivc = 0.f;
  if (r < T) {
    load_row(r, gc, xc);
    ivc = inv[r];
  }
  for (int par = 0; r < T; r += gridDim.x, par ^= 1) {
    if (beta_x) {
      const float4* go4 = reinterpret_cast<const float4*>(gx_old + (size_t)r * D);
#pragma unroll
      for (int j = 0; j < F; ++j) oc[j] = ld(go4, threadIdx.x + kThreads * j);
    }
    const int rn = r + gridDim.x;
    float ivn = 0.f;
    if (rn < T) {
      load_row(rn, gn, xn);
      ivn = inv[rn];
    }
    double dot = 0.0;
#pragma unroll
    for (int j = 0; j < F; ++j)
      dot += (double)gc[j].x * wr[j].x * xc[j].x + (double)gc[j].y * wr[j].y * xc[j].y +
             (double)gc[j].z * wr[j].z * xc[j].z + (double)gc[j].w * wr[j].w * xc[j].w;
    dot = fg_wave_sum_d(dot);
    if (lane == 0) red[par][wv] = dot;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int k = 0; k < kThreads / 64; ++k) tot += red[par][k];
    const float iv = ivc;
    const double rr = 1.0 / (double)iv;
    const double c = tot / ((double)D * rr * rr * rr);
    float4* gx4 = reinterpret_cast<float4*>(gX + (size_t)r * D);
#pragma unroll
    for (int j = 0; j < F; ++j) {
      const int cc = threadIdx.x + kThreads * j;
      if (cc < D4) {
        float4 o;
        o.x = (float)((double)gc[j].x * wr[j].x * iv - c * xc[j].x);
        o.y = (float)((double)gc[j].y * wr[j].y * iv - c * xc[j].y);
        o.z = (float)((double)gc[j].z * wr[j].z * iv - c * xc[j].z);
        o.w = (float)((double)gc[j].w * wr[j].w * iv - c * xc[j].w);
        if (beta_x) {
          o.x += oc[j].x; o.y += oc[j].y; o.z += oc[j].z; o.w += oc[j].w;
        }
        gx4[cc] = o;
        acc[j].x += gc[j].x * xc[j].x * iv;
        acc[j].y += gc[j].y * xc[j].y * iv;
        acc[j].z += gc[j].z * xc[j].z * iv;
        acc[j].w += gc[j].w * xc[j].w * iv;
      }
    }
#pragma unroll
    for (int j = 0; j < F; ++j) {
      gc[j] = gn[j];
      xc[j] = xn[j];
    }
    ivc = ivn;
  }
  if (!partial) return;
#pragma unroll
  for (int j = 0; j < F; ++j) {
    const int cc = threadIdx.x + kThreads * j;
    if (cc < D4) reinterpret_cast<float4*>(partial + (size_t)blockIdx.x * D)[cc] = acc[j];
  }
}

// Generic (any D): one workgroup per row; sum of squares in fp64.
__global__ void __launch_bounds__(kThreads) rmsnorm_fwd_kernel(float* __restrict__ Y, float* __restrict__ inv,
                                                               const float* __restrict__ X,
                                                               const float* __restrict__ w, int D, double eps) {
  __shared__ double sh[kThreads / 64];
  const size_t rb = (size_t)blockIdx.x * D;
  double ss = 0.0;
  for (int i = threadIdx.x; i < D; i += kThreads) {
    float x = X[rb + i];
    ss += (double)x * x;
  }
  ss = block_sum_d(ss, sh);
  const float iv = (float)(1.0 / sqrt(ss / D + eps));
  if (threadIdx.x == 0) inv[blockIdx.x] = iv;
  for (int i = threadIdx.x; i < D; i += kThreads) Y[rb + i] = (float)((double)X[rb + i] * iv * w[i]);
}

// Generic backward: kRowsPerBlock rows per workgroup, partial column sums of
// g*x*inv for gw.  Rows over kThreads * kMaxColsPerThread floats are cut into
// column chunks of that width (grid y); each chunk's workgroup forms the
// whole row's dot product itself and writes only its own columns.
constexpr int kRowsPerBlock = 32;
constexpr int kMaxColsPerThread = 32;  // columns per chunk: kThreads * 32
__global__ void __launch_bounds__(kThreads) rmsnorm_bwd_kernel(float* gX, const float* gx_old,
                                                               float* __restrict__ gw_partial,
                                                               const float* __restrict__ g,
                                                               const float* __restrict__ X,
                                                               const float* __restrict__ w,
                                                               const float* __restrict__ inv, int T, int D) {
  __shared__ double sh[kThreads / 64];
  float acc[kMaxColsPerThread];
#pragma unroll
  for (int j = 0; j < kMaxColsPerThread; ++j) acc[j] = 0.f;
  const int r0 = blockIdx.x * kRowsPerBlock;
  const int r1 = min(T, r0 + kRowsPerBlock);
  const int c0 = blockIdx.y * kThreads * kMaxColsPerThread;
  for (int r = r0; r < r1; ++r) {
    const size_t rb = (size_t)r * D;
    double dot = 0.0;
    for (int i = threadIdx.x; i < D; i += kThreads) dot += (double)g[rb + i] * w[i] * X[rb + i];
    dot = block_sum_d(dot, sh);
    const float iv = inv[r];
    const double rr = 1.0 / (double)iv;
    const double c = dot / ((double)D * rr * rr * rr);
#pragma unroll
    for (int j = 0; j < kMaxColsPerThread; ++j) {
      const int i = c0 + threadIdx.x + j * kThreads;
      if (i < D) {
        const float gi = g[rb + i], xi = X[rb + i];
        float v = (float)((double)gi * w[i] * iv - c * xi);
        if (gx_old) v += gx_old[rb + i];
        gX[rb + i] = v;
        acc[j] += gi * xi * iv;
      }
    }
  }
  if (gw_partial) {
#pragma unroll
    for (int j = 0; j < kMaxColsPerThread; ++j) {
      const int i = c0 + threadIdx.x + j * kThreads;
      if (i < D) gw_partial[(size_t)blockIdx.x * D + i] = acc[j];
    }
  }
}

// out[i] = (beta ? out[i] : 0) + sum_b partial[b*n + i] in a fixed order:
// 32 columns per workgroup, 8 row-groups summed in a fixed tree.
__global__ void __launch_bounds__(kThreads) colsum_kernel(float* __restrict__ out, const float* __restrict__ partial,
                                                          int nblocks, int n, int beta) {
  __shared__ float sh[8][33];
  const int c = threadIdx.x & 31, rg = threadIdx.x >> 5;
  const int i = blockIdx.x * 32 + c;
  float s = 0.f;
  if (i < n)
    for (int b = rg; b < nblocks; b += 8) s += partial[(size_t)b * n + i];
  sh[rg][c] = s;
  __syncthreads();
  if (rg == 0 && i < n) {
    float t = beta ? out[i] : 0.f;
    float u = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) u += sh[k][c];
    out[i] = t + u;
  }
}

// The same column sum for n % 4 == 0 and 16-byte aligned rows: a strip of 16
// float4 columns (256 bytes of each row) per workgroup, 16 row-groups of 16
// threads each summing rows rg, rg+16, ... in order (eight loads in flight,
// added as one at a time), then a fixed pairwise tree over the row-groups.
constexpr int kColGroups = 256;   // threads per workgroup
constexpr int kStrip4 = 16;       // float4 columns per workgroup
constexpr int kStripRows = kColGroups / kStrip4;
__device__ __forceinline__ void colsum4_body(float* __restrict__ out, const float* __restrict__ partial, int nblocks,
                                             int n, int beta, int strip, float4 (*sh)[kStrip4]) {
  const int c = threadIdx.x % kStrip4, rg = threadIdx.x / kStrip4;
  const int n4 = n >> 2;
  const int i4 = strip * kStrip4 + c;
  const bool live = i4 < n4;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  const float4* p4 = reinterpret_cast<const float4*>(partial) + (live ? i4 : 0);
  int b = rg;
  for (; b + 7 * kStripRows < nblocks; b += 8 * kStripRows) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p4[(size_t)(b + u * kStripRows) * n4];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      s.x += v[u].x; s.y += v[u].y; s.z += v[u].z; s.w += v[u].w;
    }
  }
  for (; b < nblocks; b += kStripRows) {
    const float4 v = p4[(size_t)b * n4];
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  sh[rg][c] = s;
  __syncthreads();
#pragma unroll
  for (int h = kStripRows / 2; h > 0; h >>= 1) {
    if (rg < h) {
      const float4 o = sh[rg + h][c];
      float4 t = sh[rg][c];
      t.x += o.x; t.y += o.y; t.z += o.z; t.w += o.w;
      sh[rg][c] = t;
    }
    __syncthreads();
  }
  if (rg == 0 && live) {
    float4 u = sh[0][c];
    float4* o4 = reinterpret_cast<float4*>(out) + i4;
    if (beta) {
      const float4 t = *o4;
      u.x = t.x + u.x; u.y = t.y + u.y; u.z = t.z + u.z; u.w = t.w + u.w;
    }
    *o4 = u;
  }
}

__global__ void __launch_bounds__(kColGroups) colsum4_kernel(float* __restrict__ out,
                                                             const float* __restrict__ partial, int nblocks, int n,
                                                             int beta) {
  __shared__ float4 sh[kStripRows][kStrip4];
  colsum4_body(out, partial, nblocks, n, beta, blockIdx.x, sh);
}

// Several column sums in one launch (the RMSNorm weight gradients of a
// backward pass, deferred to its end): workgroup -> (job, 16-column strip)
// by the prefix sums of the jobs' strip counts; each column is summed
// exactly as colsum4_kernel sums it.  The table travels by value in the kernel
// arguments, so a recorded graph holds it.
constexpr int kMaxColJobs = 64;
struct ColTable {
  int count;
  int start[kMaxColJobs + 1];  // first workgroup of each job; start[count] = grid size
  float* out[kMaxColJobs];
  const float* part[kMaxColJobs];
  int rows[kMaxColJobs], n[kMaxColJobs], beta[kMaxColJobs];
};
static_assert(sizeof(ColTable) <= 4096, "kernel arguments must stay within 4 KB");

__global__ void __launch_bounds__(kColGroups) colsum4_grouped(ColTable t) {
  __shared__ float4 sh[kStripRows][kStrip4];
  const int bid = blockIdx.x;
  int j = 0;
  while (j + 1 < t.count && bid >= t.start[j + 1]) ++j;  // uniform over the workgroup
  colsum4_body(t.out[j], t.part[j], t.rows[j], t.n[j], t.beta[j], bid - t.start[j], sh);
}

// ───────────────────────── ropeRows (tensor.js:133-166) ─────────────────────────
// One thread per (row, head, pair); angles from the fp64 host table, fp64 math.
__global__ void __launch_bounds__(kThreads) rope_kernel(float* __restrict__ Y, const float* __restrict__ X,
                                                        const double* __restrict__ ctab,
                                                        const double* __restrict__ stab, int64_t npairs,
                                                        int nHead, int dHead, int pos0, int posStride,
                                                        int backward, int beta) {
#pragma clang fp contract(off)
  const int half = dHead >> 1;
  const int ppr = nHead * half;  // pairs per row
  for (int64_t p = (int64_t)blockIdx.x * kThreads + threadIdx.x; p < npairs; p += (int64_t)gridDim.x * kThreads) {
    const int64_t t = p / ppr;
    const int within = (int)(p - t * ppr);
    const int i2 = within % half;  // pair index inside the head
    const int pos = pos0 + (posStride > 0 ? (int)(t % posStride) : (int)t);
    const double c = ctab[(int64_t)pos * half + i2], s = stab[(int64_t)pos * half + i2];
    const float2 v = reinterpret_cast<const float2*>(X)[p];
    const double a = v.x, b = v.y;
    float2 r;
    if (!backward) {
      r.x = (float)(a * c - b * s);
      r.y = (float)(a * s + b * c);
    } else {
      if (beta) {
        const float2 o = reinterpret_cast<const float2*>(Y)[p];
        r.x = (float)((double)o.x + (a * c + b * s));
        r.y = (float)((double)o.y + (-a * s + b * c));
      } else {
        r.x = (float)(a * c + b * s);
        r.y = (float)(-a * s + b * c);
      }
    }
    reinterpret_cast<float2*>(Y)[p] = r;
  }
}

// ───────── fused sliceCols(q,k,v) + ropeRows(q), ropeRows(k) (train.js:133-138) ─────────
// Grid (rows, ceil(pairs per row / 256)): one thread per column pair of a qkv
// row [q (nH*dH) | k (nKV*dH) | v (nKV*dH)]; q and k pairs are rotated (fp64,
// contraction off, the same arithmetic as rope_kernel), v pairs copied.
// Backward writes [R^T gq | R^T gk | gv] into gqkv (+beta); a null gradient
// pointer counts as zero.  32-bit index math only (the row is blockIdx.x).
__global__ void __launch_bounds__(kThreads) qkv_rope_kernel(float* __restrict__ Q, float* __restrict__ K,
                                                            float* __restrict__ V, float* __restrict__ G,
                                                            const double* __restrict__ ctab,
                                                            const double* __restrict__ stab, int nH, int nKV, int dH,
                                                            int pos0, int posStride, int backward, int beta) {
#pragma clang fp contract(off)
  const int half = dH >> 1;
  const int qP = nH * half, kP = nKV * half;  // pairs per row in q, k, v
  const int rowP = qP + 2 * kP;
  const int c = blockIdx.y * kThreads + threadIdx.x;
  if (c >= rowP) return;
  const int t = blockIdx.x;
  int seg, idx;
  if (c < qP) { seg = 0; idx = c; }
  else if (c < qP + kP) { seg = 1; idx = c - qP; }
  else { seg = 2; idx = c - qP - kP; }
  float* dst = seg == 0 ? Q : seg == 1 ? K : V;
  const int segP = seg == 0 ? qP : kP;
  float2* g2 = reinterpret_cast<float2*>(G) + (size_t)t * rowP + c;  // gqkv / qkv pair
  const size_t so = (size_t)t * segP + idx;                           // q / k / v pair index
  const int pos = pos0 + (posStride > 0 ? t % posStride : t);
  const int i2 = idx % half;
  if (!backward) {
    const float2 v = *g2;
    float2 r;
    if (seg < 2) {
      const double cc = ctab[(size_t)pos * half + i2], ss = stab[(size_t)pos * half + i2];
      const double a = v.x, b = v.y;
      r.x = (float)(a * cc - b * ss);
      r.y = (float)(a * ss + b * cc);
    } else {
      r = v;
    }
    reinterpret_cast<float2*>(dst)[so] = r;
  } else if (!dst) {  // no gradient for this segment: it adds zero
    if (!beta) *g2 = make_float2(0.f, 0.f);
  } else {
    const float2 gin = reinterpret_cast<const float2*>(dst)[so];
    float2 r;
    if (seg < 2) {
      const double cc = ctab[(size_t)pos * half + i2], ss = stab[(size_t)pos * half + i2];
      const double a = gin.x, b = gin.y;
      if (beta) {
        const float2 o = *g2;
        r.x = (float)((double)o.x + (a * cc + b * ss));
        r.y = (float)((double)o.y + (-a * ss + b * cc));
      } else {
        r.x = (float)(a * cc + b * ss);
        r.y = (float)(-a * ss + b * cc);
      }
    } else {
      r = gin;
      if (beta) {
        const float2 o = *g2;
        r.x = (float)((double)o.x + (double)gin.x);
        r.y = (float)((double)o.y + (double)gin.y);
      }
    }
    *g2 = r;
  }
}

// Two pairs per thread (dH % 4 == 0, 16-byte aligned tensors): thread q owns
// columns 4q' .. 4q'+3 of its row as one float4, the two pairs' table entries
// as one double2 each; a quad never straddles q | k | v (their widths are
// multiples of 4).  Grid-stride over rows * quads-per-row; the same fp64
// arithmetic per pair as qkv_rope_kernel.
typedef double d2v __attribute__((ext_vector_type(2)));
__global__ void __launch_bounds__(kThreads) qkv_rope4_kernel(float* __restrict__ Q, float* __restrict__ K,
                                                             float* __restrict__ V, float* __restrict__ G,
                                                             const double* __restrict__ ctab,
                                                             const double* __restrict__ stab, int rows, int nH,
                                                             int nKV, int dH, int pos0, int posStride, int backward,
                                                             int beta) {
#pragma clang fp contract(off)
  const int half = dH >> 1;
  const int qQ = nH * dH / 4, kQ = nKV * dH / 4;  // quads per row in q, k, v
  const int rowQ = qQ + 2 * kQ;
  const unsigned total = (unsigned)rows * (unsigned)rowQ;
  for (unsigned e = blockIdx.x * kThreads + threadIdx.x; e < total; e += gridDim.x * kThreads) {
    const unsigned t = e / (unsigned)rowQ;
    const int c = (int)(e - t * (unsigned)rowQ);
    int seg, idx;
    if (c < qQ) { seg = 0; idx = c; }
    else if (c < qQ + kQ) { seg = 1; idx = c - qQ; }
    else { seg = 2; idx = c - qQ - kQ; }
    float* dst = seg == 0 ? Q : seg == 1 ? K : V;
    const int segQ = seg == 0 ? qQ : kQ;
    float4* g4 = reinterpret_cast<float4*>(G) + e;                  // gqkv / qkv quad
    const size_t so = (size_t)t * segQ + idx;                        // q / k / v quad index
    const int pos = pos0 + (posStride > 0 ? (int)(t % (unsigned)posStride) : (int)t);
    const int i2 = (2 * idx) % half;                                 // first pair inside the head
    d2v cc = {1.0, 1.0}, ss = {0.0, 0.0};
    if (seg < 2) {
      cc = *reinterpret_cast<const d2v*>(ctab + (size_t)pos * half + i2);
      ss = *reinterpret_cast<const d2v*>(stab + (size_t)pos * half + i2);
    }
    if (!backward) {
      const v4f vv = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(g4));
      const float4 v = make_float4(vv.x, vv.y, vv.z, vv.w);
      float4 r = v;
      if (seg < 2) {
        const double a0 = v.x, b0 = v.y, a1 = v.z, b1 = v.w;
        r.x = (float)(a0 * cc.x - b0 * ss.x);
        r.y = (float)(a0 * ss.x + b0 * cc.x);
        r.z = (float)(a1 * cc.y - b1 * ss.y);
        r.w = (float)(a1 * ss.y + b1 * cc.y);
      }
      reinterpret_cast<float4*>(dst)[so] = r;
    } else if (!dst) {  // no gradient for this segment: it adds zero
      if (!beta) *g4 = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      const v4f gv = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(dst) + so);
      const float4 gin = make_float4(gv.x, gv.y, gv.z, gv.w);
      float4 r = gin;
      if (seg < 2) {
        const double a0 = gin.x, b0 = gin.y, a1 = gin.z, b1 = gin.w;
        if (beta) {
          const float4 o = *g4;
          r.x = (float)((double)o.x + (a0 * cc.x + b0 * ss.x));
          r.y = (float)((double)o.y + (-a0 * ss.x + b0 * cc.x));
          r.z = (float)((double)o.z + (a1 * cc.y + b1 * ss.y));
          r.w = (float)((double)o.w + (-a1 * ss.y + b1 * cc.y));
        } else {
          r.x = (float)(a0 * cc.x + b0 * ss.x);
          r.y = (float)(-a0 * ss.x + b0 * cc.x);
          r.z = (float)(a1 * cc.y + b1 * ss.y);
          r.w = (float)(-a1 * ss.y + b1 * cc.y);
        }
      } else if (beta) {
        const float4 o = *g4;
        r.x = (float)((double)o.x + (double)gin.x);
        r.y = (float)((double)o.y + (double)gin.y);
        r.z = (float)((double)o.z + (double)gin.z);
        r.w = (float)((double)o.w + (double)gin.w);
      }
      *g4 = r;
    }
  }
}

// ───────────────────────── swigluRows (tensor.js:272-290) ─────────────────────────
using fg::swiglu_grad1;
__device__ __forceinline__ float sigmoidf_(float x) { return fg::swiglu_sigmoid(x); }

__global__ void __launch_bounds__(kThreads) swiglu_fwd_kernel(float* __restrict__ O, const float* __restrict__ G,
                                                              const float* __restrict__ U, int64_t n) {
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 g = reinterpret_cast<const float4*>(G)[i];
    const float4 u = reinterpret_cast<const float4*>(U)[i];
    float4 o;
    o.x = g.x * sigmoidf_(g.x) * u.x;
    o.y = g.y * sigmoidf_(g.y) * u.y;
    o.z = g.z * sigmoidf_(g.z) * u.z;
    o.w = g.w * sigmoidf_(g.w) * u.w;
    reinterpret_cast<float4*>(O)[i] = o;
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
    O[i] = G[i] * sigmoidf_(G[i]) * U[i];
}


__global__ void __launch_bounds__(kThreads) swiglu_bwd_kernel(float* __restrict__ gG, int beta_g,
                                                              float* __restrict__ gU, int beta_u,
                                                              const float* __restrict__ g,
                                                              const float* __restrict__ G,
                                                              const float* __restrict__ U, int64_t n) {
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
    const float4 gy = reinterpret_cast<const float4*>(g)[i];
    const float4 gv = reinterpret_cast<const float4*>(G)[i];
    const float4 uv = reinterpret_cast<const float4*>(U)[i];
    float4 dg, du;
    swiglu_grad1(gy.x, gv.x, uv.x, dg.x, du.x);
    swiglu_grad1(gy.y, gv.y, uv.y, dg.y, du.y);
    swiglu_grad1(gy.z, gv.z, uv.z, dg.z, du.z);
    swiglu_grad1(gy.w, gv.w, uv.w, dg.w, du.w);
    if (gG) {
      if (beta_g) {
        const float4 o = reinterpret_cast<const float4*>(gG)[i];
        dg.x += o.x; dg.y += o.y; dg.z += o.z; dg.w += o.w;
      }
      reinterpret_cast<float4*>(gG)[i] = dg;
    }
    if (gU) {
      if (beta_u) {
        const float4 o = reinterpret_cast<const float4*>(gU)[i];
        du.x += o.x; du.y += o.y; du.z += o.z; du.w += o.w;
      }
      reinterpret_cast<float4*>(gU)[i] = du;
    }
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
    float dg, du;
    swiglu_grad1(g[i], G[i], U[i], dg, du);
    if (gG) gG[i] = beta_g ? gG[i] + dg : dg;
    if (gU) gU[i] = beta_u ? gU[i] + du : du;
  }
}

// ───── swigluRows on a fused gate/up projection GU[rows, 2H] = [G | U] ─────
// Same element arithmetic as swiglu_fwd_kernel / swiglu_grad1; grid (rows,
// ceil(H / 1024)), one float4 of a row per thread (H % 4 == 0).
__global__ void __launch_bounds__(kThreads) swiglu_gu_fwd_kernel(float* __restrict__ O, const float* __restrict__ GU,
                                                                 int H) {
  const int c4 = blockIdx.y * kThreads + threadIdx.x;
  if (c4 >= H / 4) return;
  const size_t r = blockIdx.x;
  const float4 g = reinterpret_cast<const float4*>(GU + r * 2 * H)[c4];
  const float4 u = reinterpret_cast<const float4*>(GU + r * 2 * H + H)[c4];
  float4 o;
  o.x = g.x * sigmoidf_(g.x) * u.x;
  o.y = g.y * sigmoidf_(g.y) * u.y;
  o.z = g.z * sigmoidf_(g.z) * u.z;
  o.w = g.w * sigmoidf_(g.w) * u.w;
  reinterpret_cast<float4*>(O + r * H)[c4] = o;
}

__global__ void __launch_bounds__(kThreads) swiglu_gu_bwd_kernel(float* __restrict__ gGU, int beta,
                                                                 const float* __restrict__ g,
                                                                 const float* __restrict__ GU, int H) {
  const int c4 = blockIdx.y * kThreads + threadIdx.x;
  if (c4 >= H / 4) return;
  const size_t r = blockIdx.x;
  // g and [G | U] are read for the last time: nontemporal loads
  const v4f gy = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(g + r * H) + c4);
  const v4f gv = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(GU + r * 2 * H) + c4);
  const v4f uv = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(GU + r * 2 * H + H) + c4);
  v4f dg, du;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float a, b;
    swiglu_grad1(gy[e], gv[e], uv[e], a, b);
    dg[e] = a;
    du[e] = b;
  }
  v4f* pg = reinterpret_cast<v4f*>(gGU + r * 2 * H) + c4;
  v4f* pu = reinterpret_cast<v4f*>(gGU + r * 2 * H + H) + c4;
  if (beta) {
    dg += *pg;
    du += *pu;
  }
  *pg = dg;
  *pu = du;
}

// swiglu_gu_bwd_kernel that also leaves the partial maxima of its output's
// finite magnitudes for the input-gradient GEMM that reads it (FG_XP_PARTS
// floats, the layout the GEMMs' operand maxima take): workgroup w writes
// part w after its rows w, w + 256, ... (two rows in flight per thread).
constexpr int kXpParts = FG_XP_PARTS;
constexpr int kSwXpThreads = 512;
__device__ __forceinline__ float finite_abs_(float x) {
  const float a = fabsf(x);
  return a < __builtin_inff() ? a : 0.f;  // inf and NaN count as 0
}
__device__ __forceinline__ void swiglu_bwd4(float* __restrict__ gGU, int beta, const float* __restrict__ g,
                                            const float* __restrict__ GU, size_t r, int c4, int H, float& m) {
  const v4f gy = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(g + r * H) + c4);
  const v4f gv = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(GU + r * 2 * H) + c4);
  const v4f uv = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(GU + r * 2 * H + H) + c4);
  v4f dg, du;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float a, b;
    swiglu_grad1(gy[e], gv[e], uv[e], a, b);
    dg[e] = a;
    du[e] = b;
  }
  v4f* pg = reinterpret_cast<v4f*>(gGU + r * 2 * H) + c4;
  v4f* pu = reinterpret_cast<v4f*>(gGU + r * 2 * H + H) + c4;
  if (beta) {
    dg += *pg;
    du += *pu;
  }
  *pg = dg;
  *pu = du;
#pragma unroll
  for (int e = 0; e < 4; ++e) m = fmaxf(m, fmaxf(finite_abs_(dg[e]), finite_abs_(du[e])));
}
__global__ void __launch_bounds__(kSwXpThreads) swiglu_gu_bwd_xp_kernel(float* __restrict__ gGU, int beta,
                                                                        const float* __restrict__ g,
                                                                        const float* __restrict__ GU, int rows, int H,
                                                                        float* __restrict__ xp) {
  const int h4 = H / 4;
  float m = 0.f;
  int r = blockIdx.x;
  for (; r + kXpParts < rows; r += 2 * kXpParts)
    for (int c4 = threadIdx.x; c4 < h4; c4 += kSwXpThreads) {
      swiglu_bwd4(gGU, beta, g, GU, r, c4, H, m);
      swiglu_bwd4(gGU, beta, g, GU, r + kXpParts, c4, H, m);
    }
  if (r < rows)
    for (int c4 = threadIdx.x; c4 < h4; c4 += kSwXpThreads) swiglu_bwd4(gGU, beta, g, GU, r, c4, H, m);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  __shared__ float wm[kSwXpThreads / 64];
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = wm[0];
#pragma unroll
    for (int w = 1; w < kSwXpThreads / 64; ++w) b = fmaxf(b, wm[w]);
    xp[blockIdx.x] = b;
  }
}

// The same two passes for any H and alignment: one element per thread.
__global__ void __launch_bounds__(kThreads) swiglu_gu_fwd_any(float* __restrict__ O, const float* __restrict__ GU,
                                                              int64_t n, int H) {
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kThreads) {
    const int64_t r = e / H, c = e - r * H;
    const float g = GU[r * 2 * H + c], u = GU[r * 2 * H + H + c];
    O[e] = g * sigmoidf_(g) * u;
  }
}

__global__ void __launch_bounds__(kThreads) swiglu_gu_bwd_any(float* __restrict__ gGU, int beta,
                                                              const float* __restrict__ g,
                                                              const float* __restrict__ GU, int64_t n, int H) {
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kThreads) {
    const int64_t r = e / H, c = e - r * H;
    float dg, du;
    swiglu_grad1(g[e], GU[r * 2 * H + c], GU[r * 2 * H + H + c], dg, du);
    float* pg = gGU + r * 2 * H + c;
    float* pu = pg + H;
    *pg = beta ? *pg + dg : dg;
    *pu = beta ? *pu + du : du;
  }
}

// ───────────────────────── embedLookup (tensor.js:85-99) ─────────────────────────
__global__ void __launch_bounds__(kThreads) embed_fwd_kernel(float* __restrict__ X, const float* __restrict__ W,
                                                             const int32_t* __restrict__ ids, int T, int V, int D) {
  const int64_t n = (int64_t)T * D;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kThreads) {
    const int t = (int)(e / D), d = (int)(e - (int64_t)t * D);
    const int id = ids[t];
    X[e] = (id >= 0 && id < V) ? W[(int64_t)id * D + d] : NAN;
  }
}

// D % 4 == 0 and 16-byte aligned rows: one wave per row, lane l copying
// float4 columns l, l+64, ... (the id read once per row, all of a lane's
// loads issued before its stores).
constexpr int kEmbedJ = 4;  // float4 per lane per pass
__global__ void __launch_bounds__(kThreads) embed_fwd4_kernel(float* __restrict__ X, const float* __restrict__ W,
                                                              const int32_t* __restrict__ ids, int T, int V, int D4) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6));
  const int nw = gridDim.x * (kThreads / 64);
  for (int t = wave; t < T; t += nw) {
    const int id = ids[t];
    const bool ok = id >= 0 && id < V;
    const float4* src = reinterpret_cast<const float4*>(W) + (int64_t)(ok ? id : 0) * D4;
    float4* dst = reinterpret_cast<float4*>(X) + (int64_t)t * D4;
    for (int c0 = lane; c0 < D4; c0 += 64 * kEmbedJ) {
      float4 v[kEmbedJ];
#pragma unroll
      for (int j = 0; j < kEmbedJ; ++j) {
        const int c = c0 + 64 * j;
        v[j] = src[c < D4 ? c : 0];
      }
#pragma unroll
      for (int j = 0; j < kEmbedJ; ++j) {
        const int c = c0 + 64 * j;
        if (c < D4) dst[c] = ok ? v[j] : make_float4(NAN, NAN, NAN, NAN);
      }
    }
  }
}

// One workgroup per segment of equal ids; rows summed in increasing t order
// onto the existing gradient row, exactly the reference's sequence of fp32 +=.
__global__ void __launch_bounds__(kThreads) embed_bwd_kernel(float* __restrict__ gW, const float* __restrict__ g,
                                                             const int32_t* __restrict__ perm,
                                                             const int32_t* __restrict__ seg_start,
                                                             const int32_t* __restrict__ seg_id, int D) {
  const int s = blockIdx.x;
  const int k0 = seg_start[s], k1 = seg_start[s + 1];
  float* row = gW + (int64_t)seg_id[s] * D;
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float acc = row[d];
    for (int k = k0; k < k1; ++k) acc += g[(int64_t)perm[k] * D + d];
    row[d] = acc;
  }
}

// ───────────────────────── sliceCols (tensor.js:170-183) ─────────────────────────
__global__ void __launch_bounds__(kThreads) slice_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                         int M, int K, int off, int len, int backward) {
  const int64_t n = (int64_t)M * len;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kThreads) {
    const int64_t m = e / len;
    const int i = (int)(e - m * len);
    const int64_t xi = m * K + off + i;
    if (!backward) dst[e] = src[xi];
    else dst[xi] += src[e];
  }
}

// ───────────────────────── add / accumulate (train.js:230-238) ─────────────────────────
__global__ void __launch_bounds__(kThreads) add_kernel(float* __restrict__ Y, const float* __restrict__ A,
                                                       const float* __restrict__ B, int64_t n, int vec) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i0 = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (vec) {
    const int64_t n4 = n / 4;
    for (int64_t i = i0; i < n4; i += stride) {
      float4 a = reinterpret_cast<const float4*>(A)[i], b = reinterpret_cast<const float4*>(B)[i];
      reinterpret_cast<float4*>(Y)[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    }
    for (int64_t i = n4 * 4 + i0; i < n; i += stride) Y[i] = A[i] + B[i];
  } else {
    for (int64_t i = i0; i < n; i += stride) Y[i] = A[i] + B[i];
  }
}

__global__ void __launch_bounds__(kThreads) accum_kernel(float* __restrict__ Y, const float* __restrict__ X,
                                                         int64_t n, int beta, int vec) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i0 = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (vec) {
    // two float4 per thread per iteration, streamed (nontemporal)
    const int64_t n4 = n / 4;
    v4f* y4 = reinterpret_cast<v4f*>(Y);
    const v4f* x4 = reinterpret_cast<const v4f*>(X);
    for (int64_t i = i0; i < n4; i += 2 * stride) {
      const int64_t i2 = i + stride;
      v4f a = __builtin_nontemporal_load(x4 + i), b = {0.f, 0.f, 0.f, 0.f};
      if (i2 < n4) b = __builtin_nontemporal_load(x4 + i2);
      if (beta) {
        a += __builtin_nontemporal_load(y4 + i);
        if (i2 < n4) b += __builtin_nontemporal_load(y4 + i2);
      }
      __builtin_nontemporal_store(a, y4 + i);
      if (i2 < n4) __builtin_nontemporal_store(b, y4 + i2);
    }
    for (int64_t i = n4 * 4 + i0; i < n; i += stride) Y[i] = beta ? Y[i] + X[i] : X[i];
  } else {
    for (int64_t i = i0; i < n; i += stride) Y[i] = beta ? Y[i] + X[i] : X[i];
  }
}

// ───────────────────────── weightedSum (tensor.js:380-389) ─────────────────────────
constexpr int kWsBlocks = 256;
__global__ void __launch_bounds__(kThreads) wsum_partial_kernel(double* __restrict__ part, const float* __restrict__ Y,
                                                                const float* __restrict__ t, int64_t n) {
  __shared__ double sh[kThreads / 64];
  double acc = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    acc += (double)Y[i] * t[i];
  acc = block_sum_d(acc, sh);
  if (threadIdx.x == 0) part[blockIdx.x] = acc;
}
__global__ void __launch_bounds__(kThreads) wsum_final_kernel(float* __restrict__ out, const double* __restrict__ part,
                                                              int nparts) {
  __shared__ double sh[kThreads / 64];
  double acc = 0.0;
  for (int i = threadIdx.x; i < nparts; i += kThreads) acc += part[i];
  acc = block_sum_d(acc, sh);
  if (threadIdx.x == 0) *out = (float)acc;
}
__global__ void __launch_bounds__(kThreads) wsum_bwd_kernel(float* __restrict__ gY, const float* __restrict__ gout,
                                                            const float* __restrict__ t, int64_t n, int beta) {
  const double k = *gout;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const float v = (float)(k * t[i]);
    gY[i] = beta ? (float)((double)gY[i] + k * t[i]) : v;
  }
}

}  // namespace

// ─────────────────────────────── C ABI ───────────────────────────────

template <int NJ>
static int rms_fwd_launch(float* Y, float* inv, const float* X, const float* w, int T, int D, double eps) {
  // 16 waves per CU, each pipelining its rows (measured best at 8192 x 768)
  const int waves = (fg::device_cu_count() > 0 ? fg::device_cu_count() : 256) * 16;
  int blocks = (min(T, waves) + 3) / 4;
  FG_LAUNCH((rmsnorm_fwd_wave<NJ>), dim3(blocks), dim3(kThreads), 0, Y, inv, X, w, T, D, eps);
  return FG_OK;
}
template <int NJ>
static int rms_bwd_launch(float* gX, const float* gx_old, float* part, int nb, const float* g, const float* g2,
                          const float* X, const float* w, const float* inv, int T, int D) {
  if (g2)
    FG_LAUNCH((rmsnorm_bwd_wave<NJ, true>), dim3(nb), dim3(kThreads), 0, gX, gx_old, part, g, g2, X, w, inv, T, D);
  else
    FG_LAUNCH((rmsnorm_bwd_wave<NJ, false>), dim3(nb), dim3(kThreads), 0, gX, gx_old, part, g, g2, X, w, inv, T,
              D);
  return FG_OK;
}
template <int F>
static int rms_bwd_row_launch(float* gX, const float* gx_old, float* part, int nb, const float* g, const float* g2,
                              const float* X, const float* w, const float* inv, int T, int D) {
  if (g2)
    FG_LAUNCH((rmsnorm_bwd_rowwg<F, true>), dim3(nb), dim3(kThreads), 0, gX, gx_old, part, g, g2, X, w, inv, T, D);
  else
    FG_LAUNCH((rmsnorm_bwd_rowwg<F, false>), dim3(nb), dim3(kThreads), 0, gX, gx_old, part, g, g2, X, w, inv, T,
              D);
  return FG_OK;
}
static bool rms_vec(const void* a, const void* b, const void* c, int D) {
  return D % 4 == 0 && D <= 4096 && al16(a) && al16(b) && al16(c);
}

extern "C" int fg_rmsnorm_fwd(float* Y, float* inv, const float* X, const float* w, int T, int D, double eps) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(T > 0 && D > 0, "fg_rmsnorm_fwd: bad shape T=%d D=%d", T, D);
  FG_ARG_CHECK(Y && inv && X && w, "fg_rmsnorm_fwd: null pointer");
  fg::KProfScope prof("rmsnorm_fwd", 0.0, 8.0 * T * (double)D + 4.0 * D + 4.0 * T);
  if (rms_vec(Y, X, w, D)) {
    const int nj = (D / 4 + 63) / 64;
    if (nj <= 1) return rms_fwd_launch<1>(Y, inv, X, w, T, D, eps);
    if (nj <= 2) return rms_fwd_launch<2>(Y, inv, X, w, T, D, eps);
    if (nj <= 3) return rms_fwd_launch<3>(Y, inv, X, w, T, D, eps);
    if (nj <= 4) return rms_fwd_launch<4>(Y, inv, X, w, T, D, eps);
    // rows over 1024 floats: a workgroup per row, rows strided over 4
    // workgroups per CU
    const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
    const int nb = max(1, min(T, 4 * cus));
    const int F = (D / 4 + kThreads - 1) / kThreads;
    if (F <= 2) FG_LAUNCH((rmsnorm_fwd_rowwg<2>), dim3(nb), dim3(kThreads), 0, Y, inv, X, w, T, D, eps);
    else FG_LAUNCH((rmsnorm_fwd_rowwg<4>), dim3(nb), dim3(kThreads), 0, Y, inv, X, w, T, D, eps);
    return FG_OK;
  }
  FG_LAUNCH(rmsnorm_fwd_kernel, dim3(T), dim3(kThreads), 0, Y, inv, X, w, D, eps);
  return FG_OK;
}

// Rows of the partial column-sum matrix of the wave kernels: ~2 workgroups
// per CU, so the matrix stays <= 2*CUs rows.
static int rms_wave_blocks(int T) {
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  return max(1, min((T + 3) / 4, 2 * cus));
}

// g2: null, or the second half of an incoming gradient g + g2 (summed in
// that order, in fp32, before use).  part_out: null (gw is summed here), or
// the caller's [rms_wave_blocks(T) x D] matrix that receives the partial
// column sums of gw instead (the wave kernels only; gw is then unused).
static int rmsnorm_bwd_impl(float* gX, const float* gx_old, float* gw, int beta_w, const float* g, const float* X,
                            const float* w, const float* inv, int T, int D, const float* g2 = nullptr,
                            float* part_out = nullptr) {
  const int beta_x = gx_old != nullptr;
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(T > 0 && D > 0, "fg_rmsnorm_bwd: bad shape T=%d D=%d", T, D);
  FG_ARG_CHECK(gX && g && X && w && inv, "fg_rmsnorm_bwd: null pointer");
  const bool vec = rms_vec(gX, g, X, D) && al16(w) && (gx_old == nullptr || al16(gx_old)) && (g2 == nullptr || al16(g2));
  FG_ARG_CHECK(!part_out || (vec && al16(part_out)),
               "fg_rmsnorm_bwd_partial: needs D %% 4 == 0, D <= 4096 and 16-byte aligned tensors (D=%d)", D);
  fg::KProfScope prof("rmsnorm_bwd", 0.0,
                      (beta_x ? 16.0 : 12.0) * T * (double)D + (g2 ? 4.0 * T * (double)D : 0.0) + 4.0 * T +
                          (part_out ? 0.0 : (beta_w ? 8.0 : 4.0) * D));
  fg::Workspace gsum;
  if (g2 && !vec) {  // generic kernel: add the halves first
    const int64_t n = (int64_t)T * D;
    int rc = gsum.get(sizeof(float) * (size_t)n);
    if (rc) return rc;
    FG_LAUNCH(add_kernel, dim3(grid_1d(n, kThreads)), dim3(kThreads), 0, (float*)gsum.ptr, g, g2, n, 0);
    g = (const float*)gsum.ptr;
    g2 = nullptr;
  }
  // wave path: up to 4 rows per wave per workgroup slot; generic path: 32 rows per workgroup
  const int nb = vec ? rms_wave_blocks(T) : (T + kRowsPerBlock - 1) / kRowsPerBlock;
  fg::Workspace ws;
  float* part = part_out;
  if (part_out) {
    gw = nullptr;
  } else if (gw) {
    int rc = ws.get(sizeof(float) * (size_t)nb * D);
    if (rc) return rc;
    part = (float*)ws.ptr;
  }
  if (vec) {
    const int nj = (D / 4 + 63) / 64;
    int rc;
    if (nj <= 1) rc = rms_bwd_launch<1>(gX, gx_old, part, nb, g, g2, X, w, inv, T, D);
    else if (nj <= 2) rc = rms_bwd_launch<2>(gX, gx_old, part, nb, g, g2, X, w, inv, T, D);
    else if (nj <= 3) rc = rms_bwd_launch<3>(gX, gx_old, part, nb, g, g2, X, w, inv, T, D);
    else if (nj <= 4) rc = rms_bwd_launch<4>(gX, gx_old, part, nb, g, g2, X, w, inv, T, D);
    else if (nj <= 8) rc = rms_bwd_row_launch<2>(gX, gx_old, part, nb, g, g2, X, w, inv, T, D);
    else rc = rms_bwd_row_launch<4>(gX, gx_old, part, nb, g, g2, X, w, inv, T, D);
    if (rc) return rc;
  } else {
    const int chunks = (D + kThreads * kMaxColsPerThread - 1) / (kThreads * kMaxColsPerThread);
    FG_LAUNCH(rmsnorm_bwd_kernel, dim3(nb, chunks), dim3(kThreads), 0, gX, gx_old, part, g, X, w, inv, T, D);
  }
  if (gw) {
    if (D % 4 == 0 && al16(gw))
      FG_LAUNCH(colsum4_kernel, dim3((D / 4 + kStrip4 - 1) / kStrip4), dim3(kColGroups), 0, gw, part, nb, D, beta_w);
    else
      FG_LAUNCH(colsum_kernel, dim3((D + 31) / 32), dim3(kThreads), 0, gw, part, nb, D, beta_w);
  }
  return FG_OK;
}

extern "C" int fg_rmsnorm_bwd(float* gX, int beta_x, float* gw, int beta_w, const float* g, const float* X,
                              const float* w, const float* inv, int T, int D) {
  return rmsnorm_bwd_impl(gX, beta_x ? gX : nullptr, gw, beta_w, g, X, w, inv, T, D);
}

extern "C" int fg_rmsnorm_bwd_from(float* gX, const float* gX_in, float* gw, int beta_w, const float* g,
                                   const float* X, const float* w, const float* inv, int T, int D) {
  return rmsnorm_bwd_impl(gX, gX_in, gw, beta_w, g, X, w, inv, T, D);
}

extern "C" int fg_rmsnorm_bwd_from_halves(float* gX, const float* gX_in, float* gw, int beta_w, const float* g_halves,
                                          const float* X, const float* w, const float* inv, int T, int D) {
  FG_ARG_CHECK(g_halves, "fg_rmsnorm_bwd_from_halves: null pointer");
  return rmsnorm_bwd_impl(gX, gX_in, gw, beta_w, g_halves, X, w, inv, T, D, g_halves + (size_t)T * D);
}

extern "C" int fg_rmsnorm_bwd_parts(int T, int D) {
  FG_REQUIRE_INIT();
  if (T <= 0 || D <= 0 || D % 4 != 0 || D > 4096) return 0;
  return rms_wave_blocks(T);
}

extern "C" int fg_rmsnorm_bwd_partial(float* gX, const float* gX_in, float* partial, const float* g, int g_halves,
                                      const float* X, const float* w, const float* inv, int T, int D) {
  FG_ARG_CHECK(partial && g, "fg_rmsnorm_bwd_partial: null pointer");
  return rmsnorm_bwd_impl(gX, gX_in, nullptr, 0, g, X, w, inv, T, D, g_halves ? g + (size_t)T * D : nullptr,
                          partial);
}

extern "C" int fg_colsum_grouped(const fg_colsum_job* jobs, int count) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(count >= 0 && (count == 0 || jobs), "fg_colsum_grouped: bad job list");
  double bytes = 0.0;
  for (int i = 0; i < count; ++i) {
    const fg_colsum_job& j = jobs[i];
    FG_ARG_CHECK(j.out && j.partial && j.rows > 0 && j.n > 0 && j.n % 4 == 0 && al16(j.out) && al16(j.partial),
                 "fg_colsum_grouped: job %d needs rows > 0, n %% 4 == 0 and 16-byte aligned buffers (rows=%d n=%d)",
                 i, j.rows, j.n);
    bytes += 4.0 * j.rows * (double)j.n + (j.beta ? 8.0 : 4.0) * j.n;
  }
  if (count == 0) return FG_OK;
  fg::KProfScope prof("rmsnorm_dw_colsum", 0.0, bytes);
  // Jobs run in launches of at most kMaxColJobs; a job whose output is
  // already written by an earlier job of the current launch starts the next
  // launch, so jobs on one output apply in order (the later ones accumulate).
  for (int b0 = 0; b0 < count;) {
    ColTable t{};
    int64_t blocks = 0;
    while (t.count < kMaxColJobs && b0 + t.count < count) {
      const fg_colsum_job& j = jobs[b0 + t.count];
      bool clash = false;
      for (int k = 0; k < t.count; ++k) clash = clash || t.out[k] == j.out;
      if (clash) break;
      const int i = t.count++;
      t.start[i] = (int)blocks;
      t.out[i] = j.out;
      t.part[i] = j.partial;
      t.rows[i] = j.rows;
      t.n[i] = j.n;
      t.beta[i] = j.beta ? 1 : 0;
      blocks += (j.n / 4 + kStrip4 - 1) / kStrip4;
    }
    FG_ARG_CHECK(blocks < (1ll << 31), "fg_colsum_grouped: too many columns in one launch");
    t.start[t.count] = (int)blocks;
    FG_LAUNCH(colsum4_grouped, dim3((unsigned)blocks), dim3(kColGroups), 0, t);
    b0 += t.count;
  }
  return FG_OK;
}

extern "C" int fg_rope_table(double* cos_tab, double* sin_tab, int npos, int dHead, double theta) {
  FG_ARG_CHECK(cos_tab && sin_tab && npos >= 0 && dHead > 0 && dHead % 2 == 0, "fg_rope_table: bad arguments");
  const int half = dHead / 2;
  for (int p = 0; p < npos; ++p)
    for (int i = 0; i < dHead; i += 2) {
      const double freq = 1.0 / pow(theta, (double)i / dHead);
      const double ang = (double)p * freq;
      cos_tab[(int64_t)p * half + i / 2] = cos(ang);
      sin_tab[(int64_t)p * half + i / 2] = sin(ang);
    }
  return FG_OK;
}

static int rope_common(const char* name, float* Y, const float* X, const double* ct, const double* st, int npos,
                       int T, int nHead, int dHead, int pos0, int posStride, int backward, int beta) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(T > 0 && nHead > 0 && dHead > 0 && dHead % 2 == 0, "%s: bad shape", name);
  FG_ARG_CHECK(Y && X && ct && st, "%s: null pointer", name);
  FG_ARG_CHECK(((uintptr_t)X % 8 == 0) && ((uintptr_t)Y % 8 == 0), "%s: tensors must be 8-byte aligned", name);
  const int maxpos = pos0 + (posStride > 0 ? (T < posStride ? T : posStride) : T) - 1;
  FG_ARG_CHECK(pos0 >= 0 && maxpos < npos, "%s: positions up to %d exceed the %d-entry table", name, maxpos, npos);
  const int64_t npairs = (int64_t)T * nHead * dHead / 2;
  fg::KProfScope prof(name, 0.0, (backward && beta ? 12.0 : 8.0) * npairs * 2.0);
  FG_LAUNCH(rope_kernel, dim3(grid_1d(npairs, kThreads)), dim3(kThreads), 0, Y, X, ct, st, npairs, nHead, dHead, pos0,
            posStride, backward, beta);
  return FG_OK;
}

extern "C" int fg_rope_fwd(float* Y, const float* X, const double* cos_tab, const double* sin_tab, int npos, int T,
                           int nHead, int dHead, int pos0, int posStride) {
  return rope_common("rope_fwd", Y, X, cos_tab, sin_tab, npos, T, nHead, dHead, pos0, posStride, 0, 0);
}

extern "C" int fg_rope_bwd(float* gX, const float* g, const double* cos_tab, const double* sin_tab, int npos, int T,
                           int nHead, int dHead, int pos0, int posStride, int beta) {
  return rope_common("rope_bwd", gX, g, cos_tab, sin_tab, npos, T, nHead, dHead, pos0, posStride, 1, beta);
}

extern "C" int fg_swiglu_fwd(float* O, const float* G, const float* U, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && O && G && U, "fg_swiglu_fwd: bad arguments");
  FG_ARG_CHECK(al16(O) && al16(G) && al16(U), "fg_swiglu_fwd: tensors must be 16-byte aligned");
  if (n == 0) return FG_OK;
  fg::KProfScope prof("swiglu_fwd", 0.0, 12.0 * n);
  FG_LAUNCH(swiglu_fwd_kernel, dim3(grid_1d(n / 4 + 1, kThreads)), dim3(kThreads), 0, O, G, U, n);
  return FG_OK;
}

extern "C" int fg_swiglu_bwd(float* gG, int beta_g, float* gU, int beta_u, const float* g, const float* G,
                             const float* U, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && g && G && U && (gG || gU), "fg_swiglu_bwd: bad arguments");
  FG_ARG_CHECK(al16(g) && al16(G) && al16(U) && (!gG || al16(gG)) && (!gU || al16(gU)),
               "fg_swiglu_bwd: tensors must be 16-byte aligned");
  if (n == 0) return FG_OK;
  fg::KProfScope prof("swiglu_bwd", 0.0, (20.0 + 4.0 * ((beta_g ? 1 : 0) + (beta_u ? 1 : 0))) * n);
  FG_LAUNCH(swiglu_bwd_kernel, dim3(grid_1d(n / 4 + 1, kThreads)), dim3(kThreads), 0, gG, beta_g, gU, beta_u, g, G, U,
            n);
  return FG_OK;
}

extern "C" int fg_embed_fwd(float* X, const float* W, const int32_t* ids, int T, int V, int D) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(T > 0 && V > 0 && D > 0 && X && W && ids, "fg_embed_fwd: bad arguments");
  fg::KProfScope prof("embed_fwd", 0.0, 8.0 * T * (double)D + 4.0 * T);
  if (D % 4 == 0 && al16(X) && al16(W)) {
    const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
    const int blocks = max(1, min((T + 3) / 4, 32 * cus));  // one wave per row, up to 128 waves per CU
    FG_LAUNCH(embed_fwd4_kernel, dim3(blocks), dim3(kThreads), 0, X, W, ids, T, V, D / 4);
    return FG_OK;
  }
  FG_LAUNCH(embed_fwd_kernel, dim3(grid_1d((int64_t)T * D, kThreads)), dim3(kThreads), 0, X, W, ids, T, V, D);
  return FG_OK;
}

extern "C" int fg_embed_plan(const int32_t* ids, int T, int V, int32_t* perm, int32_t* seg_start, int32_t* seg_id,
                             int* nseg) {
  FG_ARG_CHECK(ids && perm && seg_start && seg_id && nseg && T >= 0 && V > 0, "fg_embed_plan: bad arguments");
  std::vector<int32_t> count((size_t)V + 1, 0);
  for (int t = 0; t < T; ++t) {
    const int id = ids[t];
    FG_ARG_CHECK(id >= 0 && id < V, "fg_embed_plan: id %d at position %d is outside [0,%d)", id, t, V);
    count[id + 1]++;
  }
  for (int v = 0; v < V; ++v) count[v + 1] += count[v];
  std::vector<int32_t> fill(count.begin(), count.end() - 1);
  for (int t = 0; t < T; ++t) perm[fill[ids[t]]++] = t;  // stable: increasing t per id
  int ns = 0;
  for (int v = 0; v < V; ++v)
    if (count[v + 1] > count[v]) {
      seg_id[ns] = v;
      seg_start[ns] = count[v];
      ++ns;
    }
  seg_start[ns] = T;
  *nseg = ns;
  return FG_OK;
}

extern "C" int fg_embed_bwd(float* gW, const float* g, const int32_t* perm, const int32_t* seg_start,
                            const int32_t* seg_id, int nseg, int D) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(nseg >= 0 && D > 0 && gW && g && perm && seg_start && seg_id, "fg_embed_bwd: bad arguments");
  if (nseg == 0) return FG_OK;
  fg::KProfScope prof("embed_bwd", 0.0, 8.0 * nseg * (double)D);
  FG_LAUNCH(embed_bwd_kernel, dim3(nseg), dim3(kThreads), 0, gW, g, perm, seg_start, seg_id, D);
  return FG_OK;
}

extern "C" int fg_slice_cols_fwd(float* Y, const float* X, int M, int K, int off, int len) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(M > 0 && len > 0 && off >= 0 && off + len <= K && Y && X, "fg_slice_cols_fwd: bad arguments");
  fg::KProfScope prof("slice_cols_fwd", 0.0, 8.0 * M * (double)len);
  FG_LAUNCH(slice_kernel, dim3(grid_1d((int64_t)M * len, kThreads)), dim3(kThreads), 0, Y, X, M, K, off, len, 0);
  return FG_OK;
}

extern "C" int fg_slice_cols_bwd(float* gX, const float* g, int M, int K, int off, int len) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(M > 0 && len > 0 && off >= 0 && off + len <= K && gX && g, "fg_slice_cols_bwd: bad arguments");
  fg::KProfScope prof("slice_cols_bwd", 0.0, 12.0 * M * (double)len);
  FG_LAUNCH(slice_kernel, dim3(grid_1d((int64_t)M * len, kThreads)), dim3(kThreads), 0, gX, g, M, K, off, len, 1);
  return FG_OK;
}

extern "C" int fg_add_fwd(float* Y, const float* A, const float* B, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && Y && A && B, "fg_add_fwd: bad arguments");
  if (n == 0) return FG_OK;
  fg::KProfScope prof("add_fwd", 0.0, 12.0 * n);
  FG_LAUNCH(add_kernel, dim3(grid_1d(n / 4 + 1, kThreads)), dim3(kThreads), 0, Y, A, B, n,
            (int)(al16(Y) && al16(A) && al16(B)));
  return FG_OK;
}

extern "C" int fg_accum(float* Y, const float* X, int64_t n, int beta) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && Y && X, "fg_accum: bad arguments");
  if (n == 0) return FG_OK;
  fg::KProfScope prof("accum", 0.0, (beta ? 12.0 : 8.0) * n);
  // two float4 per thread, at most 32 workgroups per CU (measured best for
  // the 6-25M-element gradient adds of a step)
  int64_t g = (n / 8 + kThreads) / kThreads;
  const int64_t cap = (int64_t)(fg::device_cu_count() > 0 ? fg::device_cu_count() : 256) * 32;
  if (g > cap) g = cap;
  FG_LAUNCH(accum_kernel, dim3((unsigned)(g < 1 ? 1 : g)), dim3(kThreads), 0, Y, X, n, beta,
            (int)(al16(Y) && al16(X)));
  return FG_OK;
}

extern "C" int fg_weighted_sum_fwd(float* out, const float* Y, const float* t, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && out && Y && t, "fg_weighted_sum_fwd: bad arguments");
  fg::KProfScope prof("weighted_sum_fwd", 0.0, 8.0 * n);
  fg::Workspace ws;
  int rc = ws.get(sizeof(double) * kWsBlocks);
  if (rc) return rc;
  FG_LAUNCH(wsum_partial_kernel, dim3(kWsBlocks), dim3(kThreads), 0, (double*)ws.ptr, Y, t, n);
  FG_LAUNCH(wsum_final_kernel, dim3(1), dim3(kThreads), 0, out, (const double*)ws.ptr, kWsBlocks);
  return FG_OK;
}

extern "C" int fg_weighted_sum_bwd(float* gY, const float* gout, const float* t, int64_t n, int beta) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && gY && gout && t, "fg_weighted_sum_bwd: bad arguments");
  if (n == 0) return FG_OK;
  fg::KProfScope prof("weighted_sum_bwd", 0.0, (beta ? 12.0 : 8.0) * n);
  FG_LAUNCH(wsum_bwd_kernel, dim3(grid_1d(n, kThreads)), dim3(kThreads), 0, gY, gout, t, n, beta);
  return FG_OK;
}

static int qkv_rope_common(const char* name, float* Q, float* K, float* V, float* G, const double* ct,
                           const double* st, int npos, int rows, int nH, int nKV, int dH, int pos0, int posStride,
                           int backward, int beta) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && nH > 0 && nKV > 0 && dH > 0 && dH % 2 == 0, "%s: bad shape", name);
  FG_ARG_CHECK(G && ct && st && (backward || (Q && K && V)), "%s: null pointer", name);
  FG_ARG_CHECK(((uintptr_t)G % 8 == 0) && (!Q || (uintptr_t)Q % 8 == 0) && (!K || (uintptr_t)K % 8 == 0) &&
                   (!V || (uintptr_t)V % 8 == 0),
               "%s: tensors must be 8-byte aligned", name);
  const int maxpos = pos0 + (posStride > 0 ? (rows < posStride ? rows : posStride) : rows) - 1;
  FG_ARG_CHECK(pos0 >= 0 && maxpos < npos, "%s: positions up to %d exceed the %d-entry table", name, maxpos, npos);
  const int64_t pairs = (int64_t)rows * (nH + 2 * nKV) * dH / 2;
  fg::KProfScope prof(name, 0.0, (backward && beta ? 24.0 : 16.0) * pairs);
  const int rowP = (nH + 2 * nKV) * dH / 2;
  const bool quad = dH % 4 == 0 && ((uintptr_t)G % 16 == 0) && ((uintptr_t)ct % 16 == 0) && ((uintptr_t)st % 16 == 0) && (!Q || (uintptr_t)Q % 16 == 0) &&
                    (!K || (uintptr_t)K % 16 == 0) && (!V || (uintptr_t)V % 16 == 0) &&
                    (int64_t)rows * (rowP / 2) < ((int64_t)1 << 31) - (int64_t)kThreads * 65536;
  if (quad) {
    FG_LAUNCH(qkv_rope4_kernel, dim3(grid_1d((int64_t)rows * (rowP / 2), kThreads)), dim3(kThreads), 0, Q, K, V, G,
              ct, st, rows, nH, nKV, dH, pos0, posStride, backward, beta);
    return FG_OK;
  }
  FG_LAUNCH(qkv_rope_kernel, dim3(rows, (rowP + kThreads - 1) / kThreads), dim3(kThreads), 0, Q, K, V, G, ct, st, nH,
            nKV, dH, pos0, posStride, backward, beta);
  return FG_OK;
}

extern "C" int fg_qkv_rope_fwd(float* Q, float* K, float* V, const float* qkv, const double* cos_tab,
                               const double* sin_tab, int npos, int rows, int nH, int nKV, int dH, int pos0,
                               int posStride) {
  return qkv_rope_common("qkv_rope_fwd", Q, K, V, const_cast<float*>(qkv), cos_tab, sin_tab, npos, rows, nH, nKV, dH,
                         pos0, posStride, 0, 0);
}

extern "C" int fg_qkv_rope_bwd(float* gqkv, const float* gQ, const float* gK, const float* gV, const double* cos_tab,
                               const double* sin_tab, int npos, int rows, int nH, int nKV, int dH, int pos0,
                               int posStride, int beta) {
  return qkv_rope_common("qkv_rope_bwd", const_cast<float*>(gQ), const_cast<float*>(gK), const_cast<float*>(gV), gqkv,
                         cos_tab, sin_tab, npos, rows, nH, nKV, dH, pos0, posStride, 1, beta);
}

extern "C" int fg_swiglu_gu_fwd(float* O, const float* GU, int rows, int H) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && H > 0 && O && GU, "fg_swiglu_gu_fwd: bad arguments rows=%d H=%d", rows, H);
  fg::KProfScope prof("swiglu_fwd", 0.0, 12.0 * rows * (double)H);
  if (H % 4 == 0 && al16(O) && al16(GU)) {
    FG_LAUNCH(swiglu_gu_fwd_kernel, dim3(rows, (H / 4 + kThreads - 1) / kThreads), dim3(kThreads), 0, O, GU, H);
    return FG_OK;
  }
  const int64_t n = (int64_t)rows * H;
  FG_LAUNCH(swiglu_gu_fwd_any, dim3(grid_1d(n, kThreads)), dim3(kThreads), 0, O, GU, n, H);
  return FG_OK;
}

extern "C" int fg_swiglu_gu_bwd(float* gGU, int beta, const float* g, const float* GU, int rows, int H) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && H > 0 && gGU && g && GU, "fg_swiglu_gu_bwd: bad arguments rows=%d H=%d", rows, H);
  fg::KProfScope prof("swiglu_bwd", 0.0, (20.0 + (beta ? 8.0 : 0.0)) * rows * (double)H);
  if (H % 4 == 0 && al16(gGU) && al16(g) && al16(GU)) {
    FG_LAUNCH(swiglu_gu_bwd_kernel, dim3(rows, (H / 4 + kThreads - 1) / kThreads), dim3(kThreads), 0, gGU, beta, g,
              GU, H);
    return FG_OK;
  }
  const int64_t n = (int64_t)rows * H;
  FG_LAUNCH(swiglu_gu_bwd_any, dim3(grid_1d(n, kThreads)), dim3(kThreads), 0, gGU, beta, g, GU, n, H);
  return FG_OK;
}

// fg_swiglu_gu_bwd that also leaves the partial maxima of gGU in xp_out.
extern "C" int fg_swiglu_gu_bwd_p(float* gGU, int beta, const float* g, const float* GU, int rows, int H,
                                  float* xp_out) {
  if (!xp_out) return fg_swiglu_gu_bwd(gGU, beta, g, GU, rows, H);
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(rows > 0 && H > 0 && gGU && g && GU, "fg_swiglu_gu_bwd_p: bad arguments rows=%d H=%d", rows, H);
  if (H % 4 == 0 && al16(gGU) && al16(g) && al16(GU)) {
    fg::KProfScope prof("swiglu_bwd", 0.0, (20.0 + (beta ? 8.0 : 0.0)) * rows * (double)H);
    FG_LAUNCH(swiglu_gu_bwd_xp_kernel, dim3(kXpParts), dim3(kSwXpThreads), 0, gGU, beta, g, GU, rows, H, xp_out);
    return FG_OK;
  }
  const int rc = fg_swiglu_gu_bwd(gGU, beta, g, GU, rows, H);
  if (rc != FG_OK) return rc;
  const fg::XpSpec sp{gGU, xp_out, rows, 2 * H, 2 * H};
  return fg::absmax_parts(&sp, 1, "gemm_absmax");
}
