// Single-token inference forward (Transformer.forward, transformer.js:134-184)
// for gfx950.  One decode step is four launches per layer plus one:
//
//   per layer:
//     qkv        xn = rmsnorm(x, ln1); [q|k|v] = Wqkv·xn; RoPE on q, k with the
//                fp32 table (special.js:116-127); k, v written into the cache
//                at pos.  Layer 0 reads x as tok_emb[token] (transformer.js:
//                120-129) and also stores it.
//     attn       per (q head, 64-position chunk): scores q·K/√dH, the chunk's
//                softmax partials and p·V (attentionDecode, attention.js:31-61)
//     wo         the per-head combine of the partials, then x += Wo·att
//                (transformer.js:176-177)
//     gateup     xn = rmsnorm(x, ln2); h = silu(Wg·xn) * (Wu·xn)     (nn.js:56-66)
//     down       x += Wd·h                                           (:179-180)
//   head         logits = Wcls·rmsnorm(x, ln_f)                      (:182-183)
//
// Token and position are read from device memory (`state` = {token, pos}),
// so a recorded graph of one step replays every later step unchanged.
//
// A decode step reads every weight once: the matvecs are HBM-bound, so they
// accumulate in fp64 (free at 2 flop per 4 bytes), round each output once to
// fp32 and apply the reference's epilogues in fp64 (RMSNorm x·ss·w, RoPE
// a·c − b·s on the fp32 table, residual x + fp32(y), SwiGLU (g/(1+e^−g))·u).
// The reference sums in fp64 too, in another order, so outputs agree with it
// except where an fp64 sum sits on an fp32 rounding tie.  The attention sums
// p·V in fp64 over position chunks (the reference accumulates in fp32, one
// position after another), within 1e-7 relative of it.
//
// At batch 1 each launch is short, so the kernels are built around latency:
// every matvec issues the loads of its first rows before its prologue (the
// norm of x, or the attention combine) so the two overlap, and the attention
// loads K and V rows together.
#include "common.h"
#include "qformat.h"

#include <math.h>

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPF = 4;      // float4 per lane and row loaded ahead of a prologue (K <= 1024 in full)
constexpr int kChunk = 64;  // cache positions per attention workgroup

__device__ __forceinline__ double block_sum_d(double v, double* sh) {
  v = fg_wave_sum_d(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < kWaves; ++i) t += sh[i];
  return t;
}

__device__ __forceinline__ double wave_max_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const double u = __shfl_xor(v, o, 64);
    v = u > v ? u : v;
  }
  return v;
}

// xn[0..K) = fp32(x·ss·w), ss = 1/sqrt(rms² + eps), rms = sqrt(Σx²/K) in fp64
// (special.js:46-50, numeric.js:74-78).
__device__ void rmsnorm_to_lds(float* xn, const float* __restrict__ x, const float* __restrict__ w, int K,
                               double eps, double* sh) {
#pragma clang fp contract(off)
  double s = 0.0;
  for (int i = threadIdx.x; i < K; i += kThreads) {
    const double v = x[i];
    s += v * v;
  }
  s = block_sum_d(s, sh);
  const double rms = sqrt(s / K);
  const double ss = 1.0 / sqrt(rms * rms + eps);
  for (int i = threadIdx.x; i < K; i += kThreads) xn[i] = (float)(((double)x[i] * ss) * (double)w[i]);
  __syncthreads();
}

// R weight rows of one wave, the first PF float4 per lane loaded ahead.
template <int R, int PF = kPF>
struct Rows {
  const float* p[R];
  float4 pf[R][PF];
};

template <int R, int PF>
__device__ __forceinline__ void rows_prefetch(Rows<R, PF>& rw, int K) {
  if ((K & 3) != 0) return;
  const int lane = threadIdx.x & 63, K4 = K >> 2;
#pragma unroll
  for (int t = 0; t < PF; ++t) {
    const int k = lane + 64 * t;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (k < K4) rw.pf[r][t] = reinterpret_cast<const float4*>(rw.p[r])[k];
  }
}

// out[r] = W[row r]·xn (xn in LDS), fp64 per lane, reduced across the wave
// (every lane gets the sums).
template <int R, int PF>
__device__ __forceinline__ void rows_finish(double (&out)[R], const Rows<R, PF>& rw, const float* xn, int K) {
  const int lane = threadIdx.x & 63;
  double acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0;
  if ((K & 3) == 0) {
    const float4* x4 = reinterpret_cast<const float4*>(xn);
    const int K4 = K >> 2;
#pragma unroll
    for (int t = 0; t < PF; ++t) {
      const int k = lane + 64 * t;
      if (k < K4) {
        const float4 xv = x4[k];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          acc[r] += (double)rw.pf[r][t].x * xv.x;
          acc[r] += (double)rw.pf[r][t].y * xv.y;
          acc[r] += (double)rw.pf[r][t].z * xv.z;
          acc[r] += (double)rw.pf[r][t].w * xv.w;
        }
      }
    }
    for (int k = lane + 64 * PF; k < K4; k += 64) {
      float4 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r) wv[r] = reinterpret_cast<const float4*>(rw.p[r])[k];
      const float4 xv = x4[k];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        acc[r] += (double)wv[r].x * xv.x;
        acc[r] += (double)wv[r].y * xv.y;
        acc[r] += (double)wv[r].z * xv.z;
        acc[r] += (double)wv[r].w * xv.w;
      }
    }
  } else {
    for (int k = lane; k < K; k += 64) {
      const double xv = xn[k];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += (double)rw.p[r][k] * xv;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = fg_wave_sum_d(acc[r]);
}

// R weight rows of a matrix of ggml type QT (rows of rb bytes): f32 rows use
// the prefetching path above, quantized rows the block dots of qformat.h.
template <int QT, int R, int PF = kPF>
struct WRows {
  Rows<R, PF> f;
  const uint8_t* p[R];
  __device__ __forceinline__ void set(int r, const uint8_t* W, int64_t row, int64_t rb) {
    if constexpr (QT == fgq::kF32) f.p[r] = reinterpret_cast<const float*>(W + row * rb);
    else p[r] = W + row * rb;
  }
  __device__ __forceinline__ void prefetch(int K) {
    if constexpr (QT == fgq::kF32) rows_prefetch(f, K);
  }
  __device__ __forceinline__ void finish(double (&out)[R], const float* xs, int K) {
    if constexpr (QT == fgq::kF32) {
      rows_finish<R, PF>(out, f, xs, K);
    } else {
      double acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.0;
      fgq::qrows_dot<QT, R>(acc, p, xs, K);
#pragma unroll
      for (int r = 0; r < R; ++r) out[r] = fg_wave_sum_d(acc[r]);
    }
  }
};

// x = the embedding row of the token (a quantized tok_emb, decoded as
// Transformer._embed does, transformer.js:121-131); NaN for a token outside [0,V).
template <int QT>
__global__ void __launch_bounds__(kThreads) dec_embed_kernel(float* __restrict__ x, const uint8_t* __restrict__ emb,
                                                             int64_t rb, int V, const int32_t* __restrict__ state,
                                                             int D) {
  const int tok = state[0];
  const bool ok = tok >= 0 && tok < V;
  for (int i = blockIdx.x * kThreads + threadIdx.x; i < D; i += gridDim.x * kThreads)
    x[i] = ok ? fgq::dq_elem<QT>(emb + (int64_t)tok * rb, i) : NAN;
}

// Row pairs (n, n+1) per wave: RoPE rotates adjacent pairs, so a pair's two
// dot products are all its rotation needs.  With emb (layer 0) the input
// vector is the token's embedding row (NaN for a token outside [0,V)), which
// workgroup 0 also stores into x for the residual stream.
template <int QT>
__global__ void __launch_bounds__(kThreads) dec_qkv_kernel(float* __restrict__ q, float* __restrict__ kc,
                                                           float* __restrict__ vc, float* __restrict__ x,
                                                           const float* __restrict__ emb, int V,
                                                           const float* __restrict__ ln1, double eps,
                                                           const uint8_t* __restrict__ W, int64_t rb,
                                                           const float* __restrict__ rcos,
                                                           const float* __restrict__ rsin,
                                                           const int32_t* __restrict__ state, int D, int qD, int kvD,
                                                           int dH, int maxSeq, int64_t layer_off) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) float xn[];
  __shared__ double sh[kWaves];
  const int pairs = (qD + 2 * kvD) >> 1;
  const int stride = gridDim.x * kWaves;
  int pr = blockIdx.x * kWaves + (threadIdx.x >> 6);
  WRows<QT, 2> rw;
  if (pr < pairs) {
    rw.set(0, W, 2 * pr, rb);
    rw.set(1, W, 2 * pr + 1, rb);
    rw.prefetch(D);
  }
  const float* xin = x;
  if (emb) {
    const int tok = state[0];
    const bool ok = tok >= 0 && tok < V;
    float* xs = xn + D;  // the embedding row, staged in LDS
    for (int i = threadIdx.x; i < D; i += kThreads) {
      const float v = ok ? emb[(int64_t)tok * D + i] : NAN;
      xs[i] = v;
      if (blockIdx.x == 0) x[i] = v;
    }
    __syncthreads();
    xin = xs;
  }
  rmsnorm_to_lds(xn, xin, ln1, D, eps, sh);
  const int pos = state[1];
  if (pos < 0 || pos >= maxSeq) return;  // the host rejects such positions
  const int half = dH >> 1;
  const int64_t cache_off = layer_off + (int64_t)pos * kvD;
  for (bool first = true; pr < pairs; pr += stride, first = false) {
    const int n = 2 * pr;
    if (!first) {
      rw.set(0, W, n, rb);
      rw.set(1, W, n + 1, rb);
      rw.prefetch(D);
    }
    double s[2];
    rw.finish(s, xn, D);
    if ((threadIdx.x & 63) != 0) continue;
    const float a = (float)s[0], b = (float)s[1];
    if (n < qD + kvD) {
      const int i2 = (n % dH) >> 1;
      const double c = rcos[pos * half + i2], sn = rsin[pos * half + i2];
      const float o0 = (float)((double)a * c - (double)b * sn);
      const float o1 = (float)((double)a * sn + (double)b * c);
      if (n < qD) {
        q[n] = o0;
        q[n + 1] = o1;
      } else {
        kc[cache_off + n - qD] = o0;
        kc[cache_off + n - qD + 1] = o1;
      }
    } else {
      vc[cache_off + n - qD - kvD] = a;
      vc[cache_off + n - qD - kvD + 1] = b;
    }
  }
}

// Attention over the cache prefix n = pos + 1, flash-decoding style: one
// workgroup per (q head, chunk of kChunk positions).  Each position's score
// is computed by a group of LP lanes (LP a power of two >= dH/4 up to 64; each
// lane takes four dims, or C groups of four above 256 dims), reduced in fp64,
// scaled and kept in fp64 (for the max, as the reference) and as fp32 (the
// reference's Float32Array score buffer,
// from which it takes p = exp(score − max)).  The chunk's p·V is summed in
// fp64 by the same lane groups, position groups reduced in a fixed order.
// Each chunk writes {m, l, acc[dH]} (fp64) to `part`; the wo kernel combines.
template <int LP, int C>
__global__ void __launch_bounds__(kThreads) dec_attn_part_kernel(double* __restrict__ part,
                                                                 const float* __restrict__ q,
                                                                 const float* __restrict__ kc,
                                                                 const float* __restrict__ vc,
                                                                 const int32_t* __restrict__ state, int nH, int nKV,
                                                                 int dH, int maxSeq, int64_t layer_off,
                                                                 double scale, int S) {
#pragma clang fp contract(off)
  constexpr int PP = kThreads / LP;            // positions per pass
  constexpr int NPT = (kChunk + PP - 1) / PP;  // passes per chunk
  constexpr int NPF0 = NPT < 8 ? NPT : 8;
  constexpr int NPF = NPF0 / C > 0 ? NPF0 / C : 1;  // passes whose K, V rows are loaded up front
  constexpr int W4 = 4 * LP * C;                    // head dims covered: lane lc, chunk cc -> 4(lc + LP cc) ..
  __shared__ float qh[W4];
  __shared__ double vsc[kChunk];
  __shared__ double pj[kChunk];
  __shared__ double red[PP][W4];
  const int h = blockIdx.x, c = blockIdx.y;
  const int pos = state[1];
  const int n = (pos >= 0 && pos < maxSeq) ? pos + 1 : 0;
  const int j0 = c * kChunk;
  if (j0 >= n) return;
  const int cnt = n - j0 < kChunk ? n - j0 : kChunk;
  const int kvh = h / (nH / nKV), kvD = nKV * dH;
  const int pg = threadIdx.x / LP, lc = threadIdx.x % LP;
  const bool vec = (dH & 3) == 0;
  bool lane_on[C];
#pragma unroll
  for (int cc = 0; cc < C; ++cc) lane_on[cc] = 4 * (lc + LP * cc) < dH;
  const float* kbase = kc + layer_off + (int64_t)kvh * dH + 4 * lc;
  const float* vbase = vc + layer_off + (int64_t)kvh * dH + 4 * lc;
  float4 kq[NPF][C], vq[NPF][C];
  if (vec) {
#pragma unroll
    for (int t = 0; t < NPF; ++t) {
      const int jj = pg + t * PP;
      if (jj < cnt) {
#pragma unroll
        for (int cc = 0; cc < C; ++cc)
          if (lane_on[cc]) {
            kq[t][cc] = *reinterpret_cast<const float4*>(kbase + 4 * LP * cc + (int64_t)(j0 + jj) * kvD);
            vq[t][cc] = *reinterpret_cast<const float4*>(vbase + 4 * LP * cc + (int64_t)(j0 + jj) * kvD);
          }
      }
    }
  }
  for (int i = threadIdx.x; i < W4; i += kThreads) qh[i] = i < dH ? q[h * dH + i] : 0.f;
  __syncthreads();
  // scores
#pragma unroll
  for (int t = 0; t < NPT; ++t) {
    const int jj = pg + t * PP;
    if (jj >= cnt) break;  // uniform within a lane group
    double s = 0.0;
    if (vec) {
#pragma unroll
      for (int cc = 0; cc < C; ++cc)
        if (lane_on[cc]) {
          const int d0 = 4 * (lc + LP * cc);
          const float4 k4 = t < NPF ? kq[t][cc]
                                    : *reinterpret_cast<const float4*>(kbase + 4 * LP * cc + (int64_t)(j0 + jj) * kvD);
          const double e = (double)qh[d0] * k4.x + (double)qh[d0 + 1] * k4.y + (double)qh[d0 + 2] * k4.z +
                           (double)qh[d0 + 3] * k4.w;
          s = cc == 0 ? e : s + e;
        }
    } else {
      const float* kr = kbase + (int64_t)(j0 + jj) * kvD;
#pragma unroll
      for (int cc = 0; cc < C; ++cc)
        for (int e = 0; e < 4; ++e)
          if (4 * (lc + LP * cc) + e < dH) s += (double)qh[4 * (lc + LP * cc) + e] * (double)kr[4 * LP * cc + e];
    }
#pragma unroll
    for (int o = LP / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lc == 0) vsc[jj] = s * scale;
  }
  __syncthreads();
  // chunk max (fp64 scores) and p = exp(fp32 score − m)
  if (threadIdx.x < 64) {
    double m = threadIdx.x < cnt ? vsc[threadIdx.x] : -INFINITY;
    if (!(m > -INFINITY)) m = -INFINITY;  // NaN scores never raise the max
    m = wave_max_d(m);
    double p = 0.0;
    if (threadIdx.x < cnt) {
      const float sf = (float)vsc[threadIdx.x];
      p = sf == -INFINITY ? 0.0 : exp((double)sf - m);
      pj[threadIdx.x] = p;
    }
    const double l = fg_wave_sum_d(p);
    if (threadIdx.x == 0) {
      double* out = part + ((int64_t)h * S + c) * (dH + 2);
      out[0] = m;
      out[1] = l;
    }
  }
  __syncthreads();
  // Σ p·V
  double acc[4 * C];
#pragma unroll
  for (int e = 0; e < 4 * C; ++e) acc[e] = 0.0;
#pragma unroll
  for (int t = 0; t < NPT; ++t) {
    const int jj = pg + t * PP;
    if (jj >= cnt) break;
    const double p = pj[jj];
    if (p == 0.0) continue;  // the reference skips p = 0 (attention.js:48)
    if (vec) {
#pragma unroll
      for (int cc = 0; cc < C; ++cc)
        if (lane_on[cc]) {
          const float4 v4 = t < NPF ? vq[t][cc]
                                    : *reinterpret_cast<const float4*>(vbase + 4 * LP * cc + (int64_t)(j0 + jj) * kvD);
          acc[4 * cc] += p * (double)v4.x;
          acc[4 * cc + 1] += p * (double)v4.y;
          acc[4 * cc + 2] += p * (double)v4.z;
          acc[4 * cc + 3] += p * (double)v4.w;
        }
    } else {
      const float* vr = vbase + (int64_t)(j0 + jj) * kvD;
#pragma unroll
      for (int cc = 0; cc < C; ++cc)
        for (int e = 0; e < 4; ++e)
          if (4 * (lc + LP * cc) + e < dH) acc[4 * cc + e] += p * (double)vr[4 * LP * cc + e];
    }
  }
#pragma unroll
  for (int cc = 0; cc < C; ++cc)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[pg][4 * (lc + LP * cc) + e] = acc[4 * cc + e];
  __syncthreads();
  double* out = part + ((int64_t)h * S + c) * (dH + 2) + 2;
  for (int i = threadIdx.x; i < dH; i += kThreads) {
    double o = 0.0;
    for (int g = 0; g < PP; ++g) o += red[g][i];
    out[i] = o;
  }
}

// x[n] = fp32(x[n] + fp32(Wo[n]·att)), where att is first combined from the
// attention partials: per head M = max m, w_s = e^(m_s − M), l = Σ l_s·w_s,
// att = fp32(fp32(Σ acc_s·w_s) · (1 / (l || 1))) (attention.js:55-57).
// Dynamic LDS: att[D] floats (rounded up to 4), then w[nH·S], M[nH], inv[nH]
// doubles.
template <int QT>
__global__ void __launch_bounds__(kThreads) dec_wo_kernel(float* __restrict__ x, const double* __restrict__ part,
                                                          const int32_t* __restrict__ state,
                                                          const uint8_t* __restrict__ W, int64_t rb, int D, int nH,
                                                          int dH, int maxSeq, int S) {
  extern __shared__ __attribute__((aligned(16))) float att[];
  double* wsh = reinterpret_cast<double*>(att + ((D + 3) & ~3));
  double* Mh = wsh + nH * S;
  double* invh = Mh + nH;
  const int stride = gridDim.x * kWaves;
  int r = blockIdx.x * kWaves + (threadIdx.x >> 6);
  WRows<QT, 1> rw;
  if (r < D) {
    rw.set(0, W, r, rb);
    rw.prefetch(D);
  }
  const int pos = state[1];
  const int n = (pos >= 0 && pos < maxSeq) ? pos + 1 : 0;
  const int Sa = (n + kChunk - 1) / kChunk;
  for (int hh = threadIdx.x; hh < nH; hh += kThreads) {
    double M = -INFINITY;
    for (int s = 0; s < Sa; ++s) {
      const double m = part[((int64_t)hh * S + s) * (dH + 2)];
      M = m > M ? m : M;
    }
    Mh[hh] = M;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nH * Sa; i += kThreads) {
    const int hh = i / Sa, s = i - hh * Sa;
    wsh[hh * S + s] = exp(part[((int64_t)hh * S + s) * (dH + 2)] - Mh[hh]);
  }
  __syncthreads();
  for (int hh = threadIdx.x; hh < nH; hh += kThreads) {
    double l = 0.0;
    for (int s = 0; s < Sa; ++s) l += part[((int64_t)hh * S + s) * (dH + 2) + 1] * wsh[hh * S + s];
    invh[hh] = (l != 0.0 && l == l) ? 1.0 / l : 1.0;  // `1 / (l || 1)`
  }
  __syncthreads();
  for (int i = threadIdx.x; i < D; i += kThreads) {
    const int hh = i / dH, d = i - hh * dH;
    double o = 0.0;
    for (int s = 0; s < Sa; ++s) o += part[((int64_t)hh * S + s) * (dH + 2) + 2 + d] * wsh[hh * S + s];
    att[i] = (float)((double)(float)o * invh[hh]);
  }
  __syncthreads();
  for (bool first = true; r < D; r += stride, first = false) {
    if (!first) {
      rw.set(0, W, r, rb);
      rw.prefetch(D);
    }
    double s[1];
    rw.finish(s, att, D);
    if ((threadIdx.x & 63) == 0) x[r] = (float)((double)x[r] + (double)(float)s[0]);
  }
}

// x[n] = fp32(x[n] + fp32(W[n]·in)) (the FFN down projection): one row per
// wave with up to kPFDown float4 per lane loaded before the LDS fill of `in`
// (all of a 2048-float row), so a D-row output still gives every CU work.
constexpr int kPFDown = 8;
template <int QT>
__global__ void __launch_bounds__(kThreads) dec_down_kernel(float* __restrict__ x, const float* __restrict__ in,
                                                            const uint8_t* __restrict__ W, int64_t rb, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  const int stride = gridDim.x * kWaves;
  int r = blockIdx.x * kWaves + (threadIdx.x >> 6);
  WRows<QT, 1, kPFDown> rw;
  if (r < N) {
    rw.set(0, W, r, rb);
    rw.prefetch(K);
  }
  for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = in[i];
  __syncthreads();
  for (bool first = true; r < N; r += stride, first = false) {
    if (!first) {
      rw.set(0, W, r, rb);
      rw.prefetch(K);
    }
    double s[1];
    rw.finish(s, xs, K);
    if ((threadIdx.x & 63) == 0) x[r] = (float)((double)x[r] + (double)(float)s[0]);
  }
}

// h[n] = fp32((g / (1 + exp(−g))) · u), g = fp32(Wg[n]·xn), u = fp32(Wu[n]·xn).
template <int QT>
__global__ void __launch_bounds__(kThreads) dec_gateup_kernel(float* __restrict__ hout, const float* __restrict__ x,
                                                              const float* __restrict__ ln2, double eps,
                                                              const uint8_t* __restrict__ Wg,
                                                              const uint8_t* __restrict__ Wu, int64_t rb, int H,
                                                              int D) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) float xn[];
  __shared__ double sh[kWaves];
  const int stride = gridDim.x * kWaves;
  int r = blockIdx.x * kWaves + (threadIdx.x >> 6);
  WRows<QT, 2> rw;
  if (r < H) {
    rw.set(0, Wg, r, rb);
    rw.set(1, Wu, r, rb);
    rw.prefetch(D);
  }
  rmsnorm_to_lds(xn, x, ln2, D, eps, sh);
  for (bool first = true; r < H; r += stride, first = false) {
    if (!first) {
      rw.set(0, Wg, r, rb);
      rw.set(1, Wu, r, rb);
      rw.prefetch(D);
    }
    double s[2];
    rw.finish(s, xn, D);
    if ((threadIdx.x & 63) == 0) {
      const double g = (double)(float)s[0], u = (double)(float)s[1];
      hout[r] = (float)((g / (1.0 + exp(-g))) * u);
    }
  }
}

// logits[n] = fp32(W[n]·rmsnorm(x, ln_f)), two rows per wave.
template <int QT>
__global__ void __launch_bounds__(kThreads) dec_head_kernel(float* __restrict__ logits, const float* __restrict__ x,
                                                            const float* __restrict__ lnf, double eps,
                                                            const uint8_t* __restrict__ W, int64_t rb, int V, int D) {
  extern __shared__ __attribute__((aligned(16))) float xn[];
  __shared__ double sh[kWaves];
  const int pairs = (V + 1) >> 1;
  const int stride = gridDim.x * kWaves;
  int pr = blockIdx.x * kWaves + (threadIdx.x >> 6);
  WRows<QT, 2> rw;
  if (pr < pairs) {
    rw.set(0, W, 2 * pr, rb);
    rw.set(1, W, 2 * pr + 1 < V ? 2 * pr + 1 : 2 * pr, rb);
    rw.prefetch(D);
  }
  rmsnorm_to_lds(xn, x, lnf, D, eps, sh);
  for (bool first = true; pr < pairs; pr += stride, first = false) {
    const int r0 = 2 * pr, r1 = 2 * pr + 1 < V ? 2 * pr + 1 : 2 * pr;
    if (!first) {
      rw.set(0, W, r0, rb);
      rw.set(1, W, r1, rb);
      rw.prefetch(D);
    }
    double s[2];
    rw.finish(s, xn, D);
    if ((threadIdx.x & 63) == 0) {
      logits[r0] = (float)s[0];
      if (r1 != r0) logits[r1] = (float)s[1];
    }
  }
}

unsigned grid_for_waves(int64_t waves) {
  int64_t g = (waves + kWaves - 1) / kWaves;
  const int64_t cap = (int64_t)(fg::device_cu_count() > 0 ? fg::device_cu_count() : 256) * 16;
  if (g > cap) g = cap;
  return (unsigned)(g < 1 ? 1 : g);
}

template <int LP, int C = 1>
int launch_attn(const fg_decode_model* m, float* kcache, float* vcache, const int32_t* state, int dH,
                int64_t layer_off, double scale, int S) {
  FG_LAUNCH((dec_attn_part_kernel<LP, C>), dim3(m->nHeads, S), dim3(kThreads), 0, m->attn_part, m->q, kcache, vcache,
            state, m->nHeads, m->nKvHeads, dH, m->maxSeq, layer_off, scale, S);
  return FG_OK;
}

}  // namespace

extern "C" int fg_decode_step(const fg_decode_model* m, float* kcache, float* vcache, const int32_t* state,
                              float* logits) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(m && kcache && vcache && state && logits, "fg_decode_step: null argument");
  const int D = m->dim, H = m->hidden, L = m->nLayers, nH = m->nHeads, nKV = m->nKvHeads, V = m->vocab;
  FG_ARG_CHECK(D > 0 && H > 0 && L > 0 && nH > 0 && nKV > 0 && V > 0 && m->maxSeq > 0,
               "fg_decode_step: bad dimensions");
  FG_ARG_CHECK(nH % nKV == 0 && D % nH == 0, "fg_decode_step: nHeads %d must divide dim %d and be a multiple of "
               "nKvHeads %d", nH, D, nKV);
  const int dH = D / nH, qD = nH * dH, kvD = nKV * dH;
  FG_ARG_CHECK(dH % 2 == 0 && dH <= 1024, "fg_decode_step: head dim %d must be even and <= 1024", dH);
  const int S = (m->maxSeq + kChunk - 1) / kChunk;
  const size_t lds_qkv = 2 * (size_t)D * sizeof(float);
  const size_t lds_wo = (size_t)((D + 3) & ~3) * sizeof(float) + ((size_t)nH * S + 2 * nH) * sizeof(double);
  FG_ARG_CHECK(lds_qkv <= 64 * 1024 && lds_wo <= 64 * 1024 && (size_t)H * sizeof(float) <= 64 * 1024,
               "fg_decode_step: dim %d / hidden %d / %d heads x %d chunks exceed the 64 KiB LDS of a launch", D, H,
               nH, S);
  FG_ARG_CHECK(m->layers && m->tok_emb && m->ln_f && m->wcls && m->rope_cos && m->rope_sin && m->x && m->q &&
                   m->h && m->attn_part,
               "fg_decode_step: null model pointer");
  // Every matrix: a known ggml type whose blocks tile its rows (K = dim, or hidden for down).
  auto type_ok = [](int t, int K) { return fgq::known_type(t) && K % fgq::block_elems(t) == 0; };
  FG_ARG_CHECK(type_ok(m->emb_type, D) && type_ok(m->cls_type, D),
               "fg_decode_step: tok_emb type %d / wcls type %d is unsupported or does not tile dim %d", m->emb_type,
               m->cls_type, D);
  int64_t wbytes = fgq::row_bytes(m->cls_type, D) * (int64_t)V;
  for (int l = 0; l < L; ++l) {
    const fg_decode_layer& ly = m->layers[l];
    FG_ARG_CHECK(ly.ln1 && ly.wqkv && ly.wo && ly.ln2 && ly.gate && ly.up && ly.down,
                 "fg_decode_step: layer %d has a null weight", l);
    FG_ARG_CHECK(type_ok(ly.wqkv_type, D) && type_ok(ly.wo_type, D) && type_ok(ly.gate_type, D) &&
                     type_ok(ly.down_type, H) && ly.up_type == ly.gate_type,
                 "fg_decode_step: layer %d: weight types wqkv %d wo %d gate %d up %d down %d (gate and up must "
                 "match; each type must tile its rows of %d / %d)", l, ly.wqkv_type, ly.wo_type, ly.gate_type,
                 ly.up_type, ly.down_type, D, H);
    wbytes += fgq::row_bytes(ly.wqkv_type, D) * (qD + 2 * kvD) + fgq::row_bytes(ly.wo_type, D) * D +
              2 * fgq::row_bytes(ly.gate_type, D) * H + fgq::row_bytes(ly.down_type, H) * D;
  }
  const double eps = m->normEps;
  const double scale = 1.0 / sqrt((double)dH);
  int LP = 1;
  while (4 * LP < dH && LP < 64) LP <<= 1;
  fg::KProfScope prof("decode_step", 0.0, (double)wbytes);
  const bool emb_f32 = m->emb_type == fgq::kF32;
  if (!emb_f32) {
    const uint8_t* emb = static_cast<const uint8_t*>(m->tok_emb);
    const int64_t erb = fgq::row_bytes(m->emb_type, D);
    const unsigned g = (unsigned)((D + kThreads - 1) / kThreads);
    FGQ_DISPATCH(m->emb_type, {
      FG_LAUNCH(dec_embed_kernel<QT>, dim3(g), dim3(kThreads), 0, m->x, emb, erb, V, state, D);
    });
  }
  for (int l = 0; l < L; ++l) {
    const fg_decode_layer& ly = m->layers[l];
    const int64_t layer_off = (int64_t)l * m->maxSeq * kvD;
    const float* emb0 = (l == 0 && emb_f32) ? static_cast<const float*>(m->tok_emb) : nullptr;
    {
      const uint8_t* W = static_cast<const uint8_t*>(ly.wqkv);
      const int64_t rb = fgq::row_bytes(ly.wqkv_type, D);
      FGQ_DISPATCH(ly.wqkv_type, {
        FG_LAUNCH(dec_qkv_kernel<QT>, dim3(grid_for_waves((qD + 2 * kvD) / 2)), dim3(kThreads), lds_qkv, m->q,
                  kcache, vcache, m->x, emb0, V, ly.ln1, eps, W, rb, m->rope_cos, m->rope_sin, state, D, qD, kvD,
                  dH, m->maxSeq, layer_off);
      });
    }
    int rc;
    switch (LP) {
      case 1: rc = launch_attn<1>(m, kcache, vcache, state, dH, layer_off, scale, S); break;
      case 2: rc = launch_attn<2>(m, kcache, vcache, state, dH, layer_off, scale, S); break;
      case 4: rc = launch_attn<4>(m, kcache, vcache, state, dH, layer_off, scale, S); break;
      case 8: rc = launch_attn<8>(m, kcache, vcache, state, dH, layer_off, scale, S); break;
      case 16: rc = launch_attn<16>(m, kcache, vcache, state, dH, layer_off, scale, S); break;
      case 32: rc = launch_attn<32>(m, kcache, vcache, state, dH, layer_off, scale, S); break;
      default:  // 64 lanes per position, 1, 2 or 4 float4 each
        rc = dH <= 256   ? launch_attn<64>(m, kcache, vcache, state, dH, layer_off, scale, S)
             : dH <= 512 ? launch_attn<64, 2>(m, kcache, vcache, state, dH, layer_off, scale, S)
                         : launch_attn<64, 4>(m, kcache, vcache, state, dH, layer_off, scale, S);
        break;
    }
    if (rc) return rc;
    {
      const uint8_t* W = static_cast<const uint8_t*>(ly.wo);
      const int64_t rb = fgq::row_bytes(ly.wo_type, D);
      FGQ_DISPATCH(ly.wo_type, {
        FG_LAUNCH(dec_wo_kernel<QT>, dim3(grid_for_waves(D)), dim3(kThreads), lds_wo, m->x,
                  (const double*)m->attn_part, state, W, rb, D, nH, dH, m->maxSeq, S);
      });
    }
    {
      const uint8_t* Wg = static_cast<const uint8_t*>(ly.gate);
      const uint8_t* Wu = static_cast<const uint8_t*>(ly.up);
      const int64_t rb = fgq::row_bytes(ly.gate_type, D);
      FGQ_DISPATCH(ly.gate_type, {
        FG_LAUNCH(dec_gateup_kernel<QT>, dim3(grid_for_waves(H)), dim3(kThreads), D * sizeof(float), m->h, m->x,
                  ly.ln2, eps, Wg, Wu, rb, H, D);
      });
    }
    {
      const uint8_t* W = static_cast<const uint8_t*>(ly.down);
      const int64_t rb = fgq::row_bytes(ly.down_type, H);
      FGQ_DISPATCH(ly.down_type, {
        FG_LAUNCH(dec_down_kernel<QT>, dim3(grid_for_waves(D)), dim3(kThreads), H * sizeof(float), m->x,
                  m->h, W, rb, D, H);
      });
    }
  }
  {
    const uint8_t* W = static_cast<const uint8_t*>(m->wcls);
    const int64_t rb = fgq::row_bytes(m->cls_type, D);
    FGQ_DISPATCH(m->cls_type, {
      FG_LAUNCH(dec_head_kernel<QT>, dim3(grid_for_waves((V + 1) / 2)), dim3(kThreads), D * sizeof(float), logits,
                m->x, m->ln_f, eps, W, rb, V, D);
    });
  }
  return FG_OK;
}

extern "C" int fg_decode_part_len(int nHeads, int dHead, int maxSeq, int64_t* doubles) {
  FG_ARG_CHECK(nHeads > 0 && dHead > 0 && maxSeq > 0 && doubles, "fg_decode_part_len: bad arguments");
  *doubles = (int64_t)nHeads * ((maxSeq + kChunk - 1) / kChunk) * (dHead + 2);
  return FG_OK;
}
