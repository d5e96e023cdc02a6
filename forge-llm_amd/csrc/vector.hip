// Vector-level autograd ops, single-query-row attention and the one-row
// RMSNorm helper on the device.
//
// forge-llm's autograd module also exports element-wise vector ops (mul,
// silu, dot, scale, ropeNode, softmaxVec: autograd.js:70-190) and its
// attention module three single-row attention helpers over host arrays
// (attentionDecode, attentionNaive, flashAttention: attention.js:31-126), and
// its nn module a one-row RMSNorm over host arrays (rmsnormInto, nn.js:42-44).
// None of them is on the training step, so they are written for exact
// agreement with the reference's arithmetic rather than for bandwidth: fp32
// operands are widened to fp64, every JS number expression is evaluated in
// fp64 in the reference's order (contraction off), a Float32Array store
// rounds once, and `g[i] += term` is fp32(g_old + term) in fp64.  Reductions
// that the reference runs as one sequential fp64 (or fp32) sum run
// sequentially here too, so the results equal the reference's bit for bit
// up to the last-ulp differences of fp64 exp between libraries.
#include "common.h"

namespace {

constexpr int kThreads = 256;

int64_t grid_for(int64_t n) {
  int64_t g = (n + kThreads - 1) / kThreads;
  const int64_t cap = (int64_t)(fg::device_cu_count() > 0 ? fg::device_cu_count() : 256) * 16;
  if (g > cap) g = cap;
  return g < 1 ? 1 : g;
}

// fp32(old + term) when the gradient already holds a value (beta), else fp32(term).
__device__ __forceinline__ float acc_store(float old, int beta, double term) {
  return (float)((beta ? (double)old : 0.0) + term);
}

// ── mul (autograd.js:70-79): out = a * b, b of length n or 1 ──────────────
__global__ void __launch_bounds__(kThreads) mul_fwd_kernel(float* __restrict__ out, const float* __restrict__ a,
                                                           const float* __restrict__ b, int64_t n, int bscalar) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    out[i] = (float)((double)a[i] * (double)b[bscalar ? 0 : i]);
}

// ga (+)= g * b; gb (+)= g * a (elementwise b).  ga and gb are one buffer
// for mul(x, x): each element then takes both updates in the reference's
// order (no __restrict__ on them).
__global__ void __launch_bounds__(kThreads) mul_bwd_kernel(float* ga, int beta_a, float* gb,
                                                           int beta_b, const float* __restrict__ g,
                                                           const float* __restrict__ a, const float* __restrict__ b,
                                                           int64_t n, int bscalar) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    ga[i] = acc_store(ga[i], beta_a, (double)g[i] * (double)b[bscalar ? 0 : i]);
    if (!bscalar) gb[i] = acc_store(gb[i], beta_b, (double)g[i] * (double)a[i]);
  }
}

// A scalar b's gradient: gb[0] += g[i] * a[i] for i = 0..n-1, each `+=` an
// fp32 store (the reference's running Float32Array sum), one thread.
__global__ void __launch_bounds__(64) mul_bwd_scalar_kernel(float* __restrict__ gb, int beta_b,
                                                            const float* __restrict__ g,
                                                            const float* __restrict__ a, int64_t n) {
#pragma clang fp contract(off)
  if (threadIdx.x != 0) return;
  float s = beta_b ? gb[0] : 0.f;
  for (int64_t i = 0; i < n; ++i) s = (float)((double)s + (double)g[i] * (double)a[i]);
  gb[0] = s;
}

// ── silu (autograd.js:81-89) ────────────────────────────────────────────
// sig = fp32(1 / (1 + exp(-x))), out = fp32(x * sig) with the stored sig.
__global__ void __launch_bounds__(kThreads) silu_fwd_kernel(float* __restrict__ out, float* __restrict__ sig,
                                                            const float* __restrict__ x, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const double xv = x[i];
    const float s = (float)(1.0 / (1.0 + exp(-xv)));
    sig[i] = s;
    out[i] = (float)(xv * (double)s);
  }
}

// gx (+)= g * (s + x * s * (1 - s))
__global__ void __launch_bounds__(kThreads) silu_bwd_kernel(float* __restrict__ gx, int beta,
                                                            const float* __restrict__ g,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ sig, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const double s = sig[i], xv = x[i];
    const double t = (double)g[i] * (s + xv * s * (1.0 - s));
    gx[i] = acc_store(gx[i], beta, t);
  }
}

// ── dot (autograd.js:136-146): one sequential fp64 sum, fp32 result ──────
__global__ void __launch_bounds__(64) dot_fwd_kernel(float* __restrict__ out, const float* __restrict__ a,
                                                     const float* __restrict__ b, int64_t n) {
#pragma clang fp contract(off)
  if (threadIdx.x != 0) return;
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)a[i] * (double)b[i];
  out[0] = (float)s;
}

// ga (+)= k * b, gb (+)= k * a with k = g[0] (ga and gb one buffer for dot(x, x))
__global__ void __launch_bounds__(kThreads) dot_bwd_kernel(float* ga, int beta_a, float* gb,
                                                           int beta_b, const float* __restrict__ g,
                                                           const float* __restrict__ a, const float* __restrict__ b,
                                                           int64_t n) {
#pragma clang fp contract(off)
  const double k = g[0];
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    ga[i] = acc_store(ga[i], beta_a, k * (double)b[i]);
    gb[i] = acc_store(gb[i], beta_b, k * (double)a[i]);
  }
}

// ── scale (autograd.js:148-153): out = s * x, s an fp64 scalar ───────────
__global__ void __launch_bounds__(kThreads) scale_fwd_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                             double s, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    out[i] = (float)(s * (double)x[i]);
}

__global__ void __launch_bounds__(kThreads) scale_bwd_kernel(float* __restrict__ gx, int beta,
                                                             const float* __restrict__ g, double s, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    gx[i] = acc_store(gx[i], beta, (double)g[i] * s);
}

// ── ropeNode (autograd.js:156-172) ─────────────────────────────────────────
// Pairs (i, i+1), i = 0, 2, .. < dH, turned by (cos[i/2], sin[i/2]) (fp64
// tables); the other outputs are zero.  One thread per output element.
__global__ void __launch_bounds__(kThreads) rope_fwd_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                            const double* __restrict__ c,
                                                            const double* __restrict__ s, int64_t n, int dH) {
#pragma clang fp contract(off)
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kThreads) {
    const int64_t i = e & ~(int64_t)1;
    if (i >= dH) {
      out[e] = 0.f;
      continue;
    }
    const double a = x[i], b = x[i + 1], cc = c[i >> 1], ss = s[i >> 1];
    out[e] = (e == i) ? (float)(a * cc - b * ss) : (float)(a * ss + b * cc);
  }
}

// gx[i] += g[i] c + g[i+1] s; gx[i+1] += -g[i] s + g[i+1] c (pairs below dH;
// a fresh gradient is zero elsewhere)
__global__ void __launch_bounds__(kThreads) rope_bwd_kernel(float* __restrict__ gx, int beta,
                                                            const float* __restrict__ g,
                                                            const double* __restrict__ c,
                                                            const double* __restrict__ s, int64_t n, int dH) {
#pragma clang fp contract(off)
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kThreads) {
    const int64_t i = e & ~(int64_t)1;
    if (i >= dH) {
      if (!beta) gx[e] = 0.f;
      continue;
    }
    const double g0 = g[i], g1 = g[i + 1], cc = c[i >> 1], ss = s[i >> 1];
    const double t = (e == i) ? g0 * cc + g1 * ss : -g0 * ss + g1 * cc;
    gx[e] = acc_store(gx[e], beta, t);
  }
}

// ── softmaxVec (autograd.js:174-190) ──────────────────────────────────────
// One thread: m = max, p_i = fp32(exp(x_i - m)), S = sum of the stored p_i in
// fp64 (in order), then p_i = fp32(p_i / S); out = p and the saved copy.
__global__ void __launch_bounds__(64) softmax_fwd_kernel(float* __restrict__ out, float* __restrict__ p,
                                                         const float* __restrict__ x, int64_t n) {
#pragma clang fp contract(off)
  if (threadIdx.x != 0) return;
  float m = -INFINITY;
  for (int64_t i = 0; i < n; ++i)
    if (x[i] > m) m = x[i];
  double S = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const float e = (float)exp((double)x[i] - (double)m);
    p[i] = e;
    S += (double)e;
  }
  for (int64_t i = 0; i < n; ++i) {
    const float v = (float)((double)p[i] / S);
    p[i] = v;
    out[i] = v;
  }
}

// gx_i (+)= sum_j g_j (p_i ((i == j) - p_j)), summed over j in order in fp64:
// one thread per i, (g, p) streamed through LDS in chunks.
constexpr int kSmChunk = 1024;
__global__ void __launch_bounds__(kThreads) softmax_bwd_kernel(float* __restrict__ gx, int beta,
                                                               const float* __restrict__ g,
                                                               const float* __restrict__ p, int64_t n) {
#pragma clang fp contract(off)
  __shared__ float gs[kSmChunk], ps[kSmChunk];
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const double pi = i < n ? (double)p[i] : 0.0;
  double acc = 0.0;
  for (int64_t j0 = 0; j0 < n; j0 += kSmChunk) {
    const int len = (int)min((int64_t)kSmChunk, n - j0);
    __syncthreads();
    for (int u = threadIdx.x; u < len; u += kThreads) {
      gs[u] = g[j0 + u];
      ps[u] = p[j0 + u];
    }
    __syncthreads();
    if (i < n)
      for (int u = 0; u < len; ++u) {
        const double d = (j0 + u == i) ? 1.0 : 0.0;
        acc += (double)gs[u] * (pi * (d - (double)ps[u]));
      }
  }
  if (i < n) gx[i] = acc_store(gx[i], beta, acc);
}

// Long vectors (n > kSmExactMax): the same Jacobian product in its O(n)
// form, gx_i (+)= p_i (g_i - c) with c = sum_j g_j p_j (in order, fp64, one
// thread); it equals the O(n^2) sum up to fp64 rounding, so the fp32 results
// differ from it only where a value sits on an fp32 rounding tie.
constexpr int64_t kSmExactMax = 1 << 16;
__global__ void __launch_bounds__(64) softmax_dot_kernel(double* __restrict__ c, const float* __restrict__ g,
                                                         const float* __restrict__ p, int64_t n) {
#pragma clang fp contract(off)
  if (threadIdx.x != 0) return;
  double s = 0.0;
  for (int64_t j = 0; j < n; ++j) s += (double)g[j] * (double)p[j];
  c[0] = s;
}
__global__ void __launch_bounds__(kThreads) softmax_bwd_long_kernel(float* __restrict__ gx, int beta,
                                                                    const float* __restrict__ g,
                                                                    const float* __restrict__ p,
                                                                    const double* __restrict__ c, int64_t n) {
#pragma clang fp contract(off)
  const double cc = c[0];
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    gx[i] = acc_store(gx[i], beta, (double)p[i] * ((double)g[i] - cc));
}

// ── single-query-row attention (attention.js:31-126) ─────────────────────
// out[0..d) = sum_j softmax_j(scale q·K_j) V_j over keys j < n (rows of d
// floats), keys after qOff masked when causal.  One workgroup: scores in
// parallel (each an in-order fp64 dot), the softmax constants by thread 0 in
// key order, then one thread per output column accumulating over keys in
// order with an fp32 store per step, as each reference variant does:
//   mode 0  attentionDecode: two passes, p = exp(score - max), 1/l at the end;
//   mode 1  attentionNaive:  softmax of the fp32 scores, then the sum of p V;
//   mode 2  flashAttention:  blocks of `block` keys with the online rescale.
// Scratch: v (fp64 scores), sf (fp32 scores), p (fp64 weights), and per block
// alpha (fp64).
__global__ void __launch_bounds__(kThreads) row_attn_kernel(float* __restrict__ out, const float* __restrict__ q,
                                                            const float* __restrict__ K,
                                                            const float* __restrict__ V, int n, int d, double scale,
                                                            int causal, int qOff, int mode, int block,
                                                            double* __restrict__ v, float* __restrict__ sf,
                                                            double* __restrict__ p, double* __restrict__ alpha,
                                                            float* __restrict__ scores) {
#pragma clang fp contract(off)
  __shared__ double sh_l;
  const int end = mode == 2 ? (causal ? min(n, qOff + 1) : n) : n;
  // scores
  for (int j = threadIdx.x; j < end; j += kThreads) {
    if (mode != 2 && causal && j > qOff) {
      v[j] = -INFINITY;
      sf[j] = -INFINITY;
      continue;
    }
    const float* kr = K + (size_t)j * d;
    double acc = 0.0;
    for (int i = 0; i < d; ++i) acc += (double)q[i] * (double)kr[i];
    const double vj = acc * scale;
    v[j] = vj;
    sf[j] = (float)vj;
  }
  __syncthreads();
  if (scores && mode == 0)  // attentionDecode's optional score buffer
    for (int j = threadIdx.x; j < n; j += kThreads) scores[j] = sf[j];
  if (threadIdx.x == 0) {
    if (mode == 0) {
      double mx = -INFINITY;
      for (int j = 0; j < n; ++j)
        if (!(causal && j > qOff) && v[j] > mx) mx = v[j];
      double l = 0.0;
      for (int j = 0; j < n; ++j) {
        const double pj = sf[j] == -INFINITY ? 0.0 : exp((double)sf[j] - mx);
        p[j] = pj;
        if (pj != 0.0) l += pj;
      }
      sh_l = l;
    } else if (mode == 1) {
      float m = -INFINITY;
      for (int j = 0; j < n; ++j)
        if (sf[j] > m) m = sf[j];
      double S = 0.0;
      for (int j = 0; j < n; ++j) {
        const double e = exp((double)sf[j] - (double)m);
        sf[j] = (float)e;
        S += e;
      }
      const double inv = 1.0 / S;
      for (int j = 0; j < n; ++j) p[j] = (double)(float)((double)sf[j] * inv);
      sh_l = 1.0;
    } else {
      double m = -INFINITY, l = 0.0;
      for (int b = 0, bi = 0; b < end; b += block, ++bi) {
        const int e = min(b + block, end);
        double mb = -INFINITY;
        for (int j = b; j < e; ++j)
          if (v[j] > mb) mb = v[j];
        const double mNew = fmax(m, mb);
        const double al = m == -INFINITY ? 0.0 : exp(m - mNew);
        alpha[bi] = al;
        double lNew = l * al;
        for (int j = b; j < e; ++j) {
          const double pj = exp((double)sf[j] - mNew);
          p[j] = pj;
          lNew += pj;
        }
        m = mNew;
        l = lNew;
      }
      sh_l = l;
    }
  }
  __syncthreads();
  const double l = sh_l;
  for (int i = threadIdx.x; i < d; i += kThreads) {
    float o = 0.f;
    if (mode == 2) {
      for (int b = 0, bi = 0; b < end; b += block, ++bi) {
        const double al = alpha[bi];
        if (al != 1.0) o = (float)((double)o * al);
        const int e = min(b + block, end);
        for (int j = b; j < e; ++j) o = (float)((double)o + p[j] * (double)V[(size_t)j * d + i]);
      }
    } else {
      for (int j = 0; j < n; ++j) {
        const double pj = p[j];
        if (pj == 0.0) continue;
        o = (float)((double)o + pj * (double)V[(size_t)j * d + i]);
      }
    }
    if (mode != 1) {
      const double inv = 1.0 / (l != 0.0 ? l : 1.0);
      o = (float)((double)o * inv);
    }
    out[i] = o;
  }
}

// ── rmsnormInto (nn.js:42-44 → special.js:46-50, numeric.js:74-78) ────────
// rms = sqrt(S / n) with S the in-order fp64 sum of x_i^2, ss = 1 / sqrt(rms^2
// + eps), out_i = fp32(x_i ss w_i).  S by thread 0, the outputs in parallel.
__global__ void __launch_bounds__(kThreads) row_rmsnorm_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                               const float* __restrict__ w, int n, double eps) {
#pragma clang fp contract(off)
  __shared__ double sh_ss;
  if (threadIdx.x == 0) {
    double S = 0.0;
    for (int i = 0; i < n; ++i) {
      const double v = x[i];
      S += v * v;
    }
    const double r = sqrt(S / (double)n);
    sh_ss = 1.0 / sqrt(r * r + eps);
  }
  __syncthreads();
  const double ss = sh_ss;
  for (int i = threadIdx.x; i < n; i += kThreads) out[i] = (float)((double)x[i] * ss * (double)w[i]);
}

}  // namespace

extern "C" int fg_vec_mul_fwd(float* out, const float* a, const float* b, int64_t n, int64_t nb) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && (nb == 1 || nb == n) && out && a && b, "fg_vec_mul_fwd: bad arguments (n=%lld nb=%lld)",
               (long long)n, (long long)nb);
  if (n == 0) return FG_OK;
  FG_LAUNCH(mul_fwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, out, a, b, n, (int)(nb == 1 && n != 1));
  return FG_OK;
}

extern "C" int fg_vec_mul_bwd(float* ga, int beta_a, float* gb, int beta_b, const float* g, const float* a,
                              const float* b, int64_t n, int64_t nb) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && (nb == 1 || nb == n) && ga && gb && g && a && b,
               "fg_vec_mul_bwd: bad arguments (n=%lld nb=%lld)", (long long)n, (long long)nb);
  if (n == 0) {
    // an empty a against a one-element b: gb is the empty sum, 0 (a fresh
    // gradient is still written)
    if (nb == 1 && !beta_b) FG_LAUNCH(mul_bwd_scalar_kernel, dim3(1), dim3(64), 0, gb, 0, g, a, (int64_t)0);
    return FG_OK;
  }
  const int bscalar = nb == 1 && n != 1;
  FG_LAUNCH(mul_bwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, ga, beta_a, gb, beta_b, g, a, b, n,
            bscalar);
  if (bscalar) FG_LAUNCH(mul_bwd_scalar_kernel, dim3(1), dim3(64), 0, gb, beta_b, g, a, n);
  return FG_OK;
}

extern "C" int fg_vec_silu_fwd(float* out, float* sig, const float* x, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && out && sig && x, "fg_vec_silu_fwd: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(silu_fwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, out, sig, x, n);
  return FG_OK;
}

extern "C" int fg_vec_silu_bwd(float* gx, int beta, const float* g, const float* x, const float* sig, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && gx && g && x && sig, "fg_vec_silu_bwd: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(silu_bwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, gx, beta, g, x, sig, n);
  return FG_OK;
}

extern "C" int fg_vec_dot_fwd(float* out, const float* a, const float* b, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && out && a && b, "fg_vec_dot_fwd: bad arguments");
  FG_LAUNCH(dot_fwd_kernel, dim3(1), dim3(64), 0, out, a, b, n);
  return FG_OK;
}

extern "C" int fg_vec_dot_bwd(float* ga, int beta_a, float* gb, int beta_b, const float* g, const float* a,
                              const float* b, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && ga && gb && g && a && b, "fg_vec_dot_bwd: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(dot_bwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, ga, beta_a, gb, beta_b, g, a, b, n);
  return FG_OK;
}

extern "C" int fg_vec_scale_fwd(float* out, const float* x, double s, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && out && x, "fg_vec_scale_fwd: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(scale_fwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, out, x, s, n);
  return FG_OK;
}

extern "C" int fg_vec_scale_bwd(float* gx, int beta, const float* g, double s, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && gx && g, "fg_vec_scale_bwd: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(scale_bwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, gx, beta, g, s, n);
  return FG_OK;
}

extern "C" int fg_vec_rope_fwd(float* out, const float* x, const double* cos_t, const double* sin_t, int64_t n,
                               int dH) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && dH >= 0 && (int64_t)((dH + 1) & ~1) <= n && out && x && (dH == 0 || (cos_t && sin_t)),
               "fg_vec_rope_fwd: bad arguments (n=%lld dHead=%d: the pairs below dHead must lie inside the vector)",
               (long long)n, dH);
  if (n == 0) return FG_OK;
  FG_LAUNCH(rope_fwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, out, x, cos_t, sin_t, n, dH);
  return FG_OK;
}

extern "C" int fg_vec_rope_bwd(float* gx, int beta, const float* g, const double* cos_t, const double* sin_t,
                               int64_t n, int dH) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && dH >= 0 && (int64_t)((dH + 1) & ~1) <= n && gx && g && (dH == 0 || (cos_t && sin_t)),
               "fg_vec_rope_bwd: bad arguments (n=%lld dHead=%d)", (long long)n, dH);
  if (n == 0) return FG_OK;
  FG_LAUNCH(rope_bwd_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, gx, beta, g, cos_t, sin_t, n, dH);
  return FG_OK;
}

extern "C" int fg_vec_softmax_fwd(float* out, float* p, const float* x, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && out && p && x, "fg_vec_softmax_fwd: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(softmax_fwd_kernel, dim3(1), dim3(64), 0, out, p, x, n);
  return FG_OK;
}

extern "C" int fg_vec_softmax_bwd(float* gx, int beta, const float* g, const float* p, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && gx && g && p, "fg_vec_softmax_bwd: bad arguments");
  if (n == 0) return FG_OK;
  if (n > kSmExactMax) {
    fg::Workspace ws;
    int rc = ws.get(sizeof(double));
    if (rc) return rc;
    FG_LAUNCH(softmax_dot_kernel, dim3(1), dim3(64), 0, (double*)ws.ptr, g, p, n);
    FG_LAUNCH(softmax_bwd_long_kernel, dim3((unsigned)grid_for(n)), dim3(kThreads), 0, gx, beta, g, p,
              (const double*)ws.ptr, n);
    return FG_OK;
  }
  const int64_t blocks = (n + kThreads - 1) / kThreads;
  FG_LAUNCH(softmax_bwd_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, gx, beta, g, p, n);
  return FG_OK;
}

extern "C" int fg_row_attention(float* out, const float* q, const float* K, const float* V, int n, int d,
                                double scale, int causal, int qOff, int mode, int block, float* scores) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n >= 0 && d > 0 && out && q && (n == 0 || (K && V)) && mode >= 0 && mode <= 2 &&
                   (mode != 2 || block > 0),
               "fg_row_attention: bad arguments (n=%d d=%d mode=%d block=%d)", n, d, mode, block);
  const int nb = mode == 2 ? (n + block - 1) / block : 1;
  fg::Workspace ws;
  const size_t nn = (size_t)(n > 0 ? n : 1);
  int rc = ws.get(nn * (sizeof(double) * 2 + sizeof(float)) + sizeof(double) * (size_t)(nb > 0 ? nb : 1) + 64);
  if (rc) return rc;
  double* v = (double*)ws.ptr;
  double* p = v + nn;
  double* alpha = p + nn;
  float* sf = (float*)(alpha + (nb > 0 ? nb : 1));
  FG_LAUNCH(row_attn_kernel, dim3(1), dim3(kThreads), 0, out, q, K, V, n, d, scale, causal, qOff, mode, block, v, sf,
            p, alpha, scores);
  return FG_OK;
}

extern "C" int fg_row_rmsnorm(float* out, const float* x, const float* w, int n, double eps) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(n > 0 && out && x && w, "fg_row_rmsnorm: bad arguments (n=%d)", n);
  FG_LAUNCH(row_rmsnorm_kernel, dim3(1), dim3(kThreads), 0, out, x, w, n, eps);
  return FG_OK;
}
