/*
 * vector_oracle.c — CPU restatement of forge-llm's vector-level autograd ops
 * (src/L2/autograd.js:70-190), its single-query-row attention helpers
 * (src/L5/attention.js:31-126, softmax from src/L1/special.js:66-74) and
 * rmsnormInto (src/L4/nn.js:42-44 → special.js:46-50, numeric.js:74-78).
 *
 * TEST INFRASTRUCTURE ONLY (see forge_oracle.c): the parity reference of the
 * device entry points fg_vec_*, fg_row_attention and fg_row_rmsnorm.
 *
 * JS numbers are fp64 and Float32Array stores round to fp32: every
 * expression below is evaluated in double in the reference's order (built
 * with -ffp-contract=off) and every array store goes through a float.  A
 * gradient `g[i] += t` is g[i] = (float)((double)g[i] + t); `grad ??= zeros`
 * is a zero-initialised output (the caller passes zeros for a fresh grad).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

/* mul — autograd.js:70-79 (nb == 1 broadcasts b[0]) */
void or_vec_mul_fwd(float* out, const float* a, const float* b, int64_t n, int64_t nb) {
  for (int64_t i = 0; i < n; i++) out[i] = (float)((double)a[i] * (double)b[nb == 1 ? 0 : i]);
}
void or_vec_mul_bwd(float* ga, float* gb, const float* g, const float* a, const float* b, int64_t n, int64_t nb) {
  for (int64_t i = 0; i < n; i++) ga[i] = (float)((double)ga[i] + (double)g[i] * (double)b[nb == 1 ? 0 : i]);
  if (nb > 1) {
    for (int64_t i = 0; i < n; i++) gb[i] = (float)((double)gb[i] + (double)g[i] * (double)a[i]);
  } else {
    for (int64_t i = 0; i < n; i++) gb[0] = (float)((double)gb[0] + (double)g[i] * (double)a[i]);
  }
}

/* silu — autograd.js:81-89 */
void or_vec_silu_fwd(float* out, float* s, const float* x, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    s[i] = (float)(1.0 / (1.0 + exp(-(double)x[i])));
    out[i] = (float)((double)x[i] * (double)s[i]);
  }
}
void or_vec_silu_bwd(float* gx, const float* g, const float* x, const float* s, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    const double si = s[i], xi = x[i];
    gx[i] = (float)((double)gx[i] + (double)g[i] * (si + xi * si * (1.0 - si)));
  }
}

/* dot — autograd.js:136-146 */
void or_vec_dot_fwd(float* out, const float* a, const float* b, int64_t n) {
  double s = 0.0;
  for (int64_t i = 0; i < n; i++) s += (double)a[i] * (double)b[i];
  out[0] = (float)s;
}
void or_vec_dot_bwd(float* ga, float* gb, const float* g, const float* a, const float* b, int64_t n) {
  const double k = g[0];
  for (int64_t i = 0; i < n; i++) {
    ga[i] = (float)((double)ga[i] + k * (double)b[i]);
    gb[i] = (float)((double)gb[i] + k * (double)a[i]);
  }
}

/* scale — autograd.js:148-153 */
void or_vec_scale_fwd(float* out, const float* x, double s, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = (float)(s * (double)x[i]);
}
void or_vec_scale_bwd(float* gx, const float* g, double s, int64_t n) {
  for (int64_t i = 0; i < n; i++) gx[i] = (float)((double)gx[i] + (double)g[i] * s);
}

/* ropeNode — autograd.js:156-172 (out is a fresh zero array of n) */
void or_vec_rope_fwd(float* out, const float* x, const double* c, const double* sn, int64_t n, int dH) {
  for (int64_t i = 0; i < n; i++) out[i] = 0.f;
  for (int i = 0; i < dH; i += 2) {
    const double a = x[i], b = x[i + 1];
    out[i] = (float)(a * c[i >> 1] - b * sn[i >> 1]);
    out[i + 1] = (float)(a * sn[i >> 1] + b * c[i >> 1]);
  }
}
void or_vec_rope_bwd(float* gx, const float* g, const double* c, const double* sn, int dH) {
  for (int i = 0; i < dH; i += 2) {
    const double ci = c[i >> 1], si = sn[i >> 1];
    gx[i] = (float)((double)gx[i] + ((double)g[i] * ci + (double)g[i + 1] * si));
    gx[i + 1] = (float)((double)gx[i + 1] + (-(double)g[i] * si + (double)g[i + 1] * ci));
  }
}

/* softmaxVec — autograd.js:174-190 (p is the saved probability vector) */
void or_vec_softmax_fwd(float* out, float* p, const float* x, int64_t n) {
  double m = -INFINITY;
  for (int64_t i = 0; i < n; i++)
    if ((double)x[i] > m) m = x[i];
  double s = 0.0;
  for (int64_t i = 0; i < n; i++) {
    p[i] = (float)exp((double)x[i] - m);
    s += (double)p[i];
  }
  for (int64_t i = 0; i < n; i++) p[i] = (float)((double)p[i] / s);
  for (int64_t i = 0; i < n; i++) out[i] = p[i];
}
void or_vec_softmax_bwd(float* gx, const float* g, const float* p, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    double acc = 0.0;
    for (int64_t j = 0; j < n; j++) acc += (double)g[j] * ((double)p[i] * ((i == j ? 1.0 : 0.0) - (double)p[j]));
    gx[i] = (float)((double)gx[i] + acc);
  }
}

/* softmax in place over fp32 storage — special.js:66-74 */
static void sp_softmax(float* x, int n) {
  double m = -INFINITY;
  for (int i = 0; i < n; i++)
    if ((double)x[i] > m) m = x[i];
  double s = 0.0;
  for (int i = 0; i < n; i++) {
    const double e = exp((double)x[i] - m);
    x[i] = (float)e;
    s += e;
  }
  const double inv = 1.0 / s;
  for (int i = 0; i < n; i++) x[i] = (float)((double)x[i] * inv);
}

static double qk(const float* q, const float* kr, int d) {
  double acc = 0.0;
  for (int i = 0; i < d; i++) acc += (double)q[i] * (double)kr[i];
  return acc;
}

/* attentionDecode — attention.js:31-57 (sc: n floats of scratch, left with the scores) */
void or_attention_decode(float* out, const float* q, const float* K, const float* V, int n, int d, double scale,
                         int causal, int qOff, float* sc) {
  double mx = -INFINITY;
  for (int j = 0; j < n; j++) {
    if (causal && j > qOff) {
      sc[j] = -INFINITY;
      continue;
    }
    const double v = qk(q, K + (size_t)j * d, d) * scale;
    sc[j] = (float)v;
    if (v > mx) mx = v;
  }
  for (int i = 0; i < d; i++) out[i] = 0.f;
  double l = 0.0;
  for (int j = 0; j < n; j++) {
    const double p = sc[j] == -INFINITY ? 0.0 : exp((double)sc[j] - mx);
    if (p == 0.0) continue;
    l += p;
    for (int i = 0; i < d; i++) out[i] = (float)((double)out[i] + p * (double)V[(size_t)j * d + i]);
  }
  const double inv = 1.0 / (l != 0.0 ? l : 1.0);
  for (int i = 0; i < d; i++) out[i] = (float)((double)out[i] * inv);
}

/* attentionNaive — attention.js:63-79 */
void or_attention_naive(float* out, const float* q, const float* K, const float* V, int n, int d, double scale,
                        int causal, int qOff) {
  float* s = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  for (int j = 0; j < n; j++) {
    if (causal && j > qOff) {
      s[j] = -INFINITY;
      continue;
    }
    s[j] = (float)(qk(q, K + (size_t)j * d, d) * scale);
  }
  sp_softmax(s, n);
  for (int i = 0; i < d; i++) out[i] = 0.f;
  for (int j = 0; j < n; j++) {
    const double p = s[j];
    if (p == 0.0) continue;
    for (int i = 0; i < d; i++) out[i] = (float)((double)out[i] + p * (double)V[(size_t)j * d + i]);
  }
  free(s);
}

/* flashAttention — attention.js:89-126 */
void or_flash_attention(float* out, const float* q, const float* K, const float* V, int n, int d, double scale,
                        int causal, int qOff, int block) {
  const int end = causal ? (n < qOff + 1 ? n : qOff + 1) : n;
  for (int i = 0; i < d; i++) out[i] = 0.f;
  if (end <= 0) return;
  float* s = (float*)malloc(sizeof(float) * (size_t)block);
  double m = -INFINITY, l = 0.0;
  for (int b = 0; b < end; b += block) {
    const int e = b + block < end ? b + block : end;
    double mb = -INFINITY;
    for (int j = b; j < e; j++) {
      const double v = qk(q, K + (size_t)j * d, d) * scale;
      s[j - b] = (float)v;
      if (v > mb) mb = v;
    }
    const double mNew = m > mb ? m : mb;
    const double alpha = m == -INFINITY ? 0.0 : exp(m - mNew);
    double lNew = l * alpha;
    if (alpha != 1.0)
      for (int i = 0; i < d; i++) out[i] = (float)((double)out[i] * alpha);
    for (int j = b; j < e; j++) {
      const double p = exp((double)s[j - b] - mNew);
      lNew += p;
      for (int i = 0; i < d; i++) out[i] = (float)((double)out[i] + p * (double)V[(size_t)j * d + i]);
    }
    m = mNew;
    l = lNew;
  }
  const double inv = 1.0 / (l != 0.0 ? l : 1.0);
  for (int i = 0; i < d; i++) out[i] = (float)((double)out[i] * inv);
  free(s);
}

/* rmsnormInto — nn.js:42-44 → special.js:46-50 with rms from numeric.js:74-78 */
void or_row_rmsnorm(float* out, const float* x, const float* w, int n, double eps) {
  double s = 0.0;
  for (int i = 0; i < n; i++) {
    const double v = x[i];
    s += v * v;
  }
  const double r = sqrt(s / n);
  const double ss = 1.0 / sqrt(r * r + eps);
  for (int i = 0; i < n; i++) out[i] = (float)((double)x[i] * ss * (double)w[i]);
}
