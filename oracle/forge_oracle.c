/*
 * forge_oracle.c — CPU restatement of forge-llm's fused training path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the parity reference or the timed CPU baseline.  The product path
 * (forge-llm_amd/) never links, loads or falls back to it.
 *
 * Semantics follow the reference JavaScript exactly where it matters for
 * parity: arithmetic in fp64 (JS numbers), storage in fp32 (Float32Array), so
 * every store — including every `+=` into a gradient — rounds to fp32; loop
 * orders and reduction orders are the reference's.  Build with
 * -ffp-contract=off (JS never fuses a multiply-add).
 *
 * Each function cites the reference file:line it restates.  How each one is
 * pinned (golden vectors, closed forms, finite differences, known answers)
 * is recorded in oracle/README.md.
 *
 * Threads: the large loops run under OpenMP, split only over indices whose
 * outputs are independent (GEMM rows, gradient rows or columns, attention
 * heads, CE rows).  Every output element still sees exactly the reference's
 * sequence of operations in the reference's order, so results do not depend
 * on the thread count (tests/test_oracle.py checks 1 thread against many).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define F32(x) ((float)(x))

/* ───────────── RNG: splitmix32-seeded xorshift128+ (numeric.js:27-49) ───────────── */
typedef struct {
  uint32_t s0, s1;
} or_rng;

static uint32_t splitmix32_next(uint32_t* s) {
  *s = *s + 0x9e3779b9u;
  uint32_t z = *s;
  z = (z ^ (z >> 16)) * 0x21f0aaadu;
  z = (z ^ (z >> 15)) * 0x735a2d97u;
  return z ^ (z >> 15);
}

void or_rng_init(or_rng* r, uint32_t seed) {
  uint32_t s = seed ? seed : 1u; /* `seed >>> 0 || 1` */
  r->s0 = splitmix32_next(&s);
  r->s1 = splitmix32_next(&s);
}

double or_rng_next(or_rng* r) {
  uint32_t x = r->s0, y = r->s1;
  r->s0 = y;
  x ^= x << 23;
  x ^= x >> 17;
  x ^= y;
  x ^= y >> 26;
  r->s1 = x;
  return (double)(uint32_t)(r->s1 + y) / 4294967296.0;
}

double or_rng_normal(or_rng* r) {
  double u = or_rng_next(r);
  if (u < 1e-12) u = 1e-12;
  double v = or_rng_next(r);
  return sqrt(-2.0 * log(u)) * cos(2.0 * M_PI * v);
}

int or_rng_int(or_rng* r, int n) { return (int)floor(or_rng_next(r) * n); }

/* Convenience for callers: a heap RNG handle and bulk draws. */
or_rng* or_rng_new(uint32_t seed) {
  or_rng* r = (or_rng*)malloc(sizeof(or_rng));
  or_rng_init(r, seed);
  return r;
}
void or_rng_free(or_rng* r) { free(r); }
/* a[i] = fp32(normal() * scale)  — the reference's randArr / initWeights norm(). */
void or_rng_fill_normal(or_rng* r, float* out, int64_t n, double scale) {
  for (int64_t i = 0; i < n; i++) out[i] = F32(or_rng_normal(r) * scale);
}
void or_rng_fill_next(or_rng* r, double* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = or_rng_next(r);
}
void or_rng_fill_int(or_rng* r, int32_t* out, int64_t n, int range) {
  for (int64_t i = 0; i < n; i++) out[i] = or_rng_int(r, range);
}

/* ───────────── matmulT (tensor.js:34-53; gemm numeric.js:111-130) ───────────── */
/* C[M,N] = A[M,K] · B[N,K]^T with four fp64 partial sums, rounded once. */
/* One output: the four partial sums over k (k mod 4), added once, then the
 * k tail (numeric.js:116-127). */
static inline float gemm_dot(const float* a, const float* b, int K) {
  double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  int k = 0;
  for (; k + 4 <= K; k += 4) {
    s0 += (double)a[k] * b[k];
    s1 += (double)a[k + 1] * b[k + 1];
    s2 += (double)a[k + 2] * b[k + 2];
    s3 += (double)a[k + 3] * b[k + 3];
  }
  double s = s0 + s1 + s2 + s3;
  for (; k < K; k++) s += (double)a[k] * b[k];
  return F32(s);
}

void or_gemm(float* C, const float* A, const float* B, int M, int N, int K) {
  /* Rows of C are independent: blocks of 8 rows share each row of B, and
   * four outputs of a row are formed together (each with its own four
   * partial sums in the order gemm_dot uses, so the same bits). */
#pragma omp parallel for schedule(dynamic, 1) if ((int64_t)M * N * K > (1 << 20))
  for (int m0 = 0; m0 < M; m0 += 8) {
    int m1 = m0 + 8 < M ? m0 + 8 : M;
    int n = 0;
    for (; n + 4 <= N; n += 4) {
      const float* b0 = B + (int64_t)n * K;
      const float *b1 = b0 + K, *b2 = b1 + K, *b3 = b2 + K;
      for (int m = m0; m < m1; m++) {
        const float* a = A + (int64_t)m * K;
        double s[4][4] = {{0}};
        int k = 0;
        for (; k + 4 <= K; k += 4) {
          for (int u = 0; u < 4; u++) {
            double x = a[k + u];
            s[0][u] += x * b0[k + u];
            s[1][u] += x * b1[k + u];
            s[2][u] += x * b2[k + u];
            s[3][u] += x * b3[k + u];
          }
        }
        const float* bs[4] = {b0, b1, b2, b3};
        for (int v = 0; v < 4; v++) {
          double t = s[v][0] + s[v][1] + s[v][2] + s[v][3];
          for (int kk = k; kk < K; kk++) t += (double)a[kk] * bs[v][kk];
          C[(int64_t)m * N + n + v] = F32(t);
        }
      }
    }
    for (; n < N; n++)
      for (int m = m0; m < m1; m++) C[(int64_t)m * N + n] = gemm_dot(A + (int64_t)m * K, B + (int64_t)n * K, K);
  }
}

/* Backward: gX[M,K] += g·W, gW[N,K] += g^T·X, one shared m,n,k loop with an
 * fp32 store per +=; rows of g equal to 0 are skipped (tensor.js:37-52).
 * Either gradient may be NULL. */
void or_matmulT_bwd_serial(float* gX, float* gW, const float* g, const float* X, const float* W, int M,
                           int K, int N) {
  for (int m = 0; m < M; m++) {
    int64_t xb = (int64_t)m * K, gb = (int64_t)m * N;
    for (int n = 0; n < N; n++) {
      double gn = g[gb + n];
      if (gn == 0.0) continue;
      int64_t wb = (int64_t)n * K;
      for (int k = 0; k < K; k++) {
        if (gX) gX[xb + k] = F32((double)gX[xb + k] + gn * W[wb + k]);
        if (gW) gW[wb + k] = F32((double)gW[wb + k] + gn * X[xb + k]);
      }
    }
  }
}

void or_matmulT_bwd(float* gX, float* gW, const float* g, const float* X, const float* W, int M, int K,
                    int N) {
  /* gX == gW (matmulT(X, X)): the two updates interleave on one buffer. */
  if ((gX && gX == gW) || (int64_t)M * N * K <= (1 << 20)) {
    or_matmulT_bwd_serial(gX, gW, g, X, W, M, K, N);
    return;
  }
  /* Otherwise gX[m,k] only depends on its own += sequence over n (in
   * increasing n) and gW[n,k] on its own over m (increasing m): the two are
   * run as separate loops, blocked so that a W or X row is reused from cache. */
  enum { BM = 8, BN = 8 };
  if (gX) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int m0 = 0; m0 < M; m0 += BM) {
      int m1 = m0 + BM < M ? m0 + BM : M;
      for (int n = 0; n < N; n++) {
        const float* w = W + (int64_t)n * K;
        for (int m = m0; m < m1; m++) {
          double gn = g[(int64_t)m * N + n];
          if (gn == 0.0) continue;
          float* gx = gX + (int64_t)m * K;
          for (int k = 0; k < K; k++) gx[k] = F32((double)gx[k] + gn * w[k]);
        }
      }
    }
  }
  if (gW) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int n0 = 0; n0 < N; n0 += BN) {
      int n1 = n0 + BN < N ? n0 + BN : N;
      for (int m = 0; m < M; m++) {
        const float* x = X + (int64_t)m * K;
        const float* gr = g + (int64_t)m * N;
        for (int n = n0; n < n1; n++) {
          double gn = gr[n];
          if (gn == 0.0) continue;
          float* gw = gW + (int64_t)n * K;
          for (int k = 0; k < K; k++) gw[k] = F32((double)gw[k] + gn * x[k]);
        }
      }
    }
  }
}

/* ───────────── embedLookup (tensor.js:85-99) ───────────── */
void or_embed_fwd(float* out, const float* W, const int32_t* ids, int T, int D) {
  for (int t = 0; t < T; t++)
    for (int d = 0; d < D; d++) out[(int64_t)t * D + d] = W[(int64_t)ids[t] * D + d];
}
void or_embed_bwd(float* gW, const float* g, const int32_t* ids, int T, int D) {
  for (int t = 0; t < T; t++) {
    int64_t o = (int64_t)ids[t] * D, go = (int64_t)t * D;
    for (int d = 0; d < D; d++) gW[o + d] = F32((double)gW[o + d] + g[go + d]);
  }
}

/* ───────────── rmsNorm (tensor.js:103-128) ───────────── */
void or_rmsnorm_fwd(float* out, float* inv, const float* X, const float* w, int T, int D, double eps) {
#pragma omp parallel for schedule(static) if ((int64_t)T * D > (1 << 16))
  for (int t = 0; t < T; t++) {
    int64_t xb = (int64_t)t * D;
    double ss = 0;
    for (int i = 0; i < D; i++) ss += (double)X[xb + i] * X[xb + i];
    double r = sqrt(ss / D + eps);
    inv[t] = F32(1.0 / r);
    for (int i = 0; i < D; i++) out[xb + i] = F32((double)X[xb + i] * inv[t] * w[i]);
  }
}
void or_rmsnorm_bwd(float* gX, float* gw, const float* g, const float* X, const float* w, const float* inv,
                    int T, int D) {
  /* gX rows are independent; gw[i] takes its += over t in increasing t */
#pragma omp parallel for schedule(static) if ((int64_t)T * D > (1 << 16))
  for (int t = 0; t < T; t++) {
    int64_t xb = (int64_t)t * D;
    double r = 1.0 / (double)inv[t];
    double dot = 0;
    for (int i = 0; i < D; i++) dot += (double)g[xb + i] * w[i] * X[xb + i];
    double c = dot / ((double)D * r * r * r);
    for (int i = 0; i < D; i++)
      gX[xb + i] = F32((double)gX[xb + i] + ((double)g[xb + i] * w[i] * inv[t] - c * X[xb + i]));
  }
  for (int t = 0; t < T; t++) {
    int64_t xb = (int64_t)t * D;
    for (int i = 0; i < D; i++) gw[i] = F32((double)gw[i] + (double)g[xb + i] * X[xb + i] * inv[t]);
  }
}

/* ───────────── ropeRows (tensor.js:133-166) ───────────── */
static int rope_pos(int t, int pos0, int posStride) { return pos0 + (posStride > 0 ? (t % posStride) : t); }

void or_rope_fwd(float* out, const float* X, int T, int nHead, int dHead, int pos0, double theta,
                 int posStride) {
  int D = nHead * dHead;
  memcpy(out, X, sizeof(float) * (size_t)T * D);
#pragma omp parallel for schedule(static) if ((int64_t)T * nHead * dHead > (1 << 16))
  for (int t = 0; t < T; t++) {
    double pos = rope_pos(t, pos0, posStride);
    int64_t xb = (int64_t)t * D;
    for (int h = 0; h < nHead; h++) {
      int64_t hb = xb + (int64_t)h * dHead;
      for (int i = 0; i < dHead; i += 2) {
        double freq = 1.0 / pow(theta, (double)i / dHead);
        double ang = pos * freq, c = cos(ang), s = sin(ang);
        double a = out[hb + i], b = out[hb + i + 1];
        out[hb + i] = F32(a * c - b * s);
        out[hb + i + 1] = F32(a * s + b * c);
      }
    }
  }
}
void or_rope_bwd(float* gX, const float* g, int T, int nHead, int dHead, int pos0, double theta, int posStride) {
  int D = nHead * dHead;
#pragma omp parallel for schedule(static) if ((int64_t)T * nHead * dHead > (1 << 16))
  for (int t = 0; t < T; t++) {
    double pos = rope_pos(t, pos0, posStride);
    int64_t xb = (int64_t)t * D;
    for (int h = 0; h < nHead; h++) {
      int64_t hb = xb + (int64_t)h * dHead;
      for (int i = 0; i < dHead; i += 2) {
        double freq = 1.0 / pow(theta, (double)i / dHead);
        double ang = pos * freq, c = cos(ang), s = sin(ang);
        double ga = g[hb + i], gb = g[hb + i + 1];
        gX[hb + i] = F32((double)gX[hb + i] + (ga * c + gb * s));
        gX[hb + i + 1] = F32((double)gX[hb + i + 1] + (-ga * s + gb * c));
      }
    }
  }
}
/* The fp64 angle table the GPU kernels consume (same expression as above). */
void or_rope_table(double* cos_tab, double* sin_tab, int npos, int dHead, double theta) {
  int half = dHead / 2;
  for (int p = 0; p < npos; p++)
    for (int i = 0; i < dHead; i += 2) {
      double freq = 1.0 / pow(theta, (double)i / dHead);
      double ang = (double)p * freq;
      cos_tab[(int64_t)p * half + i / 2] = cos(ang);
      sin_tab[(int64_t)p * half + i / 2] = sin(ang);
    }
}

/* ───────────── sliceCols (tensor.js:170-183) ───────────── */
void or_slice_fwd(float* out, const float* X, int M, int K, int off, int len) {
  for (int m = 0; m < M; m++)
    for (int i = 0; i < len; i++) out[(int64_t)m * len + i] = X[(int64_t)m * K + off + i];
}
void or_slice_bwd(float* gX, const float* g, int M, int K, int off, int len) {
  for (int m = 0; m < M; m++)
    for (int i = 0; i < len; i++) {
      int64_t xi = (int64_t)m * K + off + i;
      gX[xi] = F32((double)gX[xi] + g[(int64_t)m * len + i]);
    }
}

/* ───────────── causalAttn / causalAttnBatch (tensor.js:191-268, 299-376) ───────────── */
/* P[B*nH*T*T] receives the probabilities (zero above the diagonal).  With B=1
 * this is exactly causalAttn; with B>1 it is the block-diagonal batch form. */
void or_attn_fwd(float* out, float* P, const float* Q, const float* K, const float* V, int B, int T, int nH,
                 int nKV, int dH) {
  double scale = 1.0 / sqrt((double)dH);
  int group = nH / nKV > 1 ? nH / nKV : 1;
  int qD = nH * dH, kvD = nKV * dH;
  int64_t N = (int64_t)B * T;
  memset(out, 0, sizeof(float) * (size_t)(N * qD));
  memset(P, 0, sizeof(float) * (size_t)B * nH * T * T);
  /* every (b, h, t) row of O and P is independent */
#pragma omp parallel if ((int64_t)B * nH * T * T > (1 << 16))
  {
  float* s = (float*)malloc(sizeof(float) * (size_t)T);
#pragma omp for collapse(3) schedule(dynamic, 16)
  for (int b = 0; b < B; b++) {
    for (int h = 0; h < nH; h++) {
      for (int t = 0; t < T; t++) {
        int64_t base = (int64_t)b * T;
        int kvh = h / group;
        int64_t pb = ((int64_t)b * nH + h) * T * T;
        int64_t qb = (base + t) * qD + (int64_t)h * dH;
        double mx = -INFINITY;
        int j = 0;
        /* four keys at a time: four independent sums, each over d in order */
        for (; j + 4 <= t + 1; j += 4) {
          const float* k0 = K + (base + j) * kvD + (int64_t)kvh * dH;
          const float *k1 = k0 + kvD, *k2 = k1 + kvD, *k3 = k2 + kvD;
          double a[4] = {0, 0, 0, 0};
          for (int d = 0; d < dH; d++) {
            double q = Q[qb + d];
            a[0] += q * k0[d];
            a[1] += q * k1[d];
            a[2] += q * k2[d];
            a[3] += q * k3[d];
          }
          for (int u = 0; u < 4; u++) {
            double acc = a[u] * scale;
            s[j + u] = F32(acc);
            if (acc > mx) mx = acc;
          }
        }
        for (; j <= t; j++) {
          int64_t kb = (base + j) * kvD + (int64_t)kvh * dH;
          double acc = 0;
          for (int d = 0; d < dH; d++) acc += (double)Q[qb + d] * K[kb + d];
          acc *= scale;
          s[j] = F32(acc);
          if (acc > mx) mx = acc;
        }
        double sum = 0;
        for (int j = 0; j <= t; j++) {
          s[j] = F32(exp((double)s[j] - mx));
          sum += s[j];
        }
        double inv = 1.0 / sum;
        for (int j = 0; j <= t; j++) {
          s[j] = F32((double)s[j] * inv);
          P[pb + (int64_t)t * T + j] = s[j];
        }
        int64_t ob = (base + t) * qD + (int64_t)h * dH;
        for (int j = 0; j <= t; j++) {
          double p = s[j];
          if (p == 0.0) continue;
          int64_t vb = (base + j) * kvD + (int64_t)kvh * dH;
          for (int d = 0; d < dH; d++) out[ob + d] = F32((double)out[ob + d] + p * V[vb + d]);
        }
      }
    }
  }
  free(s);
  }
}

/* Accumulates into gQ, gK, gV (callers zero fresh gradients). */
void or_attn_bwd(float* gQ, float* gK, float* gV, const float* g, const float* P, const float* Q, const float* K,
                 const float* V, int B, int T, int nH, int nKV, int dH) {
  double scale = 1.0 / sqrt((double)dH);
  int group = nH / nKV > 1 ? nH / nKV : 1;
  int qD = nH * dH, kvD = nKV * dH;
  /* One task per (b, kv head): its gK/gV rows receive the heads h of its
   * group in increasing h (then t, then j) exactly as the serial loops
   * over b, h, t, j order them, and gQ of head h is written only there. */
#pragma omp parallel if ((int64_t)B * nH * T * T > (1 << 16))
  {
  float* dP = (float*)malloc(sizeof(float) * (size_t)T);
#pragma omp for collapse(2) schedule(dynamic, 1)
  for (int b = 0; b < B; b++) {
    for (int kv = 0; kv < nKV; kv++) {
    int64_t base = (int64_t)b * T;
    for (int h = 0; h < nH; h++) {
      int kvh = h / group;
      if (kvh != kv) continue;
      int64_t pb = ((int64_t)b * nH + h) * T * T;
      for (int t = 0; t < T; t++) {
        int64_t ob = (base + t) * qD + (int64_t)h * dH;
        double dotP = 0;
        int j = 0;
        /* four values at a time: independent sums over d, added to dotP in j order */
        for (; j + 4 <= t + 1; j += 4) {
          const float* v0 = V + (base + j) * kvD + (int64_t)kvh * dH;
          const float *v1 = v0 + kvD, *v2 = v1 + kvD, *v3 = v2 + kvD;
          double a[4] = {0, 0, 0, 0};
          for (int d = 0; d < dH; d++) {
            double gd = g[ob + d];
            a[0] += gd * v0[d];
            a[1] += gd * v1[d];
            a[2] += gd * v2[d];
            a[3] += gd * v3[d];
          }
          for (int u = 0; u < 4; u++) {
            dP[j + u] = F32(a[u]);
            dotP += a[u] * P[pb + (int64_t)t * T + j + u];
          }
        }
        for (; j <= t; j++) {
          int64_t vb = (base + j) * kvD + (int64_t)kvh * dH;
          double acc = 0;
          for (int d = 0; d < dH; d++) acc += (double)g[ob + d] * V[vb + d];
          dP[j] = F32(acc);
          dotP += acc * P[pb + (int64_t)t * T + j];
        }
        int64_t qb = (base + t) * qD + (int64_t)h * dH;
        for (int j = 0; j <= t; j++) {
          double pj = P[pb + (int64_t)t * T + j];
          if (pj == 0.0) continue;
          double dS = pj * ((double)dP[j] - dotP);
          int64_t vb = (base + j) * kvD + (int64_t)kvh * dH;
          int64_t kb = vb;
          for (int d = 0; d < dH; d++) {
            gV[vb + d] = F32((double)gV[vb + d] + pj * g[ob + d]);
            gQ[qb + d] = F32((double)gQ[qb + d] + dS * K[kb + d] * scale);
            gK[kb + d] = F32((double)gK[kb + d] + dS * Q[qb + d] * scale);
          }
        }
      }
    }
    }
  }
  free(dP);
  }
}

/* ───────────── swigluRows (tensor.js:272-290) ───────────── */
void or_swiglu_fwd(float* out, float* sig, const float* G, const float* U, int64_t n) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
  for (int64_t i = 0; i < n; i++) {
    double g = G[i];
    double s = 1.0 / (1.0 + exp(-g));
    sig[i] = F32(s);
    out[i] = F32(g * s * U[i]);
  }
}
void or_swiglu_bwd(float* gG, float* gU, const float* g, const float* sig, const float* G, const float* U,
                   int64_t n) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
  for (int64_t i = 0; i < n; i++) {
    double s = sig[i], gv = G[i];
    gG[i] = F32((double)gG[i] + (double)g[i] * U[i] * (s + gv * s * (1.0 - s)));
    gU[i] = F32((double)gU[i] + (double)g[i] * (gv * s));
  }
}

/* ───────────── weightedSum (tensor.js:380-389) ───────────── */
void or_weighted_sum_fwd(float* out, const float* Y, const float* t, int64_t n) {
  out[0] = 0.f;
  for (int64_t i = 0; i < n; i++) out[0] = F32((double)out[0] + (double)Y[i] * t[i]);
}
void or_weighted_sum_bwd(float* gY, double g0, const float* t, int64_t n) {
  for (int64_t i = 0; i < n; i++) gY[i] = F32((double)gY[i] + g0 * t[i]);
}

/* ───────────── crossEntropyMean (tensor.js:393-417) ───────────── */
void or_ce_fwd(float* loss_out, float* probs, const float* logits, const int32_t* targets, int T, int V) {
  /* rows are independent; their losses are added afterwards in row order */
  double* row_loss = (double*)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
#pragma omp parallel for schedule(static) if ((int64_t)T * V > (1 << 16))
  for (int t = 0; t < T; t++) {
    int64_t lb = (int64_t)t * V;
    float mxf = -INFINITY;
    for (int i = 0; i < V; i++)
      if (logits[lb + i] > mxf) mxf = logits[lb + i];
    double mx = mxf, s = 0;
    for (int i = 0; i < V; i++) {
      double e = exp((double)logits[lb + i] - mx);
      probs[lb + i] = F32(e);
      s += e;
    }
    double lse = mx + log(s);
    row_loss[t] = -((double)logits[lb + targets[t]] - lse);
    for (int i = 0; i < V; i++) probs[lb + i] = F32((double)probs[lb + i] / s);
  }
  double loss = 0;
  for (int t = 0; t < T; t++) loss += row_loss[t];
  free(row_loss);
  loss_out[0] = F32(loss / T);
}
void or_ce_bwd(float* gL, double g0, const float* probs, const int32_t* targets, int T, int V) {
  double k = g0 / T;
#pragma omp parallel for schedule(static) if ((int64_t)T * V > (1 << 16))
  for (int t = 0; t < T; t++) {
    int64_t lb = (int64_t)t * V;
    for (int i = 0; i < V; i++) gL[lb + i] = F32((double)gL[lb + i] + k * probs[lb + i]);
    gL[lb + targets[t]] = F32((double)gL[lb + targets[t]] - k);
  }
}

/* ───────────── addTensors (train.js:230-238) ───────────── */
void or_add_fwd(float* out, const float* a, const float* b, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = F32((double)a[i] + b[i]);
}
void or_accum(float* y, const float* x, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = F32((double)y[i] + x[i]);
}

/* ───────────── Adam.step (autograd.js:221-243) ───────────── */
/* Tensors with g == NULL are skipped, as params without a grad are.  t is the
 * post-increment step; out[0..2] = {lr, gnorm, scale}. */
void or_adam_step_given_norm(int count, float** p, float** g, float** m, float** v, const int64_t* n, int t,
                             double lr, double b1, double b2, double eps, double wd, double clip, double total,
                             double gnorm, double* out);
void or_adam_step(int count, float** p, float** g, float** m, float** v, const int64_t* n, int t, double lr,
                  double b1, double b2, double eps, double wd, double clip, double total, double* out) {
  double tot = 0;
  for (int j = 0; j < count; j++)
    if (g[j])
      for (int64_t i = 0; i < n[j]; i++) tot += (double)g[j][i] * g[j][i];
  or_adam_step_given_norm(count, p, g, m, v, n, t, lr, b1, b2, eps, wd, clip, total, sqrt(tot), out);
}

/* The update of or_adam_step with the global gradient norm given: for a step
 * checked on a subset of the parameters, whose norm covers them all. */
void or_adam_step_given_norm(int count, float** p, float** g, float** m, float** v, const int64_t* n, int t,
                             double lr, double b1, double b2, double eps, double wd, double clip, double total,
                             double gnorm, double* out) {
  double scale = gnorm > clip ? clip / gnorm : 1.0;
  double tt = (double)t / total;
  double lr_t = lr * 0.5 * (1.0 + cos(M_PI * (tt < 1.0 ? tt : 1.0)));
  for (int j = 0; j < count; j++) {
    if (!g[j]) continue;
#pragma omp parallel for schedule(static) if (n[j] > (1 << 16))
    for (int64_t i = 0; i < n[j]; i++) {
      double gi = (double)g[j][i] * scale + wd * p[j][i];
      m[j][i] = F32(b1 * m[j][i] + (1.0 - b1) * gi);
      v[j][i] = F32(b2 * v[j][i] + (1.0 - b2) * gi * gi);
      double mh = (double)m[j][i] / (1.0 - pow(b1, t));
      double vh = (double)v[j][i] / (1.0 - pow(b2, t));
      p[j][i] = F32((double)p[j][i] - lr_t * mh / (sqrt(vh) + eps));
    }
  }
  out[0] = lr_t;
  out[1] = gnorm;
  out[2] = scale;
}

/* ───────────── model (train.js:33-227, transformer.js:29-53) ───────────── */
typedef struct {
  int dim, hidden, nLayers, nHeads, nKvHeads, vocab;
  double normEps, ropeTheta;
  int tied; /* 1: LM head reuses tok_emb (wcls null, train.js:97) */
} or_cfg;

typedef struct {
  int dHead, kvDim, qkvOut, qD;
} or_dims;

static or_dims dims_of(const or_cfg* c) {
  or_dims d;
  d.dHead = c->dim / c->nHeads;
  d.kvDim = c->nKvHeads * d.dHead;
  d.qkvOut = (c->nHeads + 2 * c->nKvHeads) * d.dHead;
  d.qD = c->nHeads * d.dHead;
  return d;
}

/* Number of floats of the flat parameter vector, in paramList order
 * (train.js:60-78): tok_emb, ln_f, [wcls], per layer ln1, ln2, wqkv, wo,
 * ffn_gate, ffn_up, ffn_down. */
int64_t or_param_count(const or_cfg* c) {
  or_dims d = dims_of(c);
  int64_t n = (int64_t)c->vocab * c->dim + c->dim + (c->tied ? 0 : (int64_t)c->vocab * c->dim);
  int64_t per = 2LL * c->dim + (int64_t)d.qkvOut * c->dim + (int64_t)c->dim * c->dim +
                2LL * c->hidden * c->dim + (int64_t)c->dim * c->hidden;
  return n + per * c->nLayers;
}

typedef struct {
  float *tok_emb, *ln_f, *wcls;
  struct {
    float *ln1, *ln2, *wqkv, *wo, *gate, *up, *down;
  } L[64];
} or_wview;

static or_wview view_params(const or_cfg* c, float* flat) {
  or_dims d = dims_of(c);
  or_wview w;
  float* p = flat;
  w.tok_emb = p; p += (int64_t)c->vocab * c->dim;
  w.ln_f = p; p += c->dim;
  if (c->tied) w.wcls = w.tok_emb;
  else { w.wcls = p; p += (int64_t)c->vocab * c->dim; }
  for (int l = 0; l < c->nLayers; l++) {
    w.L[l].ln1 = p; p += c->dim;
    w.L[l].ln2 = p; p += c->dim;
    w.L[l].wqkv = p; p += (int64_t)d.qkvOut * c->dim;
    w.L[l].wo = p; p += (int64_t)c->dim * c->dim;
    w.L[l].gate = p; p += (int64_t)c->hidden * c->dim;
    w.L[l].up = p; p += (int64_t)c->hidden * c->dim;
    w.L[l].down = p; p += (int64_t)c->dim * c->hidden;
  }
  return w;
}

/* initWeights (train.js:33-57): RNG draw order tok_emb, then per layer wqkv,
 * wo, ffn_gate, ffn_up, ffn_down; norms = 1; wo, ffn_down scaled by
 * 1/sqrt(2L) (fp32 multiply-assign).  When !tied, wcls is drawn afterwards
 * from the same stream with the same std (how the untied configurations build
 * their weights object). */
void or_init_weights(const or_cfg* c, uint32_t seed, double std, float* flat) {
  or_rng r;
  or_rng_init(&r, seed);
  or_dims d = dims_of(c);
  or_wview w = view_params(c, flat);
  double resScale = 1.0 / sqrt(2.0 * c->nLayers);
  or_rng_fill_normal(&r, w.tok_emb, (int64_t)c->vocab * c->dim, std);
  for (int i = 0; i < c->dim; i++) w.ln_f[i] = 1.f;
  for (int l = 0; l < c->nLayers; l++) {
    for (int i = 0; i < c->dim; i++) { w.L[l].ln1[i] = 1.f; w.L[l].ln2[i] = 1.f; }
    or_rng_fill_normal(&r, w.L[l].wqkv, (int64_t)d.qkvOut * c->dim, std);
    int64_t nwo = (int64_t)c->dim * c->dim;
    or_rng_fill_normal(&r, w.L[l].wo, nwo, std);
    for (int64_t i = 0; i < nwo; i++) w.L[l].wo[i] = F32((double)w.L[l].wo[i] * resScale);
    or_rng_fill_normal(&r, w.L[l].gate, (int64_t)c->hidden * c->dim, std);
    or_rng_fill_normal(&r, w.L[l].up, (int64_t)c->hidden * c->dim, std);
    int64_t nd = (int64_t)c->dim * c->hidden;
    or_rng_fill_normal(&r, w.L[l].down, nd, std);
    for (int64_t i = 0; i < nd; i++) w.L[l].down[i] = F32((double)w.L[l].down[i] * resScale);
  }
  if (!c->tied) or_rng_fill_normal(&r, w.wcls, (int64_t)c->vocab * c->dim, std);
}

static float* zalloc(int64_t n) { return (float*)calloc((size_t)(n > 0 ? n : 1), sizeof(float)); }

/*
 * One training forward+backward (TrainableTransformer.lossBatch + backward,
 * train.js:120-159, 177-191) on B rows of T input ids and B*T targets.
 * Writes logits[B*T*V], *loss, and grads (flat, paramList order; accumulated
 * onto what grads holds, as param grads are until zeroGrad); with grads NULL
 * only the forward and the loss run.
 * Backward runs in the reverse order of the reference's tape.
 */
void or_model_fwd_bwd(const or_cfg* c, const float* params, const int32_t* ids, const int32_t* targets, int B,
                      int T, float* logits, float* loss, float* grads) {
  or_dims d = dims_of(c);
  int64_t BT = (int64_t)B * T;
  int D = c->dim, H = c->hidden, nL = c->nLayers, V = c->vocab;
  or_wview w = view_params(c, (float*)params);
  or_wview gw;
  memset(&gw, 0, sizeof(gw));
  if (grads) gw = view_params(c, grads);

  typedef struct {
    float *x_in, *xn, *inv1, *qkv, *q, *k, *v, *qr, *kr, *att, *P, *ao, *x1, *xn2, *inv2, *g, *u, *act, *sig,
        *ff, *x2;
  } act_t;
  act_t* A = (act_t*)calloc((size_t)nL, sizeof(act_t));
  float* x0 = zalloc(BT * D);
  or_embed_fwd(x0, w.tok_emb, ids, (int)BT, D);
  float* x = x0;
  for (int l = 0; l < nL; l++) {
    act_t* a = &A[l];
    a->x_in = x;
    a->xn = zalloc(BT * D); a->inv1 = zalloc(BT);
    or_rmsnorm_fwd(a->xn, a->inv1, x, w.L[l].ln1, (int)BT, D, c->normEps);
    a->qkv = zalloc(BT * d.qkvOut);
    or_gemm(a->qkv, a->xn, w.L[l].wqkv, (int)BT, d.qkvOut, D);
    a->q = zalloc(BT * d.qD); a->k = zalloc(BT * d.kvDim); a->v = zalloc(BT * d.kvDim);
    or_slice_fwd(a->q, a->qkv, (int)BT, d.qkvOut, 0, d.qD);
    or_slice_fwd(a->k, a->qkv, (int)BT, d.qkvOut, d.qD, d.kvDim);
    or_slice_fwd(a->v, a->qkv, (int)BT, d.qkvOut, d.qD + d.kvDim, d.kvDim);
    a->qr = zalloc(BT * d.qD); a->kr = zalloc(BT * d.kvDim);
    or_rope_fwd(a->qr, a->q, (int)BT, c->nHeads, d.dHead, 0, c->ropeTheta, T);
    or_rope_fwd(a->kr, a->k, (int)BT, c->nKvHeads, d.dHead, 0, c->ropeTheta, T);
    a->att = zalloc(BT * d.qD);
    a->P = zalloc((int64_t)B * c->nHeads * T * T);
    or_attn_fwd(a->att, a->P, a->qr, a->kr, a->v, B, T, c->nHeads, c->nKvHeads, d.dHead);
    if (!grads) { free(a->P); a->P = NULL; } /* only the backward reads P */
    a->ao = zalloc(BT * D);
    or_gemm(a->ao, a->att, w.L[l].wo, (int)BT, D, d.qD);
    a->x1 = zalloc(BT * D);
    or_add_fwd(a->x1, x, a->ao, BT * D);
    a->xn2 = zalloc(BT * D); a->inv2 = zalloc(BT);
    or_rmsnorm_fwd(a->xn2, a->inv2, a->x1, w.L[l].ln2, (int)BT, D, c->normEps);
    a->g = zalloc(BT * H); a->u = zalloc(BT * H);
    or_gemm(a->g, a->xn2, w.L[l].gate, (int)BT, H, D);
    or_gemm(a->u, a->xn2, w.L[l].up, (int)BT, H, D);
    a->act = zalloc(BT * H); a->sig = zalloc(BT * H);
    or_swiglu_fwd(a->act, a->sig, a->g, a->u, BT * H);
    a->ff = zalloc(BT * D);
    or_gemm(a->ff, a->act, w.L[l].down, (int)BT, D, H);
    a->x2 = zalloc(BT * D);
    or_add_fwd(a->x2, a->x1, a->ff, BT * D);
    x = a->x2;
  }
  float* xf = zalloc(BT * D);
  float* invf = zalloc(BT);
  or_rmsnorm_fwd(xf, invf, x, w.ln_f, (int)BT, D, c->normEps);
  or_gemm(logits, xf, w.wcls, (int)BT, V, D);
  float* probs = zalloc(BT * V);
  or_ce_fwd(loss, probs, logits, targets, (int)BT, V);
  if (!grads) { /* forward and loss only */
    free(probs); free(xf); free(invf);
    for (int l = 0; l < nL; l++) {
      act_t* a = &A[l];
      free(a->xn); free(a->inv1); free(a->qkv); free(a->q); free(a->k); free(a->v); free(a->qr); free(a->kr);
      free(a->att); free(a->P); free(a->ao); free(a->x1); free(a->xn2); free(a->inv2); free(a->g); free(a->u);
      free(a->act); free(a->sig); free(a->ff); free(a->x2);
    }
    free(x0);
    free(A);
    return;
  }

  /* backward (reverse tape) */
  float* glog = zalloc(BT * V);
  or_ce_bwd(glog, 1.0, probs, targets, (int)BT, V);
  free(probs);
  float* gxf = zalloc(BT * D);
  or_matmulT_bwd(gxf, gw.wcls, glog, xf, w.wcls, (int)BT, D, V);
  free(glog);
  float* gx = zalloc(BT * D); /* grad of the residual stream x (current) */
  or_rmsnorm_bwd(gx, gw.ln_f, gxf, x, w.ln_f, invf, (int)BT, D);
  free(gxf); free(xf); free(invf);
  for (int l = nL - 1; l >= 0; l--) {
    act_t* a = &A[l];
    /* x2 = add(x1, ff) */
    float* gx1 = zalloc(BT * D);
    float* gff = zalloc(BT * D);
    or_accum(gx1, gx, BT * D);
    or_accum(gff, gx, BT * D);
    free(gx);
    /* ff = matmulT(act, down) */
    float* gact = zalloc(BT * H);
    or_matmulT_bwd(gact, gw.L[l].down, gff, a->act, w.L[l].down, (int)BT, H, D);
    free(gff);
    /* act = swiglu(g, u) */
    float* gg = zalloc(BT * H);
    float* gu = zalloc(BT * H);
    or_swiglu_bwd(gg, gu, gact, a->sig, a->g, a->u, BT * H);
    free(gact);
    /* u then g = matmulT(xn2, ·) */
    float* gxn2 = zalloc(BT * D);
    or_matmulT_bwd(gxn2, gw.L[l].up, gu, a->xn2, w.L[l].up, (int)BT, D, H);
    or_matmulT_bwd(gxn2, gw.L[l].gate, gg, a->xn2, w.L[l].gate, (int)BT, D, H);
    free(gg); free(gu);
    /* xn2 = rmsNorm(x1) */
    or_rmsnorm_bwd(gx1, gw.L[l].ln2, gxn2, a->x1, w.L[l].ln2, a->inv2, (int)BT, D);
    free(gxn2);
    /* x1 = add(x, ao) */
    float* gxin = zalloc(BT * D);
    float* gao = zalloc(BT * D);
    or_accum(gxin, gx1, BT * D);
    or_accum(gao, gx1, BT * D);
    free(gx1);
    /* ao = matmulT(att, wo) */
    float* gatt = zalloc(BT * d.qD);
    or_matmulT_bwd(gatt, gw.L[l].wo, gao, a->att, w.L[l].wo, (int)BT, d.qD, D);
    free(gao);
    /* att = attention(qr, kr, v) */
    float* gqr = zalloc(BT * d.qD);
    float* gkr = zalloc(BT * d.kvDim);
    float* gv = zalloc(BT * d.kvDim);
    or_attn_bwd(gqr, gkr, gv, gatt, a->P, a->qr, a->kr, a->v, B, T, c->nHeads, c->nKvHeads, d.dHead);
    free(gatt);
    /* kr, qr = rope(k), rope(q) */
    float* gk = zalloc(BT * d.kvDim);
    float* gq = zalloc(BT * d.qD);
    or_rope_bwd(gk, gkr, (int)BT, c->nKvHeads, d.dHead, 0, c->ropeTheta, T);
    or_rope_bwd(gq, gqr, (int)BT, c->nHeads, d.dHead, 0, c->ropeTheta, T);
    free(gkr); free(gqr);
    /* v, k, q = sliceCols(qkv) */
    float* gqkv = zalloc(BT * d.qkvOut);
    or_slice_bwd(gqkv, gv, (int)BT, d.qkvOut, d.qD + d.kvDim, d.kvDim);
    or_slice_bwd(gqkv, gk, (int)BT, d.qkvOut, d.qD, d.kvDim);
    or_slice_bwd(gqkv, gq, (int)BT, d.qkvOut, 0, d.qD);
    free(gv); free(gk); free(gq);
    /* qkv = matmulT(xn, wqkv) */
    float* gxn = zalloc(BT * D);
    or_matmulT_bwd(gxn, gw.L[l].wqkv, gqkv, a->xn, w.L[l].wqkv, (int)BT, D, d.qkvOut);
    free(gqkv);
    /* xn = rmsNorm(x) */
    or_rmsnorm_bwd(gxin, gw.L[l].ln1, gxn, a->x_in, w.L[l].ln1, a->inv1, (int)BT, D);
    free(gxn);
    gx = gxin;
    free(a->xn); free(a->inv1); free(a->qkv); free(a->q); free(a->k); free(a->v); free(a->qr); free(a->kr);
    free(a->att); free(a->P); free(a->ao); free(a->x1); free(a->xn2); free(a->inv2); free(a->g); free(a->u);
    free(a->act); free(a->sig); free(a->ff); free(a->x2);
  }
  or_embed_bwd(gw.tok_emb, gx, ids, (int)BT, D);
  free(gx);
  free(x0);
  free(A);
}

/* ───────────── inference forward (transformer.js:134-184) — the I-70 partner ───────────── */
/* quant_oracle.c: dotQ / dequantize / rowBytes (quant.js:64, 102-320). */
double oq_dotq(int type, const uint8_t* u8, const float* x, int64_t n);
int oq_dequantize(int type, const uint8_t* u8, int64_t n, float* out);
int64_t oq_row_bytes(int type, int64_t n);

/* A weight matrix [N, K] stored as rows of oq_row_bytes(type, K) bytes
 * (QuantLinear, nn.js:19-40; type 0 = f32). */
typedef struct {
  int type;
  const void* data;
} or_qmat;
typedef struct {
  const float *ln1, *ln2;
  or_qmat wqkv, wo, gate, up, down;
} or_qlayer;
typedef struct {
  or_qmat tok_emb;
  const float* ln_f;
  or_qmat wcls;
  const or_qlayer* layers;
} or_qmodel;

/* QuantLinear.forward (nn.js:27-33): out[n] = fp32(dotQ(row n)); for type 0
 * dotQ is numeric.js dot, the same four-partial sum as matvec (numeric.js:85-100). */
static void qmatvec_ref(float* out, or_qmat W, const float* x, int N, int K) {
  int64_t rb = oq_row_bytes(W.type, K);
  for (int n = 0; n < N; n++) out[n] = F32(oq_dotq(W.type, (const uint8_t*)W.data + (int64_t)n * rb, x, K));
}
static void rmsnorm_l1(float* out, const float* x, const float* w, int n, double eps) { /* special.js:46-50 */
  double s = 0;
  for (int i = 0; i < n; i++) s += (double)x[i] * x[i];
  double rms = sqrt(s / n);
  double ss = 1.0 / sqrt(rms * rms + eps);
  for (int i = 0; i < n; i++) out[i] = F32((double)x[i] * ss * w[i]);
}

/* Single-token decode with a contiguous KV cache, token by token, writing
 * logits[T*V], over weights of any QuantLinear type.  Uses the fp32 RoPE
 * table (special.js:116-127), attentionDecode (attention.js:31-61) and the
 * embedding row copy / dequantize of Transformer._embed (transformer.js:121-131). */
void or_infer_forward_q(const or_cfg* c, const or_qmodel* m, const int32_t* ids, int T, float* logits) {
  or_dims d = dims_of(c);
  int D = c->dim, H = c->hidden, V = c->vocab, dH = d.dHead, half = dH / 2;
  int maxSeq = T;
  float* ctab = zalloc((int64_t)maxSeq * half);
  float* stab = zalloc((int64_t)maxSeq * half);
  for (int p = 0; p < maxSeq; p++)
    for (int i = 0; i < dH; i += 2) {
      double freq = 1.0 / pow(c->ropeTheta, (double)i / dH);
      double ang = (double)p * freq;
      ctab[p * half + i / 2] = F32(cos(ang));
      stab[p * half + i / 2] = F32(sin(ang));
    }
  float* kc = zalloc((int64_t)c->nLayers * maxSeq * d.kvDim);
  float* vc = zalloc((int64_t)c->nLayers * maxSeq * d.kvDim);
  float *x = zalloc(D), *xb = zalloc(D), *xb2 = zalloc(D), *q = zalloc(d.qkvOut), *att = zalloc(D);
  float *gbuf = zalloc(H), *ubuf = zalloc(H), *sc = zalloc(maxSeq);
  double scale = 1.0 / sqrt((double)dH);
  int group = c->nHeads / c->nKvHeads;
  int64_t emb_rb = oq_row_bytes(m->tok_emb.type, D);
  for (int pos = 0; pos < T; pos++) {
    oq_dequantize(m->tok_emb.type, (const uint8_t*)m->tok_emb.data + (int64_t)ids[pos] * emb_rb, D, x);
    for (int l = 0; l < c->nLayers; l++) {
      const or_qlayer* L = m->layers + l;
      rmsnorm_l1(xb, x, L->ln1, D, c->normEps);
      qmatvec_ref(q, L->wqkv, xb, d.qkvOut, D);
      int nh_all = c->nHeads + c->nKvHeads;
      for (int h = 0; h < nh_all; h++) {
        float* v = q + h * dH;
        for (int i = 0; i < dH; i += 2) {
          double cc = ctab[pos * half + i / 2], ss = stab[pos * half + i / 2];
          double a = v[i], b = v[i + 1];
          v[i] = F32(a * cc - b * ss);
          v[i + 1] = F32(a * ss + b * cc);
        }
      }
      int64_t co = ((int64_t)l * maxSeq + pos) * d.kvDim;
      memcpy(kc + co, q + d.qD, sizeof(float) * d.kvDim);
      memcpy(vc + co, q + d.qD + d.kvDim, sizeof(float) * d.kvDim);
      for (int i = 0; i < D; i++) att[i] = 0.f;
      int n = pos + 1;
      for (int kvh = 0; kvh < c->nKvHeads; kvh++) {
        for (int gi = 0; gi < group; gi++) {
          int h = kvh * group + gi;
          if (h >= c->nHeads) break;
          const float* qh = q + h * dH;
          float* out = att + h * dH;
          double mx = -INFINITY;
          for (int j = 0; j < n; j++) {
            const float* kr = kc + ((int64_t)l * maxSeq + j) * d.kvDim + kvh * dH;
            double acc = 0;
            for (int i = 0; i < dH; i++) acc += (double)qh[i] * kr[i];
            double v = acc * scale;
            sc[j] = F32(v);
            if (v > mx) mx = v;
          }
          for (int i = 0; i < dH; i++) out[i] = 0.f;
          double lsum = 0;
          for (int j = 0; j < n; j++) {
            double p = exp((double)sc[j] - mx);
            if (p == 0.0) continue;
            lsum += p;
            const float* vr = vc + ((int64_t)l * maxSeq + j) * d.kvDim + kvh * dH;
            for (int i = 0; i < dH; i++) out[i] = F32((double)out[i] + p * vr[i]);
          }
          double inv = 1.0 / (lsum != 0.0 ? lsum : 1.0);
          for (int i = 0; i < dH; i++) out[i] = F32((double)out[i] * inv);
        }
      }
      qmatvec_ref(xb2, L->wo, att, D, D);
      for (int i = 0; i < D; i++) x[i] = F32((double)x[i] + xb2[i]);
      rmsnorm_l1(xb, x, L->ln2, D, c->normEps);
      qmatvec_ref(gbuf, L->gate, xb, H, D);
      qmatvec_ref(ubuf, L->up, xb, H, D);
      for (int i = 0; i < H; i++) {
        double g = gbuf[i];
        gbuf[i] = F32((g / (1.0 + exp(-g))) * ubuf[i]);
      }
      qmatvec_ref(xb2, L->down, gbuf, D, H);
      for (int i = 0; i < D; i++) x[i] = F32((double)x[i] + xb2[i]);
    }
    rmsnorm_l1(xb, x, m->ln_f, D, c->normEps);
    qmatvec_ref(logits + (int64_t)pos * V, m->wcls, xb, V, D);
  }
  free(ctab); free(stab); free(kc); free(vc); free(x); free(xb); free(xb2); free(q); free(att);
  free(gbuf); free(ubuf); free(sc);
}

/* The f32 model of the flat parameter vector (paramList order). */
void or_infer_forward(const or_cfg* c, const float* params, const int32_t* ids, int T, float* logits) {
  or_wview w = view_params(c, (float*)params);
  or_qlayer* L = (or_qlayer*)calloc((size_t)(c->nLayers > 0 ? c->nLayers : 1), sizeof(or_qlayer));
  for (int l = 0; l < c->nLayers; l++) {
    L[l].ln1 = w.L[l].ln1;
    L[l].ln2 = w.L[l].ln2;
    L[l].wqkv.data = w.L[l].wqkv;
    L[l].wo.data = w.L[l].wo;
    L[l].gate.data = w.L[l].gate;
    L[l].up.data = w.L[l].up;
    L[l].down.data = w.L[l].down;
  }
  or_qmodel m;
  m.tok_emb.type = 0;
  m.tok_emb.data = w.tok_emb;
  m.ln_f = w.ln_f;
  m.wcls.type = 0;
  m.wcls.data = w.wcls;
  m.layers = L;
  or_infer_forward_q(c, &m, ids, T, logits);
  free(L);
}
