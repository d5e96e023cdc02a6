/*
 * quant_oracle.c — CPU restatement of forge-llm's quantized weight formats
 * (src/L3/quant.js, src/L1/special.js:143-168, src/L4/nn.js:19-40).
 *
 * TEST INFRASTRUCTURE ONLY, like forge_oracle.c: tests/ and the CPU baseline
 * may load it, as the parity reference; the product path never links or falls back to it.
 *
 * The reference is JavaScript: every intermediate is an fp64 number, stores
 * into Float32Array round to fp32, stores into Uint8Array / Int8Array wrap
 * modulo 256, and Math.round rounds half-way cases towards +infinity.  The
 * functions below keep those semantics, the reference's evaluation order
 * (left to right, no fused multiply-add: built with -ffp-contract=off) and its
 * loop orders, so quantized bytes are bit-identical and dot products differ
 * from the reference only through libm (none is used except sqrt, which is
 * correctly rounded in both).
 *
 * Types: 0 F32, 1 F16, 2 Q4_0, 6 Q5_0 (decode only, as the reference's
 * generic branch reads them), 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define F32(x) ((float)(x))

/* ───────────── JS number helpers ───────────── */
/* Math.round: nearest integer, ties towards +infinity (exact for |v| < 2^52). */
static double js_round(double v) {
  if (!isfinite(v)) return v;
  double f = floor(v);
  return (v - f) >= 0.5 ? f + 1.0 : f;
}
/* quant.js:322 nearest_int: half-way cases away from zero. */
static double rnd(double v) { return v < 0 ? -js_round(-v) : js_round(v); }
static double clampd(double v, double a, double b) { return v < a ? a : v > b ? b : v; }
/* ToUint8 / ToInt8 of a store into a typed array (NaN and infinities give 0). */
static uint8_t to_u8(double v) {
  if (!isfinite(v)) return 0;
  double t = trunc(v);
  double m = fmod(t, 256.0);
  if (m < 0) m += 256.0;
  return (uint8_t)m;
}
static int8_t to_i8(double v) { return (int8_t)to_u8(v); }

/* special.js:143-148, quant.js:71-84 (the table holds the same values). */
double oq_fp16_to_fp32(uint16_t h) {
  int s = (h & 0x8000) >> 15, e = (h & 0x7c00) >> 10, f = h & 0x03ff;
  if (e == 0) return (s ? -1.0 : 1.0) * 5.9604644775390625e-8 * f;
  if (e == 31) return f ? NAN : (s ? -INFINITY : INFINITY);
  return (s ? -1.0 : 1.0) * ldexp(1.0 + f / 1024.0, e - 15);
}
static double h2d(const uint8_t* p) { return oq_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8))); }

/* special.js:151-168: fp64 → half, Math.round on the mantissa (ties up in
 * magnitude), subnormals as round(x·2^24) & 0x3ff. */
uint16_t oq_fp32_to_fp16(double x) {
  if (!isfinite(x)) return x > 0 ? 0x7c00 : x < 0 ? 0xfc00 : 0x7e00;
  int s = x < 0 ? 0x8000 : 0;
  x = fabs(x);
  if (x < 6.103515625e-5) {
    double q = js_round(x * 16777216.0);
    return (uint16_t)(s | ((int64_t)q & 0x3ff));
  }
  int e = 0;
  while (x >= 2) { x /= 2; e++; }
  while (x < 1) { x *= 2; e--; }
  int m = (int)js_round((x - 1) * 1024);
  if (m == 1024) { e++; m = 0; }
  int ex = e + 15;
  if (ex >= 31) return (uint16_t)(s | 0x7c00);
  return (uint16_t)(s | (ex << 10) | m);
}
static void put_h(uint8_t* p, uint16_t h) { p[0] = h & 0xff; p[1] = h >> 8; }

/* ───────────── type table (quant.js:42-56) ───────────── */
static int block_of(int type, int* bytes) {
  switch (type) {
    case 0: *bytes = 4; return 1;
    case 1: *bytes = 2; return 1;
    case 2: *bytes = 18; return 32;
    case 6: *bytes = 22; return 32;
    case 8: *bytes = 34; return 32;
    case 12: *bytes = 144; return 256;
    case 13: *bytes = 176; return 256;
    case 14: *bytes = 210; return 256;
    default: return 0;
  }
}
/* rowBytes (quant.js:64): ceil(n / block) · block bytes; −1 for an unknown type. */
int64_t oq_row_bytes(int type, int64_t n) {
  int bb, bs = block_of(type, &bb);
  if (!bs) return -1;
  return (n + bs - 1) / bs * bb;
}

/* getScaleMinK4 (quant.js:88-94): the j-th 6-bit (scale, min) of a K-quant block. */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

/* ───────────── dequantize (quant.js:102-199) ───────────── */
/* Returns 0, or −1 for a type the reference does not decode. */
int oq_dequantize(int type, const uint8_t* u8, int64_t n, float* out) {
  switch (type) {
    case 0: memcpy(out, u8, (size_t)n * 4); return 0;
    case 1:
      for (int64_t i = 0; i < n; i++) out[i] = F32(h2d(u8 + 2 * i));
      return 0;
    case 8: {
      int64_t nb = n >> 5;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* B = u8 + b * 34;
        double d = h2d(B);
        for (int j = 0; j < 32; j++) out[b * 32 + j] = F32((double)(int8_t)B[2 + j] * d);
      }
      return 0;
    }
    case 12: case 13: {
      int64_t nb = n >> 8;
      int bb = type == 12 ? 144 : 176;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* B = u8 + b * bb;
        double d = h2d(B), dmin = h2d(B + 2);
        const uint8_t* sc = B + 4;
        const uint8_t* qh = B + 16;
        const uint8_t* qs = B + (type == 12 ? 16 : 48);
        int is = 0, u1 = 1, u2 = 2;
        float* o = out + b * 256;
        for (int j = 0; j < 256; j += 64) {
          int s, m;
          scale_min_k4(is, sc, &s, &m);
          double d1 = d * s, n1 = dmin * m;
          scale_min_k4(is + 1, sc, &s, &m);
          double d2 = d * s, n2 = dmin * m;
          for (int l = 0; l < 32; l++) {
            int q = qs[(j >> 1) + l] & 0xF;
            if (type == 13 && (qh[l] & u1)) q += 16;
            o[j + l] = F32(d1 * q - n1);
          }
          for (int l = 0; l < 32; l++) {
            int q = qs[(j >> 1) + l] >> 4;
            if (type == 13 && (qh[l] & u2)) q += 16;
            o[j + 32 + l] = F32(d2 * q - n2);
          }
          is += 2;
          u1 <<= 2;
          u2 <<= 2;
        }
      }
      return 0;
    }
    case 14: {
      int64_t nb = n >> 8;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* B = u8 + b * 210;
        double d = h2d(B + 208);
        const uint8_t *ql = B, *qh = B + 128;
        const int8_t* sc = (const int8_t*)(B + 192);
        float* o = out + b * 256;
        for (int n2 = 0; n2 < 256; n2 += 128) {
          int hB = n2 >> 2, sB = n2 >> 4;
          for (int l = 0; l < 32; l++) {
            int is = l >> 4;
            int q1 = ((ql[(n2 >> 1) + l] & 0xF) | ((qh[hB + l] & 3) << 4)) - 32;
            int q2 = ((ql[(n2 >> 1) + l + 32] & 0xF) | (((qh[hB + l] >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[(n2 >> 1) + l] >> 4) | (((qh[hB + l] >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[(n2 >> 1) + l + 32] >> 4) | (((qh[hB + l] >> 6) & 3) << 4)) - 32;
            o[n2 + l] = F32(d * sc[sB + is] * q1);
            o[n2 + 32 + l] = F32(d * sc[sB + is + 2] * q2);
            o[n2 + 64 + l] = F32(d * sc[sB + is + 4] * q3);
            o[n2 + 96 + l] = F32(d * sc[sB + is + 6] * q4);
          }
        }
      }
      return 0;
    }
    case 2: case 6: {
      int bb = type == 2 ? 18 : 22;
      int64_t nb = n >> 5;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* B = u8 + b * bb;
        double d = h2d(B);
        for (int j = 0; j < 32; j++) {
          int u = B[2 + (j >> 1)];
          int q = (j & 1) ? (u >> 4) : (u & 0xF);
          out[b * 32 + j] = F32((type == 2 ? q - 8 : q) * d);
        }
      }
      return 0;
    }
    default: return -1;
  }
}

/* ───────────── dotQ (quant.js:215-320) and dot (numeric.js:52-60) ───────────── */
static double dot4(const float* a, const float* b, int64_t n) {
  double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  int64_t i = 0;
  for (; i + 4 <= n; i += 4) {
    s0 += (double)a[i] * b[i];
    s1 += (double)a[i + 1] * b[i + 1];
    s2 += (double)a[i + 2] * b[i + 2];
    s3 += (double)a[i + 3] * b[i + 3];
  }
  double s = s0 + s1 + s2 + s3;
  for (; i < n; i++) s += (double)a[i] * b[i];
  return s;
}

/* Returns the fp64 dot product of n quantized weights with x (NaN for an
 * unknown type). */
double oq_dotq(int type, const uint8_t* u8, const float* x, int64_t n) {
  switch (type) {
    case 0: return dot4((const float*)u8, x, n);
    case 1: {
      double s = 0;
      for (int64_t i = 0; i < n; i++) s += h2d(u8 + 2 * i) * x[i];
      return s;
    }
    case 8: {
      int64_t nb = n >> 5;
      double s = 0;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* B = u8 + b * 34;
        double d = h2d(B);
        const float* xb = x + b * 32;
        double t0 = 0, t1 = 0, t2 = 0, t3 = 0;
        for (int j = 0; j < 32; j += 4) {
          t0 += (double)(int8_t)B[2 + j] * xb[j];
          t1 += (double)(int8_t)B[3 + j] * xb[j + 1];
          t2 += (double)(int8_t)B[4 + j] * xb[j + 2];
          t3 += (double)(int8_t)B[5 + j] * xb[j + 3];
        }
        s += (t0 + t1 + t2 + t3) * d;
      }
      return s;
    }
    case 12: case 13: {
      int64_t nb = n >> 8;
      int bb = type == 12 ? 144 : 176;
      double s = 0;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* B = u8 + b * bb;
        double d = h2d(B), dmin = h2d(B + 2);
        const uint8_t* sc = B + 4;
        const uint8_t* qh = B + 16;
        const uint8_t* qs = B + (type == 12 ? 16 : 48);
        const float* xb = x + b * 256;
        int is = 0, u1 = 1, u2 = 2;
        for (int j = 0; j < 256; j += 64) {
          int sv, mv;
          scale_min_k4(is, sc, &sv, &mv);
          double d1 = d * sv, m1 = dmin * mv;
          scale_min_k4(is + 1, sc, &sv, &mv);
          double d2 = d * sv, m2 = dmin * mv;
          for (int l = 0; l < 32; l++) {
            int q = qs[(j >> 1) + l] & 0xF;
            if (type == 13 && (qh[l] & u1)) q += 16;
            s += (d1 * q - m1) * xb[j + l];
          }
          for (int l = 0; l < 32; l++) {
            int q = qs[(j >> 1) + l] >> 4;
            if (type == 13 && (qh[l] & u2)) q += 16;
            s += (d2 * q - m2) * xb[j + 32 + l];
          }
          is += 2;
          u1 <<= 2;
          u2 <<= 2;
        }
      }
      return s;
    }
    case 14: {
      int64_t nb = n >> 8;
      double s = 0;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* B = u8 + b * 210;
        double d = h2d(B + 208);
        const uint8_t *ql = B, *qh = B + 128;
        const int8_t* sc = (const int8_t*)(B + 192);
        const float* xb = x + b * 256;
        for (int nn = 0; nn < 256; nn += 128) {
          int hB = nn >> 2, sB = nn >> 4, lb = nn >> 1;
          for (int l = 0; l < 32; l++) {
            int is = l >> 4;
            int h = qh[hB + l];
            int q1 = ((ql[lb + l] & 0xF) | ((h & 3) << 4)) - 32;
            int q2 = ((ql[lb + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[lb + l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[lb + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
            double s1 = sc[sB + is], s2 = sc[sB + is + 2], s3 = sc[sB + is + 4], s4 = sc[sB + is + 6];
            s += d * (s1 * q1 * xb[nn + l] + s2 * q2 * xb[nn + 32 + l] + s3 * q3 * xb[nn + 64 + l] +
                      s4 * q4 * xb[nn + 96 + l]);
          }
        }
      }
      return s;
    }
    case 2: case 6: {
      float* w = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
      oq_dequantize(type, u8, n, w);
      double s = dot4(w, x, n);
      free(w);
      return s;
    }
    default: return NAN;
  }
}

/* QuantLinear.forward (nn.js:27-33): y[n] = fp32(dotQ(row n)), rows of
 * rowBytes(type, K) bytes. */
void oq_qmatvec(int type, float* y, const uint8_t* W, const float* x, int N, int K) {
  int64_t rb = oq_row_bytes(type, K);
  for (int n = 0; n < N; n++) y[n] = F32(oq_dotq(type, W + (int64_t)n * rb, x, K));
}

/* ───────────── quantizers (quant.js:322-590) ───────────── */
/* Q8_0 (quant.js:328-339): d = amax/127, q = clamp(rnd(x/d), −128, 127). */
static void quant_q8_0(const float* x, int64_t n, uint8_t* out) {
  int64_t nb = n >> 5;
  for (int64_t b = 0; b < nb; b++) {
    const float* xb = x + b * 32;
    double amax = 0;
    for (int j = 0; j < 32; j++) {
      double v = fabs((double)xb[j]);
      if (v > amax) amax = v;
    }
    double d = amax / 127, id = (d != 0 && d == d) ? 1 / d : 0;
    put_h(out + b * 34, oq_fp32_to_fp16(d));
    for (int j = 0; j < 32; j++) out[b * 34 + 2 + j] = to_u8(clampd(rnd(xb[j] * id), -128, 127));
  }
}

/* make_qx_quants (quant.js:384-414): symmetric nmax-level search over 19 scales. */
static double make_qx_quants(int n, int nmax, const float* x, int8_t* L) {
  double max = 0, amax = 0;
  for (int i = 0; i < n; i++) {
    double ax = fabs((double)x[i]);
    if (ax > amax) { amax = ax; max = x[i]; }
  }
  if (amax < 1e-30) {
    for (int i = 0; i < n; i++) L[i] = 0;
    return 0;
  }
  double iscale = -nmax / max;
  double sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; i++) {
    double l = clampd(rnd(iscale * x[i]), -nmax, nmax - 1);
    L[i] = to_i8(l);
    double w = (double)x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  double scale = suml2 != 0 ? sumlx / suml2 : 0;
  double best = scale * sumlx;
  for (int is = -9; is <= 9; is++) {
    if (is == 0) continue;
    iscale = -(nmax + 0.1 * is) / max;
    sumlx = 0;
    suml2 = 0;
    for (int i = 0; i < n; i++) {
      double l = clampd(rnd(iscale * x[i]), -nmax, nmax - 1);
      double w = (double)x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; i++) L[i] = to_i8(clampd(rnd(iscale * x[i]), -nmax, nmax - 1));
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

/* Q6_K (quant.js:346-381): 16 sub-blocks of 16 through make_qx_quants, int8
 * sub-block scales, fp16 d at the block's end. */
static void quant_q6_k(const float* x, int64_t n, uint8_t* out) {
  int64_t nb = n >> 8;
  int8_t L[256];
  float scales[16];
  memset(out, 0, (size_t)nb * 210);
  for (int64_t b = 0; b < nb; b++) {
    const float* xb = x + b * 256;
    uint8_t* B = out + b * 210;
    double maxScale = 0, maxAbs = 0;
    for (int ib = 0; ib < 16; ib++) {
      double s = make_qx_quants(16, 32, xb + ib * 16, L + ib * 16);
      scales[ib] = F32(s);
      double a = fabs(s);
      if (a > maxAbs) { maxAbs = a; maxScale = s; }
    }
    if (maxAbs < 1e-30) continue;
    double iscale = -128 / maxScale;
    uint16_t dh = oq_fp32_to_fp16(1 / iscale);
    put_h(B + 208, dh);
    for (int ib = 0; ib < 16; ib++) {
      double v = rnd(iscale * scales[ib]);
      B[192 + ib] = to_u8(v < 127 ? v : (v != v ? v : 127));  /* Math.min(127, v) & 0xff */
    }
    double d = oq_fp16_to_fp32(dh);
    for (int j = 0; j < 16; j++) {
      double dd = d * (int8_t)B[192 + j];
      if (dd == 0 || dd != dd) {
        for (int ii = 0; ii < 16; ii++) L[j * 16 + ii] = 32;
        continue;
      }
      for (int ii = 0; ii < 16; ii++) L[j * 16 + ii] = to_i8(clampd(rnd(xb[j * 16 + ii] / dd), -32, 31) + 32);
    }
    for (int j = 0; j < 256; j += 128) {
      uint8_t* p = B + (j >> 1);
      for (int l = 0; l < 32; l++) {
        int q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF, q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
        p[l] = (uint8_t)(q1 | (q3 << 4));
        p[l + 32] = (uint8_t)(q2 | (q4 << 4));
        B[128 + (j >> 2) + l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                                          ((L[j + l + 96] >> 4) << 6));
      }
    }
  }
}

/* make_qkx2_quants (quant.js:423-469): weighted least-squares (scale, min)
 * search over nstep+1 candidate scales; returns the scale, *the_min = −min. */
static double make_qkx2_quants(int n, int nmax, const float* x, const float* weights, uint8_t* L, float* the_min,
                               uint8_t* Laux, double rmin, double rdelta, int nstep) {
  double min = x[0], max = x[0];
  double sumW = weights[0], sumX = (double)weights[0] * x[0];
  for (int i = 1; i < n; i++) {
    double v = x[i];
    if (v < min) min = v;
    if (v > max) max = v;
    double w = weights[i];
    sumW += w;
    sumX += w * v;
  }
  if (min > 0) min = 0;
  if (max == min) {
    for (int i = 0; i < n; i++) L[i] = 0;
    *the_min = F32(-min);
    return 0;
  }
  double iscale = nmax / (max - min);
  double scale = 1 / iscale;
  double best = 0;
  for (int i = 0; i < n; i++) {
    double l = clampd(rnd(iscale * (x[i] - min)), 0, nmax);
    L[i] = to_u8(l);
    double diff = scale * l + min - x[i];
    diff = diff * diff;
    best += weights[i] * diff;
  }
  if (nstep < 1) {
    *the_min = F32(-min);
    return scale;
  }
  for (int is = 0; is <= nstep; is++) {
    iscale = (rmin + rdelta * is + nmax) / (max - min);
    double sumL = 0, sumL2 = 0, sumXL = 0;
    for (int i = 0; i < n; i++) {
      double l = clampd(rnd(iscale * (x[i] - min)), 0, nmax);
      Laux[i] = to_u8(l);
      double w = weights[i];
      sumL += w * l;
      sumL2 += w * l * l;
      sumXL += w * l * x[i];
    }
    double D = sumW * sumL2 - sumL * sumL;
    if (D > 0) {
      double thisScale = (sumW * sumXL - sumX * sumL) / D;
      double thisMin = (sumL2 * sumX - sumL * sumXL) / D;
      if (thisMin > 0) {
        thisMin = 0;
        thisScale = sumXL / sumL2;
      }
      double cur = 0;
      for (int i = 0; i < n; i++) {
        double diff = thisScale * Laux[i] + thisMin - x[i];
        diff = diff * diff;
        cur += weights[i] * diff;
      }
      if (cur < best) {
        for (int i = 0; i < n; i++) L[i] = Laux[i];
        best = cur;
        scale = thisScale;
        min = thisMin;
      }
    }
  }
  *the_min = F32(-min);
  return scale;
}

/* Packs eight 6-bit (scale, min) pairs into the 12 scale bytes of a K-quant
 * block (quant.js:497-505, 558-565). */
static void pack_scales_k4(uint8_t* sc, const uint8_t* ls, const uint8_t* lm) {
  for (int j = 0; j < 8; j++) {
    if (j < 4) {
      sc[j] = ls[j];
      sc[j + 4] = lm[j];
    } else {
      sc[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
      sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
      sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
    }
  }
}

/* Q5_K (quant.js:478-534): make_qkx2_quants per sub-block of 32 with weights
 * av_x + |x|, 6-bit scales and mins, 5-bit values split into qs and qh. */
static void quant_q5_k(const float* x, int64_t n, uint8_t* out) {
  int64_t nb = n >> 8;
  uint8_t L[256], Laux[32], ls[8], lm[8];
  float weights[32], mins[8], scales[8], tm;
  memset(out, 0, (size_t)nb * 176);
  for (int64_t b = 0; b < nb; b++) {
    const float* xb = x + b * 256;
    uint8_t* B = out + b * 176;
    double maxScale = 0, maxMin = 0;
    for (int j = 0; j < 8; j++) {
      double sumX2 = 0;
      for (int l = 0; l < 32; l++) {
        double v = xb[j * 32 + l];
        sumX2 += v * v;
      }
      double avX = sqrt(sumX2 / 32);
      for (int l = 0; l < 32; l++) weights[l] = F32(avX + fabs((double)xb[j * 32 + l]));
      scales[j] = F32(make_qkx2_quants(32, 31, xb + j * 32, weights, L + j * 32, &tm, Laux, -0.5, 0.1, 15));
      mins[j] = tm;
      if (scales[j] > maxScale) maxScale = scales[j];
      if (mins[j] > maxMin) maxMin = mins[j];
    }
    double invScale = maxScale > 0 ? 63 / maxScale : 0;
    double invMin = maxMin > 0 ? 63 / maxMin : 0;
    for (int j = 0; j < 8; j++) {
      double a = rnd(invScale * scales[j]), c = rnd(invMin * mins[j]);
      ls[j] = to_u8(a < 63 ? a : (a != a ? a : 63));
      lm[j] = to_u8(c < 63 ? c : (c != c ? c : 63));
    }
    pack_scales_k4(B + 4, ls, lm);
    uint16_t dh = oq_fp32_to_fp16(maxScale / 63), dhm = oq_fp32_to_fp16(maxMin / 63);
    put_h(B, dh);
    put_h(B + 2, dhm);
    double d = oq_fp16_to_fp32(dh), dmin = oq_fp16_to_fp32(dhm);
    for (int j = 0; j < 8; j++) {
      int sc, m;
      scale_min_k4(j, B + 4, &sc, &m);
      double dd = d * sc, dm = dmin * m;
      if (dd == 0 || dd != dd) continue;
      for (int l = 0; l < 32; l++) {
        double v = xb[j * 32 + l];
        L[j * 32 + l] = to_u8(clampd(rnd((v + dm) / dd), 0, 31));
      }
    }
    int m1 = 1, m2 = 2;
    for (int jj = 0; jj < 256; jj += 64) {
      for (int l = 0; l < 32; l++) {
        int l1 = L[jj + l];
        if (l1 > 15) { l1 -= 16; B[16 + l] |= (uint8_t)m1; }
        int l2 = L[jj + l + 32];
        if (l2 > 15) { l2 -= 16; B[16 + l] |= (uint8_t)m2; }
        B[48 + (jj >> 1) + l] = (uint8_t)(l1 | (l2 << 4));
      }
      m1 <<= 2;
      m2 <<= 2;
    }
  }
}

/* Q4_K (quant.js:544-578): closed-form min/max per sub-block of 32, 15 levels,
 * 6-bit scales and mins against the unrounded super-block d and dmin. */
static void quant_q4_k(const float* x, int64_t n, uint8_t* out) {
  int64_t nb = n >> 8;
  float mins[8], scales[8];
  uint8_t L[256], ls[8], lm[8];
  memset(out, 0, (size_t)nb * 144);
  for (int64_t b = 0; b < nb; b++) {
    const float* xb = x + b * 256;
    uint8_t* B = out + b * 144;
    double maxScale = 0, maxMin = 0;
    for (int j = 0; j < 8; j++) {
      double mn = INFINITY, mx = -INFINITY;
      for (int l = 0; l < 32; l++) {
        double v = xb[j * 32 + l];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
      }
      if (mn > 0) mn = 0;
      scales[j] = F32((mx - mn) / 15);
      mins[j] = F32(-mn);
      if (scales[j] > maxScale) maxScale = scales[j];
      if (mins[j] > maxMin) maxMin = mins[j];
    }
    double d = maxScale / 63, dm = maxMin / 63;
    put_h(B, oq_fp32_to_fp16(d));
    put_h(B + 2, oq_fp32_to_fp16(dm));
    double dq = (d != 0 && d == d) ? d : 1, dmq = (dm != 0 && dm == dm) ? dm : 1;  /* `d || 1` */
    for (int j = 0; j < 8; j++) {
      ls[j] = to_u8(clampd(rnd(scales[j] / dq), 0, 63));
      lm[j] = to_u8(clampd(rnd(fabs((double)mins[j]) / dmq), 0, 63));
    }
    pack_scales_k4(B + 4, ls, lm);
    for (int j = 0; j < 8; j++) {
      int sc, m;
      scale_min_k4(j, B + 4, &sc, &m);
      double dd = d * sc, mm = dm * m;
      for (int l = 0; l < 32; l++) {
        double v = xb[j * 32 + l];
        L[j * 32 + l] = to_u8(clampd(rnd((dd != 0 && dd == dd) ? (v + mm) / dd : 0), 0, 15));
      }
    }
    for (int j = 0; j < 256; j += 64)
      for (int l = 0; l < 32; l++) B[16 + (j >> 1) + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
  }
}

/* quantizeRow (quant.js:580-590).  Writes oq_row_bytes(type, n) bytes for
 * whole blocks (trailing elements of a partial block are dropped, as the
 * reference's n >> 5 / n >> 8 block counts do).  Returns −1 for a type
 * without a quantizer. */
int oq_quantize(int type, const float* x, int64_t n, uint8_t* out) {
  switch (type) {
    case 0: memcpy(out, x, (size_t)n * 4); return 0;
    case 1:
      for (int64_t i = 0; i < n; i++) put_h(out + 2 * i, oq_fp32_to_fp16(x[i]));
      return 0;
    case 8: quant_q8_0(x, n, out); return 0;
    case 12: quant_q4_k(x, n, out); return 0;
    case 13: quant_q5_k(x, n, out); return 0;
    case 14: quant_q6_k(x, n, out); return 0;
    default: return -1;
  }
}
