// Quantized weights on the device (src/L3/quant.js, src/L4/nn.js of forge-llm):
//
//   fg_qmatvec     y[n] = fp32(dotQ(W row n, x))   QuantLinear.forward (nn.js:27-33)
//   fg_dequantize  out = dequantize(q)             quant.js:102-199, bit-exact
//   fg_quantize    q = quantizeRow(x)              quant.js:322-590, bit-exact
//
// The matvec is HBM-bound (a weight is read once per call): one wave per two
// rows, x staged once per workgroup in LDS, per-format lane mappings from
// qformat.h.  Decoding is exact integer/fp16 work; sums are fp64.
//
// The quantizers restate the reference's scalar algorithms (closed-form
// Q8_0 and Q4_K, the make_qx_quants / make_qkx2_quants searches of Q6_K and
// Q5_K) with the reference's arithmetic: fp64 intermediates, fp32 stores for
// its Float32Array temporaries, typed-array wrap-around for its byte stores,
// Math.round ties towards +infinity, no fused multiply-adds.  One thread
// quantizes one block, so the search loops run in the reference's order and
// the bytes are identical to it.  Quantization is a one-time load step, not a
// per-token cost.
#include "common.h"
#include "qformat.h"

#include <math.h>

namespace {

using namespace fgq;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// ── matvec ────────────────────────────────────────────────────────────────
// Each wave takes R rows at a time over all of K; workgroups stride over the
// row groups, and there are only a few per CU, so the x vector staged in LDS
// (X_LDS; beyond 64 KiB it is read from global memory) serves many rows.
template <int QT, int R, bool X_LDS, typename OutT>
__global__ void __launch_bounds__(kThreads) qmatvec_kernel(OutT* __restrict__ y, const uint8_t* __restrict__ W,
                                                           const float* __restrict__ x, int N, int K, int64_t rb) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  const float* xv = x;
  if constexpr (X_LDS) {
    for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = x[i];
    __syncthreads();
    xv = xs;
  }
  const int groups = (N + R - 1) / R;
  for (int g = blockIdx.x * kWaves + (threadIdx.x >> 6); g < groups; g += gridDim.x * kWaves) {
    const int r0 = g * R;
    const uint8_t* rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = W + (int64_t)(r0 + r < N ? r0 + r : N - 1) * rb;
    double acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0;
    qrows_dot<QT, R>(acc, rows, xv, K);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const double s = fg_wave_sum_d(acc[r]);
      if ((threadIdx.x & 63) == 0 && r0 + r < N) y[r0 + r] = (OutT)s;
    }
  }
}

// SwiGLU activation of nn.js:56-66: h = fp32((g / (1 + e^−g)) · u) in fp64.
__global__ void __launch_bounds__(kThreads) silu_mul_kernel(float* __restrict__ h, const float* __restrict__ g,
                                                            const float* __restrict__ u, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const double gv = g[i];
    h[i] = (float)((gv / (1.0 + exp(-gv))) * (double)u[i]);
  }
}

// ── dequantize ────────────────────────────────────────────────────────────
template <int QT>
__global__ void __launch_bounds__(kThreads) dequant_kernel(float* __restrict__ out, const uint8_t* __restrict__ q,
                                                           int64_t n) {
  constexpr int BE = block_elems(QT), BB = block_bytes(QT);
  for (int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    out[i] = dq_elem<QT>(q + (i / BE) * BB, (int)(i % BE));
}

// ── quantizers (quant.js:322-590) ──────────────────────────────────────────
#pragma clang fp contract(off)

// Math.round: nearest integer, ties towards +infinity.
__device__ double js_round(double v) {
  if (!isfinite(v)) return v;
  const double f = floor(v);
  return (v - f) >= 0.5 ? f + 1.0 : f;
}
// nearest_int (quant.js:322): ties away from zero.
__device__ double rnd(double v) { return v < 0 ? -js_round(-v) : js_round(v); }
__device__ double clampd(double v, double a, double b) { return v < a ? a : v > b ? b : v; }
// A store into a Uint8Array / Int8Array: ToUint8 (NaN, ±inf → 0).
__device__ uint8_t to_u8(double v) {
  if (!isfinite(v)) return 0;
  double m = fmod(trunc(v), 256.0);
  if (m < 0) m += 256.0;
  return (uint8_t)m;
}
__device__ double h2d(uint32_t h) { return (double)h2f(h); }

// fp32ToFp16 (special.js:151-168) of an fp64 value.
__device__ uint32_t to_half(double x) {
  if (!isfinite(x)) return x > 0 ? 0x7c00u : x < 0 ? 0xfc00u : 0x7e00u;
  const uint32_t s = x < 0 ? 0x8000u : 0u;
  x = fabs(x);
  if (x < 6.103515625e-5) return s | ((uint32_t)(int64_t)js_round(x * 16777216.0) & 0x3ffu);
  int e = 0;
  while (x >= 2) { x /= 2; e++; }
  while (x < 1) { x *= 2; e--; }
  int m = (int)js_round((x - 1) * 1024);
  if (m == 1024) { e++; m = 0; }
  const int ex = e + 15;
  if (ex >= 31) return s | 0x7c00u;
  return s | ((uint32_t)ex << 10) | (uint32_t)m;
}
__device__ void put_h(uint8_t* p, uint32_t h) {
  p[0] = h & 0xff;
  p[1] = (h >> 8) & 0xff;
}
__device__ void scale_min_bytes(int j, const uint8_t* q, int& sc, int& m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}
__device__ void pack_scales_k4(uint8_t* sc, const uint8_t* ls, const uint8_t* lm) {
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

// Q8_0 (quant.js:328-339).
__device__ void quant_q8_0_block(const float* xb, uint8_t* B) {
  double amax = 0;
  for (int j = 0; j < 32; j++) {
    const double v = fabs((double)xb[j]);
    if (v > amax) amax = v;
  }
  const double d = amax / 127, id = (d != 0 && d == d) ? 1 / d : 0;
  put_h(B, to_half(d));
  for (int j = 0; j < 32; j++) B[2 + j] = to_u8(clampd(rnd(xb[j] * id), -128, 127));
}

// Q4_K (quant.js:544-578).
__device__ void quant_q4_k_block(const float* xb, uint8_t* B) {
  float mins[8], scales[8];
  uint8_t L[256], ls[8], lm[8];
  for (int i = 0; i < 144; i++) B[i] = 0;
  double maxScale = 0, maxMin = 0;
  for (int j = 0; j < 8; j++) {
    double mn = INFINITY, mx = -INFINITY;
    for (int l = 0; l < 32; l++) {
      const double v = xb[j * 32 + l];
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    if (mn > 0) mn = 0;
    scales[j] = (float)((mx - mn) / 15);
    mins[j] = (float)(-mn);
    if (scales[j] > maxScale) maxScale = scales[j];
    if (mins[j] > maxMin) maxMin = mins[j];
  }
  const double d = maxScale / 63, dm = maxMin / 63;
  put_h(B, to_half(d));
  put_h(B + 2, to_half(dm));
  const double dq = (d != 0 && d == d) ? d : 1, dmq = (dm != 0 && dm == dm) ? dm : 1;
  for (int j = 0; j < 8; j++) {
    ls[j] = to_u8(clampd(rnd(scales[j] / dq), 0, 63));
    lm[j] = to_u8(clampd(rnd(fabs((double)mins[j]) / dmq), 0, 63));
  }
  pack_scales_k4(B + 4, ls, lm);
  for (int j = 0; j < 8; j++) {
    int sc, m;
    scale_min_bytes(j, B + 4, sc, m);
    const double dd = d * sc, mm = dm * m;
    for (int l = 0; l < 32; l++) {
      const double v = xb[j * 32 + l];
      L[j * 32 + l] = to_u8(clampd(rnd((dd != 0 && dd == dd) ? (v + mm) / dd : 0), 0, 15));
    }
  }
  for (int j = 0; j < 256; j += 64)
    for (int l = 0; l < 32; l++) B[16 + (j >> 1) + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
}

// make_qkx2_quants (quant.js:423-469).
__device__ double make_qkx2_quants(int n, int nmax, const float* x, const float* weights, uint8_t* L,
                                   float* the_min, uint8_t* Laux, double rmin, double rdelta, int nstep) {
  double min = x[0], max = x[0];
  double sumW = weights[0], sumX = (double)weights[0] * x[0];
  for (int i = 1; i < n; i++) {
    const double v = x[i];
    if (v < min) min = v;
    if (v > max) max = v;
    const double w = weights[i];
    sumW += w;
    sumX += w * v;
  }
  if (min > 0) min = 0;
  if (max == min) {
    for (int i = 0; i < n; i++) L[i] = 0;
    *the_min = (float)(-min);
    return 0;
  }
  double iscale = nmax / (max - min);
  double scale = 1 / iscale;
  double best = 0;
  for (int i = 0; i < n; i++) {
    const double l = clampd(rnd(iscale * (x[i] - min)), 0, nmax);
    L[i] = to_u8(l);
    double diff = scale * l + min - x[i];
    diff = diff * diff;
    best += weights[i] * diff;
  }
  if (nstep < 1) {
    *the_min = (float)(-min);
    return scale;
  }
  for (int is = 0; is <= nstep; is++) {
    iscale = (rmin + rdelta * is + nmax) / (max - min);
    double sumL = 0, sumL2 = 0, sumXL = 0;
    for (int i = 0; i < n; i++) {
      const double l = clampd(rnd(iscale * (x[i] - min)), 0, nmax);
      Laux[i] = to_u8(l);
      const double w = weights[i];
      sumL += w * l;
      sumL2 += w * l * l;
      sumXL += w * l * x[i];
    }
    const double D = sumW * sumL2 - sumL * sumL;
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
  *the_min = (float)(-min);
  return scale;
}

// Q5_K (quant.js:478-534).
__device__ void quant_q5_k_block(const float* xb, uint8_t* B) {
  uint8_t L[256], Laux[32], ls[8], lm[8];
  float weights[32], mins[8], scales[8], tm;
  for (int i = 0; i < 176; i++) B[i] = 0;
  double maxScale = 0, maxMin = 0;
  for (int j = 0; j < 8; j++) {
    double sumX2 = 0;
    for (int l = 0; l < 32; l++) {
      const double v = xb[j * 32 + l];
      sumX2 += v * v;
    }
    const double avX = sqrt(sumX2 / 32);
    for (int l = 0; l < 32; l++) weights[l] = (float)(avX + fabs((double)xb[j * 32 + l]));
    scales[j] = (float)make_qkx2_quants(32, 31, xb + j * 32, weights, L + j * 32, &tm, Laux, -0.5, 0.1, 15);
    mins[j] = tm;
    if (scales[j] > maxScale) maxScale = scales[j];
    if (mins[j] > maxMin) maxMin = mins[j];
  }
  const double invScale = maxScale > 0 ? 63 / maxScale : 0;
  const double invMin = maxMin > 0 ? 63 / maxMin : 0;
  for (int j = 0; j < 8; j++) {
    const double a = rnd(invScale * scales[j]), c = rnd(invMin * mins[j]);
    ls[j] = to_u8(a < 63 ? a : (a != a ? a : 63));
    lm[j] = to_u8(c < 63 ? c : (c != c ? c : 63));
  }
  pack_scales_k4(B + 4, ls, lm);
  const uint32_t dh = to_half(maxScale / 63), dhm = to_half(maxMin / 63);
  put_h(B, dh);
  put_h(B + 2, dhm);
  const double d = h2d(dh), dmin = h2d(dhm);
  for (int j = 0; j < 8; j++) {
    int sc, m;
    scale_min_bytes(j, B + 4, sc, m);
    const double dd = d * sc, dm = dmin * m;
    if (dd == 0 || dd != dd) continue;
    for (int l = 0; l < 32; l++) {
      const double v = xb[j * 32 + l];
      L[j * 32 + l] = to_u8(clampd(rnd((v + dm) / dd), 0, 31));
    }
  }
  int m1 = 1, m2 = 2;
  for (int jj = 0; jj < 256; jj += 64) {
    for (int l = 0; l < 32; l++) {
      int l1 = L[jj + l];
      if (l1 > 15) {
        l1 -= 16;
        B[16 + l] |= (uint8_t)m1;
      }
      int l2 = L[jj + l + 32];
      if (l2 > 15) {
        l2 -= 16;
        B[16 + l] |= (uint8_t)m2;
      }
      B[48 + (jj >> 1) + l] = (uint8_t)(l1 | (l2 << 4));
    }
    m1 <<= 2;
    m2 <<= 2;
  }
}

// make_qx_quants (quant.js:384-414).
__device__ double make_qx_quants(int n, int nmax, const float* x, int8_t* L) {
  double max = 0, amax = 0;
  for (int i = 0; i < n; i++) {
    const double ax = fabs((double)x[i]);
    if (ax > amax) {
      amax = ax;
      max = x[i];
    }
  }
  if (amax < 1e-30) {
    for (int i = 0; i < n; i++) L[i] = 0;
    return 0;
  }
  double iscale = -nmax / max;
  double sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; i++) {
    const double l = clampd(rnd(iscale * x[i]), -nmax, nmax - 1);
    L[i] = (int8_t)to_u8(l);
    const double w = (double)x[i] * x[i];
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
      const double l = clampd(rnd(iscale * x[i]), -nmax, nmax - 1);
      const double w = (double)x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; i++) L[i] = (int8_t)to_u8(clampd(rnd(iscale * x[i]), -nmax, nmax - 1));
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

// Q6_K (quant.js:346-381).
__device__ void quant_q6_k_block(const float* xb, uint8_t* B) {
  int8_t L[256];
  float scales[16];
  for (int i = 0; i < 210; i++) B[i] = 0;
  double maxScale = 0, maxAbs = 0;
  for (int ib = 0; ib < 16; ib++) {
    const double s = make_qx_quants(16, 32, xb + ib * 16, L + ib * 16);
    scales[ib] = (float)s;
    const double a = fabs(s);
    if (a > maxAbs) {
      maxAbs = a;
      maxScale = s;
    }
  }
  if (maxAbs < 1e-30) return;
  const double iscale = -128 / maxScale;
  const uint32_t dh = to_half(1 / iscale);
  put_h(B + 208, dh);
  for (int ib = 0; ib < 16; ib++) {
    const double v = rnd(iscale * scales[ib]);
    B[192 + ib] = to_u8(v < 127 ? v : (v != v ? v : 127));
  }
  const double d = h2d(dh);
  for (int j = 0; j < 16; j++) {
    const double dd = d * (int8_t)B[192 + j];
    if (dd == 0 || dd != dd) {
      for (int ii = 0; ii < 16; ii++) L[j * 16 + ii] = 32;
      continue;
    }
    for (int ii = 0; ii < 16; ii++) L[j * 16 + ii] = (int8_t)to_u8(clampd(rnd(xb[j * 16 + ii] / dd), -32, 31) + 32);
  }
  for (int j = 0; j < 256; j += 128) {
    uint8_t* p = B + (j >> 1);
    for (int l = 0; l < 32; l++) {
      const int q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF, q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
      p[l] = (uint8_t)(q1 | (q3 << 4));
      p[l + 32] = (uint8_t)(q2 | (q4 << 4));
      B[128 + (j >> 2) + l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                                        ((L[j + l + 96] >> 4) << 6));
    }
  }
}

template <int QT>
__global__ void __launch_bounds__(64) quant_kernel(uint8_t* __restrict__ out, const float* __restrict__ x,
                                                   int64_t nblocks) {
  constexpr int BE = block_elems(QT), BB = block_bytes(QT);
  for (int64_t b = blockIdx.x * (int64_t)64 + threadIdx.x; b < nblocks; b += (int64_t)gridDim.x * 64) {
    const float* xb = x + b * BE;
    uint8_t* B = out + b * BB;
    if constexpr (QT == kF32) {
      *reinterpret_cast<float*>(B) = xb[0];
    } else if constexpr (QT == kF16) {
      put_h(B, to_half(xb[0]));
    } else if constexpr (QT == kQ8_0) {
      quant_q8_0_block(xb, B);
    } else if constexpr (QT == kQ4_K) {
      quant_q4_k_block(xb, B);
    } else if constexpr (QT == kQ5_K) {
      quant_q5_k_block(xb, B);
    } else {
      quant_q6_k_block(xb, B);
    }
  }
}

unsigned grid_for(int64_t items, int per_block) {
  int64_t g = (items + per_block - 1) / per_block;
  const int64_t cap = (int64_t)(fg::device_cu_count() > 0 ? fg::device_cu_count() : 256) * 32;
  if (g > cap) g = cap;
  return (unsigned)(g < 1 ? 1 : g);
}

template <int QT, typename OutT>
int launch_qmatvec(OutT* y, const uint8_t* W, const float* x, int N, int K) {
  constexpr int R = 2;
  const int64_t rb = row_bytes(QT, K);
  const bool lds = (size_t)K * sizeof(float) <= 64 * 1024;
  // up to 8 workgroups per CU (a launch-shape sweep over rows per wave, split
  // K and workgroups per CU at the Llama-3-8B shapes found this the fastest
  // for every type; x is staged once per workgroup)
  int64_t g = ((N + R - 1) / R + kWaves - 1) / kWaves;
  const int64_t cap = (int64_t)(fg::device_cu_count() > 0 ? fg::device_cu_count() : 256) * 8;
  if (g > cap) g = cap;
  fg::KProfScope prof("qmatvec", 2.0 * N * K, (double)rb * N + 4.0 * K + 4.0 * N);
  if (lds)
    FG_LAUNCH((qmatvec_kernel<QT, R, true, OutT>), dim3((unsigned)g), dim3(kThreads), (size_t)K * sizeof(float), y,
              W, x, N, K, rb);
  else
    FG_LAUNCH((qmatvec_kernel<QT, R, false, OutT>), dim3((unsigned)g), dim3(kThreads), 0, y, W, x, N, K, rb);
  return FG_OK;
}

}  // namespace

extern "C" int fg_qrow_bytes(int type, int64_t n, int64_t* bytes) {
  FG_ARG_CHECK(bytes && n >= 0, "fg_qrow_bytes: bad arguments");
  FG_ARG_CHECK(known_type(type), "fg_qrow_bytes: unsupported ggml type %d", type);
  *bytes = row_bytes(type, n);
  return FG_OK;
}

namespace {
template <typename OutT>
int qmatvec_entry(const char* fn, int type, OutT* y, const void* W, const float* x, int N, int K) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(y && W && x && N > 0 && K > 0, "%s: bad arguments", fn);
  FG_ARG_CHECK(known_type(type), "%s: unsupported ggml type %d", fn, type);
  FG_ARG_CHECK(K % block_elems(type) == 0, "%s: K=%d is not a whole number of %d-element blocks (type %d)", fn, K,
               block_elems(type), type);
  const uint8_t* w = static_cast<const uint8_t*>(W);
  FGQ_DISPATCH(type, { return launch_qmatvec<QT, OutT>(y, w, x, N, K); });
  return FG_OK;
}
}  // namespace

extern "C" int fg_qmatvec(int type, float* y, const void* W, const float* x, int N, int K) {
  return qmatvec_entry("fg_qmatvec", type, y, W, x, N, K);
}

extern "C" int fg_qmatvec_f64(int type, double* y, const void* W, const float* x, int N, int K) {
  return qmatvec_entry("fg_qmatvec_f64", type, y, W, x, N, K);
}

extern "C" int fg_silu_mul(float* h, const float* g, const float* u, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(h && g && u && n >= 0, "fg_silu_mul: bad arguments");
  if (n == 0) return FG_OK;
  FG_LAUNCH(silu_mul_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, h, g, u, n);
  return FG_OK;
}

extern "C" int fg_dequantize(int type, float* out, const void* q, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(out && q && n >= 0, "fg_dequantize: bad arguments");
  FG_ARG_CHECK(known_type(type), "fg_dequantize: unsupported ggml type %d", type);
  FG_ARG_CHECK(n % block_elems(type) == 0, "fg_dequantize: n=%lld is not a whole number of %d-element blocks",
               (long long)n, block_elems(type));
  if (n == 0) return FG_OK;
  const uint8_t* qb = static_cast<const uint8_t*>(q);
  FGQ_DISPATCH(type, {
    FG_LAUNCH(dequant_kernel<QT>, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, out, qb, n);
  });
  return FG_OK;
}

extern "C" int fg_quantize(int type, void* out, const float* x, int64_t n) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(out && x && n >= 0, "fg_quantize: bad arguments");
  FG_ARG_CHECK(type == kF32 || type == kF16 || type == kQ8_0 || type == kQ4_K || type == kQ5_K || type == kQ6_K,
               "fg_quantize: no quantizer for ggml type %d (F32, F16, Q8_0, Q4_K, Q5_K and Q6_K have one)", type);
  FG_ARG_CHECK(n % block_elems(type) == 0, "fg_quantize: n=%lld is not a whole number of %d-element blocks",
               (long long)n, block_elems(type));
  if (n == 0) return FG_OK;
  const int64_t nb = n / block_elems(type);
  uint8_t* ob = static_cast<uint8_t*>(out);
  switch (type) {
    case kF32: FG_LAUNCH(quant_kernel<kF32>, dim3(grid_for(nb, 64)), dim3(64), 0, ob, x, nb); break;
    case kF16: FG_LAUNCH(quant_kernel<kF16>, dim3(grid_for(nb, 64)), dim3(64), 0, ob, x, nb); break;
    case kQ8_0: FG_LAUNCH(quant_kernel<kQ8_0>, dim3(grid_for(nb, 64)), dim3(64), 0, ob, x, nb); break;
    case kQ4_K: FG_LAUNCH(quant_kernel<kQ4_K>, dim3(grid_for(nb, 64)), dim3(64), 0, ob, x, nb); break;
    case kQ5_K: FG_LAUNCH(quant_kernel<kQ5_K>, dim3(grid_for(nb, 64)), dim3(64), 0, ob, x, nb); break;
    default: FG_LAUNCH(quant_kernel<kQ6_K>, dim3(grid_for(nb, 64)), dim3(64), 0, ob, x, nb); break;
  }
  return FG_OK;
}
