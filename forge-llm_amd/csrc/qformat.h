// GGML block formats of QuantLinear weights on the device (quant.js:42-56,
// 102-320 of forge-llm): element decode, bit-exact with the reference's
// dequantize, and wave-cooperative row dot products for the matvecs.
//
// A weight matrix [N, K] is N rows of row_bytes(type, K) bytes (K a whole
// number of blocks).  Types: 0 F32, 1 F16, 2 Q4_0 and 6 Q5_0 (as the
// reference's generic decode reads them), 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K.
//
// Row dots accumulate in fp64 like the reference's dotQ (a JS number sum), in
// another order: per lane, the products q·x of a sub-block are summed (each
// product is exact in fp64: a ≤ 8-bit integer times an fp32 value) and the
// block's scales applied to the sums, d·Σq·x − m·Σx, then the lanes are summed
// across the wave.  Results agree with the reference to ~1e-16 relative before
// the final fp32 rounding.
#pragma once

#include <hip/hip_fp16.h>

#include "common.h"

namespace fgq {

enum : int { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14 };

__host__ __device__ constexpr int block_elems(int t) {
  return t == kF32 || t == kF16 ? 1 : (t == kQ4_0 || t == kQ5_0 || t == kQ8_0) ? 32 : 256;
}
__host__ __device__ constexpr int block_bytes(int t) {
  return t == kF32 ? 4 : t == kF16 ? 2 : t == kQ4_0 ? 18 : t == kQ5_0 ? 22 : t == kQ8_0 ? 34
       : t == kQ4_K ? 144 : t == kQ5_K ? 176 : t == kQ6_K ? 210 : 0;
}
inline bool known_type(int t) {
  return t == kF32 || t == kF16 || t == kQ4_0 || t == kQ5_0 || t == kQ8_0 || t == kQ4_K || t == kQ5_K ||
         t == kQ6_K;
}
inline int64_t row_bytes(int t, int64_t K) {
  const int be = block_elems(t);
  return (K + be - 1) / be * block_bytes(t);
}

// ── loads at 2-byte alignment (Q8_0, Q6_K, Q4_0 and Q5_0 blocks are only
//    2-byte aligned) ──────────────────────────────────────────────────────
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ uint32_t ld32a2(const uint8_t* p) {
  const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
  return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}

// IEEE half → float, exact (fp16 values are fp32 values; fp16 subnormals are
// normal in fp32).  Matches fp16Table (quant.js:71-84) for every non-NaN.
__device__ __forceinline__ float h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

// getScaleMinK4 (quant.js:88-94) over the 12 scale bytes held in three words.
__device__ __forceinline__ uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int k) {
  const uint32_t w = k < 4 ? s0 : k < 8 ? s1 : s2;
  return (w >> (8 * (k & 3))) & 0xffu;
}
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int& sc, int& m) {
  if (j < 4) {
    sc = (int)(sbyte(s0, s1, s2, j) & 63);
    m = (int)(sbyte(s0, s1, s2, j + 4) & 63);
  } else {
    sc = (int)((sbyte(s0, s1, s2, j + 4) & 0xF) | ((sbyte(s0, s1, s2, j - 4) >> 6) << 4));
    m = (int)((sbyte(s0, s1, s2, j + 4) >> 4) | ((sbyte(s0, s1, s2, j) >> 6) << 4));
  }
}

// ── element decode (dequantize, quant.js:102-199), bit-exact ──────────────
// Element i of a row: the reference's fp64 expression, rounded once to fp32.
template <int QT>
__device__ __forceinline__ float dq_elem(const uint8_t* __restrict__ row, int i) {
#pragma clang fp contract(off)
  if constexpr (QT == kF32) {
    return reinterpret_cast<const float*>(row)[i];
  } else if constexpr (QT == kF16) {
    return h2f(ld16(row + 2 * i));
  } else if constexpr (QT == kQ8_0) {
    const uint8_t* B = row + 34 * (i >> 5);
    return (float)((double)(int8_t)B[2 + (i & 31)] * (double)h2f(ld16(B)));
  } else if constexpr (QT == kQ4_K || QT == kQ5_K) {
    constexpr int BB = QT == kQ4_K ? 144 : 176;
    const uint8_t* B = row + BB * (i >> 8);
    const int j = i & 255, c = j >> 6, hi = (j >> 5) & 1, l = j & 31;
    const uint8_t* qs = B + (QT == kQ4_K ? 16 : 48);
    int q = hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 0xF);
    if constexpr (QT == kQ5_K) {
      if (B[16 + l] & (1 << (2 * c + hi))) q += 16;
    }
    const uint32_t s0 = ld32a2(B + 4), s1 = ld32a2(B + 8), s2 = ld32a2(B + 12);
    int sc, m;
    scale_min_k4(2 * c + hi, s0, s1, s2, sc, m);
    const double d = h2f(ld16(B)), dmin = h2f(ld16(B + 2));
    return (float)((d * sc) * q - dmin * m);
  } else if constexpr (QT == kQ6_K) {
    const uint8_t* B = row + 210 * (i >> 8);
    const int j = i & 255, n2 = j & 128, g = (j >> 5) & 3, l = j & 31, is = l >> 4;
    const int qlb = B[(n2 >> 1) + l + ((g & 1) ? 32 : 0)];
    const int nib = g < 2 ? (qlb & 0xF) : (qlb >> 4);
    const int hb = (B[128 + (n2 >> 2) + l] >> (2 * g)) & 3;
    const int q = (nib | (hb << 4)) - 32;
    const int sc = (int8_t)B[192 + (n2 >> 4) + is + 2 * g];
    const double d = h2f(ld16(B + 208));
    return (float)((d * sc) * q);
  } else {  // Q4_0 / Q5_0 as the reference's generic branch (quant.js:184-196)
    constexpr int BB = QT == kQ4_0 ? 18 : 22;
    const uint8_t* B = row + BB * (i >> 5);
    const int j = i & 31, u = B[2 + (j >> 1)];
    const int q = (j & 1) ? (u >> 4) : (u & 0xF);
    return (float)((double)(QT == kQ4_0 ? q - 8 : q) * (double)h2f(ld16(B)));
  }
}

// ── row dot products, R rows per wave, x in LDS (fp32) ─────────────────────
// acc[r] += this lane's part of row r · x; the caller sums acc over the wave.
// K is a whole number of blocks; rows[r] points at row r's first block.

template <int R>
__device__ __forceinline__ void dot_f32(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K) {
  const int lane = threadIdx.x & 63;
  if ((K & 3) == 0) {
    for (int k = lane; k < (K >> 2); k += 64) {
      const float4 xv = reinterpret_cast<const float4*>(xs)[k];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float4 w = reinterpret_cast<const float4*>(rows[r])[k];
        acc[r] += (double)w.x * xv.x;
        acc[r] += (double)w.y * xv.y;
        acc[r] += (double)w.z * xv.z;
        acc[r] += (double)w.w * xv.w;
      }
    }
  } else {
    for (int k = lane; k < K; k += 64) {
      const double xv = xs[k];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += (double)reinterpret_cast<const float*>(rows[r])[k] * xv;
    }
  }
}

template <int R>
__device__ __forceinline__ void dot_f16(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K) {
  const int lane = threadIdx.x & 63;
  if ((K & 7) == 0) {
    for (int k = lane; k < (K >> 3); k += 64) {
      const float4 x0 = reinterpret_cast<const float4*>(xs)[2 * k];
      const float4 x1 = reinterpret_cast<const float4*>(xs)[2 * k + 1];
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint4 h = reinterpret_cast<const uint4*>(rows[r])[k];
        const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r] += (double)h2f((hw[i >> 1] >> (16 * (i & 1))) & 0xffffu) * xv[i];
      }
    }
  } else {
    for (int k = lane; k < K; k += 64) {
      const double xv = xs[k];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += (double)h2f(ld16(rows[r] + 2 * k)) * xv;
    }
  }
}

// Q8_0: 8 lanes per 32-element block, 4 elements (one dword of qs) per lane.
template <int R>
__device__ __forceinline__ void dot_q8_0(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K) {
  const int lane = threadIdx.x & 63, sub = lane & 7;
  const int nb = K >> 5;
  for (int b = lane >> 3; b < nb; b += 8) {
    const float4 xv = reinterpret_cast<const float4*>(xs + 32 * b)[sub];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + 34 * b;
      const uint32_t q = ld32a2(B + 2 + 4 * sub);
      const double d = h2f(ld16(B));
      double a = (double)(int8_t)(q & 0xff) * xv.x;
      a += (double)(int8_t)((q >> 8) & 0xff) * xv.y;
      a += (double)(int8_t)((q >> 16) & 0xff) * xv.z;
      a += (double)(int8_t)(q >> 24) * xv.w;
      acc[r] += a * d;
    }
  }
}

// Q4_0 / Q5_0 (generic branch of dotQ: dot of the fp32-rounded decoded values).
template <int QT, int R>
__device__ __forceinline__ void dot_q4_0(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K) {
  constexpr int BB = QT == kQ4_0 ? 18 : 22;
  const int lane = threadIdx.x & 63, sub = lane & 7;
  const int nb = K >> 5;
  for (int b = lane >> 3; b < nb; b += 8) {
    const float4 xv = reinterpret_cast<const float4*>(xs + 32 * b)[sub];
    const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + BB * b;
      const uint32_t u = ld16(B + 2 + 2 * sub);
      const double d = h2f(ld16(B));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int by = (u >> (8 * (i >> 1))) & 0xff;
        const int q = (i & 1) ? (by >> 4) : (by & 0xF);
        const float w = (float)((double)(QT == kQ4_0 ? q - 8 : q) * d);
        acc[r] += (double)w * xa[i];
      }
    }
  }
}

// Q4_K / Q5_K: 16 lanes per 256-element block.  Lane `sub` takes qs bytes
// [8 sub, 8 sub + 8): elements 64c + l0 + i (low nibbles) and 64c + 32 + l0 + i
// (high nibbles), c = sub / 4, l0 = 8 (sub % 4), sub-blocks 2c and 2c + 1.
template <int QT, int R>
__device__ __forceinline__ void dot_k4(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K) {
  constexpr int BB = QT == kQ4_K ? 144 : 176;
  constexpr int QS = QT == kQ4_K ? 16 : 48;
  const int lane = threadIdx.x & 63, sub = lane & 15, c = sub >> 2, l0 = (sub & 3) * 8;
  const int nb = K >> 8;
  for (int b = lane >> 4; b < nb; b += 4) {
    const float* xb = xs + 256 * b + 64 * c + l0;
    const float4 a0 = reinterpret_cast<const float4*>(xb)[0], a1 = reinterpret_cast<const float4*>(xb)[1];
    const float4 h0 = reinterpret_cast<const float4*>(xb + 32)[0], h1 = reinterpret_cast<const float4*>(xb + 32)[1];
    const float xl[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float xh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    double sxl = 0.0, sxh = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sxl += xl[i];
      sxh += xh[i];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + BB * b;
      const uint4 hd = *reinterpret_cast<const uint4*>(B);  // d, dmin, scales[12]
      const uint2 q = *reinterpret_cast<const uint2*>(B + QS + 8 * sub);
      uint2 qh = make_uint2(0, 0);
      if constexpr (QT == kQ5_K) qh = *reinterpret_cast<const uint2*>(B + 16 + l0);
      int sc1, m1, sc2, m2;
      scale_min_k4(2 * c, hd.y, hd.z, hd.w, sc1, m1);
      scale_min_k4(2 * c + 1, hd.y, hd.z, hd.w, sc2, m2);
      const double d = h2f(hd.x & 0xffffu), dmin = h2f(hd.x >> 16);
      double al = 0.0, ah = 0.0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t by = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xffu;
        int lo = (int)(by & 0xF), hi = (int)(by >> 4);
        if constexpr (QT == kQ5_K) {
          const uint32_t hb = ((i < 4 ? qh.x : qh.y) >> (8 * (i & 3))) & 0xffu;
          lo += (hb >> (2 * c)) & 1 ? 16 : 0;
          hi += (hb >> (2 * c + 1)) & 1 ? 16 : 0;
        }
        al += (double)lo * xl[i];
        ah += (double)hi * xh[i];
      }
      acc[r] += (d * sc1) * al - (dmin * m1) * sxl + (d * sc2) * ah - (dmin * m2) * sxh;
    }
  }
}

// Q6_K: 16 lanes per 256-element block.  Lane `sub` takes half h = sub / 8 and
// l = l0 .. l0 + 3, l0 = 4 (sub % 8): elements 128h + l + 32g for g = 0..3 (the
// reference's q1..q4), scales 8h + l/16 + 2g.
template <int R>
__device__ __forceinline__ void dot_q6_k(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K) {
  const int lane = threadIdx.x & 63, sub = lane & 15, h = sub >> 3, l0 = (sub & 7) * 4, is = l0 >> 4;
  const int nb = K >> 8;
  for (int b = lane >> 4; b < nb; b += 4) {
    const float* xb = xs + 256 * b + 128 * h + l0;
    float xg[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 v = *reinterpret_cast<const float4*>(xb + 32 * g);
      xg[g][0] = v.x;
      xg[g][1] = v.y;
      xg[g][2] = v.z;
      xg[g][3] = v.w;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + 210 * b;
      const uint32_t qa = ld32a2(B + 64 * h + l0), qb = ld32a2(B + 64 * h + 32 + l0);
      const uint32_t qh = ld32a2(B + 128 + 32 * h + l0);
      const uint32_t s01 = ld32a2(B + 192 + 8 * h), s23 = ld32a2(B + 196 + 8 * h);
      const double d = h2f(ld16(B + 208));
      double a[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ba = (qa >> (8 * i)) & 0xff, bb = (qb >> (8 * i)) & 0xff, hh = (qh >> (8 * i)) & 0xff;
        a[0] += (double)(((ba & 0xF) | ((hh & 3) << 4)) - 32) * xg[0][i];
        a[1] += (double)(((bb & 0xF) | (((hh >> 2) & 3) << 4)) - 32) * xg[1][i];
        a[2] += (double)(((ba >> 4) | (((hh >> 4) & 3) << 4)) - 32) * xg[2][i];
        a[3] += (double)(((bb >> 4) | (((hh >> 6) & 3) << 4)) - 32) * xg[3][i];
      }
      // scale bytes 8h + is + 2g, g = 0..3: bytes is, is+2 of s01 and is, is+2 of s23
      const double sg0 = (int8_t)((s01 >> (8 * is)) & 0xff), sg1 = (int8_t)((s01 >> (8 * (is + 2))) & 0xff);
      const double sg2 = (int8_t)((s23 >> (8 * is)) & 0xff), sg3 = (int8_t)((s23 >> (8 * (is + 2))) & 0xff);
      acc[r] += d * (sg0 * a[0] + sg1 * a[1] + sg2 * a[2] + sg3 * a[3]);
    }
  }
}

template <int QT, int R>
__device__ __forceinline__ void qrows_dot(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K) {
  if constexpr (QT == kF32) dot_f32<R>(acc, rows, xs, K);
  else if constexpr (QT == kF16) dot_f16<R>(acc, rows, xs, K);
  else if constexpr (QT == kQ8_0) dot_q8_0<R>(acc, rows, xs, K);
  else if constexpr (QT == kQ4_0 || QT == kQ5_0) dot_q4_0<QT, R>(acc, rows, xs, K);
  else if constexpr (QT == kQ4_K || QT == kQ5_K) dot_k4<QT, R>(acc, rows, xs, K);
  else dot_q6_k<R>(acc, rows, xs, K);
}

}  // namespace fgq

// Expands the statement(s) for the runtime type t with a constexpr QT, inside
// a function returning int; an unknown type is an argument error.
#define FGQ_DISPATCH(t, ...)                                                           \
  switch (t) {                                                                       \
    case fgq::kF32: { constexpr int QT = fgq::kF32; __VA_ARGS__; } break;                      \
    case fgq::kF16: { constexpr int QT = fgq::kF16; __VA_ARGS__; } break;                      \
    case fgq::kQ4_0: { constexpr int QT = fgq::kQ4_0; __VA_ARGS__; } break;                    \
    case fgq::kQ5_0: { constexpr int QT = fgq::kQ5_0; __VA_ARGS__; } break;                    \
    case fgq::kQ8_0: { constexpr int QT = fgq::kQ8_0; __VA_ARGS__; } break;                    \
    case fgq::kQ4_K: { constexpr int QT = fgq::kQ4_K; __VA_ARGS__; } break;                    \
    case fgq::kQ5_K: { constexpr int QT = fgq::kQ5_K; __VA_ARGS__; } break;                    \
    case fgq::kQ6_K: { constexpr int QT = fgq::kQ6_K; __VA_ARGS__; } break;                    \
    default: return fg::set_error(FG_ERR_ARG, "unsupported ggml type %d", (int)(t)); \
  }
