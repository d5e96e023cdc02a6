// GGML block formats of QuantLinear weights on the device (quant.js:42-56,
// 102-320 of forge-llm): element decode, bit-exact with the reference's
// dequantize, and wave-cooperative row dot products for the matvecs.
//
// A weight matrix [N, K] is N rows of row_bytes(type, K) bytes (K a whole
// number of blocks).  Types: 0 F32, 1 F16, 2 Q4_0 and 6 Q5_0 (as the
// reference's generic decode reads them), 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K.
//
// Row dots: the reference's dotQ sums in fp64 (a JS number).  Here f32 and
// f16 rows sum in fp64; quantized rows sum the integer-times-x products of a
// lane's sub-block (8 to 16 of them) in fp32, then apply the block scales and
// sum across blocks and lanes in fp64: d·Σq·x − m·Σx.  The fp32 partial sums
// keep the unpacking (v_cvt_f32_ubyte of masked bytes) and the multiply-adds
// at full VALU rate, which the HBM stream of 4.5-8.5 bits per weight needs;
// fp64 conversions per element would bound the kernel at a fifth of HBM
// bandwidth.  Their rounding (~1e-7 of a partial) keeps outputs well inside
// the forward tolerance (1e-5 relative L2).
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

// The four bytes of w as floats (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ void bytes_f32(uint32_t w, float (&f)[4]) {
  f[0] = (float)(w & 0xffu);
  f[1] = (float)((w >> 8) & 0xffu);
  f[2] = (float)((w >> 16) & 0xffu);
  f[3] = (float)(w >> 24);
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
// acc[r] += this lane's part of row r · x; the caller sums acc over the wave
// (and over the `nparts` waves that split the row: wave `part` takes every
// nparts-th group of blocks).  K is a whole number of blocks; rows[r] points
// at row r's first block.

template <int R>
__device__ __forceinline__ void dot_f32(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K,
                                         int part = 0, int nparts = 1) {
  const int lane = threadIdx.x & 63;
  if ((K & 3) == 0) {
    for (int k = lane + 64 * part; k < (K >> 2); k += 64 * nparts) {
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
    for (int k = lane + 64 * part; k < K; k += 64 * nparts) {
      const double xv = xs[k];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += (double)reinterpret_cast<const float*>(rows[r])[k] * xv;
    }
  }
}

template <int R>
__device__ __forceinline__ void dot_f16(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K,
                                         int part = 0, int nparts = 1) {
  const int lane = threadIdx.x & 63;
  if ((K & 7) == 0) {
    for (int k = lane + 64 * part; k < (K >> 3); k += 64 * nparts) {
      const float4 x0 = reinterpret_cast<const float4*>(xs)[2 * k];
      const float4 x1 = reinterpret_cast<const float4*>(xs)[2 * k + 1];
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint4 h = reinterpret_cast<const uint4*>(rows[r])[k];
        const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) a = fmaf(h2f((hw[i >> 1] >> (16 * (i & 1))) & 0xffffu), xv[i], a);
        acc[r] += (double)a;
      }
    }
  } else {
    for (int k = lane + 64 * part; k < K; k += 64 * nparts) {
      const double xv = xs[k];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += (double)h2f(ld16(rows[r] + 2 * k)) * xv;
    }
  }
}

// Q8_0: 8 lanes per 32-element block, 4 elements (one dword of qs) per lane.
template <int R>
__device__ __forceinline__ void dot_q8_0(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K,
                                         int part = 0, int nparts = 1) {
  const int lane = threadIdx.x & 63, sub = lane & 7;
  const int nb = K >> 5;
  for (int b = (lane >> 3) + 8 * part; b < nb; b += 8 * nparts) {
    const float4 xv = reinterpret_cast<const float4*>(xs + 32 * b)[sub];
    const float sx = (xv.x + xv.y) + (xv.z + xv.w);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + 34 * b;
      // int8 q = (q ^ 0x80) − 128: unsigned bytes convert at full rate
      float u[4];
      bytes_f32(ld32a2(B + 2 + 4 * sub) ^ 0x80808080u, u);
      const double d = h2f(ld16(B));
      float a = u[0] * xv.x;
      a = fmaf(u[1], xv.y, a);
      a = fmaf(u[2], xv.z, a);
      a = fmaf(u[3], xv.w, a);
      acc[r] += ((double)a - 128.0 * (double)sx) * d;
    }
  }
}

// Q4_0 / Q5_0 (generic branch of dotQ: dot of the fp32-rounded decoded values).
template <int QT, int R>
__device__ __forceinline__ void dot_q4_0(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K,
                                         int part = 0, int nparts = 1) {
  constexpr int BB = QT == kQ4_0 ? 18 : 22;
  const int lane = threadIdx.x & 63, sub = lane & 7;
  const int nb = K >> 5;
  for (int b = (lane >> 3) + 8 * part; b < nb; b += 8 * nparts) {
    const float4 xv = reinterpret_cast<const float4*>(xs + 32 * b)[sub];
    const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + BB * b;
      const uint32_t u = ld16(B + 2 + 2 * sub);
      const double d = h2f(ld16(B));
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int by = (u >> (8 * (i >> 1))) & 0xff;
        const int q = (i & 1) ? (by >> 4) : (by & 0xF);
        a = fmaf((float)(QT == kQ4_0 ? q - 8 : q), xa[i], a);
      }
      acc[r] += (double)a * d;  // the decoded weights (q − 8)·d are exact in fp32
    }
  }
}

// Q4_K / Q5_K: 8 lanes per 256-element block.  Lane `s` takes qs bytes
// [16 s, 16 s + 16): elements 64c + l0 + i (low nibbles) and 64c + 32 + l0 + i
// (high nibbles), i < 16, c = s / 2, l0 = 16 (s % 2), sub-blocks 2c and 2c + 1.
template <int QT, int R>
__device__ __forceinline__ void dot_k4(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K,
                                         int part = 0, int nparts = 1) {
  constexpr int BB = QT == kQ4_K ? 144 : 176;
  constexpr int QS = QT == kQ4_K ? 16 : 48;
  const int lane = threadIdx.x & 63, s = lane & 7, c = s >> 1, l0 = (s & 1) * 16;
  const int nb = K >> 8;
  for (int b = (lane >> 3) + 8 * part; b < nb; b += 8 * nparts) {
    const float* xb = xs + 256 * b + 64 * c + l0;
    float xl[16], xh[16];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 a = reinterpret_cast<const float4*>(xb)[v], h = reinterpret_cast<const float4*>(xb + 32)[v];
      xl[4 * v] = a.x; xl[4 * v + 1] = a.y; xl[4 * v + 2] = a.z; xl[4 * v + 3] = a.w;
      xh[4 * v] = h.x; xh[4 * v + 1] = h.y; xh[4 * v + 2] = h.z; xh[4 * v + 3] = h.w;
    }
    float sxl = 0.f, sxh = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sxl += xl[i];
      sxh += xh[i];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + BB * b;
      const uint4 hd = *reinterpret_cast<const uint4*>(B);  // d, dmin, scales[12]
      const uint4 q = *reinterpret_cast<const uint4*>(B + QS + 16 * s);
      uint4 qh = make_uint4(0, 0, 0, 0);
      if constexpr (QT == kQ5_K) qh = *reinterpret_cast<const uint4*>(B + 16 + l0);
      int sc1, m1, sc2, m2;
      scale_min_k4(2 * c, hd.y, hd.z, hd.w, sc1, m1);
      scale_min_k4(2 * c + 1, hd.y, hd.z, hd.w, sc2, m2);
      const double d = h2f(hd.x & 0xffffu), dmin = h2f(hd.x >> 16);
      const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
      const uint32_t hw[4] = {qh.x, qh.y, qh.z, qh.w};
      float al = 0.f, ah = 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        uint32_t lo = qw[v] & 0x0F0F0F0Fu, hi = (qw[v] >> 4) & 0x0F0F0F0Fu;
        if constexpr (QT == kQ5_K) {  // the fifth bit: bit 2c (low) / 2c+1 (high) of qh[l]
          lo |= ((hw[v] >> (2 * c)) & 0x01010101u) << 4;
          hi |= ((hw[v] >> (2 * c + 1)) & 0x01010101u) << 4;
        }
        float fl[4], fh[4];
        bytes_f32(lo, fl);
        bytes_f32(hi, fh);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          al = fmaf(fl[i], xl[4 * v + i], al);
          ah = fmaf(fh[i], xh[4 * v + i], ah);
        }
      }
      acc[r] += (d * sc1) * (double)al - (dmin * m1) * (double)sxl + (d * sc2) * (double)ah -
                (dmin * m2) * (double)sxh;
    }
  }
}

// Q6_K: 16 lanes per 256-element block.  Lane `sub` takes half h = sub / 8 and
// l = l0 .. l0 + 3, l0 = 4 (sub % 8): elements 128h + l + 32g for g = 0..3 (the
// reference's q1..q4), scales 8h + l/16 + 2g.
template <int R>
__device__ __forceinline__ void dot_q6_k(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K,
                                         int part = 0, int nparts = 1) {
  const int lane = threadIdx.x & 63, sub = lane & 15, h = sub >> 3, l0 = (sub & 7) * 4, is = l0 >> 4;
  const int nb = K >> 8;
  for (int b = (lane >> 4) + 4 * part; b < nb; b += 4 * nparts) {
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
    float sg[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) sg[g] = (xg[g][0] + xg[g][1]) + (xg[g][2] + xg[g][3]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* B = rows[r] + 210 * b;
      const uint32_t qa = ld32a2(B + 64 * h + l0), qb = ld32a2(B + 64 * h + 32 + l0);
      const uint32_t qh = ld32a2(B + 128 + 32 * h + l0);
      const uint32_t s01 = ld32a2(B + 192 + 8 * h), s23 = ld32a2(B + 196 + 8 * h);
      const double d = h2f(ld16(B + 208));
      // 6-bit values q + 32 in four bytes per group: low / high nibbles of ql
      // with two bits of qh above them
      const uint32_t v[4] = {(qa & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4),
                             (qb & 0x0F0F0F0Fu) | (((qh >> 2) & 0x03030303u) << 4),
                             ((qa >> 4) & 0x0F0F0F0Fu) | (((qh >> 4) & 0x03030303u) << 4),
                             ((qb >> 4) & 0x0F0F0F0Fu) | (((qh >> 6) & 0x03030303u) << 4)};
      double a[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float f[4];
        bytes_f32(v[g], f);
        float t = f[0] * xg[g][0];
        t = fmaf(f[1], xg[g][1], t);
        t = fmaf(f[2], xg[g][2], t);
        t = fmaf(f[3], xg[g][3], t);
        a[g] = (double)t - 32.0 * (double)sg[g];
      }
      // scale bytes 8h + is + 2g, g = 0..3: bytes is, is+2 of s01 and is, is+2 of s23
      const double sg0 = (int8_t)((s01 >> (8 * is)) & 0xff), sg1 = (int8_t)((s01 >> (8 * (is + 2))) & 0xff);
      const double sg2 = (int8_t)((s23 >> (8 * is)) & 0xff), sg3 = (int8_t)((s23 >> (8 * (is + 2))) & 0xff);
      acc[r] += d * (sg0 * a[0] + sg1 * a[1] + sg2 * a[2] + sg3 * a[3]);
    }
  }
}

template <int QT, int R>
__device__ __forceinline__ void qrows_dot(double (&acc)[R], const uint8_t* const (&rows)[R], const float* xs, int K,
                                          int part = 0, int nparts = 1) {
  if constexpr (QT == kF32) dot_f32<R>(acc, rows, xs, K, part, nparts);
  else if constexpr (QT == kF16) dot_f16<R>(acc, rows, xs, K, part, nparts);
  else if constexpr (QT == kQ8_0) dot_q8_0<R>(acc, rows, xs, K, part, nparts);
  else if constexpr (QT == kQ4_0 || QT == kQ5_0) dot_q4_0<QT, R>(acc, rows, xs, K, part, nparts);
  else if constexpr (QT == kQ4_K || QT == kQ5_K) dot_k4<QT, R>(acc, rows, xs, K, part, nparts);
  else dot_q6_k<R>(acc, rows, xs, K, part, nparts);
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
