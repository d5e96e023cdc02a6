// Two-piece fp16 splits of power-of-two-scaled fp32 values for the fp16 MFMA
// pipes (the fp16 "hi + lo" emulation of fp32 products: Markidis et al., "NVIDIA
// Tensor Core Programmability, Performance & Precision", IPDPSW 2018; Ootomo &
// Yokota, "Recovering single precision accuracy from Tensor Cores while
// surpassing the FP32 theoretical peak performance", IJHPCA 2022).
//
// Every element x of an operand is first scaled by 2^e, e fixed per operand
// from its largest finite magnitude m so that m * 2^e lies in [2^14, 2^15)
// (xp_exponent): the scaled values fit fp16's range (max 65504) and a power of
// two changes no significand bit.  Then
//
//   hi = fp16(x * 2^e),  lo = fp16(x * 2^e - hi)      (RNE each)
//
// x * 2^e - hi is exact in fp32.  hi keeps 11 significant bits and lo the next
// 11, so |x 2^e - hi - lo| <= max(2^-22 |x 2^e|, 2^-25): elements within
// 2^-16 of m carry the 23-bit split, smaller ones an absolute error of at most
// 2^-25 in scaled units (2^-39 m; the MFMA takes fp16 subnormals exactly).
// x * y is accumulated as the three products hi*hi + hi*lo + lo*hi (each exact
// in fp32; the dropped lo*lo is below 2^-22 |x y|), in fp32 by the MFMA, and
// the sum is scaled back by 2^-(ex + ey), exactly.  Non-finite elements give
// NaN pieces (inf - inf) and are left out of m.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// hi and lo of two scaled values: one v_cvt_pk per piece, the fp16 hi values
// widened back with v_cvt_f32_f16.
__device__ __forceinline__ void split2h(float x0, float x1, int e, uint32_t& h, uint32_t& l) {
  const float a = __builtin_amdgcn_ldexpf(x0, e), b = __builtin_amdgcn_ldexpf(x1, e);
  const f16x2 hh = __builtin_convertvector((f32x2){a, b}, f16x2);
  const f16x2 ll = __builtin_convertvector((f32x2){a - (float)hh[0], b - (float)hh[1]}, f16x2);
  h = __builtin_bit_cast(uint32_t, hh);
  l = __builtin_bit_cast(uint32_t, ll);
}

__device__ __forceinline__ void split8h(const float (&x)[8], int e, u32x4& h, u32x4& l) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t a, b;
    split2h(x[2 * q], x[2 * q + 1], e, a, b);
    h[q] = a;
    l[q] = b;
  }
}

// 4 values (two packed pairs per piece).
__device__ __forceinline__ void split4h(float x0, float x1, float x2, float x3, int e, u32x2& h, u32x2& l) {
  uint32_t a, b;
  split2h(x0, x1, e, a, b);
  h[0] = a; l[0] = b;
  split2h(x2, x3, e, a, b);
  h[1] = a; l[1] = b;
}

// The exponent e of an operand from its largest finite magnitude m:
// m * 2^e in [2^14, 2^15) (m = f 2^q, f in [0.5, 1): e = 15 - q); 0 for m = 0.
__device__ __forceinline__ int exponent_of_max(float m) {
  if (!(m > 0.f)) return 0;
  return 15 - __builtin_amdgcn_frexp_expf(m);
}

// Magnitude bounds as powers of two: q with m < 2^q (kQZero for m = 0), and
// the exponent that brings values below 2^q under 2^15.  A bound built from
// several (q1 + q2 + ...) stays below -500 when any factor is zero.
constexpr int kQZero = -1000;
__device__ __forceinline__ int bound_q(float m) { return m > 0.f ? __builtin_amdgcn_frexp_expf(m) : kQZero; }
__device__ __forceinline__ int exponent_of_bound(int q) { return q < -500 ? 0 : 15 - q; }

// The largest magnitude recorded in FG_XP_PARTS = 256 partial maxima (four
// per lane, folded over the wave; wave-uniform).
__device__ __forceinline__ float fold_parts(const float* __restrict__ parts) {
  const float4 v = *reinterpret_cast<const float4*>(parts + (threadIdx.x & 63) * 4);
  float m = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, m)));
}

// An 8-wide MFMA operand fragment as its fp16 pieces, and products of them.
struct Pair {
  f16x8 h, l;
};
__device__ __forceinline__ Pair split_pair(const float (&x)[8], int e) {
  u32x4 h, l;
  split8h(x, e, h, l);
  return Pair{__builtin_bit_cast(f16x8, h), __builtin_bit_cast(f16x8, l)};
}
// Pieces of a fragment stored as [piece][...] rows `pstride` bytes apart.
__device__ __forceinline__ Pair lds_pair(const char* p, int pstride) {
  return Pair{*reinterpret_cast<const f16x8*>(p), *reinterpret_cast<const f16x8*>(p + pstride)};
}
// acc += A·B for 32x32x16 fragments given as pairs (small terms first).
__device__ __forceinline__ f32x16 mfma3(const Pair& a, const Pair& b, f32x16 acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.l, b.h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.h, b.l, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.h, b.h, acc, 0, 0, 0);
  return acc;
}

}  // namespace fg
