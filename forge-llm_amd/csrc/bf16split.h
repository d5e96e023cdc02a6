// Exact three-piece bf16 splits of fp32 values for the bf16 MFMA pipes.
//
//   hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid)   (RNE each)
//
// x == hi + mid + lo exactly: hi keeps the top 8 significant bits, x - hi is
// exact in fp32 and has at most 16 significant bits, mid keeps 8 of them and
// the remainder (<= 8 bits) is exact in bf16.  A product x*y is then the sum
// of nine exact bf16 x bf16 products; the six kept by mfma6 are every term of
// weight >= 2^-16 |x*y| (the three dropped ones sum to < 2^-23 |x*y|, one fp32
// rounding), accumulated in fp32 by the MFMA.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Two elements at a time: one v_cvt_pk_bf16_f32 (RNE) per plane, the bf16
// values widened back to fp32 with a shift / mask.
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& h, uint32_t& m, uint32_t& l) {
  h = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0, x1}, bf16x2));
  const float r0 = x0 - __builtin_bit_cast(float, h << 16);
  const float r1 = x1 - __builtin_bit_cast(float, h & 0xffff0000u);
  m = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){r0, r1}, bf16x2));
  const float s0 = r0 - __builtin_bit_cast(float, m << 16);
  const float s1 = r1 - __builtin_bit_cast(float, m & 0xffff0000u);
  l = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){s0, s1}, bf16x2));
}

__device__ __forceinline__ void split8(const float (&x)[8], u32x4& h, u32x4& m, u32x4& l) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t a, b, c;
    split2(x[2 * e], x[2 * e + 1], a, b, c);
    h[e] = a;
    m[e] = b;
    l[e] = c;
  }
}

__device__ __forceinline__ void split4(float x0, float x1, float x2, float x3, u32x2& h, u32x2& m, u32x2& l) {
  uint32_t a, b, c;
  split2(x0, x1, a, b, c);
  h[0] = a; m[0] = b; l[0] = c;
  split2(x2, x3, a, b, c);
  h[1] = a; m[1] = b; l[1] = c;
}

// One 8-wide MFMA operand fragment as its three planes.
struct Planes {
  bf16x8 h, m, l;
};

__device__ __forceinline__ Planes split_planes(const float (&x)[8]) {
  u32x4 h, m, l;
  split8(x, h, m, l);
  return Planes{__builtin_bit_cast(bf16x8, h), __builtin_bit_cast(bf16x8, m), __builtin_bit_cast(bf16x8, l)};
}

// Planes of a fragment stored as [plane][...] rows `pstride` bytes apart.
__device__ __forceinline__ Planes lds_planes(const char* p, int pstride) {
  return Planes{*reinterpret_cast<const bf16x8*>(p), *reinterpret_cast<const bf16x8*>(p + pstride),
                *reinterpret_cast<const bf16x8*>(p + 2 * pstride)};
}

// acc += A·B for 32x32x16 fragments given as planes (small terms first).
__device__ __forceinline__ f32x16 mfma6(const Planes& a, const Planes& b, f32x16 acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.l, b.h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.l, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.m, b.m, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.m, b.h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.m, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.h, acc, 0, 0, 0);
  return acc;
}

}  // namespace fg
