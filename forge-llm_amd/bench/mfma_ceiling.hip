// The MFMA issue ceiling of the split-bf16 product stream on this card, with
// no memory traffic at all: every wave of a full grid (one 8-wave workgroup
// per CU, two waves per SIMD) runs the GEMM's per-k-step MFMA pattern — two
// 16-wide substeps of six bf16 piece products on a 2 x 2 block of 32x32
// accumulators (48 v_mfma_f32_32x32x16_bf16 per step, four independent
// accumulators between dependent issues) — on operand fragments held in
// registers, one of which changes every step.  Random operands (bf16 values
// with random mantissas) and all-zero operands are timed separately: the
// sustained clock under MFMA load depends on the data.
//
//   forge-llm_amd/lib/mfma_ceiling            (built by forge-llm_amd/build.py)
//
// Prints the time per launch and the rate as bf16 TFLOP/s and as fp32
// TFLOP/s of the six-product scheme (bf16 rate / 6).
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Pieces {
  bf16x8 h, m, l;
};

__device__ __forceinline__ bf16x8 random_fragment(uint32_t s) {
  u32x4 v;
  for (int i = 0; i < 4; ++i) {
    s = s * 1664525u + 1013904223u;
    v[i] = (s & 0x3fff3fffu) | 0x3c003c00u;  // two bf16 of magnitude ~1 with random mantissas
  }
  return __builtin_bit_cast(bf16x8, v);
}

__global__ void __launch_bounds__(512) mfma_stream(float* __restrict__ out, int steps, int zero) {
  const uint32_t seed = (blockIdx.x * 512 + threadIdx.x) * 2654435761u;
  Pieces a[2][2], b[2][2];
  for (int ss = 0; ss < 2; ++ss)
    for (int r = 0; r < 2; ++r) {
      const uint32_t o = seed + r + 4 * ss;
      a[ss][r] = Pieces{random_fragment(o + 1), random_fragment(o + 2), random_fragment(o + 3)};
      b[ss][r] = Pieces{random_fragment(o + 11), random_fragment(o + 12), random_fragment(o + 13)};
      if (zero) {
        const bf16x8 z = a[ss][r].h * (__bf16)0.f;
        a[ss][r] = Pieces{z, z, z};
        b[ss][r] = Pieces{z, z, z};
      }
    }
  f32x16 acc[2][2] = {};
  for (int it = 0; it < steps; ++it) {
    for (int ss = 0; ss < 2; ++ss) {
#define FG_X3(F, G)                                                                                     \
  for (int i = 0; i < 2; ++i)                                                                          \
    for (int j = 0; j < 2; ++j)                                                                        \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ss][i].F, b[ss][j].G, acc[i][j], 0, 0, 0);
      FG_X3(l, h) FG_X3(h, l) FG_X3(m, m) FG_X3(m, h) FG_X3(h, m) FG_X3(h, h)
#undef FG_X3
    }
    // one operand fragment changes every step (a fixed register: no scratch)
    a[0][0].h = __builtin_bit_cast(
        bf16x8, __builtin_bit_cast(u32x4, a[0][0].h) ^ (u32x4){0x00010001u * (it & 7), 0u, 0x00020002u, 0u});
  }
  float s = 0.f;
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j)
      for (int v = 0; v < 16; ++v) s += acc[i][j][v];
  out[blockIdx.x * 512 + threadIdx.x] = s;
}

int main() {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || cus <= 0) {
    printf("no device\n");
    return 1;
  }
  float* d = nullptr;
  if (hipMalloc(&d, (size_t)cus * 512 * sizeof(float)) != hipSuccess) return 1;
  const int steps = 4000;
  for (int zero = 0; zero < 2; ++zero)
    for (int rep = 0; rep < 2; ++rep) {
      hipEvent_t e0, e1;
      (void)hipEventCreate(&e0);
      (void)hipEventCreate(&e1);
      mfma_stream<<<cus, 512>>>(d, 100, zero);
      (void)hipEventRecord(e0);
      mfma_stream<<<cus, 512>>>(d, steps, zero);
      (void)hipEventRecord(e1);
      (void)hipEventSynchronize(e1);
      float ms = 0.f;
      (void)hipEventElapsedTime(&ms, e0, e1);
      const double macs = (double)cus * 8 * steps * 48 * 16384.0;  // 48 MFMAs of 32x32x16 per wave-step
      const double bf16 = 2 * macs / (ms * 1e-3) / 1e12;
      printf("%s operands, run %d: %.3f ms, %.1f TFLOP/s bf16, %.1f TFLOP/s fp32 as six bf16 products\n",
             zero ? "zero" : "random", rep, ms, bf16, bf16 / 6);
      (void)hipEventDestroy(e0);
      (void)hipEventDestroy(e1);
    }
  const hipError_t e = hipDeviceSynchronize();
  printf("status %s\n", hipGetErrorString(e));
  (void)hipFree(d);
  return e == hipSuccess ? 0 : 1;
}
