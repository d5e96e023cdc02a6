// The SwiGLU element arithmetic (swigluRows, tensor.js:272-290) shared by the
// elementwise kernels and the GEMM epilogue that fuses it: one set of fp32
// expressions, so the fused form stores the separate kernels' bits.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

namespace fg {

__device__ __forceinline__ float swiglu_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

// O = G * sigmoid(G) * U
__device__ __forceinline__ float swiglu_fwd1(float g, float u) { return g * swiglu_sigmoid(g) * u; }

// dG = gy * U * (s + G s (1 - s)),  dU = gy * (G s),  s = sigmoid(G)
__device__ __forceinline__ void swiglu_grad1(float gy, float gv, float uv, float& dg, float& du) {
  const float s = swiglu_sigmoid(gv);
  dg = gy * uv * (s + gv * s * (1.f - s));
  du = gy * (gv * s);
}

}  // namespace fg
