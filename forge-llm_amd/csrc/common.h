// Internal helpers shared by the HIP translation units of libforge_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/forge_hip.h"

namespace fg {

// ── error reporting ────────────────────────────────────────────────────────
int set_error(int code, const char* fmt, ...);   // returns code
hipStream_t stream();                             // library stream (after init)
bool initialized();
int device_cu_count();
bool capturing();  // a graph capture (fg_graph_begin) is in progress

// Workspace from the caching allocator; freed back to the pool at the end of
// the entry point.  Stream-ordered reuse is safe because every kernel of the
// library runs on the one library stream.
struct Workspace {
  void* ptr = nullptr;
  ~Workspace();
  int get(size_t bytes);
};

// ── per-entry-point profiling (fg_kprof_*) ─────────────────────────────────
// While profiling, each entry point's scope brackets its launches with two
// events (launch gaps included), and every launch inside the scope gets its
// own start / stop events from hipExtLaunchKernelGGL (kernel time only).
bool kprof_launch_events(hipEvent_t* start, hipEvent_t* stop);  // false: not profiling
struct KProfScope {
  int slot = -1, pend = -1;
  KProfScope(const char* name, double flop, double bytes);  // name null: no scope
  ~KProfScope() { end(); }
  void end();  // records the stop event (idempotent)
};

// C[M,N] (beta: +)= op(A)·op(B) on the GEMM kernels, for other kernels of
// the library; the layouts of launch_gemm in gemm.hip: a_k / b_k = the
// contraction index is contiguous in A / B (true, true: C = A·B^T with A
// [M][lda], B [N][ldb]; true, false: C = A·B with B [K][ldb]; false, false:
// C = A^T·B with A [K][lda], B [K][ldb]).  C is contiguous (row stride N).
// Its launches count toward the caller's profiler scope; split-K partials
// live in `ws` (see Workspace).
int gemm_inner(bool a_k, bool b_k, Workspace& ws, float* C, const float* A, const float* B, int M, int N, int K,
               int lda, int ldb, int beta);

// A batch of equal-shaped GEMMs in one launch (attention per head): problem
// zl = 0 .. nz-1 of a chunk is z = z0 + zl = b * nh + h; an operand starts at
// base + zl * sz (local: a buffer holding the chunk) or at base + b * sb +
// (h / g) * sh (a view into [b][rows][heads] activations, g query heads per
// kv head).  C of problem zl starts at C + zl * sc (contiguous [M][N]).
// `causal` restricts each output tile (128-row origin m0, column origin n0)
// to the causal half of square attention matrices: 1 skips tiles with
// n0 >= m0 + 128 (scores past the diagonal, left unwritten), 2 sums k only
// below m0 + 128 (P·V: P is zero past the diagonal), 3 sums k only from m0
// (P^T·dO: P^T is zero before it); the terms dropped by 2 and 3 are exact
// zeros, so the sums are those of the full range.
struct BatchOperand {
  int64_t sz, sb, sh;
  int g, local;
};
struct GemmBatch {
  int nh, z0;
  BatchOperand a, b;
  int64_t sc;
  int causal;  // 0: every tile over the whole K range
};
int gemm_batched(bool a_k, bool b_k, float* C, const float* A, const float* B, int M, int N, int K, int lda, int ldb,
                 const GemmBatch& bt, int nz);

// Partial maxima of the finite magnitudes of row-strided fp32 matrices (rows
// x cols, row stride ld): FG_XP_PARTS floats per matrix into `out`, for the
// operand exponents of the split-fp16 contractions (f16split.h).  One launch
// for up to kMaxXpSpecs matrices, profiled under `prof_name` (null: none).
struct XpSpec {
  const float* p;
  float* out;
  int64_t rows;
  int ld, cols;
};
constexpr int kMaxXpSpecs = 8;
int absmax_parts(const XpSpec* specs, int count, const char* prof_name);

}  // namespace fg

#define FG_HIP_CHECK(expr)                                                          \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess)                                                           \
      return fg::set_error(FG_ERR_HIP, "%s failed: %s (%s:%d)", #expr,              \
                           hipGetErrorString(e_), __FILE__, __LINE__);              \
  } while (0)

#define FG_REQUIRE_INIT()                                                           \
  do {                                                                              \
    if (!fg::initialized()) return fg::set_error(FG_ERR_INIT, "fg_init has not been called"); \
  } while (0)

#define FG_ARG_CHECK(cond, ...)                                                     \
  do {                                                                              \
    if (!(cond)) return fg::set_error(FG_ERR_ARG, __VA_ARGS__);                     \
  } while (0)

// Entry points that synchronise with the host, or copy through host staging
// memory, cannot be recorded into a graph: they fail while a capture runs.
#define FG_NO_CAPTURE(fn)                                                           \
  do {                                                                              \
    if (fg::capturing())                                                            \
      return fg::set_error(FG_ERR_ARG, "%s cannot run while a graph is being captured", fn); \
  } while (0)

// Launch on the library stream (with the kernel's own timing events while
// profiling); FG_LAUNCH also checks the launch status.
#define FG_LAUNCH_NOCHECK(kernel, grid, block, shmem, ...)                          \
  do {                                                                              \
    hipEvent_t fg_ev0_ = nullptr, fg_ev1_ = nullptr;                                \
    if (fg::kprof_launch_events(&fg_ev0_, &fg_ev1_))                                \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, fg::stream(), fg_ev0_, fg_ev1_, 0, __VA_ARGS__); \
    else                                                                            \
      hipLaunchKernelGGL(kernel, grid, block, shmem, fg::stream(), __VA_ARGS__);    \
  } while (0)
#define FG_LAUNCH(kernel, grid, block, shmem, ...)                                  \
  do {                                                                              \
    FG_LAUNCH_NOCHECK(kernel, grid, block, shmem, __VA_ARGS__);                     \
    FG_HIP_CHECK(hipGetLastError());                                                \
  } while (0)

// Wave-level reductions (64-wide wavefronts).
__device__ __forceinline__ float fg_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ double fg_wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float fg_wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
