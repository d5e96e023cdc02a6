// fp32 GEMMs behind matmulT (tensor.js:34-53) for gfx950, on the fp16 MFMA
// pipes with split operands.
//
//   forward  Y [M,N]  = X[M,K]  · W[N,K]^T      A k-contiguous, B k-contiguous ("NT")
//   input    gX[M,K] (+)= gY[M,N] · W[N,K]      A k-contiguous, B j-contiguous ("NN")
//   weight   gW[N,K] (+)= gY[M,N]^T · X[M,K]    A i-contiguous, B j-contiguous ("TN")
//
// Kernel templates cover the three layouts: C[i,j] = sum_r A(i,r) B(r,j).
// Every fp32 operand element is scaled by a power of two fixed per operand
// and split, while it is staged from registers to LDS, into an fp16 hi and lo
// pair (23 significant bits); three fp16 MFMA products per pair are
// accumulated in fp32 (f16split.h), which gives fp32-level accuracy at the
// fp16 MFMA rate: v_mfma_f32_32x32x16_f16 retires 16x the multiply-adds of
// v_mfma_f32_32x32x2_f32 per cycle, so three of them per product cost ~5x
// less MFMA time than the fp32 instruction.
//
// Kernel shapes, with operand tiles register-prefetched one k-step ahead:
//   * gemm_x3_kernel: 256 threads, workgroup tile 128x128 / 128x256 / 256x128,
//     64x64 wave tiles, k-step 32, one LDS stage (store, barrier, compute,
//     barrier);
//   * gemm_pp_kernel: 512 threads, 128x256 / 256x128, 64x64 wave tiles,
//     k-step 32, two LDS stages: the split + store of k-step it+1 and the
//     loads of it+2 are interleaved with the MFMAs of k-step it (one barrier
//     per k-step);
//   * gemm_pq_kernel: the ping-pong pipeline on 128x192 tiles of 16x16 MFMA
//     blocks (outputs whose 128x256 tiles fill the CUs poorly);
//   * gemm_w_kernel: the ping-pong pipeline on 256x256 tiles, 64x128 wave
//     tiles, k-step 16 (outputs of at least two full rounds of such tiles).
// plan_gemm picks the shape and the K split per call.
//
// Launch shape: 1-D grid of tiles remapped so each of the 8 XCDs gets a
// contiguous range, then grouped 8 tile-rows at a time for L2 reuse.  When the
// tile count cannot fill the chip, K is split across gridDim.y and partial
// tiles are summed by a second kernel in a fixed order (deterministic).
#include "common.h"
#include "f16split.h"
#include "swiglu_math.h"

namespace {

using fg::f32x16;

constexpr int BM = 128, BK = 32;
constexpr int kThreads = 256;
constexpr int kXCD = 8;
constexpr int kGroupM = 8;

__device__ __forceinline__ int remap_xcd(int pid, int npid) {
  int per = (npid + kXCD - 1) / kXCD;
  int tall = npid % kXCD;
  if (tall == 0) tall = kXCD;
  int xcd = pid % kXCD, local = pid / kXCD;
  return xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
}

// Origin (m0, n0) of output tile pid of an M x N output in TM x TN tiles,
// tile-rows taken kGroupM at a time (grouped-M order, for L2 reuse).
__device__ __forceinline__ void tile_origin(int pid, int M, int N, int TM, int TN, int& m0, int& n0) {
  const int nTm = (M + TM - 1) / TM, nTn = (N + TN - 1) / TN;
  const int in_group = kGroupM * nTn;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int gsize = min(nTm - first_m, kGroupM);
  m0 = (first_m + (pid % in_group) % gsize) * TM;
  n0 = ((pid % in_group) / gsize) * TN;
}

// ───────── operand exponents ─────────
// absmax_kernel reduces each listed operand (a rows x cols matrix, row stride
// ld) over kXpParts workgroups to partial maxima of its finite magnitudes,
// out[part] (FG_XP_PARTS floats per operand); every wave of a GEMM workgroup
// folds its operands' partials itself (xp_exponent).  The partials come from
// the caller (the *_p entry points, which reuse them across the forward and
// backward GEMMs of one operand) or from a workspace filled just before the
// GEMM on the same stream.
constexpr int kXpParts = FG_XP_PARTS;
static_assert(kXpParts == 256, "xp_exponent folds four partials per lane");
constexpr int kMaxJobs = 52;  // jobs per grouped launch (see GTable)
constexpr int kXpMaxJobs = 2 * kMaxJobs;

struct XpJob {
  const float* p;
  float* out;
  int64_t rows;
  int ld, cols;
};
struct XpTable {
  int count;
  XpJob job[kXpMaxJobs];
};
static_assert(sizeof(XpTable) <= 4096, "the operand table travels as a kernel argument (4 KB at most)");

__device__ __forceinline__ float finite_abs(float x) {
  const float a = fabsf(x);
  return a < __builtin_inff() ? a : 0.f;  // inf and NaN count as 0
}

constexpr int kXpThreads = 512;
__global__ void __launch_bounds__(kXpThreads) absmax_kernel(XpTable t) {
  const XpJob& j = t.job[blockIdx.y];
  float m = 0.f;
  if (j.ld == j.cols) {  // contiguous: one flat range, float4 where aligned
    const int64_t n = j.rows * j.cols;
    int64_t done = 0;
    if (((uintptr_t)j.p & 15) == 0) {
      const float4* p4 = reinterpret_cast<const float4*>(j.p);
      const int64_t n4 = n / 4, step = (int64_t)kXpParts * kXpThreads;
      int64_t i = (int64_t)blockIdx.x * kXpThreads + threadIdx.x;
      for (; i + 3 * step < n4; i += 4 * step) {
        const float4 a = p4[i], b = p4[i + step], c = p4[i + 2 * step], d = p4[i + 3 * step];
        m = fmaxf(m, fmaxf(fmaxf(finite_abs(a.x), finite_abs(a.y)), fmaxf(finite_abs(a.z), finite_abs(a.w))));
        m = fmaxf(m, fmaxf(fmaxf(finite_abs(b.x), finite_abs(b.y)), fmaxf(finite_abs(b.z), finite_abs(b.w))));
        m = fmaxf(m, fmaxf(fmaxf(finite_abs(c.x), finite_abs(c.y)), fmaxf(finite_abs(c.z), finite_abs(c.w))));
        m = fmaxf(m, fmaxf(fmaxf(finite_abs(d.x), finite_abs(d.y)), fmaxf(finite_abs(d.z), finite_abs(d.w))));
      }
      for (; i < n4; i += step) {
        const float4 a = p4[i];
        m = fmaxf(m, fmaxf(fmaxf(finite_abs(a.x), finite_abs(a.y)), fmaxf(finite_abs(a.z), finite_abs(a.w))));
      }
      done = n4 * 4;
    }
    for (int64_t i = done + (int64_t)blockIdx.x * kXpThreads + threadIdx.x; i < n; i += (int64_t)kXpParts * kXpThreads)
      m = fmaxf(m, finite_abs(j.p[i]));
  } else if (((uintptr_t)j.p & 15) == 0 && (j.ld & 3) == 0 && (j.cols & 3) == 0) {  // rows of float4
    // this workgroup's rows blockIdx.x + 256 i as one flat range of float4
    // (row i, column c), four loads in flight per thread
    const int c4 = j.cols / 4;
    const int64_t nr = j.rows > blockIdx.x ? (j.rows - blockIdx.x + kXpParts - 1) / kXpParts : 0;
    const int64_t n = nr * c4;
    auto at = [&](int64_t e) {
      const int64_t i = e / c4;
      return reinterpret_cast<const float4*>(j.p + (blockIdx.x + i * kXpParts) * (int64_t)j.ld)[e - i * c4];
    };
    int64_t e = threadIdx.x;
    for (; e + 3 * kXpThreads < n; e += 4 * kXpThreads) {
      const float4 a = at(e), b = at(e + kXpThreads), c = at(e + 2 * kXpThreads), d = at(e + 3 * kXpThreads);
      m = fmaxf(m, fmaxf(fmaxf(finite_abs(a.x), finite_abs(a.y)), fmaxf(finite_abs(a.z), finite_abs(a.w))));
      m = fmaxf(m, fmaxf(fmaxf(finite_abs(b.x), finite_abs(b.y)), fmaxf(finite_abs(b.z), finite_abs(b.w))));
      m = fmaxf(m, fmaxf(fmaxf(finite_abs(c.x), finite_abs(c.y)), fmaxf(finite_abs(c.z), finite_abs(c.w))));
      m = fmaxf(m, fmaxf(fmaxf(finite_abs(d.x), finite_abs(d.y)), fmaxf(finite_abs(d.z), finite_abs(d.w))));
    }
    for (; e < n; e += kXpThreads) {
      const float4 a = at(e);
      m = fmaxf(m, fmaxf(fmaxf(finite_abs(a.x), finite_abs(a.y)), fmaxf(finite_abs(a.z), finite_abs(a.w))));
    }
  } else {
    for (int64_t r = blockIdx.x; r < j.rows; r += kXpParts)
      for (int c = threadIdx.x; c < j.cols; c += kXpThreads) m = fmaxf(m, finite_abs(j.p[r * (int64_t)j.ld + c]));
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  __shared__ float wm[kXpThreads / 64];
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = wm[0];
#pragma unroll
    for (int w = 1; w < kXpThreads / 64; ++w) b = fmaxf(b, wm[w]);
    j.out[blockIdx.x] = b;
  }
}

// The exponent of an operand (wave-uniform): fold its 256 partial maxima
// (four per lane) and take exponent_of_max.
__device__ __forceinline__ int xp_exponent(const float* __restrict__ parts) {
  const float4 v = *reinterpret_cast<const float4*>(parts + (threadIdx.x & 63) * 4);
  float m = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  return __builtin_amdgcn_readfirstlane(fg::exponent_of_max(m));
}

// The stored matrix behind a GEMM operand: kc (element (i, r) at p[i*ld + r])
// is `nk` rows of K; otherwise K rows of `nk`.
inline XpJob xp_job(const float* p, bool kc, int nk, int K, int ld, float* out) {
  return kc ? XpJob{p, out, (int64_t)nk, ld, K} : XpJob{p, out, (int64_t)K, ld, nk};
}

// Queues absmax_kernel over the table's operands (profiled as one
// "gemm_absmax" launch: 4 bytes per element read).
inline int queue_absmax(const XpTable& t, bool scoped) {
  if (t.count == 0) return FG_OK;
  double bytes = 0.0;
  for (int i = 0; i < t.count; ++i) bytes += 4.0 * (double)t.job[i].rows * t.job[i].cols;
  fg::KProfScope prof(scoped ? "gemm_absmax" : nullptr, 0.0, bytes);
  FG_LAUNCH(absmax_kernel, dim3(kXpParts, t.count), dim3(kXpThreads), 0, t);
  return FG_OK;
}

// Operand maxima of one GEMM: the caller's buffers (FG_XP_PARTS floats each,
// or null) and which of them already hold their operand's partial maxima
// (have bit 0: A, bit 1: B).  A buffer without its bit is filled before the
// GEMM; a null one is replaced by workspace.
struct XpArgs {
  float* a = nullptr;
  float* b = nullptr;
  int have = 0;
};

// Resolves x for operands described by ja / jb (their `out` ignored): queues
// the maxima that are missing and returns the buffers the GEMM reads.
inline int resolve_xp(const XpArgs& x, XpJob ja, XpJob jb, fg::Workspace& wsx, bool scoped, const float*& pa,
                      const float*& pb) {
  float* oa = x.a;
  float* ob = x.b;
  const bool need_a = !(x.have & 1) || !oa, need_b = !(x.have & 2) || !ob;
  if ((need_a && !oa) || (need_b && !ob)) {
    int rc = wsx.get(2 * kXpParts * sizeof(float));
    if (rc) return rc;
    if (!oa) oa = static_cast<float*>(wsx.ptr);
    if (!ob) ob = static_cast<float*>(wsx.ptr) + kXpParts;
  }
  XpTable t;
  t.count = 0;
  if (need_a) {
    ja.out = oa;
    t.job[t.count++] = ja;
  }
  if (need_b) {
    jb.out = ob;
    t.job[t.count++] = jb;
  }
  pa = oa;
  pb = ob;
  return queue_absmax(t, scoped);
}

// ───────── split-fp16 operands: scaled fp32 values as hi + lo fp16 pairs ─────────
// Every fp32 operand element x is scaled by the operand's power of two 2^e
// and split while it is staged to LDS (f16split.h):
//   hi = fp16(x 2^e), lo = fp16(x 2^e - hi)   (RNE each)
// The product x*y is accumulated as three fp16 MFMA products
//   lo*hi + hi*lo + hi*hi   (small terms first)
// each exact in fp32, accumulated in fp32 by v_mfma_f32_32x32x16_f16; the
// epilogue scales the sum back by 2^-(ea + eb) (exact).  The dropped lo*lo
// and the split's remainders are below 3 * 2^-22 |x*y|.
//
// The exponents come from the operands' largest finite magnitudes, reduced by
// absmax_kernel into per-workgroup partial maxima ahead of the GEMM; each
// wave of a GEMM workgroup folds its operands' 256 partials itself
// (xp_exponent).
//
// LDS rows are k-contiguous for both operands ([row][hi 32 | lo 32] fp16 + 16
// B pad = 144 B: 9 16-byte slots, so 16 consecutive rows start in distinct
// bank groups); one MFMA operand fragment (8 consecutive k of one row) is one
// ds_read_b128 per piece.  Operand lane layout (32x32x16 f16): lane l feeds
// A[i = l%32][k = 8*(l/32) + e], B[k = 8*(l/32) + e][j = l%32]; the
// accumulator layout is that of the fp32 32x32 MFMA.
constexpr int kXRow = 144;              // bytes per LDS row (2 planes x 64 B + 16 B pad)
constexpr int kXTile = BM * kXRow;      // bytes per operand tile

using fg::f16x8;
using fg::split8h;
using fg::u32x4;

// The thread's share of an operand's ROWS x 32 tile (ROWS = 128 or 256),
// loaded one k-step ahead.  KC (element (i,k) at base[i*ld + k]): rows
// (t>>2) + 64u, k = (t&3)*8 .. +7 (two float4 per row).  Otherwise (element at
// base[k*ld + i]): rows 128u + 2*(t&63) + e, e = 0,1, k = (t>>6)*8 .. +7 (one
// float2 per k; a wave reads 512 contiguous bytes per k).
template <int ROWS>
struct XFrag {
  float v[ROWS / 64][8];  // [row slot][k offset]
};

template <int ROWS, bool KC, bool CHECKED>
__device__ __forceinline__ void xload(XFrag<ROWS>& f, const float* __restrict__ base, int ld, int rows, int kdim,
                                      int row0, int k0) {
  const int t = threadIdx.x;
  if (KC) {
#pragma unroll
    for (int u = 0; u < ROWS / 64; ++u) {
      const int i = row0 + (t >> 2) + 64 * u, k = k0 + (t & 3) * 8;
      if (!CHECKED) {
        const float4 p = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k);
        const float4 q = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k + 4);
        f.v[u][0] = p.x; f.v[u][1] = p.y; f.v[u][2] = p.z; f.v[u][3] = p.w;
        f.v[u][4] = q.x; f.v[u][5] = q.y; f.v[u][6] = q.z; f.v[u][7] = q.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          f.v[u][e] = (i < rows && k + e < kdim) ? base[(size_t)i * ld + k + e] : 0.f;
      }
    }
  } else {
#pragma unroll
    for (int u2 = 0; u2 < ROWS / 128; ++u2) {
      const int i = row0 + 128 * u2 + 2 * (t & 63), k = k0 + (t >> 6) * 8;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        if (!CHECKED) {
          const float2 p = *reinterpret_cast<const float2*>(base + (size_t)(k + kk) * ld + i);
          f.v[2 * u2][kk] = p.x; f.v[2 * u2 + 1][kk] = p.y;
        } else {
          const bool kin = k + kk < kdim;
          f.v[2 * u2][kk] = (kin && i < rows) ? base[(size_t)(k + kk) * ld + i] : 0.f;
          f.v[2 * u2 + 1][kk] = (kin && i + 1 < rows) ? base[(size_t)(k + kk) * ld + i + 1] : 0.f;
        }
      }
    }
  }
}

template <int ROWS, bool KC>
__device__ __forceinline__ void xstore(char* __restrict__ lds, const XFrag<ROWS>& f, int e) {
  const int t = threadIdx.x;
#pragma unroll
  for (int u = 0; u < ROWS / 64; ++u) {
    const int row = KC ? (t >> 2) + 64 * u : 128 * (u >> 1) + 2 * (t & 63) + (u & 1);
    const int kq = KC ? (t & 3) : (t >> 6);
    u32x4 h, l;
    split8h(f.v[u], e, h, l);
    char* p = lds + row * kXRow + kq * 16;
    *reinterpret_cast<u32x4*>(p) = h;
    *reinterpret_cast<u32x4*>(p + 64) = l;
  }
}

// Workgroup tile TM x TN (128x128, 128x256 or 256x128), 4 waves in a 2x2
// grid, wave tile (TM/2) x (TN/2) = (TM/64) x (TN/64) 32x32 accumulators.
// Epilogue of a wave's MA x NB accumulator tiles (rows from i0, columns from
// j0): out = acc (+ out when use_beta) (+ rs), added in that order.  Per
// 32x32 tile, its 16 C and 16 residual loads are issued before the adds and
// stores, so a wave waits once per tile rather than once per element.
template <int MA, int NB, bool CHECKED>
__device__ __forceinline__ void store_acc(float* __restrict__ out, const float* __restrict__ rs, f32x16 (&acc)[MA][NB],
                                          int M, int N, int i0, int j0, int use_beta, int esc) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int a = 0; a < MA; ++a)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int j = j0 + b * 32 + (lane & 31);
      size_t o[16];
      bool ok[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = i0 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        ok[v] = !CHECKED || (i < M && j < N);
        o[v] = ok[v] ? (size_t)i * N + j : 0;  // a clamped, always valid address
      }
      float c[16], r[16];
      if (use_beta) {
#pragma unroll
        for (int v = 0; v < 16; ++v) c[v] = out[o[v]];
      }
      if (rs) {
#pragma unroll
        for (int v = 0; v < 16; ++v) r[v] = rs[o[v]];
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float x = __builtin_amdgcn_ldexpf(acc[a][b][v], esc);
        if (use_beta) x += c[v];
        if (rs) x += r[v];
        if (ok[v]) out[o[v]] = x;
      }
    }
}

// Larger tiles cut LDS bytes per MFMA (reads 64*(wm+wn) B per wave per 16 k,
// writes 128*(TM+TN) B per workgroup per 32 k); 128x128 keeps more tiles in
// flight for small outputs.
// One output tile: tile index pid (grouped-M order within the M x N output),
// K range [kbeg, kend); out (+)= the tile (use_beta), plus rs (the residual);
// ea, eb: the operands' exponents.
template <int TM, int TN, bool AK, bool BKc, bool CHECKED>
__device__ __forceinline__ void x3_tile(char* __restrict__ As, char* __restrict__ Bs, const float* __restrict__ A,
                                        const float* __restrict__ B, int M, int N, int lda, int ldb, int pid,
                                        int kbeg, int kend, float* __restrict__ out, int use_beta,
                                        const float* __restrict__ rs, int ea, int eb) {
  constexpr int MA = TM / 64, NB = TN / 64;  // accumulators per wave along i, j
  const int nTm = (M + TM - 1) / TM, nTn = (N + TN - 1) / TN;
  const int in_group = kGroupM * nTn;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int gsize = min(nTm - first_m, kGroupM);
  const int tm = first_m + (pid % in_group) % gsize;
  const int tn = (pid % in_group) / gsize;
  const int m0 = tm * TM, n0 = tn * TN;
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  f32x16 acc[MA][NB];
#pragma unroll
  for (int a = 0; a < MA; ++a)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

  XFrag<TM> fa;
  XFrag<TN> fb;
  if (nk > 0) {
    xload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg);
    xload<TN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kbeg);
  }
  // fragment base: row (lane%32) of a 32-row block, k half (lane/32)
  const int fofs = (lane & 31) * kXRow + (lane >> 5) * 16;
  const char* Ab = As + (wm * (TM / 2)) * kXRow + fofs;
  const char* Bb = Bs + (wn * (TN / 2)) * kXRow + fofs;
  for (int it = 0; it < nk; ++it) {
    xstore<TM, AK>(As, fa, ea);
    xstore<TN, BKc>(Bs, fb, eb);
    __syncthreads();
    if (it + 1 < nk) {
      xload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg + (it + 1) * BK);
      xload<TN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kbeg + (it + 1) * BK);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      f16x8 ah[MA], al[MA], bh[NB], bl[NB];
#pragma unroll
      for (int r = 0; r < MA; ++r) {
        const char* pa = Ab + r * 32 * kXRow + s * 32;
        ah[r] = *reinterpret_cast<const f16x8*>(pa);
        al[r] = *reinterpret_cast<const f16x8*>(pa + 64);
      }
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        const char* pb = Bb + r * 32 * kXRow + s * 32;
        bh[r] = *reinterpret_cast<const f16x8*>(pb);
        bl[r] = *reinterpret_cast<const f16x8*>(pb + 64);
      }
#define FG_X3(X, Y)                                                                       \
  _Pragma("unroll") for (int a = 0; a < MA; ++a) _Pragma("unroll") for (int b = 0; b < NB; ++b) \
      acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(X[a], Y[b], acc[a][b], 0, 0, 0);
      FG_X3(al, bh)
      FG_X3(ah, bl)
      FG_X3(ah, bh)
#undef FG_X3
    }
    __syncthreads();
  }

  store_acc<MA, NB, CHECKED>(out, rs, acc, M, N, m0 + wm * (TM / 2), n0 + wn * (TN / 2), use_beta, -(ea + eb));
}

template <int TM, int TN, bool AK, bool BKc, bool CHECKED>
__global__ void __launch_bounds__(kThreads, 2)
    gemm_x3_kernel(float* __restrict__ C, const float* __restrict__ A, const float* __restrict__ B, int M, int N,
                   int K, int lda, int ldb, int beta, int ksplit, float* __restrict__ partial,
                   const float* __restrict__ resid, const float* __restrict__ xpa, const float* __restrict__ xpb) {
  __shared__ __attribute__((aligned(16))) char As[TM * kXRow];
  __shared__ __attribute__((aligned(16))) char Bs[TN * kXRow];
  const int ea = xp_exponent(xpa), eb = xp_exponent(xpb);
  const int ntiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
  const int pid = remap_xcd(blockIdx.x, ntiles);
  const int kbeg = blockIdx.y * ksplit;
  const int kend = min(K, kbeg + ksplit);
  x3_tile<TM, TN, AK, BKc, CHECKED>(As, Bs, A, B, M, N, lda, ldb, pid, kbeg, kend,
                                    partial ? partial + (size_t)blockIdx.y * M * N : C, partial ? 0 : beta,
                                    partial ? nullptr : resid, ea, eb);
}

// A batch of 128x128-tile GEMMs (fg::GemmBatch): grid (tiles, 1, problems),
// no residual; each problem's operands located from blockIdx.z; the K range
// (or the tile itself) cut to the causal half when bt.causal is set.
__host__ __device__ __forceinline__ int64_t batch_offset(const fg::BatchOperand& o, int zl, int b, int h) {
  return o.local ? (int64_t)zl * o.sz : (int64_t)b * o.sb + (int64_t)(h / o.g) * o.sh;
}

template <bool AK, bool BKc, bool CHECKED>
__global__ void __launch_bounds__(kThreads, 2)
    gemm_x3_batch_kernel(float* __restrict__ C, const float* __restrict__ A, const float* __restrict__ B, int M, int N,
                         int K, int lda, int ldb, fg::GemmBatch bt, const float* __restrict__ xpa, const float* __restrict__ xpb) {
  __shared__ __attribute__((aligned(16))) char As[BM * kXRow];
  __shared__ __attribute__((aligned(16))) char Bs[BM * kXRow];
  const int ea = xp_exponent(xpa), eb = xp_exponent(xpb);
  const int zl = blockIdx.z, z = bt.z0 + zl, b = z / bt.nh, h = z - b * bt.nh;
  const int ntiles = ((M + BM - 1) / BM) * ((N + BM - 1) / BM);
  const int pid = remap_xcd(blockIdx.x, ntiles);
  int m0, n0, kbeg = 0, kend = K;
  tile_origin(pid, M, N, BM, BM, m0, n0);
  if (bt.causal == 1 && n0 >= m0 + BM) return;  // the whole workgroup: no barrier reached
  if (bt.causal == 2) kend = min(K, m0 + BM);
  if (bt.causal == 3) kbeg = min(K, m0);
  x3_tile<BM, BM, AK, BKc, CHECKED>(As, Bs, A + batch_offset(bt.a, zl, b, h), B + batch_offset(bt.b, zl, b, h), M, N,
                                    lda, ldb, pid, kbeg, kend, C + (int64_t)zl * bt.sc, 0, nullptr, ea, eb);
}

// ───────── ping-pong variant: 512 threads, double-buffered LDS ─────────
// Workgroup tile TM x TN (256x128 or 128x256), 8 waves in a (TM/64) x (TN/64)
// grid, wave tile 64x64.  Two LDS stages: while the waves compute k-step it
// from one stage they split and store k-step it+1 into the other and issue
// the global loads of k-step it+2, so each load has a whole k-step to land
// and there is one barrier per k-step.  2 x (TM+TN) x 144 B = 108 KB of LDS:
// one workgroup (two waves per SIMD) per CU.
constexpr int kPPThreads = 512;

// The thread's share of a ROWS x 32 operand tile (512 threads).  KC: rows
// (t>>2) + 128u, k = (t&3)*8 .. +7.  Otherwise ROWS = 256: rows
// 128*(t>>8) + 2*(t&63) + e, k = ((t>>6)&3)*8 .. +7 (float2 per k);
// ROWS = 128: row t&127, k = (t>>7)*8 .. +7 (one float per k).
template <int ROWS>
struct PFrag {
  float v[ROWS / 128][8];
};

template <int ROWS, bool KC, bool CHECKED>
__device__ __forceinline__ void pload(PFrag<ROWS>& f, const float* __restrict__ base, int ld, int rows, int kdim,
                                      int row0, int k0) {
  const int t = threadIdx.x;
  if (KC) {
#pragma unroll
    for (int u = 0; u < ROWS / 128; ++u) {
      const int i = row0 + (t >> 2) + 128 * u, k = k0 + (t & 3) * 8;
      if (!CHECKED) {
        const float4 p = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k);
        const float4 q = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k + 4);
        f.v[u][0] = p.x; f.v[u][1] = p.y; f.v[u][2] = p.z; f.v[u][3] = p.w;
        f.v[u][4] = q.x; f.v[u][5] = q.y; f.v[u][6] = q.z; f.v[u][7] = q.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          f.v[u][e] = (i < rows && k + e < kdim) ? base[(size_t)i * ld + k + e] : 0.f;
      }
    }
  } else if (ROWS == 256) {
    const int i = row0 + 128 * (t >> 8) + 2 * (t & 63), k = k0 + ((t >> 6) & 3) * 8;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      if (!CHECKED) {
        const float2 p = *reinterpret_cast<const float2*>(base + (size_t)(k + kk) * ld + i);
        f.v[0][kk] = p.x; f.v[ROWS / 128 - 1][kk] = p.y;
      } else {
        const bool kin = k + kk < kdim;
        f.v[0][kk] = (kin && i < rows) ? base[(size_t)(k + kk) * ld + i] : 0.f;
        f.v[ROWS / 128 - 1][kk] = (kin && i + 1 < rows) ? base[(size_t)(k + kk) * ld + i + 1] : 0.f;
      }
    }
  } else {
    const int i = row0 + (t & 127), k = k0 + (t >> 7) * 8;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      f.v[0][kk] = (!CHECKED || (k + kk < kdim && i < rows)) ? base[(size_t)(k + kk) * ld + i] : 0.f;
  }
}

template <int ROWS, bool KC>
__device__ __forceinline__ void pstore(char* __restrict__ lds, const PFrag<ROWS>& f, int e) {
  const int t = threadIdx.x;
#pragma unroll
  for (int u = 0; u < ROWS / 128; ++u) {
    int row, kq;
    if (KC) {
      row = (t >> 2) + 128 * u;
      kq = t & 3;
    } else if (ROWS == 256) {
      row = 128 * (t >> 8) + 2 * (t & 63) + u;
      kq = (t >> 6) & 3;
    } else {
      row = t & 127;
      kq = t >> 7;
    }
    u32x4 h, l;
    split8h(f.v[u], e, h, l);
    char* p = lds + row * kXRow + kq * 16;
    *reinterpret_cast<u32x4*>(p) = h;
    *reinterpret_cast<u32x4*>(p + 64) = l;
  }
}

template <int TM, int TN, bool AK, bool BKc, bool CHECKED>
__device__ __forceinline__ void pp_tile(char* __restrict__ lds_pp, const float* __restrict__ A,
                                        const float* __restrict__ B, int M, int N, int lda, int ldb, int pid,
                                        int kbeg, int kend, float* __restrict__ out, int use_beta,
                                        const float* __restrict__ rs, int ea, int eb,
                                        float* __restrict__ slab = nullptr) {
  constexpr int WGN = TN / 64;               // waves along j
  constexpr int kStage = (TM + TN) * kXRow;  // bytes per stage
  int m0, n0;
  tile_origin(pid, M, N, TM, TN, m0, n0);
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

  PFrag<TM> fa;
  PFrag<TN> fb;
  if (nk > 0) {
    pload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg);
    pload<TN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kbeg);
    pstore<TM, AK>(lds_pp, fa, ea);
    pstore<TN, BKc>(lds_pp + TM * kXRow, fb, eb);
    if (nk > 1) {
      pload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg + BK);
      pload<TN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kbeg + BK);
    }
  }
  __syncthreads();
  const int fofs = (lane & 31) * kXRow + (lane >> 5) * 16;
  // Body of one k-step: the 16 fragment reads of both 16-k substeps, the 24
  // MFMAs, and (STORE) the split + store of the next k-step and the loads of
  // the one after, interleaved with the MFMAs so the VALU and LDS work of a
  // wave issues while its MFMAs execute.
#define FG_PP_STEP(STORE, it)                                                                        \
  {                                                                                                  \
    const char* stage = lds_pp + ((it) & 1) * kStage;                                                \
    char* next = lds_pp + (((it) + 1) & 1) * kStage;                                                 \
    const char* Ab = stage + (wm * 64) * kXRow + fofs;                                               \
    const char* Bb = stage + (TM + wn * 64) * kXRow + fofs;                                          \
    f16x8 ah[2][2], al[2][2], bh[2][2], bl[2][2]; /* [substep][block] */                             \
    _Pragma("unroll") for (int ss = 0; ss < 2; ++ss) _Pragma("unroll") for (int r = 0; r < 2; ++r) { \
      const char* pa = Ab + r * 32 * kXRow + ss * 32;                                                \
      const char* pb = Bb + r * 32 * kXRow + ss * 32;                                                \
      ah[ss][r] = *reinterpret_cast<const f16x8*>(pa);                                               \
      al[ss][r] = *reinterpret_cast<const f16x8*>(pa + 64);                                          \
      bh[ss][r] = *reinterpret_cast<const f16x8*>(pb);                                               \
      bl[ss][r] = *reinterpret_cast<const f16x8*>(pb + 64);                                          \
    }                                                                                                \
    _Pragma("unroll") for (int ss = 0; ss < 2; ++ss) {                                               \
      FG_X3(al[ss], bh[ss])                                                                          \
      FG_X3(ah[ss], bl[ss])                                                                          \
      FG_X3(ah[ss], bh[ss])                                                                          \
    }                                                                                                \
    if (STORE) {                                                                                     \
      pstore<TM, AK>(next, fa, ea);                                                                  \
      pstore<TN, BKc>(next + TM * kXRow, fb, eb);                                                    \
      const int kl = kbeg + min((it) + 2, nk - 1) * BK; /* past the end: reload the last step */   \
      pload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kl);                                           \
      pload<TN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kl);                                          \
      /* 16 fragment reads first, then each MFMA followed by a share of the split */                 \
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);                                            \
      _Pragma("unroll") for (int q = 0; q < 12; ++q) {                                               \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);                                           \
        if (q % 2 == 1) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                          \
      }                                                                                              \
      _Pragma("unroll") for (int q = 0; q < 12; ++q) {                                               \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);                                           \
      }                                                                                              \
    }                                                                                                \
    __syncthreads();                                                                                 \
  }
#define FG_X3(X, Y)                                                                  \
  _Pragma("unroll") for (int a = 0; a < 2; ++a) _Pragma("unroll") for (int b = 0; b < 2; ++b) \
      acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(X[a], Y[b], acc[a][b], 0, 0, 0);
  for (int it = 0; it + 1 < nk; ++it) FG_PP_STEP(true, it)
  if (nk > 0) FG_PP_STEP(false, nk - 1)
#undef FG_X3
#undef FG_PP_STEP

  if (slab)  // a K piece of a tail tile: the whole TM x TN tile, row stride TN
    store_acc<2, 2, false>(slab, nullptr, acc, TM, TN, wm * 64, wn * 64, 0, -(ea + eb));
  else
    store_acc<2, 2, CHECKED>(out, rs, acc, M, N, m0 + wm * 64, n0 + wn * 64, use_beta, -(ea + eb));
}

// Tail split (ping-pong kernels, one workgroup per CU).  When the tiles fill
// at least one whole round of CUs and leave a last round at most half full,
// the last `r` tiles (in tile order) are cut along K into `c` pieces each
// (r * c <= CUs), and piece p = q * c + z (tile n_full + q, k-steps
// [z * kc, (z+1) * kc) of that tile's K, kc = ceil(k-steps / c)) writes its
// TM x TN partial to slab[p].  The grid is n_full full-K tiles then the r * c
// pieces, so the pieces run as one short last round; tail_reduce_kernel then
// adds each tail tile's c partials in order z = 0..c-1.
__device__ __forceinline__ void tail_piece(int K, int c, int z, int& kbeg, int& kend) {
  const int nk = (K + BK - 1) / BK;
  const int kc = (nk + c - 1) / c * BK;
  kbeg = z * kc;
  kend = min(K, kbeg + kc);
}

template <int TM, int TN, bool AK, bool BKc, bool CHECKED>
__global__ void __launch_bounds__(kPPThreads, 1)
    gemm_pp_kernel(float* __restrict__ C, const float* __restrict__ A, const float* __restrict__ B, int M, int N,
                   int K, int lda, int ldb, int beta, int ksplit, float* __restrict__ partial,
                   const float* __restrict__ resid, int n_full, int tail_c, float* __restrict__ slab, const float* __restrict__ xpa, const float* __restrict__ xpb) {
  __shared__ __attribute__((aligned(16))) char lds_pp[2 * (TM + TN) * kXRow];
  const int ea = xp_exponent(xpa), eb = xp_exponent(xpb);
  if ((int)blockIdx.x >= n_full) {  // a K piece of a tail tile
    const int p = blockIdx.x - n_full, q = p / tail_c, z = p % tail_c;
    int kbeg, kend;
    tail_piece(K, tail_c, z, kbeg, kend);
    pp_tile<TM, TN, AK, BKc, CHECKED>(lds_pp, A, B, M, N, lda, ldb, n_full + q, kbeg, kend, C, 0, nullptr, ea, eb,
                                      slab + (size_t)p * TM * TN);
    return;
  }
  const int pid = remap_xcd(blockIdx.x, n_full);
  const int kbeg = blockIdx.y * ksplit;
  const int kend = min(K, kbeg + ksplit);
  pp_tile<TM, TN, AK, BKc, CHECKED>(lds_pp, A, B, M, N, lda, ldb, pid, kbeg, kend,
                                    partial ? partial + (size_t)blockIdx.y * M * N : C, partial ? 0 : beta,
                                    partial ? nullptr : resid, ea, eb);
}

// ───────── wide variant: 256xTN tiles, 8 waves of 64x(TN/2), k-step 16 ─────────
// The ping-pong pipeline on a 256x256 (or 256x192) workgroup tile with
// k-steps of 16: each wave's 64x128 tile (2x4 32x32 accumulators) reads 12
// fragments per 24 MFMAs (16 for the 64x64 wave), and the workgroup loads and
// splits 16 values per thread per 24 MFMAs of each wave (24 for 128x256
// tiles); a 64x96 wave reads 10 per 18.  Per 16-k chunk every output element
// gets the same three products in the same order as in the other kernels.
// LDS rows of [hi 16 | lo 16] fp16 + 16 B (80 B, a stride of 5 16-byte
// slots: 16 consecutive rows of a fragment read fall on 16 distinct 4-bank
// groups); S stages x (256 + TN) rows x 80 B <= 160 KB.  With S = 2 a
// barrier follows every k-step (step s reads stage s % 2 and stores step
// s + 1's tile into the other).  With S = 4 the k-steps run in pairs between
// barriers: step s reads stage s % 4 and stores the split tile of step s + 2
// into stage (s + 2) % 4, whose last reader (step s - 2) is separated from it
// by the barrier after the odd step of {s - 2, s - 1}.  Four stages measured
// 2-3% faster for the forward (NT) and weight-gradient (TN) layouts and 2%
// slower for the input gradients (NN) in the training step.
constexpr int kWRow = 80;
template <bool AK, bool BKc>
constexpr int w_stages() { return AK && !BKc ? 2 : 4; }
constexpr int WK = 16;

// The thread's share (8 values) of a ROWS x 16 operand tile (ROWS = 256 or
// 192: 2 * ROWS units of 8 values, threads past them idle).  KC: row t>>1,
// k = (t&1)*8 .. +7 (two float4).  Otherwise row t % ROWS, k = (t / ROWS)*8
// .. +7 (one float per k; consecutive threads read consecutive rows).
// Row of the stacked [Wg; Wu] (2H rows) that output column c of the fused
// gate/up GEMM reads when the columns are ordered for the SwiGLU epilogue:
// within each 256-column tile, wave half wn takes hidden units
// c0/2 + 64 wn .. +63 as four 32-column blocks [G | U | G | U], so a lane
// holds the gate and up values of the same unit in accumulator blocks
// 2p and 2p + 1.
__device__ __forceinline__ int swiglu_row(int c, int H) {
  const int j = (c >> 8) * 128 + ((c >> 7) & 1) * 64 + ((c >> 6) & 1) * 32 + (c & 31);
  return ((c >> 5) & 1) ? H + j : j;
}

template <int ROWS, bool KC, bool CHECKED, bool SWR = false>
__device__ __forceinline__ void wload(float (&f)[8], const float* __restrict__ base, int ld, int rows, int kdim,
                                      int row0, int k0, int swh = 0) {
  const int t = threadIdx.x;
  if (ROWS < 256 && t >= 2 * ROWS) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = 0.f;
    return;
  }
  if (KC) {
    const int i = SWR ? swiglu_row(row0 + (t >> 1), swh) : row0 + (t >> 1), k = k0 + (t & 1) * 8;
    if (!CHECKED) {
      const float4 p = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k);
      const float4 q = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k + 4);
      f[0] = p.x; f[1] = p.y; f[2] = p.z; f[3] = p.w;
      f[4] = q.x; f[5] = q.y; f[6] = q.z; f[7] = q.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (i < rows && k + e < kdim) ? base[(size_t)i * ld + k + e] : 0.f;
    }
  } else {
    const int i = row0 + t % ROWS, k = k0 + (t / ROWS) * 8;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      f[kk] = (!CHECKED || (k + kk < kdim && i < rows)) ? base[(size_t)(k + kk) * ld + i] : 0.f;
  }
}

template <int ROWS, bool KC>
__device__ __forceinline__ void wstore(char* __restrict__ lds, const float (&f)[8], int e) {
  const int t = threadIdx.x;
  if (ROWS < 256 && t >= 2 * ROWS) return;
  const int row = KC ? (t >> 1) : t % ROWS, kq = KC ? (t & 1) : t / ROWS;
  u32x4 h, l;
  split8h(f, e, h, l);
  char* p = lds + row * kWRow + kq * 16;
  *reinterpret_cast<u32x4*>(p) = h;
  *reinterpret_cast<u32x4*>(p + 32) = l;
}

// SWG: the fused gate/up projection — B rows read in swiglu_row order, and
// the epilogue stores G and U into out = GU[M, 2H] in their plain [G | U]
// places and sw_out[M, H] = SwiGLU(G, U) (sw_h = H).
template <int TN, bool AK, bool BKc, bool CHECKED, bool SWG = false>
__device__ __forceinline__ void w_tile(char* __restrict__ lds_w, const float* __restrict__ A,
                                       const float* __restrict__ B, int M, int N, int lda, int ldb, int pid,
                                       int kbeg, int kend, float* __restrict__ out, int use_beta,
                                       const float* __restrict__ rs, int ea, int eb,
                                       float* __restrict__ slab = nullptr, float* __restrict__ sw_out = nullptr,
                                       int sw_h = 0) {
  constexpr int TM = 256;
  constexpr int NB = TN / 64;          // 32-column accumulator blocks per wave
  constexpr int kMf = 6 * NB;          // MFMAs per wave per k-step
  constexpr int kStage = (TM + TN) * kWRow;
  constexpr int S = w_stages<AK, BKc>();
  int m0, n0;
  tile_origin(pid, M, N, TM, TN, m0, n0);
  const int nk = kend > kbeg ? (kend - kbeg + WK - 1) / WK : 0;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves of 64 x TN/2

  f32x16 acc[2][NB];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

  float fa[8], fb[8];
  if (nk > 0) {
    wload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg);
    wload<TN, BKc, CHECKED, SWG>(fb, B, ldb, N, kend, n0, kbeg, sw_h);
    wstore<TM, AK>(lds_w, fa, ea);
    wstore<TN, BKc>(lds_w + TM * kWRow, fb, eb);
    if (nk > 1) {
      wload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg + WK);
      wload<TN, BKc, CHECKED, SWG>(fb, B, ldb, N, kend, n0, kbeg + WK, sw_h);
    }
    if (S == 4 && nk > 1) {
      wstore<TM, AK>(lds_w + kStage, fa, ea);
      wstore<TN, BKc>(lds_w + kStage + TM * kWRow, fb, eb);
      if (nk > 2) {
        wload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg + 2 * WK);
        wload<TN, BKc, CHECKED, SWG>(fb, B, ldb, N, kend, n0, kbeg + 2 * WK, sw_h);
      }
    }
  }
  __syncthreads();
  const int fofs = (lane & 31) * kWRow + (lane >> 5) * 16;
  // One k-step: 4 + 2 NB fragment reads, kMf MFMAs, and (STORE) the split + store of
  // the next k-step and the loads of the one after, interleaved with the MFMAs.
#define FG_W_STEP(STORE, it)                                                                           \
  {                                                                                                    \
    const char* stage = lds_w + ((it) % S) * kStage;                                                   \
    char* next = lds_w + (((it) + S / 2) % S) * kStage;                                                \
    const char* Ab = stage + (wm * 64) * kWRow + fofs;                                                 \
    const char* Bb = stage + (TM + wn * (TN / 2)) * kWRow + fofs;                                      \
    f16x8 ah[2], al[2], bh[NB], bl[NB];                                                                \
    _Pragma("unroll") for (int r = 0; r < 2; ++r) {                                                    \
      const char* pa = Ab + r * 32 * kWRow;                                                            \
      ah[r] = *reinterpret_cast<const f16x8*>(pa);                                                     \
      al[r] = *reinterpret_cast<const f16x8*>(pa + 32);                                                \
    }                                                                                                  \
    _Pragma("unroll") for (int r = 0; r < NB; ++r) {                                                   \
      const char* pb = Bb + r * 32 * kWRow;                                                            \
      bh[r] = *reinterpret_cast<const f16x8*>(pb);                                                     \
      bl[r] = *reinterpret_cast<const f16x8*>(pb + 32);                                                \
    }                                                                                                  \
    FG_X3(al, bh)                                                                                      \
    FG_X3(ah, bl)                                                                                      \
    FG_X3(ah, bh)                                                                                      \
    if (STORE) {                                                                                       \
      wstore<TM, AK>(next, fa, ea);                                                                    \
      wstore<TN, BKc>(next + TM * kWRow, fb, eb);                                                      \
      const int kl = kbeg + min((it) + 1 + S / 2, nk - 1) * WK; /* past the end: reload the last */  \
      wload<TM, AK, CHECKED>(fa, A, lda, M, kend, m0, kl);                                             \
      wload<TN, BKc, CHECKED, SWG>(fb, B, ldb, N, kend, n0, kl, sw_h);                                 \
      /* k-contiguous B (forward): the fragment reads first, then six VALU     */                         \
      /* per MFMA with a split store every third; other layouts (whose B loads */                         \
      /* are scalar) measured faster left to the compiler's schedule          */                         \
      if constexpr (BKc) {                                                                             \
        __builtin_amdgcn_sched_group_barrier(0x100, 4 + 2 * NB, 0);                                    \
        _Pragma("unroll") for (int q = 0; q < kMf / 2; ++q) {                                          \
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);                                           \
          if (q % 3 == 2) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                          \
        }                                                                                              \
        _Pragma("unroll") for (int q = 0; q < kMf / 2; ++q) {                                          \
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                           \
          __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);                                           \
        }                                                                                              \
      }                                                                                                \
    }                                                                                                  \
    if (S == 2 || !(STORE) || ((it) & 1)) __syncthreads(); /* S = 4: pairs of steps, and the last */ \
  }
#define FG_X3(X, Y)                                                                  \
  _Pragma("unroll") for (int a = 0; a < 2; ++a) _Pragma("unroll") for (int b = 0; b < NB; ++b) \
      acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(X[a], Y[b], acc[a][b], 0, 0, 0);
  for (int it = 0; it + 1 < nk; ++it) FG_W_STEP(true, it)
  if (nk > 0) FG_W_STEP(false, nk - 1)
#undef FG_X3
#undef FG_W_STEP

  if constexpr (SWG) {
    // accumulator blocks (2p, 2p+1) hold G and U of hidden units
    // n0/2 + 64 wn + 32 p + lane%32 (swiglu_row); rows as in store_acc
    static_assert(NB == 4, "the SwiGLU epilogue takes the 64x128 wave tile");
    const int H = sw_h;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        const int j = n0 / 2 + wn * 64 + pr * 32 + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int i = m0 + wm * 64 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          const float g = __builtin_amdgcn_ldexpf(acc[a][2 * pr][v], -(ea + eb));
          const float u = __builtin_amdgcn_ldexpf(acc[a][2 * pr + 1][v], -(ea + eb));
          out[(size_t)i * 2 * H + j] = g;
          out[(size_t)i * 2 * H + H + j] = u;
          sw_out[(size_t)i * H + j] = fg::swiglu_fwd1(g, u);
        }
      }
    return;
  }
  if (slab)  // a K piece of a tail tile: the whole 256 x TN tile, row stride TN
    store_acc<2, NB, false>(slab, nullptr, acc, TM, TN, wm * 64, wn * (TN / 2), 0, -(ea + eb));
  else
    store_acc<2, NB, CHECKED>(out, rs, acc, M, N, m0 + wm * 64, n0 + wn * (TN / 2), use_beta, -(ea + eb));
}

// The fused gate/up projection: GU[M, 2H] = X[M,K] · [Wg; Wu]^T and
// O[M, H] = SwiGLU(G, U) from the accumulators (full tiles only: M % 256,
// H % 128, K % 32 == 0).
__global__ void __launch_bounds__(kPPThreads, 1)
    gemm_w_swiglu_kernel(float* __restrict__ O, float* __restrict__ GU, const float* __restrict__ X,
                         const float* __restrict__ W, int M, int K, int H, const float* __restrict__ xpa, const float* __restrict__ xpb) {
  __shared__ __attribute__((aligned(16))) char lds_w[w_stages<true, true>() * 512 * kWRow];
  const int ea = xp_exponent(xpa), eb = xp_exponent(xpb);
  const int ntiles = (M / 256) * (2 * H / 256);
  const int pid = remap_xcd(blockIdx.x, ntiles);
  w_tile<256, true, true, false, true>(lds_w, X, W, M, 2 * H, K, K, pid, 0, K, GU, 0, nullptr, ea, eb, nullptr, O,
                                       H);
}

template <int TN, bool AK, bool BKc, bool CHECKED>
__global__ void __launch_bounds__(kPPThreads, 1)
    gemm_w_kernel(float* __restrict__ C, const float* __restrict__ A, const float* __restrict__ B, int M, int N,
                  int K, int lda, int ldb, int beta, int ksplit, float* __restrict__ partial,
                  const float* __restrict__ resid, int n_full, int tail_c, float* __restrict__ slab, const float* __restrict__ xpa, const float* __restrict__ xpb) {
  __shared__ __attribute__((aligned(16))) char lds_w[w_stages<AK, BKc>() * (256 + TN) * kWRow];
  const int ea = xp_exponent(xpa), eb = xp_exponent(xpb);
  if ((int)blockIdx.x >= n_full) {  // a K piece of a tail tile
    const int p = blockIdx.x - n_full, q = p / tail_c, z = p % tail_c;
    int kbeg, kend;
    tail_piece(K, tail_c, z, kbeg, kend);
    w_tile<TN, AK, BKc, CHECKED>(lds_w, A, B, M, N, lda, ldb, n_full + q, kbeg, kend, C, 0, nullptr, ea, eb,
                                 slab + (size_t)p * 256 * TN);
    return;
  }
  const int pid = remap_xcd(blockIdx.x, n_full);
  const int kbeg = blockIdx.y * ksplit;
  const int kend = min(K, kbeg + ksplit);
  w_tile<TN, AK, BKc, CHECKED>(lds_w, A, B, M, N, lda, ldb, pid, kbeg, kend,
                           partial ? partial + (size_t)blockIdx.y * M * N : C, partial ? 0 : beta,
                           partial ? nullptr : resid, ea, eb);
}

// C (+)= the sum of a tail tile's pieces (+ resid, added last): one
// workgroup row per tail tile q (blockIdx.y), elements grid-strided.
// Sums one tail tile's c pieces into C, float4 at a time where the row stride
// allows: acc = (beta ? C : 0) + piece 0 + ... + piece c-1 (in that order,
// four pieces' loads issued together), then resid + acc.  Work split over
// nx workgroups (index x) per tile.
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ void tail_sum_tile(float* __restrict__ C, const float* __restrict__ resid,
                                              const float* __restrict__ sq, int M, int N, int TM, int TN, int m0,
                                              int n0, int c, int beta, int x, int nx) {
  const size_t piece = (size_t)TM * TN;
  const bool vec = (N & 3) == 0 && ((uintptr_t)C & 15) == 0 && (resid == nullptr || ((uintptr_t)resid & 15) == 0);
  if (vec) {
    for (int e4 = x * 256 + threadIdx.x; e4 < TM * TN / 4; e4 += nx * 256) {
      const int e = 4 * e4;
      const int i = m0 + e / TN, j = n0 + e % TN;  // j % 4 == 0 and N % 4 == 0: j < N covers j .. j+3
      if (i >= M || j >= N) continue;
      const size_t o = (size_t)i * N + j;
      float4 acc = beta ? *reinterpret_cast<const float4*>(C + o) : make_float4(0.f, 0.f, 0.f, 0.f);
      int z = 0;
      for (; z + 4 <= c; z += 4) {
        const float4 a0 = *reinterpret_cast<const float4*>(sq + (size_t)z * piece + e);
        const float4 a1 = *reinterpret_cast<const float4*>(sq + (size_t)(z + 1) * piece + e);
        const float4 a2 = *reinterpret_cast<const float4*>(sq + (size_t)(z + 2) * piece + e);
        const float4 a3 = *reinterpret_cast<const float4*>(sq + (size_t)(z + 3) * piece + e);
        acc = add4(add4(add4(add4(acc, a0), a1), a2), a3);
      }
      for (; z < c; ++z) acc = add4(acc, *reinterpret_cast<const float4*>(sq + (size_t)z * piece + e));
      if (resid) acc = add4(*reinterpret_cast<const float4*>(resid + o), acc);
      *reinterpret_cast<float4*>(C + o) = acc;
    }
    return;
  }
  for (int e = x * 256 + threadIdx.x; e < TM * TN; e += nx * 256) {
    const int i = m0 + e / TN, j = n0 + e % TN;
    if (i >= M || j >= N) continue;
    const size_t o = (size_t)i * N + j;
    float acc = beta ? C[o] : 0.f;
    for (int z = 0; z < c; ++z) acc += sq[(size_t)z * piece + e];
    C[o] = resid ? resid[o] + acc : acc;
  }
}

__global__ void __launch_bounds__(256) tail_reduce_kernel(float* __restrict__ C, const float* __restrict__ resid,
                                                          const float* __restrict__ slab, int M, int N, int TM,
                                                          int TN, int n_full, int tail_c, int beta) {
  const int q = blockIdx.y;
  int m0, n0;
  tile_origin(n_full + q, M, N, TM, TN, m0, n0);
  tail_sum_tile(C, resid, slab + (size_t)q * tail_c * TM * TN, M, N, TM, TN, m0, n0, tail_c, beta, blockIdx.x,
                gridDim.x);
}

// ───────── RoPE of the q and k columns of a fused qkv projection ─────────
// ropeRows (tensor.js:133-148) applied in place to the matmulT outputs of
// columns [0, cols) — heads of dH — of Y[M, N]: pair p = (j % dH)/2 of row i
// turns by the table angle of position pos0 + (i % posStride, or i when
// posStride is 0), in fp64 with contraction off (the arithmetic of
// qkv_rope_kernel, so the values equal fg_qkv_rope_fwd's bit for bit).
struct RopeEpi {
  const double* c;
  const double* s;
  int cols, dH, pos0, posStride;
};

__device__ __forceinline__ void rope_turn(float& a, float& b, double cc, double ss) {
#pragma clang fp contract(off)
  const double da = a, db = b;
  a = (float)(da * cc - db * ss);
  b = (float)(da * ss + db * cc);
}

// Two pairs per thread (dH % 4 == 0, N % 4 == 0, 16-byte aligned Y and tables).
typedef double d2v __attribute__((ext_vector_type(2)));
__global__ void __launch_bounds__(256) rope_cols4_kernel(float* __restrict__ Y, int M, int N, RopeEpi re) {
  const int half = re.dH >> 1, q4 = re.cols >> 2;
  const int64_t total = (int64_t)M * q4;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int i = (int)(e / q4), j = 4 * (int)(e - (int64_t)i * q4);
    const int pos = re.pos0 + (re.posStride > 0 ? i % re.posStride : i);
    const size_t t = (size_t)pos * half + (j % re.dH) / 2;
    const d2v cc = *reinterpret_cast<const d2v*>(re.c + t), ss = *reinterpret_cast<const d2v*>(re.s + t);
    float4* y = reinterpret_cast<float4*>(Y + (size_t)i * N + j);
    float4 v = *y;
    rope_turn(v.x, v.y, cc.x, ss.x);
    rope_turn(v.z, v.w, cc.y, ss.y);
    *y = v;
  }
}

// One pair per thread (any even dH).
__global__ void __launch_bounds__(256) rope_cols_kernel(float* __restrict__ Y, int M, int N, RopeEpi re) {
  const int half = re.dH >> 1, pairs = re.cols >> 1;
  const int64_t total = (int64_t)M * pairs;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int i = (int)(e / pairs), j = 2 * (int)(e - (int64_t)i * pairs);
    const int pos = re.pos0 + (re.posStride > 0 ? i % re.posStride : i);
    const size_t t = (size_t)pos * half + (j % re.dH) / 2;
    float* y = Y + (size_t)i * N + j;
    float a = y[0], b = y[1];
    rope_turn(a, b, re.c[t], re.s[t]);
    y[0] = a;
    y[1] = b;
  }
}

// ───────── 128x192 tiles: 8 waves of 64x48, 16x16x32 MFMA blocks ─────────
// An 8192 x 768 output is 256 tiles of 128x192, one per CU, where 128x256
// tiles leave a quarter of the CUs idle.  Eight waves in a 2 (i) x 4 (j) grid,
// each 64x48 = 4 x 3 blocks of v_mfma_f32_16x16x32_f16 (lane l feeds
// A[i = l%16][k = 8*(l/16) + e] and B[k = 8*(l/16) + e][j = l%16]; the
// accumulator holds D[i = 4*(l/16) + v][j = l%16]).  One MFMA covers a whole
// 32-k step, so a fragment is still one ds_read_b128 per piece from the
// 144-byte LDS rows.  Per wave and k-step: 14 fragment reads for 36 MFMAs of
// 16 cycles (the 64x64 ping-pong wave: 16 reads for 24 of 32 cycles).  Two
// LDS stages (2 x 320 x 144 B = 90 KB), the same ping-pong pipeline: the
// split + store of k-step it+1 and the loads of it+2 overlap the MFMAs of it.
constexpr int QM = 128, QN = 192;
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The thread's share of a ROWS x 32 operand tile (512 threads, ROWS = 128 or
// 192): units u = t + 512*s (s < QU), unit -> (row, k-octet).  KC: row =
// unit/4, k = (unit%4)*8 .. +7 (two float4); otherwise row = unit % ROWS, k =
// (unit/ROWS)*8 .. +7 (one float per k, consecutive threads on consecutive
// rows).  Units past 4*ROWS (t >= 256 at ROWS = 192) are idle.
template <int ROWS>
struct QFrag {
  static constexpr int kU = (ROWS * 4 + kPPThreads - 1) / kPPThreads;
  float v[kU][8];
};

template <int ROWS, bool KC>
__device__ __forceinline__ void q_unit(int unit, int& row, int& kq) {
  if (KC) {
    row = unit >> 2;
    kq = unit & 3;
  } else {
    row = unit % ROWS;
    kq = unit / ROWS;
  }
}

template <int ROWS, bool KC, bool CHECKED>
__device__ __forceinline__ void qload(QFrag<ROWS>& f, const float* __restrict__ base, int ld, int rows, int kdim,
                                      int row0, int k0) {
#pragma unroll
  for (int s = 0; s < QFrag<ROWS>::kU; ++s) {
    const int unit = threadIdx.x + kPPThreads * s;
    if (unit >= 4 * ROWS) break;  // wave-uniform (256 | 512 units)
    int row, kq;
    q_unit<ROWS, KC>(unit, row, kq);
    const int i = row0 + row, k = k0 + kq * 8;
    if (KC) {
      if (!CHECKED) {
        const float4 p = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k);
        const float4 q = *reinterpret_cast<const float4*>(base + (size_t)i * ld + k + 4);
        f.v[s][0] = p.x; f.v[s][1] = p.y; f.v[s][2] = p.z; f.v[s][3] = p.w;
        f.v[s][4] = q.x; f.v[s][5] = q.y; f.v[s][6] = q.z; f.v[s][7] = q.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f.v[s][e] = (i < rows && k + e < kdim) ? base[(size_t)i * ld + k + e] : 0.f;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        f.v[s][e] = (!CHECKED || (i < rows && k + e < kdim)) ? base[(size_t)(k + e) * ld + i] : 0.f;
    }
  }
}

template <int ROWS, bool KC>
__device__ __forceinline__ void qstore(char* __restrict__ lds, const QFrag<ROWS>& f, int e) {
#pragma unroll
  for (int s = 0; s < QFrag<ROWS>::kU; ++s) {
    const int unit = threadIdx.x + kPPThreads * s;
    if (unit >= 4 * ROWS) break;
    int row, kq;
    q_unit<ROWS, KC>(unit, row, kq);
    u32x4 h, l;
    split8h(f.v[s], e, h, l);
    char* p = lds + row * kXRow + kq * 16;
    *reinterpret_cast<u32x4*>(p) = h;
    *reinterpret_cast<u32x4*>(p + 64) = l;
  }
}

// Epilogue of a wave's 4 x 3 16x16 blocks (rows from i0, columns from j0):
// out = acc (+ out when use_beta) (+ rs), per block its loads issued first.
template <bool CHECKED>
__device__ __forceinline__ void store_acc16(float* __restrict__ out, const float* __restrict__ rs,
                                            f32x4 (&acc)[4][3], int M, int N, int i0, int j0, int use_beta,
                                            int esc) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      const int j = j0 + 16 * b + (lane & 15);
      size_t o[4];
      bool ok[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 16 * a + 4 * (lane >> 4) + v;
        ok[v] = !CHECKED || (i < M && j < N);
        o[v] = ok[v] ? (size_t)i * N + j : 0;
      }
      float c[4], r[4];
      if (use_beta) {
#pragma unroll
        for (int v = 0; v < 4; ++v) c[v] = out[o[v]];
      }
      if (rs) {
#pragma unroll
        for (int v = 0; v < 4; ++v) r[v] = rs[o[v]];
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float x = __builtin_amdgcn_ldexpf(acc[a][b][v], esc);
        if (use_beta) x += c[v];
        if (rs) x += r[v];
        if (ok[v]) out[o[v]] = x;
      }
    }
}

template <bool AK, bool BKc, bool CHECKED>
__global__ void __launch_bounds__(kPPThreads, 1)
    gemm_pq_kernel(float* __restrict__ C, const float* __restrict__ A, const float* __restrict__ B, int M, int N,
                   int K, int lda, int ldb, int beta, int ksplit, float* __restrict__ partial,
                   const float* __restrict__ resid, const float* __restrict__ xpa, const float* __restrict__ xpb) {
  __shared__ __attribute__((aligned(16))) char lds_pq[2 * (QM + QN) * kXRow];
  constexpr int kStage = (QM + QN) * kXRow;
  const int ea = xp_exponent(xpa), eb = xp_exponent(xpb);
  const int ntiles = ((M + QM - 1) / QM) * ((N + QN - 1) / QN);
  const int pid = remap_xcd(blockIdx.x, ntiles);
  const int kbeg = blockIdx.y * ksplit;
  const int kend = min(K, kbeg + ksplit);
  float* out = partial ? partial + (size_t)blockIdx.y * M * N : C;
  const int use_beta = partial ? 0 : beta;
  const float* rs = partial ? nullptr : resid;
  int m0, n0;
  tile_origin(pid, M, N, QM, QN, m0, n0);
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  f32x4 acc[4][3];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[a][b][v] = 0.f;

  QFrag<QM> fa;
  QFrag<QN> fb;
  if (nk > 0) {
    qload<QM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg);
    qload<QN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kbeg);
    qstore<QM, AK>(lds_pq, fa, ea);
    qstore<QN, BKc>(lds_pq + QM * kXRow, fb, eb);
    if (nk > 1) {
      qload<QM, AK, CHECKED>(fa, A, lda, M, kend, m0, kbeg + BK);
      qload<QN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kbeg + BK);
    }
  }
  __syncthreads();
  // fragment base: row (lane%16) of a 16-row block, k octet (lane/16)
  const int fofs = (lane & 15) * kXRow + (lane >> 4) * 16;
#define FG_PQ_STEP(STORE, it)                                                                        \
  {                                                                                                  \
    const char* stage = lds_pq + ((it) & 1) * kStage;                                                \
    char* next = lds_pq + (((it) + 1) & 1) * kStage;                                                 \
    const char* Ab = stage + (wm * 64) * kXRow + fofs;                                               \
    const char* Bb = stage + (QM + wn * 48) * kXRow + fofs;                                          \
    f16x8 ah[4], al[4], bh[3], bl[3];                                                                \
    _Pragma("unroll") for (int r = 0; r < 4; ++r) {                                                  \
      const char* pa = Ab + r * 16 * kXRow;                                                          \
      ah[r] = *reinterpret_cast<const f16x8*>(pa);                                                   \
      al[r] = *reinterpret_cast<const f16x8*>(pa + 64);                                              \
    }                                                                                                \
    _Pragma("unroll") for (int r = 0; r < 3; ++r) {                                                  \
      const char* pb = Bb + r * 16 * kXRow;                                                          \
      bh[r] = *reinterpret_cast<const f16x8*>(pb);                                                   \
      bl[r] = *reinterpret_cast<const f16x8*>(pb + 64);                                              \
    }                                                                                                \
    FG_Q3(al, bh)                                                                                    \
    FG_Q3(ah, bl)                                                                                    \
    FG_Q3(ah, bh)                                                                                    \
    if (STORE) {                                                                                     \
      qstore<QM, AK>(next, fa, ea);                                                                  \
      qstore<QN, BKc>(next + QM * kXRow, fb, eb);                                                    \
      const int kl = kbeg + min((it) + 2, nk - 1) * BK; /* past the end: reload the last step */   \
      qload<QM, AK, CHECKED>(fa, A, lda, M, kend, m0, kl);                                           \
      qload<QN, BKc, CHECKED>(fb, B, ldb, N, kend, n0, kl);                                          \
      /* 14 fragment reads first, then the MFMAs with the split interleaved */                       \
      __builtin_amdgcn_sched_group_barrier(0x100, 14, 0);                                            \
      _Pragma("unroll") for (int q = 0; q < 18; ++q) {                                               \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);                                           \
        if (q % 4 == 3) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                          \
      }                                                                                              \
      _Pragma("unroll") for (int q = 0; q < 18; ++q) {                                               \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);                                           \
      }                                                                                              \
    }                                                                                                \
    __syncthreads();                                                                                 \
  }
#define FG_Q3(X, Y)                                                                  \
  _Pragma("unroll") for (int a = 0; a < 4; ++a) _Pragma("unroll") for (int b = 0; b < 3; ++b) \
      acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(X[a], Y[b], acc[a][b], 0, 0, 0);
  for (int it = 0; it + 1 < nk; ++it) FG_PQ_STEP(true, it)
  if (nk > 0) FG_PQ_STEP(false, nk - 1)
#undef FG_Q3
#undef FG_PQ_STEP

  store_acc16<CHECKED>(out, rs, acc, M, N, m0 + wm * 64, n0 + wn * 48, use_beta, -(ea + eb));
}

// Several independent GEMMs of one layout in one launch (the weight
// gradients of a step, deferred to the end of backward): the table travels
// by value as the kernel argument (no device upload, so a recorded graph
// holds it), block b -> (job, tile) through the tiles' prefix sums after the
// XCD remap.  Every job runs its full K: no split, no partial slabs.
struct GJob {  // kMaxJobs per table
  float* C;
  const float* A;
  const float* B;
  const float* xpa;  // the operands' partial maxima
  const float* xpb;
  int M, N, K, lda, ldb, beta, even;
};
struct GTable {
  int count;
  int n_full, tail_c;  // tail split (see gemm_pp_kernel): tiles n_full.. are cut into tail_c K pieces
  float* slab;
  int prefix[kMaxJobs + 1];
  GJob job[kMaxJobs];
};
static_assert(sizeof(GTable) <= 4096, "the job table travels as a kernel argument (4 KB at most)");

__device__ __forceinline__ int job_of(const GTable& t, int g) {
  int j = 0;
  while (j + 1 < t.count && g >= t.prefix[j + 1]) ++j;
  return j;
}

template <int TM, int TN, bool AK, bool BKc>
__global__ void __launch_bounds__(kPPThreads, 1) gemm_pp_grouped(GTable t) {
  __shared__ __attribute__((aligned(16))) char lds_pp[2 * (TM + TN) * kXRow];
  int g, kbeg = 0, kend = -1;
  float* slab = nullptr;
  if ((int)blockIdx.x >= t.n_full) {  // a K piece of a tail tile
    const int p = blockIdx.x - t.n_full;
    g = t.n_full + p / t.tail_c;
    slab = t.slab + (size_t)p * TM * TN;
    tail_piece(t.job[job_of(t, g)].K, t.tail_c, p % t.tail_c, kbeg, kend);
  } else {
    g = remap_xcd(blockIdx.x, t.n_full);
  }
  const int j = job_of(t, g);
  const GJob& jb = t.job[j];
  const int pid = g - t.prefix[j];
  const int ea = xp_exponent(jb.xpa), eb = xp_exponent(jb.xpb);
  if (!slab) kend = jb.K;
  if (jb.even)
    pp_tile<TM, TN, AK, BKc, false>(lds_pp, jb.A, jb.B, jb.M, jb.N, jb.lda, jb.ldb, pid, kbeg, kend, jb.C, jb.beta,
                                    nullptr, ea, eb, slab);
  else
    pp_tile<TM, TN, AK, BKc, true>(lds_pp, jb.A, jb.B, jb.M, jb.N, jb.lda, jb.ldb, pid, kbeg, kend, jb.C, jb.beta,
                                   nullptr, ea, eb, slab);
}

// The grouped launch on 256x256 tiles (w_tile).
template <bool AK, bool BKc>
__global__ void __launch_bounds__(kPPThreads, 1) gemm_w_grouped(GTable t) {
  __shared__ __attribute__((aligned(16))) char lds_w[w_stages<AK, BKc>() * 512 * kWRow];
  int g, kbeg = 0, kend = -1;
  float* slab = nullptr;
  if ((int)blockIdx.x >= t.n_full) {  // a K piece of a tail tile
    const int p = blockIdx.x - t.n_full;
    g = t.n_full + p / t.tail_c;
    slab = t.slab + (size_t)p * 256 * 256;
    tail_piece(t.job[job_of(t, g)].K, t.tail_c, p % t.tail_c, kbeg, kend);
  } else {
    g = remap_xcd(blockIdx.x, t.n_full);
  }
  const int j = job_of(t, g);
  const GJob& jb = t.job[j];
  const int pid = g - t.prefix[j];
  const int ea = xp_exponent(jb.xpa), eb = xp_exponent(jb.xpb);
  if (!slab) kend = jb.K;
  if (jb.even)
    w_tile<256, AK, BKc, false>(lds_w, jb.A, jb.B, jb.M, jb.N, jb.lda, jb.ldb, pid, kbeg, kend, jb.C, jb.beta,
                                nullptr, ea, eb, slab);
  else
    w_tile<256, AK, BKc, true>(lds_w, jb.A, jb.B, jb.M, jb.N, jb.lda, jb.ldb, pid, kbeg, kend, jb.C, jb.beta,
                               nullptr, ea, eb, slab);
}

// The grouped launch's tail tiles: job lookup per tail tile, then as
// tail_reduce_kernel (no residual).
template <int TM, int TN>
__global__ void __launch_bounds__(256) tail_reduce_grouped(GTable t) {
  const int q = blockIdx.y, g = t.n_full + q;
  const int jx = job_of(t, g);
  const GJob& jb = t.job[jx];
  int m0, n0;
  tile_origin(g - t.prefix[jx], jb.M, jb.N, TM, TN, m0, n0);
  tail_sum_tile(jb.C, nullptr, t.slab + (size_t)q * t.tail_c * TM * TN, jb.M, jb.N, TM, TN, m0, n0, t.tail_c,
                jb.beta, blockIdx.x, gridDim.x);
}

// C = resid + ((beta ? C : 0) + sum_z partial[z])  (fixed order over z).
// The slab loads of four z at a time are issued together (the sum keeps the
// z order); each slab is read once, so it is streamed (nontemporal).
typedef float v4f __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256) splitk_reduce_kernel(float* __restrict__ C, const float* __restrict__ partial,
                                                            int64_t n, int splits, int beta,
                                                            const float* __restrict__ resid) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  // float4 path: C and resid 16-byte aligned, every partial slab too (pool-aligned base, n % 4 == 0)
  const bool vec = (((uintptr_t)C | (uintptr_t)resid) & 15) == 0 && (n & 3) == 0;
  for (; i < n; i += stride) {
    if (vec && i + 4 <= n) {
      v4f s = beta ? *reinterpret_cast<const v4f*>(C + i) : v4f{0.f, 0.f, 0.f, 0.f};
      const v4f* p = reinterpret_cast<const v4f*>(partial + i);
      const int64_t zs = n / 4;  // slab stride in float4
      int z = 0;
      for (; z + 4 <= splits; z += 4) {
        const v4f p0 = __builtin_nontemporal_load(p + (z + 0) * zs);
        const v4f p1 = __builtin_nontemporal_load(p + (z + 1) * zs);
        const v4f p2 = __builtin_nontemporal_load(p + (z + 2) * zs);
        const v4f p3 = __builtin_nontemporal_load(p + (z + 3) * zs);
        s += p0;
        s += p1;
        s += p2;
        s += p3;
      }
      for (; z < splits; ++z) s += __builtin_nontemporal_load(p + z * zs);
      if (resid) {  // added last: the value of resid + (the product as matmulT stores it)
        const v4f q = *reinterpret_cast<const v4f*>(resid + i);
        s = q + s;
      }
      *reinterpret_cast<v4f*>(C + i) = s;
    } else {
      for (int64_t e = i; e < n && e < i + 4; ++e) {
        float s = beta ? C[e] : 0.f;
        for (int z = 0; z < splits; ++z) s += partial[(size_t)z * n + e];
        if (resid) s = resid[e] + s;
        C[e] = s;
      }
    }
  }
}

// Tile shape and K split for one GEMM (rules from measurements of the three
// layouts at the transformer shapes on MI355X):
//   * outputs below 8M elements use 128x128 tiles (up to three workgroups per
//     CU), except weight gradients (TN) with >= 2048 output rows;
//   * large outputs use 256-wide tiles: the ping-pong kernel for the NT and
//     TN layouts, the 128x256 / 256x128 single-stage kernel for NN (whose
//     j-contiguous B operand loads narrower vectors in the 512-thread
//     mapping).
// The K split then brings the grid to ~2 resident workgroups per CU (one for
// ping-pong), keeping >= 8 k-steps per split.
struct GemmPlan {
  int tm, tn, splits, ksplit, pp, pq, w;
};

// Fraction of the CU slots the tiles use over their rounds (one workgroup per CU).
inline double round_fill(int64_t tiles, int cus) {
  const int64_t rounds = (tiles + cus - 1) / cus;
  return (double)tiles / (double)(rounds * cus);
}

// Below this K the two pieces' partial sums cost more than the wider tile
// saves (8192 x 768 at K = 768: 68 against 58 us; at K = 2048 ... 32000: 2-7%
// faster than the 128x192 kernel).
constexpr int kW192MinK = 2048;
GemmPlan plan_gemm(bool AK, bool BKc, int M, int N, int K, int cus) {
  const bool nn = AK && !BKc, tn = !AK;
  const int64_t outs = (int64_t)M * N;
  GemmPlan p{128, 128, 1, K, 0, 0, 0};
  // Outputs with at least one full round of 256x256 tiles: the wide kernel
  // (fewer LDS reads, splits and loads per MFMA), tail-split like the
  // ping-pong kernels.
  const int64_t w_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
  if (outs >= ((int64_t)1 << 23) && (w_tiles >= 2 * cus || w_tiles == cus)) {
    p.tm = p.tn = 256;
    p.pp = p.w = 1;
    return p;
  }
  if (outs >= (int64_t)1 << 23) {
    if (nn) {
      p.tm = M >= N ? 256 : 128;
      p.tn = M >= N ? 128 : 256;
    } else {
      p.tn = 256;
      p.pp = 1;
    }
  } else if (tn && M >= 2048 && N >= 256) {
    p.tn = 256;
    p.pp = 1;
  }
  // Mid-size NT / NN outputs whose 256x192 tiles make half a round of CUs
  // (8192 x 768: 128 tiles): the wide kernel with K split in two.
  if (AK && outs < ((int64_t)1 << 23) && K >= kW192MinK) {
    const int64_t t192 = (int64_t)((M + 255) / 256) * ((N + 191) / 192);
    if (2 * t192 <= cus && 2 * t192 >= cus - cus / 8) {
      p.tm = 256;
      p.tn = 192;
      p.pp = p.w = 1;
      p.ksplit = ((K + 1) / 2 + BK - 1) / BK * BK;
      p.splits = (K + p.ksplit - 1) / p.ksplit;
      return p;
    }
  }
  // Mid-size NT / NN outputs (8192 x 768 in the 125M step): the ping-pong
  // 128x256 kernel at under one tile per CU beats the 128x128 kernel split over
  // K (a plan sweep with random operands at M = 8192, N = 768, K = 768 ... 32000:
  // 5-19% faster); long K still splits in four.
  if (AK && outs < ((int64_t)1 << 23)) {
    const int64_t pp_tiles = (int64_t)((M + 127) / 128) * ((N + 255) / 256);
    // 128x192 tiles when they fill the rounds clearly better (8192 x 768:
    // 256 tiles on 256 CUs against 192), over the whole K: 2-5% faster than
    // 128x256 at K = 768 ... 4096 (measured); at K = 32000 the 128x256 kernel
    // split four ways is 3% faster
    const int64_t pq_tiles = (int64_t)((M + QM - 1) / QM) * ((N + QN - 1) / QN);
    if (K < 16384 && pq_tiles >= cus / 2 && round_fill(pq_tiles, cus) >= round_fill(pp_tiles, cus) + 0.1) {
      p.tm = QM;
      p.tn = QN;
      p.pq = 1;
      p.splits = 1;
      p.ksplit = K;
      return p;
    }
    if (2 * pp_tiles >= cus) {
      p.tm = 128;
      p.tn = 256;
      p.pp = 1;
      const int splits = K >= 4096 ? 4 : 1;
      p.ksplit = ((K + splits - 1) / splits + BK - 1) / BK * BK;
      p.splits = (K + p.ksplit - 1) / p.ksplit;
      return p;
    }
    // Smaller outputs whose 128x256 tiles split four ways over K make exactly
    // one round of CUs (2048 x 1024: 64 tiles): the ping-pong kernel split
    // that way beats the 128x128 kernel split to two pieces per CU (random
    // operands: 2048 x 1024 over K = 4096 104 against 116 us as an input
    // gradient, 95 against 106 us forward; 1024 x 2048 over K = 1024 36.0
    // against 37.9 us).  Splits that leave part of the round idle (72 tiles
    // in 2 or 4 pieces) measured slower than the 128x128 kernel.
    if (M >= 1024 && N >= 512 && 4 * pp_tiles == cus && K >= 4 * 8 * BK) {
      p.tm = 128;
      p.tn = 256;
      p.pp = 1;
      p.ksplit = ((K + 3) / 4 + BK - 1) / BK * BK;
      p.splits = (K + p.ksplit - 1) / p.ksplit;
      return p;
    }
  }
  const int64_t tiles = (int64_t)((M + p.tm - 1) / p.tm) * ((N + p.tn - 1) / p.tn);
  const int64_t slots = (int64_t)cus * (p.pp ? 1 : 2);
  int splits = 1;
  while (tiles * splits < slots && K / (splits * 2) >= 8 * BK) splits *= 2;
  p.ksplit = ((K + splits - 1) / splits + BK - 1) / BK * BK;
  p.splits = (K + p.ksplit - 1) / p.ksplit;
  return p;
}

template <int TM, int TN, bool AK, bool BKc>
void launch_x3(bool even, dim3 grid, float* C, const float* A, const float* B, int M, int N, int K, int lda,
               int ldb, int beta, int ksplit, float* partial, const float* resid, const float* xpa,
               const float* xpb) {
  if (even)
    FG_LAUNCH_NOCHECK((gemm_x3_kernel<TM, TN, AK, BKc, false>), grid, dim3(kThreads), 0, C, A, B, M,
                       N, K, lda, ldb, beta, ksplit, partial, resid, xpa, xpb);
  else
    FG_LAUNCH_NOCHECK((gemm_x3_kernel<TM, TN, AK, BKc, true>), grid, dim3(kThreads), 0, C, A, B, M,
                       N, K, lda, ldb, beta, ksplit, partial, resid, xpa, xpb);
}

template <bool AK, bool BKc>
void launch_pq(bool even, dim3 grid, float* C, const float* A, const float* B, int M, int N, int K, int lda,
               int ldb, int beta, int ksplit, float* partial, const float* resid, const float* xpa,
               const float* xpb) {
  if (even)
    FG_LAUNCH_NOCHECK((gemm_pq_kernel<AK, BKc, false>), grid, dim3(kPPThreads), 0, C, A, B, M, N, K,
                       lda, ldb, beta, ksplit, partial, resid, xpa, xpb);
  else
    FG_LAUNCH_NOCHECK((gemm_pq_kernel<AK, BKc, true>), grid, dim3(kPPThreads), 0, C, A, B, M, N, K,
                       lda, ldb, beta, ksplit, partial, resid, xpa, xpb);
}

template <int TN, bool AK, bool BKc>
void launch_w(bool even, dim3 grid, float* C, const float* A, const float* B, int M, int N, int K, int lda, int ldb,
              int beta, int ksplit, float* partial, const float* resid, int n_full, int tail_c, float* slab,
              const float* xpa, const float* xpb) {
  if (even)
    FG_LAUNCH_NOCHECK((gemm_w_kernel<TN, AK, BKc, false>), grid, dim3(kPPThreads), 0, C, A, B, M, N, K, lda, ldb,
                       beta, ksplit, partial, resid, n_full, tail_c, slab, xpa, xpb);
  else
    FG_LAUNCH_NOCHECK((gemm_w_kernel<TN, AK, BKc, true>), grid, dim3(kPPThreads), 0, C, A, B, M, N, K, lda, ldb,
                       beta, ksplit, partial, resid, n_full, tail_c, slab, xpa, xpb);
}

template <int TM, int TN, bool AK, bool BKc>
void launch_pp(bool even, dim3 grid, float* C, const float* A, const float* B, int M, int N, int K, int lda,
               int ldb, int beta, int ksplit, float* partial, const float* resid, int n_full, int tail_c,
               float* slab, const float* xpa, const float* xpb) {
  if (even)
    FG_LAUNCH_NOCHECK((gemm_pp_kernel<TM, TN, AK, BKc, false>), grid, dim3(kPPThreads), 0, C, A, B,
                       M, N, K, lda, ldb, beta, ksplit, partial, resid, n_full, tail_c, slab, xpa, xpb);
  else
    FG_LAUNCH_NOCHECK((gemm_pp_kernel<TM, TN, AK, BKc, true>), grid, dim3(kPPThreads), 0, C, A, B,
                       M, N, K, lda, ldb, beta, ksplit, partial, resid, n_full, tail_c, slab, xpa, xpb);
}

// Tail split plan for `tiles` one-per-CU tiles of K k-range: number of tail
// tiles r (the last, partial round) and pieces per tile c (c = 1: none).
// The full rounds run first, then the r * c pieces (each 1/c of a tile's
// k-steps).  A last round at most half full is cut into c = CUs / r pieces
// (>= 4 k-steps of 32 each): one round of pieces.  A fuller last round is cut
// only over a long K (pieces of >= 16 k-steps, where a piece's fixed cost and
// its partial slab are small against its MFMA work): c minimises the
// ceil(r c / CUs) rounds of 1/c length, plus a small charge per piece (ties
// go to fewer pieces) — e.g. 135 tail tiles over K = 8192 on 256 CUs take 5
// rounds of 1/9 with c = 9 instead of one whole round.
struct TailPlan {
  int r, c;
};
TailPlan plan_tail(int64_t tiles, int K, int cus) {
  TailPlan t{0, 1};
  const int64_t r = tiles % cus;
  if (tiles < cus || r == 0) return t;
  const int nk = (K + BK - 1) / BK;
  if (2 * r <= cus) {
    int c = (int)(cus / r);
    if (c > nk / 4) c = nk / 4;
    if (c < 2) return t;
    t.r = (int)r;
    t.c = c;
    return t;
  }
  const int cmax = min(nk / 16, 32);
  double best = 1.0;
  for (int c = 2; c <= cmax; ++c) {
    const double cost = (double)((r * c + cus - 1) / cus) / c + 0.005 * c;
    if (cost < best - 1e-9) {
      best = cost;
      t.r = (int)r;
      t.c = c;
    }
  }
  return t;
}

// Queues C (+)= A·B on fg::stream(); split-K partials live in `ws`, which
// the caller keeps until the kernels are ordered before any later reuse.
// parts_out: the plan must split K in two; the two pieces' M x N partial sums
// are left in parts_out[0 .. 2MN) (piece z at z*M*N, nothing reduced, C not
// written): C = parts_out[0 .. MN) + parts_out[MN .. 2MN) in fp32 is what the
// reduce would store.
template <bool AK, bool BKc>
int launch_gemm(const char* name, fg::Workspace& ws, float* C, const float* A, const float* B, int M, int N, int K,
                int lda, int ldb, int beta, const float* resid = nullptr, float* parts_out = nullptr,
                bool scoped = true, const XpArgs& xp = XpArgs()) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(M > 0 && N > 0 && K >= 0 && (K > 0 || !parts_out), "%s: bad shape M=%d N=%d K=%d", name, M, N, K);
  FG_ARG_CHECK(C && (K == 0 || (A && B)), "%s: null pointer", name);
  if (K == 0) {
    if (!beta) {
      FG_LAUNCH(splitk_reduce_kernel, dim3(1), dim3(256), 0, C, C, (int64_t)M * N, 0, 0, resid);
    }
    return FG_OK;
  }
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  const GemmPlan pl = plan_gemm(AK, BKc, M, N, K, cus);
  FG_ARG_CHECK(!parts_out || (pl.splits == 2 && !beta && !resid),
               "%s: the plan for M=%d N=%d K=%d takes %d K pieces, not two", name, M, N, K, pl.splits);
  const int tiles = ((M + pl.tm - 1) / pl.tm) * ((N + pl.tn - 1) / pl.tn);
  // Fast path: every tile full and every vector access aligned.
  const bool even = (M % pl.tm == 0) && (N % pl.tn == 0) && (K % BK == 0) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                    ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0) && ((uintptr_t)C % 16 == 0) &&
                    (resid == nullptr || (uintptr_t)resid % 16 == 0);
  float* partial = parts_out;
  if (pl.splits > 1 && !partial) {
    int rc = ws.get(sizeof(float) * (size_t)pl.splits * M * N);
    if (rc) return rc;
    partial = (float*)ws.ptr;
  }
  TailPlan tp{0, 1};
  if (pl.pp && pl.splits == 1) tp = plan_tail(tiles, K, cus);
  float* slab = nullptr;
  if (tp.c > 1) {
    int rc = ws.get(sizeof(float) * (size_t)tp.r * tp.c * pl.tm * pl.tn);
    if (rc) return rc;
    slab = (float*)ws.ptr;
  }
  const int n_full = tiles - tp.r;
  dim3 grid(n_full + tp.r * tp.c, pl.splits);
  fg::Workspace wsx;
  const float *xpa, *xpb;
  {
    int rc = resolve_xp(xp, xp_job(A, AK, M, K, lda, nullptr), xp_job(B, BKc, N, K, ldb, nullptr), wsx, scoped, xpa,
                        xpb);
    if (rc) return rc;
  }
  // Profiler scope per layout family (gemm_x3_kernel<*, *, AK, BK, *>);
  // algorithmic work = 2MNK flop, compulsory bytes = A + B + C (+ C read when
  // accumulating, + the residual).
  fg::KProfScope prof(!scoped ? nullptr : AK ? (BKc ? "gemm_nt" : "gemm_nn") : "gemm_tn", 2.0 * M * N * (double)K,
                      4.0 * ((double)M * K + (double)N * K + (1.0 + (beta ? 1.0 : 0.0) + (resid ? 1.0 : 0.0)) * M * N));
  if (pl.w && pl.tn == 192)
    launch_w<192, AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, n_full, tp.c,
                           slab, xpa, xpb);
  else if (pl.w)
    launch_w<256, AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, n_full, tp.c,
                           slab, xpa, xpb);
  else if (pl.pq)
    launch_pq<AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, xpa, xpb);
  else if (pl.pp && pl.tm == 256)
    launch_pp<256, 128, AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, n_full,
                                 tp.c, slab, xpa, xpb);
  else if (pl.pp)
    launch_pp<128, 256, AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, n_full,
                                 tp.c, slab, xpa, xpb);
  else if (pl.tm == 128 && pl.tn == 128)
    launch_x3<128, 128, AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, xpa, xpb);
  else if (pl.tm == 128)
    launch_x3<128, 256, AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, xpa, xpb);
  else
    launch_x3<256, 128, AK, BKc>(even, grid, C, A, B, M, N, K, lda, ldb, beta, pl.ksplit, partial, resid, xpa, xpb);
  FG_HIP_CHECK(hipGetLastError());
  if (tp.c > 1) {
    const int per = pl.tm * pl.tn;
    FG_LAUNCH(tail_reduce_kernel, dim3((per + 255) / 256 < 32 ? (per + 255) / 256 : 32, tp.r), dim3(256), 0, C,
              resid, slab, M, N, pl.tm, pl.tn, n_full, tp.c, beta);
  }
  prof.end();
  if (pl.splits > 1 && !parts_out) {
    fg::KProfScope prof2(scoped ? "gemm_splitk_reduce" : nullptr, 0.0,
                         4.0 * (double)M * N * (pl.splits + 1 + (beta ? 1 : 0) + (resid ? 1 : 0)));
    int64_t n = (int64_t)M * N;
    int64_t blocks = (n / 4 + 255) / 256 + 1;
    if (blocks > 8LL * cus) blocks = 8LL * cus;
    FG_LAUNCH(splitk_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, C, partial, n, pl.splits, beta, resid);
  }
  return FG_OK;
}

}  // namespace

namespace fg {
int gemm_inner(bool a_k, bool b_k, Workspace& ws, float* C, const float* A, const float* B, int M, int N, int K,
               int lda, int ldb, int beta) {
  if (a_k && b_k)
    return launch_gemm<true, true>("gemm_inner", ws, C, A, B, M, N, K, lda, ldb, beta, nullptr, nullptr, false);
  if (a_k) return launch_gemm<true, false>("gemm_inner", ws, C, A, B, M, N, K, lda, ldb, beta, nullptr, nullptr, false);
  FG_ARG_CHECK(!b_k, "gemm_inner: A^T·B^T is not a layout of the GEMM kernels");
  return launch_gemm<false, false>("gemm_inner", ws, C, A, B, M, N, K, lda, ldb, beta, nullptr, nullptr, false);
}
int absmax_parts(const XpSpec* specs, int count, const char* prof_name) {
  FG_ARG_CHECK(count >= 0 && count <= kMaxXpSpecs, "absmax_parts: %d matrices", count);
  XpTable t;
  t.count = count;
  for (int i = 0; i < count; ++i) {
    FG_ARG_CHECK(specs[i].p && specs[i].out && specs[i].rows >= 0 && specs[i].cols >= 0 &&
                     (specs[i].rows <= 1 || specs[i].ld >= specs[i].cols),
                 "absmax_parts: bad matrix %d", i);
    t.job[i] = XpJob{specs[i].p, specs[i].out, specs[i].rows, specs[i].ld, specs[i].cols};
  }
  if (count == 0) return FG_OK;
  double bytes = 0.0;
  for (int i = 0; i < count; ++i) bytes += 4.0 * (double)t.job[i].rows * t.job[i].cols;
  KProfScope prof(prof_name, 0.0, bytes);
  FG_LAUNCH(absmax_kernel, dim3(kXpParts, t.count), dim3(kXpThreads), 0, t);
  return FG_OK;
}

template <bool AK, bool BKc>
int launch_batch(bool even, dim3 grid, float* C, const float* A, const float* B, int M, int N, int K, int lda, int ldb,
                 const GemmBatch& bt, const float* xpa, const float* xpb) {
  if (even)
    FG_LAUNCH((gemm_x3_batch_kernel<AK, BKc, false>), grid, dim3(kThreads), 0, C, A, B, M, N, K, lda, ldb, bt, xpa,
              xpb);
  else
    FG_LAUNCH((gemm_x3_batch_kernel<AK, BKc, true>), grid, dim3(kThreads), 0, C, A, B, M, N, K, lda, ldb, bt, xpa,
              xpb);
  return FG_OK;
}

int gemm_batched(bool a_k, bool b_k, float* C, const float* A, const float* B, int M, int N, int K, int lda, int ldb,
                 const GemmBatch& bt, int nz) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(M > 0 && N > 0 && K > 0 && nz > 0 && nz <= 65535 && bt.nh > 0 && bt.a.g > 0 && bt.b.g > 0,
               "gemm_batched: bad shape M=%d N=%d K=%d nz=%d", M, N, K, nz);
  FG_ARG_CHECK(C && A && B, "gemm_batched: null pointer");
  FG_ARG_CHECK(a_k || !b_k, "gemm_batched: A^T·B^T is not a layout of the GEMM kernels");
  FG_ARG_CHECK(bt.causal >= 0 && bt.causal <= 3 && (bt.causal != 1 || M == N) && (bt.causal < 2 || M == K),
               "gemm_batched: causal mode %d needs a square attention matrix (M=%d N=%d K=%d)", bt.causal, M, N, K);
  auto al4 = [](const BatchOperand& o) { return o.local ? o.sz % 4 == 0 : (o.sb % 4 == 0 && o.sh % 4 == 0); };
  const bool even = (M % BM == 0) && (N % BM == 0) && (K % BK == 0) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                    ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0) && ((uintptr_t)C % 16 == 0) && al4(bt.a) &&
                    al4(bt.b) && bt.sc % 4 == 0;
  const dim3 grid(((M + BM - 1) / BM) * ((N + BM - 1) / BM), 1, nz);
  fg::Workspace wsx;
  const float *xpa, *xpb;
  {  // exponents over the memory every problem's operand lies in
    auto span = [&](const BatchOperand& o, const float* p, int64_t extent) {
      int64_t lo = INT64_MAX, hi = 0;
      for (int zl = 0; zl < nz; ++zl) {
        const int z = bt.z0 + zl, b = z / bt.nh, h = z - b * bt.nh;
        const int64_t off = batch_offset(o, zl, b, h);
        lo = off < lo ? off : lo;
        hi = off > hi ? off : hi;
      }
      return XpJob{p + lo, nullptr, hi + extent - lo, 1, 1};
    };
    int rc = resolve_xp(XpArgs(), span(bt.a, A, a_k ? (int64_t)(M - 1) * lda + K : (int64_t)(K - 1) * lda + M),
                        span(bt.b, B, b_k ? (int64_t)(N - 1) * ldb + K : (int64_t)(K - 1) * ldb + N), wsx, false, xpa,
                        xpb);
    if (rc) return rc;
  }
  if (a_k && b_k) return launch_batch<true, true>(even, grid, C, A, B, M, N, K, lda, ldb, bt, xpa, xpb);
  if (a_k) return launch_batch<true, false>(even, grid, C, A, B, M, N, K, lda, ldb, bt, xpa, xpb);
  return launch_batch<false, false>(even, grid, C, A, B, M, N, K, lda, ldb, bt, xpa, xpb);
}
}  // namespace fg

extern "C" int fg_matmulT_fwd_p(float* Y, const float* X, const float* W, int M, int K, int N, float* xp_x,
                                float* xp_w, int have) {
  // Y[M,N] = X[M,K] · W[N,K]^T : A(i=m, r=k) = X[m*K+k], B(r=k, j=n) = W[n*K+k]
  fg::Workspace ws;
  return launch_gemm<true, true>("matmulT_fwd", ws, Y, X, W, M, N, K, K, K, 0, nullptr, nullptr, true,
                                 XpArgs{xp_x, xp_w, have});
}

extern "C" int fg_matmulT_fwd(float* Y, const float* X, const float* W, int M, int K, int N) {
  return fg_matmulT_fwd_p(Y, X, W, M, K, N, nullptr, nullptr, 0);
}

extern "C" int fg_matmulT_fwd_swiglu(float* O, float* GU, const float* X, const float* Wgu, int M, int K, int H) {
  return fg_matmulT_fwd_swiglu_p(O, GU, X, Wgu, M, K, H, nullptr, nullptr, 0);
}

extern "C" int fg_matmulT_fwd_swiglu_p(float* O, float* GU, const float* X, const float* Wgu, int M, int K, int H,
                                       float* xp_x, float* xp_w, int have) {
  // GU[M, 2H] = X[M,K] · Wgu[2H,K]^T (Wgu = [Wg; Wu]), O[M,H] = SwiGLU(GU[:, :H], GU[:, H:])
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(M > 0 && K > 0 && H > 0, "fg_matmulT_fwd_swiglu: bad shape M=%d K=%d H=%d", M, K, H);
  FG_ARG_CHECK(O && GU && X && Wgu, "fg_matmulT_fwd_swiglu: null pointer");
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  const GemmPlan pl = plan_gemm(true, true, M, 2 * H, K, cus);
  const bool fused = pl.w && pl.tn == 256 && pl.splits == 1 && M % 256 == 0 && H % 128 == 0 && K % BK == 0 &&
                     (int64_t)(M / 256) * (2 * H / 256) % cus == 0 && (uintptr_t)X % 16 == 0 &&
                     (uintptr_t)Wgu % 16 == 0 && (uintptr_t)GU % 16 == 0;
  if (!fused) {  // the GEMM, then the SwiGLU pass
    fg::Workspace ws;
    int rc = launch_gemm<true, true>("matmulT_fwd", ws, GU, X, Wgu, M, 2 * H, K, K, K, 0, nullptr, nullptr, true,
                                     XpArgs{xp_x, xp_w, have});
    if (rc) return rc;
    return fg_swiglu_gu_fwd(O, GU, M, H);
  }
  fg::Workspace wsx;
  const float *xpa, *xpb;
  {
    int rc = resolve_xp(XpArgs{xp_x, xp_w, have}, xp_job(X, true, M, K, K, nullptr),
                        xp_job(Wgu, true, 2 * H, K, K, nullptr), wsx, true, xpa, xpb);
    if (rc) return rc;
  }
  fg::KProfScope prof("gemm_nt", 2.0 * M * 2.0 * H * K,
                      4.0 * ((double)M * K + 2.0 * H * K + 3.0 * (double)M * H));
  const int ntiles = (M / 256) * (2 * H / 256);
  FG_LAUNCH(gemm_w_swiglu_kernel, dim3(ntiles), dim3(kPPThreads), 0, O, GU, X, Wgu, M, K, H, xpa, xpb);
  return FG_OK;
}

extern "C" int fg_matmulT_bwd_x_p(float* gX, const float* gY, const float* W, int M, int K, int N, int beta,
                                  float* xp_gy, float* xp_w, int have) {
  // gX[M,K] = gY[M,N] · W[N,K] : A(i=m, r=n) = gY[m*N+n], B(r=n, j=k) = W[n*K+k]
  fg::Workspace ws;
  return launch_gemm<true, false>("matmulT_bwd_x", ws, gX, gY, W, M, K, N, N, K, beta, nullptr, nullptr, true,
                                  XpArgs{xp_gy, xp_w, have});
}

extern "C" int fg_matmulT_bwd_x(float* gX, const float* gY, const float* W, int M, int K, int N, int beta) {
  return fg_matmulT_bwd_x_p(gX, gY, W, M, K, N, beta, nullptr, nullptr, 0);
}

extern "C" int fg_matmulT_bwd_x_pieces(int M, int K, int N) {
  FG_ARG_CHECK(M > 0 && K > 0 && N > 0, "fg_matmulT_bwd_x_pieces: bad shape M=%d K=%d N=%d", M, K, N);
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  return plan_gemm(true, false, M, K, N, cus).splits;
}

extern "C" int fg_matmulT_bwd_x_halves_p(float* gX_halves, const float* gY, const float* W, int M, int K, int N,
                                         float* xp_gy, float* xp_w, int have) {
  // fg_matmulT_bwd_x's two K pieces, unreduced: gX = gX_halves[0 .. MK) + gX_halves[MK .. 2MK)
  fg::Workspace ws;
  FG_ARG_CHECK(gX_halves, "fg_matmulT_bwd_x_halves: null pointer");
  return launch_gemm<true, false>("matmulT_bwd_x_halves", ws, gX_halves, gY, W, M, K, N, N, K, 0, nullptr, gX_halves,
                                  true, XpArgs{xp_gy, xp_w, have});
}

extern "C" int fg_matmulT_bwd_x_halves(float* gX_halves, const float* gY, const float* W, int M, int K, int N) {
  return fg_matmulT_bwd_x_halves_p(gX_halves, gY, W, M, K, N, nullptr, nullptr, 0);
}

extern "C" int fg_matmulT_bwd_w_p(float* gW, const float* gY, const float* X, int M, int K, int N, int beta,
                                  float* xp_gy, float* xp_x, int have) {
  // gW[N,K] = gY^T · X : A(i=n, r=m) = gY[m*N+n], B(r=m, j=k) = X[m*K+k]
  fg::Workspace ws;
  return launch_gemm<false, false>("matmulT_bwd_w", ws, gW, gY, X, N, K, M, N, K, beta, nullptr, nullptr, true,
                                   XpArgs{xp_gy, xp_x, have});
}

extern "C" int fg_matmulT_bwd_w(float* gW, const float* gY, const float* X, int M, int K, int N, int beta) {
  return fg_matmulT_bwd_w_p(gW, gY, X, M, K, N, beta, nullptr, nullptr, 0);
}

extern "C" int fg_matmulT_bwd_w_grouped(const fg_wgrad_job* jobs, int count) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(count >= 0 && (count == 0 || jobs), "fg_matmulT_bwd_w_grouped: bad job list");
  // 256x256 tiles (gemm_w_grouped) when they make at least two rounds of
  // CUs, else 128x256 ping-pong tiles (twice as many to spread)
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  int64_t w_tiles = 0;
  for (int i = 0; i < count; ++i)
    w_tiles += (int64_t)((jobs[i].N + 255) / 256) * ((jobs[i].K + 255) / 256);
  const bool wide = w_tiles >= 2 * cus;
  const int TM = wide ? 256 : 128, TN = 256;
  GTable t;
  double flop = 0.0, bytes = 0.0;
  auto flush = [&]() -> int {
    if (t.count == 0) return FG_OK;
    // the maxima the jobs do not bring, into one workspace
    fg::Workspace wsx;
    {
      int missing = 0;
      for (int j = 0; j < t.count; ++j) missing += (t.job[j].xpa == nullptr) + (t.job[j].xpb == nullptr);
      XpTable xt;
      xt.count = 0;
      if (missing) {
        int rc = wsx.get((size_t)missing * kXpParts * sizeof(float));
        if (rc) return rc;
        float* next = static_cast<float*>(wsx.ptr);
        for (int j = 0; j < t.count; ++j) {
          GJob& g = t.job[j];
          if (!g.xpa) {
            xt.job[xt.count++] = xp_job(g.A, false, g.M, g.K, g.lda, next);
            g.xpa = next;
            next += kXpParts;
          }
          if (!g.xpb) {
            xt.job[xt.count++] = xp_job(g.B, false, g.N, g.K, g.ldb, next);
            g.xpb = next;
            next += kXpParts;
          }
        }
      }
      int rc = queue_absmax(xt, true);
      if (rc) return rc;
    }
    fg::KProfScope prof("gemm_tn", flop, bytes);
    // tail split over the whole launch, pieces sized by the smallest job K
    const int tiles = t.prefix[t.count];
    int kmin = t.job[0].K;
    for (int j = 1; j < t.count; ++j) kmin = min(kmin, t.job[j].K);
    const TailPlan tp = plan_tail(tiles, kmin, cus);
    fg::Workspace ws;
    t.n_full = tiles - tp.r;
    t.tail_c = tp.c;
    t.slab = nullptr;
    if (tp.c > 1) {
      int rc = ws.get(sizeof(float) * (size_t)tp.r * tp.c * TM * TN);
      if (rc) return rc;
      t.slab = (float*)ws.ptr;
    }
    if (wide) {
      FG_LAUNCH((gemm_w_grouped<false, false>), dim3(t.n_full + tp.r * tp.c), dim3(kPPThreads), 0, t);
      if (tp.c > 1) FG_LAUNCH((tail_reduce_grouped<256, 256>), dim3(32, tp.r), dim3(256), 0, t);
    } else {
      FG_LAUNCH((gemm_pp_grouped<128, 256, false, false>), dim3(t.n_full + tp.r * tp.c), dim3(kPPThreads), 0, t);
      if (tp.c > 1) FG_LAUNCH((tail_reduce_grouped<128, 256>), dim3(32, tp.r), dim3(256), 0, t);
    }
    t.count = 0;
    flop = bytes = 0.0;
    return FG_OK;
  };
  t.count = 0;
  t.prefix[0] = 0;
  for (int i = 0; i < count; ++i) {
    const fg_wgrad_job& jb = jobs[i];
    FG_ARG_CHECK(jb.gW && jb.gY && jb.X && jb.M > 0 && jb.K > 0 && jb.N > 0,
                 "fg_matmulT_bwd_w_grouped: job %d has a null pointer or a bad shape (M=%d K=%d N=%d)", i, jb.M,
                 jb.K, jb.N);
    // a job on a gW already written by this table's jobs starts the next
    // launch, so jobs on one output apply in list order
    for (int j = 0; j < t.count; ++j) {
      if (t.job[j].C == jb.gW) {
        int rc = flush();
        if (rc) return rc;
        break;
      }
    }
    // gW[N,K] (+)= gY^T · X: the TN layout of fg_matmulT_bwd_w, M_gemm = N, N_gemm = K, K_gemm = M
    const int Mg = jb.N, Ng = jb.K, Kg = jb.M;
    const int tiles = ((Mg + TM - 1) / TM) * ((Ng + TN - 1) / TN);
    FG_ARG_CHECK((int64_t)t.prefix[t.count] + tiles < (1ll << 31), "fg_matmulT_bwd_w_grouped: too many tiles");
    GJob& g = t.job[t.count];
    g.C = jb.gW;
    g.A = jb.gY;
    g.B = jb.X;
    g.xpa = jb.xp_gy;
    g.xpb = jb.xp_x;
    g.M = Mg;
    g.N = Ng;
    g.K = Kg;
    g.lda = jb.N;
    g.ldb = jb.K;
    g.beta = jb.beta ? 1 : 0;
    g.even = (Mg % TM == 0) && (Ng % TN == 0) && (Kg % BK == 0) && (g.lda % 4 == 0) && (g.ldb % 4 == 0) &&
             ((uintptr_t)g.A % 16 == 0) && ((uintptr_t)g.B % 16 == 0) && ((uintptr_t)g.C % 16 == 0);
    t.prefix[t.count + 1] = t.prefix[t.count] + tiles;
    t.count += 1;
    flop += 2.0 * Mg * Ng * (double)Kg;
    bytes += 4.0 * ((double)Mg * Kg + (double)Ng * Kg + (1.0 + g.beta) * Mg * Ng);
    if (t.count == kMaxJobs) {
      int rc = flush();
      if (rc) return rc;
    }
  }
  return flush();
}

extern "C" int fg_matmulT_bwd_p(float* gX, int beta_x, float* gW, int beta_w, const float* gY, const float* X,
                                const float* W, int M, int K, int N, float* xp_gy, float* xp_x, float* xp_w,
                                int have) {
  // Both gradients of Y = X·W^T, gX first (so an aliased gW accumulates onto it);
  // gY's maxima, filled for the first GEMM, serve the second.
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(gX && gW && gY && X && W, "fg_matmulT_bwd: null pointer");
  fg::Workspace wsg;
  if (!xp_gy) {
    int rc = wsg.get(kXpParts * sizeof(float));
    if (rc) return rc;
    xp_gy = static_cast<float*>(wsg.ptr);
    have &= ~1;
  }
  {
    fg::Workspace ws;
    int rc = launch_gemm<true, false>("matmulT_bwd_x", ws, gX, gY, W, M, K, N, N, K, beta_x, nullptr, nullptr, true,
                                      XpArgs{xp_gy, xp_w, (have & 1) | ((have >> 1) & 2)});
    if (rc) return rc;
  }
  fg::Workspace ws;
  return launch_gemm<false, false>("matmulT_bwd_w", ws, gW, gY, X, N, K, M, N, K, beta_w, nullptr, nullptr, true,
                                   XpArgs{xp_gy, xp_x, 1 | (have & 2)});
}

extern "C" int fg_matmulT_bwd(float* gX, int beta_x, float* gW, int beta_w, const float* gY, const float* X,
                              const float* W, int M, int K, int N) {
  return fg_matmulT_bwd_p(gX, beta_x, gW, beta_w, gY, X, W, M, K, N, nullptr, nullptr, nullptr, 0);
}

extern "C" int fg_matmulT_fwd_rope(float* Y, const float* X, const float* W, int M, int K, int N,
                                   const double* cos_tab, const double* sin_tab, int npos, int nH, int nKV, int dH,
                                   int pos0, int posStride) {
  return fg_matmulT_fwd_rope_p(Y, X, W, M, K, N, cos_tab, sin_tab, npos, nH, nKV, dH, pos0, posStride, nullptr,
                               nullptr, 0);
}

extern "C" int fg_matmulT_fwd_rope_p(float* Y, const float* X, const float* W, int M, int K, int N,
                                     const double* cos_tab, const double* sin_tab, int npos, int nH, int nKV, int dH,
                                     int pos0, int posStride, float* xp_x, float* xp_w, int have) {
  // Y[M,N] = X·W^T, then the q and k column pairs of each row rotated in place
  // (one pass over those columns: 8 B per element, against the 16 B per pair
  // plus the v copy of a separate q/k/v split)
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(cos_tab && sin_tab, "fg_matmulT_fwd_rope: null table");
  FG_ARG_CHECK(nH > 0 && nKV > 0 && dH > 0 && dH % 2 == 0 && (int64_t)(nH + nKV) * dH <= N,
               "fg_matmulT_fwd_rope: heads nH=%d nKV=%d dH=%d do not fit N=%d", nH, nKV, dH, N);
  FG_ARG_CHECK(M > 0 && pos0 >= 0 && posStride >= 0, "fg_matmulT_fwd_rope: bad rows/positions");
  const int maxpos = pos0 + (posStride > 0 ? (M < posStride ? M : posStride) : M) - 1;
  FG_ARG_CHECK(maxpos < npos, "fg_matmulT_fwd_rope: positions up to %d exceed the %d-entry table", maxpos, npos);
  {
    fg::Workspace ws;
    int rc = launch_gemm<true, true>("matmulT_fwd_rope", ws, Y, X, W, M, N, K, K, K, 0, nullptr, nullptr, true,
                                     XpArgs{xp_x, xp_w, have});
    if (rc) return rc;
  }
  const RopeEpi re{cos_tab, sin_tab, (nH + nKV) * dH, dH, pos0, posStride};
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  fg::KProfScope prof("qkv_rope_fwd", 0.0, 8.0 * M * (double)re.cols);
  const bool quad = dH % 4 == 0 && N % 4 == 0 && (uintptr_t)Y % 16 == 0 && (uintptr_t)cos_tab % 16 == 0 &&
                    (uintptr_t)sin_tab % 16 == 0;
  const int64_t work = (int64_t)M * (quad ? re.cols / 4 : re.cols / 2);
  int64_t blocks = (work + 255) / 256;
  if (blocks > 16LL * cus) blocks = 16LL * cus;
  if (quad)
    FG_LAUNCH(rope_cols4_kernel, dim3((unsigned)blocks), dim3(256), 0, Y, M, N, re);
  else
    FG_LAUNCH(rope_cols_kernel, dim3((unsigned)blocks), dim3(256), 0, Y, M, N, re);
  return FG_OK;
}

extern "C" int fg_matmulT_fwd_resid_p(float* Y, const float* R, const float* X, const float* W, int M, int K, int N,
                                      float* xp_x, float* xp_w, int have) {
  // Y[M,N] = R[M,N] + X[M,K] · W[N,K]^T
  FG_ARG_CHECK(R != nullptr, "fg_matmulT_fwd_resid: null residual");
  fg::Workspace ws;
  return launch_gemm<true, true>("matmulT_fwd_resid", ws, Y, X, W, M, N, K, K, K, 0, R, nullptr, true,
                                 XpArgs{xp_x, xp_w, have});
}

extern "C" int fg_matmulT_fwd_resid(float* Y, const float* R, const float* X, const float* W, int M, int K, int N) {
  return fg_matmulT_fwd_resid_p(Y, R, X, W, M, K, N, nullptr, nullptr, 0);
}
