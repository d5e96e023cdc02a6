// fp32 MFMA GEMMs behind matmulT (tensor.js:34-53) for gfx950.
//
//   forward  Y [M,N]  = X[M,K]  · W[N,K]^T      A k-contiguous, B k-contiguous ("NT")
//   input    gX[M,K] (+)= gY[M,N] · W[N,K]      A k-contiguous, B j-contiguous ("NN")
//   weight   gW[N,K] (+)= gY[M,N]^T · X[M,K]    A i-contiguous, B j-contiguous ("TN")
//
// One kernel template covers the three layouts: C[i,j] = sum_r A(i,r) B(r,j).
// Workgroup tile 128x128, k-step 32, 256 threads = 4 waves in a 2x2 grid; each
// wave owns a 64x64 sub-tile = 2x2 v_mfma_f32_32x32x2_f32 accumulators (64
// fp32 accumulators per lane).  Global tiles are loaded as float4 into
// registers one k-step ahead, then written to LDS (+4 float padding per row);
// MFMA operands are read from LDS with ds_read_b128 (k-contiguous operand) or
// ds_read_b32 (i/j-contiguous operand).
//
// Reduction order inside a k-step is permuted (lane half h of the wave feeds
// k = h*16 + s at MFMA step s); the sum is over the same terms.
//
// Launch shape: 1-D grid of tiles remapped so each of the 8 XCDs gets a
// contiguous range, then grouped 8 tile-rows at a time for L2 reuse.  When the
// tile count cannot fill the chip, K is split across gridDim.y and partial
// tiles are summed by a second kernel in a fixed order (deterministic).
#include "common.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int kThreads = 256;
constexpr int PADK = 4;         // k-contiguous LDS rows: BK + 4 floats
constexpr int PADI = 4;         // i/j-contiguous LDS rows: BM + 4 floats
constexpr int kXCD = 8;
constexpr int kGroupM = 8;

template <bool KC>
struct Tile {
  // LDS footprint of one operand tile (floats)
  static constexpr int kFloats = KC ? BM * (BK + PADK) : BK * (BM + PADI);
};

// One float4 of the 128xBK tile of an operand starting at (row0, k0); u in
// [0,4) selects which of the thread's four.  KC: element (i,k) at
// base[i*ld + k]; else base[k*ld + i].  Returned by value so the prefetch
// stays in VGPRs.
template <bool KC, bool CHECKED>
__device__ __forceinline__ float4 load4(const float* __restrict__ base, int ld, int rows, int kdim, int row0, int k0,
                                        int u) {
  const int t = threadIdx.x;
  int i, k;
  if (KC) {
    i = row0 + (t >> 3) + 32 * u;
    k = k0 + (t & 7) * 4;
  } else {
    k = k0 + (t >> 5) + 8 * u;
    i = row0 + (t & 31) * 4;
  }
  if (!CHECKED) {
    const float* p = KC ? base + (size_t)i * ld + k : base + (size_t)k * ld + i;
    return *reinterpret_cast<const float4*>(p);
  }
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int ii = KC ? i : i + e, kk = KC ? k + e : k;
    v[e] = (ii < rows && kk < kdim) ? (KC ? base[(size_t)ii * ld + kk] : base[(size_t)kk * ld + ii]) : 0.f;
  }
  return make_float4(v[0], v[1], v[2], v[3]);
}

template <bool KC>
__device__ __forceinline__ void store4(float* __restrict__ lds, int u, float4 v) {
  const int t = threadIdx.x;
  const int off = KC ? ((t >> 3) + 32 * u) * (BK + PADK) + (t & 7) * 4 : ((t >> 5) + 8 * u) * (BM + PADI) + (t & 31) * 4;
  *reinterpret_cast<float4*>(lds + off) = v;
}

// Operand fragment for rows [rb*32, rb*32+32) of the tile: frag[s] is the
// value this lane feeds at MFMA step s (row = lane%32, k = h*16 + s).
template <bool KC>
__device__ __forceinline__ void read_frag(float (&f)[16], const float* __restrict__ lds, int rowbase) {
  const int lane = threadIdx.x & 63;
  const int i = rowbase + (lane & 31), h = lane >> 5;
  if (KC) {
    const float4* p = reinterpret_cast<const float4*>(lds + i * (BK + PADK) + h * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 v = p[q];
      f[4 * q + 0] = v.x; f[4 * q + 1] = v.y; f[4 * q + 2] = v.z; f[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int s = 0; s < 16; ++s) f[s] = lds[(h * 16 + s) * (BM + PADI) + i];
  }
}

__device__ __forceinline__ int remap_xcd(int pid, int npid) {
  int per = (npid + kXCD - 1) / kXCD;
  int tall = npid % kXCD;
  if (tall == 0) tall = kXCD;
  int xcd = pid % kXCD, local = pid / kXCD;
  return xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
}

// C = (beta ? C : 0) + (resid ? resid : 0) + A·B over the K range of split
// blockIdx.y.  When `partial` is set the raw tile is written to
// partial + blockIdx.y*M*N (the reduce kernel applies beta and resid).
template <bool AK, bool BKc, bool CHECKED>
__global__ void __launch_bounds__(kThreads, 2)
    gemm_kernel(float* __restrict__ C, const float* __restrict__ A, const float* __restrict__ B, int M, int N,
                int K, int lda, int ldb, int beta, int ksplit, float* __restrict__ partial,
                const float* __restrict__ resid) {
  __shared__ __attribute__((aligned(16))) float As[Tile<AK>::kFloats];
  __shared__ __attribute__((aligned(16))) float Bs[Tile<BKc>::kFloats];

  const int nTm = (M + BM - 1) / BM, nTn = (N + BN - 1) / BN;
  const int ntiles = nTm * nTn;
  int pid = remap_xcd(blockIdx.x, ntiles);
  const int in_group = kGroupM * nTn;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int gsize = min(nTm - first_m, kGroupM);
  const int tm = first_m + (pid % in_group) % gsize;
  const int tn = (pid % in_group) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int kbeg = blockIdx.y * ksplit;
  const int kend = min(K, kbeg + ksplit);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.f;

  float4 a0, a1, a2, a3, b0, b1, b2, b3;
#define FG_GEMM_LOAD(k0)                                       \
  a0 = load4<AK, CHECKED>(A, lda, M, kend, m0, (k0), 0);       \
  a1 = load4<AK, CHECKED>(A, lda, M, kend, m0, (k0), 1);       \
  a2 = load4<AK, CHECKED>(A, lda, M, kend, m0, (k0), 2);       \
  a3 = load4<AK, CHECKED>(A, lda, M, kend, m0, (k0), 3);       \
  b0 = load4<BKc, CHECKED>(B, ldb, N, kend, n0, (k0), 0);      \
  b1 = load4<BKc, CHECKED>(B, ldb, N, kend, n0, (k0), 1);      \
  b2 = load4<BKc, CHECKED>(B, ldb, N, kend, n0, (k0), 2);      \
  b3 = load4<BKc, CHECKED>(B, ldb, N, kend, n0, (k0), 3);
  if (nk > 0) {
    FG_GEMM_LOAD(kbeg)
  }
  for (int it = 0; it < nk; ++it) {
    store4<AK>(As, 0, a0); store4<AK>(As, 1, a1); store4<AK>(As, 2, a2); store4<AK>(As, 3, a3);
    store4<BKc>(Bs, 0, b0); store4<BKc>(Bs, 1, b1); store4<BKc>(Bs, 2, b2); store4<BKc>(Bs, 3, b3);
    __syncthreads();
    if (it + 1 < nk) {
      FG_GEMM_LOAD(kbeg + (it + 1) * BK)
    }
#undef FG_GEMM_LOAD
    float fa[2][16], fb[2][16];
    read_frag<AK>(fa[0], As, wm * 64);
    read_frag<AK>(fa[1], As, wm * 64 + 32);
    read_frag<BKc>(fb[0], Bs, wn * 64);
    read_frag<BKc>(fb[1], Bs, wn * 64 + 32);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[0][s], fb[0][s], acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[0][s], fb[1][s], acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[1][s], fb[0][s], acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[1][s], fb[1][s], acc[1][1], 0, 0, 0);
    }
    __syncthreads();
  }

  // Epilogue: lane holds C[i][j] with j = lane%32, i = 8*(v/4) + 4*(lane/32) + v%4.
  const int lane = threadIdx.x & 63;
  float* out = partial ? partial + (size_t)blockIdx.y * M * N : C;
  const int use_beta = partial ? 0 : beta;
  const float* rs = partial ? nullptr : resid;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int j = n0 + wn * 64 + b * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = m0 + wm * 64 + a * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (!CHECKED || (i < M && j < N)) {
          float* p = out + (size_t)i * N + j;
          float r = acc[a][b][v];
          if (use_beta) r += *p;
          if (rs) r += rs[(size_t)i * N + j];
          *p = r;
        }
      }
    }
}

// C = resid + ((beta ? C : 0) + sum_z partial[z])  (fixed order over z).
__global__ void __launch_bounds__(256) splitk_reduce_kernel(float* __restrict__ C, const float* __restrict__ partial,
                                                            int64_t n, int splits, int beta,
                                                            const float* __restrict__ resid) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  // float4 path: C and resid 16-byte aligned, every partial slab too (pool-aligned base, n % 4 == 0)
  const bool vec = (((uintptr_t)C | (uintptr_t)resid) & 15) == 0 && (n & 3) == 0;
  for (; i < n; i += stride) {
    if (vec && i + 4 <= n) {
      float4 s = beta ? *reinterpret_cast<const float4*>(C + i) : make_float4(0.f, 0.f, 0.f, 0.f);
      for (int z = 0; z < splits; ++z) {
        float4 p = *reinterpret_cast<const float4*>(partial + (size_t)z * n + i);
        s.x += p.x; s.y += p.y; s.z += p.z; s.w += p.w;
      }
      if (resid) {  // added last: the value of resid + (the product as matmulT stores it)
        const float4 q = *reinterpret_cast<const float4*>(resid + i);
        s.x = q.x + s.x; s.y = q.y + s.y; s.z = q.z + s.z; s.w = q.w + s.w;
      }
      *reinterpret_cast<float4*>(C + i) = s;
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

template <bool AK, bool BKc>
int launch_gemm(const char* name, float* C, const float* A, const float* B, int M, int N, int K, int lda, int ldb,
                int beta, const float* resid = nullptr) {
  FG_REQUIRE_INIT();
  FG_ARG_CHECK(M > 0 && N > 0 && K >= 0, "%s: bad shape M=%d N=%d K=%d", name, M, N, K);
  FG_ARG_CHECK(C && (K == 0 || (A && B)), "%s: null pointer", name);
  if (K == 0) {
    if (!beta) {
      FG_LAUNCH(splitk_reduce_kernel, dim3(1), dim3(256), 0, C, C, (int64_t)M * N, 0, 0, resid);
    }
    return FG_OK;
  }
  const int nTm = (M + BM - 1) / BM, nTn = (N + BN - 1) / BN;
  const int tiles = nTm * nTn;
  // Fast path: every tile full and every float4 aligned.
  const bool even = (M % BM == 0) && (N % BN == 0) && (K % BK == 0) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                    ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0) && ((uintptr_t)C % 16 == 0) &&
                    (resid == nullptr || (uintptr_t)resid % 16 == 0);
  // Split K until the grid holds ~2 workgroups per CU, keeping >= 8 k-steps per split.
  const int cus = fg::device_cu_count() > 0 ? fg::device_cu_count() : 256;
  int splits = 1;
  while ((int64_t)tiles * splits < 2LL * cus && K / (splits * 2) >= 8 * BK) splits *= 2;
  int ksplit = ((K + splits - 1) / splits + BK - 1) / BK * BK;
  splits = (K + ksplit - 1) / ksplit;
  fg::Workspace ws;
  float* partial = nullptr;
  if (splits > 1) {
    int rc = ws.get(sizeof(float) * (size_t)splits * M * N);
    if (rc) return rc;
    partial = (float*)ws.ptr;
  }
  dim3 grid(tiles, splits);
  // Profiler scope per kernel family: the name matches the launched symbol
  // (gemm_kernel<AK,BK,*>); algorithmic work = 2MNK flop, compulsory bytes =
  // A + B + C (+ C read when accumulating).
  fg::KProfScope prof(AK ? (BKc ? "gemm_nt" : "gemm_nn") : "gemm_tn", 2.0 * M * N * (double)K,
                      4.0 * ((double)M * K + (double)N * K + (1.0 + (beta ? 1.0 : 0.0) + (resid ? 1.0 : 0.0)) * M * N));
  if (even)
    FG_LAUNCH((gemm_kernel<AK, BKc, false>), grid, dim3(kThreads), 0, C, A, B, M, N, K, lda, ldb, beta, ksplit,
              partial, resid);
  else
    FG_LAUNCH((gemm_kernel<AK, BKc, true>), grid, dim3(kThreads), 0, C, A, B, M, N, K, lda, ldb, beta, ksplit,
              partial, resid);
  prof.end();
  if (splits > 1) {
    fg::KProfScope prof2("gemm_splitk_reduce", 0.0,
                         4.0 * (double)M * N * (splits + 1 + (beta ? 1 : 0) + (resid ? 1 : 0)));
    int64_t n = (int64_t)M * N;
    int64_t blocks = (n / 4 + 255) / 256 + 1;
    if (blocks > 8LL * cus) blocks = 8LL * cus;
    FG_LAUNCH(splitk_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, C, partial, n, splits, beta, resid);
  }
  return FG_OK;
}

}  // namespace

extern "C" int fg_matmulT_fwd(float* Y, const float* X, const float* W, int M, int K, int N) {
  // Y[M,N] = X[M,K] · W[N,K]^T : A(i=m, r=k) = X[m*K+k], B(r=k, j=n) = W[n*K+k]
  return launch_gemm<true, true>("matmulT_fwd", Y, X, W, M, N, K, K, K, 0);
}

extern "C" int fg_matmulT_bwd_x(float* gX, const float* gY, const float* W, int M, int K, int N, int beta) {
  // gX[M,K] = gY[M,N] · W[N,K] : A(i=m, r=n) = gY[m*N+n], B(r=n, j=k) = W[n*K+k]
  return launch_gemm<true, false>("matmulT_bwd_x", gX, gY, W, M, K, N, N, K, beta);
}

extern "C" int fg_matmulT_bwd_w(float* gW, const float* gY, const float* X, int M, int K, int N, int beta) {
  // gW[N,K] = gY^T · X : A(i=n, r=m) = gY[m*N+n], B(r=m, j=k) = X[m*K+k]
  return launch_gemm<false, false>("matmulT_bwd_w", gW, gY, X, N, K, M, N, K, beta);
}

extern "C" int fg_matmulT_fwd_resid(float* Y, const float* R, const float* X, const float* W, int M, int K, int N) {
  // Y[M,N] = R[M,N] + X[M,K] · W[N,K]^T
  FG_ARG_CHECK(R != nullptr, "fg_matmulT_fwd_resid: null residual");
  return launch_gemm<true, true>("matmulT_fwd_resid", Y, X, W, M, N, K, K, K, 0, R);
}
