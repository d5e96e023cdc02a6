/*
 * forge_hip.h — C ABI of the MI355X (gfx950) training-path library.
 *
 * This is the drop-in boundary for the tensor-level fused forward+backward
 * training path of forge-llm (src/L2/tensor.js, src/L2/autograd.js,
 * src/L6/train.js).  The JavaScript host (forge-llm_amd/src) reaches it through
 * the N-API addon forge-llm_amd/csrc/napi_addon.cpp; any other FFI (ctypes,
 * cgo, JNI) can bind it directly: plain pointers, sizes and scalars only.
 *
 * Conventions
 *  - Every entry point returns int: 0 on success, a negative FG_ERR_* code on
 *    failure; fg_last_error() then returns a message (thread-local).
 *  - Tensors are fp32, row-major, resident in device memory obtained from
 *    fg_malloc (or any hipMalloc'd memory of the current device).
 *  - All kernels run in order on one internal HIP stream; entry points return
 *    as soon as the work is queued.  fg_d2h / fg_h2d / fg_sync synchronise.
 *  - "beta" arguments select first-write (0: out = result) or accumulate
 *    (1: out += result); they implement the reference's `grad ??= zeros`
 *    followed by `+=` without a separate zero-fill pass.
 *  - Scalar hyper-parameters (eps, lr_t, bias corrections, RoPE tables) are
 *    computed on the host in fp64 and passed by value / as tables.
 */
#ifndef FORGE_HIP_H
#define FORGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FG_OK 0
#define FG_ERR_ARG (-1)   /* invalid shape / argument (nothing was queued) */
#define FG_ERR_HIP (-2)   /* HIP runtime error */
#define FG_ERR_OOM (-3)   /* device allocation failed */
#define FG_ERR_INIT (-4)  /* fg_init not called / no device */

/* ───────────────────────── runtime ───────────────────────── */

/* Select the device and create the library stream.  Idempotent. */
int fg_init(int device);
/* Number of visible devices (0 when no GPU; does not require fg_init). */
int fg_device_count(int* count);
/* Message describing the most recent failure on this thread. */
const char* fg_last_error(void);

/* Caching device allocator (size-class free lists, stream-ordered reuse). */
int fg_malloc(void** ptr, size_t bytes);
int fg_free(void* ptr);
int fg_empty_cache(void);
int fg_mem_stats(size_t* bytes_in_use, size_t* bytes_cached);

/* Copies ordered after all queued work.  fg_h2d returns once `src` may be
 * reused: copies up to 1 MiB are staged through pinned memory and queued
 * without draining the stream; larger ones complete before returning.
 * fg_d2h returns with the data in `dst`. */
int fg_h2d(void* dst, const void* src, size_t bytes);
int fg_d2h(void* dst, const void* src, size_t bytes);
/* Queued device-to-device copy and zero fill (a fill kernel, not hipMemset). */
int fg_d2d(void* dst, const void* src, size_t bytes);
int fg_zero(void* ptr, size_t bytes);
int fg_sync(void);

/* Asynchronous small read-back (<= 4096 bytes) through pinned staging:
 * fg_read_async queues the copy and returns a ticket; fg_read_wait blocks only
 * until that copy (not the whole stream) has completed.  Used for the loss
 * scalar (train.js:188-191) and Adam's gnorm (autograd.js:242). */
int fg_read_async(const void* src, size_t bytes, int* ticket);
int fg_read_wait(int ticket, void* dst, size_t bytes);

/* Events on the library stream (for timing). */
int fg_event_create(void** ev);
int fg_event_record(void* ev);
int fg_event_elapsed_ms(void* start, void* stop, float* ms);
int fg_event_destroy(void* ev);

/* Per-entry-point profiling: when enabled, each op entry point brackets its
 * launches with events and accumulates calls, time and algorithmic flop/byte
 * counts per kernel family.  fg_kprof_report writes a JSON array into buf. */
int fg_kprof_enable(int on);
int fg_kprof_reset(void);
int fg_kprof_report(char* buf, size_t len);

/* ───────────────────────── fused ops ───────────────────────── */

/* matmulT forward — tensor.js:34-36 (gemm, numeric.js:111-130).
 * Y[M,N] = X[M,K] · W[N,K]^T in fp32 arithmetic on the fp16 matrix pipes:
 * every operand is scaled by a power of two 2^e fixed per operand (its
 * largest finite magnitude m lands in [2^14, 2^15)), each scaled element is
 * split into fp16 hi = fp16(x 2^e) and lo = fp16(x 2^e - hi) (23 significant
 * bits; |x 2^e - hi - lo| <= max(2^-22 |x 2^e|, 2^-25)), each product x·y is
 * formed as hi·hi + hi·lo + lo·hi (v_mfma_f32_32x32x16_f16 / 16x16x32_f16
 * into fp32 accumulators; the dropped lo·lo is below 2^-22 |xy|), and the
 * sum is scaled back by 2^-(ex + ey) exactly.  The maxima m come from one
 * read of each operand before the GEMM (the *_p forms below can reuse them).
 * Non-finite elements are left out of m and give NaN products. */
int fg_matmulT_fwd(float* Y, const float* X, const float* W, int M, int K, int N);
/* Operand maxima for the *_p forms: FG_XP_PARTS floats of device memory per
 * operand, the partial maxima of its finite magnitudes.  Each *_p entry point
 * takes one such buffer per operand (or NULL: computed into workspace) and a
 * mask `have` of the buffers that already hold their operand's maxima, filled
 * by an earlier *_p call over the same, unchanged data; a non-NULL buffer
 * whose bit is clear is filled (the operands' bits are listed per entry
 * point).  No counterpart in the reference: the training step passes the
 * maxima of X and W from the forward GEMM to its input and weight gradients,
 * and those of gY from the input gradient to the weight gradient. */
#define FG_XP_PARTS 256
/* fg_matmulT_fwd; have bit 0: xp_x, bit 1: xp_w. */
int fg_matmulT_fwd_p(float* Y, const float* X, const float* W, int M, int K, int N, float* xp_x, float* xp_w,
                     int have);
/* matmulT input gradient — tensor.js:38,47.  gX[M,K] (+)= gY[M,N] · W[N,K]. */
int fg_matmulT_bwd_x(float* gX, const float* gY, const float* W, int M, int K, int N, int beta);
/* fg_matmulT_bwd_x; have bit 0: xp_gy, bit 1: xp_w. */
int fg_matmulT_bwd_x_p(float* gX, const float* gY, const float* W, int M, int K, int N, int beta, float* xp_gy,
                       float* xp_w, int have);
/* The number of K pieces fg_matmulT_bwd_x splits its contraction into for
 * this shape (1 = no split); a split's pieces are summed in order. */
int fg_matmulT_bwd_x_pieces(int M, int K, int N);
/* The input gradient of tensor.js:38,47 for shapes split in two K pieces,
 * left unreduced: gX = gX_halves[0 .. MK) + gX_halves[MK .. 2MK) in fp32
 * (the value fg_matmulT_bwd_x stores with beta 0), for a consumer that adds
 * the halves itself (fg_rmsnorm_bwd_from_halves).  Fails unless
 * fg_matmulT_bwd_x_pieces(M, K, N) == 2. */
int fg_matmulT_bwd_x_halves(float* gX_halves, const float* gY, const float* W, int M, int K, int N);
/* fg_matmulT_bwd_x_halves; have bit 0: xp_gy, bit 1: xp_w. */
int fg_matmulT_bwd_x_halves_p(float* gX_halves, const float* gY, const float* W, int M, int K, int N, float* xp_gy,
                              float* xp_w, int have);
/* matmulT weight gradient — tensor.js:39,48.  gW[N,K] (+)= gY[M,N]^T · X[M,K]. */
int fg_matmulT_bwd_w(float* gW, const float* gY, const float* X, int M, int K, int N, int beta);
/* fg_matmulT_bwd_w; have bit 0: xp_gy, bit 1: xp_x. */
int fg_matmulT_bwd_w_p(float* gW, const float* gY, const float* X, int M, int K, int N, int beta, float* xp_gy,
                       float* xp_x, int have);
/* Several matmulT weight gradients in one launch — tensor.js:49-51 per job:
 * gW[N,K] (+)= gY[M,N]^T · X[M,K] (beta per job), each over its full M (no
 * K split).  The training step defers the weight gradients of its layer
 * matmuls to the end of backward() and issues them here: thousands of output
 * tiles in one grid fill the GPU without the split-K partial slabs that a
 * single small-output gradient needs.  Jobs on one gW (a weight used twice
 * in one pass) apply in list order, a later job's beta accumulating onto the
 * earlier result; gW must not partially overlap another job's gW.  xp_gy /
 * xp_x: the operands' maxima (FG_XP_PARTS floats each, as filled by a *_p
 * entry point over the same data) or NULL (computed here). */
typedef struct fg_wgrad_job {
  float* gW;
  const float* gY;
  const float* X;
  int M, K, N, beta;
  const float* xp_gy;
  const float* xp_x;
} fg_wgrad_job;
int fg_matmulT_bwd_w_grouped(const fg_wgrad_job* jobs, int count);

/* matmulT backward (tensor.js:44-51) in one call: gX (+)= gY·W, then
 * gW (+)= gY^T·X (beta_* as in the separate entry points).  gX == gW is
 * allowed (matmulT(X, X)): the second GEMM accumulates onto the first. */
int fg_matmulT_bwd(float* gX, int beta_x, float* gW, int beta_w, const float* gY, const float* X,
                   const float* W, int M, int K, int N);
/* fg_matmulT_bwd; have bit 0: xp_gy, bit 1: xp_x, bit 2: xp_w. */
int fg_matmulT_bwd_p(float* gX, int beta_x, float* gW, int beta_w, const float* gY, const float* X, const float* W,
                     int M, int K, int N, float* xp_gy, float* xp_x, float* xp_w, int have);

/* Fused residual projection — the addTensors(x, matmulT(a, W)) pair of
 * TrainableTransformer._forward (train.js:144-145, 152-153):
 * Y[M,N] = R[M,N] + X[M,K] · W[N,K]^T with the residual added in the GEMM
 * epilogue.  Backward is matmulT's plus the pass-through R.grad += Y.grad. */
int fg_matmulT_fwd_resid(float* Y, const float* R, const float* X, const float* W, int M, int K, int N);
/* fg_matmulT_fwd_resid; have bit 0: xp_x, bit 1: xp_w. */
int fg_matmulT_fwd_resid_p(float* Y, const float* R, const float* X, const float* W, int M, int K, int N,
                           float* xp_x, float* xp_w, int have);

/* Fused qkv projection with RoPE — the matmulT(xn, wqkv) of
 * TrainableTransformer._forward (train.js:131) followed by the ropeRows of
 * its q and k column blocks (train.js:133-138, tensor.js:133-148):
 * Y[M,N] = X[M,K] · W[N,K]^T, then in every row the (even, odd) column pairs
 * of [0, (nH + nKV) dH) — heads of dH — turned by the angle of position
 * pos0 + (row % posStride, or row when posStride is 0) from the fp64 tables
 * of fg_rope_table (npos entries), in fp64: bit for bit fg_matmulT_fwd then
 * the rotation fg_qkv_rope_fwd applies, done in place over the q and k
 * columns after the GEMM.  The v columns are left as they are. */
int fg_matmulT_fwd_rope(float* Y, const float* X, const float* W, int M, int K, int N, const double* cos_tab,
                        const double* sin_tab, int npos, int nH, int nKV, int dH, int pos0, int posStride);
/* fg_matmulT_fwd_rope; have bit 0: xp_x, bit 1: xp_w. */
int fg_matmulT_fwd_rope_p(float* Y, const float* X, const float* W, int M, int K, int N, const double* cos_tab,
                          const double* sin_tab, int npos, int nH, int nKV, int dH, int pos0, int posStride,
                          float* xp_x, float* xp_w, int have);

/* causalAttn / causalAttnBatch over the column blocks of a fused projection
 * (tensor.js:191-229, 299-337 on the q, k, v that train.js:133-138 cuts out
 * of qkv): qkv[B*T, (nH + 2 nKV) dH] = [q | k | v] with q and k already
 * rotated; O and lse as fg_attn_fwd.  dH in {32, 64, 96, 128}, 16-byte aligned. */
int fg_attn_fwd_qkv(float* O, float* lse, const float* qkv, int B, int T, int nH, int nKV, int dH);
/* fg_attn_fwd_qkv that also leaves the partial maxima of q, k and v (the
 * operand powers of two of the split-fp16 products, see fg_matmulT_fwd) in
 * xp_qkv (3 * FG_XP_PARTS floats of device memory, or NULL), for
 * fg_attn_bwd_qkv_p over the same, unchanged qkv.  No counterpart in the
 * reference: the training step's attention backward reuses them. */
int fg_attn_fwd_qkv_p(float* O, float* lse, const float* qkv, int B, int T, int nH, int nKV, int dH, float* xp_qkv);
/* Its backward (tensor.js:231-267, 339-375, then the ropeRows and sliceCols
 * backwards of train.js:133-138): gqkv = [R^T dQ | R^T dK | dV], written (not
 * accumulated) — the value fg_attn_bwd followed by fg_qkv_rope_bwd stores. */
int fg_attn_bwd_qkv(float* gqkv, const float* dO, const float* qkv, const float* O, const float* lse, int B, int T,
                    int nH, int nKV, int dH, const double* cos_tab, const double* sin_tab, int npos, int pos0,
                    int posStride);
/* fg_attn_bwd_qkv with the maxima fg_attn_fwd_qkv_p left in xp_qkv (NULL:
 * computed here). */
int fg_attn_bwd_qkv_p(float* gqkv, const float* dO, const float* qkv, const float* O, const float* lse, int B, int T,
                      int nH, int nKV, int dH, const double* cos_tab, const double* sin_tab, int npos, int pos0,
                      int posStride, const float* xp_qkv);

/* causalAttn / causalAttnBatch forward — tensor.js:191-229, 299-337.
 * Any head size (MFMA kernels for 32, 64, 96 and 128 on 16-byte aligned
 * tensors, the next of those on head-padded copies for other sizes from 33
 * to 127, batched GEMM launches over T×T workspaces above 128,
 * one-row-per-thread kernels otherwise), and any nH, nKV whose head map
 * stays below nKV (with nH < nKV the kv heads no query head uses get zero
 * gradients).
 * Q[B*T, nH*dH], K,V[B*T, nKV*dH] → O[B*T, nH*dH] with a block-diagonal causal
 * mask (row b*T+t sees b*T..b*T+t), GQA head map kvh = h / max(1, nH/nKV),
 * scale 1/sqrt(dH).  P is not kept between the calls; lse[B*nH*T] receives the
 * natural-log row log-sum-exp of the scaled scores (layout [b][h][t]). */
int fg_attn_fwd(float* O, float* lse, const float* Q, const float* K, const float* V,
                int B, int T, int nH, int nKV, int dH);
/* causalAttn* backward — tensor.js:231-267, 339-375.  Recomputes P from lse.
 * dQ (+)= ..., dK (+)= ..., dV (+)= ... (per-tensor beta).  dK/dV of a kv head
 * sum over the nH/nKV query heads of its group.  The head sizes with MFMA
 * kernels keep dS = P∘(dP − D) of every causal 32×32 block in a workspace
 * (4 bytes per causal pair and head) and form dQ from it in a second launch;
 * when that workspace would exceed the limit of fg_attn_set_ds_limit
 * (8 GiB by default) dQ recomputes S and dP instead. */
/* Largest stored-dS workspace of the attention backward, in bytes (0: always
 * recompute).  Applies to calls queued afterwards; no reference counterpart
 * (the reference keeps the whole P matrix). */
int fg_attn_set_ds_limit(size_t bytes);
int fg_attn_bwd(float* dQ, int beta_q, float* dK, int beta_k, float* dV, int beta_v,
                const float* dO, const float* Q, const float* K, const float* V,
                const float* O, const float* lse, int B, int T, int nH, int nKV, int dH);

/* crossEntropyMean forward — tensor.js:393-407.  loss (device scalar) =
 * mean over rows of (lse_r - logits[r, targets[r]]); lse[rows] is saved for
 * the backward.  targets are int32 on the device. */
int fg_ce_fwd(float* loss, float* lse, const float* logits, const int32_t* targets, int rows, int V);
/* crossEntropyMean forward together with its backward for a seed gradient of
 * 1 — the loss of a training step, whose backward always follows
 * (train.js:265-269, autograd.js:126-133): loss and lse as fg_ce_fwd, and
 * dlogits = (1/rows)(softmax(logits) - onehot(targets)) written (not
 * accumulated): bit for bit fg_ce_fwd then fg_ce_bwd with *gloss = 1 and
 * beta 0, reading the logits from HBM once instead of twice. */
int fg_ce_fwd_bwd(float* loss, float* lse, float* dlogits, const float* logits, const int32_t* targets, int rows,
                  int V);
/* fg_ce_fwd_bwd that also fills xp_grad (FG_XP_PARTS floats of device
 * memory, or NULL) with a bound of the gradient's magnitudes, 1/rows
 * (|softmax - onehot| <= 1), in the form the *_p GEMM entry points take as
 * operand maxima: the gradient's GEMM then skips reading it for its maxima.
 * No counterpart in the reference. */
int fg_ce_fwd_bwd_p(float* loss, float* lse, float* dlogits, const float* logits, const int32_t* targets, int rows,
                    int V, float* xp_grad);
/* fg_ce_fwd_bwd that allocates nothing: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under graph capture,
 * serving loops, harnesses that forbid allocation): the per-row losses go to a
 * static device array of 65536 fp64 entries (512 KiB per device, held until
 * the process ends) instead of an allocator workspace.  rows > 65536 fail
 * with FG_ERR_ARG.  Same kernels, same bits as fg_ce_fwd_bwd.  Every call on a
 * device shares that device's array: calls that overlap (queued from several
 * host threads at once) race on it. */
int fg_ce_fwd_bwd_noalloc(float* loss, float* lse, float* dlogits, const float* logits, const int32_t* targets,
                          int rows, int V);
/* crossEntropyMean backward — tensor.js:408-416.
 * dlogits (+)= (g/rows) * (softmax(logits) - onehot(targets)), g = *gloss
 * (device scalar, the loss node's gradient). */
int fg_ce_bwd(float* dlogits, const float* logits, const float* lse, const int32_t* targets,
              const float* gloss, int rows, int V, int beta);
/* fg_ce_bwd with beta 0 that also fills xp_grad (FG_XP_PARTS floats of
 * device memory) with the gradient's bound |gloss| / rows as GEMM operand
 * maxima (see fg_ce_fwd_bwd_p); beta must be 0.  No counterpart in the
 * reference. */
int fg_ce_bwd_p(float* dlogits, const float* logits, const float* lse, const int32_t* targets, const float* gloss,
                int rows, int V, int beta, float* xp_grad);

/* rmsNorm forward — tensor.js:103-113.  Y = X * inv_t * w with
 * inv_t = 1/sqrt(sum(x^2)/D + eps); inv[T] is saved for the backward. */
int fg_rmsnorm_fwd(float* Y, float* inv, const float* X, const float* w, int T, int D, double eps);
/* rmsNorm backward — tensor.js:114-127.  gX (+)= g*w*inv - c*x with
 * c = sum(g*w*x)*inv^3/D;  gw (+)= sum_t g*x*inv (column reduction). */
int fg_rmsnorm_bwd(float* gX, int beta_x, float* gw, int beta_w, const float* g, const float* X,
                   const float* w, const float* inv, int T, int D);
/* The same backward writing gX = gX_in + dX (gX_in may be gX itself, or
 * NULL for gX = dX): a gradient that still shares another node's buffer is
 * accumulated into a fresh one without a copy first. */
int fg_rmsnorm_bwd_from(float* gX, const float* gX_in, float* gw, int beta_w, const float* g, const float* X,
                        const float* w, const float* inv, int T, int D);
/* fg_rmsnorm_bwd_from with the incoming gradient given as two halves,
 * g = g_halves[0 .. TD) + g_halves[TD .. 2TD) (summed in fp32, in that
 * order, as fg_matmulT_bwd_x_halves' pieces would be). */
int fg_rmsnorm_bwd_from_halves(float* gX, const float* gX_in, float* gw, int beta_w, const float* g_halves,
                               const float* X, const float* w, const float* inv, int T, int D);
/* The rmsNorm weight gradient deferred — tensor.js:114-127 split in two:
 * fg_rmsnorm_bwd_partial writes gX as fg_rmsnorm_bwd_from does (with
 * g_halves set, g holds the incoming gradient as two halves, as in
 * fg_rmsnorm_bwd_from_halves) and leaves
 * gw's column sum as a partial matrix[fg_rmsnorm_bwd_parts(T, D) x D]; one
 * fg_colsum_grouped launch at the end of the backward pass then forms every
 * deferred gw (+)= column sums of its matrix, the same sums in the same
 * order as the one-call form.  fg_rmsnorm_bwd_parts returns 0 for shapes
 * without the deferred form (D % 4 != 0 or D > 4096). */
int fg_rmsnorm_bwd_parts(int T, int D);
int fg_rmsnorm_bwd_partial(float* gX, const float* gX_in, float* partial, const float* g, int g_halves,
                           const float* X, const float* w, const float* inv, int T, int D);
typedef struct fg_colsum_job {
  float* out;            /* out[n] (+)= sum over rows of partial[rows x n] (beta) */
  const float* partial;
  int rows, n, beta;     /* n % 4 == 0, 16-byte aligned buffers */
} fg_colsum_job;
/* Jobs on one output are applied in list order (a later job's beta
 * accumulates onto the earlier result). */
int fg_colsum_grouped(const fg_colsum_job* jobs, int count);

/* RoPE angle table (host helper): cos/sin[p*(dHead/2) + i/2] of
 * p * theta^(-i/dHead) for even i, in fp64 — tensor.js:142-143. */
int fg_rope_table(double* cos_tab, double* sin_tab, int npos, int dHead, double theta);
/* ropeRows forward — tensor.js:133-149.  Interleaved-pair rotation of every
 * head; position = pos0 + (posStride > 0 ? t % posStride : t); the device
 * tables hold npos positions. */
int fg_rope_fwd(float* Y, const float* X, const double* cos_tab, const double* sin_tab, int npos,
                int T, int nHead, int dHead, int pos0, int posStride);
/* ropeRows backward — tensor.js:150-165.  gX (+)= R^T g. */
int fg_rope_bwd(float* gX, const float* g, const double* cos_tab, const double* sin_tab, int npos,
                int T, int nHead, int dHead, int pos0, int posStride, int beta);

/* Fused q/k/v split + RoPE — the sliceCols×3 + ropeRows×2 sequence of
 * TrainableTransformer._forward (train.js:133-138, tensor.js:133-183): from
 * qkv[rows, (nH+2nKV)*dH] write Q = rope(q) [rows, nH*dH], K = rope(k)
 * [rows, nKV*dH] and V = v [rows, nKV*dH] in one pass. */
int fg_qkv_rope_fwd(float* Q, float* K, float* V, const float* qkv, const double* cos_tab,
                    const double* sin_tab, int npos, int rows, int nH, int nKV, int dH, int pos0,
                    int posStride);
/* Its backward: gqkv (+)= [R^T gQ | R^T gK | gV]; a NULL gradient counts as zero. */
int fg_qkv_rope_bwd(float* gqkv, const float* gQ, const float* gK, const float* gV, const double* cos_tab,
                    const double* sin_tab, int npos, int rows, int nH, int nKV, int dH, int pos0,
                    int posStride, int beta);

/* swigluRows on a fused gate/up projection — the matmulT(gate), matmulT(up),
 * swigluRows sequence of TrainableTransformer._forward (train.js:149-151)
 * with the two projections as one GEMM: GU[rows, 2H] = [G | U] (row r holds
 * G[r, 0..H) then U[r, 0..H)).  O[rows, H] = silu(G)·U, the same element
 * arithmetic as fg_swiglu_fwd.  Any H (float4 rows when H % 4 == 0 and the
 * tensors are 16-byte aligned). */
int fg_swiglu_gu_fwd(float* O, const float* GU, int rows, int H);
/* The fused gate/up projection and swigluRows (tensor.js:34-36 twice, then
 * tensor.js:272-283): GU[M, 2H] = X[M,K] · Wgu[2H,K]^T with Wgu = [Wg; Wu]
 * stacked, and O[M,H] = SwiGLU(GU[:, :H], GU[:, H:]).  Where the output
 * makes whole rounds of 256x256 tiles, the SwiGLU is formed in the GEMM's
 * epilogue (the gate and up columns of one hidden unit computed side by
 * side); elsewhere the GEMM and fg_swiglu_gu_fwd.  Both give the bits of
 * fg_matmulT_fwd followed by fg_swiglu_gu_fwd. */
int fg_matmulT_fwd_swiglu(float* O, float* GU, const float* X, const float* Wgu, int M, int K, int H);
/* fg_matmulT_fwd_swiglu; have bit 0: xp_x, bit 1: xp_w (of Wgu). */
int fg_matmulT_fwd_swiglu_p(float* O, float* GU, const float* X, const float* Wgu, int M, int K, int H, float* xp_x,
                            float* xp_w, int have);
/* Its backward: gGU[rows, 2H] (+)= [dG | dU] (one beta for both halves). */
int fg_swiglu_gu_bwd(float* gGU, int beta, const float* g, const float* GU, int rows, int H);
/* fg_swiglu_gu_bwd that also leaves the partial maxima of the finite
 * magnitudes of gGU (FG_XP_PARTS floats of device memory, or NULL) for the
 * input- and weight-gradient GEMMs that read it (bit 0 of their `have`).  No
 * counterpart in the reference: it saves those GEMMs a read of gGU. */
int fg_swiglu_gu_bwd_p(float* gGU, int beta, const float* g, const float* GU, int rows, int H, float* xp_out);

/* swigluRows forward — tensor.js:272-280.  O = G * sigmoid(G) * U. */
int fg_swiglu_fwd(float* O, const float* G, const float* U, int64_t n);
/* swigluRows backward — tensor.js:281-289.
 * gG (+)= g*U*(s + G*s*(1-s)),  gU (+)= g*G*s,  s = sigmoid(G). */
int fg_swiglu_bwd(float* gG, int beta_g, float* gU, int beta_u, const float* g, const float* G,
                  const float* U, int64_t n);

/* embedLookup forward — tensor.js:85-91.  X[t,:] = W[ids[t],:]; an id outside
 * [0,V) yields a NaN row (the reference reads `undefined`). */
int fg_embed_fwd(float* X, const float* W, const int32_t* ids, int T, int V, int D);
/* embedLookup backward plan (host helper): stable counting sort of ids into
 * segments of equal id; perm[T], seg_start[nseg+1], seg_id[nseg].  Returns
 * FG_ERR_ARG for an id outside [0,V). */
int fg_embed_plan(const int32_t* ids, int T, int V, int32_t* perm, int32_t* seg_start,
                  int32_t* seg_id, int* nseg);
/* embedLookup backward — tensor.js:92-98.  gW[id,:] += g[t,:] for every t,
 * summed per id in increasing t (the reference's order), no atomics.
 * Device arrays come from fg_embed_plan.  Always accumulates. */
int fg_embed_bwd(float* gW, const float* g, const int32_t* perm, const int32_t* seg_start,
                 const int32_t* seg_id, int nseg, int D);

/* sliceCols forward — tensor.js:170-175.  Y[M,len] = X[:, off:off+len]. */
int fg_slice_cols_fwd(float* Y, const float* X, int M, int K, int off, int len);
/* sliceCols backward — tensor.js:176-182.  gX[:, off:off+len] += g.  Always
 * accumulates (a fresh gX must be zeroed first). */
int fg_slice_cols_bwd(float* gX, const float* g, int M, int K, int off, int len);

/* addTensors forward — train.js:230-232.  Y = A + B. */
int fg_add_fwd(float* Y, const float* A, const float* B, int64_t n);
/* Gradient pass-through — train.js:233-237.  Y (+)= X. */
int fg_accum(float* Y, const float* X, int64_t n, int beta);

/* weightedSum forward — tensor.js:380-384.  *out = sum_i Y[i]*t[i]
 * (fp64 accumulation, deterministic order of partials). */
int fg_weighted_sum_fwd(float* out, const float* Y, const float* t, int64_t n);
/* weightedSum backward — tensor.js:384-388.  gY (+)= (*gout) * t. */
int fg_weighted_sum_bwd(float* gY, const float* gout, const float* t, int64_t n, int beta);

/* ── vector-level autograd ops (autograd.js:70-190) ──────────────────────
 * Element-wise helpers of the autograd module, off the training step.  They
 * follow the reference's arithmetic: fp32 operands widened to fp64, each
 * Float32Array store rounded once, a gradient update g (+)= term stored as
 * fp32(g_old + term) (beta = 0: fp32(term)), and the reference's sequential
 * sums kept sequential.  Backward calls may pass one buffer as both
 * gradients (mul(x, x), dot(x, x)); each element then takes both updates in
 * the reference's order. */
/* mul — autograd.js:70-79.  out = a * b; b has nb = n elements or nb = 1 (broadcast). */
int fg_vec_mul_fwd(float* out, const float* a, const float* b, int64_t n, int64_t nb);
/* mul backward: ga (+)= g * b; gb (+)= g * a, or for nb = 1 the running
 * fp32 sum gb[0] += g[i] * a[i] over i in order. */
int fg_vec_mul_bwd(float* ga, int beta_a, float* gb, int beta_b, const float* g, const float* a, const float* b,
                   int64_t n, int64_t nb);
/* silu — autograd.js:81-89.  sig = fp32(1 / (1 + exp(-x))) (saved for the
 * backward), out = x * sig. */
int fg_vec_silu_fwd(float* out, float* sig, const float* x, int64_t n);
/* silu backward: gx (+)= g * (sig + x * sig * (1 - sig)). */
int fg_vec_silu_bwd(float* gx, int beta, const float* g, const float* x, const float* sig, int64_t n);
/* dot — autograd.js:136-146.  out[0] = sum a_i b_i (one sequential fp64 sum). */
int fg_vec_dot_fwd(float* out, const float* a, const float* b, int64_t n);
/* dot backward: ga (+)= g[0] * b, gb (+)= g[0] * a (g a device scalar). */
int fg_vec_dot_bwd(float* ga, int beta_a, float* gb, int beta_b, const float* g, const float* a, const float* b,
                   int64_t n);
/* scale — autograd.js:148-153.  out = s * x (s an fp64 host scalar). */
int fg_vec_scale_fwd(float* out, const float* x, double s, int64_t n);
/* scale backward: gx (+)= g * s. */
int fg_vec_scale_bwd(float* gx, int beta, const float* g, double s, int64_t n);
/* ropeNode — autograd.js:156-172.  Pairs (i, i+1), i = 0, 2, .. < dHead,
 * turned by cos_t[i/2], sin_t[i/2] (fp64 device tables of ceil(dHead/2)
 * entries); the outputs past the pairs are zero.  The pairs must lie inside
 * the vector (2 ceil(dHead/2) <= n), else FG_ERR_ARG. */
int fg_vec_rope_fwd(float* out, const float* x, const double* cos_t, const double* sin_t, int64_t n, int dHead);
/* ropeNode backward: R^T of each pair into gx; with beta = 0 the elements
 * past the pairs are set to zero. */
int fg_vec_rope_bwd(float* gx, int beta, const float* g, const double* cos_t, const double* sin_t, int64_t n,
                    int dHead);
/* softmaxVec — autograd.js:174-190.  p = softmax(x) (exp of x - max stored
 * in fp32, their fp64 sum in order, then each divided); out and the saved p
 * hold the same values. */
int fg_vec_softmax_fwd(float* out, float* p, const float* x, int64_t n);
/* softmaxVec backward: gx_i (+)= sum_j g_j (p_i ((i == j) - p_j)), summed
 * over j in order in fp64 (O(n^2) work, as in the reference) for n <= 65536;
 * longer vectors take the O(n) form p_i (g_i - sum_j g_j p_j), equal up to
 * fp64 rounding. */
int fg_vec_softmax_bwd(float* gx, int beta, const float* g, const float* p, int64_t n);

/* Single-query-row attention over host-side helpers' operands —
 * attentionDecode (attention.js:31-57, mode 0), attentionNaive (:63-79,
 * mode 1), flashAttention (:89-126, mode 2, `block` keys per block):
 * out[0..d) = sum_j softmax_j(scale * q·K_j) V_j over keys j < n, K and V
 * holding rows of d floats (the caller's kOff already applied); with causal
 * set, keys j > qOff are masked.  Each mode keeps its reference's order of
 * operations (fp64 dots and weights, fp32 stores).  scores (nullable, mode
 * 0 only) receives the n fp32 scores, -inf where masked, as attentionDecode
 * leaves them in its optional buffer.  Uses a workspace of about 20 n bytes. */
int fg_row_attention(float* out, const float* q, const float* K, const float* V, int n, int d, double scale,
                     int causal, int qOff, int mode, int block, float* scores);
/* rmsnormInto — nn.js:42-44 (special.js:46-50): out[i] = x[i] * ss * w[i]
 * with ss = 1 / sqrt(rms^2 + eps), rms = sqrt(sum x^2 / n) (in-order fp64 sum). */
int fg_row_rmsnorm(float* out, const float* x, const float* w, int n, double eps);

/* Adam.step — autograd.js:221-243 (one call per optimizer step).
 * Per tensor: p (fp32 params), g (grad), m, v (moments), n (elements).
 * gnorm = sqrt(sum over all g^2) in fp64; scale = gnorm > clip ? clip/gnorm : 1;
 * g' = g*scale + wd*p;  m = b1*m + (1-b1)*g';  v = b2*v + (1-b2)*g'^2;
 * p -= lr_t * (m/bc1) / (sqrt(v/bc2) + eps).  Computed in fp64, stored fp32.
 * lr_t (cosine schedule) and bc1 = 1-b1^t, bc2 = 1-b2^t come from the host.
 * stats_dev (device, 2 doubles, may be NULL) receives {gnorm, scale}. */
typedef struct fg_adam_tensor {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
} fg_adam_tensor;
int fg_adam_step(const fg_adam_tensor* tensors, int count, double lr_t, double b1, double b2,
                 double eps, double wd, double clip, double bc1, double bc2, double* stats_dev);

/* Adam.step with the per-step scalars in device memory: sched_dev = {lr_t,
 * bc1, bc2} (3 doubles), read by the update kernel, so that a recorded graph
 * step (fg_graph_*) uses the values the host writes there before each replay.
 * Same arithmetic as fg_adam_step — autograd.js:221-243. */
int fg_adam_step_sched(const fg_adam_tensor* tensors, int count, const double* sched_dev, double b1,
                       double b2, double eps, double wd, double clip, double* stats_dev);

/* Adam.step over a plan: the chunk table of one tensor list (pointers, sizes)
 * uploaded once into device memory by fg_adam_plan_create, together with the
 * norm partials, so that a step allocates nothing and each optimizer owns
 * its table (a recorded graph keeps using the table it was recorded with
 * until the plan is destroyed).  No counterpart in the reference, whose Adam
 * (autograd.js:214-244) walks its JS arrays; same arithmetic as fg_adam_step.
 * fg_adam_plan_matches tells whether a tensor list (the same pointers and
 * sizes, in order) is the one the plan was built for.  fg_adam_plan_destroy
 * returns the memory to the allocator in stream order (steps already queued
 * still see the table). */
typedef struct fg_adam_plan fg_adam_plan;
int fg_adam_plan_create(const fg_adam_tensor* tensors, int count, fg_adam_plan** plan);
int fg_adam_plan_matches(const fg_adam_plan* plan, const fg_adam_tensor* tensors, int count, int* match);
int fg_adam_plan_destroy(fg_adam_plan* plan);
int fg_adam_step_plan(fg_adam_plan* plan, double lr_t, double b1, double b2, double eps, double wd, double clip,
                      double bc1, double bc2, double* stats_dev);
int fg_adam_step_sched_plan(fg_adam_plan* plan, const double* sched_dev, double b1, double b2, double eps,
                            double wd, double clip, double* stats_dev);

/* ──────────── device-resident training loop (train.js:246-276) ──────────── */

/* Batch sampling of train() — train.js:255-260.  data[n] is the token buffer
 * resident in device memory, starts[B] (device) the window starts drawn on
 * the host with the reference's RNG.  ids[b*T+i] = row[i], targets[b*T+i] =
 * row[i+1] with row[i] = data[s_b+i], or data[n-1] past the end
 * (`data[s+i] ?? data[data.length-1]`).  Values outside [0,V) become -1. */
int fg_batch_gather(int32_t* ids, int32_t* targets, const int32_t* data, int64_t n,
                    const int32_t* starts, int B, int T, int V);
/* Number of 64-bit keys fg_embed_sort_keys needs for T ids (a power of two). */
int fg_embed_keys_len(int T, int64_t* len);
/* Device replacement of the embedLookup backward plan (tensor.js:92-98):
 * keys[0..len) = ascending (id << 32 | t) for every id in [0,V), then ~0. */
int fg_embed_sort_keys(uint64_t* keys, int64_t len, const int32_t* ids, int T, int V);
/* embedLookup backward over sorted keys — tensor.js:92-98.  gW[id,:] +=
 * g[t,:] summed per id in increasing t; the same sums, in the same order, as
 * fg_embed_bwd.  beta 0: the rows of the ids present are written with their
 * sums (started from +0, without reading them: the same bits as accumulating
 * into a zero row) and every other row is left as it is — for a gradient
 * the caller has just zero-filled. */
int fg_embed_bwd_sorted(float* gW, const float* g, const uint64_t* keys, int T, int V, int D, int beta);

/* ptr[0..n) = value (a kernel; the loss-gradient seed of backward(),
 * autograd.js:127). */
int fg_fill_f32(float* ptr, float value, int64_t n);

/* Recorded steps (hipGraph).  No reference counterpart: the reference's
 * train() loop re-issues every op each step.  Between fg_graph_begin and
 * fg_graph_end the library's queued work is recorded instead of run;
 * fg_graph_launch replays it.  Entry points that synchronise or copy through
 * host staging (fg_h2d, fg_d2h, fg_sync, fg_read_*, events, profiling, a
 * first fg_adam_step over a new tensor list) fail during a capture, so a
 * recorded step must take every per-step input from device memory.  Memory
 * allocated by recorded work stays reserved for the graph until
 * fg_graph_destroy.  fg_graph_abort discards a capture that failed. */
int fg_graph_begin(void);
int fg_graph_end(void** graph);
int fg_graph_launch(void* graph);
int fg_graph_destroy(void* graph);
int fg_graph_abort(void);

/* ──────────── inference forward: one decode step (transformer.js:134-184) ──────────── */

/* Weights of one layer, in the reference's layouts: wqkv [(nH+2nKV)·dH, dim],
 * wo [dim, dim], gate/up [hidden, dim], down [dim, hidden] (device).  Each
 * matrix is a QuantLinear (nn.js:19-40): rows of fg_qrow_bytes(type, K)
 * bytes of its ggml type (0 F32, 1 F16, 2 Q4_0, 6 Q5_0, 8 Q8_0, 12 Q4_K,
 * 13 Q5_K, 14 Q6_K); gate and up share one type. */
typedef struct fg_decode_layer {
  const float* ln1;
  const void* wqkv;
  const void* wo;
  const float* ln2;
  const void* gate;
  const void* up;
  const void* down;
  int wqkv_type, wo_type, gate_type, up_type, down_type;
} fg_decode_layer;
/* A loaded Transformer (transformer.js:69-118): Config dims, weights (the
 * embedding and the LM head typed like the layer matrices; the embedding row
 * of a quantized tok_emb is decoded as Transformer._embed does,
 * transformer.js:121-131), the fp32 RoPE table (special.js:116-127,
 * [maxSeq][dHead/2] cos and sin, device) and device scratch: x[dim],
 * q[nH·dH], h[hidden] (fp32) and attn_part (fp64, fg_decode_part_len
 * doubles: the attention's per-chunk partials).  `layers` is a host array of
 * nLayers. */
typedef struct fg_decode_model {
  int dim, hidden, nLayers, nHeads, nKvHeads, vocab, maxSeq;
  int emb_type, cls_type;
  double normEps;
  const void* tok_emb;
  const float* ln_f;
  const void* wcls; /* = tok_emb for a tied head */
  const fg_decode_layer* layers;
  const float* rope_cos;
  const float* rope_sin;
  float* x;
  float* q;
  float* h;
  double* attn_part;
} fg_decode_model;
/* Doubles of fg_decode_model.attn_part for nHeads, dHead and the cache's maxSeq. */
int fg_decode_part_len(int nHeads, int dHead, int maxSeq, int64_t* doubles);
/* Transformer.forward(token, pos, cache) — transformer.js:134-184, with
 * attentionDecode (attention.js:31-61) and KVCache.put (attention.js:137-141).
 * state (device) = {token, pos}; kcache / vcache (device) are the KVCache's
 * [nLayers][maxSeq][nKV·dH] arrays (maxSeq = model->maxSeq); logits[vocab]
 * (device).  Reading token and position from device memory lets a recorded
 * graph of one step serve every step.  A token outside [0,vocab) gives NaN
 * logits; a position outside [0,maxSeq) writes nothing.  Head dims: even, up
 * to 1024.  Each launch stages its input vector in LDS, so dim <= 8192,
 * hidden <= 16384 and 4·dim + 8·nHeads·(ceil(maxSeq/64) + 2) <= 65536 bytes
 * (maxSeq up to 12160 at 32 heads and dim 4096); larger models are rejected
 * with an error. */
int fg_decode_step(const fg_decode_model* m, float* kcache, float* vcache, const int32_t* state,
                   float* logits);

/* ──────────── quantized weights (src/L3/quant.js, src/L4/nn.js) ──────────── */

/* rowBytes (quant.js:64): bytes of n elements of a ggml type, whole blocks. */
int fg_qrow_bytes(int type, int64_t n, int64_t* bytes);
/* QuantLinear.forward (nn.js:27-33) / dotQ (quant.js:215-320):
 * y[n] = fp32(Σ_k W[n,k]·x[k]) for n < N, W rows of fg_qrow_bytes(type, K)
 * bytes, K a whole number of blocks (device pointers).  F32 / F16 rows sum in
 * fp64; quantized rows sum each sub-block's integer·x products in fp32 and
 * apply the block scales and the sums across blocks in fp64 (~1e-7 relative). */
int fg_qmatvec(int type, float* y, const void* W, const float* x, int N, int K);
/* dotQ (quant.js:215-320) as the reference returns it: the same sums as
 * fg_qmatvec, kept in fp64 (y[N] doubles, device). */
int fg_qmatvec_f64(int type, double* y, const void* W, const float* x, int N, int K);
/* SwiGLU.forward's activation (nn.js:56-66): h[i] = fp32((g/(1+e^-g))·u) in
 * fp64 (device pointers). */
int fg_silu_mul(float* h, const float* g, const float* u, int64_t n);
/* dequantize (quant.js:102-199): out[i] = fp32 value of element i of the
 * quantized array q (n a whole number of blocks), bit-identical to the
 * reference (device pointers). */
int fg_dequantize(int type, float* out, const void* q, int64_t n);
/* quantizeRow (quant.js:580-590) for F32, F16, Q8_0, Q4_K, Q5_K and Q6_K:
 * the fg_qrow_bytes(type, n) bytes of x[n] (n a whole number of blocks),
 * bit-identical to the reference (device pointers). */
int fg_quantize(int type, void* out, const float* x, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_HIP_H */
