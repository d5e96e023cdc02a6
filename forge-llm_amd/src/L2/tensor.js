/**
 * L2b · tensor-level fused ops on MI355X (gfx950).
 *
 * Drop-in for forge-llm's src/L2/tensor.js: same exports, same positional
 * signatures, same forward values and backward semantics (gradients are
 * created on first write and accumulated afterwards).  Every op queues HIP
 * kernels through the C ABI (include/forge_hip.h) and returns a Node whose
 * value stays in device memory; backward closures run device kernels.
 *
 * Shapes are validated on the host before anything is queued (a mismatch
 * throws instead of reading out of bounds).
 */
import { hip, allocF32, graphState } from "./device.js";
import { Node, _deviceNode, _tapeEnabled, _deferWeightGrad, _deferring, _deferColsum } from "./autograd.js";

function need(node, n, what) {
  if (!(node instanceof Node)) throw new TypeError(`${what}: expected a Node`);
  if (node.n !== n) throw new RangeError(`${what}: expected ${n} elements, got ${node.n}`);
}
function posInt(v, what) {
  if (!Number.isInteger(v) || v <= 0) throw new RangeError(`${what} must be a positive integer, got ${v}`);
}
/** Attach the device backward, or drop saved tensors when nothing records. */
function attach(out, saved, bwd) {
  if (_tapeEnabled()) {
    out._saved = saved;
    out._bdev = bwd;
  } else if (saved) {
    const a = hip();
    for (const h of saved) a.free(h);
  }
  return out;
}

// ── GEMM operand maxima ─────────────────────────────────────────────────
// The GEMMs scale each operand by a power of two taken from its largest
// finite magnitude, which costs one read of the operand.  A recorded GEMM
// keeps the maxima of its forward operands (FG_XP_PARTS floats each) for its
// backward, and the maxima of the output gradient serve both gradient GEMMs.
const XP_BYTES = 256 * 4;

/** Buffers for the forward maxima of X and W (filled by the forward GEMM),
 *  with the value versions they describe; null when nothing records. */
function xpForward(a, X, W) {
  if (!_tapeEnabled()) return null;
  return { x: a.alloc(XP_BYTES), vx: X._ver, w: a.alloc(XP_BYTES), vw: W._ver };
}
/** The forward GEMM's trailing maxima arguments. */
function xpArgs(xp) { return xp ? [xp.x, xp.w, 0] : []; }
/** The forward maxima of X / W if the value is unchanged since, else null. */
function xpX(xp, X) { return xp && X._ver === xp.vx ? xp.x : null; }
function xpW(xp, W) { return xp && W._ver === xp.vw ? xp.w : null; }

/**
 * Y[M,N] = X[M,K] · W[N,K]ᵀ (tensor.js:34-53).
 * Backward: dX (+)= dY·W, dW (+)= dYᵀ·X.  The GEMMs compute in fp32 on the
 * fp16 MFMA pipes: each operand is scaled by a power of two and split into
 * an fp16 hi/lo pair (23 significant bits), and every product is the sum of
 * hi·hi, hi·lo and lo·hi (the dropped lo·lo is below 2⁻²² of the product).
 */
export function matmulT(X, W, M, K, N) {
  posInt(M, "M"); posInt(K, "K"); posInt(N, "N");
  need(X, M * K, "matmulT X"); need(W, N * K, "matmulT W");
  const a = hip();
  const Y = _deviceNode(M * N);
  const xd = X._devData(), wd = W._devData();
  const xp = xpForward(a, X, W);
  a.matmulTFwd(Y._dev, xd, wd, M, K, N, ...xpArgs(xp));
  return attach(Y, xp && [xp.x, xp.w], () => {
    const g = Y._gradDev();
    const gxp = Y._gxp;  // handed over: freed with the GEMMs' temporaries
    Y._gxp = null;
    matmulTGrads(a, g, X, W, M, K, N, xp, false, gxp);
  });
}

/** True when X's first gradient, dY·W, should stay as the two unreduced K
 *  pieces of its GEMM: X is an RMSNorm output (whose backward adds the
 *  halves itself, saving the GEMM's partial-sum pass) and the GEMM splits K
 *  in two. */
function takesHalves(a, X, M, K, N) {
  return X._rmsOut === true && !X._hasGrad() && a.matmulTBwdXPieces(M, K, N) === 2;
}

/** X.grad (+)= g[M,N]·W[N,K] (W a device buffer; wx its maxima or null;
 *  xg g's maxima, held already when hg is 1, else filled by the GEMM), as
 *  two halves when takesHalves. */
function bwdX(a, X, g, W, M, K, N, xg, wx, hg = 0) {
  if (takesHalves(a, X, M, K, N)) {
    const h = a.alloc(2 * M * K * 4);
    a.matmulTBwdXHalves(h, g, W, M, K, N, xg, wx, hg | (wx ? 2 : 0));
    X._adoptHalves(h);
    return;
  }
  const gx = X._gradAcc();
  a.matmulTBwdX(gx.h, g, W, M, K, N, gx.beta, xg, wx, hg | (wx ? 2 : 0));
}

/** dX now; dW now, or deferred to the end of backward() for a weight marked
 *  _deferGrad (its gradient has no other writer in the step).  xp: the
 *  forward's operand maxima (or null); the maxima of g (gxp when its writer
 *  left them, else filled by the first gradient GEMM) serve both.  gTemp: g
 *  is a temporary buffer to free once both gradients are queued. */
function matmulTGrads(a, g, X, W, M, K, N, xp, gTemp = false, gxp = null) {
  // g's maxima: handed over by the op that wrote g (gxp, now owned here), else
  // filled by the first GEMM
  const xg = gxp || a.alloc(XP_BYTES);
  const hg = gxp ? 1 : 0;
  const temps = gTemp ? [g, xg] : [xg];
  const done = () => { for (const h of temps) a.free(h); };
  const wd = W._devData(), wx = xpW(xp, W);
  if (X !== W && takesHalves(a, X, M, K, N)) {
    bwdX(a, X, g, wd, M, K, N, xg, wx, hg);
    const gw = W._gradAcc();
    const xd = X._devData(), xx = xpX(xp, X);
    if (W._deferGrad && _deferWeightGrad([gw.h, g, xd, M, K, N, gw.beta, xg, xx], temps, [W])) return;
    a.matmulTBwdW(gw.h, g, xd, M, K, N, gw.beta, xg, xx, xx ? 3 : 1);
    done();
    return;
  }
  const gx = X._gradAcc();
  const gw = W._gradAcc();
  const xd = X._devData(), xx = xpX(xp, X);
  if (W._deferGrad && X !== W && _deferWeightGrad([gw.h, g, xd, M, K, N, gw.beta, xg, xx], temps, [W])) {
    // the job reads xg at the end of backward(), after this GEMM has filled it
    a.matmulTBwdX(gx.h, g, wd, M, K, N, gx.beta, xg, wx, hg | (wx ? 2 : 0));
    return;
  }
  a.matmulTBwd(gx.h, gx.beta, gw.h, gw.beta, g, xd, wd, M, K, N, xg, xx, wx, hg | (xx ? 2 : 0) | (wx ? 4 : 0));
  done();
}

/** Y[M,N] = X[M,K] · B[K,N] with B row-major (tensor.js:56-81). */
export function matmul(X, B, M, K, N) {
  posInt(M, "M"); posInt(K, "K"); posInt(N, "N");
  need(X, M * K, "matmul X"); need(B, K * N, "matmul B");
  const a = hip();
  const Y = _deviceNode(M * N);
  // C[M,N] = A[M,K]·B[K,N] is the dX form of the NT kernels.
  a.matmulTBwdX(Y._dev, X._devData(), B._devData(), M, N, K, 0);
  return attach(Y, null, () => {
    const g = Y._gradDev();
    const tmp = allocF32(M * K);
    a.matmulTFwd(tmp, g, B._devData(), M, N, K);  // dY[M,N]·B[K,N]ᵀ
    const gx = X._gradAcc();
    a.accum(gx.h, tmp, M * K, gx.beta);
    a.free(tmp);
    const gb = B._gradAcc();
    a.matmulTBwdW(gb.h, X._devData(), g, M, N, K, gb.beta);  // Xᵀ·dY
  });
}

// ── token ids resident in device memory ─────────────────────────────────
/**
 * n int32 token ids in device memory (-1 marks an id outside [0,V)).  The
 * device-resident train() loop cuts its batches into two of these each step;
 * embedLookup and crossEntropyMean accept one wherever they take a host id
 * array, and then build nothing on the host.
 */
export class DeviceIds {
  constructor(h, n) { this.h = h; this.n = n; }
  /** Uploads host ids (values that are not integers in [0,V) become -1). */
  static from(ids, V) {
    const n = ids.length;
    posInt(n, "ids.length");
    const v = new Int32Array(n);
    for (let t = 0; t < n; t++) {
      const id = ids[t];
      v[t] = Number.isInteger(id) && id >= 0 && id < V ? id : -1;
    }
    const a = hip();
    const h = a.alloc(n * 4);
    a.h2d(h, v);
    return new DeviceIds(h, n);
  }
  free() { if (this.h) { hip().free(this.h); this.h = null; } }
}

// ── embedding lookup ────────────────────────────────────────────────────
/**
 * X[T,D] = W[ids[t], :] (tensor.js:85-99); backward scatter-adds into W.grad
 * in increasing t per id (the reference's order), without atomics.  With host
 * ids the grouping plan is built on the host and travels with the ids in one
 * upload; with DeviceIds the positions are grouped by a device sort of
 * (id, t) keys — the same sums in the same order.  An id outside [0,V) gives
 * a NaN row and no gradient, as in the reference.
 */
export function embedLookup(W, ids, V, D) {
  posInt(V, "V"); posInt(D, "D");
  need(W, V * D, "embedLookup W");
  if (ids instanceof DeviceIds) return embedLookupDevice(W, ids, V, D);
  const T = ids.length;
  posInt(T, "ids.length");
  const a = hip();
  // counting sort of valid ids: perm (t in increasing order per id), segments
  const count = new Int32Array(V + 1);
  const idv = new Int32Array(T);
  for (let t = 0; t < T; t++) {
    const id = ids[t];
    if (Number.isInteger(id) && id >= 0 && id < V) { idv[t] = id; count[id + 1]++; } else idv[t] = -1;
  }
  let nseg = 0;
  for (let v = 0; v < V; v++) { if (count[v + 1] > 0) nseg++; count[v + 1] += count[v]; }
  const buf = new Int32Array(2 * T + 2 * nseg + 2);
  buf.set(idv, 0);
  const perm = buf.subarray(T, 2 * T), segStart = buf.subarray(2 * T, 2 * T + nseg + 1);
  const segId = buf.subarray(2 * T + nseg + 1, 2 * T + 2 * nseg + 1);
  const fill = count.slice(0, V);
  for (let t = 0; t < T; t++) if (idv[t] >= 0) perm[fill[idv[t]]++] = t;
  let s = 0;
  for (let v = 0; v < V; v++) if (count[v + 1] > count[v]) { segId[s] = v; segStart[s] = count[v]; s++; }
  segStart[nseg] = count[V];
  const h = a.alloc(buf.byteLength);
  a.h2d(h, buf);
  const hIds = a.view(h, 0, T * 4), hPerm = a.view(h, T * 4, T * 4);
  const hStart = a.view(h, 2 * T * 4, (nseg + 1) * 4), hSeg = a.view(h, (2 * T + nseg + 1) * 4, Math.max(1, nseg) * 4);
  const X = _deviceNode(T * D);
  a.embedFwd(X._dev, W._devData(), hIds, T, V, D);
  return attach(X, [h], () => {
    const gW = W._gradZeroed();
    if (nseg > 0) a.embedBwd(gW, X._gradDev(), hPerm, hStart, hSeg, nseg, D);
  });
}

function embedLookupDevice(W, ids, V, D) {
  const T = ids.n;
  posInt(T, "ids.n");
  const a = hip();
  const X = _deviceNode(T * D);
  a.embedFwd(X._dev, W._devData(), ids.h, T, V, D);
  return attach(X, null, () => {
    const { h: gW, zeroed } = W._gradZeroedInfo();
    const len = a.embedKeysLen(T);
    const keys = a.alloc(len * 8);
    a.embedSortKeys(keys, len, ids.h, T, V);
    a.embedBwdSorted(gW, X._gradDev(), keys, T, V, D, zeroed ? 0 : 1);
    a.free(keys);
  });
}

// ── RMSNorm (per token) ─────────────────────────────────────────────────
/** Y[T,D] = X[T,D] / rms(X[t]) · w[D], eps inside the root (tensor.js:103-128). */
export function rmsNorm(X, w, T, D, eps = 1e-6) {
  posInt(T, "T"); posInt(D, "D");
  need(X, T * D, "rmsNorm X"); need(w, D, "rmsNorm w");
  const a = hip();
  const Y = _deviceNode(T * D);
  const inv = allocF32(T);
  a.rmsnormFwd(Y._dev, inv, X._devData(), w._devData(), T, D, eps);
  Y._rmsOut = true;  // its gradient may arrive as two halves (bwdX)
  return attach(Y, [inv], () => {
    const gx = X._gradAccFrom();
    const hv = Y._gradHalves();
    // A weight whose only gradient is this norm's (w._deferGrad) gets its
    // column sum at the end of backward(), grouped with the other norms'.
    const parts = w._deferGrad && _deferring() ? a.rmsnormBwdParts(T, D) : 0;
    if (parts > 0) {
      const part = allocF32(parts * D);
      const g = hv || Y._gradDev();
      a.rmsnormBwdPartial(gx.h, gx.src, part, g, hv ? 1 : 0, X._devData(), w._devData(), inv, T, D);
      const gw = w._gradAcc();
      _deferColsum([gw.h, part, parts, D, gw.beta], [part], [w]);
      return;
    }
    const gw = w._gradAcc();
    if (hv) a.rmsnormBwdFromHalves(gx.h, gx.src, gw.h, gw.beta, hv, X._devData(), w._devData(), inv, T, D);
    else a.rmsnormBwdFrom(gx.h, gx.src, gw.h, gw.beta, Y._gradDev(), X._devData(), w._devData(), inv, T, D);
  });
}

// ── RoPE ────────────────────────────────────────────────────────────────
const _ropeTables = new Map();
/** Device cos/sin tables for (theta, dHead) covering npos positions; the
 *  angles use the reference's expression 1/θ^(i/dHead)·pos in fp64. */
function ropeTable(theta, dHead, npos) {
  const key = `${theta}|${dHead}`;
  let e = _ropeTables.get(key);
  if (e && e.npos >= npos) return e;
  const half = dHead / 2;
  const n = Math.max(npos, e ? 2 * e.npos : 0);
  const c = new Float64Array(n * half), s = new Float64Array(n * half);
  for (let p = 0; p < n; p++) {
    for (let i = 0; i < dHead; i += 2) {
      const freq = 1 / Math.pow(theta, i / dHead);
      const ang = p * freq;
      c[p * half + i / 2] = Math.cos(ang);
      s[p * half + i / 2] = Math.sin(ang);
    }
  }
  const a = hip();
  const hc = a.alloc(c.byteLength), hs = a.alloc(s.byteLength);
  a.h2d(hc, c); a.h2d(hs, s);
  if (e) { a.free(e.c); a.free(e.s); }
  e = { npos: n, c: hc, s: hs };
  _ropeTables.set(key, e);
  return e;
}

/** Rotates interleaved pairs of every head; position = pos0 + (t % posStride)
 *  when posStride > 0 (tensor.js:133-166).  Backward applies Rᵀ. */
export function ropeRows(X, T, nHead, dHead, pos0, theta = 10000, posStride = 0) {
  posInt(T, "T"); posInt(nHead, "nHead"); posInt(dHead, "dHead");
  if (dHead % 2) throw new RangeError(`ropeRows: dHead must be even, got ${dHead}`);
  if (!Number.isInteger(pos0) || pos0 < 0) throw new RangeError(`ropeRows: pos0 must be a non-negative integer`);
  need(X, T * nHead * dHead, "ropeRows X");
  const npos = pos0 + (posStride > 0 ? Math.min(T, posStride) : T);
  const tab = ropeTable(theta, dHead, npos);
  const a = hip();
  const Y = _deviceNode(T * nHead * dHead);
  a.ropeFwd(Y._dev, X._devData(), tab.c, tab.s, tab.npos, T, nHead, dHead, pos0, posStride);
  return attach(Y, null, () => {
    const gx = X._gradAcc();
    const t2 = ropeTable(theta, dHead, npos);
    a.ropeBwd(gx.h, Y._gradDev(), t2.c, t2.s, t2.npos, T, nHead, dHead, pos0, posStride, gx.beta);
  });
}

/**
 * Fused q/k/v split + RoPE of a fused projection qkv[rows, (nH+2·nKV)·dHead]:
 * returns [ropeRows(sliceCols(q)), ropeRows(sliceCols(k)), sliceCols(v)] —
 * the train.js:133-138 sequence — reading qkv once.  The three outputs share
 * one backward, attached to q (the first created, so it runs after every
 * consumer of q, k and v has accumulated its gradient): it writes
 * qkv.grad (+)= [Rᵀ·gq | Rᵀ·gk | gv] in one pass, the value the reference's
 * ropeRows and sliceCols backwards add up to.
 */
export function qkvRope(qkv, rows, nH, nKV, dHead, pos0, theta = 10000, posStride = 0) {
  posInt(rows, "rows"); posInt(nH, "nH"); posInt(nKV, "nKV"); posInt(dHead, "dHead");
  if (dHead % 2) throw new RangeError(`qkvRope: dHead must be even, got ${dHead}`);
  if (!Number.isInteger(pos0) || pos0 < 0) throw new RangeError(`qkvRope: pos0 must be a non-negative integer`);
  need(qkv, rows * (nH + 2 * nKV) * dHead, "qkvRope qkv");
  const npos = pos0 + (posStride > 0 ? Math.min(rows, posStride) : rows);
  const tab = ropeTable(theta, dHead, npos);
  const a = hip();
  const q = _deviceNode(rows * nH * dHead);
  const k = _deviceNode(rows * nKV * dHead);
  const v = _deviceNode(rows * nKV * dHead);
  a.qkvRopeFwd(q._dev, k._dev, v._dev, qkv._devData(), tab.c, tab.s, tab.npos, rows, nH, nKV, dHead, pos0, posStride);
  attach(q, null, () => {
    if (!q._hasGrad() && !k._hasGrad() && !v._hasGrad()) return;
    const g = qkv._gradAcc();
    const t2 = ropeTable(theta, dHead, npos);
    a.qkvRopeBwd(g.h, q._hasGrad() ? q._gradDev() : null, k._hasGrad() ? k._gradDev() : null,
      v._hasGrad() ? v._gradDev() : null, t2.c, t2.s, t2.npos, rows, nH, nKV, dHead, pos0, posStride, g.beta);
  });
  q._bdevAlways = _tapeEnabled();
  return [q, k, v];
}

/**
 * The qkv projection, q/k RoPE and causal attention of a decoder layer
 * (train.js:131-142: matmulT → sliceCols×3 + ropeRows×2 → causalAttn(Batch))
 * as one node.  Forward: one GEMM whose epilogue rotates the q and k columns
 * (fg_matmulT_fwd_rope), then attention reading q, k, v as column blocks of
 * that qkv buffer.  Backward: attention writes [Rᵀ·dQ | Rᵀ·dK | dV] straight
 * into the qkv gradient (fg_attn_bwd_qkv), then the projection's input and
 * weight gradients.  Values and gradients equal the separate ops' bit for
 * bit.  Needs dHead ∈ {32, 64, 96, 128} (the MFMA attention) and nH ≥ nKV;
 * returns null otherwise, and the caller composes the separate ops.
 */
export function qkvRopeAttention(xn, Wqkv, B, T, nH, nKV, dHead, D, pos0, theta = 10000, posStride = 0) {
  if (!(dHead === 32 || dHead === 64 || dHead === 96 || dHead === 128) || nH < nKV) return null;
  posInt(B, "B"); posInt(T, "T"); posInt(nH, "nH"); posInt(nKV, "nKV"); posInt(D, "D");
  if (!Number.isInteger(pos0) || pos0 < 0) throw new RangeError(`qkvRopeAttention: pos0 must be a non-negative integer`);
  const rows = B * T, W = (nH + 2 * nKV) * dHead;
  need(xn, rows * D, "qkvRopeAttention xn"); need(Wqkv, W * D, "qkvRopeAttention Wqkv");
  const npos = pos0 + (posStride > 0 ? Math.min(rows, posStride) : rows);
  const tab = ropeTable(theta, dHead, npos);
  const a = hip();
  const qkv = allocF32(rows * W);
  const xd = xn._devData(), wd = Wqkv._devData();
  const xp = xpForward(a, xn, Wqkv);
  a.matmulTFwdRope(qkv, xd, wd, rows, D, W, tab.c, tab.s, tab.npos, nH, nKV, dHead, pos0, posStride, ...xpArgs(xp));
  const O = _deviceNode(rows * nH * dHead);
  const lse = allocF32(B * nH * T);
  // the maxima of q, k, v (the attention's operand powers of two), kept for the backward
  const xa = xp ? a.alloc(3 * XP_BYTES) : null;
  a.attnFwdQkv(O._dev, lse, qkv, B, T, nH, nKV, dHead, xa);
  return attach(O, xp ? [qkv, lse, xp.x, xp.w, xa] : [qkv, lse], () => {
    const g = allocF32(rows * W);
    const t2 = ropeTable(theta, dHead, npos);
    a.attnBwdQkv(g, O._gradDev(), qkv, O._devData(), lse, B, T, nH, nKV, dHead, t2.c, t2.s, t2.npos, pos0,
      posStride, xa);
    matmulTGrads(a, g, xn, Wqkv, rows, D, W, xp, true);
  });
}

// ── column slice ────────────────────────────────────────────────────────
/** Columns [off, off+len) of X[M,K] → [M,len]; backward adds back (tensor.js:170-183). */
export function sliceCols(X, M, K, off, len) {
  posInt(M, "M"); posInt(K, "K"); posInt(len, "len");
  if (!Number.isInteger(off) || off < 0 || off + len > K) throw new RangeError(`sliceCols: [${off}, ${off + len}) outside ${K} columns`);
  need(X, M * K, "sliceCols X");
  const a = hip();
  const Y = _deviceNode(M * len);
  a.sliceColsFwd(Y._dev, X._devData(), M, K, off, len);
  return attach(Y, null, () => {
    a.sliceColsBwd(X._gradZeroed(), Y._gradDev(), M, K, off, len);
  });
}

// ── causal attention ────────────────────────────────────────────────────
function attention(Q, K, V, B, T, nH, nKV, dHead, what) {
  posInt(B, "B"); posInt(T, "T"); posInt(nH, "nH"); posInt(nKV, "nKV"); posInt(dHead, "dHead");
  need(Q, B * T * nH * dHead, `${what} Q`);
  need(K, B * T * nKV * dHead, `${what} K`);
  need(V, B * T * nKV * dHead, `${what} V`);
  const a = hip();
  const O = _deviceNode(B * T * nH * dHead);
  const lse = allocF32(B * nH * T);
  a.attnFwd(O._dev, lse, Q._devData(), K._devData(), V._devData(), B, T, nH, nKV, dHead);
  return attach(O, [lse], () => {
    const gq = Q._gradAcc(), gk = K._gradAcc(), gv = V._gradAcc();
    a.attnBwd(gq.h, gq.beta, gk.h, gk.beta, gv.h, gv.beta, O._gradDev(), Q._devData(), K._devData(),
      V._devData(), O._devData(), lse, B, T, nH, nKV, dHead);
  });
}

/** Causal self-attention with GQA, one sequence (tensor.js:191-268). */
export function causalAttn(Q, K, V, T, nH, nKV, dHead) {
  return attention(Q, K, V, 1, T, nH, nKV, dHead, "causalAttn");
}

/** Batched causal attention with a block-diagonal mask (tensor.js:299-376). */
export function causalAttnBatch(Q, K, V, B, T, nH, nKV, dHead) {
  return attention(Q, K, V, B, T, nH, nKV, dHead, "causalAttnBatch");
}

// ── SwiGLU ──────────────────────────────────────────────────────────────
/** O[T,H] = silu(G) ⊙ U (tensor.js:272-290). */
export function swigluRows(G, U, T, H) {
  posInt(T, "T"); posInt(H, "H");
  need(G, T * H, "swigluRows G"); need(U, T * H, "swigluRows U");
  const a = hip();
  const O = _deviceNode(T * H);
  a.swigluFwd(O._dev, G._devData(), U._devData(), T * H);
  return attach(O, null, () => {
    const gg = G._gradAcc(), gu = U._gradAcc();
    a.swigluBwd(gg.h, gg.beta, gu.h, gu.beta, O._gradDev(), G._devData(), U._devData(), T * H);
  });
}

// ── fused gate/up projection + SwiGLU (train.js:149-151) ────────────────
/**
 * Stores two parameters of equal width back to back in one device buffer
 * (A's rows, then B's), so a GEMM can treat them as one [A; B] weight.  The
 * host arrays stay as they are; each Node keeps a view of its half.
 */
export function packPair(A, B) {
  if (!(A instanceof Node) || !(B instanceof Node)) throw new TypeError("packPair: expected Nodes");
  const a = hip();
  const parent = a.alloc((A.n + B.n) * 4);
  const va = a.view(parent, 0, A.n * 4), vb = a.view(parent, A.n * 4, B.n * 4);
  const pr = { parent, a: A, b: B, va, vb, gparent: null, ga: null, gb: null };
  for (const [N, v] of [[A, va], [B, vb]]) {
    if (!N._hostValid) N.data;  // bring a device-only value to the host before rebinding
    if (N._dev) a.free(N._dev);
    N._dev = v;
    N._exposed = true;          // the next device use uploads the host value into the view
    N._pair = pr;
  }
  return pr;
}

/** {h, beta} for writing both gradients of a pair with one GEMM, or null. */
function pairGradAcc(pr) {
  const A = pr.a, B = pr.b;
  if (!A._hasGrad() && !B._hasGrad()) {
    const a = hip();
    pr.gparent = a.alloc((A.n + B.n) * 4);
    pr.ga = a.view(pr.gparent, 0, A.n * 4);
    pr.gb = a.view(pr.gparent, A.n * 4, B.n * 4);
    A._gdev = pr.ga; B._gdev = pr.gb;
    A._gHostValid = false; B._gHostValid = false;
    return { h: pr.ga, beta: 0 };
  }
  if (pr.ga && A._gdev === pr.ga && B._gdev === pr.gb) {
    const ga = A._gradAcc(), gb = B._gradAcc();
    if (ga.beta === gb.beta) return { h: pr.ga, beta: ga.beta };
    return { split: [ga, gb] };
  }
  return null;
}

/**
 * act[T,H] = swigluRows(matmulT(X, Wg), matmulT(X, Wu)) with the two
 * projections as one GEMM over [Wg; Wu] when the pair is packed
 * (packPair), the same values as the three separate ops (each output is the
 * same dot product).  Backward: one swiglu pass writes [dG | dU], then one
 * input-gradient GEMM over K = 2H and one weight-gradient GEMM for both
 * weights.  Falls back to the separate ops when the weights are not packed.
 */
export function swigluGateUp(X, Wg, Wu, T, D, H) {
  posInt(T, "T"); posInt(D, "D"); posInt(H, "H");
  need(X, T * D, "swigluGateUp X"); need(Wg, H * D, "swigluGateUp Wg"); need(Wu, H * D, "swigluGateUp Wu");
  const pr = Wg._pair;
  const packed = pr && pr.a === Wg && pr.b === Wu && Wg._dev === pr.va && Wu._dev === pr.vb;
  if (!packed) return swigluRows(matmulT(X, Wg, T, D, H), matmulT(X, Wu, T, D, H), T, H);
  const a = hip();
  Wu._devData();
  const GU = allocF32(T * 2 * H);
  const O = _deviceNode(T * H);
  const xd = X._devData(), wd = Wg._devData();
  // the packed [Wg; Wu] maxima describe both halves' versions
  const xp = xpForward(a, X, Wg);
  const vu = Wu._ver;
  a.matmulTFwdSwiglu(O._dev, GU, xd, wd, T, D, H, ...xpArgs(xp));
  return attach(O, xp ? [GU, xp.x, xp.w] : [GU], () => {
    const gGU = allocF32(T * 2 * H);
    // the SwiGLU backward leaves the maxima of [dG | dU] for both GEMMs
    const xg = a.alloc(XP_BYTES);
    a.swigluGuBwd(gGU, 0, O._gradDev(), GU, T, H, xg);
    Wu._devData();
    const w = Wg._devData();
    const wx = Wu._ver === vu ? xpW(xp, Wg) : null;
    bwdX(a, X, gGU, w, T, D, 2 * H, xg, wx, 1);
    const gw = pairGradAcc(pr);
    const xd2 = X._devData(), xx = xpX(xp, X);
    if (gw && !gw.split) {
      if (Wg._deferGrad && _deferWeightGrad([gw.h, gGU, xd2, T, D, 2 * H, gw.beta, xg, xx], [gGU, xg], [Wg, Wu])) return;
      a.matmulTBwdW(gw.h, gGU, xd2, T, D, 2 * H, gw.beta, xg, xx, xx ? 3 : 1);
    } else {
      const tmp = allocF32(2 * H * D);
      a.matmulTBwdW(tmp, gGU, xd2, T, D, 2 * H, 0, xg, xx, xx ? 3 : 1);
      const [gg, gu] = gw ? gw.split : [Wg._gradAcc(), Wu._gradAcc()];
      a.accum(gg.h, a.view(tmp, 0, H * D * 4), H * D, gg.beta);
      a.accum(gu.h, a.view(tmp, H * D * 4, H * D * 4), H * D, gu.beta);
      a.free(tmp);
    }
    a.free(gGU);
    a.free(xg);
  });
}

// ── weighted sum (test/custom objectives) ───────────────────────────────
/** out[0] = Σ Y[i]·t[i]; backward passes g·t to Y (tensor.js:380-389). */
export function weightedSum(Y, t) {
  const n = Y.n;
  if (!t || t.length < n) throw new RangeError(`weightedSum: weights of length ${t ? t.length : 0} < ${n}`);
  const a = hip();
  const tw = t instanceof Float32Array && t.length === n ? t : Float32Array.from(Array.prototype.slice.call(t, 0, n));
  const ht = allocF32(n);
  a.h2d(ht, tw);
  const out = _deviceNode(1);
  a.weightedSumFwd(out._dev, Y._devData(), ht, n);
  if (!graphState.capturing) out._ticket = a.readAsync(out._dev, 4);
  return attach(out, [ht], () => {
    const gy = Y._gradAcc();
    a.weightedSumBwd(gy.h, out._gradDev(), ht, n, gy.beta);
  });
}

// ── cross-entropy (mean) ────────────────────────────────────────────────
/** L = -(1/T) Σ log softmax(logits[t])[targets[t]]; dLogits = (P − OneHot)/T
 *  (tensor.js:393-417).  Softmax is recomputed from the saved row LSE. */
export function crossEntropyMean(logits, targets, T, V) {
  posInt(T, "T"); posInt(V, "V");
  need(logits, T * V, "crossEntropyMean logits");
  const a = hip();
  let ht, saved;
  if (targets instanceof DeviceIds) {
    if (targets.n !== T) throw new RangeError(`crossEntropyMean: ${targets.n} device targets for T=${T}`);
    ht = targets.h;
    saved = [];
  } else {
    const tg = new Int32Array(T);
    for (let t = 0; t < T; t++) {
      const v = targets[t];
      tg[t] = Number.isInteger(v) && v >= 0 && v < V ? v : -1;
    }
    ht = a.alloc(T * 4);
    a.h2d(ht, tg);
    saved = [ht];
  }
  const lse = allocF32(T);
  saved.push(lse);
  const L = _deviceNode(1);
  a.ceFwd(L._dev, lse, logits._devData(), ht, T, V);
  if (!graphState.capturing) L._ticket = a.readAsync(L._dev, 4);
  return attach(L, saved, () => ceBwdInto(a, logits, lse, ht, L, T, V));
}

/** logits.grad (+)= the CE gradient of loss node L; a fresh gradient also
 *  gets its magnitude bound |L.grad| / T as GEMM operand maxima, which the
 *  LM head's gradient GEMMs take instead of reading the gradient for them. */
function ceBwdInto(a, logits, lse, ht, L, T, V) {
  const gl = logits._gradAcc();
  const ld = logits._devData(), gL = L._gradDev();
  if (gl.beta === 0) {
    const xp = a.alloc(XP_BYTES);
    a.ceBwd(gl.h, ld, lse, ht, gL, T, V, 0, xp);
    logits._gxp = xp;
  } else {
    a.ceBwd(gl.h, ld, lse, ht, gL, T, V, gl.beta);
  }
}

/**
 * crossEntropyMean for a loss whose backward always follows (the training
 * step): the forward also writes the gradient of a seed of 1,
 * (1/T)(softmax − onehot), in the same pass over the logits
 * (fg_ce_fwd_bwd: the logits are read from HBM once, not twice).  When
 * backward() seeds this node and the logits have no gradient yet, that buffer
 * becomes logits.grad; otherwise the backward runs as crossEntropyMean's.
 * Values and gradients equal crossEntropyMean's bit for bit.
 */
export function crossEntropyMeanFused(logits, targets, T, V) {
  posInt(T, "T"); posInt(V, "V");
  need(logits, T * V, "crossEntropyMean logits");
  const a = hip();
  let ht, saved;
  if (targets instanceof DeviceIds) {
    if (targets.n !== T) throw new RangeError(`crossEntropyMean: ${targets.n} device targets for T=${T}`);
    ht = targets.h;
    saved = [];
  } else {
    const tg = new Int32Array(T);
    for (let t = 0; t < T; t++) {
      const v = targets[t];
      tg[t] = Number.isInteger(v) && v >= 0 && v < V ? v : -1;
    }
    ht = a.alloc(T * 4);
    a.h2d(ht, tg);
    saved = [ht];
  }
  const lse = allocF32(T), pre = allocF32(T * V);
  // the bound of the precomputed gradient's magnitudes (1/T), as GEMM operand maxima
  const xpre = a.alloc(XP_BYTES);
  saved.push(lse, pre, xpre);
  const L = _deviceNode(1);
  a.ceFwdBwd(L._dev, lse, pre, logits._devData(), ht, T, V, xpre);
  if (!graphState.capturing) L._ticket = a.readAsync(L._dev, 4);
  return attach(L, saved, () => {
    if (L._seeded && !logits._hasGrad() && L._saved.includes(pre)) {
      L._seeded = false;
      logits._adoptGrad(pre);
      logits._gxp = xpre;
      L._saved = L._saved.filter((h) => h !== pre && h !== xpre);  // now owned by logits
      return;
    }
    ceBwdInto(a, logits, lse, ht, L, T, V);
  });
}

/**
 * R + X·Wᵀ in one GEMM (the addTensors(x, matmulT(a, W)) residual pair of
 * train.js:144-145, 152-153): the residual is added in the GEMM epilogue.
 * Backward: R.grad (+)= g, then matmulT's dX/dW.
 */
export function matmulTResid(R, X, W, M, K, N) {
  posInt(M, "M"); posInt(K, "K"); posInt(N, "N");
  need(R, M * N, "matmulTResid R"); need(X, M * K, "matmulTResid X"); need(W, N * K, "matmulTResid W");
  const a = hip();
  const Y = _deviceNode(M * N);
  const rd = R._devData(), xd = X._devData(), wd = W._devData();
  const xp = xpForward(a, X, W);
  a.matmulTFwdResid(Y._dev, rd, xd, wd, M, K, N, ...xpArgs(xp));
  return attach(Y, xp && [xp.x, xp.w], () => {
    const g = Y._gradDev();
    if (!R._hasGrad() && R !== X && R !== W) {
      R._shareGrad(Y);  // R's gradient starts as g: share Y's buffer (copy on write)
    } else {
      const gr = R._gradAcc();
      a.accum(gr.h, g, M * N, gr.beta);
    }
    matmulTGrads(a, g, X, W, M, K, N, xp);
  });
}

// ── residual add (train.js:230-238, autograd.js:60-67) ──────────────────
export function _addTensors(A, B, n) {
  need(A, n, "add a"); need(B, n, "add b");
  const a = hip();
  const Y = _deviceNode(n);
  a.addFwd(Y._dev, A._devData(), B._devData(), n);
  return attach(Y, null, () => {
    const g = Y._gradDev();
    const ga = A._gradAcc();
    a.accum(ga.h, g, n, ga.beta);
    const gb = B._gradAcc();
    a.accum(gb.h, g, n, gb.beta);
  });
}
