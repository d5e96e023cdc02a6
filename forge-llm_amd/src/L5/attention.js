/**
 * L5 · KV cache of the inference forward, resident in device memory.
 *
 * Same interface as forge-llm's contiguous KVCache (src/L5/attention.js:
 * 128-156): nLayers × maxSeq × kvDim keys and values, `put`, `kView`/`vView`,
 * `sliceK`/`sliceV`, `reset`, `bytes`, `len`.  The arrays live in HBM, where
 * Transformer.forward's kernels write each position's K and V; `k` / `v` and
 * the views download a copy on access (writing into that copy does not
 * change the cache — use `put`).  The reference's single-row attention
 * helpers over host arrays (attentionDecode, attentionNaive, flashAttention)
 * are kept with their signatures and compute on the device; the model's own
 * decode attention runs inside Transformer.forward.
 */
import { hip } from "../L2/device.js";

export class KVCache {
  constructor(nLayers, maxSeq, kvDim) {
    for (const [k, v] of [["nLayers", nLayers], ["maxSeq", maxSeq], ["kvDim", kvDim]])
      if (!Number.isInteger(v) || v <= 0) throw new RangeError(`KVCache: ${k} must be a positive integer, got ${v}`);
    this.nLayers = nLayers; this.maxSeq = maxSeq; this.kvDim = kvDim;
    const a = hip();
    const bytes = nLayers * maxSeq * kvDim * 4;
    this.kd = a.alloc(bytes); this.vd = a.alloc(bytes);
    a.zero(this.kd, bytes); a.zero(this.vd, bytes);
    this.len = 0;
  }
  _off(layer, pos) {
    if (!Number.isInteger(layer) || layer < 0 || layer >= this.nLayers) throw new RangeError(`KVCache: layer ${layer} out of range`);
    if (!Number.isInteger(pos) || pos < 0 || pos > this.maxSeq) throw new RangeError(`KVCache: position ${pos} out of range`);
    return (layer * this.maxSeq + pos) * this.kvDim;
  }
  _read(h, off, n) {
    const out = new Float32Array(n);
    if (n > 0) hip().d2h(h, out, off * 4);
    return out;
  }
  put(layer, pos, k, v) {
    const o = this._off(layer, pos);
    if (pos >= this.maxSeq) throw new RangeError(`KVCache: position ${pos} out of range`);
    const a = hip();
    a.h2d(this.kd, Float32Array.from(k.subarray ? k.subarray(0, this.kvDim) : k.slice(0, this.kvDim)), o * 4);
    a.h2d(this.vd, Float32Array.from(v.subarray ? v.subarray(0, this.kvDim) : v.slice(0, this.kvDim)), o * 4);
    if (pos + 1 > this.len) this.len = pos + 1;
  }
  get k() { return this._read(this.kd, 0, this.nLayers * this.maxSeq * this.kvDim); }
  get v() { return this._read(this.vd, 0, this.nLayers * this.maxSeq * this.kvDim); }
  kView(layer, upto) { return this._read(this.kd, this._off(layer, 0), upto * this.kvDim); }
  vView(layer, upto) { return this._read(this.vd, this._off(layer, 0), upto * this.kvDim); }
  sliceK(layer, pos) { return this._read(this.kd, this._off(layer, pos), this.kvDim); }
  sliceV(layer, pos) { return this._read(this.vd, this._off(layer, pos), this.kvDim); }
  reset() { this.len = 0; }
  bytes() { return 2 * this.nLayers * this.maxSeq * this.kvDim * 4; }
  /** Frees the device arrays (the cache is unusable afterwards). */
  free() {
    const a = hip();
    if (this.kd) { a.free(this.kd); a.free(this.vd); this.kd = null; this.vd = null; }
  }
}

// ── single-query-row attention over host arrays (attention.js:31-126) ──
// out[0..d) = Σ_j softmax_j(scale · q·K_j) V_j over keys j < n (rows of d
// floats at K[kOff + j d], V[kOff + j d]); with causal, keys j > qOff are
// masked.  The operands are copied to the device, fg_row_attention computes
// the row there with the variant's own order of operations (mode 0: the
// two-pass decode loop, 1: softmax then Σ p V, 2: blocks of `block` keys with
// the online rescale), and the d results are written into `out`.
function f32Slice(x, off, len, what) {
  if (len === 0) return new Float32Array(0);
  if (!x || typeof x.length !== "number" || x.length < off + len)
    throw new RangeError(`${what}: needs ${off + len} elements, has ${x ? x.length : 0}`);
  if (x instanceof Float32Array) return x.subarray(off, off + len);
  return Float32Array.from(Array.prototype.slice.call(x, off, off + len));
}

function rowAttention(name, mode, out, q, K, V, n, d, scale, causal, qOff, kOff, block, scores) {
  if (!Number.isInteger(n) || n < 0) throw new RangeError(`${name}: n must be a non-negative integer, got ${n}`);
  if (!Number.isInteger(d) || d <= 0) throw new RangeError(`${name}: d must be a positive integer, got ${d}`);
  if (!Number.isInteger(qOff)) throw new RangeError(`${name}: qOff must be an integer, got ${qOff}`);
  if (!Number.isInteger(kOff) || kOff < 0) throw new RangeError(`${name}: kOff must be a non-negative integer, got ${kOff}`);
  if (!Number.isInteger(block) || block <= 0) throw new RangeError(`${name}: block must be a positive integer, got ${block}`);
  if (typeof scale !== "number") throw new TypeError(`${name}: scale must be a number`);
  if (!out || out.length < d) throw new RangeError(`${name}: out needs ${d} elements`);
  const qh = f32Slice(q, 0, d, `${name} q`);
  const kh = f32Slice(K, kOff, n * d, `${name} K`);
  const vh = f32Slice(V, kOff, n * d, `${name} V`);
  const a = hip();
  const held = [];
  const alloc = (bytes) => { const h = a.alloc(bytes); held.push(h); return h; };
  try {
    const bq = alloc(d * 4), bk = alloc(Math.max(1, n * d) * 4), bv = alloc(Math.max(1, n * d) * 4);
    const bo = alloc(d * 4);
    const bs = scores ? alloc(Math.max(1, n) * 4) : null;
    a.h2d(bq, qh);
    if (n > 0) { a.h2d(bk, kh); a.h2d(bv, vh); }
    a.rowAttention(bo, bq, bk, bv, n, d, scale, causal ? 1 : 0, qOff, mode, block, bs);
    const r = new Float32Array(d);
    a.d2h(bo, r);
    for (let i = 0; i < d; i++) out[i] = r[i];
    if (scores && n > 0) {
      const sc = new Float32Array(n);
      a.d2h(bs, sc);
      for (let j = 0; j < n; j++) scores[j] = sc[j];
    }
  } finally {
    for (const h of held) a.free(h);
  }
  return out;
}

/** Two-pass single-row attention (attention.js:31-57); `s` (length >= n),
 *  when given, receives the scores as the reference leaves them. */
export function attentionDecode(out, q, K, V, n, d, scale, causal = true, qOff = 0, kOff = 0, s = null) {
  return rowAttention("attentionDecode", 0, out, q, K, V, n, d, scale, causal, qOff, kOff, 1,
                      s && s.length >= n ? s : null);
}
/** Reference single-row attention: softmax of the scores, then Σ p V (attention.js:63-79). */
export function attentionNaive(out, q, K, V, n, d, scale, causal = true, qOff = 0, kOff = 0) {
  return rowAttention("attentionNaive", 1, out, q, K, V, n, d, scale, causal, qOff, kOff, 1, null);
}
/** Online-softmax single-row attention over blocks of `block` keys (attention.js:89-126). */
export function flashAttention(out, q, K, V, n, d, scale, causal = true, qOff = 0, kOff = 0, block = 64) {
  return rowAttention("flashAttention", 2, out, q, K, V, n, d, scale, causal, qOff, kOff, block, null);
}
