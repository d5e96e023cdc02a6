/**
 * L5 · KV cache of the inference forward, resident in device memory.
 *
 * Same interface as forge-llm's contiguous KVCache (src/L5/attention.js:
 * 128-156): nLayers × maxSeq × kvDim keys and values, `put`, `kView`/`vView`,
 * `sliceK`/`sliceV`, `reset`, `bytes`, `len`.  The arrays live in HBM, where
 * Transformer.forward's kernels write each position's K and V; `k` / `v` and
 * the views download a copy on access (writing into that copy does not
 * change the cache — use `put`).  The reference's single-row attention
 * helpers (attentionDecode, attentionNaive, flashAttention) are CPU code: the
 * decode attention runs inside Transformer.forward on the device.
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

function onCpu(name) {
  return function () {
    throw new Error(`forge-llm_amd: ${name} is a CPU single-row helper of the reference; the decode attention runs inside Transformer.forward on the device`);
  };
}
export const attentionDecode = onCpu("attentionDecode");
export const attentionNaive = onCpu("attentionNaive");
export const flashAttention = onCpu("flashAttention");
