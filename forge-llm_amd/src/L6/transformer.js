/**
 * L6 · model hyper-parameters and the inference model.  Config has the same
 * fields, defaults and derived dimensions as forge-llm's Config
 * (src/L6/transformer.js:29-53), including the GQA divisibility check;
 * Transformer is its inference forward (:69-184) on the device.
 */
import { hip } from "../L2/device.js";
import { KVCache } from "../L5/attention.js";
import { info, rowBytes } from "../L3/quant.js";

function pick(o, k, d) { return o[k] === undefined || o[k] === null ? d : o[k]; }

export class Config {
  constructor(o = {}) {
    this.dim = pick(o, "dim", 288);
    this.hidden = pick(o, "hidden", 768);
    this.nLayers = pick(o, "nLayers", 6);
    this.nHeads = pick(o, "nHeads", 6);
    this.nKvHeads = pick(o, "nKvHeads", 6);
    this.vocabSize = pick(o, "vocabSize", 32000);
    this.maxSeq = pick(o, "maxSeq", 1024);
    this.normEps = pick(o, "normEps", 1e-5);
    this.ropeTheta = pick(o, "ropeTheta", 10000);
    this.bosId = pick(o, "bosId", 1);
    this.eosId = pick(o, "eosId", 2);
    this._derive();
  }
  _derive() {
    if (this.nHeads % this.nKvHeads !== 0) {
      throw new Error(`GQA needs nHeads (${this.nHeads}) divisible by nKvHeads (${this.nKvHeads})`);
    }
    this.dHead = Math.floor(this.dim / this.nHeads);
    this.kvDim = this.nKvHeads * this.dHead;
    this.qkvOut = (this.nHeads + 2 * this.nKvHeads) * this.dHead;
    this.groupSize = this.nHeads / this.nKvHeads;
  }
}

// ── inference forward (transformer.js:69-184) ───────────────────────────────

/** fp32 RoPE table of the inference path (special.js:116-127): angles in
 *  fp64, cos/sin rounded to fp32. */
function ropeTableF32(maxPos, dim, theta) {
  const half = dim / 2;
  const cos = new Float32Array(maxPos * half), sin = new Float32Array(maxPos * half);
  for (let p = 0; p < maxPos; p++) {
    for (let i = 0; i < dim; i += 2) {
      const freq = 1 / Math.pow(theta, i / dim);
      const ang = p * freq;
      cos[p * half + i / 2] = Math.cos(ang);
      sin[p * half + i / 2] = Math.sin(ang);
    }
  }
  return { cos, sin };
}

/** f32 vectors (norm weights): a Float32Array / array, or a QuantLinear of
 *  type 0. */
function f32Weights(w, n, what) {
  if (w && typeof w === "object" && !ArrayBuffer.isView(w) && !Array.isArray(w) && "type" in w) {
    if (w.type !== 0) throw new Error(`Transformer.loadWeights: ${what} must be f32, got type ${w.type}`);
    w = w.bytes;
  }
  if (!w || w.length !== n) throw new RangeError(`Transformer.loadWeights: ${what} needs ${n} values, got ${w ? w.length : 0}`);
  return w instanceof Float32Array ? w : Float32Array.from(w);
}

/** A weight matrix [N, K]: f32 values, or a QuantLinear ({type, bytes, N, K},
 *  nn.js:19-40) of any type the decode kernels read (asQuantLinear,
 *  transformer.js:66-70).  Returns {type, data} with data the bytes to upload. */
function matWeights(w, N, K, what) {
  if (w && typeof w === "object" && !ArrayBuffer.isView(w) && !Array.isArray(w) && "type" in w) {
    if ((w.N !== undefined && w.N !== N) || (w.K !== undefined && w.K !== K))
      throw new RangeError(`Transformer.loadWeights: ${what} is [${w.N}, ${w.K}], [${N}, ${K}] expected`);
    if (w.type === 0) return { type: 0, data: f32Weights(w.bytes, N * K, what) };
    if (!DEVICE_TYPES.has(w.type)) throw new Error(`Transformer.loadWeights: ${what} has ggml type ${w.type}, which the device decode does not read`);
    const bs = info(w.type).blockSize;
    if (K % bs !== 0) throw new RangeError(`Transformer.loadWeights: ${what}: rows of ${K} are not whole ${bs}-element blocks`);
    const need = rowBytes(w.type, K) * N;
    const b = w.bytes instanceof Uint8Array ? w.bytes : new Uint8Array(w.bytes.buffer, w.bytes.byteOffset, w.bytes.byteLength);
    if (b.byteLength < need) throw new RangeError(`Transformer.loadWeights: ${what} holds ${b.byteLength} bytes, ${need} needed`);
    return { type: w.type, data: b.subarray(0, need) };
  }
  return { type: 0, data: f32Weights(w, N * K, what) };
}
const DEVICE_TYPES = new Set([0, 1, 2, 6, 8, 12, 13, 14]);

const GRAPHS_KEPT = 4;

/**
 * Inference model (transformer.js:69-184) on the device: `loadWeights(w)`
 * uploads the weights once; `forward(token, pos, cache)` runs one decode step
 * (fg_decode_step: embed, per layer RMSNorm → QKV → RoPE → KV write →
 * attention → Wo + residual → RMSNorm → SwiGLU FFN + residual, final norm,
 * LM head: 4 launches per layer + 1) and returns the logits as a host Float32Array (the same array
 * every call, like the reference's `this.logits`).  The first step with a
 * cache runs op by op; the second is recorded as a HIP graph that later
 * steps with that cache replay (token and position are read from device
 * memory); `opts.graph = false` issues every step op by op.  `cache` must be
 * this package's device KVCache.
 */
export class Transformer {
  constructor(config, opts = {}) {
    this.cfg = config instanceof Config ? config : new Config(config);
    this._graphOn = !(opts && opts.graph === false);
    const c = this.cfg;
    if (c.dim % c.nHeads !== 0) throw new Error(`Transformer: dim ${c.dim} must be a multiple of nHeads ${c.nHeads}`);
    this.logits = new Float32Array(c.vocabSize);
    this._w = null; this._model = null; this._graphs = [];
  }

  loadWeights(w) {
    const c = this.cfg, a = hip();
    this.release();
    const D = c.dim, H = c.hidden, V = c.vocabSize;
    const bufs = [];
    const up = (arr) => { const h = a.alloc(Math.max(1, arr.byteLength)); a.h2d(h, arr); bufs.push(h); return h; };
    const mat = (x, N, K, what) => { const m = matWeights(x, N, K, what); return { type: m.type, h: up(m.data) }; };
    const tok = mat(w.tok_emb, V, D, "tok_emb");
    const wcls = w.wcls ? mat(w.wcls, V, D, "wcls") : tok;
    const layers = [];
    for (let l = 0; l < c.nLayers; l++) {
      const L = w[`layer.${l}`];
      if (!L) throw new Error(`Transformer.loadWeights: layer.${l} missing`);
      const qkv = mat(L.wqkv, c.qkvOut, D, `layer.${l}.wqkv`), wo = mat(L.wo, D, D, `layer.${l}.wo`);
      const g = mat(L.ffn_gate, H, D, `layer.${l}.ffn_gate`), u = mat(L.ffn_up, H, D, `layer.${l}.ffn_up`);
      const dn = mat(L.ffn_down, D, H, `layer.${l}.ffn_down`);
      if (g.type !== u.type)
        throw new Error(`Transformer.loadWeights: layer.${l} ffn_gate (type ${g.type}) and ffn_up (type ${u.type}) must share a type on the device`);
      layers.push({
        ln1: up(f32Weights(L.ln1, D, `layer.${l}.ln1`)), ln2: up(f32Weights(L.ln2, D, `layer.${l}.ln2`)),
        wqkv: qkv.h, wo: wo.h, gate: g.h, up: u.h, down: dn.h,
        wqkv_type: qkv.type, wo_type: wo.type, gate_type: g.type, up_type: u.type, down_type: dn.type,
      });
    }
    const rt = ropeTableF32(c.maxSeq, c.dHead, c.ropeTheta);
    const scratch = (n) => { const h = a.alloc(Math.max(1, n) * 4); bufs.push(h); return h; };
    this._w = {
      bufs, tok: tok.h, wcls: wcls.h, emb_type: tok.type, cls_type: wcls.type, layers,
      ln_f: up(f32Weights(w.ln_f, D, "ln_f")), rope_cos: up(rt.cos), rope_sin: up(rt.sin),
      x: scratch(D), q: scratch(c.nHeads * c.dHead), h: scratch(H), logits: scratch(V),
      state: a.alloc(8), stateHost: new Int32Array(2), part: null, partSeq: 0,
    };
    bufs.push(this._w.state);
    return this;
  }

  _modelFor(cache) {
    const c = this.cfg, W = this._w, a = hip();
    if (W.partSeq < cache.maxSeq || this._model === null || this._modelSeq !== cache.maxSeq) {
      this._dropGraphs();
      if (W.partSeq < cache.maxSeq) {
        if (W.part) a.free(W.part);
        W.part = a.alloc(a.decodePartLen(c.nHeads, c.dHead, cache.maxSeq) * 8);
        W.partSeq = cache.maxSeq;
      }
      this._model = a.decodeModel({
        dim: c.dim, hidden: c.hidden, nLayers: c.nLayers, nHeads: c.nHeads, nKvHeads: c.nKvHeads,
        vocab: c.vocabSize, maxSeq: cache.maxSeq, normEps: c.normEps, tok_emb: W.tok, ln_f: W.ln_f, wcls: W.wcls,
        emb_type: W.emb_type, cls_type: W.cls_type,
        rope_cos: W.rope_cos, rope_sin: W.rope_sin, x: W.x, q: W.q, h: W.h, attn_part: W.part,
        layers: W.layers,
      });
      this._modelSeq = cache.maxSeq;
    }
    return this._model;
  }

  /** One decode step: logits of `token` at position `pos`, K/V appended to `cache`. */
  forward(token, pos, cache) {
    this._step(token, pos, cache);
    hip().d2h(this._w.logits, this.logits);
    return this.logits;
  }

  /** Queues one decode step (logits stay in device memory, `_w.logits`). */
  _step(token, pos, cache) {
    const c = this.cfg, W = this._w, a = hip();
    if (!W) throw new Error("Transformer.forward: call loadWeights first");
    if (!(cache instanceof KVCache)) throw new TypeError("Transformer.forward: cache must be a device KVCache");
    if (!cache.kd) throw new Error("Transformer.forward: the cache has been freed");
    if (cache.nLayers !== c.nLayers || cache.kvDim !== c.kvDim) throw new RangeError("Transformer.forward: cache shape does not match the Config");
    if (!Number.isInteger(pos) || pos < 0 || pos >= Math.min(cache.maxSeq, c.maxSeq))
      throw new RangeError(`Transformer.forward: position ${pos} outside [0, ${Math.min(cache.maxSeq, c.maxSeq)})`);
    const model = this._modelFor(cache);
    W.stateHost[0] = Number.isInteger(token) && token >= 0 && token < c.vocabSize ? token : -1;
    W.stateHost[1] = pos;
    a.h2d(W.state, W.stateHost);
    let g = this._graphOn ? this._graphs.find((e) => e.cache === cache) : null;
    if (!this._graphOn) {
      a.decodeStep(model, cache.kd, cache.vd, W.state, W.logits);
    } else if (g && g.graph) {
      a.graphLaunch(g.graph);
    } else if (g) {
      a.graphBegin();
      try {
        a.decodeStep(model, cache.kd, cache.vd, W.state, W.logits);
        g.graph = a.graphEnd();
      } catch (e) {
        a.graphAbort();
        throw e;
      }
      a.graphLaunch(g.graph);
    } else {
      a.decodeStep(model, cache.kd, cache.vd, W.state, W.logits);
      this._graphs.push({ cache, graph: null });
      if (this._graphs.length > GRAPHS_KEPT) {
        const old = this._graphs.shift();
        if (old.graph) a.graphDestroy(old.graph);
      }
    }
    if (pos + 1 > cache.len) cache.len = pos + 1;
  }

  _dropGraphs() {
    const a = hip();
    for (const e of this._graphs) if (e.graph) a.graphDestroy(e.graph);
    this._graphs = [];
  }

  /** Frees the device weights, scratch and recorded graphs. */
  release() {
    if (!this._w) return;
    const a = hip();
    this._dropGraphs();
    for (const h of this._w.bufs) a.free(h);
    if (this._w.part) a.free(this._w.part);
    this._w = null; this._model = null;
  }
}
