/**
 * L6b · trainable transformer on MI355X.
 *
 * Same API and topology as forge-llm's src/L6/train.js: `initWeights`
 * (:33-57, GPT-2 style N(0, 0.02) with the 1/√(2L) residual scaling and the
 * same RNG draw order), `toParams` (:60-78, paramList order), the
 * `TrainableTransformer` class (:83-227) whose `_forward` chains
 * embedLookup → [rmsNorm → matmulT(wqkv) → sliceCols×3 → ropeRows×2 →
 * causalAttn(Batch) → matmulT(wo) → add → rmsNorm → matmulT(gate, up) →
 * swigluRows → matmulT(down) → add] × L → rmsNorm → matmulT(LM head), and the
 * `train()` loop (:246-276).  Three fusions keep the values and gradients of
 * that chain: the slices + RoPEs run as one qkvRope pass, each residual add is
 * the epilogue of the GEMM before it (matmulTResid), and the gate and up
 * projections are one GEMM over the packed [gate; up] weights followed by one
 * SwiGLU pass (swigluGateUp).  Every op runs on the device (src/L2/tensor.js);
 * parameters, gradients and Adam moments stay resident in HBM across steps.
 *
 * train() runs device-resident (DeviceTrainLoop): the token data is uploaded
 * once, each step's B windows are cut on the device at starts drawn on the
 * host with the reference's RNG (the same draws, so the same batches), and
 * from the second step on the whole step — gather, forward, loss, backward,
 * Adam — is replayed as one recorded HIP graph.  Per step the host uploads
 * B starts and {lr, bc1, bc2} (one small copy) and launches the graph; it
 * reads the loss and gnorm back only on logged steps.
 */
import { Config } from "./transformer.js";
import { RNG } from "../L0/numeric.js";
import { hip, graphState } from "../L2/device.js";
import { param, resetTape, backward, Adam } from "../L2/autograd.js";
import {
  matmulT, matmulTResid, embedLookup, rmsNorm, qkvRope, qkvRopeAttention, causalAttn, causalAttnBatch,
  crossEntropyMeanFused,
  swigluGateUp, packPair, crossEntropyMean, DeviceIds,
} from "../L2/tensor.js";

/** GPT-2 style init: N(0, 0.02); wo and ffn_down additionally × 1/√(2·nLayers). */
export function initWeights(cfg, seed = 1337) {
  const rng = new RNG(seed);
  const std = 0.02;
  const resScale = 1 / Math.sqrt(2 * cfg.nLayers);
  const norm = (n) => { const a = new Float32Array(n); for (let i = 0; i < n; i++) a[i] = rng.normal() * std; return a; };
  const ones = (n) => new Float32Array(n).fill(1);
  const scaled = (n) => { const a = norm(n); for (let i = 0; i < n; i++) a[i] *= resScale; return a; };
  const w = { tok_emb: norm(cfg.vocabSize * cfg.dim), ln_f: ones(cfg.dim), wcls: null };
  for (let l = 0; l < cfg.nLayers; l++) {
    const ln1 = ones(cfg.dim), ln2 = ones(cfg.dim);
    const wqkv = norm(cfg.qkvOut * cfg.dim);
    const wo = scaled(cfg.dim * cfg.dim);
    const ffn_gate = norm(cfg.hidden * cfg.dim);
    const ffn_up = norm(cfg.hidden * cfg.dim);
    const ffn_down = scaled(cfg.dim * cfg.hidden);
    w[`layer.${l}`] = { ln1, ln2, wqkv, wo, ffn_gate, ffn_up, ffn_down };
  }
  return w;
}

/** f32 weights object → parameter Nodes in paramList order. */
export function toParams(w, cfg) {
  const P = [];
  const mk = (arr) => { const p = param(arr); P.push(p); return p; };
  const ps = { tok_emb: mk(w.tok_emb), ln_f: mk(w.ln_f), wcls: w.wcls ? mk(w.wcls) : null, layers: [] };
  for (let l = 0; l < cfg.nLayers; l++) {
    const L = w[`layer.${l}`];
    ps.layers.push({
      ln1: mk(L.ln1), ln2: mk(L.ln2),
      wqkv: mk(L.wqkv), wo: mk(L.wo),
      ffn_gate: mk(L.ffn_gate), ffn_up: mk(L.ffn_up), ffn_down: mk(L.ffn_down),
    });
  }
  return { ps, all: P };
}

export class TrainableTransformer {
  constructor(config, weights = null, seed = 1337) {
    this.cfg = config instanceof Config ? config : new Config(config);
    const c = this.cfg;
    const w = weights === null || weights === undefined ? initWeights(c, seed) : weights;
    const { ps, all } = toParams(w, c);
    this.params = ps;
    this.paramList = all;
    this.w = w;
    this._build();
  }

  _build() {
    const ps = this.params;
    this.wclsNode = ps.wcls ? ps.wcls : ps.tok_emb;  // tied LM head when wcls is null
    this._packed = false;
    // Weights whose only gradient is their matmul's: their dW GEMMs are
    // deferred to the end of backward() and run as one grouped launch.
    for (const L of ps.layers) for (const p of [L.wqkv, L.wo, L.ffn_gate, L.ffn_up, L.ffn_down]) p._deferGrad = true;
    if (ps.wcls) ps.wcls._deferGrad = true;
  }

  /** ids[T] → logits[T, V] */
  forward(ids, pos0 = 0) {
    return this._forward(ids, 1, ids.length, pos0);
  }

  /** ids[B][T] → logits[B, T, V] with a block-diagonal causal mask. */
  forwardBatch(batchIds) {
    const B = batchIds.length, T = batchIds[0].length;
    const flat = [];
    for (const row of batchIds) for (const id of row) flat.push(id);
    return this._forward(flat, B, T, 0);
  }

  _forward(flatIds, B, T, pos0) {
    const c = this.cfg, ps = this.params;
    const BT = B * T, qD = c.nHeads * c.dHead, kvD = c.nKvHeads * c.dHead;
    if (!this._packed) {  // ffn_gate and ffn_up of a layer back to back on the device (one GEMM for both)
      for (const L of ps.layers) packPair(L.ffn_gate, L.ffn_up);
      this._packed = true;
    }
    let x = embedLookup(ps.tok_emb, flatIds, c.vocabSize, c.dim);
    for (let l = 0; l < c.nLayers; l++) {
      const L = ps.layers[l];
      const xn = rmsNorm(x, L.ln1, BT, c.dim, c.normEps);
      // matmulT(xn, wqkv), the q/k RoPE and the attention as one node (the
      // RoPE in the GEMM epilogue and in attention's gradient stores), or for
      // head sizes without the MFMA attention: matmulT, then sliceCols×3 +
      // ropeRows×2 in one pass over qkv, then the attention (same values and
      // gradients either way)
      let att = qkvRopeAttention(xn, L.wqkv, B, T, c.nHeads, c.nKvHeads, c.dHead, c.dim, pos0, c.ropeTheta, T);
      if (!att) {
        const qkv = matmulT(xn, L.wqkv, BT, c.dim, c.qkvOut);
        const [qr, kr, v] = qkvRope(qkv, BT, c.nHeads, c.nKvHeads, c.dHead, pos0, c.ropeTheta, T);
        att = B === 1
          ? causalAttn(qr, kr, v, T, c.nHeads, c.nKvHeads, c.dHead)
          : causalAttnBatch(qr, kr, v, B, T, c.nHeads, c.nKvHeads, c.dHead);
      }
      x = matmulTResid(x, att, L.wo, BT, qD, c.dim);  // x + att·woᵀ, residual in the GEMM epilogue
      const xn2 = rmsNorm(x, L.ln2, BT, c.dim, c.normEps);
      // matmulT(gate), matmulT(up), swigluRows as one [gate; up] GEMM + one SwiGLU pass
      const act = swigluGateUp(xn2, L.ffn_gate, L.ffn_up, BT, c.dim, c.hidden);
      x = matmulTResid(x, act, L.ffn_down, BT, c.hidden, c.dim);
    }
    const xf = rmsNorm(x, ps.ln_f, BT, c.dim, c.normEps);
    return matmulT(xf, this.wclsNode, BT, c.dim, c.vocabSize);
  }

  /** Next-token loss of one sequence: inputs ids[0..T), targets[T]. */
  loss(ids, targets) {
    const T = targets.length;
    const logits = this.forward(ids.slice(0, T));
    return crossEntropyMean(logits, targets, T, this.cfg.vocabSize);
  }

  /** Batched next-token loss: rows of T+1 ids, samples isolated by the mask. */
  lossBatch(batchIds) {
    const B = batchIds.length, T = batchIds[0].length - 1;
    const flatIds = [], flatTgt = [];
    for (const row of batchIds) {
      for (let i = 0; i < T; i++) { flatIds.push(row[i]); flatTgt.push(row[i + 1]); }
    }
    const logits = this._forward(flatIds, B, T, 0);
    return crossEntropyMean(logits, flatTgt, B * T, this.cfg.vocabSize);
  }

  /** lossBatch over ids already in device memory (DeviceIds of B·T inputs
   *  and B·T targets, as cut by fg_batch_gather). */
  _lossBatchIds(ids, targets, B, T) {
    const logits = this._forward(ids, B, T, 0);
    // the device loop always runs backward next: the CE gradient is formed in
    // the forward's pass over the logits (same values as crossEntropyMean)
    return crossEntropyMeanFused(logits, targets, B * T, this.cfg.vocabSize);
  }

  /** Backpropagates and returns the loss value. */
  backward(lossNode) {
    backward(lossNode);
    return lossNode.data[0];
  }

  zeroGrad() {
    for (const p of this.paramList) p.zeroGrad();
  }

  /** Weights as host f32 arrays (downloaded from the device). */
  exportWeights() {
    const c = this.cfg;
    const out = {
      tok_emb: Float32Array.from(this.params.tok_emb.data),
      ln_f: Float32Array.from(this.params.ln_f.data),
      wcls: this.params.wcls ? Float32Array.from(this.params.wcls.data) : null,
    };
    for (let l = 0; l < c.nLayers; l++) {
      const L = this.params.layers[l];
      out[`layer.${l}`] = {
        ln1: Float32Array.from(L.ln1.data),
        ln2: Float32Array.from(L.ln2.data),
        wqkv: Float32Array.from(L.wqkv.data),
        wo: Float32Array.from(L.wo.data),
        ffn_gate: Float32Array.from(L.ffn_gate.data),
        ffn_up: Float32Array.from(L.ffn_up.data),
        ffn_down: Float32Array.from(L.ffn_down.data),
      };
    }
    return out;
  }

  countParams() {
    let n = 0;
    for (const p of this.paramList) n += p.n;
    return n;
  }
}

/**
 * The device-resident form of train()'s loop body (train.js:255-266).
 *
 * The token data lives in device memory; step(starts) uploads the B window
 * starts together with Adam's {lr, bc1, bc2} in one small copy, and queues
 * gather → zeroGrad → lossBatch → backward → Adam.  The first step runs op by
 * op (it also warms the allocator and uploads every one-time table); with
 * `graph` the second step is recorded into a HIP graph as it is queued, and
 * later steps replay it.  Every step runs the same kernels on the same
 * inputs as the op-by-op path, so losses and parameters are bit-identical.
 */
export class DeviceTrainLoop {
  constructor(model, opt, data, B, T, opts = {}) {
    const o = opts || {};
    const a = hip();
    const n = data.length;
    if (!(n >= 1)) throw new RangeError("train: data holds no tokens");
    const V = model.cfg.vocabSize;
    const last = data[n - 1];
    const d = new Int32Array(n);
    for (let i = 0; i < n; i++) {
      let v = data[i];
      if (v === undefined || v === null) v = last;  // `data[s+i] ?? data[len-1]`
      d[i] = Number.isInteger(v) && v >= 0 && v < V ? v : -1;
    }
    this.model = model; this.opt = opt; this.B = B; this.T = T; this.V = V; this.n = n;
    this.graphOn = o.graph === undefined || o.graph === null ? true : !!o.graph;
    this.data = a.alloc(n * 4);
    a.h2d(this.data, d);
    // step inputs: {lr, bc1, bc2} as 3 doubles, then B int32 window starts
    this.host = new ArrayBuffer(32 + 4 * B);
    this.sched64 = new Float64Array(this.host, 0, 3);
    this.starts32 = new Int32Array(this.host, 32, B);
    this.u8 = new Uint8Array(this.host);
    this.inputs = a.alloc(32 + 4 * B);
    this.sched = a.view(this.inputs, 0, 24);
    this.starts = a.view(this.inputs, 32, 4 * B);
    this.ids = new DeviceIds(a.alloc(B * T * 4), B * T);
    this.tgt = new DeviceIds(a.alloc(B * T * 4), B * T);
    this.graph = null; this.loss = null; this.steps = 0; this.lr = 0;
  }

  _body() {
    hip().batchGather(this.ids.h, this.tgt.h, this.data, this.n, this.starts, this.B, this.T, this.V);
    this.model.zeroGrad();
    const L = this.model._lossBatchIds(this.ids, this.tgt, this.B, this.T);
    backward(L);
    this.opt._stepSched(this.sched);
    return L;
  }

  /** Queues one training step over the windows at `starts` (B ints in [0, n)). */
  step(starts) {
    const a = hip();
    for (let b = 0; b < this.B; b++) {
      const s = starts[b];
      if (!Number.isInteger(s) || s < 0 || s >= this.n) throw new RangeError(`train: window start ${s} outside [0, ${this.n})`);
      this.starts32[b] = s;
    }
    const sc = this.opt._advance();
    this.sched64[0] = sc.lr; this.sched64[1] = sc.bc1; this.sched64[2] = sc.bc2;
    this.lr = sc.lr;
    a.h2d(this.inputs, this.u8);
    if (!this.graphOn || this.steps === 0) {
      resetTape();
      this.loss = this._body();
    } else if (this.graph === null) {
      resetTape();
      graphState.capturing = true;
      try {
        a.graphBegin();
        try {
          this.loss = this._body();
          this.graph = a.graphEnd();
        } catch (e) {
          a.graphAbort();
          throw e;
        }
      } finally {
        graphState.capturing = false;
      }
      a.graphLaunch(this.graph);
    } else {
      a.graphLaunch(this.graph);
    }
    this.steps++;
  }

  /** {loss, lr, gnorm, scale} of the latest step (waits for that step only). */
  read() {
    const a = hip();
    const lt = a.readAsync(this.loss._dev, 4), st = a.readAsync(this.opt._stats, 16);
    const lv = new Float32Array(1), sv = new Float64Array(2);
    a.readWait(lt, lv);
    a.readWait(st, sv);
    return { loss: lv[0], lr: this.lr, gnorm: sv[0], scale: sv[1] };
  }

  /** Destroys the graph (after the queued replays finish) and frees the buffers. */
  close() {
    const a = hip();
    if (this.graph !== null) { a.graphDestroy(this.graph); this.graph = null; }
    resetTape();
    this.ids.free(); this.tgt.free();
    if (this.inputs) { a.free(this.inputs); this.inputs = null; }
    if (this.data) { a.free(this.data); this.data = null; }
  }
}

/**
 * Training loop (train.js:246-276): per step sample B windows of seqLen+1
 * ids (the reference's RNG draws), resetTape, zeroGrad, lossBatch, backward,
 * Adam step; logs and returns the history every logEvery steps.  The loop is
 * device-resident (DeviceTrainLoop) unless opts.deviceLoop is false, which
 * runs the op-by-op loop over host-built batches; opts.graph = false keeps
 * the device loop but issues every step op by op.
 */
export function train(model, data, opts = {}) {
  const o = opts || {};
  const pick = (k, d) => (o[k] === undefined || o[k] === null ? d : o[k]);
  const steps = pick("steps", 100);
  const B = pick("batchSize", 8);
  const seqLen = pick("seqLen", 32);
  const lr = pick("lr", 1e-2);
  const logEvery = pick("logEvery", 10);
  const rng = new RNG(pick("seed", 7));

  const opt = new Adam(model.paramList, { lr, totalSteps: steps, clip: 1.0, wd: 0.01 });
  const history = [];
  const log = (step, l, lrv, gnorm) => {
    history.push({ step, loss: l, lr: lrv, gnorm });
    console.log(`  step ${String(step).padStart(4)}  loss ${l.toFixed(4)}  lr ${lrv.toExponential(2)}  |g| ${gnorm.toFixed(3)}`);
  };
  const drawStart = () => rng.int(Math.max(1, data.length - seqLen - 1));

  if (!pick("deviceLoop", true)) {
    for (let step = 0; step < steps; step++) {
      const batch = [];
      for (let b = 0; b < B; b++) {
        const s = drawStart();
        const row = new Array(seqLen + 1);
        for (let i = 0; i <= seqLen; i++) {
          const v = data[s + i];
          row[i] = v === undefined || v === null ? data[data.length - 1] : v;
        }
        batch.push(row);
      }
      resetTape();
      model.zeroGrad();
      const lossNode = model.lossBatch(batch);
      const l = model.backward(lossNode);
      const info = opt.step();
      if (step % logEvery === 0 || step === steps - 1) log(step, l, info.lr, info.gnorm);
    }
    return history;
  }

  const loop = new DeviceTrainLoop(model, opt, data, B, seqLen, { graph: pick("graph", true) });
  try {
    const starts = new Array(B);
    for (let step = 0; step < steps; step++) {
      for (let b = 0; b < B; b++) starts[b] = drawStart();
      loop.step(starts);
      if (step % logEvery === 0 || step === steps - 1) {
        const r = loop.read();
        log(step, r.loss, r.lr, r.gnorm);
      }
    }
  } finally {
    loop.close();
  }
  return history;
}
