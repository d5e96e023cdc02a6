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

// ── the parameter table ─────────────────────────────────────────────────
/**
 * Every parameter tensor of the model, one row each, in paramList order
 * (train.js:60-78).  The table is the one description of the weights:
 * initWeights fills them in its order (which is the reference's RNG draw
 * order, since the `ones` rows draw nothing), toParams builds the paramList
 * from it, exportWeights downloads by it, and checkpoints name tensors by
 * its `gguf` column.
 *   key    name in the weights object (layer rows under `layer.<l>`)
 *   count  number of elements for a Config
 *   init   "ones" (norm weights), "normal" (N(0, 0.02)), "scaled" (N(0, 0.02),
 *          then × 1/√(2·nLayers): the residual projections) or "given" (the
 *          untied LM head, supplied by the caller; null means tied)
 *   gguf   its tensor name in a GGUF file
 */
const MODEL_ROWS = [
  { key: "tok_emb", count: (c) => c.vocabSize * c.dim, init: "normal", gguf: () => "token_embd.weight" },
  { key: "ln_f", count: (c) => c.dim, init: "ones", gguf: () => "output_norm.weight" },
  { key: "wcls", count: (c) => c.vocabSize * c.dim, init: "given", gguf: () => "output.weight" },
];
const LAYER_ROWS = [
  { key: "ln1", count: (c) => c.dim, init: "ones", gguf: (l) => `blk.${l}.attn_norm.weight` },
  { key: "ln2", count: (c) => c.dim, init: "ones", gguf: (l) => `blk.${l}.ffn_norm.weight` },
  { key: "wqkv", count: (c) => c.qkvOut * c.dim, init: "normal", gguf: (l) => `blk.${l}.attn_qkv.weight` },
  { key: "wo", count: (c) => c.dim * c.dim, init: "scaled", gguf: (l) => `blk.${l}.attn_output.weight` },
  { key: "ffn_gate", count: (c) => c.hidden * c.dim, init: "normal", gguf: (l) => `blk.${l}.ffn_gate.weight` },
  { key: "ffn_up", count: (c) => c.hidden * c.dim, init: "normal", gguf: (l) => `blk.${l}.ffn_up.weight` },
  { key: "ffn_down", count: (c) => c.dim * c.hidden, init: "scaled", gguf: (l) => `blk.${l}.ffn_down.weight` },
];
const INIT_STD = 0.02;

/** The parameter slots of a config in paramList order, {row, layer} with
 *  layer -1 for the model-level tensors; `tied` leaves out the LM head. */
export function parameterSlots(cfg, tied) {
  const slots = [];
  for (const row of MODEL_ROWS) if (!(tied && row.init === "given")) slots.push({ row, layer: -1 });
  for (let l = 0; l < cfg.nLayers; l++) for (const row of LAYER_ROWS) slots.push({ row, layer: l });
  return slots;
}
/** GGUF tensor name of a slot. */
export const slotName = (slot) => slot.row.gguf(slot.layer);

/** Reads / writes a slot's entry in a weights-shaped object (model-level
 *  entries at the top, layer entries under `layer.<l>`). */
function slotGet(w, slot) {
  return slot.layer < 0 ? w[slot.row.key] : w[`layer.${slot.layer}`][slot.row.key];
}
function slotSet(w, slot, v) {
  if (slot.layer < 0) { w[slot.row.key] = v; return; }
  const k = `layer.${slot.layer}`;
  if (!w[k]) w[k] = {};
  w[k][slot.row.key] = v;
}

/** A weights object (initWeights' shape, wcls null when tied) whose every
 *  tensor is fill(slot), in the table's order. */
export function weightsFromSlots(cfg, tied, fill) {
  const w = { tok_emb: null, ln_f: null, wcls: null };
  for (const slot of parameterSlots(cfg, tied)) slotSet(w, slot, fill(slot));
  return w;
}

/** Weights drawn by the table (train.js:33-57): N(0, 0.02) from one RNG in
 *  table order, the residual projections then scaled (a second fp32
 *  rounding, as the reference multiplies the stored values), norms = 1 and
 *  wcls null (tied). */
export function initWeights(cfg, seed = 1337) {
  const rng = new RNG(seed);
  const resScale = 1 / Math.sqrt(2 * cfg.nLayers);
  const w = {};
  for (const slot of parameterSlots(cfg, false)) {
    const n = slot.row.count(cfg);
    let a = null;
    if (slot.row.init === "ones") {
      a = new Float32Array(n).fill(1);
    } else if (slot.row.init !== "given") {
      a = new Float32Array(n);
      for (let i = 0; i < n; i++) a[i] = rng.normal() * INIT_STD;
      if (slot.row.init === "scaled") for (let i = 0; i < n; i++) a[i] *= resScale;
    }
    slotSet(w, slot, a);
  }
  return w;
}

/** Weights object → parameter Nodes: `ps` shaped like the weights (layers
 *  as an array) and `all`, the paramList (the table's order). */
export function toParams(w, cfg) {
  const ps = { tok_emb: null, ln_f: null, wcls: null, layers: [] };
  const all = [];
  for (const slot of parameterSlots(cfg, !w.wcls)) {
    const node = param(slotGet(w, slot));
    all.push(node);
    if (slot.layer < 0) ps[slot.row.key] = node;
    else (ps.layers[slot.layer] = ps.layers[slot.layer] || {})[slot.row.key] = node;
  }
  return { ps, all };
}

/** Rows of T+1 ids → the flat next-token pairs of a batch (train.js:177-185):
 *  inputs row[0..T), targets row[1..T], rows back to back. */
function nextTokenPairs(rows) {
  const T = rows[0].length - 1, inputs = new Array(rows.length * T), targets = new Array(rows.length * T);
  rows.forEach((row, b) => {
    for (let i = 0; i < T; i++) { inputs[b * T + i] = row[i]; targets[b * T + i] = row[i + 1]; }
  });
  return { inputs, targets, T };
}

function flatten(rows) {
  const out = [];
  for (const row of rows) for (let i = 0; i < row.length; i++) out.push(row[i]);
  return out;
}

export class TrainableTransformer {
  constructor(config, weights = null, seed = 1337) {
    this.cfg = config instanceof Config ? config : new Config(config);
    this.w = weights === null || weights === undefined ? initWeights(this.cfg, seed) : weights;
    const { ps, all } = toParams(this.w, this.cfg);
    this.params = ps;
    this.paramList = all;
    this._build();
  }

  _build() {
    const ps = this.params;
    this.wclsNode = ps.wcls ? ps.wcls : ps.tok_emb;  // tied LM head when wcls is null
    this._packed = false;
    // Weights whose only gradient is one op's: the dW GEMMs of the matmul
    // weights and the column sums of the norm weights are deferred to the
    // end of backward() and run as one grouped launch each.
    for (const L of ps.layers) {
      for (const p of [L.wqkv, L.wo, L.ffn_gate, L.ffn_up, L.ffn_down, L.ln1, L.ln2]) p._deferGrad = true;
    }
    if (ps.wcls) ps.wcls._deferGrad = true;
    ps.ln_f._deferGrad = true;
  }

  /** One sequence: ids[T] → logits[T, V], positions from pos0. */
  forward(ids, pos0 = 0) { return this._forward(ids, 1, ids.length, pos0); }

  /** B sequences of equal length, each seeing only itself (block-diagonal
   *  causal mask): ids[B][T] → logits[B·T, V]. */
  forwardBatch(batchIds) { return this._forward(flatten(batchIds), batchIds.length, batchIds[0].length, 0); }

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

  /** Next-token loss of one sequence (train.js:164-171): the logits of
   *  ids[0..T) against targets[0..T), T = targets.length. */
  loss(ids, targets) {
    const T = targets.length;
    return crossEntropyMean(this.forward(ids.slice(0, T)), targets, T, this.cfg.vocabSize);
  }

  /** Mean next-token loss over B rows of T+1 ids (train.js:177-185). */
  lossBatch(batchIds) {
    const { inputs, targets, T } = nextTokenPairs(batchIds);
    const B = batchIds.length;
    return crossEntropyMean(this._forward(inputs, B, T, 0), targets, B * T, this.cfg.vocabSize);
  }

  /** lossBatch over ids already in device memory (DeviceIds of B·T inputs
   *  and B·T targets, as cut by fg_batch_gather). */
  _lossBatchIds(ids, targets, B, T) {
    const logits = this._forward(ids, B, T, 0);
    // the device loop always runs backward next: the CE gradient is formed in
    // the forward's pass over the logits (same values as crossEntropyMean)
    return crossEntropyMeanFused(logits, targets, B * T, this.cfg.vocabSize);
  }

  /** backward() from the loss, then its value (train.js:188-191). */
  backward(lossNode) {
    backward(lossNode);
    return lossNode.data[0];
  }

  zeroGrad() { this.paramList.forEach((p) => p.zeroGrad()); }

  /** The weights as host f32 arrays, shaped as initWeights returns them
   *  (wcls null when tied), downloaded without marking the parameters as
   *  edited on the host. */
  exportWeights() {
    const out = {};
    for (const slot of parameterSlots(this.cfg, false)) {
      const node = slot.layer < 0 ? this.params[slot.row.key] : this.params.layers[slot.layer][slot.row.key];
      slotSet(out, slot, node ? node._download() : null);
    }
    return out;
  }

  countParams() { return this.paramList.reduce((n, p) => n + p.n, 0); }
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
    // the latest step's loss, copied out of the tape: read() still finds it
    // after other code has reset the tape (another loop stepping in turn)
    this.lossBuf = a.alloc(4);
    this.graph = null; this.loss = null; this.steps = 0; this.lr = 0;
  }

  _body() {
    const a = hip();
    a.batchGather(this.ids.h, this.tgt.h, this.data, this.n, this.starts, this.B, this.T, this.V);
    this.model.zeroGrad();
    const L = this.model._lossBatchIds(this.ids, this.tgt, this.B, this.T);
    backward(L);
    this.opt._stepSched(this.sched);
    a.accum(this.lossBuf, L._dev, 1, 0);  // a copy kernel (a recorded graph holds it)
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
    const lt = a.readAsync(this.lossBuf, 4), st = a.readAsync(this.opt._stats, 16);
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
    if (this.lossBuf) { a.free(this.lossBuf); this.lossBuf = null; }
    if (this.inputs) { a.free(this.inputs); this.inputs = null; }
    if (this.data) { a.free(this.data); this.data = null; }
  }
}

/**
 * train()'s batch sampling (train.js:255-260): each of a step's B windows
 * starts at rng.int(max(1, len − seqLen − 1)) and holds seqLen + 1 ids, with
 * the last token standing in past the end (`data[s+i] ?? data[len−1]`).
 */
class WindowSampler {
  constructor(data, seqLen, seed) {
    this.data = data;
    this.seqLen = seqLen;
    this.rng = new RNG(seed);
    this.span = Math.max(1, data.length - seqLen - 1);
  }
  /** The next B window starts (B draws of the RNG). */
  starts(B) {
    const s = new Array(B);
    for (let b = 0; b < B; b++) s[b] = this.rng.int(this.span);
    return s;
  }
  /** The windows at `starts` as rows of seqLen + 1 ids. */
  rows(starts) {
    const d = this.data, fill = d[d.length - 1];
    return starts.map((s) => {
      const row = new Array(this.seqLen + 1);
      for (let i = 0; i <= this.seqLen; i++) {
        const v = d[s + i];
        row[i] = v === undefined || v === null ? fill : v;
      }
      return row;
    });
  }
}

const TRAIN_DEFAULTS = { steps: 100, batchSize: 8, seqLen: 32, lr: 1e-2, logEvery: 10, seed: 7, deviceLoop: true, graph: true };

/**
 * Training loop (train.js:246-276): each step samples B windows, then
 * resetTape → zeroGrad → lossBatch → backward → Adam (lr, cosine over
 * `steps`, clip 1, weight decay 0.01); every logEvery-th step and the last
 * are logged and returned as {step, loss, lr, gnorm}.  The steps run in the
 * device-resident DeviceTrainLoop (recorded as a HIP graph unless
 * opts.graph is false); opts.deviceLoop = false runs them op by op over
 * host-built batches instead.  Every path draws the same windows.
 */
export function train(model, data, opts = {}) {
  const o = Object.assign({}, TRAIN_DEFAULTS);
  for (const [k, v] of Object.entries(opts || {})) if (v !== undefined && v !== null) o[k] = v;
  const opt = new Adam(model.paramList, { lr: o.lr, totalSteps: o.steps, clip: 1.0, wd: 0.01 });
  const sampler = new WindowSampler(data, o.seqLen, o.seed);
  const history = [];
  const logged = (step) => step % o.logEvery === 0 || step === o.steps - 1;
  const log = (step, loss, lr, gnorm) => {
    history.push({ step, loss, lr, gnorm });
    console.log(`  step ${String(step).padStart(4)}  loss ${loss.toFixed(4)}  lr ${lr.toExponential(2)}  |g| ${gnorm.toFixed(3)}`);
  };

  if (!o.deviceLoop) {
    for (let step = 0; step < o.steps; step++) {
      const rows = sampler.rows(sampler.starts(o.batchSize));
      resetTape();
      model.zeroGrad();
      const loss = model.backward(model.lossBatch(rows));
      const info = opt.step();
      if (logged(step)) log(step, loss, info.lr, info.gnorm);
    }
    return history;
  }

  const loop = new DeviceTrainLoop(model, opt, data, o.batchSize, o.seqLen, { graph: o.graph });
  try {
    for (let step = 0; step < o.steps; step++) {
      loop.step(sampler.starts(o.batchSize));
      if (logged(step)) {
        const r = loop.read();
        log(step, r.loss, r.lr, r.gnorm);
      }
    }
  } finally {
    loop.close();
  }
  return history;
}
