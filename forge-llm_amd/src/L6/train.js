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
 */
import { Config } from "./transformer.js";
import { RNG } from "../L0/numeric.js";
import { param, resetTape, backward, Adam } from "../L2/autograd.js";
import {
  matmulT, matmulTResid, embedLookup, rmsNorm, qkvRope, causalAttn, causalAttnBatch,
  swigluGateUp, packPair, crossEntropyMean,
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
      const qkv = matmulT(xn, L.wqkv, BT, c.dim, c.qkvOut);
      // sliceCols×3 + ropeRows×2 in one pass over qkv (same values and gradients)
      const [qr, kr, v] = qkvRope(qkv, BT, c.nHeads, c.nKvHeads, c.dHead, pos0, c.ropeTheta, T);
      const att = B === 1
        ? causalAttn(qr, kr, v, T, c.nHeads, c.nKvHeads, c.dHead)
        : causalAttnBatch(qr, kr, v, B, T, c.nHeads, c.nKvHeads, c.dHead);
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
 * Training loop (train.js:246-276): per step sample B windows of seqLen+1
 * ids, resetTape, zeroGrad, lossBatch, backward, Adam step; logs and returns
 * the history every logEvery steps.
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
  for (let step = 0; step < steps; step++) {
    const batch = [];
    for (let b = 0; b < B; b++) {
      const s = rng.int(Math.max(1, data.length - seqLen - 1));
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
    if (step % logEvery === 0 || step === steps - 1) {
      history.push({ step, loss: l, lr: info.lr, gnorm: info.gnorm });
      console.log(`  step ${String(step).padStart(4)}  loss ${l.toFixed(4)}  lr ${info.lr.toExponential(2)}  |g| ${info.gnorm.toFixed(3)}`);
    }
  }
  return history;
}
