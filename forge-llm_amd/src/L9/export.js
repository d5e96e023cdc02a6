/**
 * L9 · trained-weight export and training checkpoints.
 *
 * exportGGUF (engine.js:126-228): f32 weights (a TrainableTransformer's
 * exportWeights(), downloaded from the device) → a llama-architecture GGUF v3
 * file with the reference's metadata keys, key order, tensor names and
 * dimension order, so the bytes equal the reference's for the same weights.
 * The fused wqkv is written as the three attn_q / attn_k / attn_v tensors.
 * Quantized exports run the reference's quantizers on the device.
 *
 * loadGGUF (engine.js:236-300): GGUF bytes → {config, transformer (the
 * device inference model, quantized matrices kept quantized), vocab (the
 * tokenizer metadata as arrays, or null), metadata}.
 *
 * saveCheckpoint / loadCheckpoint (no counterpart in the reference, which
 * exports weights only): the same GGUF with every parameter (fused wqkv kept
 * fused) plus Adam's moments m and v as `forge.adam.m.<name>` /
 * `forge.adam.v.<name>` tensors and Adam's step, schedule and
 * hyper-parameters as FLOAT64 / UINT32 metadata.  Loading restores the
 * parameters, m, v and t bit for bit, so training resumed from a checkpoint
 * continues exactly as if it had not stopped.
 */
import { Config, Transformer } from "../L6/transformer.js";
import { TrainableTransformer, parameterSlots, slotName, weightsFromSlots } from "../L6/train.js";
import { Adam } from "../L2/autograd.js";
import { writeGGUF, readGGUF, GGUFValueType, GGML_F32 } from "./gguf.js";
import { QuantLinear } from "../L4/nn.js";
import { info, rowBytes, quantizeRow } from "../L3/quant.js";

const NAMES = {
  emb: "token_embd.weight",
  lnF: "output_norm.weight",
  out: "output.weight",
  ln1: (l) => `blk.${l}.attn_norm.weight`,
  wq: (l) => `blk.${l}.attn_q.weight`,
  wk: (l) => `blk.${l}.attn_k.weight`,
  wv: (l) => `blk.${l}.attn_v.weight`,
  wqkv: (l) => `blk.${l}.attn_qkv.weight`,
  wo: (l) => `blk.${l}.attn_output.weight`,
  ln2: (l) => `blk.${l}.ffn_norm.weight`,
  fg: (l) => `blk.${l}.ffn_gate.weight`,
  fu: (l) => `blk.${l}.ffn_up.weight`,
  fd: (l) => `blk.${l}.ffn_down.weight`,
};

const f32 = (a) => (a instanceof Float32Array ? a : Float32Array.from(a));
const bytesOf = (a) => new Uint8Array(a.buffer, a.byteOffset, a.byteLength);
const mat = (name, a, N, K) => ({ name, dims: [K, N], type: GGML_F32, data: bytesOf(f32(a)) });
const vec = (name, a, n) => ({ name, dims: [n], type: GGML_F32, data: bytesOf(f32(a)) });

function llamaMeta(c, name, fileType) {
  const A = "llama";
  const m = new Map();
  m.set("general.architecture", A);
  m.set("general.name", name);
  m.set("general.quantization_version", 2);
  m.set("general.alignment", 32);
  m.set(`${A}.block_count`, c.nLayers);
  m.set(`${A}.embedding_length`, c.dim);
  m.set(`${A}.feed_forward_length`, c.hidden);
  m.set(`${A}.attention.head_count`, c.nHeads);
  m.set(`${A}.attention.head_count_kv`, c.nKvHeads);
  m.set(`${A}.context_length`, c.maxSeq);
  m.set(`${A}.attention.layer_norm_rms_epsilon`, c.normEps);
  m.set(`${A}.vocab_size`, c.vocabSize);
  m.set(`${A}.rope.freq_base`, c.ropeTheta);
  m.set("general.file_type", fileType);
  return m;
}

function vocabMeta(m, vocab) {
  if (!vocab) return;
  m.set("tokenizer.ggml.model", "llama");
  m.set("tokenizer.ggml.tokens", vocab.tokenBytes.map((b) => new TextDecoder().decode(b)));
  m.set("tokenizer.ggml.scores", vocab.scores.map((s) => s));
  m.set("tokenizer.ggml.token_type", vocab.types);
  m.set("tokenizer.ggml.bos_token_id", vocab.bos);
  m.set("tokenizer.ggml.eos_token_id", vocab.eos);
  m.set("tokenizer.ggml.add_bos_token", vocab.addBos);
  m.set("tokenizer.ggml.add_eos_token", vocab.addEos);
}

const QUANT_TYPES = new Set([0, 1, 8, 12, 13, 14]);

/**
 * Weights (exportWeights() layout) → GGUF v3 bytes (engine.js:126-228).
 * quantType 0 writes f32; 1, 8, 12, 13, 14 (F16, Q8_0, Q4_K, Q5_K, Q6_K)
 * quantize every matrix whose rows are whole blocks on the device, with the
 * reference's quantizers (so the bytes are the reference's), and keep the
 * others f32; the fused wqkv is quantized whole and cut into q / k / v rows.
 */
export function exportGGUF(weights, config, vocab = null, quantType = 0, name = "forge-model") {
  const c = config instanceof Config ? config : new Config(config);
  const qt = quantType === undefined || quantType === null ? 0 : quantType;
  if (!QUANT_TYPES.has(qt)) throw new Error(`exportGGUF: no quantizer for type ${qt} (0, 1, 8, 12, 13, 14 are supported)`);
  const meta = llamaMeta(c, name, qt);
  const D = c.dim, H = c.hidden, qD = c.nHeads * c.dHead, kvD = c.nKvHeads * c.dHead;
  const bs = info(qt).blockSize;
  const pushT = (list, nm, a, N, K) => {
    if (qt === 0 || K % bs !== 0) list.push(mat(nm, a, N, K));
    else list.push({ name: nm, dims: [K, N], type: qt, data: quantizeRow(qt, f32(a), N * K) });
  };
  const t = [];
  pushT(t, NAMES.emb, weights.tok_emb, c.vocabSize, D);
  t.push(vec(NAMES.lnF, weights.ln_f, D));
  for (let l = 0; l < c.nLayers; l++) {
    const L = weights[`layer.${l}`];
    const wqkv = f32(L.wqkv);
    t.push(vec(NAMES.ln1(l), L.ln1, D));
    if (qt === 0 || D % bs !== 0) {
      t.push(mat(NAMES.wq(l), wqkv.subarray(0, qD * D), qD, D));
      t.push(mat(NAMES.wk(l), wqkv.subarray(qD * D, (qD + kvD) * D), kvD, D));
      t.push(mat(NAMES.wv(l), wqkv.subarray((qD + kvD) * D, (qD + 2 * kvD) * D), kvD, D));
    } else {
      const bytes = quantizeRow(qt, wqkv, c.qkvOut * D), rb = rowBytes(qt, D);
      const rows = (nm, r0, n) => t.push({ name: nm, dims: [D, n], type: qt, data: bytes.subarray(r0 * rb, (r0 + n) * rb) });
      rows(NAMES.wq(l), 0, qD);
      rows(NAMES.wk(l), qD, kvD);
      rows(NAMES.wv(l), qD + kvD, kvD);
    }
    pushT(t, NAMES.wo(l), L.wo, D, D);
    t.push(vec(NAMES.ln2(l), L.ln2, D));
    pushT(t, NAMES.fg(l), L.ffn_gate, H, D);
    pushT(t, NAMES.fu(l), L.ffn_up, H, D);
    pushT(t, NAMES.fd(l), L.ffn_down, D, H);
  }
  if (weights.wcls) pushT(t, NAMES.out, weights.wcls, c.vocabSize, D);
  vocabMeta(meta, vocab);
  return writeGGUF({ meta, tensors: t }).bytes;
}

function configFrom(g) {
  const M = (k, d) => (g.meta.has(k) ? g.meta.get(k) : d);
  const A = M("general.architecture", "llama");
  const K = (s) => `${A}.${s}`;
  return new Config({
    dim: M(K("embedding_length")), hidden: M(K("feed_forward_length")), nLayers: M(K("block_count")),
    nHeads: M(K("attention.head_count")), nKvHeads: M(K("attention.head_count_kv"), M(K("attention.head_count"))),
    vocabSize: M(K("vocab_size")), maxSeq: M(K("context_length"), 512),
    normEps: M(K("attention.layer_norm_rms_epsilon"), 1e-5), ropeTheta: M(K("rope.freq_base"), 10000),
    bosId: M("tokenizer.ggml.bos_token_id", 1), eosId: M("tokenizer.ggml.eos_token_id", 2),
  });
}

function f32Tensor(g, name, n) {
  const t = g.getTensor(name);
  if (!t) throw new Error(`GGUF: tensor ${name} missing`);
  if (t.type !== GGML_F32) throw new Error(`GGUF: tensor ${name} has ggml type ${t.type}; only f32 tensors load here`);
  const n0 = t.dims.reduce((a, b) => a * b, 1);
  if (n0 !== n) throw new Error(`GGUF: tensor ${name} holds ${n0} values, ${n} expected`);
  return new Float32Array(t.data.slice().buffer);
}

/** exportWeights()-layout f32 weights from GGUF bytes (fused or split QKV). */
export function weightsFromGGUF(g, c) {
  const D = c.dim, H = c.hidden, qD = c.nHeads * c.dHead, kvD = c.nKvHeads * c.dHead;
  const w = {
    tok_emb: f32Tensor(g, NAMES.emb, c.vocabSize * D), ln_f: f32Tensor(g, NAMES.lnF, D),
    wcls: g.getTensor(NAMES.out) ? f32Tensor(g, NAMES.out, c.vocabSize * D) : null,
  };
  for (let l = 0; l < c.nLayers; l++) {
    let wqkv;
    if (g.getTensor(NAMES.wqkv(l))) wqkv = f32Tensor(g, NAMES.wqkv(l), c.qkvOut * D);
    else {
      wqkv = new Float32Array(c.qkvOut * D);
      wqkv.set(f32Tensor(g, NAMES.wq(l), qD * D), 0);
      wqkv.set(f32Tensor(g, NAMES.wk(l), kvD * D), qD * D);
      wqkv.set(f32Tensor(g, NAMES.wv(l), kvD * D), (qD + kvD) * D);
    }
    w[`layer.${l}`] = {
      ln1: f32Tensor(g, NAMES.ln1(l), D), ln2: f32Tensor(g, NAMES.ln2(l), D), wqkv,
      wo: f32Tensor(g, NAMES.wo(l), D * D), ffn_gate: f32Tensor(g, NAMES.fg(l), H * D),
      ffn_up: f32Tensor(g, NAMES.fu(l), H * D), ffn_down: f32Tensor(g, NAMES.fd(l), D * H),
    };
  }
  return w;
}

/** A matrix tensor as a QuantLinear [N, K] (GGUF dims [K, N]; engine.js:251-256, 313-321). */
function qlTensor(g, name, N, K) {
  const t = g.getTensor(name);
  if (!t) throw new Error(`GGUF: tensor ${name} missing`);
  const n0 = t.dims.reduce((a, b) => a * b, 1);
  if (n0 !== N * K) throw new Error(`GGUF: tensor ${name} holds ${n0} values, ${N * K} expected`);
  if (t.type === GGML_F32) return new QuantLinear(0, new Float32Array(t.data.slice().buffer), N, K);
  return new QuantLinear(t.type, t.data, N, K);
}

/** Fused wqkv: attn_qkv, or the q / k / v rows concatenated byte for byte
 *  (engine.js:260-268, 62-73: all three must share a type). */
function fusedQKV(g, c, l) {
  const D = c.dim;
  if (g.getTensor(NAMES.wqkv(l))) return qlTensor(g, NAMES.wqkv(l), c.qkvOut, D);
  const parts = [NAMES.wq(l), NAMES.wk(l), NAMES.wv(l)].map((nm) => {
    const t = g.getTensor(nm);
    if (!t) throw new Error(`GGUF: layer ${l} lacks attn_q/k/v`);
    return t;
  });
  const types = new Set(parts.map((p) => p.type));
  if (types.size !== 1) throw new Error(`GGUF: layer ${l} q/k/v quantization types differ: ${[...types]}`);
  const total = parts.reduce((a, p) => a + p.data.byteLength, 0);
  const out = new Uint8Array(total);
  let o = 0;
  for (const p of parts) { out.set(p.data, o); o += p.data.byteLength; }
  const type = parts[0].type;
  if (type === GGML_F32) return new QuantLinear(0, new Float32Array(out.buffer), c.qkvOut, D);
  return new QuantLinear(type, out, c.qkvOut, D);
}

/** GGUF bytes → {config, transformer, vocab, metadata} (engine.js:236-300):
 *  f32 and quantized (F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K) matrices load
 *  into the device decode model as they are; norm vectors are f32. */
export function loadGGUF(buf) {
  const g = readGGUF(buf);
  const c = configFrom(g);
  const D = c.dim, H = c.hidden;
  const w = {
    tok_emb: qlTensor(g, NAMES.emb, c.vocabSize, D), ln_f: f32Tensor(g, NAMES.lnF, D),
    wcls: g.getTensor(NAMES.out) ? qlTensor(g, NAMES.out, c.vocabSize, D) : null,
  };
  for (let l = 0; l < c.nLayers; l++) {
    w[`layer.${l}`] = {
      ln1: f32Tensor(g, NAMES.ln1(l), D), ln2: f32Tensor(g, NAMES.ln2(l), D), wqkv: fusedQKV(g, c, l),
      wo: qlTensor(g, NAMES.wo(l), D, D), ffn_gate: qlTensor(g, NAMES.fg(l), H, D),
      ffn_up: qlTensor(g, NAMES.fu(l), H, D), ffn_down: qlTensor(g, NAMES.fd(l), D, H),
    };
  }
  const transformer = new Transformer(c).loadWeights(w);
  const vocab = g.meta.has("tokenizer.ggml.tokens") ? {
    tokens: g.meta.get("tokenizer.ggml.tokens"),
    types: g.meta.get("tokenizer.ggml.token_type") || null,
    scores: g.meta.get("tokenizer.ggml.scores") || null,
    bos: g.meta.get("tokenizer.ggml.bos_token_id"), eos: g.meta.get("tokenizer.ggml.eos_token_id"),
  } : null;
  return { config: c, transformer, vocab, metadata: g.meta };
}

// ── checkpoints ────────────────────────────────────────────────────────────
/** GGUF name of each entry of a TrainableTransformer's paramList (the
 *  model's parameter table, train.js:60-78 order). */
function paramNames(model) {
  const out = parameterSlots(model.cfg, !model.params.wcls).map(slotName);
  if (out.length !== model.paramList.length) throw new Error("checkpoint: unexpected parameter list");
  return out;
}

const F64 = (v) => ({ ggufType: GGUFValueType.FLOAT64, value: v });
const ADAM_KEYS = ["lr", "b1", "b2", "eps", "wd", "clip"];

/**
 * model (TrainableTransformer) + opt (its Adam) → GGUF bytes holding the
 * parameters, Adam's m and v and its state.  Downloads from the device; the
 * training state itself is not changed.
 */
export function saveCheckpoint(model, opt, name = "forge-checkpoint") {
  const c = model.cfg;
  if (!(opt instanceof Adam) || opt.p.length !== model.paramList.length) throw new Error("saveCheckpoint: opt must be the model's Adam");
  const meta = llamaMeta(c, name, 0);
  meta.set("forge.checkpoint.version", 1);
  meta.set("forge.checkpoint.tied", !model.params.wcls);
  // the llama keys hold eps as FLOAT32; the checkpoint keeps the exact values
  meta.set("forge.config.norm_eps", F64(c.normEps));
  meta.set("forge.config.rope_theta", F64(c.ropeTheta));
  meta.set("forge.adam.t", opt.t);
  meta.set("forge.adam.total_steps", opt.total);
  for (const k of ADAM_KEYS) meta.set(`forge.adam.${k}`, F64(opt[k]));
  const names = paramNames(model);
  const m = opt.m, v = opt.v;
  const tensors = [];
  model.paramList.forEach((p, j) => tensors.push({ name: names[j], dims: [p.n], type: GGML_F32, data: bytesOf(p._download()) }));
  model.paramList.forEach((p, j) => tensors.push({ name: `forge.adam.m.${names[j]}`, dims: [p.n], type: GGML_F32, data: bytesOf(m[j]) }));
  model.paramList.forEach((p, j) => tensors.push({ name: `forge.adam.v.${names[j]}`, dims: [p.n], type: GGML_F32, data: bytesOf(v[j]) }));
  return writeGGUF({ meta, tensors }).bytes;
}

/** Checkpoint bytes → {model, opt}: a TrainableTransformer with the saved
 *  parameters and an Adam with the saved m, v, t and hyper-parameters. */
export function loadCheckpoint(buf) {
  const g = readGGUF(buf);
  if (g.meta.get("forge.checkpoint.version") !== 1) throw new Error("loadCheckpoint: not a forge-llm_amd checkpoint");
  const c0 = configFrom(g);
  const c = new Config(Object.assign({}, c0, {
    normEps: g.meta.get("forge.config.norm_eps"), ropeTheta: g.meta.get("forge.config.rope_theta"),
  }));
  const tied = g.meta.get("forge.checkpoint.tied");
  const get = (nm) => {
    const t = g.getTensor(nm);
    if (!t || t.type !== GGML_F32) throw new Error(`loadCheckpoint: tensor ${nm} missing`);
    return new Float32Array(t.data.slice().buffer);
  };
  const names = parameterSlots(c, tied).map(slotName);
  const model = new TrainableTransformer(c, weightsFromSlots(c, tied, (slot) => get(slotName(slot))));
  const M = (k) => g.meta.get(`forge.adam.${k}`);
  const opt = new Adam(model.paramList, {
    lr: M("lr"), b1: M("b1"), b2: M("b2"), eps: M("eps"), wd: M("wd"), clip: M("clip"), totalSteps: M("total_steps"),
  });
  opt._restore(M("t"), names.map((nm) => get(`forge.adam.m.${nm}`)), names.map((nm) => get(`forge.adam.v.${nm}`)));
  return { model, opt };
}
