// Times the inference forward (Transformer.forward, one token per step with a
// KV cache) on the GPU.  Prints one JSON object.
//
//   node decode.mjs '{"preset":"125m","tokens":256,"warmup":8,"graph":true}'
//   node decode.mjs '{"preset":"b5"}'
//   node decode.mjs '{"preset":"llama8b_slice","quant":12}'   (matrices as Q4_K)
//
// `quant` (a ggml type: 1 F16, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K) quantizes
// every matrix, embedding and head included, with QuantLinear.fromF32 (the
// reference's quantizers, on the device) before loadWeights.
//
// preset b5 repeats the reference's B5 end-to-end measurement
// (bench/bench.mjs:187-215): Config dim 256, hidden 512, 4 layers, 8/4 heads,
// vocab 4096, maxSeq 512, initWeights(777), tied head; prefill = 32 forward
// calls on a fresh cache (best of 8 after 5 warm-ups); decode = forward(7,
// 200, cache) after 128 positions (best of 30 after 25 warm-ups).
//
// Pass 1: `tokens` API calls forward(token, pos, cache) — each returns the
// logits on the host (one device-to-host copy per token).  Pass 2: the same
// number of steps queued back to back (logits left in device memory) between
// two events, the device time per step.  Positions continue from the warmup,
// so pass 2 runs at positions warmup+tokens .. warmup+2·tokens−1.
import { RNG, Config, Transformer, KVCache, initWeights, hip, QuantLinear, rowBytes } from "../src/index.js";

const PRESETS = {
  "125m": { dim: 768, hidden: 2048, nLayers: 12, nHeads: 12, nKvHeads: 12, vocab: 32000, maxSeq: 1024, theta: 1e4, tied: false },
  llama8b_slice: { dim: 4096, hidden: 14336, nLayers: 1, nHeads: 32, nKvHeads: 8, vocab: 128256, maxSeq: 4096, theta: 5e5, tied: false },
};
const args = JSON.parse(process.argv[2] || "{}");
if (args.preset === "b5") {
  const cfg = new Config({ dim: 256, hidden: 512, nLayers: 4, nHeads: 8, nKvHeads: 4, vocabSize: 4096, maxSeq: 512 });
  const w = initWeights(cfg, 777);
  const weights = { tok_emb: w.tok_emb, ln_f: w.ln_f, wcls: null };
  for (let l = 0; l < cfg.nLayers; l++) weights[`layer.${l}`] = w[`layer.${l}`];
  const tr = new Transformer(cfg, { graph: args.graph !== false }).loadWeights(weights);
  const best = (fn, iters) => {
    const warm = iters <= 3 ? 5 : 25;
    for (let i = 0; i < warm; i++) fn();
    let b = Infinity, sum = 0;
    for (let i = 0; i < iters; i++) {
      const t0 = process.hrtime.bigint();
      fn();
      const dt = Number(process.hrtime.bigint() - t0) / 1e6;
      sum += dt;
      if (dt < b) b = dt;
    }
    return { best: b, mean: sum / iters };
  };
  const caches = [];
  const tPre = best(() => {
    const cache = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
    for (let i = 0; i < 32; i++) tr.forward(i % cfg.vocabSize, i, cache);
    cache.free();
  }, 8);
  const cache = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
  for (let i = 0; i < 128; i++) tr.forward(i % cfg.vocabSize, i, cache);
  const tDec = best(() => { tr.forward(7, 200, cache); }, 30);
  console.log(JSON.stringify({
    preset: "b5", graph: args.graph !== false, prefill_ms: tPre.best, prefill_tok_s: 32 / (tPre.best / 1e3),
    decode_ms: tDec.best, decode_ms_mean: tDec.mean, decode_tok_s: 1e3 / tDec.best,
    reference_cpu: { prefill_tok_s: 329, decode_tok_s: 268, source: "docs/PERFORMANCE.md:96-97 (B5)" },
  }));
  tr.release();
  cache.free();
  process.exit(0);
}
const P = Object.assign({}, PRESETS[args.preset || "125m"], args.override || {});
const tokens = args.tokens || 256, warmup = args.warmup === undefined ? 8 : args.warmup;
const a = hip();
const cfg = new Config({ dim: P.dim, hidden: P.hidden, nLayers: P.nLayers, nHeads: P.nHeads, nKvHeads: P.nKvHeads,
                         vocabSize: P.vocab, maxSeq: P.maxSeq, normEps: 1e-5, ropeTheta: P.theta });
if (warmup + 2 * tokens > cfg.maxSeq) throw new Error("warmup + 2*tokens exceeds maxSeq");
const w = initWeights(cfg, 1337);
if (!P.tied) {
  const r = new RNG(4242);
  w.wcls = new Float32Array(cfg.vocabSize * cfg.dim);
  for (let i = 0; i < w.wcls.length; i++) w.wcls[i] = r.normal() * 0.02;
}
const qt = args.quant || 0;
const D = cfg.dim, H = cfg.hidden, V = cfg.vocabSize, L = cfg.nLayers;
const q = (x, N, K) => (qt ? QuantLinear.fromF32(x, N, K, qt) : x);
const weights = { tok_emb: q(w.tok_emb, V, D), ln_f: w.ln_f, wcls: w.wcls ? q(w.wcls, V, D) : null };
for (let l = 0; l < cfg.nLayers; l++) {
  const Lw = w[`layer.${l}`];
  weights[`layer.${l}`] = { ln1: Lw.ln1, ln2: Lw.ln2, wqkv: q(Lw.wqkv, cfg.qkvOut, D), wo: q(Lw.wo, D, D),
    ffn_gate: q(Lw.ffn_gate, H, D), ffn_up: q(Lw.ffn_up, H, D), ffn_down: q(Lw.ffn_down, D, H) };
}
const tr = new Transformer(cfg, { graph: args.graph !== false }).loadWeights(weights);
const cache = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
const rng = new RNG(3);
let pos = 0;
for (let i = 0; i < warmup; i++) tr.forward(rng.int(cfg.vocabSize), pos++, cache);
a.sync();
const h0 = process.hrtime.bigint();
for (let i = 0; i < tokens; i++) tr.forward(rng.int(cfg.vocabSize), pos++, cache);
const apiMs = Number(process.hrtime.bigint() - h0) / 1e6;
const pos1 = pos;
const e0 = a.eventCreate(), e1 = a.eventCreate();
a.eventRecord(e0);
for (let i = 0; i < tokens; i++) tr._step(rng.int(cfg.vocabSize), pos++, cache);
a.eventRecord(e1);
a.sync();
const devMs = a.eventElapsed(e0, e1);
// bytes one step reads: every matrix once (the head; the embedding row only),
// the norm vectors
const rbD = rowBytes(qt, D), rbH = rowBytes(qt, H);
const weightBytes = L * (rbD * (cfg.qkvOut + D + 2 * H) + rbH * D + 8 * D) + rbD * V + rbD + 4 * D;
// KV bytes read by the attention at the mean position of pass 2
const meanN = (pos1 + pos - 1) / 2 + 1;
const kvBytes = 2 * 4 * L * cfg.kvDim * meanN;
console.log(JSON.stringify({
  preset: args.preset || "125m", cfg: P, quant: qt, graph: args.graph !== false, tokens, warmup,
  api_ms_per_token: apiMs / tokens, api_tokens_per_s: 1e3 * tokens / apiMs,
  device_ms_per_token: devMs / tokens, device_tokens_per_s: 1e3 * tokens / devMs,
  positions_pass2: [pos1, pos - 1], weight_bytes: weightBytes, kv_bytes_mean: kvBytes,
  device_gbs: (weightBytes + kvBytes) / (devMs / tokens * 1e-3) / 1e9,
}));
tr.release();
cache.free();
