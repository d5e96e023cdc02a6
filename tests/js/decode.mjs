// The inference forward on the device (Transformer / KVCache of
// forge-llm_amd/src): I-70 with both sides on the GPU (verify.js:288-310),
// graph replay equal to op-by-op steps, the KVCache interface, and errors.
// Prints one JSON line per case.
import {
  Config, Transformer, KVCache, TrainableTransformer, initWeights, resetTape, RNG,
} from "../../forge-llm_amd/src/index.js";

const out = [];
function rec(test, fn) {
  try {
    const r = fn();
    out.push({ test, ok: !!r.ok, detail: r.detail });
  } catch (e) {
    out.push({ test, ok: false, error: String(e && e.stack || e) });
  }
}
function weightsFor(cfg, w) {
  const o = { tok_emb: w.tok_emb, ln_f: w.ln_f, wcls: w.wcls || null };
  for (let l = 0; l < cfg.nLayers; l++) o[`layer.${l}`] = w[`layer.${l}`];
  return o;
}
function decodeAll(tr, cfg, ids, cache) {
  const rows = [];
  for (let t = 0; t < ids.length; t++) rows.push(Float32Array.from(tr.forward(ids[t], t, cache)));
  return rows;
}
function maxDiff(rows, flat, V) {
  let m = 0;
  rows.forEach((r, t) => { for (let v = 0; v < V; v++) m = Math.max(m, Math.abs(r[v] - flat[t * V + v])); });
  return m;
}

// I-70: training forward (GPU) == token-by-token inference forward (GPU)
rec("I-70 on the device: TrainableTransformer.forward == Transformer.forward", () => {
  const cfg = new Config({ dim: 32, hidden: 64, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 40, maxSeq: 16, normEps: 1e-5 });
  const w = initWeights(cfg, 4242);
  const ids = [1, 5, 9, 13, 2, 7];
  const tm = new TrainableTransformer(cfg, w);
  resetTape();
  const logitsT = tm.forward(ids).data;
  const tr = new Transformer(cfg).loadWeights(weightsFor(cfg, w));
  const cache = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
  const d = maxDiff(decodeAll(tr, cfg, ids, cache), logitsT, cfg.vocabSize);
  return { ok: d < 2e-3 && cache.len === ids.length, detail: `maxLogitsDiff=${d.toExponential(2)}` };
});

// a larger GQA model with an untied head (dH 64), 48 positions
rec("I-70 on the device, dH 64 GQA untied head, 48 positions", () => {
  const cfg = new Config({ dim: 256, hidden: 512, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 300, maxSeq: 64, normEps: 1e-5 });
  const w = initWeights(cfg, 17);
  const r = new RNG(5);
  w.wcls = new Float32Array(cfg.vocabSize * cfg.dim);
  for (let i = 0; i < w.wcls.length; i++) w.wcls[i] = r.normal() * 0.02;
  const ids = [];
  for (let t = 0; t < 48; t++) ids.push(r.int(cfg.vocabSize));
  const tm = new TrainableTransformer(cfg, w);
  resetTape();
  const logitsT = tm.forward(ids).data;
  const tr = new Transformer(cfg).loadWeights(weightsFor(cfg, w));
  const d = maxDiff(decodeAll(tr, cfg, ids, new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim)), logitsT, cfg.vocabSize);
  return { ok: d < 2e-3, detail: `maxLogitsDiff=${d.toExponential(2)}` };
});

// graph replay == op-by-op, bit for bit; a second cache records its own graph
rec("graph replay == op-by-op decode (bit-identical), two caches", () => {
  const cfg = new Config({ dim: 128, hidden: 256, nLayers: 2, nHeads: 2, nKvHeads: 1, vocabSize: 97, maxSeq: 40, normEps: 1e-5 });
  const w = weightsFor(cfg, initWeights(cfg, 23));
  const ids = [];
  const r = new RNG(9);
  for (let t = 0; t < 30; t++) ids.push(r.int(cfg.vocabSize));
  const G = new Transformer(cfg).loadWeights(w), E = new Transformer(cfg, { graph: false }).loadWeights(w);
  const cA = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim), cB = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
  const cE = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
  const a = [], b = [], e = [];
  for (let t = 0; t < ids.length; t++) {  // interleave the two caches on one model
    a.push(Float32Array.from(G.forward(ids[t], t, cA)));
    b.push(Float32Array.from(G.forward(ids[(t + 7) % ids.length], t, cB)));
    e.push(Float32Array.from(E.forward(ids[t], t, cE)));
  }
  const same = (x, y) => x.every((v, i) => Object.is(v, y[i]));
  const ok = a.every((row, t) => same(row, e[t])) && same(cA.k, cE.k) && same(cA.v, cE.v);
  const E2 = new Transformer(cfg, { graph: false }).loadWeights(w);
  const cE2 = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
  const okB = b.every((row, t) => same(row, E2.forward(ids[(t + 7) % ids.length], t, cE2)));
  G.release(); E.release(); E2.release();
  return { ok: ok && okB && G._graphs.length === 0, detail: `graphs ok=${ok} second cache ok=${okB}` };
});

rec("KVCache interface (put / slice / views / reset / bytes)", () => {
  const c = new KVCache(2, 8, 6);
  const k = Float32Array.from([1, 2, 3, 4, 5, 6]), v = Float32Array.from([6, 5, 4, 3, 2, 1]);
  c.put(1, 3, k, v);
  const ok = c.len === 4 && c.sliceK(1, 3).every((x, i) => x === k[i]) && c.sliceV(1, 3).every((x, i) => x === v[i]) &&
    c.kView(1, 4).length === 24 && c.kView(1, 4)[18] === 1 && c.bytes() === 2 * 2 * 8 * 6 * 4 && c.k.length === 96;
  c.reset();
  return { ok: ok && c.len === 0, detail: "" };
});

rec("errors: position range, freed cache, short quantized weights, cache shape", () => {
  const cfg = new Config({ dim: 32, hidden: 64, nLayers: 1, nHeads: 4, nKvHeads: 2, vocabSize: 40, maxSeq: 8, normEps: 1e-5 });
  const w = weightsFor(cfg, initWeights(cfg, 1));
  const tr = new Transformer(cfg).loadWeights(w);
  const c = new KVCache(cfg.nLayers, 8, cfg.kvDim);
  const throws = (fn, T) => { try { fn(); return false; } catch (e) { return e instanceof T; } };
  const e1 = throws(() => tr.forward(1, 8, c), RangeError);
  const e2 = throws(() => tr.forward(1, 0, new KVCache(2, 8, cfg.kvDim)), RangeError);
  const q = Object.assign({}, w, { tok_emb: { type: 8, bytes: new Uint8Array(10) } });
  const e3 = throws(() => new Transformer(cfg).loadWeights(q), Error);
  tr.forward(1, 0, c); tr.forward(2, 1, c); tr.forward(3, 2, c);  // eager, recorded, replayed
  c.free();
  const e4 = throws(() => tr.forward(1, 3, c), Error);
  const nan = tr.forward(40, 0, new KVCache(cfg.nLayers, 8, cfg.kvDim)).every((x) => Number.isNaN(x));
  tr.release();
  return { ok: e1 && e2 && e3 && e4 && nan, detail: `${e1} ${e2} ${e3} ${e4} nan=${nan}` };
});

for (const r of out) console.log(JSON.stringify(r));
process.exit(out.every((r) => r.ok) ? 0 : 1);
