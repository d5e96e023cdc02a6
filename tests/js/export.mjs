// GGUF export / load and training checkpoints on the GPU.
//  * loadGGUF(exportGGUF(w)) gives a device Transformer whose decode logits
//    are bit-identical to new Transformer(cfg).loadWeights(w) (the llama
//    metadata stores eps as FLOAT32, so the direct model is given that value).
//  * Training resumed from a checkpoint is the training that never stopped:
//    6 steps straight and 3 steps + saveCheckpoint + loadCheckpoint + 3 steps
//    give bit-identical losses, gradient norms, parameters and Adam moments;
//    saving the loaded state again reproduces the file byte for byte.
// Prints one JSON line per case.
import {
  Config, TrainableTransformer, initWeights, RNG, Adam, resetTape, Transformer, KVCache,
  exportGGUF, loadGGUF, saveCheckpoint, loadCheckpoint,
} from "../../forge-llm_amd/src/index.js";

const out = [];
function rec(test, fn) {
  try { const r = fn(); out.push({ test, ok: !!r.ok, detail: r.detail || "" }); }
  catch (e) { out.push({ test, ok: false, error: String(e && e.stack || e) }); }
}

function sameBits(x, y) {
  if (x.length !== y.length) return false;
  const a = new Uint32Array(x.buffer, x.byteOffset, x.length), b = new Uint32Array(y.buffer, y.byteOffset, y.length);
  for (let i = 0; i < a.length; i++) if (a[i] !== b[i]) return false;
  return true;
}

function weightsFor(cfg, seed, untied) {
  const w = initWeights(cfg, seed);
  if (untied) {
    const r = new RNG(seed + 1);
    w.wcls = new Float32Array(cfg.vocabSize * cfg.dim);
    for (let i = 0; i < w.wcls.length; i++) w.wcls[i] = r.normal() * 0.02;
  }
  return w;
}

const SPECS = [
  { name: "demo tied GQA", dim: 64, hidden: 128, nLayers: 2, nHeads: 4, nKvHeads: 2, vocab: 31, untied: false },
  { name: "untied MHA dH=64", dim: 128, hidden: 256, nLayers: 2, nHeads: 2, nKvHeads: 2, vocab: 97, untied: true },
];

function cfgOf(s, eps = 1e-5) {
  return new Config({ dim: s.dim, hidden: s.hidden, nLayers: s.nLayers, nHeads: s.nHeads, nKvHeads: s.nKvHeads,
                      vocabSize: s.vocab, maxSeq: 64, normEps: eps, ropeTheta: 1e4 });
}

function decode(tr, cfg, toks) {
  const cache = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.nKvHeads * cfg.dHead);
  const logits = [];
  try {
    toks.forEach((t, p) => logits.push(Float32Array.from(tr.forward(t, p, cache))));
  } finally { cache.free(); }
  return logits;
}

for (const s of SPECS) {
  rec(`loadGGUF decode == loadWeights decode (${s.name})`, () => {
    const cfg = cfgOf(s);
    const w = weightsFor(cfg, 20260101, s.untied);
    const m = loadGGUF(exportGGUF(w, cfg, null, 0, "export-test"));
    const c = m.config;
    const cfgOk = c.dim === cfg.dim && c.hidden === cfg.hidden && c.nLayers === cfg.nLayers && c.nHeads === cfg.nHeads &&
      c.nKvHeads === cfg.nKvHeads && c.vocabSize === cfg.vocabSize && c.maxSeq === cfg.maxSeq &&
      c.normEps === Math.fround(1e-5) && c.ropeTheta === 1e4 && m.vocab === null &&
      m.metadata.get("general.name") === "export-test";
    const direct = new Transformer(cfgOf(s, Math.fround(1e-5))).loadWeights(w);
    const toks = [1, 5, 3, 9, 0, 2, 7, s.vocab - 1];
    const a = decode(m.transformer, c, toks), b = decode(direct, c, toks);
    m.transformer.release(); direct.release();
    const bad = a.map((x, i) => (sameBits(x, b[i]) ? -1 : i)).filter((i) => i >= 0);
    return { ok: cfgOk && bad.length === 0, detail: cfgOk ? `positions differing: [${bad}]` : "config mismatch" };
  });
}

function batches(n, B, T, V, seed) {
  const r = new RNG(seed);
  const out = [];
  for (let k = 0; k < n; k++) {
    const b = [];
    for (let i = 0; i < B; i++) { const row = []; for (let t = 0; t <= T; t++) row.push(r.int(V)); b.push(row); }
    out.push(b);
  }
  return out;
}

function steps(model, opt, list) {
  const hist = [];
  for (const batch of list) {
    resetTape();
    model.zeroGrad();
    const loss = model.backward(model.lossBatch(batch));
    const info = opt.step();
    hist.push([loss, info.lr, info.gnorm]);
  }
  resetTape();
  return hist;
}

for (const s of SPECS) {
  rec(`checkpoint resume is bit-identical (${s.name})`, () => {
    const cfg = cfgOf(s);
    const w = weightsFor(cfg, 7, s.untied);
    const data = batches(6, 3, 16, s.vocab, 11);
    const hyper = { lr: 5e-3, totalSteps: 6, clip: 1.0, wd: 0.01 };

    const A = new TrainableTransformer(cfg, w);
    const optA = new Adam(A.paramList, hyper);
    const hA = steps(A, optA, data);

    const B0 = new TrainableTransformer(cfg, weightsFor(cfg, 7, s.untied));
    const optB0 = new Adam(B0.paramList, hyper);
    const hB = steps(B0, optB0, data.slice(0, 3));
    const file = saveCheckpoint(B0, optB0, "resume-test");
    const { model: B, opt: optB } = loadCheckpoint(file);
    const again = saveCheckpoint(B, optB, "resume-test");
    hB.push(...steps(B, optB, data.slice(3)));

    const bad = [];
    if (Buffer.compare(Buffer.from(file), Buffer.from(again)) !== 0) bad.push("re-saved file differs");
    if (B.cfg.normEps !== cfg.normEps || B.cfg.ropeTheta !== cfg.ropeTheta || !!B.params.wcls !== s.untied) bad.push("config");
    hA.forEach((h, i) => { if (!h.every((v, k) => Object.is(v, hB[i][k]))) bad.push(`step ${i}: ${h} vs ${hB[i]}`); });
    const mA = optA.m, vA = optA.v, mB = optB.m, vB = optB.v;
    A.paramList.forEach((p, j) => {
      if (!sameBits(Float32Array.from(p.data), Float32Array.from(B.paramList[j].data))) bad.push(`param ${j}`);
      if (!sameBits(mA[j], mB[j]) || !sameBits(vA[j], vB[j])) bad.push(`moments ${j}`);
    });
    if (optA.t !== optB.t) bad.push(`t ${optA.t} vs ${optB.t}`);
    return { ok: bad.length === 0, detail: bad.slice(0, 5).join("; ") || `${hA.length} steps, ${file.length} bytes` };
  });
}

rec("loadCheckpoint rejects a plain export", () => {
  const cfg = cfgOf(SPECS[0]);
  try { loadCheckpoint(exportGGUF(initWeights(cfg, 1), cfg)); return { ok: false }; } catch (e) { return { ok: /checkpoint/.test(e.message) }; }
});

for (const r of out) console.log(JSON.stringify(r));
process.exit(out.every((r) => r.ok) ? 0 : 1);
