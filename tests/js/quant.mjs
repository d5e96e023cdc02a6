// Quantized weights through the JS API (forge-llm_amd/src/L3/quant.js,
// L4/nn.js, L6/transformer.js, L9/export.js) on the GPU:
//  * the reference's own L3/L4 tests and invariants, restated over the device
//    API (test/l3-l5.test.js:17-172; verify.js I-20, I-22, I-23, I-40, I-41);
//  * QuantLinear matrices in Transformer.loadWeights, and a quantized GGUF
//    export loaded back by loadGGUF, decode the same logits bit for bit;
//  * a binary dump (argv[2]) of quantizeRow bytes, dotQ values,
//    QuantLinear.forward outputs and quantized-model logits, which the Python
//    side checks against the oracle.
// Prints one JSON line per case.
import { writeFileSync } from "fs";
import {
  RNG, Config, initWeights, Transformer, KVCache, QuantLinear, SwiGLU, GGMLType, info, rowBytes, dequantize,
  quantizeRow, dotQ, qualityReport, fp16Table, quantizeRowQ8_0, quantizeRowQ5K, quantizeRowQ6K, quantizeRowF16,
  exportGGUF, loadGGUF, readGGUF, writeGGUF,
} from "../../forge-llm_amd/src/index.js";

const out = [];
function rec(test, fn) {
  try { const r = fn(); out.push({ test, ok: !!r.ok, detail: r.detail || "" }); }
  catch (e) { out.push({ test, ok: false, error: String(e && e.stack || e) }); }
}
const normals = (seed, n, s = 1) => { const r = new RNG(seed), x = new Float32Array(n); for (let i = 0; i < n; i++) x[i] = r.normal() * s; return x; };
function dot(a, b, n) { let s = 0; for (let i = 0; i < n; i++) s += a[i] * b[i]; return s; }
function matvec(o, W, x, N, K) { for (let n = 0; n < N; n++) { let s = 0; for (let k = 0; k < K; k++) s += W[n * K + k] * x[k]; o[n] = s; } return o; }
const cos = (a, b) => dot(a, b, a.length) / Math.sqrt(dot(a, a, a.length) * dot(b, b, b.length));
const sameBits = (x, y) => x.length === y.length && Buffer.compare(Buffer.from(x.buffer, x.byteOffset, x.byteLength), Buffer.from(y.buffer, y.byteOffset, y.byteLength)) === 0;

rec("bpw and rowBytes tables (l3-l5.test.js:17-33, I-23)", () => {
  const ok = info(12).bpw === 4.5 && info(13).bpw === 5.5 && info(14).bpw === 6.5625 && info(8).bpw === 8.5 &&
    info(1).bpw === 16 && info(0).bpw === 32 && rowBytes(12, 256) === 144 && rowBytes(12, 512) === 288 &&
    rowBytes(14, 256) === 210 && rowBytes(8, 32) === 34 && rowBytes(8, 64) === 68 && rowBytes(0, 100) === 400;
  return { ok };
});

rec("F16 round trip (l3-l5.test.js:35-45)", () => {
  const x = normals(1, 64);
  const dq = dequantize(1, quantizeRowF16(x, 64), 64);
  let m = 0; for (let i = 0; i < 64; i++) m = Math.max(m, Math.abs(dq[i] - x[i]) / (Math.abs(x[i]) + 1e-3));
  return { ok: m < 1e-3, detail: `maxRel ${m}` };
});

rec("Q8_0 error bound amax/254 (l3-l5.test.js:47-58)", () => {
  const x = normals(2, 256);
  const dq = dequantize(8, quantizeRowQ8_0(x, 256), 256);
  let amax = 0, worst = 0;
  for (let i = 0; i < 256; i++) { amax = Math.max(amax, Math.abs(x[i])); worst = Math.max(worst, Math.abs(dq[i] - x[i])); }
  return { ok: worst <= amax / 254 + 1e-6, detail: `${worst} <= ${amax / 254}` };
});

rec("dotQ == dequantize-then-dot (l3-l5.test.js:60-72, I-22)", () => {
  const r = new RNG(3), x = new Float32Array(512), y = new Float32Array(512);
  for (let i = 0; i < 512; i++) { x[i] = r.normal() * 0.8; y[i] = r.normal(); }
  const bad = [];
  for (const t of [1, 8, 12, 13, 14]) {
    const q = quantizeRow(t, x, 512);
    const a = dot(dequantize(t, q, 512), y, 512), b = dotQ(t, q, y, 512);
    if (!(Math.abs(a - b) <= 1e-3 * (Math.abs(a) + 1))) bad.push(`${t}: ${a} vs ${b}`);
  }
  return { ok: bad.length === 0, detail: bad.join("; ") };
});

rec("Q5_K size, error and fifth bit (l3-l5.test.js:74-90)", () => {
  const x = normals(7, 256, 0.5);
  const q = quantizeRowQ5K(x, 256);
  const dq = dequantize(13, q, 256);
  let se = 0, sx = 0; for (let i = 0; i < 256; i++) { se += (dq[i] - x[i]) ** 2; sx += x[i] ** 2; }
  let qh = 0; for (let i = 0; i < 32; i++) if (q[16 + i] !== 0) qh++;
  return { ok: q.length === 176 && quantizeRow(13, x, 256).length === 176 && Math.sqrt(se / sx) < 0.05 && qh > 0, detail: `rel ${Math.sqrt(se / sx)}` };
});

rec("Q6_K d at the block end (l3-l5.test.js:92-112)", () => {
  const x = normals(8, 256), y = new Float32Array(256);
  for (let i = 0; i < 256; i++) y[i] = x[i] * 4;
  const qx = quantizeRowQ6K(x, 256), qy = quantizeRowQ6K(y, 256);
  let head = true; for (let i = 0; i < 208; i++) if (qx[i] !== qy[i]) head = false;
  const T = fp16Table();
  const dx = T[qx[208] | (qx[209] << 8)], dy = T[qy[208] | (qy[209] << 8)];
  return { ok: qx.length === 210 && head && (qx[208] !== qy[208] || qx[209] !== qy[209]) && Math.abs(dy / dx - 4) < 0.02, detail: `${dy / dx}` };
});

rec("quality report ratios and cosines (l3-l5.test.js:114-125, I-20)", () => {
  const x = normals(4, 1024, 0.6);
  const q8 = qualityReport(8, x, 1024), q4 = qualityReport(12, x, 1024);
  const x7 = normals(9, 1024, 0.7);
  const bounds = { 8: 0.02, 12: 0.06, 13: 0.04, 14: 0.02 };
  const i20 = [8, 12, 13, 14].every((t) => qualityReport(t, x7, 1024).rmse < bounds[t]);
  return { ok: q8.ratio > 3.5 && q8.ratio < 4 && q4.ratio > 6.5 && q4.ratio < 7.5 && q8.cos > 0.999 && q4.cos > 0.995 && i20, detail: `q8 cos ${q8.cos} q4 cos ${q4.cos}` };
});

rec("QuantLinear Q8_0 vs f32, toF32 (l3-l5.test.js:127-149, I-40)", () => {
  const r = new RNG(5), N = 64, K = 128;
  const W = new Float32Array(N * K); for (let i = 0; i < W.length; i++) W[i] = r.normal();
  const x = new Float32Array(K); for (let i = 0; i < K; i++) x[i] = r.normal();
  const f = QuantLinear.fromF32(W, N, K, 0), q8 = QuantLinear.fromF32(W, N, K, GGMLType.Q8_0);
  const o1 = f.forward(x, new Float32Array(N)), o2 = q8.forward(x, new Float32Array(N));
  const ref = matvec(new Float32Array(N), W, x, N, K);
  let rel = 0; for (let i = 0; i < N; i++) rel = Math.max(rel, Math.abs(o1[i] - ref[i]) / Math.abs(ref[i]));
  const toF = sameBits(q8.toF32(), dequantize(8, q8.bytes, N * K));
  return { ok: cos(o1, o2) > 0.999 && rel < 1e-6 && toF && q8.bytesSize() === N * 136, detail: `cos ${cos(o1, o2)}, f32 max rel ${rel}` };
});

rec("SwiGLU block == decomposition (l3-l5.test.js:151-172, I-41)", () => {
  const dim = 32, hidden = 64, r = new RNG(7);
  const gW = new Float32Array(hidden * dim), uW = new Float32Array(hidden * dim), dW = new Float32Array(dim * hidden);
  for (let i = 0; i < gW.length; i++) { gW[i] = r.normal(); uW[i] = r.normal(); }
  for (let i = 0; i < dW.length; i++) dW[i] = r.normal();
  const x = new Float32Array(dim); for (let i = 0; i < dim; i++) x[i] = r.normal();
  const sw = new SwiGLU(QuantLinear.fromF32(gW, hidden, dim, 0), QuantLinear.fromF32(uW, hidden, dim, 0), QuantLinear.fromF32(dW, dim, hidden, 0), dim, hidden);
  const o = sw.forward(x, new Float32Array(dim));
  const gv = matvec(new Float32Array(hidden), gW, x, hidden, dim), uv = matvec(new Float32Array(hidden), uW, x, hidden, dim);
  const act = new Float32Array(hidden); for (let i = 0; i < hidden; i++) act[i] = (gv[i] / (1 + Math.exp(-gv[i]))) * uv[i];
  const ref = matvec(new Float32Array(dim), dW, act, dim, hidden);
  let m = 0; for (let i = 0; i < dim; i++) m = Math.max(m, Math.abs(o[i] - ref[i]));
  return { ok: m < 1e-5, detail: `maxErr ${m}` };
});

// ── quantized models ──
const cfg = new Config({ dim: 256, hidden: 512, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 96, maxSeq: 32, normEps: 1e-5 });
const w0 = initWeights(cfg, 5);
const ids = [3, 17, 0, 95, 5, 40, 41, 8];
function decode(tr) {
  const c = new KVCache(cfg.nLayers, cfg.maxSeq, cfg.kvDim);
  const rows = ids.map((t, p) => Float32Array.from(tr.forward(t, p, c)));
  c.free();
  return rows;
}
const dumps = [];
for (const qt of [8, 12, 13, 14]) {
  rec(`QuantLinear weights == loadGGUF(exportGGUF(w, ${qt})) decode, bit for bit`, () => {
    const D = cfg.dim, H = cfg.hidden;
    const ql = (a, N, K) => QuantLinear.fromF32(a, N, K, qt);
    const w = { tok_emb: ql(w0.tok_emb, cfg.vocabSize, D), ln_f: w0.ln_f, wcls: null };
    for (let l = 0; l < cfg.nLayers; l++) {
      const L = w0[`layer.${l}`];
      w[`layer.${l}`] = { ln1: L.ln1, ln2: L.ln2, wqkv: ql(L.wqkv, cfg.qkvOut, D), wo: ql(L.wo, D, D),
        ffn_gate: ql(L.ffn_gate, H, D), ffn_up: ql(L.ffn_up, H, D), ffn_down: ql(L.ffn_down, D, H) };
    }
    const direct = new Transformer(cfg).loadWeights(w);
    dumps.push(...decode(direct));
    direct.release();
    // the llama metadata holds eps as FLOAT32: compare with a model given that eps
    const cfg32 = new Config(Object.assign({}, cfg, { normEps: Math.fround(cfg.normEps) }));
    const direct32 = new Transformer(cfg32).loadWeights(w);
    const file = exportGGUF(w0, cfg, null, qt, "q-test");
    const g = readGGUF(file);
    const typed = g.tensors.filter((t) => t.dims.length === 2).every((t) => t.type === qt);
    const m = loadGGUF(file);
    const a = decode(direct32), b = decode(m.transformer);
    direct32.release(); m.transformer.release();
    const bad = a.map((r, i) => (sameBits(r, b[i]) ? -1 : i)).filter((i) => i >= 0);
    return { ok: typed && bad.length === 0 && m.config.dim === D, detail: `${file.length} bytes; differing positions [${bad}]` };
  });
}

// I-60 / I-61 (verify.js:415-443): a model with N(0, 1) weights decoded in f32
// and in Q8_0 (cosine >= 0.99 at every position, argmax flips at most once),
// and two separate f32 models on the same input give the same logits.
{
  const c2 = new Config({ dim: 128, hidden: 256, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 64, maxSeq: 32, normEps: 1e-5 });
  const r2 = new RNG(99);
  const mat = (n) => { const a = new Float32Array(n); for (let i = 0; i < n; i++) a[i] = r2.normal(); return a; };
  const ones = (n) => new Float32Array(n).fill(1);
  const D = c2.dim, H = c2.hidden;
  const W = { tok_emb: mat(c2.vocabSize * D), ln_f: ones(D), wcls: null };
  for (let l = 0; l < c2.nLayers; l++)
    W[`layer.${l}`] = { ln1: ones(D), ln2: ones(D), wqkv: mat(c2.qkvOut * D), wo: mat(D * D), ffn_gate: mat(H * D),
                        ffn_up: mat(H * D), ffn_down: mat(D * H) };
  const asType = (qt) => {
    if (qt === 0) return W;
    const ql = (a, N, K) => QuantLinear.fromF32(a, N, K, qt);
    const w = { tok_emb: ql(W.tok_emb, c2.vocabSize, D), ln_f: W.ln_f, wcls: null };
    for (let l = 0; l < c2.nLayers; l++) {
      const L = W[`layer.${l}`];
      w[`layer.${l}`] = { ln1: L.ln1, ln2: L.ln2, wqkv: ql(L.wqkv, c2.qkvOut, D), wo: ql(L.wo, D, D),
        ffn_gate: ql(L.ffn_gate, H, D), ffn_up: ql(L.ffn_up, H, D), ffn_down: ql(L.ffn_down, D, H) };
    }
    return w;
  };
  const argmax = (a) => { let b = 0; for (let i = 1; i < a.length; i++) if (a[i] > a[b]) b = i; return b; };
  rec("I-60 f32 vs Q8_0 decode: cosine >= 0.99, argmax flips at most once", () => {
    const t32 = new Transformer(c2).loadWeights(asType(0)), t8 = new Transformer(c2).loadWeights(asType(8));
    const k32 = new KVCache(c2.nLayers, c2.maxSeq, c2.kvDim), k8 = new KVCache(c2.nLayers, c2.maxSeq, c2.kvDim);
    let cosMin = 1, match = 0;
    const nPos = 8;
    for (let pos = 0; pos < nPos; pos++) {
      const a = Float32Array.from(t32.forward(pos, pos, k32)), b = Float32Array.from(t8.forward(pos, pos, k8));
      cosMin = Math.min(cosMin, cos(a, b));
      if (argmax(a) === argmax(b)) match++;
    }
    t32.release(); t8.release(); k32.free(); k8.free();
    return { ok: cosMin >= 0.99 && match >= nPos - 1, detail: `minCos ${cosMin} argmax match ${match}/${nPos}` };
  });
  rec("I-61 same input, two models -> same logits (< 1e-6)", () => {
    const ta = new Transformer(c2).loadWeights(asType(0)), tb = new Transformer(c2).loadWeights(asType(0));
    const ca = new KVCache(c2.nLayers, c2.maxSeq, c2.kvDim), cb = new KVCache(c2.nLayers, c2.maxSeq, c2.kvDim);
    const la = Float32Array.from(ta.forward(5, 0, ca)), lb = Float32Array.from(tb.forward(5, 0, cb));
    ta.release(); tb.release(); ca.free(); cb.free();
    let m = 0;
    for (let i = 0; i < la.length; i++) m = Math.max(m, Math.abs(la[i] - lb[i]));
    return { ok: m < 1e-6, detail: `maxErr ${m}` };
  });
}

rec("q/k/v of different types are rejected by loadGGUF, as the reference does", () => {
  const file = exportGGUF(w0, cfg, null, 0, "mixed");
  const g = readGGUF(file);
  const tensors = g.tensors.map((t) => {
    const s = g.getTensor(t.name);
    if (t.name === "blk.0.attn_v.weight") {
      const n = t.dims[0] * t.dims[1];
      return { name: t.name, dims: t.dims, type: 8, data: quantizeRow(8, new Float32Array(s.data.slice().buffer), n) };
    }
    return { name: t.name, dims: t.dims, type: s.type, data: s.data };
  });
  const bytes = writeGGUF({ meta: g.meta, tensors }).bytes;
  try { loadGGUF(bytes); return { ok: false, detail: "loaded" }; } catch (e) { return { ok: /types differ/.test(e.message), detail: e.message }; }
});

// dump for the oracle comparison: quantizeRow bytes and dotQ / forward of a seeded matrix, then logits
if (process.argv[2]) {
  const N = 40, K = 512, W = normals(11, N * K, 0.05), x = normals(12, K);
  const parts = [];
  for (const t of [1, 8, 12, 13, 14]) {
    const q = quantizeRow(t, W, N * K);
    const ql = new QuantLinear(t, q, N, K);
    const y = ql.forward(x, new Float32Array(N));
    const d = new Float64Array([dotQ(t, q, x, K, 0, 0), dotQ(t, q, x, K, 0, rowBytes(t, K) * 7)]);
    parts.push(new Uint8Array(q), new Uint8Array(y.buffer), new Uint8Array(d.buffer));
  }
  for (const r of dumps) parts.push(new Uint8Array(r.buffer));
  writeFileSync(process.argv[2], Buffer.concat(parts.map((p) => Buffer.from(p.buffer, p.byteOffset, p.byteLength))));
}

for (const r of out) console.log(JSON.stringify(r));
process.exit(out.every((r) => r.ok) ? 0 : 1);
