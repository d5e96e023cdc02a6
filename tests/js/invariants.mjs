// The reference's own checks for the training path, run with the GPU ops:
// the L10 invariants I-30, I-31, I-32, I-33a–d, I-34, I-35, I-36, I-71
// (src/L10/verify.js:91-325) and the hot-path unit tests of
// test/l2-l6.test.js (gradient checks, closed forms, batch == per-sample,
// overfit, Adam first step, tape isolation), with the same thresholds.
// Inputs replay the reference's seeded RNG draws where it uses one.
import { test, assert, run } from "./harness.mjs";
import {
  RNG, Config, TrainableTransformer, initWeights, resetTape, backward, gradCheck, param, leaf, Adam, op,
  add, linear, softmaxCE, matmulT, embedLookup, rmsNorm, ropeRows, causalAttn, causalAttnBatch, swigluRows,
  crossEntropyMean, weightedSum, sliceCols, matmul, qkvRope, qkvRopeAttention, matmulTResid, swigluGateUp, packPair,
  crossEntropyMeanFused,
} from "../../forge-llm_amd/src/index.js";

const randArr = (n, rng, scale = 1) => { const a = new Float32Array(n); for (let i = 0; i < n; i++) a[i] = rng.normal() * scale; return a; };

// verify.js:141-162 / l2-l6.test.js:19-40: central differences, error relative to the gradient scale.
function numGrad(lossFn, params, eps = 2e-3) {
  resetTape();
  const base = lossFn();
  backward(base);
  let worst = 0, at = "";
  for (const name of Object.keys(params)) {
    const p = params[name];
    const g = p.grad;
    const ana = Float32Array.from(g || new Float32Array(p.n));
    let gmax = 0;
    for (let i = 0; i < ana.length; i++) gmax = Math.max(gmax, Math.abs(ana[i]));
    const floor = Math.max(gmax, 1e-3);
    for (let i = 0; i < p.n; i++) {
      const o = p.data[i];
      p.data[i] = o + eps; const lp = lossFn().data[0];
      p.data[i] = o - eps; const lm = lossFn().data[0];
      p.data[i] = o;
      const num = (lp - lm) / (2 * eps);
      const rel = Math.abs(num - ana[i]) / floor;
      if (rel > worst) { worst = rel; at = `${name}[${i}]`; }
    }
  }
  return { maxRelErr: worst, at };
}

// ── L10 invariants (verify.js) with the RNG(12345) draw sequence ──
const vr = new RNG(12345);
randArr(8 * 12 + 16 * 12 + 12, vr);  // I-00/I-01 inputs
randArr(7 + 8 + 16, vr);            // I-10, I-12, I-13 inputs

test("I-30 linear+softmaxCE gradCheck < 1e-4", () => {
  resetTape();
  const K = 5, N = 4;
  const W = param(new Float32Array([0.3, -0.2, 0.1, 0.4, 0.0, 0.2, -0.1, 0.5, 0.3, -0.4, 0.1, 0.2, 0.6, -0.3, 0.2, 0.4, -0.5, 0.1, 0.3, 0.2]));
  const x = leaf(new Float32Array([1, 0.5, -0.3, 0.2, 0.4]));
  const lossFn = () => { resetTape(); return softmaxCE(linear(W, x, N, K), 2); };
  const gc = gradCheck(lossFn, { W });
  assert(gc.maxRelErr < 1e-4, `maxRelErr=${gc.maxRelErr} @ ${gc.at}`);
  return gc;
});

test("I-31 softmaxCE gradient = p − onehot (1e-5)", () => {
  resetTape();
  const logits = leaf(new Float32Array([1.2, 0.3, -0.5, 2.1]));
  backward(softmaxCE(logits, 1));
  const x = logits.data, g = logits.grad;
  let mx = -Infinity; for (const v of x) mx = Math.max(mx, v);
  let s = 0; const p = []; for (const v of x) { const e = Math.exp(v - mx); p.push(e); s += e; }
  let worst = 0;
  for (let i = 0; i < p.length; i++) worst = Math.max(worst, Math.abs(g[i] - (p[i] / s - (i === 1 ? 1 : 0))));
  assert(worst <= 1e-5, `max |grad - (p - onehot)| = ${worst}`);
  return { worst };
});

test("I-32 Adam first step ≈ lr", () => {
  const p1 = param(new Float32Array([1.0]));
  p1.grad = new Float32Array([1.0]);
  const opt = new Adam([p1], { lr: 0.1, totalSteps: 100 });
  opt.step();
  const upd = Math.abs(1.0 - p1.data[0]);
  assert(upd > 0 && upd < 0.2, `dw=${upd}`);
  return { dw: upd };
});

test("I-33a matmulT grad = central difference", () => {
  const M = 3, K = 5, N = 4;
  const X = param(randArr(M * K, vr, 0.5)), W = param(randArr(N * K, vr, 0.5));
  const t = randArr(M * N, vr);
  const gc = numGrad(() => { resetTape(); return weightedSum(matmulT(X, W, M, K, N), t); }, { X, W });
  assert(gc.maxRelErr < 2e-3, `maxRelErr=${gc.maxRelErr} @ ${gc.at}`);
  return gc;
});

test("I-33b rmsNorm grad = central difference", () => {
  const T = 2, D = 6;
  const X = param(randArr(T * D, vr, 0.5)), Wt = param(new Float32Array(D).fill(1));
  const t = randArr(T * D, vr);
  const gc = numGrad(() => { resetTape(); return weightedSum(rmsNorm(X, Wt, T, D, 1e-5), t); }, { X, Wt });
  assert(gc.maxRelErr < 2e-3, `maxRelErr=${gc.maxRelErr} @ ${gc.at}`);
  return gc;
});

test("I-33c ropeRows grad = central difference", () => {
  const T = 3, nH = 2, dH = 4;
  const X = param(randArr(T * nH * dH, vr, 0.5));
  const t = randArr(T * nH * dH, vr);
  const gc = numGrad(() => { resetTape(); return weightedSum(ropeRows(X, T, nH, dH, 0, 10000), t); }, { X });
  assert(gc.maxRelErr < 2e-3, `maxRelErr=${gc.maxRelErr} @ ${gc.at}`);
  return gc;
});

test("I-33d causalAttn (GQA) grad = central difference", () => {
  const T = 4, nH = 4, nKV = 2, dH = 4;
  const Q = param(randArr(T * nH * dH, vr, 0.5));
  const K = param(randArr(T * nKV * dH, vr, 0.5));
  const V = param(randArr(T * nKV * dH, vr, 0.5));
  const t = randArr(T * nH * dH, vr);
  const gc = numGrad(() => { resetTape(); return weightedSum(causalAttn(Q, K, V, T, nH, nKV, dH), t); }, { Q, K, V });
  assert(gc.maxRelErr < 2e-3, `maxRelErr=${gc.maxRelErr} @ ${gc.at}`);
  return gc;
});

test("I-34 crossEntropyMean grad = (P−OneHot)/T", () => {
  const T = 3, V = 5;
  const L = param(randArr(T * V, vr, 0.5));
  const targets = [1, 3, 0];
  resetTape();
  backward(crossEntropyMean(L, targets, T, V));
  const g = L.grad, x = L.data;
  let worst = 0;
  for (let t = 0; t < T; t++) {
    let mx = -Infinity; for (let i = 0; i < V; i++) mx = Math.max(mx, x[t * V + i]);
    let s = 0; const p = new Float64Array(V);
    for (let i = 0; i < V; i++) { p[i] = Math.exp(x[t * V + i] - mx); s += p[i]; }
    for (let i = 0; i < V; i++) worst = Math.max(worst, Math.abs(g[t * V + i] - (p[i] / s - (i === targets[t] ? 1 : 0)) / T));
  }
  assert(worst <= 1e-6, `maxΔ=${worst}`);
  return { maxDelta: worst };
});

test("I-35 swigluRows grad = central difference", () => {
  const T = 2, H = 5;
  const G = param(randArr(T * H, vr, 0.5)), U = param(randArr(T * H, vr, 0.5));
  const t = randArr(T * H, vr);
  const gc = numGrad(() => { resetTape(); return weightedSum(swigluRows(G, U, T, H), t); }, { G, U });
  assert(gc.maxRelErr < 2e-3, `maxRelErr=${gc.maxRelErr} @ ${gc.at}`);
  return gc;
});

test("I-36 embedLookup grad = scatter-add", () => {
  const V = 5, D = 3;
  const E = param(randArr(V * D, vr, 0.5));
  const ids = [0, 3, 3];
  resetTape();
  const X = embedLookup(E, ids, V, D);
  const t = new Float32Array(X.n); for (let i = 0; i < t.length; i++) t[i] = i + 1;
  backward(weightedSum(X, t));
  const g = E.grad;
  let worst = 0;
  for (let v = 0; v < V; v++) for (let d = 0; d < D; d++) {
    let want = 0;
    for (let tt = 0; tt < ids.length; tt++) if (ids[tt] === v) want += tt * D + d + 1;
    worst = Math.max(worst, Math.abs(g[v * D + d] - want));
  }
  assert(worst <= 1e-5, `maxΔ=${worst}`);
  return { maxDelta: worst };
});

test("I-71 overfit: loss < 0.6 × first", () => {
  const cfg2 = new Config({ dim: 32, hidden: 64, nLayers: 1, nHeads: 4, nKvHeads: 4, vocabSize: 20, maxSeq: 16, normEps: 1e-5 });
  const m2 = new TrainableTransformer(cfg2, initWeights(cfg2, 777));
  const data = [1, 2, 3, 4, 5, 6, 7, 8];
  resetTape();
  const first = m2.backward(m2.loss(data, data.slice(1)));
  const opt = new Adam(m2.paramList, { lr: 0.05, totalSteps: 60, clip: 1.0 });
  let last = first;
  for (let s = 0; s < 60; s++) {
    resetTape(); m2.zeroGrad();
    last = m2.backward(m2.loss(data, data.slice(1)));
    opt.step();
  }
  assert(last < first * 0.6, `${first} -> ${last}`);
  return { first, last };
});

// ── test/l2-l6.test.js ──
test("l2-l6 linear grad", () => {
  const rng = new RNG(1);
  const K = 6, N = 5;
  const W = param(randArr(K * N, rng)), x = leaf(randArr(K, rng));
  const t = randArr(N, rng);
  const { maxRelErr, at } = numGrad(() => { resetTape(); return weightedSum(linear(W, x, N, K), t); }, { W });
  assert(maxRelErr < 2e-3, `worst=${maxRelErr} @ ${at}`);
  return { maxRelErr };
});

test("l2-l6 softmaxCE grad = p − onehot", () => {
  resetTape();
  const logits = leaf(new Float32Array([1.2, 0.3, -0.5, 2.1]));
  backward(softmaxCE(logits, 1));
  const x = logits.data, g = logits.grad;
  let mx = -Infinity; for (const v of x) mx = Math.max(mx, v);
  let s = 0; const p = []; for (const v of x) { const e = Math.exp(v - mx); p.push(e); s += e; }
  for (let i = 0; i < p.length; i++) assert(Math.abs(g[i] - (p[i] / s - (i === 1 ? 1 : 0))) < 1e-5, `i=${i}`);
});

test("l2-l6 matmulT grad", () => {
  const rng = new RNG(2);
  const M = 4, K = 5, N = 3;
  const X = param(randArr(M * K, rng)), W = param(randArr(N * K, rng));
  const t = randArr(M * N, rng);
  const r = numGrad(() => { resetTape(); return weightedSum(matmulT(X, W, M, K, N), t); }, { X, W });
  assert(r.maxRelErr < 2e-3, JSON.stringify(r));
  return r;
});

test("l2-l6 rmsNorm grad", () => {
  const rng = new RNG(3);
  const T = 3, D = 8;
  const X = param(randArr(T * D, rng)), W = param(new Float32Array(D).fill(1));
  const t = randArr(T * D, rng);
  const r = numGrad(() => { resetTape(); return weightedSum(rmsNorm(X, W, T, D, 1e-5), t); }, { X, W });
  assert(r.maxRelErr < 2e-3, JSON.stringify(r));
  return r;
});

test("l2-l6 ropeRows grad", () => {
  const rng = new RNG(4);
  const T = 3, nH = 2, dH = 4;
  const X = param(randArr(T * nH * dH, rng));
  const t = randArr(T * nH * dH, rng);
  const r = numGrad(() => { resetTape(); return weightedSum(ropeRows(X, T, nH, dH, 0, 10000), t); }, { X });
  assert(r.maxRelErr < 2e-3, JSON.stringify(r));
  return r;
});

test("l2-l6 causalAttn grad (tol 5e-3)", () => {
  const rng = new RNG(5);
  const T = 4, nH = 4, nKV = 2, dH = 4;
  const Q = param(randArr(T * nH * dH, rng)), K = param(randArr(T * nKV * dH, rng)), V = param(randArr(T * nKV * dH, rng));
  const t = randArr(T * nH * dH, rng);
  const r = numGrad(() => { resetTape(); return weightedSum(causalAttn(Q, K, V, T, nH, nKV, dH), t); }, { Q, K, V });
  assert(r.maxRelErr < 5e-3, JSON.stringify(r));
  return r;
});

test("causalAttn (MFMA dH=64) grad = central difference", () => {
  const rng = new RNG(15);
  const T = 40, nH = 2, nKV = 1, dH = 64;
  const Q = param(randArr(T * nH * dH, rng, 0.3)), K = param(randArr(T * nKV * dH, rng, 0.3)), V = param(randArr(T * nKV * dH, rng, 0.3));
  const t = randArr(T * nH * dH, rng);
  // check a strided subset of elements (the full sweep is 3·T·dH·(nH+2nKV) losses)
  const lossFn = () => { resetTape(); return weightedSum(causalAttn(Q, K, V, T, nH, nKV, dH), t); };
  resetTape();
  const base = lossFn();
  backward(base);
  let worst = 0;
  for (const [name, p] of Object.entries({ Q, K, V })) {
    const ana = Float32Array.from(p.grad);
    let gmax = 0; for (const v of ana) gmax = Math.max(gmax, Math.abs(v));
    for (let i = 0; i < p.n; i += 97) {
      const o = p.data[i];
      p.data[i] = o + 2e-3; const lp = lossFn().data[0];
      p.data[i] = o - 2e-3; const lm = lossFn().data[0];
      p.data[i] = o;
      worst = Math.max(worst, Math.abs((lp - lm) / 4e-3 - ana[i]) / Math.max(gmax, 1e-3));
    }
  }
  assert(worst < 2e-2, `worst=${worst}`);
  return { worst };
});

test("l2-l6 swigluRows grad", () => {
  const rng = new RNG(6);
  const T = 2, H = 5;
  const G = param(randArr(T * H, rng)), U = param(randArr(T * H, rng));
  const t = randArr(T * H, rng);
  const r = numGrad(() => { resetTape(); return weightedSum(swigluRows(G, U, T, H), t); }, { G, U });
  assert(r.maxRelErr < 2e-3, JSON.stringify(r));
  return r;
});

test("l2-l6 crossEntropyMean grad = (P−OneHot)/T", () => {
  resetTape();
  const rng = new RNG(7);
  const T = 3, V = 6;
  const L = param(randArr(T * V, rng));
  const targets = [1, 3, 0];
  backward(crossEntropyMean(L, targets, T, V));
  const g = L.grad, x = L.data;
  for (let t = 0; t < T; t++) {
    let mx = -Infinity; for (let i = 0; i < V; i++) mx = Math.max(mx, x[t * V + i]);
    let s = 0; const p = new Float64Array(V);
    for (let i = 0; i < V; i++) { p[i] = Math.exp(x[t * V + i] - mx); s += p[i]; }
    for (let i = 0; i < V; i++) assert(Math.abs(g[t * V + i] - (p[i] / s - (i === targets[t] ? 1 : 0)) / T) < 1e-5);
  }
});

test("l2-l6 embedLookup grad = scatter-add", () => {
  resetTape();
  const V = 4, D = 3;
  const E = param(new Float32Array(V * D).map((_, i) => i * 0.1));
  const ids = [0, 2, 2];
  const X = embedLookup(E, ids, V, D);
  const t = new Float32Array(X.n).map((_, i) => i + 1);
  backward(weightedSum(X, t));
  const g = E.grad;
  for (let v = 0; v < V; v++) for (let d = 0; d < D; d++) {
    let want = 0;
    for (let tt = 0; tt < ids.length; tt++) if (ids[tt] === v) want += tt * D + d + 1;
    assert(Math.abs(g[v * D + d] - want) < 1e-5);
  }
});

test("I-33e batch block-diagonal == per-sample", () => {
  const cfg = new Config({ dim: 32, hidden: 64, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 20, maxSeq: 32 });
  const m = new TrainableTransformer(cfg, initWeights(cfg, 11));
  const rows = [[1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12]];
  resetTape();
  const batchLoss = m.backward(m.lossBatch(rows));
  let sum = 0;
  for (const r of rows) { resetTape(); sum += m.backward(m.loss(r.slice(0, -1), r.slice(1))); }
  assert(Math.abs(batchLoss - sum / rows.length) < 1e-5, `${batchLoss} vs ${sum / rows.length}`);
  return { batchLoss, perSample: sum / rows.length };
});

test("I-33e at MFMA shapes: batch == per-sample (dH 64, T 96)", () => {
  const cfg = new Config({ dim: 128, hidden: 256, nLayers: 1, nHeads: 2, nKvHeads: 1, vocabSize: 50, maxSeq: 128 });
  const m = new TrainableTransformer(cfg, initWeights(cfg, 21));
  const rng = new RNG(3);
  const rows = [0, 1, 2].map(() => Array.from({ length: 97 }, () => rng.int(50)));
  resetTape();
  const batchLoss = m.backward(m.lossBatch(rows));
  let sum = 0;
  for (const r of rows) { resetTape(); sum += m.backward(m.loss(r.slice(0, -1), r.slice(1))); }
  assert(Math.abs(batchLoss - sum / rows.length) < 1e-5, `${batchLoss} vs ${sum / rows.length}`);
  return { batchLoss, perSample: sum / rows.length };
});

test("l2-l6 single-batch overfit", () => {
  const cfg = new Config({ dim: 32, hidden: 64, nLayers: 1, nHeads: 4, nKvHeads: 4, vocabSize: 20, maxSeq: 16 });
  const m = new TrainableTransformer(cfg, initWeights(cfg, 13));
  const data = [1, 2, 3, 4, 5, 6, 7, 8];
  resetTape();
  const first = m.backward(m.loss(data, data.slice(1)));
  const opt = new Adam(m.paramList, { lr: 0.05, totalSteps: 60 });
  let last = first;
  for (let i = 0; i < 60; i++) {
    resetTape(); m.zeroGrad();
    last = m.backward(m.loss(data, data.slice(1)));
    opt.step();
  }
  assert(last < first * 0.6, `${first} -> ${last}`);
  return { first, last };
});

test("l2-l6 Adam bias correction: first step ≈ lr", () => {
  const p = param(new Float32Array([1.0]));
  p.grad = new Float32Array([1.0]);
  const opt = new Adam([p], { lr: 0.1, totalSteps: 100 });
  const info = opt.step();
  const dw = 1.0 - p.data[0];
  assert(Math.abs(dw - 0.1) < 1e-4, `dw=${dw}`);
  const exact = 0.1 * 0.5 * (1 + Math.cos(Math.PI / 100)) / (1 + 1e-8);
  assert(Math.abs(dw - exact) < 1e-7, `dw=${dw} exact=${exact}`);
  assert(info.gnorm === 1 && info.scale === 1, `gnorm=${info.gnorm} scale=${info.scale}`);
  return { dw, exact };
});

test("l2-l6 tape isolation: old nodes are not back-propagated", () => {
  resetTape();
  const p = param(new Float32Array([1.0]));
  let called = false;
  op(new Float32Array([p.data[0]]), () => { called = true; });
  resetTape();
  const l2 = op(new Float32Array([p.data[0] * 2]), () => {});
  backward(l2);
  assert(l2.grad && !called);
});

test("device tensors: host edits of .data are seen by the next op", () => {
  resetTape();
  const X = param(new Float32Array([1, 2, 3, 4])), W = param(new Float32Array([1, 1]));
  const y1 = matmulT(X, W, 2, 2, 1).data;
  X.data[0] = 10;
  const y2 = matmulT(X, W, 2, 2, 1).data;
  assert(y1[0] === 3 && y2[0] === 12 && y2[1] === 7, `${y1} ${y2}`);
});

test("gradients accumulate across backward calls until zeroGrad", () => {
  const W = param(new Float32Array([1, 2, 3]));
  const x = leaf(new Float32Array([1, 1, 1]));
  const t = [1];
  for (let k = 0; k < 2; k++) { resetTape(); backward(weightedSum(linear(W, x, 1, 3), t)); }
  const g = Array.from(W.grad);
  assert(g.join() === "2,2,2", `grad ${g}`);
  W.zeroGrad();
  assert(Array.from(W.grad).join() === "0,0,0");
});

test("matmul (non-transposed) forward and grads", () => {
  resetTape();
  const rng = new RNG(9);
  const M = 3, K = 4, N = 5;
  const X = param(randArr(M * K, rng)), B = param(randArr(K * N, rng));
  const t = randArr(M * N, rng);
  const Y = matmul(X, B, M, K, N);
  const y = Y.data, xd = X.data, bd = B.data;
  for (let m = 0; m < M; m++) for (let n = 0; n < N; n++) {
    let s = 0; for (let k = 0; k < K; k++) s += xd[m * K + k] * bd[k * N + n];
    assert(Math.abs(y[m * N + n] - s) < 1e-5, "matmul value");
  }
  const r = numGrad(() => { resetTape(); return weightedSum(matmul(X, B, M, K, N), t); }, { X, B });
  assert(r.maxRelErr < 2e-3, JSON.stringify(r));
  return r;
});

// The two fusions of TrainableTransformer._forward must equal the unfused
// reference sequence exactly (values and gradients, bit for bit).
function sameBits(a, b, what) {
  assert(a.length === b.length, `${what}: length ${a.length} vs ${b.length}`);
  for (let i = 0; i < a.length; i++) {
    if (!(a[i] === b[i] || (a[i] !== a[i] && b[i] !== b[i]))) throw new Error(`${what}[${i}]: ${a[i]} vs ${b[i]}`);
  }
}

test("qkvRope == sliceCols×3 + ropeRows×2 (values, grads; q-only and k-only grads)", () => {
  const rows = 40, T = 20, nH = 4, nKV = 2, dH = 8, W = (nH + 2 * nKV) * dH, qD = nH * dH, kvD = nKV * dH;
  const rng = new RNG(31);
  const base = randArr(rows * W, rng);
  const wq = randArr(rows * qD, rng), wk = randArr(rows * kvD, rng), wv = randArr(rows * kvD, rng);
  const run = (fused, use) => {
    resetTape();
    const qkv = param(Float32Array.from(base));
    let q, k, v;
    if (fused) [q, k, v] = qkvRope(qkv, rows, nH, nKV, dH, 3, 5e5, T);
    else {
      q = ropeRows(sliceCols(qkv, rows, W, 0, qD), rows, nH, dH, 3, 5e5, T);
      k = ropeRows(sliceCols(qkv, rows, W, qD, kvD), rows, nKV, dH, 3, 5e5, T);
      v = sliceCols(qkv, rows, W, qD + kvD, kvD);
    }
    const parts = [];
    if (use.includes("q")) parts.push(weightedSum(q, wq));
    if (use.includes("k")) parts.push(weightedSum(k, wk));
    if (use.includes("v")) parts.push(weightedSum(v, wv));
    let L = parts[0];
    for (let i = 1; i < parts.length; i++) L = add(L, parts[i]);
    backward(L);
    return { q: Float32Array.from(q.data), k: Float32Array.from(k.data), v: Float32Array.from(v.data), g: Float32Array.from(qkv.grad) };
  };
  for (const use of ["qkv", "q", "k", "v"]) {
    const a = run(true, use), b = run(false, use);
    sameBits(a.q, b.q, `q (${use})`); sameBits(a.k, b.k, `k (${use})`); sameBits(a.v, b.v, `v (${use})`);
    sameBits(a.g, b.g, `qkv.grad (${use})`);
  }
});

test("qkvRopeAttention == matmulT + qkvRope + causalAttn(Batch) (values, grads)", () => {
  const rng = new RNG(34);
  // [B, T, nH, nKV, dH, D, pos0]: ragged T, GQA, B = 1 (causalAttn), dH 32 / 64 / 128
  for (const [B, T, nH, nKV, dH, D, pos0] of [[2, 100, 4, 2, 32, 64, 0], [1, 70, 4, 1, 64, 96, 3], [2, 40, 2, 2, 128, 64, 0]]) {
    const rows = B * T, W = (nH + 2 * nKV) * dH;
    const xd = randArr(rows * D, rng), wd = randArr(W * D, rng, 0.1), t = randArr(rows * nH * dH, rng);
    const run = (fused) => {
      resetTape();
      const xn = param(Float32Array.from(xd)), Wq = param(Float32Array.from(wd));
      let att;
      if (fused) att = qkvRopeAttention(xn, Wq, B, T, nH, nKV, dH, D, pos0, 1e4, T);
      else {
        const qkv = matmulT(xn, Wq, rows, D, W);
        const [q, k, v] = qkvRope(qkv, rows, nH, nKV, dH, pos0, 1e4, T);
        att = B === 1 ? causalAttn(q, k, v, T, nH, nKV, dH) : causalAttnBatch(q, k, v, B, T, nH, nKV, dH);
      }
      backward(weightedSum(att, t));
      return [att.data, xn.grad, Wq.grad].map((z) => Float32Array.from(z));
    };
    const f = run(true), u = run(false);
    ["att", "xn.grad", "Wqkv.grad"].forEach((nm, i) => sameBits(f[i], u[i], `${nm} B${B} T${T} dH${dH}`));
  }
  resetTape();
  assert(qkvRopeAttention(leaf(new Float32Array(4 * 8)), leaf(new Float32Array(64 * 8)), 1, 4, 2, 1, 16, 8, 0) === null,
    "dH 16 has no fused path");
});

test("crossEntropyMeanFused == crossEntropyMean (seeded loss, a combined loss, an existing gradient)", () => {
  const rng = new RNG(35);
  const T = 37, V = 1000;
  const ld = randArr(T * V, rng, 2);
  const tg = Array.from({ length: T }, () => Math.floor(rng.next() * V));
  const run = (fused, mode) => {
    resetTape();
    const x = param(Float32Array.from(ld));
    if (mode === "existing") x.grad = new Float32Array(T * V).fill(0.25);
    const ce = (fused ? crossEntropyMeanFused : crossEntropyMean)(x, tg, T, V);
    const loss = mode === "combined" ? add(ce, ce) : ce;
    backward(loss);
    return [Float32Array.from(ce.data), Float32Array.from(x.grad)];
  };
  for (const mode of ["seeded", "combined", "existing"]) {
    const f = run(true, mode), u = run(false, mode);
    sameBits(f[0], u[0], `loss (${mode})`);
    sameBits(f[1], u[1], `logits.grad (${mode})`);
  }
});

test("matmulTResid == add(x, matmulT(a, W)) (values, grads)", () => {
  const rng = new RNG(32);
  for (const [M, K, N] of [[5, 7, 3], [130, 96, 40]]) {
    const xd = randArr(M * N, rng), ad = randArr(M * K, rng), wd = randArr(N * K, rng), t = randArr(M * N, rng);
    const run = (fused) => {
      resetTape();
      const x = param(Float32Array.from(xd)), a = param(Float32Array.from(ad)), W = param(Float32Array.from(wd));
      const y = fused ? matmulTResid(x, a, W, M, K, N) : add(x, matmulT(a, W, M, K, N));
      backward(weightedSum(y, t));
      return [y.data, x.grad, a.grad, W.grad].map((z) => Float32Array.from(z));
    };
    const f = run(true), u = run(false);
    ["y", "x.grad", "a.grad", "W.grad"].forEach((nm, i) => sameBits(f[i], u[i], `${nm} ${M}x${K}x${N}`));
  }
});

function closeTo(a, b, tol, what) {
  let m = 0, d = 0;
  for (let i = 0; i < a.length; i++) { m = Math.max(m, Math.abs(b[i])); d = Math.max(d, Math.abs(a[i] - b[i])); }
  assert(d <= tol * Math.max(m, 1e-30), `${what}: max|diff| ${d} vs max|ref| ${m}`);
}

test("swigluGateUp (packed [gate; up]) == matmulT×2 + swigluRows; unpacked falls back", () => {
  const T = 96, D = 64, H = 128;
  const rng = new RNG(33);
  const xd = randArr(T * D, rng), gd = randArr(H * D, rng, 0.1), ud = randArr(H * D, rng, 0.1), t = randArr(T * H, rng);
  const run = (mode) => {
    resetTape();
    const x = param(Float32Array.from(xd)), Wg = param(Float32Array.from(gd)), Wu = param(Float32Array.from(ud));
    if (mode !== "unfused") packPair(Wg, Wu);
    if (mode === "stale") Wu.grad = new Float32Array(H * D).fill(0.5);  // only one half has a gradient: fallback
    const y = mode === "unfused" ? swigluRows(matmulT(x, Wg, T, D, H), matmulT(x, Wu, T, D, H), T, H)
      : swigluGateUp(x, Wg, Wu, T, D, H);
    backward(weightedSum(y, t));
    return [y.data, x.grad, Wg.grad, Wu.grad].map((z) => Float32Array.from(z));
  };
  const f = run("fused"), u = run("unfused"), st = run("stale");
  sameBits(f[0], u[0], "act");  // each output is the same dot product and the same SwiGLU arithmetic
  closeTo(f[1], u[1], 1e-6, "x.grad");   // one K = 2H GEMM vs two accumulated GEMMs
  closeTo(f[2], u[2], 1e-6, "Wg.grad");
  closeTo(f[3], u[3], 1e-6, "Wu.grad");
  sameBits(st[0], u[0], "act (fallback)");
  closeTo(st[2], u[2], 1e-6, "Wg.grad (fallback)");
  const wu = Float32Array.from(u[3], (v) => v + 0.5);
  closeTo(st[3], wu, 1e-6, "Wu.grad accumulated onto 0.5 (fallback)");
});

test("a model used twice in one backward pass (deferred weight gradients on one output) == two passes", () => {
  // Both losses reach every weight twice: the deferred dW GEMM jobs and the
  // deferred norm column sums each hold two jobs on one gradient, which
  // must apply in order (the second accumulating onto the first).
  const cfg = new Config({ dim: 64, hidden: 128, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 40, maxSeq: 32 });
  const w = initWeights(cfg, 77);
  const m = new TrainableTransformer(cfg, w);
  const rng = new RNG(3);
  const seqA = [], seqB = [];
  for (let i = 0; i < 2; i++) {
    const a = [], b = [];
    for (let t = 0; t < 17; t++) { a.push(rng.int(40)); b.push(rng.int(40)); }
    seqA.push(a); seqB.push(b);
  }
  resetTape(); m.zeroGrad();
  backward(add(m.lossBatch(seqA), m.lossBatch(seqB)));
  const once = m.paramList.map((p) => Float32Array.from(p.grad));
  m.zeroGrad();
  resetTape(); backward(m.lossBatch(seqA));
  resetTape(); backward(m.lossBatch(seqB));
  const twice = m.paramList.map((p) => Float32Array.from(p.grad));
  let worst = 0;
  for (let k = 0; k < once.length; k++) {
    let gmax = 1e-12;
    for (let i = 0; i < twice[k].length; i++) gmax = Math.max(gmax, Math.abs(twice[k][i]));
    for (let i = 0; i < once[k].length; i++) worst = Math.max(worst, Math.abs(once[k][i] - twice[k][i]) / gmax);
  }
  assert(worst < 1e-5, `max relative difference ${worst}`);
  return { maxRel: worst };
});

test("a deferred weight gradient that another op also writes later in the tape walk == deferral off", () => {
  // Regularizers on a norm weight (deferred column sum), a matmul weight
  // (deferred dW GEMM) and the packed gate weight (deferred pair GEMM) are
  // recorded before the model's forward, so their backward runs after the
  // model's and accumulates onto gradients whose deferred jobs are queued.
  const cfg = new Config({ dim: 64, hidden: 128, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 40, maxSeq: 32 });
  const rng = new RNG(5);
  const seqs = [];
  for (let i = 0; i < 2; i++) { const a = []; for (let t = 0; t < 17; t++) a.push(rng.int(40)); seqs.push(a); }
  const run1 = (defer) => {
    const m = new TrainableTransformer(cfg, initWeights(cfg, 91));
    if (!defer) for (const p of m.paramList) p._deferGrad = false;
    const ps = m.params;
    const targets = [ps.ln_f, ps.layers[0].wo, ps.layers[1].ffn_gate, ps.layers[1].ln2];
    const wts = targets.map((p) => randArr(p.n, new RNG(p.n), 0.5));
    resetTape(); m.zeroGrad();
    let reg = weightedSum(targets[0], wts[0]);
    for (let k = 1; k < targets.length; k++) reg = add(reg, weightedSum(targets[k], wts[k]));
    backward(add(reg, m.lossBatch(seqs)));
    return m.paramList.map((p) => Float32Array.from(p.grad));
  };
  const on = run1(true), off = run1(false);
  let worst = 0;
  for (let k = 0; k < on.length; k++) {
    let gmax = 1e-12;
    for (let i = 0; i < off[k].length; i++) gmax = Math.max(gmax, Math.abs(off[k][i]));
    for (let i = 0; i < on[k].length; i++) worst = Math.max(worst, Math.abs(on[k][i] - off[k][i]) / gmax);
  }
  assert(worst < 1e-5, `max relative difference ${worst}`);
  return { maxRel: worst };
});

test("shape errors throw instead of launching", () => {
  let threw = 0;
  try { matmulT(leaf([1, 2, 3]), leaf([1, 2]), 1, 2, 1); } catch (e) { threw++; }
  try { sliceCols(leaf([1, 2, 3, 4]), 2, 2, 1, 2); } catch (e) { threw++; }
  try { causalAttn(leaf(new Float32Array(5 * 8)), leaf(new Float32Array(2 * 8)), leaf(new Float32Array(2 * 8)), 1, 5, 2, 8); } catch (e) { threw++; }
  try { qkvRope(leaf(new Float32Array(4 * 24)), 4, 2, 1, 7, 0); } catch (e) { threw++; }
  try { matmulTResid(leaf([1, 2]), leaf([1, 2]), leaf([1, 2]), 1, 2, 1); } catch (e) { threw++; }
  assert(threw === 5, `threw ${threw}`);
});

run();
