// The vector-level autograd ops (mul, siluAD, dotAD, scaleAD, ropeNode,
// softmaxVec: autograd.js:70-190), the single-row attention helpers
// (attentionDecode / attentionNaive / flashAttention: attention.js:31-126)
// and rmsnormInto (nn.js:42-44) through the public API, on the device.
// The kernels themselves are compared with the oracle in
// tests/test_gpu_vector.py; this file checks the host side: values written
// back into the caller's arrays, Node and tape behaviour, gradients that
// accumulate, a tensor used twice, central-difference gradient checks
// (verify.js:141-162), and the reference's own attention tests
// (l3-l5.test.js:174-216, verify.js:378-414) with their thresholds.
import { test, assert, run } from "./harness.mjs";
import {
  RNG, resetTape, backward, gradCheck, param, leaf, mul, siluAD, dotAD, scaleAD, ropeNode, softmaxVec,
  attentionDecode, attentionNaive, flashAttention, KVCache, rmsnormInto, maxAbsErr, add, noGrad,
} from "../../forge-llm_amd/src/index.js";

const randArr = (n, rng, s = 1) => { const a = new Float32Array(n); for (let i = 0; i < n; i++) a[i] = rng.normal() * s; return a; };
const f = Math.fround;

test("mul / scaleAD / dotAD forward values (fp32 of the fp64 expression)", () => {
  resetTape();
  const rng = new RNG(21);
  const a = randArr(300, rng), b = randArr(300, rng);
  const A = leaf(a), B = leaf(b), S = leaf(new Float32Array([0.75]));
  const m = mul(A, B).data, ms = mul(A, S).data, sc = scaleAD(A, -0.3).data, d = dotAD(A, B).data;
  let dd = 0;
  for (let i = 0; i < 300; i++) {
    assert(m[i] === f(a[i] * b[i]), `mul[${i}]`);
    assert(ms[i] === f(a[i] * 0.75), `mul scalar[${i}]`);
    assert(sc[i] === f(-0.3 * a[i]), `scale[${i}]`);
    dd += a[i] * b[i];
  }
  assert(d.length === 1 && d[0] === f(dd), `dot ${d[0]} vs ${f(dd)}`);
  return { dot: d[0] };
});

test("mul backward: elementwise and broadcast-scalar gradients, x·x", () => {
  resetTape();
  const rng = new RNG(22);
  const a = randArr(50, rng), b = randArr(50, rng);
  const A = param(a), B = param(b), S = param(new Float32Array([1.5]));
  const L = dotAD(add(mul(A, B), mul(A, S)), leaf(new Float32Array(50).fill(1)));
  backward(L);
  const ga = A.grad, gb = B.grad, gs = S.grad;
  let sum = 0;
  for (let i = 0; i < 50; i++) {
    assert(Math.abs(ga[i] - (b[i] + 1.5)) < 1e-5, `ga[${i}]`);
    assert(Math.abs(gb[i] - a[i]) < 1e-6, `gb[${i}]`);
    sum += a[i];
  }
  assert(Math.abs(gs[0] - sum) < 1e-4, `gs ${gs[0]} vs ${sum}`);
  // a tensor used twice in one op: d(Σ x²)/dx = 2x
  resetTape();
  const X = param(a);
  backward(dotAD(mul(X, X), leaf(new Float32Array(50).fill(1))));
  for (let i = 0; i < 50; i++) assert(Math.abs(X.grad[i] - 2 * a[i]) < 1e-5, `2x[${i}]`);
  resetTape();
  const Y = param(a);
  backward(dotAD(Y, Y));
  for (let i = 0; i < 50; i++) assert(Math.abs(Y.grad[i] - 2 * a[i]) < 1e-5, `dot 2x[${i}]`);
  return { gs: gs[0] };
});

test("gradCheck of a chain of the vector ops < 1e-2", () => {
  const rng = new RNG(23);
  const d = 16;
  const x = param(randArr(d, rng, 0.8)), w = param(randArr(d, rng, 0.5)), y = param(randArr(d, rng));
  const cos = new Float32Array(d / 2), sin = new Float32Array(d / 2);
  for (let i = 0; i < d / 2; i++) { const t = 3 * Math.pow(10000, -2 * i / d); cos[i] = Math.cos(t); sin[i] = Math.sin(t); }
  const lossFn = () => {
    resetTape();
    const h = softmaxVec(mul(siluAD(x), w));
    const r = ropeNode(scaleAD(y, 0.5), cos, sin, d);
    return dotAD(h, r);
  };
  const gc = gradCheck(lossFn, { x, w, y });
  assert(gc.maxRelErr < 1e-2, `maxRelErr=${gc.maxRelErr} @ ${gc.at}`);
  return gc;
});

test("ropeNode zeroes the entries past dHead, softmaxVec sums to one", () => {
  resetTape();
  const rng = new RNG(24);
  const x = leaf(randArr(12, rng));
  const out = ropeNode(x, [1, 0, 0.6], [0, 1, 0.8], 6).data;
  const xd = x.data;
  assert(out[0] === xd[0] && out[1] === xd[1], "identity pair");
  assert(out[2] === f(-xd[3]) && out[3] === xd[2], "quarter turn");
  for (let i = 6; i < 12; i++) assert(out[i] === 0, `zero[${i}]`);
  const p = softmaxVec(leaf(randArr(1000, rng, 3))).data;
  let s = 0;
  for (let i = 0; i < p.length; i++) s += p[i];
  assert(Math.abs(s - 1) < 1e-5, `sum ${s}`);
  return { sum: s };
});

test("outside the tape (noGrad) the ops return values and keep nothing for a backward", () => {
  resetTape();
  const rng = new RNG(26);
  const a = randArr(64, rng);
  const X = leaf(a);
  const out = noGrad(() => ({ s: siluAD(X).data, p: softmaxVec(X).data, r: ropeNode(X, [0.6], [0.8], 2).data }));
  for (let i = 0; i < 64; i++) {
    const sg = f(1 / (1 + Math.exp(-a[i])));
    assert(Math.abs(out.s[i] - f(a[i] * sg)) <= 1.2e-7 * Math.max(1, Math.abs(out.s[i])), `silu[${i}]`);
  }
  let s = 0;
  for (let i = 0; i < 64; i++) s += out.p[i];
  assert(Math.abs(s - 1) < 1e-6, `softmax sum ${s}`);
  assert(out.r[0] === f(a[0] * 0.6 - a[1] * 0.8) && out.r[2] === 0, "rope");
  return { sum: s };
});

// ── single-row attention (the reference's tests) ──
test("flashAttention == attentionNaive (l3-l5.test.js:174-185) < 1e-4", () => {
  const n = 64, d = 16, rng = new RNG(8);
  const q = randArr(d, rng);
  const K = new Float32Array(n * d), V = new Float32Array(n * d);
  for (let i = 0; i < n * d; i++) { K[i] = rng.normal(); V[i] = rng.normal(); }
  const o1 = new Float32Array(d), o2 = new Float32Array(d), o3 = new Float32Array(d);
  flashAttention(o1, q, K, V, n, d, 1 / Math.sqrt(d), true, n - 1, 0);
  attentionNaive(o2, q, K, V, n, d, 1 / Math.sqrt(d), true, n - 1, 0);
  attentionDecode(o3, q, K, V, n, d, 1 / Math.sqrt(d), true, n - 1, 0);
  assert(maxAbsErr(o1, o2) < 1e-4, `flash/naive ${maxAbsErr(o1, o2)}`);
  assert(maxAbsErr(o3, o2) < 1e-4, `decode/naive ${maxAbsErr(o3, o2)}`);
  return { flash: maxAbsErr(o1, o2), decode: maxAbsErr(o3, o2) };
});

test("causal mask: keys after qOff take no part (l3-l5.test.js:187-200) < 1e-5", () => {
  const n = 16, d = 8, rng = new RNG(9);
  const q = randArr(d, rng);
  const K = new Float32Array(n * d), V = new Float32Array(n * d);
  for (let i = 0; i < n * d; i++) { K[i] = rng.normal(); V[i] = rng.normal(); }
  const pos = 5, o = new Float32Array(d), oRef = new Float32Array(d);
  flashAttention(o, q, K, V, n, d, 1 / Math.sqrt(d), true, pos, 0);
  attentionNaive(oRef, q, K, V, pos + 1, d, 1 / Math.sqrt(d), true, pos, 0);
  assert(maxAbsErr(o, oRef) < 1e-5, `maxErr ${maxAbsErr(o, oRef)}`);
  // the decode variant's optional score buffer holds -Infinity past qOff
  const s = new Float32Array(n), o2 = new Float32Array(d);
  attentionDecode(o2, q, K, V, n, d, 1 / Math.sqrt(d), true, pos, 0, s);
  for (let j = pos + 1; j < n; j++) assert(s[j] === -Infinity, `s[${j}]=${s[j]}`);
  let sd = 0;
  for (let i = 0; i < d; i++) sd += q[i] * K[2 * d + i];
  assert(s[2] === f(sd * (1 / Math.sqrt(d))), `score ${s[2]}`);
  assert(maxAbsErr(o2, oRef) < 1e-5, `decode ${maxAbsErr(o2, oRef)}`);
  return { maxErr: maxAbsErr(o, oRef) };
});

test("KVCache views == full arrays (l3-l5.test.js:202-216) < 1e-5; kOff selects the keys", () => {
  const n = 32, d = 8, rng = new RNG(10);
  const K = new Float32Array(n * d), V = new Float32Array(n * d);
  for (let i = 0; i < n * d; i++) { K[i] = rng.normal(); V[i] = rng.normal(); }
  const q = randArr(d, rng);
  const cache = new KVCache(1, n, d);
  for (let p = 0; p < n; p++) cache.put(0, p, K.subarray(p * d, p * d + d), V.subarray(p * d, p * d + d));
  const oCache = new Float32Array(d), oFull = new Float32Array(d);
  flashAttention(oCache, q, cache.kView(0, n), cache.vView(0, n), n, d, 1 / Math.sqrt(d), true, n - 1, 0);
  flashAttention(oFull, q, K, V, n, d, 1 / Math.sqrt(d), true, n - 1, 0);
  cache.free();
  assert(maxAbsErr(oCache, oFull) < 1e-5, `cache ${maxAbsErr(oCache, oFull)}`);
  // kOff: the last 10 keys of K as their own sequence
  const oOff = new Float32Array(d), oSub = new Float32Array(d);
  attentionNaive(oOff, q, K, V, 10, d, 0.3, false, 0, (n - 10) * d);
  attentionNaive(oSub, q, K.slice((n - 10) * d), V.slice((n - 10) * d), 10, d, 0.3, false, 0, 0);
  assert(maxAbsErr(oOff, oSub) === 0, "kOff");
  // a plain-array out receives the values too
  const plain = new Array(d).fill(7);
  flashAttention(plain, q, K, V, n, d, 1 / Math.sqrt(d), true, n - 1, 0);
  assert(maxAbsErr(Float32Array.from(plain), oFull) === 0, "array out");
  return { maxErr: maxAbsErr(oCache, oFull) };
});

test("rmsnormInto: x·w / sqrt(rms² + eps) written into out", () => {
  const rng = new RNG(25);
  const n = 300, x = randArr(n, rng, 2), w = randArr(n, rng);
  const out = new Float32Array(n + 3).fill(5);
  rmsnormInto(out, x, w, n, 1e-5);
  let s = 0;
  for (let i = 0; i < n; i++) s += x[i] * x[i];
  const r = Math.sqrt(s / n), ss = 1 / Math.sqrt(r * r + 1e-5);
  for (let i = 0; i < n; i++) assert(out[i] === f(x[i] * ss * w[i]), `out[${i}]`);
  for (let i = n; i < n + 3; i++) assert(out[i] === 5, "past n untouched");
  return { ss };
});

run();
