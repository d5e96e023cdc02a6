// Runs the TrainableTransformer on the GPU and dumps what the parity tests
// compare against the oracle:
//   node dump_step.mjs <outdir> '<json spec>'
// spec: {dim, hidden, nLayers, nHeads, nKvHeads, vocab, normEps, ropeTheta,
//        B, T, initSeed, idsSeed, untied, mode: "step" | "forward" | "steps" | "loop" | "loop_sampled",
//        lr, totalSteps, wd, clip, ids?, nsteps?, exportTo?, dataLen?, logitsEvery?, bigRows?, chunkEvery?}
// Files: manifest.json + raw little-endian .bin arrays.
//
// "loop_sampled" is "loop" at widths whose [V, d] tensors (embedding, LM
// head: 525M floats at the Llama-3-8B widths) are too large to dump whole:
// see sampleOf below for what each array holds.
import { writeFileSync, mkdirSync } from "fs";
import { join } from "path";
import {
  RNG, Config, TrainableTransformer, initWeights, resetTape, Adam, crossEntropyMean, DeviceTrainLoop, tape, hip,
  exportGGUF,
} from "../../forge-llm_amd/src/index.js";

const out = process.argv[2];
const spec = JSON.parse(process.argv[3]);
mkdirSync(out, { recursive: true });
const manifest = {};
function dump(name, arr) {
  const file = `${name}.bin`;
  writeFileSync(join(out, file), Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));
  manifest[name] = { file, dtype: arr instanceof Float32Array ? "f4" : arr instanceof Float64Array ? "f8" : "i4", n: arr.length };
}
// spec.progress: a line on stderr as each stage ends (long runs)
const t00 = Date.now();
const stage = (what) => { if (spec.progress) console.error(`[dump_step ${((Date.now() - t00) / 1e3).toFixed(1)} s] ${what}`); };
function concat(arrs) {
  let n = 0; for (const a of arrs) n += a.length;
  const r = new Float32Array(n); let o = 0;
  for (const a of arrs) { r.set(a, o); o += a.length; }
  return r;
}

const cfg = new Config({
  dim: spec.dim, hidden: spec.hidden, nLayers: spec.nLayers, nHeads: spec.nHeads, nKvHeads: spec.nKvHeads,
  vocabSize: spec.vocab, maxSeq: Math.max(64, spec.T), normEps: spec.normEps || 1e-5, ropeTheta: spec.ropeTheta || 10000,
});
const w = initWeights(cfg, spec.initSeed);
if (spec.untied) {
  // untied LM head: drawn after the layers from the same stream (N(0, 0.02))
  const rng = new RNG(spec.initSeed);
  let skip = cfg.vocabSize * cfg.dim + cfg.nLayers * (cfg.qkvOut * cfg.dim + cfg.dim * cfg.dim + 3 * cfg.hidden * cfg.dim);
  while (skip-- > 0) rng.normal();
  const a = new Float32Array(cfg.vocabSize * cfg.dim);
  for (let i = 0; i < a.length; i++) a[i] = rng.normal() * 0.02;
  w.wcls = a;
}
stage("weights drawn");
const model = new TrainableTransformer(cfg, w);
const sampled = spec.mode === "loop_sampled";
// The sampled form of a parameter-sized array (mode "loop_sampled"): a tensor
// of V*d floats keeps the rows spec.bigRows (rows of d floats); with `whole`
// every other tensor is kept whole, else a tensor of more than 2^20 floats
// keeps every spec.chunkEvery-th run of 4096 floats (runs 0, k, 2k, ...).
const CHUNK = 4096;
function sampleOf(p, arr, whole) {
  if (!sampled) return arr;
  const D = cfg.dim;
  if (p.n === cfg.vocabSize * D) {
    const out = new Float32Array(spec.bigRows.length * D);
    spec.bigRows.forEach((r, k) => out.set(arr.subarray(r * D, (r + 1) * D), k * D));
    return out;
  }
  if (whole || p.n <= (1 << 20)) return arr;
  const k = spec.chunkEvery, nch = Math.ceil(p.n / CHUNK), keep = [];
  for (let c = 0; c < nch; c += k) keep.push(arr.subarray(c * CHUNK, Math.min(p.n, (c + 1) * CHUNK)));
  return concat(keep);
}
dump("params0", concat(model.paramList.map((p) => (sampled ? sampleOf(p, p._download(), false) : Float32Array.from(p.data)))));

const B = spec.B, T = spec.T;
if (spec.mode !== "loop" && !sampled) {
let rows;
if (spec.ids) rows = spec.ids;
else {
  const r = new RNG(spec.idsSeed);
  rows = [];
  for (let b = 0; b < B; b++) { const row = []; for (let i = 0; i <= T; i++) row.push(r.int(cfg.vocabSize)); rows.push(row); }
}
const ids = new Int32Array(B * T), tg = new Int32Array(B * T);
for (let b = 0; b < B; b++) for (let i = 0; i < T; i++) { ids[b * T + i] = rows[b][i]; tg[b * T + i] = rows[b][i + 1]; }
dump("ids", ids);
dump("targets", tg);

resetTape();
model.zeroGrad();
const logits = B === 1 ? model.forward(Array.from(ids)) : model._forward(Array.from(ids), B, T, 0);
dump("logits", Float32Array.from(logits.data));
if (spec.mode === "step") {
  const lossNode = crossEntropyMean(logits, Array.from(tg), B * T, cfg.vocabSize);
  const loss = model.backward(lossNode);
  dump("loss", new Float32Array([loss]));
  dump("grads", concat(model.paramList.map((p) => Float32Array.from(p.grad || new Float32Array(p.n)))));
  const opt = new Adam(model.paramList, { lr: spec.lr, totalSteps: spec.totalSteps, clip: spec.clip, wd: spec.wd });
  const info = opt.step();
  dump("adam_info", new Float64Array([info.lr, info.gnorm, info.scale]));
  dump("params1", concat(model.paramList.map((p) => Float32Array.from(p.data))));
  dump("m1", concat(opt.m));
  dump("v1", concat(opt.v));
}
if (spec.mode === "steps") {
  // several train() steps, a fresh batch per step (drawn from idsSeed after the first)
  const opt = new Adam(model.paramList, { lr: spec.lr, totalSteps: spec.totalSteps, clip: spec.clip, wd: spec.wd });
  const r = new RNG(spec.idsSeed + 1000);
  const allIds = [], allTg = [], losses = [], gnorms = [];
  for (let s = 0; s < spec.nsteps; s++) {
    const bIds = new Int32Array(B * T), bTg = new Int32Array(B * T);
    const rws = [];
    for (let b = 0; b < B; b++) {
      const row = []; for (let i = 0; i <= T; i++) row.push(r.int(cfg.vocabSize));
      rws.push(row);
      for (let i = 0; i < T; i++) { bIds[b * T + i] = row[i]; bTg[b * T + i] = row[i + 1]; }
    }
    resetTape();
    model.zeroGrad();
    losses.push(model.backward(model.lossBatch(rws)));
    gnorms.push(opt.step().gnorm);
    allIds.push(bIds); allTg.push(bTg);
  }
  const cat = (xs) => { const o = new Int32Array(xs.length * B * T); xs.forEach((x, i) => o.set(x, i * B * T)); return o; };
  dump("step_ids", cat(allIds));
  dump("step_targets", cat(allTg));
  dump("step_losses", new Float64Array(losses));
  dump("step_gnorms", new Float64Array(gnorms));
  dump("params_final", concat(model.paramList.map((p) => Float32Array.from(p.data))));
  if (spec.exportTo) {
    // the trained weights as the reference's llama GGUF export (engine.js:126-228)
    writeFileSync(spec.exportTo, exportGGUF(model.exportWeights(), cfg, null, 0, "forge-trained"));
  }
}
}
if (spec.mode === "loop" || sampled) {
  // One step of train()'s device-resident loop (DeviceTrainLoop, op by op):
  // the windows cut on the device, the fused CE forward + seed-1 backward,
  // the device-sorted embedding backward, the grouped weight-gradient GEMM
  // and Adam with {lr, bc1, bc2} read from device memory — the kernels of
  // the benchmark's step.  Token data and window starts come from
  // RNG(idsSeed) (data first, then the B starts, rng.int as train() draws them).
  const r = new RNG(spec.idsSeed);
  const n = spec.dataLen;
  const data = new Array(n);
  for (let i = 0; i < n; i++) data[i] = r.int(cfg.vocabSize);
  const starts = [];
  for (let b = 0; b < B; b++) starts.push(r.int(Math.max(1, n - T - 1)));
  dump("data", Int32Array.from(data));
  dump("starts", Int32Array.from(starts));
  const opt = new Adam(model.paramList, { lr: spec.lr, totalSteps: spec.totalSteps, clip: spec.clip, wd: spec.wd });
  const loop = new DeviceTrainLoop(model, opt, data, B, T, { graph: false });
  try {
    loop.step(starts);
    const res = loop.read();
    stage("step done");
    const a = hip();
    const gi = new Int32Array(B * T), gt = new Int32Array(B * T);
    a.d2h(loop.ids.h, gi);
    a.d2h(loop.tgt.h, gt);
    dump("ids", gi);
    dump("targets", gt);
    // the logits are the value the loss node was computed from: the node
    // recorded just before it
    const nodes = tape().nodes;
    const lg = nodes[nodes.indexOf(loop.loss) - 1];
    if (!lg || lg.n !== B * T * cfg.vocabSize) throw new Error("logits node not found on the tape");
    // every `logitsEvery`-th row, each downloaded from its byte offset
    const every = spec.logitsEvery || 1, V = cfg.vocabSize;
    const rowsOut = new Float32Array(Math.ceil((B * T) / every) * V);
    const dev = lg._devData();
    for (let i = 0, k = 0; i < B * T; i += every, k++) a.d2h(dev, rowsOut.subarray(k * V, (k + 1) * V), i * V * 4);
    dump("logits", rowsOut);
    dump("loss", new Float32Array([res.loss]));
    if (!sampled) {
      dump("grads", concat(model.paramList.map((p) => Float32Array.from(p.grad || new Float32Array(p.n)))));
    } else {
      // every gradient's fp64 sum of squares over the whole tensor, the rows
      // of the embedding gradient holding a nonzero value, and the gradients
      // (the [V, d] ones at the sampled rows, the others whole)
      const gs = [], sumsq = [];
      for (const p of model.paramList) {
        const g = p.grad || new Float32Array(p.n);
        let s2 = 0;
        for (let i = 0; i < g.length; i++) s2 += g[i] * g[i];
        sumsq.push(s2);
        if (p === model.params.tok_emb) {
          const nz = [], D = cfg.dim;
          for (let r0 = 0; r0 < cfg.vocabSize; r0++) {
            for (let i = r0 * D; i < (r0 + 1) * D; i++) if (g[i] !== 0) { nz.push(r0); break; }
          }
          dump("tok_emb_grad_rows", Int32Array.from(nz));
        }
        gs.push(sampleOf(p, g, true));
      }
      dump("grad_sumsq", Float64Array.from(sumsq));
      dump("grads", concat(gs));
    }
    stage("gradients written");
    dump("adam_info", new Float64Array([res.lr, res.gnorm, res.scale]));
    dump("params1", concat(model.paramList.map((p) => sampleOf(p, sampled ? p._download() : Float32Array.from(p.data), false))));
    dump("m1", concat(opt.m.map((a, j) => sampleOf(model.paramList[j], a, false))));
    dump("v1", concat(opt.v.map((a, j) => sampleOf(model.paramList[j], a, false))));
  } finally {
    loop.close();
  }
}
stage("all written");
writeFileSync(join(out, "manifest.json"), JSON.stringify(manifest));
console.log(JSON.stringify({ ok: true, params: model.countParams() }));
