// Runs the TrainableTransformer on the GPU and dumps what the parity tests
// compare against the oracle:
//   node dump_step.mjs <outdir> '<json spec>'
// spec: {dim, hidden, nLayers, nHeads, nKvHeads, vocab, normEps, ropeTheta,
//        B, T, initSeed, idsSeed, untied, mode: "step" | "forward" | "steps" | "loop",
//        lr, totalSteps, wd, clip, ids?, nsteps?, exportTo?, dataLen?, logitsEvery?}
// Files: manifest.json + raw little-endian .bin arrays.
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
const model = new TrainableTransformer(cfg, w);
dump("params0", concat(model.paramList.map((p) => Float32Array.from(p.data))));

const B = spec.B, T = spec.T;
if (spec.mode !== "loop") {
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
if (spec.mode === "loop") {
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
    dump("grads", concat(model.paramList.map((p) => Float32Array.from(p.grad || new Float32Array(p.n)))));
    dump("adam_info", new Float64Array([res.lr, res.gnorm, res.scale]));
    dump("params1", concat(model.paramList.map((p) => Float32Array.from(p.data))));
    dump("m1", concat(opt.m));
    dump("v1", concat(opt.v));
  } finally {
    loop.close();
  }
}
writeFileSync(join(out, "manifest.json"), JSON.stringify(manifest));
console.log(JSON.stringify({ ok: true, params: model.countParams() }));
