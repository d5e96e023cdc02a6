// Times full training steps of the TrainableTransformer on the GPU:
// resetTape → zeroGrad → lossBatch (embed … LM head, crossEntropyMean) →
// backward → Adam.step (global-norm clip, cosine LR, moments, update), the
// body of train() (src/L6/train.js).  Prints one JSON object.
//
//   node train_step.mjs '{"preset":"125m","steps":10,"warmup":3,"loop":"graph"}'
//
// loop "graph" (train()'s device-resident loop, DeviceTrainLoop): a token
// stream of 2^22 uniform random ids resident in device memory, B windows per
// step at RNG-drawn starts, the step replayed as one recorded HIP graph from
// the second step on; "device": the same loop issued op by op; "host": every
// step's ids drawn on the host (uniform random) and uploaded, op by op.
//
// Pass 1 (timed): `warmup` untimed steps, then `steps` steps between two
// device synchronisations.  Pass 2 (profiled): the same number of steps op
// by op with per-kernel-family HIP events on the library stream (fg_kprof),
// reported as calls / ms / algorithmic flop and bytes per family.
import {
  RNG, Config, TrainableTransformer, initWeights, resetTape, Adam, hip, DeviceTrainLoop,
} from "../src/index.js";

const PRESETS = {
  // `forge train` demo shape (vocab of the built-in corpus = 31)
  demo: { dim: 64, hidden: 128, nLayers: 2, nHeads: 4, nKvHeads: 2, vocab: 31, B: 8, T: 32, theta: 1e4, tied: true, lr: 5e-3, wd: 0.01 },
  // 125M-shaped: d768, 12 layers, 12 heads x 64, SwiGLU 2048, V 32000 untied, B8 x T1024
  "125m": { dim: 768, hidden: 2048, nLayers: 12, nHeads: 12, nKvHeads: 12, vocab: 32000, B: 8, T: 1024, theta: 1e4, tied: false, lr: 3e-4, wd: 0 },
  // Llama-3-8B-shaped slice: one layer, d4096, 32/8 heads x 128, ffn 14336, V 128256, B1 x T4096
  llama8b_slice: { dim: 4096, hidden: 14336, nLayers: 1, nHeads: 32, nKvHeads: 8, vocab: 128256, B: 1, T: 4096, theta: 5e5, tied: false, lr: 3e-4, wd: 0 },
};

const args = JSON.parse(process.argv[2] || "{}");
const P = Object.assign({}, PRESETS[args.preset || "125m"], args.override || {});
const steps = args.steps || 10, warmup = args.warmup === undefined ? 3 : args.warmup;
const loopKind = args.loop || "graph";
if (!["graph", "device", "host"].includes(loopKind)) throw new Error(`unknown loop ${loopKind}`);
const a = hip();

const cfg = new Config({
  dim: P.dim, hidden: P.hidden, nLayers: P.nLayers, nHeads: P.nHeads, nKvHeads: P.nKvHeads,
  vocabSize: P.vocab, maxSeq: P.T, normEps: 1e-5, ropeTheta: P.theta,
});
const t0 = Date.now();
const w = initWeights(cfg, 1337);
if (!P.tied) {
  const rng = new RNG(4242);
  const h = new Float32Array(cfg.vocabSize * cfg.dim);
  for (let i = 0; i < h.length; i++) h[i] = rng.normal() * 0.02;
  w.wcls = h;
}
const model = new TrainableTransformer(cfg, w);
const opt = new Adam(model.paramList, { lr: P.lr, totalSteps: 1000, clip: 1.0, wd: P.wd });
const initMs = Date.now() - t0;

const idsRng = new RNG(1);
function batch() {
  const rows = [];
  for (let b = 0; b < P.B; b++) {
    const row = new Array(P.T + 1);
    for (let i = 0; i <= P.T; i++) row[i] = idsRng.int(cfg.vocabSize);
    rows.push(row);
  }
  return rows;
}
const losses = [];
function hostStep() {
  const rows = batch();
  resetTape();
  model.zeroGrad();
  const l = model.backward(model.lossBatch(rows));
  opt.step();
  losses.push(l);
}

// device-resident token stream and window starts
let stream = null, startRng = null;
function makeLoop(graph) {
  if (stream === null) {
    stream = new Int32Array((1 << 22) + P.T + 1);
    for (let i = 0; i < stream.length; i++) stream[i] = idsRng.int(cfg.vocabSize);
    startRng = new RNG(2);
  }
  return new DeviceTrainLoop(model, opt, stream, P.B, P.T, { graph });
}
function loopStep(loop) {
  const starts = new Array(P.B);
  for (let b = 0; b < P.B; b++) starts[b] = startRng.int(stream.length - P.T - 1);
  loop.step(starts);
}

let loop = loopKind === "host" ? null : makeLoop(loopKind === "graph");
const step = () => (loop ? loopStep(loop) : hostStep());

for (let i = 0; i < warmup; i++) step();
a.sync();
const e0 = a.eventCreate(), e1 = a.eventCreate();
const h0 = process.hrtime.bigint();
a.eventRecord(e0);
for (let i = 0; i < steps; i++) step();
a.eventRecord(e1);
a.sync();
const wallMs = Number(process.hrtime.bigint() - h0) / 1e6;
const gpuMs = a.eventElapsed(e0, e1);
if (loop) { losses.push(loop.read().loss); loop.close(); }

// pass 2: per-kernel-family events (op by op: a graph replay records none)
if (loop) loop = makeLoop(false);
a.kprofReset();
a.kprofEnable(1);
const h1 = process.hrtime.bigint();
for (let i = 0; i < steps; i++) step();
a.sync();
const profWallMs = Number(process.hrtime.bigint() - h1) / 1e6;
const kernels = JSON.parse(a.kprofReport());
a.kprofEnable(0);
if (loop) { losses.push(loop.read().loss); loop.close(); }
const mem = a.memStats();

console.log(JSON.stringify({
  preset: args.preset || "125m", cfg: P, loop: loopKind, params: model.countParams(), steps, warmup,
  wall_ms: wallMs, gpu_ms: gpuMs, ms_per_step: wallMs / steps, tokens_per_step: P.B * P.T,
  profiled_ms_per_step: profWallMs / steps, kernels, init_ms: initMs,
  losses, mem_in_use: mem[0], mem_cached: mem[1],
}));
