/**
 * L2 · reverse-mode autodiff with device-resident tensors (MI355X).
 *
 * Same contract as forge-llm's src/L2/autograd.js: a module-global tape
 * (autograd.js:20-23), `Node {data, grad, _b}` (:25-34), `leaf/param/op`
 * (:36-43), `backward` walking the tape in reverse and calling each node's
 * backward only when its gradient exists (:126-133), `gradCheck` (:192-210)
 * and `Adam` with global-norm clipping, cosine schedule, L2 weight decay and
 * bias correction (:214-244).
 *
 * What changes is where the numbers live.  A Node's value and gradient live
 * in device memory; `.data` / `.grad` are getters that download on read and
 * mark the host copy as possibly modified, so host code that writes
 * `p.data[i] = v` (the gradient checks do, verify.js:152-155) is seen by the
 * next device op, which re-uploads it.  A missing gradient is allocated on
 * the device by the first op that writes it (first write, beta = 0), later
 * writers accumulate (beta = 1) — the reference's `grad ??= zeros; grad += …`.
 *
 * resetTape() releases the device memory of the previous tape's op outputs
 * (their values, gradients and saved tensors).  Outputs of at most 1024
 * elements (losses, scalars) keep a host copy; reading a larger released
 * output throws.  Leaves and params are never released by the tape.
 */
import { hip, allocF32 } from "./device.js";
import { matmulT, crossEntropyMean, rmsNorm, _addTensors } from "./tensor.js";

// ── Tape ──────────────────────────────────────────────────────────────────
let _tape = { nodes: [], enabled: true };
export function tape() { return _tape; }
export function resetTape() {
  const old = _tape.nodes;
  _tape = { nodes: [], enabled: true };
  for (let i = 0; i < old.length; i++) if (old[i]._isOp) old[i]._release();
}
export function noGrad(fn) {
  const e = _tape.enabled;
  _tape.enabled = false;
  try { return fn(); } finally { _tape.enabled = e; }
}
export function _tapeEnabled() { return _tape.enabled; }

const KEEP_ON_RELEASE = 1024;
const RELEASED = "forge-llm_amd: this tensor's device memory was released by resetTape(); read .data before resetting the tape";

/** Marker for data produced on the device (internal). */
class DeviceData {
  constructor(h, n) { this.h = h; this.n = n; }
}

export class Node {
  constructor(data, requiresGrad = true) {
    if (data instanceof DeviceData) {
      this._n = data.n; this._dev = data.h; this._host = null; this._hostValid = false; this._exposed = false;
    } else {
      const arr = data instanceof Float32Array ? data : Float32Array.from(data);
      this._n = arr.length; this._dev = null; this._host = arr; this._hostValid = true; this._exposed = true;
    }
    this._gdev = null; this._ghost = null; this._gHostValid = false; this._gExposed = false;
    this._b = null; this._bdev = null; this._saved = null;
    this._isOp = false; this._released = false; this._ticket = -1; this._bdevAlways = false; this._gZero = false;
    this._gShared = false;  // _gdev is another node's gradient, read-only (copy on write)
    this._ver = 0;  // bumped whenever the device value changes after creation (uploads, device writes)
    // Device buffer of FG_XP_PARTS floats bounding the gradient's magnitudes
    // (the GEMM operand maxima of include/forge_hip.h), set by the op that
    // wrote the whole gradient and dropped by any other gradient write.
    this._gxp = null;
    this._deferPending = false;  // a queued grouped launch still writes _gdev
    // Device buffer of 2n floats when the gradient is held as two halves
    // (the K pieces of the GEMM that wrote it): grad = first + second half,
    // summed on first use unless the consumer adds them itself.
    this._gHalves = null;
    if (requiresGrad && _tape.enabled) _tape.nodes.push(this);
  }

  get n() { return this._n; }

  get data() {
    if (!this._hostValid) {
      if (!this._dev) throw new Error(RELEASED);
      if (!this._host || this._host.length !== this._n) this._host = new Float32Array(this._n);
      const a = hip();
      if (!(this._ticket >= 0 && a.readWait(this._ticket, this._host))) a.d2h(this._dev, this._host);
      this._ticket = -1;
      this._hostValid = true;
    }
    this._exposed = true;
    return this._host;
  }

  set data(v) {
    const arr = v instanceof Float32Array ? v : Float32Array.from(v);
    if (arr.length !== this._n && this._dev) { hip().free(this._dev); this._dev = null; }
    this._n = arr.length; this._host = arr; this._hostValid = true; this._exposed = true; this._ticket = -1;
  }

  get grad() {
    this._settle();
    if (this._gdev === null && this._ghost === null) return null;
    if (this._gZero && !this._gHostValid) {
      if (!this._ghost || this._ghost.length !== this._n) this._ghost = new Float32Array(this._n);
      else this._ghost.fill(0);
      this._gHostValid = true;
    }
    if (!this._gHostValid) {
      if (!this._ghost || this._ghost.length !== this._n) this._ghost = new Float32Array(this._n);
      hip().d2h(this._gdev, this._ghost);
      this._gHostValid = true;
    }
    this._gExposed = true;
    this._seeded = false;  // the caller may edit the returned array
    return this._ghost;
  }

  set grad(v) {
    if (this._deferPending) _flushDeferred();
    this._dropGxp();
    this._seeded = false;
    this._dropHalves();
    if (v === null || v === undefined) {
      if (this._gdev && !this._gShared) hip().free(this._gdev);
      this._gdev = null; this._ghost = null; this._gHostValid = false; this._gExposed = false; this._gZero = false;
      this._gShared = false;
      return;
    }
    const arr = v instanceof Float32Array ? v : Float32Array.from(v);
    if (arr.length !== this._n) throw new Error(`grad of length ${arr.length} set on a tensor of ${this._n} elements`);
    this._ghost = arr; this._gHostValid = true; this._gExposed = true; this._gZero = false;
  }

  /** Zeroes the gradient.  A device gradient is only marked zero: the next
   *  op that writes all of it stores instead of accumulating (beta 0), and
   *  any other use fills it with zeros first. */
  zeroGrad() {
    this._dropGxp();
    this._seeded = false;
    this._settle();
    if (this._gShared) { this._gdev = null; this._gShared = false; }
    if (this._gdev) {
      this._gZero = true;
      if (this._ghost) this._ghost.fill(0);
      this._gHostValid = !!this._ghost;
      this._gExposed = false;
    } else if (this._ghost) {
      this._ghost.fill(0);
    }
  }

  // ── device protocol used by the fused ops (internal) ──
  /** Device buffer holding the current value (uploads host edits first). */
  _devData() {
    if (this._exposed || !this._dev) {
      if (!this._hostValid) throw new Error(RELEASED);
      if (!this._dev) this._dev = allocF32(this._n);
      hip().h2d(this._dev, this._host);
      this._exposed = false;
      this._ver++;
    }
    return this._dev;
  }
  /** A host copy of the current value that does not mark the host copy as
   *  edited (no re-upload at the next device use). */
  _download() {
    if (this._hostValid && !this._exposed) return Float32Array.from(this._host);
    const out = new Float32Array(this._n);
    hip().d2h(this._devData(), out);
    return out;
  }
  /** The device copy was just written by a kernel (e.g. the Adam update). */
  _deviceWrote() { this._hostValid = false; this._exposed = false; this._ticket = -1; this._ver++; }
  /** Forgets the gradient maxima (the gradient is about to change). */
  _dropGxp() { if (this._gxp) { hip().free(this._gxp); this._gxp = null; } }
  _hasGrad() { return this._gdev !== null || this._ghost !== null || this._gHalves !== null; }
  /** Takes a first gradient held as two halves (buffer of 2n floats). */
  _adoptHalves(h) {
    if (this._hasGrad()) throw new Error("_adoptHalves: the node already has a gradient");
    this._dropGxp();
    this._gHalves = h;
  }
  /** The two-halves buffer of a gradient held that way, else null. */
  _gradHalves() { return this._gHalves; }
  /** Sums a gradient held as two halves into an ordinary device gradient. */
  _settle() {
    if (this._deferPending) _flushDeferred();
    if (this._gHalves === null) return;
    const a = hip(), h = allocF32(this._n);
    a.addFwd(h, a.view(this._gHalves, 0, this._n * 4), a.view(this._gHalves, this._n * 4, this._n * 4), this._n);
    a.free(this._gHalves);
    this._gHalves = null;
    this._gdev = h; this._gShared = false; this._ghost = null;
    this._gHostValid = false; this._gExposed = false; this._gZero = false;
  }
  _dropHalves() {
    if (this._gHalves === null) return;
    hip().free(this._gHalves);
    this._gHalves = null;
  }
  /** Device gradient for reading (uploads host edits first); must exist. */
  _gradDev() {
    this._settle();
    if (this._gShared && (this._gExposed || this._gZero)) this._unshare();
    if (this._gExposed || !this._gdev) {
      this._dropGxp();
      if (!this._gdev) this._gdev = allocF32(this._n);
      hip().h2d(this._gdev, this._ghost);
      this._gExposed = false;
      this._gZero = false;
    } else if (this._gZero) {
      hip().zero(this._gdev, this._n * 4);
      this._gZero = false;
    }
    return this._gdev;
  }
  /** {h, beta} for an op that writes the whole gradient: fresh or marked zero → beta 0. */
  _gradAcc() {
    this._dropGxp();
    this._seeded = false;
    this._settle();
    this._unshare();
    if (!this._hasGrad()) {
      this._gdev = allocF32(this._n);
      this._gHostValid = false;
      return { h: this._gdev, beta: 0 };
    }
    if (this._gZero && !this._gExposed) {
      this._gZero = false;
      this._gHostValid = false;
      return { h: this._gdev, beta: 0 };
    }
    const h = this._gradDev();
    this._gHostValid = false;
    return { h, beta: 1 };
  }
  /** {h, zeroed} for ops that add into part of the gradient: zeroed when the
   *  buffer was zero-filled here (fresh, or a pending zeroGrad), so every
   *  element is 0 and such an op may write its part without reading it. */
  _gradZeroedInfo() {
    this._dropGxp();
    this._seeded = false;
    this._settle();
    this._unshare();
    const zeroed = !this._hasGrad() || (this._gdev !== null && this._gZero && !this._gExposed);
    return { h: this._gradZeroed(), zeroed };
  }
  /** Device gradient for ops that add into part of it (fresh → zero-filled). */
  _gradZeroed() {
    this._dropGxp();
    this._seeded = false;
    this._settle();
    this._unshare();
    if (!this._hasGrad()) {
      this._gdev = allocF32(this._n);
      hip().zero(this._gdev, this._n * 4);
      this._gHostValid = false;
      return this._gdev;
    }
    const h = this._gradDev();
    this._gHostValid = false;
    return h;
  }
  /** grad = ones, the seed of backward() (autograd.js:127); filled on the
   *  device for a device value, so no host upload is queued. */
  _seedGrad() {
    this._dropGxp();
    this._dropHalves();
    if (!this._dev || this._released) { this.grad = new Float32Array(this._n).fill(1); return; }
    if (!this._gdev) this._gdev = allocF32(this._n);
    hip().fillF32(this._gdev, 1, this._n);
    this._ghost = null; this._gHostValid = false; this._gExposed = false; this._gZero = false;
    this._seeded = true;  // grad is exactly the seed (an op's backward may rely on it)
  }
  /** Takes a device buffer holding this node's complete first gradient. */
  _adoptGrad(h) {
    if (this._hasGrad()) throw new Error("_adoptGrad: the node already has a gradient");
    this._dropGxp();
    this._gdev = h; this._gShared = false; this._ghost = null;
    this._gHostValid = false; this._gExposed = false; this._gZero = false;
  }
  /** This node's gradient starts equal to src's: share src's device buffer
   *  read-only (no copy).  The first op that accumulates into it writes a
   *  fresh buffer (_gradAccFrom), and any other writer copies first
   *  (_unshare), so src's gradient never changes. */
  _shareGrad(src) {
    this._dropGxp();
    this._seeded = false;
    src._settle();
    this._gdev = src._gdev; this._gShared = true; this._ghost = null;
    this._gHostValid = false; this._gExposed = false; this._gZero = false;
  }
  /** Gives a shared gradient its own buffer (a copy), before it is written. */
  _unshare() {
    if (!this._gShared) return;
    const a = hip();
    const h = allocF32(this._n);
    a.accum(h, this._gdev, this._n, 0);
    this._gdev = h; this._gShared = false;
  }
  /** {h, beta, src} for an op that writes h = src + its result (beta 1) or
   *  h = its result (beta 0, src null); a shared gradient is read from its
   *  buffer and written into a fresh one. */
  _gradAccFrom() {
    this._dropGxp();
    this._seeded = false;
    this._settle();
    if (this._gShared) {
      const src = this._gdev;
      this._gdev = allocF32(this._n); this._gShared = false; this._gHostValid = false;
      return { h: this._gdev, beta: 1, src };
    }
    const r = this._gradAcc();
    return { h: r.h, beta: r.beta, src: r.beta ? r.h : null };
  }
  /** Free device memory of an op output (small values keep a host copy). */
  _release() {
    if (this._released) return;
    this._released = true;
    this._dropGxp();
    if (this._gHalves !== null && this._n <= KEEP_ON_RELEASE) this._settle();
    this._dropHalves();
    if (this._dev) {
      if (!this._hostValid && this._n <= KEEP_ON_RELEASE) this.data;
      hip().free(this._dev);
      this._dev = null;
    }
    if (this._gdev) {
      if (!this._gHostValid && this._n <= KEEP_ON_RELEASE) this.grad;
      if (!this._gShared) hip().free(this._gdev);
      this._gdev = null; this._gShared = false;
      if (!this._gHostValid) this._ghost = null;
    }
    if (this._saved) {
      const a = hip();
      for (const h of this._saved) a.free(h);
      this._saved = null;
    }
    this._bdev = null;
  }
}

/** A Node whose value is a fresh device buffer of n fp32 (internal). */
export function _deviceNode(n) {
  const nd = new Node(new DeviceData(allocF32(n), n));
  nd._isOp = true;
  return nd;
}

export const leaf = (data) => new Node(data);
export const param = (data) => { const n = new Node(data); n.isParam = true; return n; };

/** Host-side custom op (autograd.js:39-43): `bwd(g)` receives the host gradient. */
export function op(out, bwd) {
  const n = new Node(out);
  n._b = bwd;
  n._isOp = true;
  return n;
}

// Weight gradients deferred while backward() walks the tape: the layer
// matmuls' dW GEMMs ({job, frees}) run together at its end in one grouped
// launch (fg_matmulT_bwd_w_grouped) instead of one small, K-split GEMM each.
// The RMSNorm weight gradients ({job, frees}: the column sums of their
// partial matrices) are deferred the same way and run as one grouped
// column-sum launch (fg_colsum_grouped).
// A job fixes its beta when it is queued, so any other access to a target's
// gradient before the end of backward() (another op accumulating into it, a
// read) first issues every queued job (_flushDeferred): the gradient then
// holds what the op-by-op order would have written.
let _deferred = null;
let _deferredCols = null;
let _pendingNodes = [];
function _markPending(targets) {
  for (const t of targets || []) {
    if (!t._deferPending) { t._deferPending = true; _pendingNodes.push(t); }
  }
}
function _clearPending() {
  for (const t of _pendingNodes) t._deferPending = false;
  _pendingNodes = [];
}
/** Queues gW (+)= gYᵀ·X for the end of the running backward(); false when no
 *  backward() is running (the caller computes it now).  `frees`: device
 *  buffers to release once the grouped GEMM is queued; `targets`: the Nodes
 *  whose gradient the job writes. */
export function _deferWeightGrad(job, frees, targets) {
  if (_deferred === null) return false;
  _deferred.push({ job, frees: frees || [] });
  _markPending(targets);
  return true;
}
/** True while backward() runs, i.e. while _deferColsum accepts jobs. */
export function _deferring() { return _deferredCols !== null; }
/** Queues out (+)= column sums of a partial matrix ([out, partial, rows, n,
 *  beta]) for the end of the running backward(); `frees`, `targets` as above. */
export function _deferColsum(job, frees, targets) {
  if (_deferredCols === null) return false;
  _deferredCols.push({ job, frees: frees || [] });
  _markPending(targets);
  return true;
}
/** Issues every queued job now (column sums, then the grouped GEMM, the
 *  order backward() uses) and empties the queues. */
function _flushDeferred() {
  const cols = _deferredCols, jobs = _deferred;
  _clearPending();
  if (!(cols && cols.length) && !(jobs && jobs.length)) return;
  const a = hip();
  if (cols && cols.length) {
    a.colsumGrouped(cols.map((j) => j.job));
    for (const j of cols) for (const h of j.frees) a.free(h);
    cols.length = 0;
  }
  if (jobs && jobs.length) {
    a.matmulTBwdWGrouped(jobs.map((j) => j.job));
    for (const j of jobs) for (const h of j.frees) a.free(h);
    jobs.length = 0;
  }
}

export function backward(loss) {
  loss._seedGrad();
  const nodes = _tape.nodes;
  const jobs = [], cols = [];
  _deferred = jobs;
  _deferredCols = cols;
  try {
    for (let i = nodes.length - 1; i >= 0; i--) {
      const nd = nodes[i];
      if (!nd._hasGrad() && !nd._bdevAlways) continue;
      if (nd._bdev) nd._bdev();
      else if (nd._b) nd._b(nd.grad);
    }
    _flushDeferred();
  } finally {
    _deferred = null;
    _deferredCols = null;
    _clearPending();
  }
}

// ── vector-level ops (autograd.js:47-189) on the device kernels ──────────────
/** out[N] = W[N,K] · x[K] (autograd.js:47-58) — the matmulT kernels with M = 1. */
export function linear(W, x, N, K) { return matmulT(x, W, 1, K, N); }
/** Elementwise sum (autograd.js:60-67). */
export function add(a, b) { return _addTensors(a, b, a.n); }
/** RMSNorm of one vector (autograd.js:91-107). */
export function rmsnorm(x, w, eps = 1e-6) { return rmsNorm(x, w, 1, x.n, eps); }
/** softmax + cross-entropy of one row (autograd.js:110-124).  The loss is
 *  lse - x[target]; the reference's clamp of p at 1e-40 only differs when
 *  p underflows below 1e-40. */
export function softmaxCE(logits, target) { return crossEntropyMean(logits, [target], 1, logits.n); }

// The vector-level ops (autograd.js:70-190) run on the device too (vector.js).
export { mul, silu, dot, scale, ropeNode, softmaxVec } from "./vector.js";

/**
 * Central-difference check of backward() (autograd.js:192-210): the analytic
 * gradient of lossFn() at about 24 evenly spaced entries of each named
 * parameter against (L(p + eps) − L(p − eps)) / 2eps, each error scaled by
 * max(1, |numeric|, |analytic|).  Returns the worst {maxRelErr, at} and the
 * unperturbed loss.
 */
export function gradCheck(lossFn, params, eps = 1e-3) {
  const base = lossFn();
  backward(base);
  const lossWith = (p, i, value) => {
    p.data[i] = value;  // a host edit: the next device op re-uploads p
    return lossFn().data[0];
  };
  let worst = { maxRelErr: 0, at: "" };
  for (const [name, p] of Object.entries(params)) {
    const stride = Math.max(1, Math.floor(p.n / 24));
    for (let i = 0; i < p.n; i += stride) {
      const x0 = p.data[i];
      const numeric = (lossWith(p, i, x0 + eps) - lossWith(p, i, x0 - eps)) / (2 * eps);
      p.data[i] = x0;
      const g = p.grad;
      const analytic = g ? g[i] : 0;
      const err = Math.abs(numeric - analytic) / Math.max(1, Math.abs(numeric), Math.abs(analytic));
      if (err > worst.maxRelErr) worst = { maxRelErr: err, at: `${name}[${i}]` };
    }
  }
  return { maxRelErr: worst.maxRelErr, at: worst.at, loss: base.data[0] };
}

// ── optimizer ─────────────────────────────────────────────────────────────
/** The {lr, gnorm, scale} of one step; gnorm/scale are read from the device
 *  only when asked for (the copy was queued right after the update). */
class StepInfo {
  constructor(lr, ticket, stats) { this.lr = lr; this._ticket = ticket; this._stats = stats; this._v = null; }
  _read() {
    if (this._v) return this._v;
    const v = new Float64Array(2);
    const a = hip();
    if (!a.readWait(this._ticket, v)) a.d2h(this._stats, v);
    this._v = v;
    return v;
  }
  get gnorm() { return this._read()[0]; }
  get scale() { return this._read()[1]; }
  toJSON() { return { lr: this.lr, gnorm: this.gnorm, scale: this.scale }; }
}

/** Adam + global-norm clip + cosine LR + L2 weight decay (autograd.js:214-244),
 *  one fused multi-tensor update on the device per step. */
export class Adam {
  constructor(params, opts = {}) {
    const o = opts || {};
    const pick = (k, d) => (o[k] === undefined || o[k] === null ? d : o[k]);
    this.p = params; this.lr = pick("lr", 3e-4); this.b1 = pick("b1", 0.9); this.b2 = pick("b2", 0.999);
    this.eps = pick("eps", 1e-8); this.wd = pick("wd", 0); this.clip = pick("clip", 1.0);
    this.total = pick("totalSteps", 1000); this.t = 0;
    const a = hip();
    this._sizes = params.map((p) => p.n);
    this._m = params.map((p) => { const h = allocF32(p.n); a.zero(h, p.n * 4); return h; });
    this._v = params.map((p) => { const h = allocF32(p.n); a.zero(h, p.n * 4); return h; });
    this._stats = a.alloc(16);
    this._plan = null;      // this optimizer's chunk table in device memory
    this._oldPlans = [];    // earlier tables, kept for graphs that recorded them
  }
  /** The device plan (chunk table) of the current tensor list: built on the
   *  first step and again only when the list changes (other pointers or
   *  sizes), so two optimizers never share or overwrite a table. */
  _planFor(list) {
    const a = hip();
    if (this._plan === null || !a.adamPlanMatches(this._plan, list)) {
      if (this._plan !== null) this._oldPlans.push(this._plan);
      this._plan = a.adamPlanCreate(list);
    }
    return this._plan;
  }
  _download(hs) {
    const a = hip();
    return hs.map((h, j) => { const out = new Float32Array(this._sizes[j]); a.d2h(h, out); return out; });
  }
  /** Restores t and the moments (host arrays, one per parameter, in
   *  paramList order) saved by a checkpoint. */
  _restore(t, m, v) {
    if (!Number.isInteger(t) || t < 0) throw new RangeError(`Adam._restore: bad step ${t}`);
    const a = hip();
    for (let j = 0; j < this.p.length; j++) {
      if (m[j].length !== this._sizes[j] || v[j].length !== this._sizes[j]) throw new RangeError(`Adam._restore: moment ${j} has the wrong size`);
      a.h2d(this._m[j], m[j]);
      a.h2d(this._v[j], v[j]);
    }
    this.t = t;
  }
  /** First / second moments as host arrays (downloaded on access). */
  get m() { return this._download(this._m); }
  get v() { return this._download(this._v); }

  /** Advances t and returns the step's {lr, bc1, bc2} (cosine schedule on
   *  the post-increment t, fp64 bias corrections; autograd.js:221-228). */
  _advance() {
    this.t++;
    const lr = this.lr * 0.5 * (1 + Math.cos(Math.PI * Math.min(this.t / this.total, 1)));
    return { lr, bc1: 1 - Math.pow(this.b1, this.t), bc2: 1 - Math.pow(this.b2, this.t) };
  }
  _list() {
    const list = [], touched = [];
    for (let j = 0; j < this.p.length; j++) {
      const p = this.p[j];
      if (!p._hasGrad()) continue;
      if (p.n !== this._sizes[j]) throw new Error(`Adam: parameter ${j} changed size (${this._sizes[j]} -> ${p.n})`);
      list.push([p._devData(), p._gradDev(), this._m[j], this._v[j], p.n]);
      touched.push(p);
    }
    return { list, touched };
  }

  step() {
    const { lr, bc1, bc2 } = this._advance();
    const { list, touched } = this._list();
    const a = hip();
    a.adamStepPlan(this._planFor(list), lr, this.b1, this.b2, this.eps, this.wd, this.clip, bc1, bc2, this._stats);
    for (const p of touched) p._deviceWrote();
    return new StepInfo(lr, a.readAsync(this._stats, 16), this._stats);
  }

  /** The update of step() with {lr, bc1, bc2} read from device memory
   *  (`sched`, 3 doubles written by the caller after _advance()); queues no
   *  read-back, so a recorded graph step can hold it. */
  _stepSched(sched) {
    const { list, touched } = this._list();
    hip().adamStepSchedPlan(this._planFor(list), sched, this.b1, this.b2, this.eps, this.wd, this.clip, this._stats);
    for (const p of touched) p._deviceWrote();
  }
}
