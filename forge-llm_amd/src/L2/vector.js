/**
 * L2c · vector-level autograd ops on the device: mul, silu, dot, scale,
 * ropeNode, softmaxVec (forge-llm src/L2/autograd.js:70-190).
 *
 * Same positional signatures, forward values and backward semantics as the
 * reference: each op returns a Node recorded on the tape, its gradient is
 * created on first write and accumulated afterwards, and the arithmetic is
 * the reference's (fp64 evaluation of fp32 operands, one fp32 rounding per
 * store; see the fg_vec_* entry points in include/forge_hip.h).  Values stay
 * in device memory; `.data` / `.grad` download on read like every other op.
 */
import { hip, allocF32, graphState } from "./device.js";
import { Node, _deviceNode, _tapeEnabled } from "./autograd.js";

function node(x, what) {
  if (!(x instanceof Node)) throw new TypeError(`${what}: expected a Node`);
  return x;
}
function attach(out, saved, bwd) {
  if (_tapeEnabled()) {
    out._saved = saved;
    out._bdev = bwd;
  } else if (saved) {
    const a = hip();
    for (const h of saved) a.free(h);
  }
  return out;
}
/** A scalar result: its 4 bytes are queued for the host right away (read by `.data`). */
function readSoon(a, out) {
  if (!graphState.capturing) out._ticket = a.readAsync(out._dev, 4);
  return out;
}

/** out = a ⊙ b, with b of a's length or a single element broadcast (autograd.js:70-79). */
export function mul(a, b) {
  node(a, "mul a"); node(b, "mul b");
  const n = a.n, nb = b.n;
  if (!(nb === n || nb === 1)) throw new RangeError(`mul: b has ${nb} elements, expected ${n} or 1`);
  const d = hip();
  const out = _deviceNode(n);
  d.vecMulFwd(out._dev, a._devData(), b._devData(), n, nb);
  return attach(out, null, () => {
    const g = out._gradDev();
    const ga = a._gradAcc();
    const gb = b._gradAcc();
    d.vecMulBwd(ga.h, ga.beta, gb.h, gb.beta, g, a._devData(), b._devData(), n, nb);
  });
}

/** out = x · σ(x) (autograd.js:81-89); σ is kept for the backward. */
export function silu(x) {
  node(x, "silu x");
  const n = x.n, d = hip();
  const out = _deviceNode(n);
  const sig = allocF32(n);
  d.vecSiluFwd(out._dev, sig, x._devData(), n);
  return attach(out, [sig], () => {
    const gx = x._gradAcc();
    d.vecSiluBwd(gx.h, gx.beta, out._gradDev(), x._devData(), sig, n);
  });
}

/** out = Σ aᵢ bᵢ as a one-element Node (autograd.js:136-146). */
export function dot(a, b) {
  node(a, "dot a"); node(b, "dot b");
  const n = a.n;
  if (b.n !== n) throw new RangeError(`dot: lengths ${n} and ${b.n} differ`);
  const d = hip();
  const out = _deviceNode(1);
  d.vecDotFwd(out._dev, a._devData(), b._devData(), n);
  readSoon(d, out);
  return attach(out, null, () => {
    const g = out._gradDev();
    const ga = a._gradAcc();
    const gb = b._gradAcc();
    d.vecDotBwd(ga.h, ga.beta, gb.h, gb.beta, g, a._devData(), b._devData(), n);
  });
}

/** out = s · x for a number s (autograd.js:148-153). */
export function scale(x, s) {
  node(x, "scale x");
  if (typeof s !== "number") throw new TypeError(`scale: s must be a number, got ${typeof s}`);
  const n = x.n, d = hip();
  const out = _deviceNode(n);
  d.vecScaleFwd(out._dev, x._devData(), s, n);
  return attach(out, null, () => {
    const gx = x._gradAcc();
    d.vecScaleBwd(gx.h, gx.beta, out._gradDev(), s, n);
  });
}

/**
 * RoPE of the first dHead entries of x (autograd.js:156-172): pair
 * (x[i], x[i+1]), i = 0, 2, …, turned by (cos[i/2], sin[i/2]); the entries
 * after the pairs are zero in the output.  cos / sin are constant arrays.
 */
export function ropeNode(x, cos, sin, dHead) {
  node(x, "ropeNode x");
  if (!Number.isInteger(dHead) || dHead < 0) throw new RangeError(`ropeNode: dHead must be a non-negative integer, got ${dHead}`);
  const n = x.n, half = (dHead + 1) >> 1;
  if (2 * half > n) throw new RangeError(`ropeNode: the pairs below dHead=${dHead} need ${2 * half} elements, x has ${n}`);
  if (!cos || !sin || cos.length < half || sin.length < half)
    throw new RangeError(`ropeNode: cos and sin need ${half} entries`);
  const d = hip();
  const out = _deviceNode(n);  // a Node on the tape first: released with it if the table allocation fails
  const tab = half > 0 ? d.alloc(2 * half * 8) : null;
  if (tab) {
    const t = new Float64Array(2 * half);
    for (let k = 0; k < half; k++) { t[k] = cos[k]; t[half + k] = sin[k]; }
    d.h2d(tab, t);
  }
  const ct = tab, st = tab ? d.view(tab, half * 8, half * 8) : null;
  d.vecRopeFwd(out._dev, x._devData(), ct, st, n, dHead);
  return attach(out, tab ? [tab] : null, () => {
    const gx = x._gradAcc();
    d.vecRopeBwd(gx.h, gx.beta, out._gradDev(), ct, st, n, dHead);
  });
}

/** p = softmax(x) (autograd.js:174-190); the backward applies the full softmax Jacobian. */
export function softmaxVec(x) {
  node(x, "softmaxVec x");
  const n = x.n, d = hip();
  const out = _deviceNode(n);
  const p = allocF32(n);
  d.vecSoftmaxFwd(out._dev, p, x._devData(), n);
  return attach(out, [p], () => {
    const gx = x._gradAcc();
    d.vecSoftmaxBwd(gx.h, gx.beta, out._gradDev(), p, n);
  });
}
