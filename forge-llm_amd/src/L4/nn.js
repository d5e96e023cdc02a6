/**
 * L4 · QuantLinear and the SwiGLU block (forge-llm src/L4/nn.js:19-66) on the
 * device.
 *
 * QuantLinear keeps the reference's fields — type, bytes (host, a
 * Float32Array for type 0), N, K — and uploads the bytes to the device once,
 * on first use; forward runs fg_qmatvec (fp64 sums, one fp32 rounding per
 * output, as the reference's dotQ / matvec into a Float32Array).  Change
 * `bytes` after the first forward and call `invalidate()` so the next call
 * uploads again.  Transformer.loadWeights takes QuantLinear matrices as they
 * are: the decode kernels read every supported type directly.
 */
import { hip } from "../L2/device.js";
import { info, rowBytes, quantizeRow, dequantize } from "../L3/quant.js";

const SUPPORTED = new Set([0, 1, 2, 6, 8, 12, 13, 14]);

function upload(a, typed) {
  const h = a.alloc(Math.max(1, typed.byteLength));
  if (typed.byteLength) a.h2d(h, typed);
  return h;
}

/** Quantized linear layer W[N, K] (nn.js:19-40). */
export class QuantLinear {
  constructor(type, bytes, N, K) {
    this.type = type; this.bytes = bytes; this.N = N; this.K = K;
    this._d = null;
  }

  /** QuantLinear.fromF32 (nn.js:23-25): type 0 keeps an f32 copy, other types
   *  quantize W on the device (bit-identical to the reference's quantizeRow). */
  static fromF32(W, N, K, type = 0) {
    return new QuantLinear(type, type === 0 ? Float32Array.from(W) : quantizeRow(type, W, N * K), N, K);
  }

  /** The weight bytes as a Uint8Array view. */
  _u8() {
    const b = this.bytes;
    if (b instanceof Uint8Array) return b;
    if (ArrayBuffer.isView(b)) return new Uint8Array(b.buffer, b.byteOffset, b.byteLength);
    return new Uint8Array(Float32Array.from(b).buffer);
  }

  _check() {
    if (!SUPPORTED.has(this.type)) throw new Error(`QuantLinear: type ${this.type} is not supported on the device`);
    const bs = info(this.type).blockSize;
    if (this.K % bs !== 0) throw new RangeError(`QuantLinear: K=${this.K} is not a whole number of ${bs}-element blocks`);
    const need = rowBytes(this.type, this.K) * this.N;
    if (this._u8().byteLength < need) throw new RangeError(`QuantLinear: ${need} bytes needed, ${this._u8().byteLength} given`);
  }

  /** Device copy of the weights (uploaded once). */
  _dev() {
    if (this._d) return this._d;
    this._check();
    this._d = upload(hip(), this._u8().subarray(0, rowBytes(this.type, this.K) * this.N));
    return this._d;
  }

  /** Drops the device copy (the next use uploads `bytes` again). */
  invalidate() {
    if (this._d) hip().free(this._d);
    this._d = null;
  }

  /** out[N] = W · x[xOff .. xOff+K) (nn.js:27-33). */
  forward(x, out, xOff = 0) {
    const a = hip(), W = this._dev();
    const xs = (x instanceof Float32Array ? x : Float32Array.from(x)).subarray(xOff, xOff + this.K);
    if (xs.length !== this.K) throw new RangeError(`QuantLinear.forward: x holds ${xs.length} of ${this.K} values`);
    const xd = upload(a, xs), yd = a.alloc(this.N * 4);
    try {
      a.qmatvec(this.type, yd, W, xd, this.N, this.K);
      a.d2h(yd, out.subarray ? out.subarray(0, this.N) : out);
    } finally {
      a.free(xd); a.free(yd);
    }
    return out;
  }

  /** Dequantized weights (nn.js:35-38). */
  toF32() {
    if (this.type === 0) return Float32Array.from(this.bytes);
    return dequantize(this.type, this._u8(), this.N * this.K);
  }

  bytesSize() { return rowBytes(this.type, this.K) * this.N; }
}

/** One-row RMSNorm over host arrays (nn.js:42-44): out[i] = x[i]·w[i] /
 *  sqrt(rms(x)² + eps), computed on the device, written into `out`. */
export function rmsnormInto(out, x, w, n, eps = 1e-6) {
  if (!Number.isInteger(n) || n <= 0) throw new RangeError(`rmsnormInto: n must be a positive integer, got ${n}`);
  for (const [v, what] of [[out, "out"], [x, "x"], [w, "w"]])
    if (!v || v.length < n) throw new RangeError(`rmsnormInto: ${what} needs ${n} elements`);
  if (typeof eps !== "number") throw new TypeError("rmsnormInto: eps must be a number");
  const f32 = (v) => (v instanceof Float32Array ? v.subarray(0, n) : Float32Array.from(Array.prototype.slice.call(v, 0, n)));
  const a = hip();
  const held = [];
  const alloc = () => { const h = a.alloc(n * 4); held.push(h); return h; };
  try {
    const bx = alloc(), bw = alloc(), bo = alloc();
    a.h2d(bx, f32(x));
    a.h2d(bw, f32(w));
    a.rowRmsnorm(bo, bx, bw, n, eps);
    const r = new Float32Array(n);
    a.d2h(bo, r);
    for (let i = 0; i < n; i++) out[i] = r[i];
  } finally {
    for (const h of held) a.free(h);
  }
  return out;
}

/** SwiGLU block (nn.js:50-66): out = W_down · (silu(W_gate · x) ⊙ (W_up · x)),
 *  the three matvecs and the activation on the device. */
export class SwiGLU {
  constructor(gate, up, down, dim, hidden) {
    this.gate = gate; this.up = up; this.down = down;
    this.dim = dim; this.hidden = hidden;
  }

  forward(x, out) {
    const a = hip(), H = this.hidden, D = this.dim;
    const xs = (x instanceof Float32Array ? x : Float32Array.from(x)).subarray(0, D);
    const xd = upload(a, xs), g = a.alloc(H * 4), u = a.alloc(H * 4), h = a.alloc(H * 4), o = a.alloc(D * 4);
    try {
      a.qmatvec(this.gate.type, g, this.gate._dev(), xd, H, D);
      a.qmatvec(this.up.type, u, this.up._dev(), xd, H, D);
      a.siluMul(h, g, u, H);
      a.qmatvec(this.down.type, o, this.down._dev(), h, D, H);
      a.d2h(o, out.subarray ? out.subarray(0, D) : out);
    } finally {
      a.free(xd); a.free(g); a.free(u); a.free(h); a.free(o);
    }
    return out;
  }
}
