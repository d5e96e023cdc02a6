/**
 * L3 · quantized weight formats (forge-llm src/L3/quant.js) on the device.
 *
 * The type table, `info` and `rowBytes` are host bookkeeping; everything that
 * touches weight values runs on the GPU through libforge_hip:
 *   dequantize   → fg_dequantize  (bit-identical to the reference)
 *   dotQ         → fg_qmatvec_f64 (fp64 sum, as the reference returns it)
 *   quantizeRow  → fg_quantize    (bit-identical bytes: the reference's
 *                  closed-form Q8_0 / Q4_K and its Q5_K / Q6_K searches)
 * Host arrays in, host arrays out, as in the reference: each call uploads its
 * inputs and downloads its result.  The device-resident path for whole
 * models is QuantLinear / Transformer.loadWeights, which upload once.
 *
 * Types: F32 0, F16 1, Q4_0 2, Q5_0 6, Q8_0 8, Q4_K 12, Q5_K 13, Q6_K 14
 * (Q4_0 / Q5_0 decode only, read the way the reference's generic branch
 * reads them).
 */
import { hip } from "../L2/device.js";

export const QK_K = 256;

/** GGML type ids (ggml.h numbering, as the reference's GGMLType). */
export const GGMLType = {
  F32: 0, F16: 1, Q4_0: 2, Q4_1: 3, Q5_0: 6, Q5_1: 7,
  Q8_0: 8, Q8_1: 9, Q2_K: 10, Q3_K: 11, Q4_K: 12, Q5_K: 13, Q6_K: 14, Q8_K: 15,
  IQ2_XXS: 16, IQ2_XS: 17, IQ3_XXS: 18, IQ3_S: 19, IQ2_S: 20, IQ3_M: 21, IQ4_XS: 22, IQ4_NL: 23,
};
export const TYPE_NAME = Object.fromEntries(Object.entries(GGMLType).map(([k, v]) => [v, k]));

const blk = (name, blockSize, blockBytes) => ({ name, blockSize, blockBytes, bpw: (8 * blockBytes) / blockSize });
/** {blockSize, blockBytes, bpw} per type (the GGML block layouts). */
export const TYPE_INFO = {
  0: blk("F32", 1, 4), 1: blk("F16", 1, 2), 2: blk("Q4_0", 32, 18), 3: blk("Q4_1", 32, 20),
  6: blk("Q5_0", 32, 22), 7: blk("Q5_1", 32, 24), 8: blk("Q8_0", 32, 34), 9: blk("Q8_1", 32, 36),
  12: blk("Q4_K", 256, 144), 13: blk("Q5_K", 256, 176), 14: blk("Q6_K", 256, 210), 15: blk("Q8_K", 256, 292),
};

export function info(type) {
  const t = TYPE_INFO[type];
  if (!t) throw new Error(`unsupported GGML type ${type}`);
  return t;
}
/** rowBytes (quant.js:64): bytes of n elements, whole blocks. */
export function rowBytes(type, n) { const t = info(type); return Math.ceil(n / t.blockSize) * t.blockBytes; }

const DECODABLE = new Set([0, 1, 2, 6, 8, 12, 13, 14]);
const QUANTIZABLE = new Set([0, 1, 8, 12, 13, 14]);

function bytesView(a) {
  if (a instanceof Uint8Array) return a;
  if (ArrayBuffer.isView(a)) return new Uint8Array(a.buffer, a.byteOffset, a.byteLength);
  throw new TypeError("expected a Uint8Array (or typed array) of quantized bytes");
}
function f32View(x, off, n) {
  const f = x instanceof Float32Array ? x : Float32Array.from(x);
  if (off + n > f.length) throw new RangeError(`need ${n} values from offset ${off}, array holds ${f.length}`);
  return f.subarray(off, off + n);
}
function upload(a, typed) {
  const h = a.alloc(Math.max(1, typed.byteLength));
  if (typed.byteLength) a.h2d(h, typed);
  return h;
}

/** dequantize (quant.js:102-199): n values of type `type` from u8 at byteOff. */
export function dequantize(type, u8, n, out = new Float32Array(n), byteOff = 0) {
  if (!DECODABLE.has(type)) throw new Error(`dequantize: type ${type} (${TYPE_NAME[type]}) is not supported`);
  const bs = info(type).blockSize;
  if (n % bs !== 0) throw new RangeError(`dequantize: ${n} elements are not whole ${bs}-element blocks`);
  const src = bytesView(u8).subarray(byteOff, byteOff + rowBytes(type, n));
  if (src.length !== rowBytes(type, n)) throw new RangeError("dequantize: source shorter than n elements");
  if (n === 0) return out;
  const a = hip();
  const q = upload(a, src), o = a.alloc(n * 4);
  try {
    a.dequantize(type, o, q, n);
    a.d2h(o, out.subarray(0, n));
  } finally {
    a.free(q); a.free(o);
  }
  return out;
}

/** dotQ (quant.js:215-320): Σ w·x over n quantized weights (u8 from byteOff)
 *  and x[xOff ..], as an fp64 number. */
export function dotQ(type, u8, x, n, xOff = 0, byteOff = 0) {
  if (!DECODABLE.has(type)) throw new Error(`dotQ: type ${type} (${TYPE_NAME[type]}) is not supported`);
  const bs = info(type).blockSize;
  if (n % bs !== 0) throw new RangeError(`dotQ: ${n} elements are not whole ${bs}-element blocks`);
  const src = bytesView(u8).subarray(byteOff, byteOff + rowBytes(type, n));
  const a = hip();
  const q = upload(a, src), xd = upload(a, f32View(x, xOff, n)), y = a.alloc(8);
  const r = new Float64Array(1);
  try {
    a.qmatvecF64(type, y, q, xd, 1, n);
    a.d2h(y, r);
  } finally {
    a.free(q); a.free(xd); a.free(y);
  }
  return r[0];
}

/** quantizeRow (quant.js:580-590): x[off .. off+n) → bytes.  Whole blocks are
 *  quantized (a trailing partial block is dropped, as the reference's block
 *  count n / blockSize does). */
export function quantizeRow(type, x, n, off = 0) {
  if (!QUANTIZABLE.has(type)) throw new Error(`quantizeRow: no quantizer for type ${type} (${TYPE_NAME[type]})`);
  const bs = info(type).blockSize;
  const nw = n - (n % bs);
  const out = new Uint8Array(rowBytes(type, nw));
  if (nw === 0) return out;
  const a = hip();
  const xd = upload(a, f32View(x, off, nw)), q = a.alloc(out.length);
  try {
    a.quantize(type, q, xd, nw);
    a.d2h(q, out);
  } finally {
    a.free(xd); a.free(q);
  }
  return out;
}

export const quantizeRowF16 = (x, n, off = 0) => quantizeRow(1, x, n, off);
export const quantizeRowQ8_0 = (x, n, off = 0) => quantizeRow(8, x, n, off);
export const quantizeRowQ4K = (x, n, off = 0) => quantizeRow(12, x, n, off);
export const quantizeRowQ5K = (x, n, off = 0) => quantizeRow(13, x, n, off);
export const quantizeRowQ6K = (x, n, off = 0) => quantizeRow(14, x, n, off);

/** Quality report (quant.js:593-610): RMSE, max error, relative L2, cosine
 *  and compression of a quantize → dequantize round trip on the device. */
export function qualityReport(type, orig, n = orig.length) {
  const bytes = quantizeRow(type, orig, n);
  const nq = n - (n % info(type).blockSize);
  const deq = dequantize(type, bytes, nq);
  let se = 0, mx = 0, nn = 0, dd = 0, nb = 0;
  for (let i = 0; i < nq; i++) {
    const e = deq[i] - orig[i];
    se += e * e;
    if (Math.abs(e) > mx) mx = Math.abs(e);
    nn += orig[i] * orig[i]; dd += orig[i] * deq[i]; nb += deq[i] * deq[i];
  }
  return {
    type, name: info(type).name, rmse: Math.sqrt(se / n), maxAbs: mx,
    relL2: Math.sqrt(se / (nn || 1)), cos: dd / (Math.sqrt(nn * nb) || 1),
    bpw: info(type).bpw, bytes: bytes.length, origBytes: n * 4, ratio: (n * 4) / bytes.length,
  };
}

/** fp16 → fp32 table of all 65536 halves (decoded on the device). */
let _fp16 = null;
export function fp16Table() {
  if (_fp16) return _fp16;
  const h = new Uint16Array(65536);
  for (let i = 0; i < 65536; i++) h[i] = i;
  _fp16 = dequantize(1, new Uint8Array(h.buffer), 65536);
  return _fp16;
}
