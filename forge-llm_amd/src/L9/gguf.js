/**
 * L9 · GGUF v3 container (read and write), host code.
 *
 * The on-disk format of forge-llm's exportGGUF / loadGGUF (src/L9/gguf.js:
 * 142-209 write, :89-120 read), written from the GGUF v3 layout:
 *
 *   u32 magic 0x46554747 ("GGUF") · u32 version 3 · u64 tensor count ·
 *   u64 metadata count · metadata {string key, u32 type, value}* ·
 *   tensor infos {string name, u32 n_dims, u64 dims[n_dims], u32 ggml type,
 *   u64 offset}* · zero padding to general.alignment · tensor data, each
 *   tensor padded to the alignment.
 *   string = u64 byte length + UTF-8 bytes; array = u32 element type + u64
 *   count + elements.  All integers little-endian.
 *
 * Metadata values keep the reference writer's type choice (so files match it
 * byte for byte): booleans → BOOL, integers in [0, 2^32) → UINT32, other
 * numbers → FLOAT32, strings → STRING, arrays by their first element
 * (string → STRING, integer → INT32, other → FLOAT32).  A value given as
 * {ggufType, value} is written with that type (the checkpoint's FLOAT64
 * optimizer scalars).
 */
export const GGUFValueType = {
  UINT8: 0, INT8: 1, UINT16: 2, INT16: 3, UINT32: 4, INT32: 5,
  FLOAT32: 6, BOOL: 7, STRING: 8, ARRAY: 9, UINT64: 10, INT64: 11, FLOAT64: 12,
};
export const GGML_F32 = 0;
export const GGML_F16 = 1;
export const GGML_Q8_0 = 8;
export const GGML_Q4_K = 12;
export const GGML_Q5_K = 13;
export const GGML_Q6_K = 14;

const DEFAULT_ALIGN = 32;
const MAGIC = 0x46554747;

// ggml block layouts [elements per block, bytes per block] (the GGML type
// table that quant.js:42-56 of the reference also lists).
const BLOCKS = {
  [GGML_F32]: [1, 4], [GGML_F16]: [1, 2], 2: [32, 18], 3: [32, 20], 6: [32, 22], 7: [32, 24],
  [GGML_Q8_0]: [32, 34], 9: [32, 36], [GGML_Q4_K]: [256, 144], [GGML_Q5_K]: [256, 176], [GGML_Q6_K]: [256, 210],
  15: [256, 292],
};

/** Mean bytes per element of a ggml type (gguf.js:211-218 of the reference). */
export function ggmlTypeSize(type) {
  const b = BLOCKS[type];
  if (!b) throw new Error(`GGUF: unsupported ggml type ${type}`);
  return b[1] / b[0];
}

/** Bytes of a tensor of n elements of a ggml type (block types need whole blocks). */
export function tensorBytes(type, n) {
  const b = BLOCKS[type];
  if (!b) throw new Error(`GGUF: unsupported ggml type ${type}`);
  if (n % b[0] !== 0) throw new Error(`GGUF: ${n} elements are not whole blocks of ${b[0]} (type ${type})`);
  return (n / b[0]) * b[1];
}

class ByteSink {
  constructor() { this.parts = []; this.n = 0; this.scratch = new DataView(new ArrayBuffer(8)); }
  bytes(u8) { this.parts.push(u8); this.n += u8.length; }
  _fixed(k, fn) { fn(this.scratch); this.bytes(new Uint8Array(this.scratch.buffer.slice(0, k))); }
  u8(v) { this._fixed(1, (d) => d.setUint8(0, v)); }
  i8(v) { this._fixed(1, (d) => d.setInt8(0, v)); }
  u16(v) { this._fixed(2, (d) => d.setUint16(0, v, true)); }
  i16(v) { this._fixed(2, (d) => d.setInt16(0, v, true)); }
  u32(v) { this._fixed(4, (d) => d.setUint32(0, v, true)); }
  i32(v) { this._fixed(4, (d) => d.setInt32(0, v, true)); }
  f32(v) { this._fixed(4, (d) => d.setFloat32(0, v, true)); }
  f64(v) { this._fixed(8, (d) => d.setFloat64(0, v, true)); }
  u64(v) {
    if (!Number.isInteger(v) || v < 0 || v > Number.MAX_SAFE_INTEGER) throw new RangeError(`GGUF: bad u64 ${v}`);
    this._fixed(8, (d) => { d.setUint32(0, v % 4294967296, true); d.setUint32(4, Math.floor(v / 4294967296), true); });
  }
  i64(v) {
    if (!Number.isInteger(v) || Math.abs(v) > Number.MAX_SAFE_INTEGER) throw new RangeError(`GGUF: bad i64 ${v}`);
    const hi = Math.floor(v / 4294967296), lo = v - hi * 4294967296;  // two's complement halves
    this._fixed(8, (d) => { d.setUint32(0, lo, true); d.setInt32(4, hi, true); });
  }
  str(s) { const b = new TextEncoder().encode(s); this.u64(b.length); this.bytes(b); }
  pad(align) { const k = (align - (this.n % align)) % align; if (k) this.bytes(new Uint8Array(k)); }
  concat() {
    const out = new Uint8Array(this.n);
    let o = 0;
    for (const p of this.parts) { out.set(p, o); o += p.length; }
    return out;
  }
}

function valueType(v) {
  if (v && typeof v === "object" && !Array.isArray(v) && "ggufType" in v) return v.ggufType;
  if (typeof v === "boolean") return GGUFValueType.BOOL;
  if (typeof v === "number") return Number.isInteger(v) && v >= 0 && v <= 0xffffffff ? GGUFValueType.UINT32 : GGUFValueType.FLOAT32;
  if (typeof v === "string") return GGUFValueType.STRING;
  if (Array.isArray(v)) return GGUFValueType.ARRAY;
  throw new TypeError(`GGUF: metadata value of type ${typeof v} cannot be written`);
}

function writeScalar(w, t, v) {
  switch (t) {
    case GGUFValueType.UINT8: return w.u8(v);
    case GGUFValueType.INT8: return w.i8(v);
    case GGUFValueType.UINT16: return w.u16(v);
    case GGUFValueType.INT16: return w.i16(v);
    case GGUFValueType.UINT32: return w.u32(v);
    case GGUFValueType.INT32: return w.i32(v);
    case GGUFValueType.FLOAT32: return w.f32(v);
    case GGUFValueType.BOOL: return w.u8(v ? 1 : 0);
    case GGUFValueType.STRING: return w.str(v);
    case GGUFValueType.UINT64: return w.u64(v);
    case GGUFValueType.INT64: return w.i64(v);
    case GGUFValueType.FLOAT64: return w.f64(v);
    default: throw new TypeError(`GGUF: scalar type ${t}`);
  }
}

function writeValue(w, v) {
  const t = valueType(v);
  w.u32(t);
  const raw = v && typeof v === "object" && !Array.isArray(v) && "ggufType" in v ? v.value : v;
  if (t !== GGUFValueType.ARRAY) return writeScalar(w, t, raw);
  const first = raw[0];
  const et = typeof first === "string" || Array.isArray(first) ? GGUFValueType.STRING
    : typeof first === "number" && Number.isInteger(first) ? GGUFValueType.INT32 : GGUFValueType.FLOAT32;
  w.u32(et);
  w.u64(raw.length);
  for (const e of raw) writeScalar(w, et, et === GGUFValueType.STRING && Array.isArray(e) ? String(e) : e);
}

/**
 * Serialises {meta: Map<string, value>, tensors: [{name, dims, type, data}]}
 * (data: Uint8Array of tensorBytes(type, Π dims) bytes) to GGUF v3:
 * {bytes, headerLen, dataStart} as gguf.js:142-179 of the reference returns.
 */
export function writeGGUF({ meta = new Map(), tensors = [] }) {
  const w = new ByteSink();
  w.u32(MAGIC); w.u32(3); w.u64(tensors.length); w.u64(meta.size);
  for (const [k, v] of meta) { w.str(k); writeValue(w, v); }
  const alignV = meta.get("general.alignment");
  const align = alignV === undefined ? DEFAULT_ALIGN : (typeof alignV === "object" ? alignV.value : alignV);
  let off = 0;
  for (const t of tensors) {
    const n = t.dims.reduce((a, b) => a * b, 1);
    const len = tensorBytes(t.type, n);
    if (t.data.byteLength !== len) throw new RangeError(`GGUF: tensor ${t.name} holds ${t.data.byteLength} bytes, ${len} expected`);
    w.str(t.name); w.u32(t.dims.length);
    for (const d of t.dims) w.u64(d);
    w.u32(t.type); w.u64(off);
    off += Math.ceil(len / align) * align;
  }
  const headerLen = w.n;
  w.pad(align);
  const dataStart = w.n;
  for (const t of tensors) {
    w.bytes(t.data instanceof Uint8Array ? t.data : new Uint8Array(t.data.buffer, t.data.byteOffset, t.data.byteLength));
    w.pad(align);
  }
  return { bytes: w.concat(), headerLen, dataStart };
}

class ByteSource {
  constructor(u8) { this.b = u8; this.d = new DataView(u8.buffer, u8.byteOffset, u8.byteLength); this.p = 0; }
  _need(k) { if (this.p + k > this.b.length) throw new RangeError("GGUF: truncated file"); }
  u8() { this._need(1); return this.d.getUint8(this.p++); }
  i8() { this._need(1); return this.d.getInt8(this.p++); }
  u16() { this._need(2); const v = this.d.getUint16(this.p, true); this.p += 2; return v; }
  i16() { this._need(2); const v = this.d.getInt16(this.p, true); this.p += 2; return v; }
  u32() { this._need(4); const v = this.d.getUint32(this.p, true); this.p += 4; return v; }
  i32() { this._need(4); const v = this.d.getInt32(this.p, true); this.p += 4; return v; }
  f32() { this._need(4); const v = this.d.getFloat32(this.p, true); this.p += 4; return v; }
  f64() { this._need(8); const v = this.d.getFloat64(this.p, true); this.p += 8; return v; }
  u64() { const lo = this.u32(), hi = this.u32(); return hi * 4294967296 + lo; }
  i64() { const lo = this.u32(), hi = this.i32(); return hi * 4294967296 + lo; }
  str() { const n = this.u64(); this._need(n); const s = new TextDecoder().decode(this.b.subarray(this.p, this.p + n)); this.p += n; return s; }
}

function readScalar(r, t) {
  switch (t) {
    case GGUFValueType.UINT8: return r.u8();
    case GGUFValueType.INT8: return r.i8();
    case GGUFValueType.UINT16: return r.u16();
    case GGUFValueType.INT16: return r.i16();
    case GGUFValueType.UINT32: return r.u32();
    case GGUFValueType.INT32: return r.i32();
    case GGUFValueType.FLOAT32: return r.f32();
    case GGUFValueType.BOOL: return r.u8() !== 0;
    case GGUFValueType.STRING: return r.str();
    case GGUFValueType.UINT64: return r.u64();
    case GGUFValueType.INT64: return r.i64();
    case GGUFValueType.FLOAT64: return r.f64();
    default: throw new Error(`GGUF: unknown value type ${t}`);
  }
}

/**
 * Parses GGUF (v1-v3) bytes: {version, alignment, meta (Map), tensors
 * [{name, dims, type, offset}], tensorDataStart, getTensor(name) →
 * {type, dims, data: Uint8Array view} | null}.
 */
export function readGGUF(buf) {
  const u8 = buf instanceof Uint8Array ? buf : new Uint8Array(buf.buffer || buf, buf.byteOffset || 0, buf.byteLength);
  const r = new ByteSource(u8);
  const magic = r.u32();
  // The message keeps the reference's wording (gguf.js:75), which its tests match.
  if (magic !== MAGIC) throw new Error(`非法 GGUF magic: 0x${magic.toString(16)} (GGUF: bad magic)`);
  const version = r.u32();
  if (version < 1 || version > 3) throw new Error(`GGUF: unsupported version ${version}`);
  const nT = r.u64(), nKv = r.u64();
  const meta = new Map();
  for (let i = 0; i < nKv; i++) {
    const k = r.str();
    const t = r.u32();
    if (t === GGUFValueType.ARRAY) {
      const et = r.u32(), n = r.u64();
      const arr = new Array(n);
      for (let j = 0; j < n; j++) arr[j] = readScalar(r, et);
      meta.set(k, arr);
    } else meta.set(k, readScalar(r, t));
  }
  const tensors = [];
  for (let i = 0; i < nT; i++) {
    const name = r.str();
    const nd = r.u32();
    const dims = [];
    for (let d = 0; d < nd; d++) dims.push(r.u64());
    tensors.push({ name, dims, type: r.u32(), offset: r.u64() });
  }
  const alignment = meta.has("general.alignment") ? meta.get("general.alignment") : DEFAULT_ALIGN;
  const start = Math.ceil(r.p / alignment) * alignment;
  const byName = new Map(tensors.map((t) => [t.name, t]));
  return {
    version, alignment, meta, tensors, tensorDataStart: start,
    getTensor(name) {
      const t = byName.get(name);
      if (!t) return null;
      const len = tensorBytes(t.type, t.dims.reduce((a, b) => a * b, 1));
      const s = start + t.offset;
      if (s + len > u8.length) throw new RangeError(`GGUF: tensor ${name} runs past the end of the file`);
      return { type: t.type, dims: t.dims, data: u8.subarray(s, s + len) };
    },
  };
}
