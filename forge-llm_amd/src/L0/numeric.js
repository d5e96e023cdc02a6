/**
 * L0 · host numerics used around the device path: the deterministic RNG that
 * seeds weights and synthetic inputs, and the error metrics.
 *
 * RNG restates forge-llm's src/L0/numeric.js:27-49 (splitmix32 seeding,
 * xorshift128+ stream, Box–Muller normals) so seeded weights and inputs are
 * identical to the reference's.  Metrics follow numeric.js:142-161.
 */
export class RNG {
  constructor(seed = 0x9e3779b9) {
    let state = (seed >>> 0) || 1;
    const mix = () => {
      state = (state + 0x9e3779b9) >>> 0;
      let z = state;
      z = Math.imul(z ^ (z >>> 16), 0x21f0aaad) >>> 0;
      z = Math.imul(z ^ (z >>> 15), 0x735a2d97) >>> 0;
      return (z ^ (z >>> 15)) >>> 0;
    };
    this.s0 = mix();
    this.s1 = mix();
  }
  /** Uniform in [0, 1) with 32 random bits. */
  next() {
    let a = this.s0;
    const b = this.s1;
    this.s0 = b;
    a = (a ^ (a << 23)) >>> 0;
    a = (a ^ (a >>> 17)) >>> 0;
    a = (a ^ b ^ (b >>> 26)) >>> 0;
    this.s1 = a;
    return ((a + b) >>> 0) / 4294967296;
  }
  /** Standard normal (Box–Muller). */
  normal() {
    const u = Math.max(this.next(), 1e-12), v = this.next();
    return Math.sqrt(-2 * Math.log(u)) * Math.cos(2 * Math.PI * v);
  }
  uniform(a, b) { return a + (b - a) * this.next(); }
  int(n) { return Math.floor(this.next() * n); }
}

export function maxAbsErr(a, b) {
  let m = 0;
  for (let i = 0; i < a.length; i++) { const d = Math.abs(a[i] - b[i]); if (d > m) m = d; }
  return m;
}
export function rmse(a, b) {
  let s = 0;
  for (let i = 0; i < a.length; i++) { const d = a[i] - b[i]; s += d * d; }
  return Math.sqrt(s / a.length);
}
export function relL2(a, b) {
  let ns = 0, ds = 0;
  for (let i = 0; i < a.length; i++) { const d = a[i] - b[i]; ns += d * d; ds += a[i] * a[i]; }
  return Math.sqrt(ns / (ds || 1));
}
export function cosSim(a, b) {
  let d = 0, na = 0, nb = 0;
  for (let i = 0; i < a.length; i++) { d += a[i] * b[i]; na += a[i] * a[i]; nb += b[i] * b[i]; }
  return d / (Math.sqrt(na * nb) || 1);
}
