// GGUF container and f32 export on the host (no GPU): the reference's GGUF
// tests (test/l7-l10.test.js:79-131) restated — write → read keeps every
// metadata pair and tensor (I-90), tensor data is aligned (I-91), a bad magic
// throws — plus export → re-import of initWeights weights, bit for bit.
// Writes the exported file to argv[2] for the Python-side parser check.
import { writeFileSync } from "fs";
import { writeGGUF, readGGUF, GGUFValueType, tensorBytes } from "../../forge-llm_amd/src/L9/gguf.js";
import { exportGGUF, weightsFromGGUF } from "../../forge-llm_amd/src/L9/export.js";
import { Config } from "../../forge-llm_amd/src/L6/transformer.js";
import { initWeights } from "../../forge-llm_amd/src/L6/train.js";
import { RNG } from "../../forge-llm_amd/src/L0/numeric.js";

const out = [];
function rec(test, fn) {
  try { const r = fn(); out.push({ test, ok: !!r.ok, detail: r.detail || "" }); }
  catch (e) { out.push({ test, ok: false, error: String(e && e.stack || e) }); }
}
const same = (a, b) => a.length === b.length && a.every((v, i) => Object.is(v, b[i]));

rec("I-90: write → read keeps every metadata value and tensor", () => {
  const meta = new Map([
    ["general.architecture", "llama"], ["u32", 7], ["f32", 0.25], ["neg", -3], ["big", 4294967296], ["flag", true],
    ["no", false], ["names", ["a", "b", "ü"]], ["ints", [1, 2, 3]], ["floats", [0.5, -1.5]],
    ["f64", { ggufType: GGUFValueType.FLOAT64, value: 3e-4 }], ["u8", { ggufType: GGUFValueType.UINT8, value: 200 }],
    ["i64", { ggufType: GGUFValueType.INT64, value: -5 }],
  ]);
  const t1 = Float32Array.from([1, 2, 3, 4, 5, 6]);
  const t2 = new Uint8Array(34 * 2).map((_, i) => i);
  const { bytes } = writeGGUF({ meta, tensors: [
    { name: "a", dims: [3, 2], type: 0, data: new Uint8Array(t1.buffer) },
    { name: "q", dims: [64], type: 8, data: t2 },
  ] });
  const g = readGGUF(bytes);
  const m = g.meta;
  const ok = m.get("general.architecture") === "llama" && m.get("u32") === 7 && m.get("f32") === 0.25 &&
    m.get("neg") === -3 && m.get("big") === Math.fround(4294967296) && m.get("flag") === true && m.get("no") === false &&
    same(m.get("names"), ["a", "b", "ü"]) && same(m.get("ints"), [1, 2, 3]) && same(m.get("floats"), [0.5, -1.5]) &&
    m.get("f64") === 3e-4 && m.get("u8") === 200 && m.get("i64") === -5 && g.version === 3 &&
    same(Array.from(new Float32Array(g.getTensor("a").data.slice().buffer)), Array.from(t1)) &&
    same(Array.from(g.getTensor("q").data), Array.from(t2)) && g.getTensor("zz") === null;
  return { ok, detail: `${bytes.length} bytes` };
});

rec("I-91: tensor data starts on the alignment", () => {
  const tensors = [];
  for (let i = 0; i < 5; i++) tensors.push({ name: `t${i}`, dims: [i + 1], type: 0, data: new Uint8Array(4 * (i + 1)) });
  const { bytes, headerLen, dataStart } = writeGGUF({ meta: new Map([["general.alignment", 64]]), tensors });
  const g = readGGUF(bytes);
  const ok = dataStart % 64 === 0 && dataStart === g.tensorDataStart && headerLen <= dataStart && g.alignment === 64 && g.tensorDataStart % 64 === 0 && g.tensors.every((t) => t.offset % 64 === 0);
  return { ok, detail: g.tensors.map((t) => t.offset).join(",") };
});

rec("bad magic, truncation and partial blocks throw", () => {
  const { bytes } = writeGGUF({ meta: new Map([["x", 1]]), tensors: [] });
  const bad = bytes.slice(); bad[0] = 0;
  const t = (fn) => { try { fn(); return false; } catch (e) { return true; } };
  let msg = ""; try { readGGUF(bad); } catch (e) { msg = e.message; }
  const ok = /非法 GGUF magic/.test(msg) && t(() => readGGUF(bad)) && t(() => readGGUF(bytes.slice(0, 20))) && t(() => tensorBytes(8, 33)) &&
    tensorBytes(12, 512) === 288 && tensorBytes(14, 256) === 210 && tensorBytes(8, 64) === 68;
  return { ok };
});

function weightsFor(cfg, seed, untied) {
  const w = initWeights(cfg, seed);
  if (untied) {
    const r = new RNG(seed + 1);
    w.wcls = new Float32Array(cfg.vocabSize * cfg.dim);
    for (let i = 0; i < w.wcls.length; i++) w.wcls[i] = r.normal() * 0.02;
  }
  return w;
}

for (const untied of [false, true]) {
  rec(`export → re-import, ${untied ? "untied" : "tied"} head (GQA 4/2)`, () => {
    const cfg = new Config({ dim: 64, hidden: 128, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 31, maxSeq: 64, normEps: 1e-5 });
    const w = weightsFor(cfg, 20260101, untied);
    const bytes = exportGGUF(w, cfg, null, 0, "forge-demo");
    const g = readGGUF(bytes);
    const back = weightsFromGGUF(g, cfg);
    let ok = same(Array.from(back.tok_emb), Array.from(w.tok_emb)) && same(Array.from(back.ln_f), Array.from(w.ln_f)) &&
      (untied ? same(Array.from(back.wcls), Array.from(w.wcls)) : back.wcls === null);
    for (let l = 0; l < cfg.nLayers; l++)
      for (const k of ["ln1", "ln2", "wqkv", "wo", "ffn_gate", "ffn_up", "ffn_down"])
        ok = ok && same(Array.from(back[`layer.${l}`][k]), Array.from(w[`layer.${l}`][k]));
    const names = g.tensors.map((t) => t.name);
    ok = ok && names[0] === "token_embd.weight" && names[2] === "blk.0.attn_norm.weight" && names[3] === "blk.0.attn_q.weight" &&
      (g.getTensor("blk.0.attn_k.weight").dims.join() === "64,32") && g.meta.get("general.file_type") === 0;
    if (untied && process.argv[2]) writeFileSync(process.argv[2], bytes);
    return { ok, detail: `${g.tensors.length} tensors, ${bytes.length} bytes` };
  });
}

for (const r of out) console.log(JSON.stringify(r));
process.exit(out.every((r) => r.ok) ? 0 : 1);
