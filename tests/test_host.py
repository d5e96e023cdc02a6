"""CPU tests of the boundary and the host side (no GPU needed):

* libforge_hip.so loads and exports every entry point include/forge_hip.h
  declares; device entry points fail cleanly (FG_ERR_INIT) without a GPU;
  the host helpers (RoPE table, embedding plan) match the oracle;
* the N-API addon loads in Node and exposes the ops; the JS package loads,
  its RNG / initWeights / Config reproduce the oracle's, and ops throw a
  clear error when no device is present (no CPU fallback);
* the build recipe compiles for gfx950 only with packed-fp32 disabled.
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

import forge_hip
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def node_eval(code, timeout=120):
    r = subprocess.run(["node", "--input-type=module", "-e", code], cwd=os.path.join(ROOT, "forge-llm_amd"),
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    return r.returncode, r.stdout


def test_header_symbols_all_exported():
    assert forge_hip.MISSING == []
    assert len(forge_hip.DECLS) >= 40
    for name in forge_hip.DECLS:
        assert hasattr(forge_hip.lib, name)


def test_device_entry_points_fail_cleanly_without_init():
    if forge_hip.device_count() > 0:
        pytest.skip("a GPU is visible")
    p = ctypes.c_void_p()
    assert forge_hip.lib.fg_malloc(ctypes.byref(p), 64) == -4
    assert "fg_init" in forge_hip.last_error()
    assert forge_hip.lib.fg_init(0) == -4
    assert forge_hip.lib.fg_matmulT_fwd(None, None, None, 1, 1, 1) == -4


def test_rope_table_helper_matches_oracle():
    n, d = 33, 16
    c = np.empty(n * d // 2)
    s = np.empty(n * d // 2)
    forge_hip.check(forge_hip.lib.fg_rope_table(c.ctypes.data, s.ctypes.data, n, d, 5e5), "fg_rope_table")
    oc, os_ = oracle.rope_table(n, d, 5e5)
    np.testing.assert_array_equal(c, oc)
    np.testing.assert_array_equal(s, os_)


def test_embed_plan_helper():
    ids = np.array([3, 1, 3, 0, 3, 1], np.int32)
    perm = np.empty(6, np.int32)
    start = np.empty(7, np.int32)
    seg = np.empty(6, np.int32)
    ns = ctypes.c_int()
    forge_hip.check(forge_hip.lib.fg_embed_plan(ids.ctypes.data, 6, 5, perm.ctypes.data, start.ctypes.data,
                                                seg.ctypes.data, ctypes.byref(ns)), "fg_embed_plan")
    assert ns.value == 3
    assert list(seg[:3]) == [0, 1, 3] and list(start[:4]) == [0, 1, 3, 6]
    assert list(perm) == [3, 1, 5, 0, 2, 4]  # increasing t within each id
    bad = np.array([0, 9], np.int32)
    assert forge_hip.lib.fg_embed_plan(bad.ctypes.data, 2, 5, perm.ctypes.data, start.ctypes.data,
                                       seg.ctypes.data, ctypes.byref(ns)) == -1


def test_build_recipe_flags():
    src = open(os.path.join(ROOT, "forge-llm_amd", "build.py")).read()
    assert "--offload-arch=gfx950" in src and "-packed-fp32-ops" in src


def test_napi_addon_and_js_package_load():
    rc, out = node_eval("""
import { addonUninitialised } from './src/L2/device.js';
import * as F from './src/index.js';
const a = addonUninitialised();
const need = ['init','alloc','free','h2d','d2h','matmulTFwd','matmulTBwdX','matmulTBwdW','attnFwd','attnBwd',
  'ceFwd','ceBwd','rmsnormFwd','rmsnormBwd','ropeFwd','ropeBwd','swigluFwd','swigluBwd','embedFwd','embedBwd',
  'sliceColsFwd','sliceColsBwd','addFwd','accum','weightedSumFwd','weightedSumBwd','adamStep','readAsync','readWait'];
const missing = need.filter((k) => typeof a[k] !== 'function');
let err = '';
if (a.deviceCount() === 0) { try { F.matmulT(F.leaf([1]), F.leaf([1]), 1, 1, 1); } catch (e) { err = e.message; } }
console.log(JSON.stringify({ missing, exports: Object.keys(F).length, err, devices: a.deviceCount() }));
""")
    assert rc == 0, out
    r = json.loads(out.strip().splitlines()[-1])
    assert r["missing"] == [] and r["exports"] >= 35
    if r["devices"] == 0:
        assert "no HIP device" in r["err"]


def test_js_rng_matches_oracle():
    rc, out = node_eval("""
import { RNG } from './src/L0/numeric.js';
const r = new RNG(20260101); const a = [];
for (let i = 0; i < 200; i++) a.push(r.next());
for (let i = 0; i < 200; i++) a.push(r.normal());
for (let i = 0; i < 200; i++) a.push(r.int(32000));
console.log(JSON.stringify(a));
""")
    assert rc == 0, out
    js = json.loads(out)
    o = oracle.RNG(20260101)
    ref = [o.next() for _ in range(200)] + [o.normal() for _ in range(200)] + [o.int(32000) for _ in range(200)]
    assert js[:200] == ref[:200]
    np.testing.assert_allclose(js[200:400], ref[200:400], rtol=0, atol=1e-15)
    assert js[400:] == ref[400:]


def test_js_init_weights_and_config_match_oracle(tmp_path):
    out_file = tmp_path / "w.bin"
    rc, out = node_eval("""
import { writeFileSync } from 'fs';
import { Config, initWeights } from './src/index.js';
const cfg = new Config({ dim: 64, hidden: 128, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 31, maxSeq: 64 });
const w = initWeights(cfg, 20260101);
const parts = [w.tok_emb, w.ln_f];
for (let l = 0; l < 2; l++) { const L = w['layer.' + l]; parts.push(L.ln1, L.ln2, L.wqkv, L.wo, L.ffn_gate, L.ffn_up, L.ffn_down); }
let n = 0; for (const p of parts) n += p.length;
const all = new Float32Array(n); let o = 0; for (const p of parts) { all.set(p, o); o += p.length; }
writeFileSync('%s', Buffer.from(all.buffer));
console.log(JSON.stringify({ dHead: cfg.dHead, qkvOut: cfg.qkvOut, kvDim: cfg.kvDim, n }));
""" % str(out_file))
    assert rc == 0, out
    info = json.loads(out.strip().splitlines()[-1])
    assert (info["dHead"], info["qkvOut"], info["kvDim"]) == (16, 128, 32)
    cfg = oracle.Cfg(dim=64, hidden=128, nLayers=2, nHeads=4, nKvHeads=2, vocab=31, tied=1)
    ref = oracle.init_weights(cfg, 20260101)
    got = np.fromfile(str(out_file), np.float32)
    assert info["n"] == ref.size == 76032  # the demo model's parameter count
    np.testing.assert_array_equal(got, ref)


def test_js_config_rejects_bad_gqa():
    rc, out = node_eval("""
import { Config } from './src/index.js';
try { new Config({ nHeads: 6, nKvHeads: 4 }); console.log('no error'); } catch (e) { console.log('threw'); }
""")
    assert rc == 0 and out.strip() == "threw"


def test_gguf_host_js(tmp_path):
    """GGUF container and f32 export on the host (tests/js/gguf_host.mjs)."""
    out_file = tmp_path / "demo.gguf"
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "gguf_host.mjs"), str(out_file)],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    rows = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    bad = [x for x in rows if not x["ok"]]
    assert r.returncode == 0 and len(rows) == 5 and not bad, r.stdout


def _parse_gguf(b):
    """Minimal GGUF v3 reader written from the format description (u32 magic,
    u32 version, u64 counts, {u64-length string key, u32 type, value}*,
    {name, u32 n_dims, u64 dims, u32 type, u64 offset}*, aligned data)."""
    import struct
    p = [0]

    def take(fmt):
        v = struct.unpack_from("<" + fmt, b, p[0])
        p[0] += struct.calcsize("<" + fmt)
        return v[0]

    def string():
        n = take("Q")
        s = b[p[0]:p[0] + n].decode()
        p[0] += n
        return s

    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("I"), take("Q")
            return (et, [value(et) for _ in range(n)])
        return take(scalar[t])

    assert take("I") == 0x46554747 and take("I") == 3
    nT, nKv = take("Q"), take("Q")
    meta = []
    for _ in range(nKv):
        k = string()
        t = take("I")
        meta.append((k, t, value(t)))
    tensors = []
    for _ in range(nT):
        name = string()
        dims = [take("Q") for _ in range(take("I"))]
        tensors.append((name, dims, take("I"), take("Q")))
    start = -(-p[0] // 32) * 32
    return meta, tensors, start


def test_gguf_export_layout_matches_oracle_weights(tmp_path):
    """The exported file, read by an independent parser: llama metadata with
    the reference writer's key order and value types (engine.js:127-143,
    gguf.js:181-185: integers in [0, 2^32) are UINT32, other numbers FLOAT32),
    tensor names, ggml dims [K, N], 32-byte-aligned offsets, and the tensor
    bytes equal to the oracle's initWeights (wqkv split by rows into q/k/v)."""
    out_file = tmp_path / "demo.gguf"
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "gguf_host.mjs"), str(out_file)],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    b = out_file.read_bytes()
    meta, tensors, start = _parse_gguf(b)
    U32, F32, STR = 4, 6, 8
    assert meta == [
        ("general.architecture", STR, "llama"), ("general.name", STR, "forge-demo"),
        ("general.quantization_version", U32, 2), ("general.alignment", U32, 32),
        ("llama.block_count", U32, 2), ("llama.embedding_length", U32, 64), ("llama.feed_forward_length", U32, 128),
        ("llama.attention.head_count", U32, 4), ("llama.attention.head_count_kv", U32, 2),
        ("llama.context_length", U32, 64),
        ("llama.attention.layer_norm_rms_epsilon", F32, float(np.float32(1e-5))),
        ("llama.vocab_size", U32, 31), ("llama.rope.freq_base", U32, 10000), ("general.file_type", U32, 0)]

    cfg = oracle.Cfg(dim=64, hidden=128, nLayers=2, nHeads=4, nKvHeads=2, vocab=31, tied=1)
    P = oracle.split_params(cfg, oracle.init_weights(cfg, 20260101))
    rng = oracle.RNG(20260102)
    wcls = np.array([rng.normal() * 0.02 for _ in range(31 * 64)], np.float64).astype(np.float32)
    D, H, qD, kvD = 64, 128, 64, 32
    expect = [("token_embd.weight", [D, 31], P["tok_emb"]), ("output_norm.weight", [D], P["ln_f"])]
    for l in range(2):
        L = lambda k: P["layer.%d.%s" % (l, k)]
        wqkv = L("wqkv")
        expect += [("blk.%d.attn_norm.weight" % l, [D], L("ln1")),
                   ("blk.%d.attn_q.weight" % l, [D, qD], wqkv[:qD * D]),
                   ("blk.%d.attn_k.weight" % l, [D, kvD], wqkv[qD * D:(qD + kvD) * D]),
                   ("blk.%d.attn_v.weight" % l, [D, kvD], wqkv[(qD + kvD) * D:]),
                   ("blk.%d.attn_output.weight" % l, [D, D], L("wo")),
                   ("blk.%d.ffn_norm.weight" % l, [D], L("ln2")),
                   ("blk.%d.ffn_gate.weight" % l, [D, H], L("ffn_gate")),
                   ("blk.%d.ffn_up.weight" % l, [D, H], L("ffn_up")),
                   ("blk.%d.ffn_down.weight" % l, [H, D], L("ffn_down"))]
    expect.append(("output.weight", [D, 31], wcls))
    assert [(n, d, t) for n, d, t, _ in tensors] == [(n, d, 0) for n, d, _ in expect]
    off = 0
    for (name, dims, _, o), (_, _, want) in zip(tensors, expect):
        assert o == off and (start + o) % 32 == 0, name
        got = np.frombuffer(b, np.float32, count=want.size, offset=start + o)
        np.testing.assert_array_equal(got, want, err_msg=name)
        off += -(-want.size * 4 // 32) * 32
    assert len(b) == start + off
