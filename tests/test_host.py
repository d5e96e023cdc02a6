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
