"""The inference forward (Transformer.forward, transformer.js:134-184) on the
device, through fg_decode_step, against the oracle's token-by-token decode
(oracle/forge_oracle.c or_infer_forward: the reference's matvec, RMSNorm,
fp32 RoPE table, attentionDecode and SwiGLU restated in C).

Every position's logits must be within the forward tolerance (relative L2
1e-5); the matvecs sum in fp64 like the reference, so logits agree to the
last bit at position 0; later positions carry the attention's fp64 sums
(the reference accumulates p·V in fp32), within ~1e-7.  The JavaScript
Transformer / KVCache classes (graph replay, I-70 on the device) are covered
by tests/js/decode.mjs.
"""
import ctypes
import math
import os
import subprocess

import numpy as np
import pytest

import oracle
from util import TOL_FWD, rel_l2

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def rope_f32(maxSeq, dH, theta):
    half = dH // 2
    c = np.empty(maxSeq * half, np.float32)
    s = np.empty(maxSeq * half, np.float32)
    for p in range(maxSeq):
        for i in range(0, dH, 2):
            ang = p * (1.0 / math.pow(theta, i / dH))
            c[p * half + i // 2] = math.cos(ang)
            s[p * half + i // 2] = math.sin(ang)
    return c, s


class Decoder:
    """fg_decode_model over device copies of the oracle's flat parameters.

    `types` gives ggml types for the matrices ({"emb", "cls", "wqkv", "wo",
    "gate", "down"}; up shares gate's type; absent = f32): those are
    quantized by the oracle's quantizeRow and uploaded as bytes, and
    `oracle_logits` decodes the same bytes with the oracle."""

    def __init__(self, fh, cfg, params, maxSeq, types=None):
        self.fh, self.cfg, self.maxSeq = fh, cfg, maxSeq
        self.types = types = dict(types or {})
        P = oracle.split_params(cfg, params)
        if "wcls" not in P:
            P["wcls"] = P["tok_emb"]
        up = lambda a: fh.DeviceArray.from_numpy(np.ascontiguousarray(a))  # noqa: E731
        kind = {"tok_emb": "emb", "wcls": "cls"}
        for l in range(cfg.nLayers):
            for k, t in (("wqkv", "wqkv"), ("wo", "wo"), ("ffn_gate", "gate"), ("ffn_up", "gate"),
                         ("ffn_down", "down")):
                kind["layer.%d.%s" % (l, k)] = t
        self.host = {}  # (type, bytes or f32) per matrix, for the oracle
        self.keep = {}
        for k, v in P.items():
            t = types.get(kind.get(k), 0)
            if k in kind and t:
                b = oracle.quantize(t, v)
                self.host[k] = (t, b)
                self.keep[k] = up(b)
            else:
                self.host[k] = (0, np.ascontiguousarray(v, np.float32))
                self.keep[k] = up(np.ascontiguousarray(v, np.float32))
        self.P = P
        D, H, V = cfg.dim, cfg.hidden, cfg.vocab
        c, s = rope_f32(maxSeq, cfg.dHead, cfg.ropeTheta)
        self.keep["rope_cos"], self.keep["rope_sin"] = up(c), up(s)
        for name, n in [("x", D), ("q", cfg.nHeads * cfg.dHead), ("h", H), ("logits", V)]:
            self.keep[name] = fh.DeviceArray((n,))
        nd = ctypes.c_int64(0)
        fh.check(fh.lib.fg_decode_part_len(cfg.nHeads, cfg.dHead, maxSeq, ctypes.byref(nd)), "fg_decode_part_len")
        self.keep["attn_part"] = fh.DeviceArray((nd.value,), np.float64)
        kvD = cfg.nKvHeads * cfg.dHead
        self.kc = fh.DeviceArray.zeros((cfg.nLayers * maxSeq * kvD,))
        self.vc = fh.DeviceArray.zeros((cfg.nLayers * maxSeq * kvD,))
        self.state = fh.DeviceArray((2,), np.int32)
        self.layers = (fh.DecodeLayer * cfg.nLayers)()
        for l in range(cfg.nLayers):
            g = lambda k: self.keep["layer.%d.%s" % (l, k)].ptr  # noqa: E731
            self.layers[l] = fh.DecodeLayer(g("ln1"), g("wqkv"), g("wo"), g("ln2"), g("ffn_gate"), g("ffn_up"),
                                            g("ffn_down"), types.get("wqkv", 0), types.get("wo", 0),
                                            types.get("gate", 0), types.get("gate", 0), types.get("down", 0))
        k = self.keep
        self.m = fh.DecodeModel(D, H, cfg.nLayers, cfg.nHeads, cfg.nKvHeads, V, maxSeq, types.get("emb", 0),
                                types.get("cls", 0), cfg.normEps, k["tok_emb"].ptr, k["ln_f"].ptr, k["wcls"].ptr,
                                ctypes.cast(self.layers, ctypes.c_void_p), k["rope_cos"].ptr, k["rope_sin"].ptr,
                                k["x"].ptr, k["q"].ptr, k["h"].ptr, k["attn_part"].ptr)

    def oracle_logits(self, ids):
        h, P = self.host, self.P
        layers = [{"ln1": P["layer.%d.ln1" % l], "ln2": P["layer.%d.ln2" % l],
                   "wqkv": h["layer.%d.wqkv" % l], "wo": h["layer.%d.wo" % l], "gate": h["layer.%d.ffn_gate" % l],
                   "up": h["layer.%d.ffn_up" % l], "down": h["layer.%d.ffn_down" % l]}
                  for l in range(self.cfg.nLayers)]
        model = {"tok_emb": h["tok_emb"], "ln_f": P["ln_f"], "wcls": h["wcls"], "layers": layers}
        return oracle.infer_forward_q(self.cfg, model, ids).reshape(len(ids), self.cfg.vocab)

    def step(self, token, pos):
        self.state.upload(np.array([token, pos], np.int32))
        self.fh.check(self.fh.lib.fg_decode_step(ctypes.byref(self.m), self.kc.ptr, self.vc.ptr, self.state.ptr,
                                                 self.keep["logits"].ptr), "fg_decode_step")
        return self.keep["logits"].numpy()


CASES = {
    # verify.js:288-310 (I-70) shape
    "i70": (dict(dim=32, hidden=64, nLayers=2, nHeads=4, nKvHeads=2, vocab=40, tied=1), 4242, 6),
    # dH 64, GQA 2:1, untied head, 40 positions
    "dh64_gqa": (dict(dim=256, hidden=512, nLayers=2, nHeads=4, nKvHeads=2, vocab=300, tied=0), 7, 40),
    # dH 128 (two dims per lane), hidden and dim not multiples of 256
    "dh128": (dict(dim=512, hidden=200, nLayers=1, nHeads=4, nKvHeads=1, vocab=100, tied=1), 8, 20),
    # K not a multiple of 4 (scalar dot path), dH 22
    "odd_k": (dict(dim=44, hidden=30, nLayers=2, nHeads=2, nKvHeads=1, vocab=50, tied=0), 9, 12),
    # 300 positions: five position chunks per head
    "long": (dict(dim=128, hidden=128, nLayers=1, nHeads=2, nKvHeads=1, vocab=64, tied=1, ropeTheta=5e5), 10, 300),
    # dH 48 (lane groups of 16 with idle lanes), dH 256 (64 lanes per position)
    "dh48": (dict(dim=96, hidden=64, nLayers=1, nHeads=2, nKvHeads=2, vocab=30, tied=1), 11, 70),
    "dh256": (dict(dim=512, hidden=96, nLayers=1, nHeads=2, nKvHeads=1, vocab=30, tied=1), 12, 70),
    # above 256 dims: two (dH 384, the second group half idle) and four float4 groups per lane (dH 1024)
    "dh384": (dict(dim=768, hidden=96, nLayers=1, nHeads=2, nKvHeads=1, vocab=30, tied=1), 15, 70),
    "dh1024": (dict(dim=2048, hidden=64, nLayers=1, nHeads=2, nKvHeads=2, vocab=20, tied=0), 16, 40),
    # the smallest heads: dH 2 (one lane per position) and dH 6 (two lanes, scalar dots)
    "tiny": (dict(dim=4, hidden=3, nLayers=1, nHeads=2, nKvHeads=1, vocab=5, tied=0), 13, 9),
    "dh6": (dict(dim=12, hidden=7, nLayers=2, nHeads=2, nKvHeads=2, vocab=11, tied=1), 14, 70),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CASES))
def test_decode_step_vs_oracle(fh, name):
    kw, seed, T = CASES[name]
    cfg = oracle.Cfg(**kw)
    params = oracle.init_weights(cfg, seed)
    if not cfg.tied:  # a distinct head matrix
        P = oracle.split_params(cfg, params)
        P["wcls"][:] = np.random.default_rng(seed).standard_normal(P["wcls"].size).astype(np.float32) * 0.02
    ids = np.random.default_rng(seed + 1).integers(0, cfg.vocab, T).astype(np.int32)
    ref = oracle.infer_forward(cfg, params, ids).reshape(T, cfg.vocab)
    dec = Decoder(fh, cfg, params, maxSeq=T + 3)
    got = np.stack([dec.step(int(ids[t]), t) for t in range(T)])
    err = rel_l2(got, ref)
    same0 = float(np.mean(got[0] == ref[0]))
    print("%s: rel-L2 %.2e, identical logits %.1f%% (position 0: %.1f%%)"
          % (name, err, 100 * np.mean(got == ref), 100 * same0))
    assert err <= TOL_FWD
    # At position 0 the attention is exact (one key, p = 1), so only fp64 sum
    # orders differ from the reference: the logits agree bit for bit except at
    # rounding ties.  An fp32-accumulating matvec would miss most of them.
    assert same0 > 0.95


@pytest.mark.gpu
def test_decode_bad_token_is_nan_and_bad_position_writes_nothing(fh):
    cfg = oracle.Cfg(dim=32, hidden=64, nLayers=1, nHeads=4, nKvHeads=2, vocab=40, tied=1)
    dec = Decoder(fh, cfg, oracle.init_weights(cfg, 3), maxSeq=4)
    assert np.isnan(dec.step(40, 0)).all()  # NaN row, as the reference's undefined embedding
    kc0 = dec.kc.numpy()
    dec.step(1, 4)  # outside [0, maxSeq): no cache write
    np.testing.assert_array_equal(dec.kc.numpy(), kc0)
    assert np.isfinite(dec.step(1, 0)).all()  # position 0 rewritten with a valid token
    assert np.isfinite(dec.step(2, 1)).all()


@pytest.mark.gpu
def test_decode_rejects_bad_models(fh):
    cfg = oracle.Cfg(dim=32, hidden=64, nLayers=1, nHeads=4, nKvHeads=2, vocab=40, tied=1)
    dec = Decoder(fh, cfg, oracle.init_weights(cfg, 3), maxSeq=4)
    dec.m.nKvHeads = 3
    with pytest.raises(fh.ForgeError, match="nKvHeads"):
        dec.step(1, 0)
    dec.m.nKvHeads = 2
    dec.layers[0].wo = None
    with pytest.raises(fh.ForgeError, match="null weight"):
        dec.step(1, 0)


@pytest.mark.gpu
def test_decode_js(fh):
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "decode.mjs")], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    import json
    res = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    for x in res:
        print(x["test"], "ok" if x["ok"] else "FAIL", x.get("detail") or x.get("error", ""))
    assert r.returncode == 0 and res and all(x["ok"] for x in res), r.stdout[-4000:]


def _random_decode_cases(n, seed):
    """Seeded random model shapes inside the decode step's limits: even head
    dims up to 300, GQA, odd hidden widths and vocabularies, tied or untied."""
    rs = np.random.default_rng(seed)
    out = {}
    while len(out) < n:
        dH = 2 * int(rs.integers(1, 151))
        nKV = int(rs.integers(1, 4))
        nH = nKV * int(rs.integers(1, 4))
        if nH * dH > 2048:
            continue
        kw = dict(dim=nH * dH, hidden=int(rs.integers(1, 3000)), nLayers=int(rs.integers(1, 3)), nHeads=nH,
                  nKvHeads=nKV, vocab=int(rs.integers(2, 700)), tied=int(rs.integers(0, 2)),
                  ropeTheta=float(rs.choice([1e4, 5e5])))
        out["r%d_d%d_h%dx%d" % (len(out), nH * dH, nH, dH)] = (kw, int(rs.integers(1, 1 << 20)),
                                                                int(rs.integers(1, 150)))
    return out


RANDOM_CASES = _random_decode_cases(10, 31)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(RANDOM_CASES))
def test_decode_random_shapes_vs_oracle(fh, name):
    """Every position's logits against the oracle's token-by-token decode."""
    kw, seed, T = RANDOM_CASES[name]
    cfg = oracle.Cfg(**kw)
    params = oracle.init_weights(cfg, seed)
    if not cfg.tied:
        P = oracle.split_params(cfg, params)
        P["wcls"][:] = np.random.default_rng(seed).standard_normal(P["wcls"].size).astype(np.float32) * 0.02
    ids = np.random.default_rng(seed + 1).integers(0, cfg.vocab, T).astype(np.int32)
    ref = oracle.infer_forward(cfg, params, ids).reshape(T, cfg.vocab)
    dec = Decoder(fh, cfg, params, maxSeq=T + 1)
    got = np.stack([dec.step(int(ids[t]), t) for t in range(T)])
    assert rel_l2(got, ref) <= TOL_FWD
