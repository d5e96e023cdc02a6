"""Pins the oracle's quantized-weight functions (oracle/quant_oracle.c), CPU only.

The reference's quantization (src/L3/quant.js) cannot run here (Node 12), so
its restatement is checked against:

* the reference's own L3/L4 tests (test/l3-l5.test.js:17-149), restated with
  the oracle's RNG: bits per weight, rowBytes, F16 round trip, the Q8_0 error
  bound, dotQ vs dequantize-then-dot, the Q5_K size / error / qh use, the Q6_K
  d-at-the-tail scaling test, the quality report, QuantLinear cosine and toF32;
* an independent vectorised numpy decoder written from the GGML block layouts
  (llama.cpp ggml-quants / gguf-py quants), applied both to random blocks and
  to the oracle's own quantizer output — a wrong nibble, bit or scale index in
  either the oracle's decoder or its encoder fails here;
* hand-built blocks with answers worked out from the layout by hand;
* the fp16 conversions: every one of the 65536 halves against numpy, random
  fp64 values against numpy's correctly rounded conversion, and the
  reference's own rounding at ties (Math.round: half-way goes up in
  magnitude, where IEEE rounds to even) and its subnormal wrap;
* the typed-weight decode forward against the f32 decode of the dequantized
  weights.

What no check here fixes: which candidate scale the make_qx_quants /
make_qkx2_quants searches of Q6_K / Q5_K keep when two are within rounding of
each other; for those, bytes are pinned only through the properties above.
"""
import numpy as np
import pytest

import oracle

F16, Q8_0, Q4_K, Q5_K, Q6_K, Q4_0 = 1, 8, 12, 13, 14, 2


# ── independent GGML-layout decoder (numpy, vectorised) ──────────────────
def _h(b):
    return b.view(np.float16).astype(np.float64)


def ggml_decode(t, q, n):
    q = np.asarray(q, np.uint8)
    if t == F16:
        return q.view(np.float16).astype(np.float32)[:n]
    if t == Q8_0:
        blk = q.reshape(-1, 34)
        d = _h(blk[:, :2].copy()).reshape(-1, 1)
        return ((blk[:, 2:].view(np.int8).astype(np.float64)) * d).astype(np.float32).ravel()[:n]
    if t in (Q4_K, Q5_K):
        bb = 144 if t == Q4_K else 176
        blk = q.reshape(-1, bb)
        d = _h(blk[:, 0:2].copy()).reshape(-1, 1)
        dmin = _h(blk[:, 2:4].copy()).reshape(-1, 1)
        s = blk[:, 4:16].astype(np.int64)
        sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)], axis=1)
        mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        qs = blk[:, -128:].astype(np.int64).reshape(-1, 4, 32)
        vals = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32)  # sub-block 2c: low, 2c+1: high
        if t == Q5_K:
            qh = blk[:, 16:48].astype(np.int64)  # bit i of qh[l] is bit 4 of sub-block i, element l
            bits = np.stack([(qh >> i) & 1 for i in range(8)], axis=1)
            vals = vals + 16 * bits
        out = (d[:, :, None] * sc[:, :, None]) * vals - (dmin[:, :, None] * mn[:, :, None])
        return out.astype(np.float32).ravel()[:n]
    if t == Q6_K:
        blk = q.reshape(-1, 210)
        ql = blk[:, 0:128].astype(np.int64).reshape(-1, 2, 64)
        qh = blk[:, 128:192].astype(np.int64).reshape(-1, 2, 32)
        sc = blk[:, 192:208].view(np.int8).astype(np.float64)
        d = _h(blk[:, 208:210].copy()).reshape(-1, 1)
        lo, hi = ql[:, :, :32], ql[:, :, 32:]
        g = [(lo & 0xF) | ((qh & 3) << 4), (hi & 0xF) | (((qh >> 2) & 3) << 4),
             (lo >> 4) | (((qh >> 4) & 3) << 4), (hi >> 4) | (((qh >> 6) & 3) << 4)]
        qv = (np.stack(g, axis=2) - 32).reshape(-1, 256)  # element 128h + 32g + l
        scale = np.repeat(sc, 16, axis=1)  # element e uses scale e // 16
        return ((d * scale) * qv).astype(np.float32).ravel()[:n]
    raise ValueError(t)


def random_blocks(t, nblocks, seed):
    rs = np.random.default_rng(seed)
    bs, bb = oracle.BLOCK[t]
    q = rs.integers(0, 256, size=nblocks * bb, dtype=np.uint8)
    blk = q.reshape(nblocks, bb)
    d = rs.uniform(1e-3, 1.0, size=nblocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if t == Q6_K:
        blk[:, 208:210] = d
    else:
        blk[:, 0:2] = d
    if t in (Q4_K, Q5_K):
        blk[:, 2:4] = rs.uniform(1e-3, 0.5, size=nblocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return q


# ── the reference's L3/L4 tests (test/l3-l5.test.js:17-149) ──────────────
def test_bpw_and_row_bytes():
    bpw = {t: 8.0 * bb / bs for t, (bs, bb) in oracle.BLOCK.items()}
    assert (bpw[Q4_K], bpw[Q5_K], bpw[Q6_K], bpw[Q8_0], bpw[F16], bpw[0]) == (4.5, 5.5, 6.5625, 8.5, 16, 32)
    rb = oracle.row_bytes
    assert (rb(Q4_K, 256), rb(Q4_K, 512), rb(Q6_K, 256), rb(Q8_0, 32), rb(Q8_0, 64), rb(0, 100)) == \
        (144, 288, 210, 34, 68, 400)


def _normals(seed, n, scale=1.0):
    r = oracle.RNG(seed)
    return np.array([r.normal() * scale for _ in range(n)], np.float64).astype(np.float32)


def test_f16_round_trip():
    x = _normals(1, 64)
    dq = oracle.dequantize(F16, oracle.quantize(F16, x), 64)
    assert np.max(np.abs(dq - x) / (np.abs(x) + 1e-3)) < 1e-3


def test_q8_0_error_bound():
    x = _normals(2, 256)
    dq = oracle.dequantize(Q8_0, oracle.quantize(Q8_0, x), 256)
    amax = np.max(np.abs(x))
    assert np.max(np.abs(dq - x)) <= amax / 254 + 1e-6


def test_dotq_equals_dequantize_then_dot():
    r = oracle.RNG(3)
    x, y = np.empty(512, np.float32), np.empty(512, np.float32)
    for i in range(512):
        x[i] = r.normal() * 0.8
        y[i] = r.normal()
    for t in (F16, Q8_0, Q4_K, Q5_K, Q6_K):
        q = oracle.quantize(t, x)
        a = float(np.dot(oracle.dequantize(t, q, 512).astype(np.float64), y.astype(np.float64)))
        b = oracle.dotq(t, q, y)
        assert abs(a - b) <= 1e-3 * (abs(a) + 1), (t, a, b)
        # and, tighter: the fp64 sum of the exact decoded values (before their fp32 rounding)
        assert abs(a - b) <= 1e-6 * np.sum(np.abs(y)) * np.max(np.abs(x)), (t, a, b)


def test_q5_k_size_error_and_fifth_bit():
    x = _normals(7, 256, 0.5)
    q = oracle.quantize(Q5_K, x)
    assert q.size == 176
    dq = oracle.dequantize(Q5_K, q, 256)
    assert np.sqrt(np.sum((dq - x) ** 2) / np.sum(x.astype(np.float64) ** 2)) < 0.05
    assert np.count_nonzero(q[16:48]) > 0


def test_q6_k_scale_at_block_end():
    x = _normals(8, 256)
    y = (x.astype(np.float64) * 4).astype(np.float32)
    qx, qy = oracle.quantize(Q6_K, x), oracle.quantize(Q6_K, y)
    assert qx.size == 210
    assert np.array_equal(qx[:208], qy[:208]) and not np.array_equal(qx[208:], qy[208:])
    half = lambda q: oracle.fp16_to_fp32(int(q[208]) | (int(q[209]) << 8))  # noqa: E731
    dx, dy = half(qx), half(qy)
    assert abs(dy / dx - 4) < 0.02


def _cos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return float(np.dot(a, b) / np.sqrt(np.dot(a, a) * np.dot(b, b)))


def test_quality_report():
    x = _normals(4, 1024, 0.6)
    for t, lo, hi, cmin in ((Q8_0, 3.5, 4.0, 0.999), (Q4_K, 6.5, 7.5, 0.995)):
        q = oracle.quantize(t, x)
        ratio = 4096 / q.size
        assert lo < ratio < hi and _cos(x, oracle.dequantize(t, q, 1024)) > cmin


def test_quant_linear_q8_0_close_to_f32():
    r = oracle.RNG(5)
    N, K = 64, 128
    W = np.array([r.normal() for _ in range(N * K)]).astype(np.float32)
    x = np.array([r.normal() for _ in range(K)]).astype(np.float32)
    o1 = oracle.qmatvec(0, W.view(np.uint8), x, N, K)
    o2 = oracle.qmatvec(Q8_0, oracle.quantize(Q8_0, W), x, N, K)
    assert _cos(o1, o2) > 0.999
    # type 0 is numeric.js matvec: the fp64 product sum rounded once
    np.testing.assert_allclose(o1, (W.reshape(N, K).astype(np.float64) @ x.astype(np.float64)), rtol=1e-6)


def test_to_f32_equals_dequantize():
    W = _normals(6, 32 * 64)
    q = oracle.quantize(Q8_0, W)
    assert np.array_equal(oracle.dequantize(Q8_0, q, W.size), ggml_decode(Q8_0, q, W.size))


# ── independent decoder ───────────────────────────────────────────────────
@pytest.mark.parametrize("t", [F16, Q8_0, Q4_K, Q5_K, Q6_K])
def test_dequantize_matches_ggml_layout_on_random_blocks(t):
    nb = 64 if oracle.BLOCK[t][0] == 256 else 512
    q = random_blocks(t, nb, 100 + t)
    n = nb * oracle.BLOCK[t][0]
    if t == F16:
        q = np.random.default_rng(5).uniform(-4, 4, n).astype(np.float16).view(np.uint8)
    a, b = oracle.dequantize(t, q, n), ggml_decode(t, q, n)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("t", [F16, Q8_0, Q4_K, Q5_K, Q6_K])
def test_quantizer_output_decodes_by_the_ggml_layout(t):
    rs = np.random.default_rng(t)
    x = (rs.standard_normal(4096) * 0.05).astype(np.float32)
    x[256:512] = np.abs(x[256:512]) + 0.01  # an all-positive block (the K-quants' min > 0 branch)
    x[512:768] = 0.0                         # an all-zero block
    x[768:1024] = 0.3                        # a constant block
    q = oracle.quantize(t, x)
    assert q.size == oracle.row_bytes(t, x.size)
    d = ggml_decode(t, q, x.size)
    assert np.array_equal(d.view(np.uint32), oracle.dequantize(t, q, x.size).view(np.uint32))
    err = np.sqrt(np.sum((d - x) ** 2) / np.sum(x.astype(np.float64) ** 2))
    assert err < {F16: 1e-3, Q8_0: 0.01, Q4_K: 0.12, Q5_K: 0.06, Q6_K: 0.03}[t], err
    assert np.all(d[512:768] == 0)


def test_known_answer_blocks():
    # Q4_K: d = 1, dmin = 0.5; sub-block 0 scale 2 min 3, sub-block 1 scale 1 min 0;
    # qs[0] = 0x5A: element 0 = 1·2·10 − 0.5·3 = 18.5, element 32 = 1·1·5 − 0 = 5.
    b = np.zeros(144, np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[2:4] = [0x00, 0x38]
    b[4], b[5], b[8] = 2, 1, 3
    b[16] = 0x5A
    v = oracle.dequantize(Q4_K, b, 256)
    assert (v[0], v[32], v[1]) == (18.5, 5.0, -1.5)
    # Q5_K: the same, plus qh[0] bit 0 → element 0 gains 16: 1·2·26 − 1.5 = 50.5
    b5 = np.zeros(176, np.uint8)
    b5[0:16] = b[0:16]
    b5[16] = 1
    b5[48] = 0x5A
    v = oracle.dequantize(Q5_K, b5, 256)
    assert (v[0], v[32]) == (50.5, 5.0)
    # Q6_K: d = 0.25 at bytes 208-209; scales[0] = 4, scales[4] = −1; ql[0] = 0x21,
    # qh[0] = 0b10: element 0 = 0.25·4·((1 | 2<<4) − 32) = 1.0,
    # element 64 = 0.25·(−1)·((2 | 0<<4) − 32) = 7.5.
    b6 = np.zeros(210, np.uint8)
    b6[208:210] = [0x00, 0x34]
    b6[192], b6[196] = 4, 0xFF
    b6[0], b6[128] = 0x21, 0b10
    v = oracle.dequantize(Q6_K, b6, 256)
    assert (v[0], v[64]) == (1.0, 7.5)
    # Q8_0: d = 2, qs = [−3, 127]
    b8 = np.zeros(34, np.uint8)
    b8[0:2] = [0x00, 0x40]
    b8[2], b8[3] = 0xFD, 127
    v = oracle.dequantize(Q8_0, b8, 32)
    assert (v[0], v[1]) == (-6.0, 254.0)


# ── fp16 conversions (special.js:143-168) ─────────────────────────────────
def test_fp16_to_fp32_all_halves():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float64)
    got = np.array([oracle.fp16_to_fp32(int(v)) for v in h])
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan], ref[~nan])


def test_fp32_to_fp16_rounding():
    rs = np.random.default_rng(0)
    x = np.concatenate([rs.standard_normal(20000) * 10.0 ** rs.integers(-9, 5, 20000),
                        rs.uniform(-70000, 70000, 2000)])
    got = np.array([oracle.fp32_to_fp16(v) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)  # no random value sits exactly on a tie
    # the reference's ties: Math.round sends half-way cases up in magnitude
    assert oracle.fp32_to_fp16(1 + 2 ** -11) == 0x3C01          # IEEE (even) would give 0x3C00
    assert oracle.fp32_to_fp16(-(1 + 2 ** -11)) == 0xBC01
    assert oracle.fp32_to_fp16(1 + 3 * 2 ** -11) == 0x3C02
    assert oracle.fp32_to_fp16(2.0 ** -25) == 0x0001              # half the smallest subnormal
    assert oracle.fp32_to_fp16(2.0 ** -14 - 2.0 ** -26) == 0x0000  # round(x·2^24) = 1024 wraps to 0
    assert oracle.fp32_to_fp16(65519.0) == 0x7BFF and oracle.fp32_to_fp16(65520.0) == 0x7C00
    assert oracle.fp32_to_fp16(float("nan")) == 0x7E00 and oracle.fp32_to_fp16(float("-inf")) == 0xFC00


# ── typed-weight decode forward ───────────────────────────────────────────
def _typed_model(cfg, P, types):
    tq = lambda t, w: (t, oracle.quantize(t, w))  # noqa: E731
    layers = []
    for l in range(cfg.nLayers):
        g = lambda k: P["layer.%d.%s" % (l, k)]  # noqa: E731
        layers.append({"ln1": g("ln1"), "ln2": g("ln2"), "wqkv": tq(types["wqkv"], g("wqkv")),
                       "wo": tq(types["wo"], g("wo")), "gate": tq(types["gate"], g("ffn_gate")),
                       "up": tq(types["gate"], g("ffn_up")), "down": tq(types["down"], g("ffn_down"))})
    emb = tq(types["emb"], P["tok_emb"])
    return {"tok_emb": emb, "ln_f": P["ln_f"], "layers": layers,
            "wcls": tq(types["cls"], P["wcls"]) if "wcls" in P else emb}


def _dequantized_params(cfg, model):
    dq = lambda tb, n: oracle.dequantize(tb[0], tb[1], n)  # noqa: E731
    d, h, v = cfg.dim, cfg.hidden, cfg.vocab
    parts = [dq(model["tok_emb"], v * d), model["ln_f"]]
    if not cfg.tied:
        parts.append(dq(model["wcls"], v * d))
    for L in model["layers"]:
        parts += [L["ln1"], L["ln2"], dq(L["wqkv"], cfg.qkvOut * d), dq(L["wo"], d * d), dq(L["gate"], h * d),
                  dq(L["up"], h * d), dq(L["down"], d * h)]
    return np.concatenate(parts).astype(np.float32)


@pytest.mark.parametrize("types", [
    {"emb": 0, "cls": 0, "wqkv": Q4_K, "wo": Q6_K, "gate": Q5_K, "down": Q8_0},
    {"emb": Q8_0, "cls": Q6_K, "wqkv": F16, "wo": Q4_K, "gate": Q4_K, "down": Q6_K},
])
def test_typed_decode_equals_f32_decode_of_dequantized_weights(types):
    cfg = oracle.Cfg(dim=256, hidden=512, nLayers=2, nHeads=4, nKvHeads=2, vocab=64, tied=0)
    P = oracle.split_params(cfg, oracle.init_weights(cfg, 11))
    rs = np.random.default_rng(1)
    P["wcls"] = (rs.standard_normal(64 * 256) * 0.02).astype(np.float32)
    model = _typed_model(cfg, P, types)
    ids = [3, 17, 0, 63, 5]
    a = oracle.infer_forward_q(cfg, model, ids)
    b = oracle.infer_forward(cfg, _dequantized_params(cfg, model), ids)
    rel = np.linalg.norm(a - b) / np.linalg.norm(b)
    assert rel < 1e-6, rel
    # type 0 everywhere is the f32 decode itself
    f32m = _typed_model(cfg, P, {k: 0 for k in types})
    assert np.array_equal(oracle.infer_forward_q(cfg, f32m, ids),
                          oracle.infer_forward(cfg, _dequantized_params(cfg, f32m), ids))
