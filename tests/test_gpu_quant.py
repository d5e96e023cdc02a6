"""Quantized weights on the device against the oracle (oracle/quant_oracle.c):

* fg_dequantize — bit-identical to the reference's dequantize, every type,
  random blocks, and all 65536 fp16 values;
* fg_quantize — bit-identical bytes to the reference's quantizeRow for F32,
  F16, Q8_0, Q4_K, Q5_K and Q6_K over normal data at several scales and the
  corner blocks (zeros, constants, all-positive, tiny values whose scales are
  fp16 subnormals, large values);
* fg_qmatvec — QuantLinear.forward / dotQ at ragged and real shapes (x in
  LDS and, for K > 16384, read from global memory): f32 rows sum in fp64 like
  the reference (within 1e-7 relative, almost every output bit-identical);
  quantized rows sum each lane's sub-block in fp32 before the fp64 scale and
  row sums (within the forward tolerance, ~3e-7 relative L2 at N ≥ 64);
* fg_decode_step over quantized matrices — the typed-weight decode of the
  oracle on the same bytes, at the forward tolerance.
"""
import ctypes

import numpy as np
import pytest

import oracle
from test_gpu_decode import Decoder
from util import TOL_FWD, rel_l2

TYPES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q5_0": 6, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
QUANTIZERS = ["F32", "F16", "Q8_0", "Q4_K", "Q5_K", "Q6_K"]


def _random_bytes(t, nblocks, seed):
    rs = np.random.default_rng(seed)
    bs, bb = oracle.BLOCK[t]
    q = rs.integers(0, 256, size=nblocks * bb, dtype=np.uint8)
    if t == 0:
        return rs.standard_normal(nblocks).astype(np.float32).view(np.uint8).copy()
    if t == 1:
        return rs.uniform(-8, 8, nblocks).astype(np.float16).view(np.uint8).copy()
    blk = q.reshape(nblocks, bb)
    d = rs.uniform(1e-3, 0.1, size=nblocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if t == 14:
        blk[:, 208:210] = d
    else:
        blk[:, 0:2] = d
    if t in (12, 13):
        blk[:, 2:4] = rs.uniform(1e-3, 0.05, size=nblocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return q


def _inputs(n, seed):
    """Normal data at several scales plus the corner blocks, n a multiple of 256."""
    rs = np.random.default_rng(seed)
    x = rs.standard_normal(n) * 10.0 ** rs.integers(-3, 2, n // 256).repeat(256)
    x[0:256] = 0.0
    x[256:512] = 0.25
    x[512:768] = np.abs(x[512:768]) + 0.01
    x[768:1024] *= 1e-6           # fp16-subnormal block scales
    x[1024:1280] *= 1e4           # large values
    x[1280:1312] = -3.0           # one constant Q8_0 block, negative
    return x.astype(np.float32)


@pytest.mark.gpu
def test_qrow_bytes(fh):
    for name, t in TYPES.items():
        for n in (0, 256, 4096, 14336):
            b = ctypes.c_int64()
            fh.check(fh.lib.fg_qrow_bytes(t, n, ctypes.byref(b)), "fg_qrow_bytes")
            assert b.value == oracle.row_bytes(t, n), name
    assert fh.lib.fg_qrow_bytes(3, 256, ctypes.byref(ctypes.c_int64())) != 0  # Q4_1: no decoder


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(TYPES))
def test_dequantize_bit_exact(fh, name):
    t = TYPES[name]
    bs = oracle.BLOCK[t][0]
    nblocks = 4096 if bs == 1 else (64 if bs == 256 else 512)
    q = _random_bytes(t, nblocks, 10 + t)
    n = nblocks * bs
    out, qd = fh.DeviceArray((n,)), fh.DeviceArray.from_numpy(q)
    fh.check(fh.lib.fg_dequantize(t, ctypes.c_void_p(out.ptr), ctypes.c_void_p(qd.ptr), n), "fg_dequantize")
    got, ref = out.numpy(), oracle.dequantize(t, q, n)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
def test_dequantize_every_half(fh):
    h = np.arange(65536, dtype=np.uint16)
    out, hd = fh.DeviceArray((65536,)), fh.DeviceArray.from_numpy(h)
    fh.check(fh.lib.fg_dequantize(1, ctypes.c_void_p(out.ptr), ctypes.c_void_p(hd.ptr), 65536), "fg_dequantize")
    got, ref = out.numpy(), h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", QUANTIZERS)
def test_quantize_bit_exact(fh, name):
    t = TYPES[name]
    x = _inputs(256 * 40, 20 + t)
    ref = oracle.quantize(t, x)
    out, xd = fh.DeviceArray((ref.size,), np.uint8), fh.DeviceArray.from_numpy(x)
    fh.check(fh.lib.fg_quantize(t, ctypes.c_void_p(out.ptr), ctypes.c_void_p(xd.ptr), x.size), "fg_quantize")
    got = out.numpy()
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, "%s: %d bytes differ, first at %s" % (name, bad.size, bad[:8])


@pytest.mark.gpu
def test_quantize_and_qmatvec_reject_bad_arguments(fh):
    x = fh.DeviceArray.zeros((300,))
    out = fh.DeviceArray((1024,), np.uint8)
    assert fh.lib.fg_quantize(12, ctypes.c_void_p(out.ptr), ctypes.c_void_p(x.ptr), 300) != 0  # not whole blocks
    assert "whole number" in fh.last_error()
    assert fh.lib.fg_quantize(2, ctypes.c_void_p(out.ptr), ctypes.c_void_p(x.ptr), 256) != 0  # no Q4_0 quantizer
    y = fh.DeviceArray((4,))
    assert fh.lib.fg_qmatvec(14, ctypes.c_void_p(y.ptr), ctypes.c_void_p(out.ptr), ctypes.c_void_p(x.ptr), 1,
                             300) != 0
    assert fh.lib.fg_qmatvec(99, ctypes.c_void_p(y.ptr), ctypes.c_void_p(out.ptr), ctypes.c_void_p(x.ptr), 1,
                             256) != 0


SHAPES = [(1, 256), (7, 512), (64, 768), (301, 4096), (33, 14336), (5, 20480)]


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(TYPES))
def test_qmatvec_vs_oracle(fh, name):
    t = TYPES[name]
    rs = np.random.default_rng(30 + t)
    ident, total, worst = 0, 0, 0.0
    for N, K in SHAPES + ([(9, 7), (3, 13)] if t == 0 else []):
        if K % oracle.BLOCK[t][0]:
            continue
        if t in (0, 1, 2, 6):  # random values / blocks
            W = _random_bytes(t, N * K // oracle.BLOCK[t][0], N * K)
        else:
            W = oracle.quantize(t, (rs.standard_normal(N * K) * 0.05).astype(np.float32))
        x = rs.standard_normal(K).astype(np.float32)
        ref = oracle.qmatvec(t, W, x, N, K)
        # keep every device array referenced until the results are read
        y, Wd, xd = fh.DeviceArray((N,)), fh.DeviceArray.from_numpy(W), fh.DeviceArray.from_numpy(x)
        fh.check(fh.lib.fg_qmatvec(t, ctypes.c_void_p(y.ptr), ctypes.c_void_p(Wd.ptr), ctypes.c_void_p(xd.ptr), N,
                                   K), "fg_qmatvec")
        got = y.numpy()
        err = rel_l2(got, ref)
        worst = max(worst, err)
        assert err <= (1e-7 if t == 0 else TOL_FWD), (name, N, K, err)
        ident += int(np.sum(got == ref))
        total += N
    print("%s: worst rel-L2 %.1e, %d of %d outputs bit-identical" % (name, worst, ident, total))
    if t == 0:
        assert ident >= 0.98 * total


DECODE_TYPES = {
    "k_quants": {"wqkv": 12, "wo": 14, "gate": 13, "down": 12, "cls": 14},
    "q8_f16_emb": {"emb": 8, "cls": 8, "wqkv": 8, "wo": 1, "gate": 8, "down": 1},
    "q4k_emb_tied": {"emb": 12, "cls": 12, "wqkv": 12, "wo": 12, "gate": 12, "down": 12},
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(DECODE_TYPES))
def test_decode_step_quantized_vs_oracle(fh, name):
    types = DECODE_TYPES[name]
    tied = name.endswith("tied")
    cfg = oracle.Cfg(dim=256, hidden=512, nLayers=2, nHeads=4, nKvHeads=2, vocab=96, tied=1 if tied else 0)
    params = oracle.init_weights(cfg, 5)
    if not tied:
        P = oracle.split_params(cfg, params)
        P["wcls"][:] = np.random.default_rng(5).standard_normal(P["wcls"].size).astype(np.float32) * 0.02
    T = 24
    ids = np.random.default_rng(6).integers(0, cfg.vocab, T).astype(np.int32)
    dec = Decoder(fh, cfg, params, maxSeq=T + 2, types=types)
    ref = dec.oracle_logits(ids)
    got = np.stack([dec.step(int(ids[t]), t) for t in range(T)])
    err = rel_l2(got, ref)
    same0 = float(np.mean(got[0] == ref[0]))
    print("%s: rel-L2 %.2e, position 0 identical %.1f%%" % (name, err, 100 * same0))
    assert err <= TOL_FWD


@pytest.mark.gpu
def test_decode_rejects_mismatched_gate_up_and_ragged_blocks(fh):
    cfg = oracle.Cfg(dim=64, hidden=128, nLayers=1, nHeads=4, nKvHeads=2, vocab=40, tied=1)
    dec = Decoder(fh, cfg, oracle.init_weights(cfg, 3), maxSeq=4)
    dec.layers[0].up_type = 8
    with pytest.raises(fh.ForgeError, match="gate and up"):
        dec.step(1, 0)
    dec.layers[0].up_type = 0
    dec.layers[0].wqkv_type = 12  # 64 is not a whole Q4_K block
    with pytest.raises(fh.ForgeError, match="tile"):
        dec.step(1, 0)


@pytest.mark.gpu
def test_js_quant_api(fh, tmp_path):
    """tests/js/quant.mjs: the reference's L3/L4 tests over the device API, the
    QuantLinear / quantized-GGUF decode identity, and a dump checked here
    against the oracle (quantizeRow bytes bit-exact, QuantLinear.forward and
    dotQ against the oracle's, quantized-model logits at the forward tolerance)."""
    import json
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    dump = tmp_path / "quant.bin"
    r = subprocess.run(["node", os.path.join(root, "tests", "js", "quant.mjs"), str(dump)], cwd=root,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    res = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    for x in res:
        print(x["test"], "ok" if x["ok"] else "FAIL", x.get("detail") or x.get("error", ""))
    assert r.returncode == 0 and len(res) == 16 and all(x["ok"] for x in res), r.stdout[-4000:]

    b = dump.read_bytes()
    o = 0
    N, K = 40, 512
    rng = oracle.RNG(11)
    W = np.array([rng.normal() * 0.05 for _ in range(N * K)]).astype(np.float32)
    rng = oracle.RNG(12)
    x = np.array([rng.normal() for _ in range(K)]).astype(np.float32)
    for t in (1, 8, 12, 13, 14):
        q = oracle.quantize(t, W)
        got_q = np.frombuffer(b, np.uint8, q.size, o)
        o += q.size
        np.testing.assert_array_equal(got_q, q)
        y = np.frombuffer(b, np.float32, N, o)
        o += 4 * N
        ref = oracle.qmatvec(t, q, x, N, K)
        assert rel_l2(y, ref) <= TOL_FWD
        d = np.frombuffer(b, np.float64, 2, o)
        o += 16
        rb = oracle.row_bytes(t, K)
        for j, row in enumerate((0, 7)):
            ref_d = oracle.dotq(t, q[row * rb:(row + 1) * rb], x)
            mag = float(np.dot(np.abs(oracle.dequantize(t, q[row * rb:(row + 1) * rb], K)), np.abs(x)))
            assert abs(d[j] - ref_d) <= 1e-6 * mag
    # quantized-model logits (four types, 8 positions each) against the oracle's typed decode
    cfg = oracle.Cfg(dim=256, hidden=512, nLayers=2, nHeads=4, nKvHeads=2, vocab=96, tied=1)
    P = oracle.split_params(cfg, oracle.init_weights(cfg, 5))
    ids = [3, 17, 0, 95, 5, 40, 41, 8]
    for t in (8, 12, 13, 14):
        got = np.frombuffer(b, np.float32, len(ids) * cfg.vocab, o).reshape(len(ids), cfg.vocab)
        o += 4 * got.size
        qm = lambda a: (t, oracle.quantize(t, a))  # noqa: E731
        layers = [{"ln1": P["layer.%d.ln1" % l], "ln2": P["layer.%d.ln2" % l], "wqkv": qm(P["layer.%d.wqkv" % l]),
                   "wo": qm(P["layer.%d.wo" % l]), "gate": qm(P["layer.%d.ffn_gate" % l]),
                   "up": qm(P["layer.%d.ffn_up" % l]), "down": qm(P["layer.%d.ffn_down" % l])} for l in range(2)]
        emb = qm(P["tok_emb"])
        ref = oracle.infer_forward_q(cfg, {"tok_emb": emb, "ln_f": P["ln_f"], "wcls": emb, "layers": layers}, ids)
        err = rel_l2(got, ref.reshape(got.shape))
        print("type %d: logits rel-L2 %.2e vs the oracle" % (t, err))
        assert err <= TOL_FWD
    assert o == len(b)
