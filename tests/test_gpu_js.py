"""The JavaScript host (forge-llm_amd/src) on the GPU, compared with the oracle.

* the reference's own invariants and hot-path unit tests with the GPU ops
  (tests/js/invariants.mjs);
* the vector-level autograd ops, single-row attention helpers and
  rmsnormInto through the public API (tests/js/vector_ops.mjs);
* one full TrainableTransformer training step (forward, CE, backward, Adam)
  at the `forge train` demo shape and at a shape that takes the MFMA
  attention path: logits, loss, every parameter gradient, the updated
  parameters and both Adam moments;
* I-70: the GPU training forward equals the oracle's token-by-token
  inference forward with a KV cache (verify.js:288-310).
"""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle
from util import TOL_ADAM, TOL_FWD, TOL_GRAD, max_rel, rel_l2

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "tests", "js")


def node(*args, timeout=300):
    r = subprocess.run(["node"] + list(args), cwd=ROOT, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=timeout)
    return r.returncode, r.stdout


def load_dump(d):
    man = json.load(open(os.path.join(d, "manifest.json")))
    return {k: np.fromfile(os.path.join(d, v["file"]), dtype=v["dtype"]) for k, v in man.items()}


@pytest.mark.gpu
def test_js_invariants_with_gpu_ops(fh):
    rc, out = node(os.path.join(JS, "invariants.mjs"), timeout=600)
    results = [json.loads(l) for l in out.splitlines() if l.startswith("{")]
    for r in results:
        print(r["test"], "ok" if r["ok"] else "FAIL", r.get("detail") or r.get("error", ""))
    failed = [r for r in results if not r["ok"]]
    assert rc == 0 and not failed and len(results) >= 28, out[-4000:]


@pytest.mark.gpu
def test_js_vector_ops_and_row_attention(fh):
    rc, out = node(os.path.join(JS, "vector_ops.mjs"), timeout=300)
    results = [json.loads(l) for l in out.splitlines() if l.startswith("{")]
    for r in results:
        print(r["test"], "ok" if r["ok"] else "FAIL", r.get("detail") or r.get("error", ""))
    failed = [r for r in results if not r["ok"]]
    assert rc == 0 and not failed and len(results) >= 8, out[-4000:]


def _cfg(spec):
    return oracle.Cfg(dim=spec["dim"], hidden=spec["hidden"], nLayers=spec["nLayers"], nHeads=spec["nHeads"],
                      nKvHeads=spec["nKvHeads"], vocab=spec["vocab"], normEps=spec.get("normEps", 1e-5),
                      ropeTheta=spec.get("ropeTheta", 1e4), tied=0 if spec.get("untied") else 1)


STEP_SPECS = {
    # `forge train` demo: Config{dim64,hid128,L2,nH4,nKV2,V31}, initWeights seed 20260101,
    # batch 8 x seq 32, ids uniform in [0,31) from RNG(1); Adam lr 5e-3, 60 steps, clip 1, wd 0.01.
    "demo": dict(dim=64, hidden=128, nLayers=2, nHeads=4, nKvHeads=2, vocab=31, B=8, T=32, initSeed=20260101,
                 idsSeed=1, lr=5e-3, totalSteps=60, clip=1.0, wd=0.01),
    # MFMA attention (dH 64, GQA 2:1), untied head, multi-tile GEMMs.
    "mfma": dict(dim=256, hidden=512, nLayers=2, nHeads=4, nKvHeads=2, vocab=512, B=2, T=128, initSeed=5,
                 idsSeed=2, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.0, untied=True),
    # Widths that fit no vector or tile size: dH 30 (scalar attention, GQA 3:1),
    # d 90 / SwiGLU 230 / V 77 (checked GEMM edges, scalar RMSNorm and
    # embedding rows), B3 x T37.
    "ragged": dict(dim=90, hidden=230, nLayers=2, nHeads=3, nKvHeads=1, vocab=77, B=3, T=37, initSeed=11,
                   idsSeed=4, lr=1e-3, totalSteps=100, clip=0.5, wd=0.01, untied=True),
    # The dH 32 and dH 128 MFMA attention kernels inside a step (GQA 4:1 and
    # 2:1, ragged T), tied heads.
    "dh32": dict(dim=256, hidden=384, nLayers=1, nHeads=8, nKvHeads=2, vocab=300, B=2, T=100, initSeed=12,
                 idsSeed=5, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.0),
    "dh128": dict(dim=256, hidden=512, nLayers=1, nHeads=2, nKvHeads=1, vocab=200, B=2, T=70, initSeed=13,
                  idsSeed=6, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.0),
    # dH 192 (GQA 2:1): attention as per-head GEMM launches inside a step.
    "dh192": dict(dim=768, hidden=512, nLayers=1, nHeads=4, nKvHeads=2, vocab=200, B=2, T=40, initSeed=17,
                  idsSeed=9, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.01, untied=True),
    # dH 80 (GQA 2:1): attention on the dH 96 kernels over head-padded copies
    # inside a step (qkvRope + causalAttnBatch), untied head.
    "dh80": dict(dim=320, hidden=512, nLayers=1, nHeads=4, nKvHeads=2, vocab=300, B=2, T=70, initSeed=15,
                 idsSeed=8, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.01, untied=True),
    # dH 96 (GQA 3:1): the fused qkv attention on the dH 96 kernels.
    "dh96": dict(dim=576, hidden=640, nLayers=1, nHeads=6, nKvHeads=2, vocab=250, B=2, T=90, initSeed=18,
                 idsSeed=10, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.01),
    # The smallest model the reference's Config accepts in practice: d 4,
    # dH 2, SwiGLU 3, V 5, B2 x T3, untied.
    "tiny": dict(dim=4, hidden=3, nLayers=1, nHeads=2, nKvHeads=1, vocab=5, B=2, T=3, initSeed=14,
                 idsSeed=7, lr=1e-2, totalSteps=10, clip=1.0, wd=0.01, untied=True),
}


def _random_step_specs(n, seed):
    """Seeded random model shapes for one training step: head size even in
    [2, 160] (RoPE pairs), nH a multiple of nKV, any SwiGLU width and vocab,
    tied or untied, one or two layers, ragged batch and sequence lengths."""
    rs = np.random.default_rng(seed)
    out = {}
    while len(out) < n:
        if rs.random() < 0.5:
            dH = int(rs.choice([2, 4, 16, 30, 32, 34, 64, 96, 128, 130]))
        else:
            dH = 2 * int(rs.integers(1, 81))
        nKV = int(rs.integers(1, 4))
        nH = nKV * int(rs.integers(1, 4))
        dim = nH * dH
        if dim > 1024:
            continue
        spec = dict(dim=dim, hidden=int(rs.integers(1, 700)), nLayers=int(rs.integers(1, 3)), nHeads=nH,
                    nKvHeads=nKV, vocab=int(rs.integers(2, 600)), B=int(rs.integers(1, 4)),
                    T=int(rs.integers(1, 90)), initSeed=int(rs.integers(1, 1 << 30)),
                    idsSeed=int(rs.integers(1, 1 << 30)), lr=float(rs.choice([1e-3, 3e-4])), totalSteps=100,
                    clip=float(rs.choice([0.5, 1.0])), wd=float(rs.choice([0.0, 0.01])),
                    untied=bool(rs.integers(0, 2)))
        out["r%d_d%d_h%dx%d_kv%d" % (len(out), dim, nH, dH, nKV)] = spec
    return out


RANDOM_STEP_SPECS = _random_step_specs(10, 99)


def _step_parity(tmp_path, spec):
    spec = dict(spec, mode="step")
    rc, out = node(os.path.join(JS, "dump_step.mjs"), str(tmp_path), json.dumps(spec))
    assert rc == 0, out
    d = load_dump(str(tmp_path))
    cfg = _cfg(spec)
    B, T = spec["B"], spec["T"]
    logits, loss, grads = oracle.model_fwd_bwd(cfg, d["params0"], d["ids"], d["targets"], B, T)
    assert rel_l2(d["logits"], logits) < TOL_FWD
    assert rel_l2(d["loss"], [loss]) < TOL_FWD
    shapes = cfg.param_shapes()
    g_gpu = oracle.split_params(cfg, d["grads"])
    g_ref = oracle.split_params(cfg, grads)
    worst = {k: max_rel(g_gpu[k], g_ref[k]) for k, _ in shapes}
    print("worst grad max-rel:", max(worst.values()), max(worst, key=worst.get))
    for k, _ in shapes:
        assert worst[k] < TOL_GRAD, (k, worst[k])
    # Adam on identical gradients (the GPU's): parameters and moments to 1e-6
    p = [a.copy() for a in oracle.split_params(cfg, d["params0"]).values()]
    gg = [a.copy() for a in g_gpu.values()]
    m = [np.zeros_like(a) for a in p]
    v = [np.zeros_like(a) for a in p]
    info = oracle.adam_step(p, gg, m, v, 1, lr=spec["lr"], wd=spec["wd"], clip=spec["clip"], total=spec["totalSteps"])
    assert abs(d["adam_info"][1] - info["gnorm"]) <= 1e-6 * info["gnorm"]
    for name_, a, b in [("params", d["params1"], np.concatenate(p)), ("m", d["m1"], np.concatenate(m)),
                        ("v", d["v1"], np.concatenate(v))]:
        assert rel_l2(a, b) < TOL_ADAM, name_


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(STEP_SPECS))
def test_train_step_parity(fh, tmp_path, name):
    _step_parity(tmp_path, STEP_SPECS[name])


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(RANDOM_STEP_SPECS))
def test_train_step_parity_random_shapes(fh, tmp_path, name):
    """One step at seeded random model shapes (the routes each op takes at
    widths no fixed spec names), against the oracle."""
    _step_parity(tmp_path, RANDOM_STEP_SPECS[name])


def _expected_windows(data, starts, T):
    """train()'s batch rows (train.js:255-260): row[i] = data[s+i], or the last
    token past the end; inputs row[0..T), targets row[1..T]."""
    n = len(data)
    idx = np.minimum(np.asarray(starts, np.int64)[:, None] + np.arange(T + 1)[None, :], n - 1)
    rows = np.asarray(data, np.int32)[idx]
    return rows[:, :T].ravel(), rows[:, 1:].ravel()


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_train_step_125m_widths_vs_oracle(fh, tmp_path):
    """One step of train()'s device loop at the 125M shape's widths and batch
    (d768, 12 heads x 64, SwiGLU 2048, V 32000 untied, B8 x T1024: every GEMM,
    attention and CE launch has the benchmark's shape) with two layers,
    against the oracle: the gathered windows bit for bit, logits (every 16th
    row), loss, every parameter gradient, and Adam's parameters and moments on
    identical gradients.  Kernel variants on this path: 128x192 tiles for the
    8192x768 outputs, 128x256 ping-pong tiles with the tail split (qkv
    forward), the grouped weight-gradient launch, the LM-head input gradient
    split over K, ce_fused_regs (rows of 32000 floats held in registers), the
    fused qkv + RoPE + attention at T 1024, the device-sorted embedding
    backward and Adam reading its schedule from device memory."""
    spec = dict(dim=768, hidden=2048, nLayers=2, nHeads=12, nKvHeads=12, vocab=32000, B=8, T=1024, initSeed=1337,
                idsSeed=3, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.01, untied=True, mode="loop", dataLen=40000,
                logitsEvery=16)
    rc, out = node(os.path.join(JS, "dump_step.mjs"), str(tmp_path), json.dumps(spec), timeout=600)
    assert rc == 0, out
    d = load_dump(str(tmp_path))
    cfg = _cfg(spec)
    B, T, V = spec["B"], spec["T"], spec["vocab"]
    ids, tg = _expected_windows(d["data"], d["starts"], T)
    np.testing.assert_array_equal(d["ids"], ids)
    np.testing.assert_array_equal(d["targets"], tg)
    logits, loss, grads = oracle.model_fwd_bwd(cfg, d["params0"], ids, tg, B, T)
    rows = np.arange(0, B * T, spec["logitsEvery"])
    ref_rows = logits.reshape(B * T, V)[rows]
    print("logits rel-L2 %.3g  loss gpu %.7f oracle %.7f" % (rel_l2(d["logits"], ref_rows), d["loss"][0], loss))
    assert rel_l2(d["logits"], ref_rows) < TOL_FWD
    assert abs(float(d["loss"][0]) - float(loss)) <= TOL_FWD * abs(float(loss))
    g_gpu = oracle.split_params(cfg, d["grads"])
    g_ref = oracle.split_params(cfg, grads)
    worst = {k: max_rel(g_gpu[k], g_ref[k]) for k, _ in cfg.param_shapes()}
    print("worst grad max-rel: %.3g (%s)" % (max(worst.values()), max(worst, key=worst.get)))
    for k, v in worst.items():
        assert v < TOL_GRAD, (k, v)
    p = [a.copy() for a in oracle.split_params(cfg, d["params0"]).values()]
    gg = [a.copy() for a in g_gpu.values()]
    m = [np.zeros_like(a) for a in p]
    v = [np.zeros_like(a) for a in p]
    info = oracle.adam_step(p, gg, m, v, 1, lr=spec["lr"], wd=spec["wd"], clip=spec["clip"], total=spec["totalSteps"])
    assert abs(d["adam_info"][0] - info["lr"]) <= 1e-15 * info["lr"]
    assert abs(d["adam_info"][1] - info["gnorm"]) <= 1e-6 * info["gnorm"]
    for name_, a, b in [("params", d["params1"], np.concatenate(p)), ("m", d["m1"], np.concatenate(m)),
                        ("v", d["v1"], np.concatenate(v))]:
        assert rel_l2(a, b) < TOL_ADAM, name_


def _sample_idx(cfg, n, big_rows, chunk_every, whole):
    """Flat indices of dump_step.mjs's sampleOf: [V, d] tensors at big_rows,
    other tensors whole (whole=True or at most 2^20 floats) or every
    chunk_every-th run of 4096 floats."""
    D = cfg.dim
    if n == cfg.vocab * D:
        return (np.asarray(big_rows, np.int64)[:, None] * D + np.arange(D)[None, :]).ravel()
    if whole or n <= (1 << 20):
        return np.arange(n)
    ch = np.arange(0, (n + 4095) // 4096, chunk_every, dtype=np.int64)
    idx = (ch[:, None] * 4096 + np.arange(4096)[None, :]).ravel()
    return idx[idx < n]


def _split_sampled(cfg, flat, idxs):
    out, o = {}, 0
    for (name, _), ix in zip(cfg.param_shapes(), idxs):
        out[name] = flat[o:o + ix.size]
        o += ix.size
    assert o == flat.size
    return out


@pytest.mark.gpu
@pytest.mark.timeout(1100)
def test_train_step_llama8b_widths_vs_oracle(fh, tmp_path):
    """One step of train()'s device loop at the Llama-3-8B slice's widths
    (d4096, 32 query / 8 kv heads x 128, SwiGLU 14336, V 128256 untied, RoPE
    theta 5e5, one layer, B1) at T 1024, against the oracle: the gathered
    window bit for bit; logits (every 8th row) and loss; every gradient (the
    525M-float embedding and LM-head gradients at the rows of every input and
    target id plus 256 random rows, the others whole), with the embedding
    gradient nonzero exactly at the input ids and the global gradient norm
    from every element; Adam's parameters and moments on identical
    gradients (every 16th run of 4096 floats of the layer matrices).
    Kernel variants on this path: the long-row fused CE (rows of 128256
    floats), the GQA 4:1 attention with its dK/dV partial reduce at dH 128,
    the workgroup-per-row RMSNorm backward at D 4096, the fused qkv RoPE at
    theta 5e5, the gate/up GEMM with its SwiGLU epilogue at 4096 -> 2x14336,
    the grouped weight-gradient launch and the device-sorted embedding
    backward."""
    T, V = 1024, 128256
    spec = dict(dim=4096, hidden=14336, nLayers=1, nHeads=32, nKvHeads=8, vocab=V, B=1, T=T, initSeed=1337,
                idsSeed=8, lr=3e-4, totalSteps=1000, clip=1.0, wd=0.01, untied=True, ropeTheta=5e5,
                mode="loop_sampled", dataLen=20000, logitsEvery=8, chunkEvery=16)
    cfg = _cfg(spec)
    r = oracle.RNG(spec["idsSeed"])
    data = r.ints(spec["dataLen"], V)
    starts = [r.int(max(1, spec["dataLen"] - T - 1))]
    ids, tg = _expected_windows(data, starts, T)
    big = np.union1d(np.union1d(ids, tg), np.random.default_rng(0).choice(V, 256, replace=False))
    spec["bigRows"] = [int(x) for x in big]
    spec["progress"] = True
    # stderr (the stage lines) passes through, so a long run shows progress
    r = subprocess.run(["node", os.path.join(JS, "dump_step.mjs"), str(tmp_path), json.dumps(spec)], cwd=ROOT,
                       stdout=subprocess.PIPE, text=True, timeout=900)
    assert r.returncode == 0, r.stdout
    print("oracle: step at T %d" % T, flush=True)
    d = load_dump(str(tmp_path))
    np.testing.assert_array_equal(d["data"], data)
    np.testing.assert_array_equal(d["starts"], starts)
    np.testing.assert_array_equal(d["ids"], ids)
    np.testing.assert_array_equal(d["targets"], tg)
    shapes = cfg.param_shapes()
    idx_s = [_sample_idx(cfg, n, big, spec["chunkEvery"], False) for _, n in shapes]
    idx_w = [_sample_idx(cfg, n, big, spec["chunkEvery"], True) for _, n in shapes]
    # the JS initWeights + untied head equal the oracle's init on every sampled element
    p0 = oracle.split_params(cfg, oracle.init_weights(cfg, spec["initSeed"]))
    for (name, _), ix, got in zip(shapes, idx_s, _split_sampled(cfg, d["params0"], idx_s).values()):
        np.testing.assert_array_equal(got, p0[name][ix], err_msg=name)
    params0 = np.concatenate([p0[name] for name, _ in shapes])
    del p0
    logits, loss, grads = oracle.model_fwd_bwd(cfg, params0, ids, tg, 1, T)
    print("oracle: done", flush=True)
    rows = np.arange(0, T, spec["logitsEvery"])
    ref_rows = logits.reshape(T, V)[rows]
    del logits
    print("logits rel-L2 %.3g  loss gpu %.7f oracle %.7f" % (rel_l2(d["logits"], ref_rows), d["loss"][0], loss))
    assert rel_l2(d["logits"], ref_rows) < TOL_FWD
    assert abs(float(d["loss"][0]) - float(loss)) <= TOL_FWD * abs(float(loss))
    g_ref = oracle.split_params(cfg, grads)
    g_gpu = _split_sampled(cfg, d["grads"], idx_w)
    worst = {}
    for (name, _), ix in zip(shapes, idx_w):
        worst[name] = max_rel(g_gpu[name], g_ref[name][ix])
    print("worst grad max-rel: %.3g (%s)" % (max(worst.values()), max(worst, key=worst.get)))
    for k, v in worst.items():
        assert v < TOL_GRAD, (k, v)
    # the embedding gradient is nonzero exactly at the input ids, on both sides
    np.testing.assert_array_equal(d["tok_emb_grad_rows"], np.unique(ids))
    emb = g_ref["tok_emb"].reshape(V, cfg.dim)
    np.testing.assert_array_equal(np.flatnonzero(np.any(emb != 0, axis=1)), np.unique(ids))
    # the global norm Adam clipped with: from every element, on both sides
    gnorm = float(d["adam_info"][1])
    assert abs(gnorm - float(np.sqrt(np.sum(d["grad_sumsq"])))) <= 1e-9 * gnorm
    ref_norm = float(np.sqrt(sum(float(np.dot(g.astype(np.float64), g.astype(np.float64))) for g in g_ref.values())))
    print("gnorm gpu %.9g oracle %.9g" % (gnorm, ref_norm))
    assert abs(gnorm - ref_norm) <= TOL_GRAD * ref_norm
    del grads, g_ref
    # Adam on the GPU's gradients at the sampled elements, clipped with its norm
    p = [params0[o:o + n][ix].copy() for (o, n), ix in zip(_offsets(shapes), idx_s)]
    gg = [_subsample(g_gpu[name], ixs, ixw) for (name, _), ixs, ixw in zip(shapes, idx_s, idx_w)]
    m = [np.zeros_like(a) for a in p]
    v = [np.zeros_like(a) for a in p]
    info = oracle.adam_step(p, gg, m, v, 1, lr=spec["lr"], wd=spec["wd"], clip=spec["clip"],
                            total=spec["totalSteps"], gnorm=gnorm)
    assert abs(d["adam_info"][0] - info["lr"]) <= 1e-15 * info["lr"]
    assert abs(d["adam_info"][2] - info["scale"]) <= 1e-12 * info["scale"]
    for name_, a, b in [("params", d["params1"], np.concatenate(p)), ("m", d["m1"], np.concatenate(m)),
                        ("v", d["v1"], np.concatenate(v))]:
        assert rel_l2(a, b) < TOL_ADAM, name_


def _offsets(shapes):
    o = 0
    for _, n in shapes:
        yield o, n
        o += n


def _subsample(g_whole_sampled, idx_s, idx_w):
    """The elements idx_s of a gradient dumped at idx_w (idx_s is a subset)."""
    if idx_s.size == idx_w.size:
        return g_whole_sampled.copy()
    pos = np.searchsorted(idx_w, idx_s)
    assert np.array_equal(idx_w[pos], idx_s)
    return np.ascontiguousarray(g_whole_sampled[pos])


@pytest.mark.gpu
def test_i70_train_forward_equals_inference_forward(fh, tmp_path):
    spec = dict(dim=32, hidden=64, nLayers=2, nHeads=4, nKvHeads=2, vocab=40, B=1, T=6, initSeed=4242,
                ids=[[1, 5, 9, 13, 2, 7, 0]], mode="forward")
    rc, out = node(os.path.join(JS, "dump_step.mjs"), str(tmp_path), json.dumps(spec))
    assert rc == 0, out
    d = load_dump(str(tmp_path))
    cfg = _cfg(spec)
    infer = oracle.infer_forward(cfg, d["params0"], d["ids"])
    diff = float(np.max(np.abs(d["logits"].astype(np.float64) - infer)))
    print("I-70 max|dlogits| =", diff)
    assert diff < 2e-3
    # and the oracle's training forward on the same weights
    train_logits, _, _ = oracle.model_fwd_bwd(cfg, d["params0"], d["ids"], d["ids"], 1, 6)
    assert rel_l2(d["logits"], train_logits) < TOL_FWD


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(STEP_SPECS))
def test_multi_step_training_parity(fh, tmp_path, name):
    """Several train() steps with a fresh random batch each: per-step loss and
    gradient norm, and the final parameters, against the oracle replaying the
    same steps (model forward/backward + Adam with carried moments)."""
    spec = dict(STEP_SPECS[name], mode="steps", nsteps=6)
    rc, out = node(os.path.join(JS, "dump_step.mjs"), str(tmp_path), json.dumps(spec))
    assert rc == 0, out
    d = load_dump(str(tmp_path))
    cfg = _cfg(spec)
    B, T, n = spec["B"], spec["T"], spec["nsteps"]
    params = [a.copy() for a in oracle.split_params(cfg, d["params0"]).values()]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    for s in range(n):
        ids = d["step_ids"][s * B * T:(s + 1) * B * T]
        tg = d["step_targets"][s * B * T:(s + 1) * B * T]
        _, loss, grads = oracle.model_fwd_bwd(cfg, np.concatenate(params), ids, tg, B, T)
        g = [a.copy() for a in oracle.split_params(cfg, grads).values()]
        info = oracle.adam_step(params, g, m, v, s + 1, lr=spec["lr"], wd=spec["wd"], clip=spec["clip"],
                                total=spec["totalSteps"])
        print("step", s, "loss gpu %.6f oracle %.6f" % (d["step_losses"][s], loss),
              "gnorm gpu %.6f oracle %.6f" % (d["step_gnorms"][s], info["gnorm"]))
        assert abs(d["step_losses"][s] - loss) <= 1e-4 * abs(loss)
        assert abs(d["step_gnorms"][s] - info["gnorm"]) <= 1e-3 * info["gnorm"]
    assert rel_l2(d["params_final"], np.concatenate(params)) < 1e-4
