"""GGUF export / load and training checkpoints on the GPU (tests/js/export.mjs):
loadGGUF(exportGGUF(w)) decodes bit-identically to loading w directly, and
training resumed from saveCheckpoint / loadCheckpoint is bit-identical to
training that never stopped (losses, gradient norms, parameters, Adam m/v)."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_export_and_checkpoint_js(fh):
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "export.mjs")], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    res = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    for x in res:
        print(x["test"], "ok" if x["ok"] else "FAIL", x.get("detail") or x.get("error", ""))
    assert r.returncode == 0 and len(res) == 5 and all(x["ok"] for x in res), r.stdout[-4000:]


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["demo", "untied"])
def test_trained_export_matches_oracle_training(fh, tmp_path, name):
    """Three training steps on the device, then exportGGUF of the trained
    weights (engine.js:126-228), read back by an independent GGUF parser:
    every tensor (wqkv as its attn_q / attn_k / attn_v row blocks) against
    the oracle replaying the same three steps (model forward/backward and
    Adam with carried moments, train.js:265-269)."""
    import numpy as np

    import oracle
    from test_gpu_js import STEP_SPECS, _cfg, load_dump, node
    from test_host import _parse_gguf
    from util import rel_l2

    base = dict(STEP_SPECS["demo"]) if name == "demo" else dict(STEP_SPECS["mfma"], nLayers=1)
    out_file = tmp_path / "trained.gguf"
    spec = dict(base, mode="steps", nsteps=3, exportTo=str(out_file))
    rc, out = node(os.path.join(ROOT, "tests", "js", "dump_step.mjs"), str(tmp_path), json.dumps(spec))
    assert rc == 0, out
    d = load_dump(str(tmp_path))
    cfg = _cfg(spec)
    B, T = spec["B"], spec["T"]
    params = [a.copy() for a in oracle.split_params(cfg, d["params0"]).values()]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    for s in range(3):
        sl = slice(s * B * T, (s + 1) * B * T)
        _, _, grads = oracle.model_fwd_bwd(cfg, np.concatenate(params), d["step_ids"][sl], d["step_targets"][sl], B, T)
        g = [a.copy() for a in oracle.split_params(cfg, grads).values()]
        oracle.adam_step(params, g, m, v, s + 1, lr=spec["lr"], wd=spec["wd"], clip=spec["clip"],
                         total=spec["totalSteps"])
    P = dict(zip([k for k, _ in cfg.param_shapes()], params))
    D, H, V = cfg.dim, cfg.hidden, cfg.vocab
    qD, kvD = cfg.nHeads * cfg.dHead, cfg.nKvHeads * cfg.dHead
    expect = {"token_embd.weight": P["tok_emb"], "output_norm.weight": P["ln_f"]}
    for l in range(cfg.nLayers):
        L = lambda k: P["layer.%d.%s" % (l, k)]
        expect.update({"blk.%d.attn_norm.weight" % l: L("ln1"), "blk.%d.attn_q.weight" % l: L("wqkv")[:qD * D],
                       "blk.%d.attn_k.weight" % l: L("wqkv")[qD * D:(qD + kvD) * D],
                       "blk.%d.attn_v.weight" % l: L("wqkv")[(qD + kvD) * D:],
                       "blk.%d.attn_output.weight" % l: L("wo"), "blk.%d.ffn_norm.weight" % l: L("ln2"),
                       "blk.%d.ffn_gate.weight" % l: L("ffn_gate"), "blk.%d.ffn_up.weight" % l: L("ffn_up"),
                       "blk.%d.ffn_down.weight" % l: L("ffn_down")})
    if not cfg.tied:
        expect["output.weight"] = P["wcls"]
    b = out_file.read_bytes()
    _, tensors, start = _parse_gguf(b)
    assert sorted(n for n, _, _, _ in tensors) == sorted(expect)
    for tname, dims, ttype, off in tensors:
        want = expect[tname]
        assert ttype == 0 and int(np.prod(dims)) == want.size, tname
        got = np.frombuffer(b, np.float32, count=want.size, offset=start + off)
        assert rel_l2(got, want) < 1e-4, (tname, rel_l2(got, want))
    # and the download the export was made from is the device's parameters
    np.testing.assert_array_equal(np.frombuffer(b, np.float32, count=V * D, offset=start + tensors[0][3]),
                                  oracle.split_params(cfg, d["params_final"])["tok_emb"])
