#!/usr/bin/env python3
"""Benchmark: training tokens/s of one full step (forward + CE + backward +
global-norm clip + Adam) of the 125M-shaped TrainableTransformer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

The step runs through the product path: the JavaScript host
(forge-llm_amd/src, the TrainableTransformer / train() API) driving the HIP
kernels of libforge_hip.so through the N-API addon, launched as a child
process (this process never touches the GPU).  Workload: d_model 768,
12 layers, 12 heads x 64, SwiGLU 2048, RMSNorm, RoPE base 10000, vocab 32000
with an untied LM head, batch 8 x seq 1024 of uniform random token ids,
weights N(0, 0.02); fp32 throughout.  The default loop is train()'s
device-resident one (--loop graph): the token stream resident in HBM, the
windows cut on the device, each step replayed as one recorded HIP graph;
--loop device issues the same steps op by op, --loop host uploads host-drawn
ids every step.

Printed line: the metric, value = B*T*steps / wall time of the timed region
(inputs resident on the device), plus
  roofline     — the kernel family with the largest device time in the step,
                 algorithmic flop (or bytes) per launch / its average duration,
                 measured with each launch's own start/stop HIP events on the
                 library stream during a second pass of the same steps (the
                 entry points' event brackets, launch gaps included, are
                 reported beside it as frac_bracket);
  cpu_baseline — the CPU oracle (single thread) timed on a bounded sample of
                 the same step and scaled to a full step;
  kernels      — the same measurement for every kernel family.
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "train tokens/s (fwd+bwd+Adam) 125M-shape; per-kernel % of HBM / fp32-MFMA peak"
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_FP32_MFMA_TFS = 157.3   # MI355X dense fp32 matrix
PEAK_FP16_MFMA_TFS = 2500.0  # MI355X dense fp16 matrix
# The contraction families evaluate each fp32 product as several half-width
# MFMA products of split operands, so their ceiling in fp32 flop/s is that
# instruction's peak over the products per fp32 product: three
# fp16 products of scaled hi/lo pairs.
SPLIT_BASIS = {"gemm_": ("fp16", PEAK_FP16_MFMA_TFS, 3), "attn_": ("fp16", PEAK_FP16_MFMA_TFS, 3)}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def run_gpu(preset, steps, warmup, loop):
    cmd = ["node", os.path.join(ROOT, "forge-llm_amd", "bench", "train_step.mjs"),
           json.dumps({"preset": preset, "steps": steps, "warmup": warmup, "loop": loop})]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout[-4000:] + r.stderr[-4000:])
        raise SystemExit("GPU step bench failed (exit %d)" % r.returncode)
    return json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])


def kernel_rows(kernels, steps):
    """Per kernel family: algorithmic work over the kernels' own time (each
    launch's start/stop events from hipExtLaunchKernelGGL, the basis rocprof's
    kernel durations share) and over the entry points' event brackets (which
    also hold each launch's dispatch gap)."""
    rows = []
    for k in kernels:
        kms = k.get("kernel_ms", 0.0)
        if kms <= 0:
            continue
        work = k["flop"] if k["flop"] > 0 else k["bytes"]
        if k["flop"] > 0:
            ach = work / (kms * 1e-3) / 1e12
            split = [v for p, v in SPLIT_BASIS.items() if k["name"].startswith(p)]
            if split:
                typ, tfs, prods = split[0]
                peak = tfs / prods
                basis = "%s dense MFMA %.0f TFLOP/s / %d products per fp32 product" % (typ, tfs, prods)
            else:
                peak = PEAK_FP32_MFMA_TFS
                basis = "fp32 dense MFMA %.1f TFLOP/s" % PEAK_FP32_MFMA_TFS
            row = dict(name=k["name"], bound="mfma", achieved=ach, peak=round(peak, 1), unit="TFLOP/s",
                       frac=ach / peak, frac_fp32_mfma=ach / PEAK_FP32_MFMA_TFS, peak_basis=basis)
            bracket = work / (k["ms"] * 1e-3) / 1e12
        else:
            ach = work / (kms * 1e-3) / 1e9
            peak = PEAK_HBM_GBS
            row = dict(name=k["name"], bound="hbm", achieved=ach, peak=peak, unit="GB/s", frac=ach / peak)
            bracket = work / (k["ms"] * 1e-3) / 1e9
        row.update(ms_per_step=kms / steps, calls_per_step=k["calls"] / steps,
                   launches_per_step=k.get("launches", 0) / steps,
                   avg_launch_us=1e3 * kms / k["calls"], algo_per_launch=work / k["calls"],
                   bracket_ms_per_step=k["ms"] / steps, frac_bracket=bracket / peak)
        rows.append(row)
    rows.sort(key=lambda r: -r["ms_per_step"])
    return rows


def host_cpu():
    """CPU model and logical core count of this host."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 0


def cpu_baseline():
    """Single-thread oracle timed on a bounded sample of one 125M-shaped step.

    Per-token costs are measured on row subsets of the real shapes and scaled
    by the number of rows; attention by heads; Adam by parameter count:
      t_step = B*T*(L*(gemm_tok + elem_tok) + head_tok) + B*L*nH*attn_head + adam*P/P_s
    """
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle

    oracle.set_threads(1)  # one thread, as the reference's JavaScript runs

    d, H, V, nH, dH, L, B, T = 768, 2048, 32000, 12, 64, 12, 8, 1024
    P_total = 134105856
    rng = np.random.default_rng(0)

    def rnd(n, s=1.0):
        return (rng.standard_normal(n) * s).astype(np.float32)

    t_all = time.perf_counter()
    Mg = 1536
    t0 = time.perf_counter()
    for K, N in [(d, 3 * d), (d, d), (d, H), (d, H), (H, d)]:
        X, W, g = rnd(Mg * K), rnd(N * K, 0.02), rnd(Mg * N)
        oracle.matmulT_fwd(X, W, Mg, K, N)
        oracle.matmulT_bwd(g, X, W, Mg, K, N)
    gemm_tok = (time.perf_counter() - t0) / Mg

    Te = 2048
    t0 = time.perf_counter()
    x, w1 = rnd(Te * d), np.ones(d, np.float32)
    y, inv = oracle.rmsnorm_fwd(x, w1, Te, d, 1e-5)
    oracle.rmsnorm_bwd(y, x, w1, inv, Te, d)
    qkv = rnd(Te * 3 * d)
    for off in (0, d, 2 * d):
        sl = oracle.slice_fwd(qkv, Te, 3 * d, off, d)
        oracle.slice_bwd(sl, Te, 3 * d, off, d)
    for _ in range(2):
        r = oracle.rope_fwd(sl, Te, nH, dH, 0, 1e4, T)
        oracle.rope_bwd(r, Te, nH, dH, 0, 1e4, T)
    G, U = rnd(Te * H), rnd(Te * H)
    o, sig = oracle.swiglu_fwd(G, U)
    oracle.swiglu_bwd(o, sig, G, U)
    oracle.add_fwd(x, y)
    elem_tok = 2 * (time.perf_counter() - t0) / Te  # two norms/adds per layer; rope pair covers q and k

    nh_s = 4
    t0 = time.perf_counter()
    for _ in range(nh_s):
        q, k, v, g = rnd(T * dH), rnd(T * dH), rnd(T * dH), rnd(T * dH)
        out, Pm = oracle.attn_fwd(q, k, v, 1, T, 1, 1, dH)
        oracle.attn_bwd(g, Pm, q, k, v, 1, T, 1, 1, dH)
    attn_head = (time.perf_counter() - t0) / nh_s

    Mh = 320
    t0 = time.perf_counter()
    X, W = rnd(Mh * d), rnd(V * d, 0.02)
    logits = oracle.matmulT_fwd(X, W, Mh, d, V)
    tg = rng.integers(0, V, Mh).astype(np.int32)
    loss, probs = oracle.ce_fwd(logits, tg, Mh, V)
    gl = oracle.ce_bwd(1.0, probs, tg, Mh, V)
    oracle.matmulT_bwd(gl, X, W, Mh, d, V)
    xe = rnd(Mh * d)
    oracle.rmsnorm_bwd(xe, xe, np.ones(d, np.float32), np.ones(Mh, np.float32), Mh, d)
    head_tok = (time.perf_counter() - t0) / Mh

    Ps = 1 << 23
    p, gg = [rnd(Ps)], [rnd(Ps)]
    m, vv = [np.zeros(Ps, np.float32)], [np.zeros(Ps, np.float32)]
    t0 = time.perf_counter()
    oracle.adam_step(p, gg, m, vv, 1)
    adam = (time.perf_counter() - t0) * P_total / Ps
    sample_s = time.perf_counter() - t_all

    t_step = B * T * (L * (gemm_tok + elem_tok) + head_tok) + B * L * nH * attn_head + adam
    cpu_model, cpu_count = host_cpu()
    return {
        "value": B * T / t_step,
        "unit": "tokens/s",
        "cores": 1,
        "threads": 1,
        "host_cpu": cpu_model,
        "host_logical_cores": cpu_count,
        "kind": "port",
        "sample": ("C oracle (fp64 arithmetic, fp32 stores, reference loop order), 1 thread, %.1f s measured on: "
                   "5 layer GEMMs fwd+bwd at %d rows, norms/slices/RoPE/SwiGLU/add at %d rows, attention fwd+bwd "
                   "of 4 heads at T=1024, LM head+CE fwd+bwd at %d rows, Adam on 2^23 params; scaled to B8xT1024, "
                   "12 layers, 12 heads, 134.1M params -> %.1f s per step. The reference's own JavaScript "
                   "needs Node >= 20 and this image has Node 12, so it cannot be timed here" % (sample_s, Mg, Te, Mh,
                                                                                                t_step)),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--preset", default="125m", choices=["125m", "demo", "llama8b_slice"])
    ap.add_argument("--loop", default="graph", choices=["graph", "device", "host"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print("bench.py measures one GPU: the data-parallel multi-GPU path is not implemented; "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    r = run_gpu(a.preset, a.steps, a.warmup, a.loop)
    ms = r["ms_per_step"]
    value = r["tokens_per_step"] / (ms / 1e3)
    rows = kernel_rows(r["kernels"], a.steps)
    dom = rows[0]
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        tr = json.load(open(TRAFFIC_FILE))
        traffic = tr.get(a.preset, {}).get(dom["name"])
    roofline = {"bound": dom["bound"], "achieved": round(dom["achieved"], 3), "peak": dom["peak"],
                "unit": dom["unit"], "frac": round(dom["frac"], 4), "traffic": traffic, "kernel": dom["name"],
                "peak_basis": dom.get("peak_basis", "HBM3E %.0f GB/s" % PEAK_HBM_GBS),
                "frac_fp32_mfma": (round(dom["frac_fp32_mfma"], 4) if "frac_fp32_mfma" in dom else None),
                "avg_launch_us": round(dom["avg_launch_us"], 3), "algo_per_launch": dom["algo_per_launch"],
                "timing": "kernel start/stop events of each launch (hipExtLaunchKernelGGL) on the library stream",
                "frac_bracket": round(dom["frac_bracket"], 4)}
    cfg = r["cfg"]
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic (uniform random token ids, N(0,0.02) weights)" if a.loop == "host" else
                 "synthetic (2^22 uniform random token ids resident in HBM, windows at RNG starts; "
                 "N(0,0.02) weights)"),
        "config": {
            "workload": "%s TrainableTransformer train step: d%d L%d nH%d/nKV%d dH%d ffn%d V%d %s head, "
                        "B%d x T%d, embed..LM head+CE fwd, bwd, global-norm clip, Adam" % (
                            a.preset, cfg["dim"], cfg["nLayers"], cfg["nHeads"], cfg["nKvHeads"],
                            cfg["dim"] // cfg["nHeads"], cfg["hidden"], cfg["vocab"],
                            "tied" if cfg["tied"] else "untied", cfg["B"], cfg["T"]),
            "global_batch": cfg["B"], "seq_len": cfg["T"], "params": r["params"], "parallelism": "none (1 GPU)",
            "loop": {"graph": "device-resident train() loop, step replayed as one HIP graph",
                     "device": "device-resident train() loop, op by op",
                     "host": "host-drawn ids uploaded each step, op by op"}[a.loop],
        },
        "roofline": roofline,
        "kernels": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in row.items()
                     if k in ("name", "bound", "achieved", "unit", "frac", "frac_fp32_mfma", "ms_per_step",
                              "calls_per_step", "launches_per_step", "bracket_ms_per_step", "frac_bracket")}
                    for row in rows],
        "profiled_ms_per_step": round(r["profiled_ms_per_step"], 3),
        "loss_last": r["losses"][-1],
    }
    if not a.no_cpu_baseline and a.preset == "125m":
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
