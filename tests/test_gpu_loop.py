"""The device-resident train() loop (train.js:246-276) through the C ABI.

* fg_batch_gather: the windows train() cuts from its token data, against the
  reference's row construction restated in numpy (train.js:255-260);
* fg_embed_sort_keys / fg_embed_bwd_sorted: the device plan of the embedding
  backward — sorted keys against numpy's sort, gradient rows bit-exact against
  the oracle's sequential scatter-add (tensor.js:92-98) and fg_embed_bwd;
* fg_adam_step_sched: bit-exact against fg_adam_step (the same update with
  the step scalars read from device memory);
* fg_graph_*: a recorded sequence replayed several times, with eager work and
  synchronisations between replays, equals the eager results each time; the
  capture refuses host staging copies and synchronisation;
* train() three ways in JavaScript (tests/js/train_loop.mjs): graph replay,
  op-by-op device loop and the host-batch loop, bit-identical.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NO_KEY = np.uint64(0xFFFFFFFFFFFFFFFF)


def up(fh, a):
    return fh.DeviceArray.from_numpy(np.ascontiguousarray(a))


def gather_ref(data, starts, T, V):
    """Rows of train.js:255-260: row[i] = data[s+i] ?? data[n-1]; ids = row[:T], targets = row[1:]."""
    n = len(data)
    ids, tgt = [], []
    for s in starts:
        row = [data[s + i] if s + i < n else data[n - 1] for i in range(T + 1)]
        ids += row[:T]
        tgt += row[1:]
    m = lambda v: np.where((np.asarray(v) >= 0) & (np.asarray(v) < V), v, -1).astype(np.int32)
    return m(ids), m(tgt)


@pytest.mark.gpu
@pytest.mark.parametrize("n,B,T,V", [(5000, 8, 64, 97), (20, 2, 32, 31), (1, 1, 4, 8), (70000, 4, 1024, 32000)])
def test_batch_gather(fh, n, B, T, V):
    rng = np.random.default_rng(n)
    data = rng.integers(-3, V + 3, n).astype(np.int32)  # includes ids outside [0,V)
    hi = max(1, n - T - 1)
    starts = rng.integers(0, hi, B).astype(np.int32)
    starts[0] = hi - 1
    ids, tgt = fh.DeviceArray((B * T,), np.int32), fh.DeviceArray((B * T,), np.int32)
    fh.call("batch_gather", ids, tgt, up(fh, data), n, up(fh, starts), B, T, V)
    ids_ref, tgt_ref = gather_ref(data.tolist(), starts.tolist(), T, V)
    np.testing.assert_array_equal(ids.numpy(), ids_ref)
    np.testing.assert_array_equal(tgt.numpy(), tgt_ref)


def keys_len(fh, T):
    n = ctypes.c_int64(0)
    fh.check(fh.lib.fg_embed_keys_len(T, ctypes.byref(n)), "fg_embed_keys_len")
    return n.value


@pytest.mark.gpu
@pytest.mark.parametrize("T,V", [(1, 5), (7, 3), (256, 31), (8192, 32000), (8193, 50), (40000, 128256)])
def test_embed_sort_keys(fh, T, V):
    rng = np.random.default_rng(T)
    ids = rng.integers(0, V, T).astype(np.int32)
    ids[rng.integers(0, T, max(1, T // 50))] = -1  # invalid ids sort last
    ids[rng.integers(0, T, max(1, T // 70))] = V
    P = keys_len(fh, T)
    assert P >= T and P & (P - 1) == 0
    keys = fh.DeviceArray((P,), np.uint64)
    fh.call("embed_sort_keys", keys, P, up(fh, ids), T, V)
    t = np.arange(T, dtype=np.uint64)
    exp = np.where((ids >= 0) & (ids < V), (ids.astype(np.uint64) << np.uint64(32)) | t, NO_KEY)
    exp = np.sort(np.concatenate([exp, np.full(P - T, NO_KEY, np.uint64)]))
    np.testing.assert_array_equal(keys.numpy(), exp)
    if P > 2:
        with pytest.raises(fh.ForgeError, match="needed"):
            fh.call("embed_sort_keys", keys, P // 2, up(fh, ids), T, V)


@pytest.mark.gpu
@pytest.mark.parametrize("T,V,D", [(5, 7, 3), (300, 20, 64), (8192, 32000, 768), (8192, 40, 130), (20000, 500, 32),
                                   (700, 90, 1028)])
def test_embed_bwd_sorted_bit_exact(fh, T, V, D):
    rng = oracle.RNG(31)
    g = rng.normal_f32(T * D)
    ids = np.asarray(rng.ints(T, min(V, 60)), np.int32)  # many duplicates
    ids[::97] = -1  # invalid ids contribute nothing
    ids[5::101] = V
    gW0 = rng.normal_f32(V * D, 0.1)
    P = keys_len(fh, T)
    keys = fh.DeviceArray((P,), np.uint64)
    dids = up(fh, ids)
    fh.call("embed_sort_keys", keys, P, dids, T, V)
    gW = up(fh, gW0)
    fh.call("embed_bwd_sorted", gW, up(fh, g), keys, T, V, D, 1)
    valid = (ids >= 0) & (ids < V)
    ref = oracle.embed_bwd(g.reshape(T, D)[valid].ravel(), ids[valid], V, D, gW=gW0)
    np.testing.assert_array_equal(gW.numpy(), ref)
    # beta 0: the present ids' rows hold their sums as if accumulated into a
    # zero row; every other row keeps its old value unread
    gW = up(fh, gW0)
    fh.call("embed_bwd_sorted", gW, up(fh, g), keys, T, V, D, 0)
    fresh = oracle.embed_bwd(g.reshape(T, D)[valid].ravel(), ids[valid], V, D, gW=np.zeros(V * D, np.float32))
    present = np.zeros(V, bool)
    present[ids[valid]] = True
    want = np.where(np.repeat(present, D), fresh, gW0)
    np.testing.assert_array_equal(gW.numpy(), want)


@pytest.mark.gpu
def test_fill_f32(fh):
    x = fh.DeviceArray((1001,))
    fh.call("fill_f32", x, ctypes.c_float(1.0), 1001)
    np.testing.assert_array_equal(x.numpy(), np.ones(1001, np.float32))
    fh.call("fill_f32", x, ctypes.c_float(-2.5), 3)
    assert x.numpy()[:4].tolist() == [-2.5, -2.5, -2.5, 1.0]


def _adam_tensors(fh, sizes, seed):
    rng = np.random.default_rng(seed)
    ts = []
    for n in sizes:
        p = rng.standard_normal(n).astype(np.float32)
        g = (rng.standard_normal(n) * 0.3).astype(np.float32)
        m = (rng.standard_normal(n) * 0.01).astype(np.float32)
        v = np.abs(rng.standard_normal(n) * 1e-4).astype(np.float32)
        ts.append([up(fh, p), up(fh, g), up(fh, m), up(fh, v)])
    return ts


@pytest.mark.gpu
def test_adam_sched_equals_by_value(fh):
    sizes = [3, 8192 * 3 + 5, 4096, 1]
    A, B = _adam_tensors(fh, sizes, 1), _adam_tensors(fh, sizes, 1)
    t, lr0, b1, b2 = 3, 1e-3, 0.9, 0.999
    lr = lr0 * 0.5 * (1 + np.cos(np.pi * t / 50))
    bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
    sa, sb = fh.DeviceArray((2,), np.float64), fh.DeviceArray((2,), np.float64)
    fh.adam_step([(p, g, m, v) for p, g, m, v in A], lr, b1, b2, 1e-8, 0.01, 1.0, bc1, bc2, stats=sa)
    sched = up(fh, np.array([lr, bc1, bc2], np.float64))
    arr = (fh.AdamTensor * len(sizes))()
    for i, (p, g, m, v) in enumerate(B):
        arr[i] = fh.AdamTensor(p.ptr, g.ptr, m.ptr, v.ptr, sizes[i])
    fh.check(fh.lib.fg_adam_step_sched(ctypes.cast(arr, ctypes.c_void_p), len(sizes), sched.ptr, ctypes.c_double(b1), ctypes.c_double(b2),
                                        ctypes.c_double(1e-8), ctypes.c_double(0.01), ctypes.c_double(1.0), sb.ptr),
             "fg_adam_step_sched")
    for ta, tb in zip(A, B):
        for x, y in zip(ta, tb):
            np.testing.assert_array_equal(x.numpy(), y.numpy())
    np.testing.assert_array_equal(sa.numpy(), sb.numpy())


@pytest.mark.gpu
def test_graph_replay_equals_eager(fh):
    """matmulT + residual + accumulate recorded once, replayed 4 times with new
    inputs copied in between (eager work and synchronisation between replays)."""
    M, K, N = 300, 256, 520
    rng = np.random.default_rng(5)
    X, W, R = fh.DeviceArray((M * K,)), up(fh, rng.standard_normal(N * K).astype(np.float32)), fh.DeviceArray((M * N,))
    Y, G = fh.DeviceArray((M * N,)), fh.DeviceArray((M * N,))

    def body():
        fh.call("matmulT_fwd_resid", Y, R, X, W, M, K, N)
        fh.call("accum", G, Y, M * N, 1)
        fh.call("matmulT_bwd_w", W, Y, X, M, K, N, 1)  # W += Yᵀ·X (in-place state, as Adam updates params)

    xs = [(rng.standard_normal(M * K) * 0.05).astype(np.float32) for _ in range(5)]
    rs = [rng.standard_normal(M * N).astype(np.float32) for _ in range(5)]
    W0 = W.numpy()
    # eager reference
    We = up(fh, W0)
    Ge = fh.DeviceArray.zeros((M * N,))
    eager = []
    for i in range(5):
        X.upload(xs[i]); R.upload(rs[i])
        fh.call("matmulT_fwd_resid", Y, R, X, We, M, K, N)
        fh.call("accum", Ge, Y, M * N, 1)
        fh.call("matmulT_bwd_w", We, Y, X, M, K, N, 1)
        eager.append((Y.numpy(), Ge.numpy(), We.numpy()))
    # recorded
    W.upload(W0)
    G.upload(np.zeros(M * N, np.float32))
    X.upload(xs[0]); R.upload(rs[0])
    body()
    got0 = (Y.numpy(), G.numpy(), W.numpy())
    X.upload(xs[1]); R.upload(rs[1])
    fh.call("graph_begin")
    try:
        with pytest.raises(fh.ForgeError, match="captured"):
            X.upload(xs[1])  # a host staging copy cannot be recorded
        body()
        gp = ctypes.c_void_p()
        fh.check(fh.lib.fg_graph_end(ctypes.byref(gp)), "fg_graph_end")
    except Exception:
        fh.lib.fg_graph_abort()
        raise
    outs = [got0]
    try:
        for i in range(1, 5):
            if i > 1:
                X.upload(xs[i]); R.upload(rs[i])
            fh.check(fh.lib.fg_graph_launch(gp), "fg_graph_launch")
            fh.sync()
            scratch = fh.DeviceArray((M * N,))  # eager work between replays
            fh.call("add_fwd", scratch, Y, G, M * N)
            outs.append((Y.numpy(), G.numpy(), W.numpy()))
    finally:
        fh.check(fh.lib.fg_graph_destroy(gp), "fg_graph_destroy")
    for i, (a, b) in enumerate(zip(outs, eager)):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y, err_msg="replay %d" % i)


@pytest.mark.gpu
def test_graph_abort_restores_eager_use(fh):
    fh.call("graph_begin")
    with pytest.raises(fh.ForgeError, match="captured"):
        fh.sync()
    with pytest.raises(fh.ForgeError, match="already"):
        fh.call("graph_begin")
    fh.check(fh.lib.fg_graph_abort(), "fg_graph_abort")
    x = fh.DeviceArray.from_numpy(np.arange(10, dtype=np.float32))
    fh.call("fill_f32", x, ctypes.c_float(3.0), 5)
    assert x.numpy().tolist() == [3.0] * 5 + [5.0, 6.0, 7.0, 8.0, 9.0]


def _first_loss_125m_oracle():
    """The oracle's loss for the first step of the 125M case of
    tests/js/train_loop.mjs: initWeights(cfg, 1337) with the untied head drawn
    from RNG(99), token data tokens(200000, 32000, 8), the first B = 8 window
    starts of train()'s RNG(7) (train.js:255-260), forward + CE only."""
    d, H, L, V, B, T = 768, 2048, 12, 32000, 8, 1024
    tied = oracle.Cfg(dim=d, hidden=H, nLayers=L, nHeads=12, nKvHeads=12, vocab=V, tied=1)
    parts = oracle.split_params(tied, oracle.init_weights(tied, 1337))
    wcls = oracle.RNG(99).normal_f32(V * d, 0.02)
    names = list(parts)
    flat = np.concatenate([parts["tok_emb"], parts["ln_f"], wcls] + [parts[k] for k in names[2:]])
    data = oracle.RNG(8).ints(200000, V)
    r = oracle.RNG(7)
    starts = [r.int(max(1, len(data) - T - 1)) for _ in range(B)]
    rows = np.stack([data[np.minimum(np.arange(s, s + T + 1), len(data) - 1)] for s in starts])
    untied = oracle.Cfg(dim=d, hidden=H, nLayers=L, nHeads=12, nKvHeads=12, vocab=V, tied=0)
    _, loss = oracle.model_loss(untied, flat, rows[:, :T].ravel(), rows[:, 1:].ravel(), B, T)
    return float(loss)


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_train_loop_js(fh):
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "train_loop.mjs")], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    import json
    res = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    for x in res:
        print(x["test"], "ok" if x["ok"] else "FAIL", x.get("detail") or x.get("error", ""))
    assert r.returncode == 0 and res and all(x["ok"] for x in res), r.stdout[-4000:]
    # the full 125M step (12 layers, B8 x T1024): its first loss against the
    # oracle's forward on the same weights and windows
    l0 = [x["loss0"] for x in res if x.get("spec") == "125m"]
    assert len(l0) == 1
    ref = _first_loss_125m_oracle()
    print("125m first loss: gpu %.7f oracle %.7f" % (l0[0], ref))
    assert abs(l0[0] - ref) <= 1e-5 * abs(ref)
