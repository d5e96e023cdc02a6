"""numpy-facing wrapper of the C oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the parity reference or the timed CPU baseline.  The
product (forge-llm_amd/) never imports it.

Every function takes/returns numpy arrays with the reference's layouts
(row-major fp32, int32 ids) and calls the C restatement in forge_oracle.c,
which cites the reference file:line it follows.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBPATH = os.path.join(HERE, "liboracle.so")


def build():
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


if not os.path.exists(LIBPATH):
    build()
_lib = ctypes.CDLL(LIBPATH)

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_int64
D = ctypes.c_double
U = ctypes.c_uint32


def _sig(name, res, *args):
    f = getattr(_lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


_sig("or_rng_new", P, U)
_sig("or_rng_free", None, P)
_sig("or_rng_next", D, P)
_sig("or_rng_normal", D, P)
_sig("or_rng_int", I, P, I)
_sig("or_rng_fill_normal", None, P, P, L, D)
_sig("or_rng_fill_next", None, P, P, L)
_sig("or_rng_fill_int", None, P, P, L, I)
_sig("or_gemm", None, P, P, P, I, I, I)
_sig("or_matmulT_bwd", None, P, P, P, P, P, I, I, I)
_sig("or_matmulT_bwd_serial", None, P, P, P, P, P, I, I, I)
_sig("or_embed_fwd", None, P, P, P, I, I)
_sig("or_embed_bwd", None, P, P, P, I, I)
_sig("or_rmsnorm_fwd", None, P, P, P, P, I, I, D)
_sig("or_rmsnorm_bwd", None, P, P, P, P, P, P, I, I)
_sig("or_rope_fwd", None, P, P, I, I, I, I, D, I)
_sig("or_rope_bwd", None, P, P, I, I, I, I, D, I)
_sig("or_rope_table", None, P, P, I, I, D)
_sig("or_slice_fwd", None, P, P, I, I, I, I)
_sig("or_slice_bwd", None, P, P, I, I, I, I)
_sig("or_attn_fwd", None, P, P, P, P, P, I, I, I, I, I)
_sig("or_attn_bwd", None, P, P, P, P, P, P, P, P, I, I, I, I, I)
_sig("or_swiglu_fwd", None, P, P, P, P, L)
_sig("or_swiglu_bwd", None, P, P, P, P, P, P, L)
_sig("or_weighted_sum_fwd", None, P, P, P, L)
_sig("or_weighted_sum_bwd", None, P, D, P, L)
_sig("or_ce_fwd", None, P, P, P, P, I, I)
_sig("or_ce_bwd", None, P, D, P, P, I, I)
_sig("or_add_fwd", None, P, P, P, L)
_sig("or_accum", None, P, P, L)
_sig("or_adam_step", None, I, P, P, P, P, P, I, D, D, D, D, D, D, D, P)
_sig("or_adam_step_given_norm", None, I, P, P, P, P, P, I, D, D, D, D, D, D, D, D, P)
_sig("or_param_count", L, P)
_sig("or_init_weights", None, P, U, D, P)
_sig("or_model_fwd_bwd", None, P, P, P, P, I, I, P, P, P)
_sig("or_infer_forward", None, P, P, P, I, P)
_sig("or_infer_forward_q", None, P, P, P, I, P)
_sig("oq_fp16_to_fp32", D, ctypes.c_uint16)
_sig("oq_fp32_to_fp16", ctypes.c_uint16, D)
_sig("oq_row_bytes", L, I, L)
_sig("oq_dequantize", I, I, P, L, P)
_sig("oq_dotq", D, I, P, P, L)
_sig("oq_qmatvec", None, I, P, P, P, I, I)
_sig("oq_quantize", I, I, P, L, P)
_sig("or_vec_mul_fwd", None, P, P, P, L, L)
_sig("or_vec_mul_bwd", None, P, P, P, P, P, L, L)
_sig("or_vec_silu_fwd", None, P, P, P, L)
_sig("or_vec_silu_bwd", None, P, P, P, P, L)
_sig("or_vec_dot_fwd", None, P, P, P, L)
_sig("or_vec_dot_bwd", None, P, P, P, P, P, L)
_sig("or_vec_scale_fwd", None, P, P, D, L)
_sig("or_vec_scale_bwd", None, P, P, D, L)
_sig("or_vec_rope_fwd", None, P, P, P, P, L, I)
_sig("or_vec_rope_bwd", None, P, P, P, P, I)
_sig("or_vec_softmax_fwd", None, P, P, P, L)
_sig("or_vec_softmax_bwd", None, P, P, P, L)
_sig("or_attention_decode", None, P, P, P, P, I, I, D, I, I, P)
_sig("or_attention_naive", None, P, P, P, P, I, I, D, I, I)
_sig("or_flash_attention", None, P, P, P, P, I, I, D, I, I, I)
_sig("or_row_rmsnorm", None, P, P, P, I, D)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


# ── RNG (numeric.js:27-49) ──────────────────────────────────────────────────
class RNG:
    def __init__(self, seed):
        self._h = _lib.or_rng_new(seed & 0xFFFFFFFF)

    def __del__(self):
        if getattr(self, "_h", None):
            _lib.or_rng_free(self._h)

    def next(self):
        return _lib.or_rng_next(self._h)

    def normal(self):
        return _lib.or_rng_normal(self._h)

    def int(self, n):
        return _lib.or_rng_int(self._h, n)

    def normal_f32(self, n, scale=1.0):
        out = np.empty(int(n), np.float32)
        _lib.or_rng_fill_normal(self._h, _p(out), int(n), float(scale))
        return out

    def next_many(self, n):
        out = np.empty(int(n), np.float64)
        _lib.or_rng_fill_next(self._h, _p(out), int(n))
        return out

    def ints(self, n, rng_range):
        out = np.empty(int(n), np.int32)
        _lib.or_rng_fill_int(self._h, _p(out), int(n), int(rng_range))
        return out


# ── ops ─────────────────────────────────────────────────────────────────────
def matmulT_fwd(X, W, M, K, N):
    X, W = f32(X), f32(W)
    Y = np.empty(M * N, np.float32)
    _lib.or_gemm(_p(Y), _p(X), _p(W), M, N, K)
    return Y


def matmulT_bwd(g, X, W, M, K, N, gX=None, gW=None):
    g, X, W = f32(g), f32(X), f32(W)
    gX = np.zeros(M * K, np.float32) if gX is None else f32(gX).copy()
    gW = np.zeros(N * K, np.float32) if gW is None else f32(gW).copy()
    _lib.or_matmulT_bwd(_p(gX), _p(gW), _p(g), _p(X), _p(W), M, K, N)
    return gX, gW


def matmulT_bwd_serial(g, X, W, M, K, N):
    """The reference's single interleaved m, n, k loop (no threads, no split)."""
    g, X, W = f32(g), f32(X), f32(W)
    gX = np.zeros(M * K, np.float32)
    gW = np.zeros(N * K, np.float32)
    _lib.or_matmulT_bwd_serial(_p(gX), _p(gW), _p(g), _p(X), _p(W), M, K, N)
    return gX, gW


def set_threads(n):
    """OpenMP threads of the oracle's large loops (results do not depend on it)."""
    ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))


def embed_fwd(W, ids, D):
    W, ids = f32(W), i32(ids)
    out = np.empty(len(ids) * D, np.float32)
    _lib.or_embed_fwd(_p(out), _p(W), _p(ids), len(ids), D)
    return out


def embed_bwd(g, ids, V, D, gW=None):
    g, ids = f32(g), i32(ids)
    gW = np.zeros(V * D, np.float32) if gW is None else f32(gW).copy()
    _lib.or_embed_bwd(_p(gW), _p(g), _p(ids), len(ids), D)
    return gW


def rmsnorm_fwd(X, w, T, D, eps):
    X, w = f32(X), f32(w)
    out = np.empty(T * D, np.float32)
    inv = np.empty(T, np.float32)
    _lib.or_rmsnorm_fwd(_p(out), _p(inv), _p(X), _p(w), T, D, float(eps))
    return out, inv


def rmsnorm_bwd(g, X, w, inv, T, D, gX=None, gw=None):
    g, X, w, inv = f32(g), f32(X), f32(w), f32(inv)
    gX = np.zeros(T * D, np.float32) if gX is None else f32(gX).copy()
    gw = np.zeros(D, np.float32) if gw is None else f32(gw).copy()
    _lib.or_rmsnorm_bwd(_p(gX), _p(gw), _p(g), _p(X), _p(w), _p(inv), T, D)
    return gX, gw


def rope_fwd(X, T, nHead, dHead, pos0=0, theta=10000.0, posStride=0):
    X = f32(X)
    out = np.empty(T * nHead * dHead, np.float32)
    _lib.or_rope_fwd(_p(out), _p(X), T, nHead, dHead, pos0, float(theta), posStride)
    return out


def rope_bwd(g, T, nHead, dHead, pos0=0, theta=10000.0, posStride=0, gX=None):
    g = f32(g)
    gX = np.zeros(T * nHead * dHead, np.float32) if gX is None else f32(gX).copy()
    _lib.or_rope_bwd(_p(gX), _p(g), T, nHead, dHead, pos0, float(theta), posStride)
    return gX


def rope_table(npos, dHead, theta):
    c = np.empty(npos * (dHead // 2), np.float64)
    s = np.empty(npos * (dHead // 2), np.float64)
    _lib.or_rope_table(_p(c), _p(s), npos, dHead, float(theta))
    return c, s


def slice_fwd(X, M, K, off, ln):
    X = f32(X)
    out = np.empty(M * ln, np.float32)
    _lib.or_slice_fwd(_p(out), _p(X), M, K, off, ln)
    return out


def slice_bwd(g, M, K, off, ln, gX=None):
    g = f32(g)
    gX = np.zeros(M * K, np.float32) if gX is None else f32(gX).copy()
    _lib.or_slice_bwd(_p(gX), _p(g), M, K, off, ln)
    return gX


def attn_fwd(Q, K, V, B, T, nH, nKV, dH):
    Q, K, V = f32(Q), f32(K), f32(V)
    out = np.empty(B * T * nH * dH, np.float32)
    Pm = np.empty(B * nH * T * T, np.float32)
    _lib.or_attn_fwd(_p(out), _p(Pm), _p(Q), _p(K), _p(V), B, T, nH, nKV, dH)
    return out, Pm


def attn_bwd(g, Pm, Q, K, V, B, T, nH, nKV, dH):
    g, Pm, Q, K, V = f32(g), f32(Pm), f32(Q), f32(K), f32(V)
    gQ = np.zeros(B * T * nH * dH, np.float32)
    gK = np.zeros(B * T * nKV * dH, np.float32)
    gV = np.zeros(B * T * nKV * dH, np.float32)
    _lib.or_attn_bwd(_p(gQ), _p(gK), _p(gV), _p(g), _p(Pm), _p(Q), _p(K), _p(V), B, T, nH, nKV, dH)
    return gQ, gK, gV


def swiglu_fwd(G, U):
    G, U = f32(G), f32(U)
    out = np.empty(G.size, np.float32)
    sig = np.empty(G.size, np.float32)
    _lib.or_swiglu_fwd(_p(out), _p(sig), _p(G), _p(U), G.size)
    return out, sig


def swiglu_bwd(g, sig, G, U, gG=None, gU=None):
    g, sig, G, U = f32(g), f32(sig), f32(G), f32(U)
    gG = np.zeros(G.size, np.float32) if gG is None else f32(gG).copy()
    gU = np.zeros(G.size, np.float32) if gU is None else f32(gU).copy()
    _lib.or_swiglu_bwd(_p(gG), _p(gU), _p(g), _p(sig), _p(G), _p(U), G.size)
    return gG, gU


def weighted_sum_fwd(Y, t):
    Y, t = f32(Y), f32(t)
    out = np.zeros(1, np.float32)
    _lib.or_weighted_sum_fwd(_p(out), _p(Y), _p(t), Y.size)
    return out[0]


def weighted_sum_bwd(g0, t, gY=None):
    t = f32(t)
    gY = np.zeros(t.size, np.float32) if gY is None else f32(gY).copy()
    _lib.or_weighted_sum_bwd(_p(gY), float(g0), _p(t), t.size)
    return gY


def ce_fwd(logits, targets, T, V):
    logits, targets = f32(logits), i32(targets)
    out = np.zeros(1, np.float32)
    probs = np.empty(T * V, np.float32)
    _lib.or_ce_fwd(_p(out), _p(probs), _p(logits), _p(targets), T, V)
    return out[0], probs


def ce_bwd(g0, probs, targets, T, V, gL=None):
    probs, targets = f32(probs), i32(targets)
    gL = np.zeros(T * V, np.float32) if gL is None else f32(gL).copy()
    _lib.or_ce_bwd(_p(gL), float(g0), _p(probs), _p(targets), T, V)
    return gL


def add_fwd(a, b):
    a, b = f32(a), f32(b)
    out = np.empty(a.size, np.float32)
    _lib.or_add_fwd(_p(out), _p(a), _p(b), a.size)
    return out


def adam_step(params, grads, ms, vs, t, lr=3e-4, b1=0.9, b2=0.999, eps=1e-8, wd=0.0, clip=1.0, total=1000,
              gnorm=None):
    """In place on lists of fp32 arrays (grads entries may be None).  With
    `gnorm` given, the clip uses it instead of the norm of `grads` (a step
    checked on a subset of the parameters)."""
    n = len(params)
    arrP = (ctypes.c_void_p * n)(*[_p(a) for a in params])
    arrG = (ctypes.c_void_p * n)(*[(_p(g) if g is not None else None) for g in grads])
    arrM = (ctypes.c_void_p * n)(*[_p(a) for a in ms])
    arrV = (ctypes.c_void_p * n)(*[_p(a) for a in vs])
    ns = np.array([a.size for a in params], np.int64)
    out = np.zeros(3, np.float64)
    if gnorm is None:
        _lib.or_adam_step(n, arrP, arrG, arrM, arrV, _p(ns), int(t), float(lr), float(b1), float(b2), float(eps),
                          float(wd), float(clip), float(total), _p(out))
    else:
        _lib.or_adam_step_given_norm(n, arrP, arrG, arrM, arrV, _p(ns), int(t), float(lr), float(b1), float(b2),
                                     float(eps), float(wd), float(clip), float(total), float(gnorm), _p(out))
    return {"lr": out[0], "gnorm": out[1], "scale": out[2]}


# ── model ───────────────────────────────────────────────────────────────────
class Cfg(ctypes.Structure):
    """Config (transformer.js:29-53) plus the tied/untied LM head flag."""
    _fields_ = [("dim", I), ("hidden", I), ("nLayers", I), ("nHeads", I), ("nKvHeads", I), ("vocab", I),
                ("normEps", D), ("ropeTheta", D), ("tied", I)]

    def __init__(self, dim=288, hidden=768, nLayers=6, nHeads=6, nKvHeads=6, vocab=32000, normEps=1e-5,
                 ropeTheta=10000.0, tied=1):
        super().__init__(dim, hidden, nLayers, nHeads, nKvHeads, vocab, normEps, ropeTheta, tied)

    @property
    def dHead(self):
        return self.dim // self.nHeads

    @property
    def qkvOut(self):
        return (self.nHeads + 2 * self.nKvHeads) * self.dHead

    def param_shapes(self):
        """[(name, numel)] in paramList order (train.js:60-78)."""
        d, h, v = self.dim, self.hidden, self.vocab
        out = [("tok_emb", v * d), ("ln_f", d)]
        if not self.tied:
            out.append(("wcls", v * d))
        for l in range(self.nLayers):
            out += [("layer.%d.ln1" % l, d), ("layer.%d.ln2" % l, d), ("layer.%d.wqkv" % l, self.qkvOut * d),
                    ("layer.%d.wo" % l, d * d), ("layer.%d.ffn_gate" % l, h * d),
                    ("layer.%d.ffn_up" % l, h * d), ("layer.%d.ffn_down" % l, d * h)]
        return out


def param_count(cfg):
    return _lib.or_param_count(ctypes.byref(cfg))


def init_weights(cfg, seed, std=0.02):
    out = np.empty(param_count(cfg), np.float32)
    _lib.or_init_weights(ctypes.byref(cfg), seed & 0xFFFFFFFF, float(std), _p(out))
    return out


def split_params(cfg, flat):
    out, o = {}, 0
    for name, n in cfg.param_shapes():
        out[name] = flat[o:o + n]
        o += n
    return out


def model_fwd_bwd(cfg, params, ids, targets, B, T):
    params, ids, targets = f32(params), i32(ids), i32(targets)
    logits = np.empty(B * T * cfg.vocab, np.float32)
    loss = np.zeros(1, np.float32)
    grads = np.zeros(params.size, np.float32)
    _lib.or_model_fwd_bwd(ctypes.byref(cfg), _p(params), _p(ids), _p(targets), B, T, _p(logits), _p(loss),
                          _p(grads))
    return logits, loss[0], grads


def model_loss(cfg, params, ids, targets, B, T):
    """Forward and loss only (logits, loss) of model_fwd_bwd."""
    params, ids, targets = f32(params), i32(ids), i32(targets)
    logits = np.empty(B * T * cfg.vocab, np.float32)
    loss = np.zeros(1, np.float32)
    _lib.or_model_fwd_bwd(ctypes.byref(cfg), _p(params), _p(ids), _p(targets), B, T, _p(logits), _p(loss), None)
    return logits, loss[0]


def infer_forward(cfg, params, ids):
    params, ids = f32(params), i32(ids)
    logits = np.empty(len(ids) * cfg.vocab, np.float32)
    _lib.or_infer_forward(ctypes.byref(cfg), _p(params), _p(ids), len(ids), _p(logits))
    return logits


# ── quantized weights (quant_oracle.c: quant.js, special.js:143-168, nn.js) ──
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q5_0": 6, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 6: (32, 22), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def fp16_to_fp32(h):
    return _lib.oq_fp16_to_fp32(int(h) & 0xFFFF)


def fp32_to_fp16(x):
    return _lib.oq_fp32_to_fp16(float(x))


def row_bytes(t, n):
    return _lib.oq_row_bytes(t, n)


def quantize(t, x):
    """quantizeRow(t, x, len(x)) → uint8 array of row_bytes(t, len(x))."""
    x = f32(x)
    out = np.zeros(row_bytes(t, x.size), np.uint8)
    if _lib.oq_quantize(t, _p(x), x.size, _p(out)) != 0:
        raise ValueError("no quantizer for type %d" % t)
    return out


def dequantize(t, q, n):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(n, np.float32)
    if _lib.oq_dequantize(t, _p(q), n, _p(out)) != 0:
        raise ValueError("no decoder for type %d" % t)
    return out


def dotq(t, q, x):
    q, x = np.ascontiguousarray(q, dtype=np.uint8), f32(x)
    return _lib.oq_dotq(t, _p(q), _p(x), x.size)


def qmatvec(t, W, x, N, K):
    W, x = np.ascontiguousarray(W, dtype=np.uint8), f32(x)
    y = np.empty(N, np.float32)
    _lib.oq_qmatvec(t, _p(y), _p(W), _p(x), N, K)
    return y


class _QMat(ctypes.Structure):
    _fields_ = [("type", I), ("data", P)]


class _QLayer(ctypes.Structure):
    _fields_ = [("ln1", P), ("ln2", P)] + [(n, _QMat) for n in ("wqkv", "wo", "gate", "up", "down")]


class _QModel(ctypes.Structure):
    _fields_ = [("tok_emb", _QMat), ("ln_f", P), ("wcls", _QMat), ("layers", P)]


def infer_forward_q(cfg, model, ids):
    """or_infer_forward_q over typed weights.  model: {"tok_emb": (type, bytes),
    "ln_f": f32, "wcls": (type, bytes), "layers": [{"ln1", "ln2": f32,
    "wqkv", "wo", "gate", "up", "down": (type, bytes)}]}."""
    keep = []

    def qm(tb):
        t, b = tb
        b = np.asarray(b)
        b = np.ascontiguousarray(b) if b.dtype == np.uint8 else f32(b)
        keep.append(b)
        return _QMat(t, b.ctypes.data)

    def fp(a):
        a = f32(a)
        keep.append(a)
        return a.ctypes.data

    layers = (_QLayer * cfg.nLayers)()
    for l, L_ in enumerate(model["layers"]):
        layers[l] = _QLayer(fp(L_["ln1"]), fp(L_["ln2"]), qm(L_["wqkv"]), qm(L_["wo"]), qm(L_["gate"]),
                            qm(L_["up"]), qm(L_["down"]))
    m = _QModel(qm(model["tok_emb"]), fp(model["ln_f"]), qm(model["wcls"]), ctypes.addressof(layers))
    ids = i32(ids)
    logits = np.empty(len(ids) * cfg.vocab, np.float32)
    _lib.or_infer_forward_q(ctypes.byref(cfg), ctypes.byref(m), _p(ids), len(ids), _p(logits))
    return logits


# ── vector-level autograd ops (autograd.js:70-190) ─────────────────────────
# Backward wrappers take the gradients' current values (zeros for a fresh
# gradient) and return the updated copies.
def vec_mul_fwd(a, b):
    a, b = f32(a), f32(b)
    out = np.empty(a.size, np.float32)
    _lib.or_vec_mul_fwd(_p(out), _p(a), _p(b), a.size, b.size)
    return out


def vec_mul_bwd(g, a, b, ga=None, gb=None):
    g, a, b = f32(g), f32(a), f32(b)
    ga = np.zeros(a.size, np.float32) if ga is None else f32(ga).copy()
    gb = np.zeros(b.size, np.float32) if gb is None else f32(gb).copy()
    _lib.or_vec_mul_bwd(_p(ga), _p(gb), _p(g), _p(a), _p(b), a.size, b.size)
    return ga, gb


def vec_silu_fwd(x):
    x = f32(x)
    out, s = np.empty(x.size, np.float32), np.empty(x.size, np.float32)
    _lib.or_vec_silu_fwd(_p(out), _p(s), _p(x), x.size)
    return out, s


def vec_silu_bwd(g, x, s, gx=None):
    g, x, s = f32(g), f32(x), f32(s)
    gx = np.zeros(x.size, np.float32) if gx is None else f32(gx).copy()
    _lib.or_vec_silu_bwd(_p(gx), _p(g), _p(x), _p(s), x.size)
    return gx


def vec_dot_fwd(a, b):
    a, b = f32(a), f32(b)
    out = np.zeros(1, np.float32)
    _lib.or_vec_dot_fwd(_p(out), _p(a), _p(b), a.size)
    return out[0]


def vec_dot_bwd(g0, a, b, ga=None, gb=None):
    a, b = f32(a), f32(b)
    g = np.array([g0], np.float32)
    ga = np.zeros(a.size, np.float32) if ga is None else f32(ga).copy()
    gb = np.zeros(b.size, np.float32) if gb is None else f32(gb).copy()
    _lib.or_vec_dot_bwd(_p(ga), _p(gb), _p(g), _p(a), _p(b), a.size)
    return ga, gb


def vec_scale_fwd(x, s):
    x = f32(x)
    out = np.empty(x.size, np.float32)
    _lib.or_vec_scale_fwd(_p(out), _p(x), float(s), x.size)
    return out


def vec_scale_bwd(g, s, gx=None):
    g = f32(g)
    gx = np.zeros(g.size, np.float32) if gx is None else f32(gx).copy()
    _lib.or_vec_scale_bwd(_p(gx), _p(g), float(s), g.size)
    return gx


def vec_rope_fwd(x, cos, sin, dH):
    x = f32(x)
    c, s = np.ascontiguousarray(cos, np.float64), np.ascontiguousarray(sin, np.float64)
    out = np.empty(x.size, np.float32)
    _lib.or_vec_rope_fwd(_p(out), _p(x), _p(c), _p(s), x.size, dH)
    return out


def vec_rope_bwd(g, cos, sin, dH, gx=None):
    g = f32(g)
    c, s = np.ascontiguousarray(cos, np.float64), np.ascontiguousarray(sin, np.float64)
    gx = np.zeros(g.size, np.float32) if gx is None else f32(gx).copy()
    _lib.or_vec_rope_bwd(_p(gx), _p(g), _p(c), _p(s), dH)
    return gx


def vec_softmax_fwd(x):
    x = f32(x)
    out, p = np.empty(x.size, np.float32), np.empty(x.size, np.float32)
    _lib.or_vec_softmax_fwd(_p(out), _p(p), _p(x), x.size)
    return out, p


def vec_softmax_bwd(g, p, gx=None):
    g, p = f32(g), f32(p)
    gx = np.zeros(p.size, np.float32) if gx is None else f32(gx).copy()
    _lib.or_vec_softmax_bwd(_p(gx), _p(g), _p(p), p.size)
    return gx


# ── single-row attention (attention.js:31-126) and rmsnormInto (nn.js:42-44) ──
def attention_decode(q, K, V, n, d, scale, causal=True, qOff=0):
    """Returns (out, scores) as attentionDecode leaves them."""
    q, K, V = f32(q), f32(K), f32(V)
    out, sc = np.empty(d, np.float32), np.empty(max(n, 1), np.float32)
    _lib.or_attention_decode(_p(out), _p(q), _p(K), _p(V), n, d, float(scale), int(causal), qOff, _p(sc))
    return out, sc[:n]


def attention_naive(q, K, V, n, d, scale, causal=True, qOff=0):
    q, K, V = f32(q), f32(K), f32(V)
    out = np.empty(d, np.float32)
    _lib.or_attention_naive(_p(out), _p(q), _p(K), _p(V), n, d, float(scale), int(causal), qOff)
    return out


def flash_attention(q, K, V, n, d, scale, causal=True, qOff=0, block=64):
    q, K, V = f32(q), f32(K), f32(V)
    out = np.empty(d, np.float32)
    _lib.or_flash_attention(_p(out), _p(q), _p(K), _p(V), n, d, float(scale), int(causal), qOff, block)
    return out


def row_rmsnorm(x, w, eps=1e-6):
    x, w = f32(x), f32(w)
    out = np.empty(x.size, np.float32)
    _lib.or_row_rmsnorm(_p(out), _p(x), _p(w), x.size, float(eps))
    return out
