"""Independent fp64 restatement of the training path in vectorised closed forms.

TEST INFRASTRUCTURE ONLY (pins the C oracle; generates tests/golden fixtures).
Unlike forge_oracle.c, which follows the reference's loops (fp64 arithmetic,
fp32 stores), this module computes each quantity in float64 end to end from
its mathematical definition, so the two agree to fp32 rounding and a wrong
index, sign or dropped term in either shows up as a gross mismatch:

  matmulT      Y = X W^T, dX = G W, dW = G^T X                 (tensor.js:34-53)
  rmsNorm      y = x w / sqrt(mean(x^2)+eps); grads by the chain rule  (:103-128)
  ropeRows     complex rotation (a + ib) e^{i pos theta^(-i/d)}          (:133-166)
  attention    masked softmax(Q K^T / sqrt(d)) V and its Jacobian-vector products (:191-376)
  swiglu       g sigma(g) u                                     (:272-290)
  CE           mean(lse - x_target), (softmax - onehot)/T       (:393-417)
  Adam         autograd.js:221-243 in float64
  model        train.js:120-159 forward in float64
"""
import numpy as np


def matmulT(X, W):
    return X @ W.T


def matmulT_grads(G, X, W):
    return G @ W, G.T @ X


def rmsnorm(X, w, eps):
    r = np.sqrt(np.mean(X * X, axis=1, keepdims=True) + eps)
    return X / r * w, 1.0 / r[:, 0]


def rmsnorm_grads(G, X, w, eps):
    D = X.shape[1]
    r = np.sqrt(np.mean(X * X, axis=1, keepdims=True) + eps)
    gw = np.sum(G * X / r, axis=0)
    gx = G * w / r - X * np.sum(G * w * X, axis=1, keepdims=True) / (D * r ** 3)
    return gx, gw


def rope_angles(T, dHead, pos0=0, theta=1e4, posStride=0):
    t = np.arange(T)
    pos = pos0 + (t % posStride if posStride > 0 else t)
    i = np.arange(0, dHead, 2)
    return pos[:, None].astype(np.float64) * (1.0 / np.power(theta, i / dHead))[None, :]


def rope(X, nHead, dHead, pos0=0, theta=1e4, posStride=0, inverse=False):
    T = X.shape[0]
    ang = rope_angles(T, dHead, pos0, theta, posStride)
    z = X.reshape(T, nHead, dHead // 2, 2)
    c = z[..., 0] + 1j * z[..., 1]
    rot = np.exp((-1j if inverse else 1j) * ang)[:, None, :]
    o = c * rot
    return np.stack([o.real, o.imag], -1).reshape(T, nHead * dHead)


def attention(Q, K, V, B, T, nH, nKV, dH):
    """Returns O and a closure computing (dQ, dK, dV) for an upstream dO."""
    group = max(1, nH // nKV)
    Q4 = Q.reshape(B, T, nH, dH)
    K4 = K.reshape(B, T, nKV, dH)
    V4 = V.reshape(B, T, nKV, dH)
    mask = np.triu(np.ones((T, T), bool), 1)
    O = np.zeros_like(Q4)
    Ps = {}
    for b in range(B):
        for h in range(nH):
            kv = h // group
            S = Q4[b, :, h] @ K4[b, :, kv].T / np.sqrt(dH)
            S[mask] = -np.inf
            S -= S.max(1, keepdims=True)
            P = np.exp(S)
            P /= P.sum(1, keepdims=True)
            Ps[b, h] = P
            O[b, :, h] = P @ V4[b, :, kv]

    def grads(dO):
        dO4 = dO.reshape(B, T, nH, dH)
        dQ, dK, dV = np.zeros_like(Q4), np.zeros_like(K4), np.zeros_like(V4)
        for b in range(B):
            for h in range(nH):
                kv = h // group
                P = Ps[b, h]
                dP = dO4[b, :, h] @ V4[b, :, kv].T
                dS = P * (dP - np.sum(dP * P, axis=1, keepdims=True))
                dQ[b, :, h] += dS @ K4[b, :, kv] / np.sqrt(dH)
                dK[b, :, kv] += dS.T @ Q4[b, :, h] / np.sqrt(dH)
                dV[b, :, kv] += P.T @ dO4[b, :, h]
        return dQ.reshape(Q.shape), dK.reshape(K.shape), dV.reshape(V.shape)

    return O.reshape(Q.shape), grads


def swiglu(G, U):
    s = 1.0 / (1.0 + np.exp(-G))
    return G * s * U


def swiglu_grads(dO, G, U):
    s = 1.0 / (1.0 + np.exp(-G))
    return dO * U * (s + G * s * (1 - s)), dO * G * s


def ce(logits, targets):
    T = logits.shape[0]
    m = logits.max(1, keepdims=True)
    lse = m[:, 0] + np.log(np.sum(np.exp(logits - m), axis=1))
    loss = np.mean(lse - logits[np.arange(T), targets])
    P = np.exp(logits - lse[:, None])
    P[np.arange(T), targets] -= 1.0
    return loss, P / T


def adam(p, g, m, v, t, lr, b1, b2, eps, wd, clip, total):
    """One step on lists of float64 arrays (None grads skipped)."""
    gnorm = np.sqrt(sum(float(np.sum(x * x)) for x in g if x is not None))
    scale = clip / gnorm if gnorm > clip else 1.0
    lr_t = lr * 0.5 * (1 + np.cos(np.pi * min(t / total, 1.0)))
    out = []
    for pj, gj, mj, vj in zip(p, g, m, v):
        if gj is None:
            out.append((pj, mj, vj))
            continue
        gg = gj * scale + wd * pj
        mj = b1 * mj + (1 - b1) * gg
        vj = b2 * vj + (1 - b2) * gg * gg
        pj = pj - lr_t * (mj / (1 - b1 ** t)) / (np.sqrt(vj / (1 - b2 ** t)) + eps)
        out.append((pj, mj, vj))
    return out, gnorm, scale, lr_t


def model_loss(P, ids, targets, B, T, dim, hidden, nLayers, nHeads, nKvHeads, vocab, eps=1e-5, theta=1e4,
               tied=True):
    """float64 forward of TrainableTransformer.lossBatch (train.js:120-185).
    P: dict of float64 arrays keyed like the paramList names."""
    dH = dim // nHeads
    qD, kvD = nHeads * dH, nKvHeads * dH
    x = P["tok_emb"].reshape(vocab, dim)[ids]
    for l in range(nLayers):
        pre = "layer.%d." % l
        xn, _ = rmsnorm(x, P[pre + "ln1"], eps)
        qkv = xn @ P[pre + "wqkv"].reshape(-1, dim).T
        q, k, v = qkv[:, :qD], qkv[:, qD:qD + kvD], qkv[:, qD + kvD:]
        q = rope(q, nHeads, dH, 0, theta, T)
        k = rope(k, nKvHeads, dH, 0, theta, T)
        att, _ = attention(q, k, v, B, T, nHeads, nKvHeads, dH)
        x = x + att @ P[pre + "wo"].reshape(dim, qD).T
        xn2, _ = rmsnorm(x, P[pre + "ln2"], eps)
        g = xn2 @ P[pre + "ffn_gate"].reshape(hidden, dim).T
        u = xn2 @ P[pre + "ffn_up"].reshape(hidden, dim).T
        x = x + swiglu(g, u) @ P[pre + "ffn_down"].reshape(dim, hidden).T
    xf, _ = rmsnorm(x, P["ln_f"], eps)
    W = P["tok_emb"] if tied else P["wcls"]
    logits = xf @ W.reshape(vocab, dim).T
    loss, _ = ce(logits, targets)
    return loss, logits
