"""CPU restatement of the reference's host-op reference() bodies (inference-scheduler/src/
host_nodes.py, llm_nodes.py) in numpy float64 with the C library's exp / erf / tanh through
Python's math module, as the reference computes them.  TEST INFRASTRUCTURE ONLY (the checker,
never the thing measured or shipped); nothing here imports the product.
"""
import math

import numpy as np

_LIBM = {name: np.vectorize(getattr(math, name), otypes=[np.float64]) for name in ("exp", "tanh", "erf")}


def libm(name, x):
    """Elementwise glibc exp / tanh / erf of a float64 array (host_nodes.py:151-162)."""
    x = np.asarray(x, np.float64)
    return _LIBM[name](x) if x.size else x.copy()


def quantize_q88(x):
    """DataType.host_quantize for Q8.8 (dtype.py:214-219, 367-369): NaN -> 0, clip, round half even."""
    x = np.asarray(x, np.float64)
    x = np.where(np.isnan(x), 0.0, x)
    return np.round(np.clip(x, -128.0, 127.99609375) * 256.0) / 256.0


def quantize_exp(x, f):
    """DataType.quantize_exp (dtype.py:278-286): round half even at 2^-f, saturate, NaN -> 0."""
    s = np.power(2.0, np.asarray(f, np.float64))
    x = np.asarray(x, np.float64)
    r = np.round(np.where(np.isnan(x), 0.0, x) * s)
    return np.clip(r, -32768, 32767) / s


def f32(v):
    return np.asarray(v, np.float64).astype(np.float32).astype(np.float64)


def softmax(x, n):
    """SoftmaxNode.reference (host_nodes.py:1037-1041)."""
    x = np.asarray(x, np.float64).reshape(-1, n)
    e = libm("exp", x - x.max(axis=1, keepdims=True))
    s = np.cumsum(e, axis=1)[:, -1:]
    return quantize_q88(e / s)


def layer_norm(x, n, gamma, beta, eps, tf_form):
    """LayerNormNode.reference (host_nodes.py:1134-1148)."""
    x = np.asarray(x, np.float64).reshape(-1, n)
    ga = (np.ones(n) if gamma is None else np.asarray(gamma, np.float32).astype(np.float64))[None, :]
    be = (np.zeros(n) if beta is None else np.asarray(beta, np.float32).astype(np.float64))[None, :]
    mean = np.cumsum(x, axis=1)[:, -1:] / float(n)
    d = x - mean
    var = np.cumsum(d * d, axis=1)[:, -1:] / float(n)
    inv = 1.0 / np.sqrt(var + eps)
    if tf_form:
        g = inv * ga
        y = x * g + (be - mean * g)
    else:
        y = d * inv * ga + be
    return quantize_q88(y)


def gelu(v, approximate, c1, c2, k, div):
    """GeluNode.values (host_nodes.py:1228-1240)."""
    v = np.asarray(v, np.float64).reshape(-1)
    if approximate == "tanh":
        y = v * (0.5 * (1.0 + libm("tanh", c2 * (v + c1 * (v * v * v)))))
    else:
        u = v / k if div else v * k
        y = v * (0.5 * (1.0 + libm("erf", u)))
    return quantize_q88(y)


def rms_norm(h, gamma, eps, f_out, W):
    """LlmRMSNormNode.reference (llm_nodes.py:676-688), rows of gamma's n."""
    g = np.asarray(gamma, np.float32).astype(np.float64).reshape(-1)
    n = g.size
    h = np.asarray(h, np.float64).reshape(-1, n)
    ss = np.cumsum(h * h, axis=-1)[:, -1]
    r = 1.0 / np.sqrt(ss / float(n) + eps)
    y = ((h * r[:, None]) * g[None, :]).reshape(-1, W)
    return quantize_exp(y, np.asarray(f_out)[None, :])


def silu_table(f):
    """llm_nodes.silu_table (:322-332)."""
    t = np.empty(65536)
    d = 2.0 ** f
    for i in range(65536):
        g = (i - 32768 + 0.0) / d
        t[i] = g / (1.0 + math.exp(-g)) if g > -700 else 0.0
    return t


_SILU = {}


def silu_mul(g, u, f_gate, f_out):
    """LlmSiluMulNode.reference (llm_nodes.py:741-751)."""
    n = len(f_gate)
    g = np.asarray(g, np.float64).reshape(-1, n)
    u = np.asarray(u, np.float64).reshape(-1, n)
    sil = np.empty_like(g)
    for f in np.unique(f_gate):
        cols = np.asarray(f_gate) == f
        if int(f) not in _SILU:
            _SILU[int(f)] = silu_table(int(f))
        idx = np.floor(g[:, cols] * 2.0 ** int(f)).astype(np.int64) + 32768
        sil[:, cols] = _SILU[int(f)][idx]
    return quantize_exp(sil * u, np.asarray(f_out)[None, :])


def dot8(prod):
    """llm_nodes.dot8 (:292-301): 8 lanes in order, then the pairwise tree."""
    n, hd = prod.shape
    acc = np.cumsum(prod.reshape(n, hd // 8, 8), axis=1)[:, -1, :]
    return (((acc[:, 0] + acc[:, 1]) + (acc[:, 2] + acc[:, 3]))
            + ((acc[:, 4] + acc[:, 5]) + (acc[:, 6] + acc[:, 7])))


def rope(x, cos, sin):
    """llm_nodes.rope (:304-312)."""
    half = x.shape[-1] // 2
    c = np.concatenate([cos, cos]).astype(np.float64)
    s = np.concatenate([sin, sin]).astype(np.float64)
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * c + rot * s


def attention(q0, k0, v, pos, n, ck, cv, f_ck, f_cv, f_out, cos, sin, T, H, KV, HD):
    """LlmAttentionNode.reference (llm_nodes.py:923-955); ck / cv logical [C][KV HD] values, in place."""
    C = ck.shape[0]
    q0 = np.asarray(q0, np.float64).reshape(T, H, HD)
    k0 = np.asarray(k0, np.float64).reshape(T, KV, HD)
    v = np.asarray(v, np.float64).reshape(T, KV * HD)
    n = max(0, min(n, T, C - pos))
    grp = np.arange(H) // (H // KV)
    scale = 1.0 / math.sqrt(HD)
    out = np.zeros((T, H, HD))
    for t in range(n):
        p = pos + t
        kr = rope(k0[t], cos[p], sin[p]).reshape(-1)
        ck[p] = quantize_exp(kr, f_ck)
        cv[p] = quantize_exp(v[t], f_cv)
    for t in range(n):
        p = pos + t
        qr = rope(q0[t], cos[p], sin[p])
        K = ck[:p + 1].reshape(p + 1, KV, HD)
        V = cv[:p + 1].reshape(p + 1, KV, HD)
        for h in range(H):
            g = grp[h]
            s = dot8(qr[h][None, :] * K[:, g]) * scale
            e = libm("exp", s - s.max())
            pr = e / np.cumsum(e)[-1]
            out[t, h] = np.cumsum(pr[:, None] * V[:, g], axis=0)[-1]
    return quantize_exp(out.reshape(T, -1), np.asarray(f_out)[None, :])


def embed(ids, table, scale, f_out, res32):
    """LlmEmbedNode.reference (llm_nodes.py:549-570) without image rows."""
    tab = np.asarray(table, np.float32)
    k = np.clip(np.asarray(ids, np.float64).reshape(-1).astype(np.int64), 0, tab.shape[0] - 1)
    if scale != 1.0:
        out = (tab[k] * np.float32(scale)).astype(np.float64)
    else:
        out = tab[k].astype(np.float64)
    if res32:
        f = np.asarray(f_out, np.float64)
        raw = np.clip(np.rint(out * np.power(2.0, f)), -2147483648.0, 2147483647.0) + 0.0
        out = raw / np.power(2.0, f)
    return out
