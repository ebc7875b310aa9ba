"""The row-ops node adapters' reference() for the graph-level checker, independent of the product:
each adapter kind's job constants derived here from the node's declared fields (gamma, beta,
eps, bias, the tensors' exponents) by a restatement of the reference's specification functions
(inference-scheduler/src/rowops_spec.py: gamma_scale :124-129, beta_bits :132-143, bias_bits
:146-150, bias_exp :160-179, bias_params :182-191, norm_params :211-229), then the unit's
arithmetic from the C oracle's job (oracle/cm_oracle.c, pinned by the reference's row-ops
fixtures and its own row-ops oracle); RoPE through the restated rowops_spec.rope
(oracle/attn_prep.py).  TEST INFRASTRUCTURE ONLY.  Nothing here imports the product.
"""
import math

import numpy as np

from oracle import cm
from oracle.attn_prep import rope, rope_tables_raw

P1_BITS, BQ_BITS, SILU_BITS, G_BITS, N_MAX = 24, 20, 20, 14, 4096
OP_COPY, OP_ADDX, OP_DEQUANT, OP_MULACT, OP_NORM = 1, 2, 3, 4, 5
K_I16, K_I32, K_F32 = 0, 1, 2
F_B_EN, F_RELU, F_NORM_LN = 1 << 12, 1 << 15, 1 << 16


# ---------------------------------------------------------------- the specification's constants
def gamma_scale(g_real):
    """g with max |round(g_real 2^g)| < 2^31."""
    m = float(np.abs(np.asarray(g_real, np.float64)).max())
    return 0 if m == 0.0 else 30 - int(math.floor(math.log2(m)))


def beta_bits(beta):
    """beta's scale: 2^-20 while round(beta 2^bb) fits the int22, coarser by a bit per doubling."""
    if beta is None:
        return BQ_BITS
    m = float(np.abs(np.asarray(beta, np.float64)).max()) if np.size(beta) else 0.0
    bb = BQ_BITS
    while bb > 0 and abs(round(m * 2.0 ** bb)) >= (1 << 21):
        bb -= 1
    return bb


def bias_bits(bias, f):
    return min(int(f), beta_bits(bias))


def bias_exp(bias, f_x, f_out, extra=8):
    bias = np.asarray(bias, np.float64).reshape(-1)
    n = bias.size
    lo = np.maximum(np.broadcast_to(np.asarray(f_x, np.int64), (n,)), np.broadcast_to(np.asarray(f_out, np.int64), (n,)))
    fp = np.minimum(lo + extra, 24)
    for _ in range(64):
        over = np.abs(np.rint(bias * np.power(2.0, fp.astype(np.float64)))) > (1 << 21) - 1
        if not over.any():
            break
        fp = np.where(over, fp - 1, fp)
    if (fp < lo).any():
        raise ValueError("bias_exp: the bias does not fit the int22 at the output's grid")
    return fp


def bias_params(bias, f_x, f_out):
    fp = bias_exp(bias, f_x, f_out)
    n = fp.size
    bq = np.rint(np.asarray(bias, np.float64).reshape(-1) * np.power(2.0, fp.astype(np.float64))).astype(np.int64)
    return (bq, fp - np.broadcast_to(np.asarray(f_x, np.int64), (n,)),
            fp - np.broadcast_to(np.asarray(f_out, np.int64), (n,)))


def norm_params(gamma, n, eps, f_in, beta=None, rms=False):
    """(G [n], g, Bq [n] or None, E) of a norm job."""
    gamma = np.asarray(gamma, np.float64)
    gs = gamma * math.sqrt(n) if rms else gamma
    g = gamma_scale(gs)
    G = np.rint(gs * 2.0 ** g).astype(np.int64)
    if rms:
        return G, g, None, int(round(eps * n * 2.0 ** (2 * f_in)))
    E = int(round(eps * n * n * 2.0 ** (2 * f_in)))
    bb = beta_bits(beta)
    Bq = None if beta is None else (np.rint(np.asarray(beta, np.float64) * 2.0 ** bb).astype(np.int64)
                                    << (P1_BITS + g - bb))
    return G, g, Bq, E


# ---------------------------------------------------------------- one job through the C oracle
def _params(n, G=0, Bq=0, sa=0, sb=0, sc=0):
    """n per-column 16-byte entries: int32 G, int32 Bq' (int22), u8 shifts."""
    cols = [np.broadcast_to(np.asarray(v, np.int64), (n,)) for v in (G, Bq, sa, sb, sc)]
    p = np.zeros((n, 16), np.uint8)
    p[:, 0:4] = (cols[0] & 0xFFFFFFFF).astype("<u4").view(np.uint8).reshape(n, 4)
    p[:, 4:8] = (cols[1] & 0xFFFFFFFF).astype("<u4").view(np.uint8).reshape(n, 4)
    p[:, 8], p[:, 9], p[:, 10] = cols[2], cols[3], cols[4]
    return p.reshape(-1)


_NP = {K_I16: np.int16, K_I32: np.int32, K_F32: np.float32}


def _job(op, a, b, ak, bk, ck, p, eps=0, bq_sh=0):
    """One job over the rows of a [rows][n] (and b), each row at a 16-byte multiple stride."""
    rows, n = a.shape
    kb = lambda k: 2 if k == K_I16 else 4            # noqa: E731

    def img(x, k):
        s = (kb(k) * n + 15) & ~15
        out = np.zeros((rows, s), np.uint8)
        out[:, :kb(k) * n] = np.ascontiguousarray(x.astype(_NP[k])).view(np.uint8).reshape(rows, -1)
        return out.reshape(-1), s

    a_img, a_s = img(a, ak)
    b_img, b_s = img(b, bk) if b is not None else (None, 0)
    c_s = (kb(ck) * n + 15) & ~15
    c = np.zeros(rows * c_s, np.uint8)
    word = op | (ak << 4) | (bk << 6) | (ck << 8) | (F_B_EN if b is not None else 0)
    cm.rowops_reset_params()
    cm.rowops(a_img, b_img, c, p, word, n, rows, 1, a_s, 0, b_s, 0, c_s, 0, eps, 0, bq_sh)
    return c.reshape(rows, c_s)[:, :kb(ck) * n].copy().view(_NP[ck])


# ---------------------------------------------------------------- the adapters
def _chan(t, n, F=8):
    return np.broadcast_to(np.asarray(F if t.exp is None else t.exp, np.int64).reshape(-1), (n,)).copy()


def _raw(t, v, n):
    return np.rint(np.asarray(v, np.float64).reshape(-1, n) * np.power(2.0, _chan(t, n).astype(np.float64)))


def adapter(sn, ins, host_value=None):
    """The output values of row-ops adapter ``sn`` (by its class name) for input values ``ins``;
    ``host_value(tensor)`` gives a runtime position's value."""
    kind = type(sn).__name__
    x_t, y = sn.inputs[0], sn.output
    F = getattr(sn, "F", 8)
    W = int(x_t.shape[-1])
    fo = _chan(y, W, F)
    unit = lambda r: (r.astype(np.float64) / np.power(2.0, fo.astype(np.float64))).reshape(y.shape)   # noqa: E731
    if kind in ("LayerNormRoNode", "LayerNorm32RoNode"):
        fx = _chan(x_t, W, F)
        a = _raw(x_t, ins[0], W).astype(np.int64)
        gamma = np.ones(W) if sn.gamma is None else np.asarray(sn.gamma, np.float64).reshape(-1)
        beta = np.zeros(W) if sn.beta is None else np.asarray(sn.beta, np.float64).reshape(-1)
        G, g, _bq, E = norm_params(gamma, W, sn.eps, int(fx[0]), beta=beta)
        bb = beta_bits(beta)
        bqp = np.rint(beta * 2.0 ** bb).astype(np.int64)
        ak = K_I32 if x_t.kind == "i32" else K_I16
        r = _job(OP_NORM | F_NORM_LN, a, None, ak, K_I16, K_I16, _params(W, G, bqp, 0, 0, P1_BITS + g - fo), eps=E,
                 bq_sh=P1_BITS + g - bb)
        return unit(r)
    if kind == "RMSNormRoNode":
        gamma = np.asarray(sn.gamma, np.float64).reshape(-1)
        n = gamma.size
        fx = _chan(x_t, W, F)
        a = _raw(x_t, ins[0], W).astype(np.int64).reshape(-1, n)
        G, g, _b, E = norm_params(gamma, n, sn.eps, int(fx[0]), rms=True)
        r = _job(OP_NORM, a, None, K_I32, K_I16, K_I16, _params(n, G, 0, 0, 0, P1_BITS + g - fo[:n]), eps=E)
        return unit(r.reshape(-1, W))
    if kind in ("ResAddRoNode", "ResAddBiasRoNode"):
        d_t = sn.inputs[1]
        fr = int(fo[0])
        fa, fd = _chan(x_t, W, F), _chan(d_t, W, F)
        a = _raw(x_t, ins[0], W).astype(np.int64)
        d = _raw(d_t, ins[1], W).astype(np.int64)
        ak = K_I32 if x_t.kind == "i32" else K_I16
        if kind == "ResAddRoNode":
            r = _job(OP_ADDX, a, d, ak, K_I16, K_I32, _params(W, 0, 0, 0, fr - fd, 0))
        else:
            bias = np.asarray(sn.bias, np.float64).reshape(-1)
            bb = bias_bits(bias, fr)
            r = _job(OP_ADDX, a, d, ak, K_I16, K_I32, _params(W, 0, np.rint(bias * 2.0 ** bb).astype(np.int64),
                                                               fr - fa, fr - fd, 0), bq_sh=fr - bb)
        return unit(r)
    if kind == "WidenRoNode":
        fx = _chan(x_t, W, F)
        r = _job(OP_COPY, _raw(x_t, ins[0], W).astype(np.int64), None, K_I16, K_I16, K_I32,
                 _params(W, 0, 0, int(fo[0]) - fx, 0, 0))
        return unit(r)
    if kind == "SiluMulRoNode":
        u_t = sn.inputs[1]
        fg, fu = _chan(x_t, W, F), _chan(u_t, W, F)
        r = _job(OP_MULACT, _raw(x_t, ins[0], W).astype(np.int64), _raw(u_t, ins[1], W).astype(np.int64), K_I16,
                 K_I16, K_I16, _params(W, 0, 0, G_BITS - fg, 0, SILU_BITS + fu - fo))
        return unit(r)
    if kind == "DequantRoNode":
        # float32 of raw 2^-f per column: exact for int16 raws, rounded half to even for int32
        f = _chan(x_t, W, F)
        raw = _raw(x_t, ins[0], W)
        return (raw * np.power(2.0, -f.astype(np.float64))).astype(np.float32).astype(np.float64).reshape(y.shape)
    if kind == "BiasCopyRoNode":
        fx = _chan(x_t, W, F)
        bq, sa, sc = bias_params(np.asarray(sn.bias, np.float64).reshape(-1), fx, fo)
        r = _job(OP_COPY | (F_RELU if sn.relu else 0), _raw(x_t, ins[0], W).astype(np.int64), None, K_I16, K_I16,
                 K_I16, _params(W, 0, bq, sa, 0, sc))
        return unit(r)
    if kind == "RopeRoNode":
        nh, HD = sn.heads, sn.head_dim
        fx = _chan(x_t, W, F).reshape(nh, HD)
        xr = _raw(x_t, ins[0], W).astype(np.int64).reshape(-1, nh, HD)
        rows = xr.shape[0]
        pos = int(sn.pos) if sn.pos_t is None else int(host_value(sn.pos_t))
        cos = np.asarray(sn.cos, np.float32)
        sin = np.asarray(sn.sin, np.float32)
        cr, sr = rope_tables_raw(np.concatenate([cos, cos], 1).astype(np.float64),
                                 np.concatenate([sin, sin], 1).astype(np.float64))
        idx = np.full(rows, pos) if sn.same_pos else pos + np.arange(rows)
        yr = rope(xr, fx, cr[idx], sr[idx], fo.reshape(nh, HD))
        return unit(yr.reshape(-1, W))
    raise NotImplementedError(f"row-ops adapter {kind}")
