"""The reference simulator's own CPU algorithms for the units whose cost it dominates, restated
for the ``cpu_sim_ref`` baseline: the row-ops norms with exact per-row sums in Python integers
(inference-scheduler/src/rowops_spec.py:240-284, ``layer_norm`` / ``rms_norm``: a loop over rows
with object-dtype sums, the rsqrt of ``rsqrt_bf`` :102-121 in Python integers) and the
activation unit through ``np.vectorize`` of glibc's erf / exp / tanh per element
(vectorop_act.py:60-79 with host_nodes.py:150-162 ``libm``, then DataType.host_quantize,
dtype.py:214-219).  The results equal the C oracle's bit for bit (tests/test_sim_ref.py); only
the cost differs.

TEST INFRASTRUCTURE ONLY: used by oracle/graph_sim.py's ``algo="ref"`` (the CPU baseline that
bench.py times) and by the tests; nothing here imports the product.
"""
import math
from functools import lru_cache

import numpy as np

from oracle.rowops_adapt import P1_BITS, beta_bits, norm_params

RM_BITS = 47


@lru_cache(maxsize=None)
def _rsqrt_table():
    """round(2^47 / sqrt((idx + 0.5) 2^19)) for the 13-bit index idx of Dm in [2^30, 2^32)."""
    idx = np.arange(8192, dtype=np.float64)
    with np.errstate(divide="ignore"):
        y = np.rint(2.0 ** RM_BITS / np.sqrt((idx + 0.5) * 2.0 ** 19))
    y[:2048] = 0
    return [int(v) for v in np.minimum(y, 2.0 ** 32 - 1)]


def _rsqrt(D: int):
    """(Rm, sh) with 1/sqrt(D) ~ Rm 2^-sh: the table on the leading 13 bits of D block-floated
    to an even exponent, one Newton step with every product truncated by its shift."""
    d = D.bit_length() - 32
    d += d & 1
    Dm = D >> d if d >= 0 else D << -d
    y0 = _rsqrt_table()[Dm >> 19]
    u = (((Dm * y0) >> 32) * y0) >> 32
    y1 = y0 + ((y0 * ((1 << 30) - u)) >> 31)
    return min(max(y1, 1 << 31), (1 << 32) - 1), RM_BITS + d // 2


def _rne(v: int, k: int) -> int:
    if k <= 0:
        return v << -k
    q = v >> k
    r = v - (q << k)
    h = 1 << (k - 1)
    return q + (1 if r > h or (r == h and q & 1) else 0)


def _shr(v: int, k: int) -> int:
    """floor(v / 2^k); k <= 0 shifts left."""
    return v >> k if k >= 0 else v << -k


def _sat16(v: int) -> int:
    return -32768 if v < -32768 else (32767 if v > 32767 else v)


def layer_norm(x_raw, f_x: int, gamma, beta, eps: float, f_out):
    """LayerNorm rows of the raw integers x_raw [rows][n] at 2^-f_x into int16 at 2^-f_out[c]:
    per row S1 = sum x, S2 = sum x^2, D = n S2 - S1^2 + E in Python integers, the rsqrt, and per
    element A = n x - S1, P1 = floor(A Rm / 2^(sh - 24)), y = rne((P1 G + Bq) / 2^(24 + g - f_out))."""
    x_raw = np.asarray(x_raw, np.int64)
    rows, n = x_raw.shape
    G, g, Bq, E = norm_params(gamma, n, eps, int(f_x), beta=beta)
    G = [int(v) for v in G]
    Bq = [0] * n if Bq is None else [int(v) for v in Bq]
    sh_c = [P1_BITS + g - int(f) for f in np.broadcast_to(np.asarray(f_out, np.int64), (n,))]
    out = np.empty((rows, n), np.int64)
    for r in range(rows):
        row = [int(v) for v in x_raw[r]]
        S1 = sum(row)
        S2 = sum(v * v for v in row)
        D = n * S2 - S1 * S1 + E
        Rm, sh = _rsqrt(max(D, 1))
        k = sh - P1_BITS
        out[r] = [_sat16(_rne(_shr((n * v - S1) * Rm, k) * G[c] + Bq[c], sh_c[c])) for c, v in enumerate(row)]
    return out


def rms_norm(h_raw, f_h: int, gamma, eps: float, f_out):
    """RMSNorm rows of h_raw [rows][n] at 2^-f_h: D = sum h^2 + E, P1 = floor(h Rm / 2^(sh - 24)),
    y = rne(P1 G / 2^(24 + g - f_out)) with gamma folded with sqrt(n) into G."""
    h_raw = np.asarray(h_raw, np.int64)
    rows, n = h_raw.shape
    G, g, _b, E = norm_params(gamma, n, eps, int(f_h), rms=True)
    G = [int(v) for v in G]
    sh_c = [P1_BITS + g - int(f) for f in np.broadcast_to(np.asarray(f_out, np.int64), (n,))]
    out = np.empty((rows, n), np.int64)
    for r in range(rows):
        row = [int(v) for v in h_raw[r]]
        Rm, sh = _rsqrt(sum(v * v for v in row) + E)
        k = sh - P1_BITS
        out[r] = [_sat16(_rne(_shr(v * Rm, k) * G[c], sh_c[c])) for c, v in enumerate(row)]
    return out


_LIBM = {name: np.vectorize(getattr(math, name), otypes=[np.float64]) for name in ("exp", "erf", "tanh")}
ACT_LEAKY, ACT_SILU, ACT_GELU, ACT_GELU_TANH = 3, 4, 5, 6


def act_values(act: int, x, alpha: int = 0):
    """The activation unit's unrounded double result of the values x, libm per element
    (vectorop_act.py:60-73)."""
    x = np.asarray(x, np.float64)
    if act == ACT_LEAKY:
        return np.where(x >= 0.0, x, x * ((alpha & 0xFFFF) / 65536.0))
    if act == ACT_SILU:
        return x / (1.0 + _LIBM["exp"](-x))
    if act == ACT_GELU:
        return x * (0.5 * (1.0 + _LIBM["erf"](x / math.sqrt(2.0))))
    if act == ACT_GELU_TANH:
        return x * (0.5 * (1.0 + _LIBM["tanh"](math.sqrt(2.0 / math.pi) * (x + 0.044715 * (x * x * x)))))
    raise ValueError(f"act {act} is not one of the activation unit's")


def act_unit(act: int, x_raw, alpha: int = 0):
    """The activation unit on Q8.8 raws: the double activation of x = raw / 2^8 with libm per
    element, then rounded half to even at 2^-8 and saturated (NaN to 0)."""
    v = np.nan_to_num(act_values(act, np.asarray(x_raw, np.float64) / 256.0, alpha), nan=0.0)
    return np.round(np.clip(v, -128.0, 127.99609375) * 256.0).astype(np.int64)


__all__ = ["layer_norm", "rms_norm", "act_values", "act_unit", "beta_bits"]
