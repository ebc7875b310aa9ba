"""The reference simulator's quantisation residuals restated with numpy float64: the statistics
(inference-scheduler/src/codegen/_simulate.py:77-118 ``_residual_stats``), the pooling unit's
full-precision result (``_pool2d_ref`` :273-364 with ``_pool_poly_sqrt`` :229-270, a loop over
output positions and taps as there) and the VectorOP branch's full value (:721-765).

TEST INFRASTRUCTURE ONLY: oracle/graph_sim.py's ``errors_out`` and the tests; nothing here
imports the product.
"""
import math

import numpy as np

from oracle.sim_ref import act_values

POOL_MAX, POOL_AVG = 0, 1
Q_MIN, Q_MAX = -128.0, 127.99609375


def residual_stats(full, quant, eps=1e-12):
    """(abs_max, nrmse, sqnr_db) of r = full - quant: max |r|, ||r||_2 / ||full||_2,
    20 log10(||full|| / ||r||); a zero ``full`` gives (m, 0, inf) with r = 0, else (m, inf, -inf)."""
    full = np.asarray(full, np.float64).reshape(-1)
    r = full - np.asarray(quant, np.float64).reshape(-1)
    abs_max = float(np.abs(r).max()) if r.size else 0.0
    norm_r = float(np.sqrt(np.dot(r, r)))
    norm_w = float(np.sqrt(np.dot(full, full)))
    if norm_w <= eps:
        return (abs_max, 0.0, math.inf) if norm_r <= eps else (abs_max, math.inf, -math.inf)
    return abs_max, norm_r / norm_w, (math.inf if norm_r <= eps else 20.0 * math.log10(norm_w / norm_r))


def truncate(x):
    """dtype.py:371-377: saturate, floor at 2^-8."""
    return np.floor(np.clip(np.asarray(x, np.float64), Q_MIN, Q_MAX) * 256.0) / 256.0


def truncate_div(x):
    """dtype.py:379-383: saturate, round toward zero at 2^-8."""
    return np.trunc(np.clip(np.asarray(x, np.float64), Q_MIN, Q_MAX) * 256.0) / 256.0


def host_quantize(x):
    """dtype.py:214-219: NaN to 0, saturate, round half to even at 2^-8."""
    x = np.asarray(x, np.float64)
    return np.round(np.clip(np.where(np.isnan(x), 0.0, x), Q_MIN, Q_MAX) * 256.0) / 256.0


def _floor_at(v, frac_bits):
    return np.floor(v * float(1 << frac_bits)) / float(1 << frac_bits)


def poly_sqrt(acc):
    """The pooling unit's square root: acc = m 4^k, m in [1, 4) floored at 2^-16, the cubic
    0.4434 + 0.6432 m - 0.0943 m^2 + 0.0077 m^3 (coefficients floored at 2^-15) by Horner with
    each step floored at 2^-20, times 2^k, floored at 2^-16; 0 for acc <= 0."""
    acc = np.asarray(acc, np.float64)
    out = np.zeros_like(acc)
    for idx in zip(*np.nonzero(acc > 0.0)):
        a = float(acc[idx])
        mant, e = math.frexp(a)                # a = mant 2^e, mant in [0.5, 1)
        k = e // 2
        m = mant * 2.0 ** (e - 2 * k)
        if m < 1.0:
            m, k = m * 4.0, k - 1
        m = _floor_at(m, 16)
        c0, c1, c2, c3 = (_floor_at(c, 15) for c in (0.4434, 0.6432, -0.0943, 0.0077))
        t = _floor_at(c3 * m + c2, 20)
        t = _floor_at(t * m + c1, 20)
        t = _floor_at(t * m + c0, 20)
        out[idx] = _floor_at(math.ldexp(t, k), 16)
    return out


def pool_full(x, ph, pw, sh, sw, pt, pl, dh, dw, oh, ow, pool_type, lp_order, count_include_pad):
    """_pool2d_ref: per output position, the taps inside the input; max, or the sum times
    round(2^23 / d) / 2^23 with d the window (count_include_pad) or the taps inside (at least 1),
    or sum |x| (LP1), or poly_sqrt(sum x^2) (LP2)."""
    x = np.asarray(x, np.float64)
    N, C, H, W = x.shape
    y = np.zeros((N, C, oh, ow))
    for r in range(oh):
        for c in range(ow):
            taps = [(r * sh + a * dh - pt, c * sw + b * dw - pl) for a in range(ph) for b in range(pw)]
            taps = [(i, j) for i, j in taps if 0 <= i < H and 0 <= j < W]
            if pool_type == POOL_MAX:
                acc = np.full((N, C), -np.inf)
                for i, j in taps:
                    acc = np.maximum(acc, x[:, :, i, j])
                y[:, :, r, c] = acc
                continue
            acc = np.zeros((N, C))
            for i, j in taps:
                v = x[:, :, i, j]
                acc = acc + (v if pool_type == POOL_AVG else (np.abs(v) if lp_order == 1 else v * v))
            if pool_type == POOL_AVG:
                d = max(ph * pw if count_include_pad else len(taps), 1)
                y[:, :, r, c] = acc * ((((1 << 23) + d // 2) // d) / float(1 << 23))
            else:
                y[:, :, r, c] = acc if lp_order == 1 else poly_sqrt(np.maximum(acc, 0.0))
    return y


_ACT_OF_OP = {4: 1, 5: 2, 6: 3, 7: 4, 8: 5, 9: 6}


def vectorop_full(op, act, alpha, a, b):
    """(full, quantise) of a VectorOP node on numpy-broadcast operand values: the op (DIV rounds
    toward zero), the fused RELU / RELU6 clamp, or for an activation of the unit its double value
    on the truncated op result, quantised to nearest."""
    q = truncate
    if op == 0:
        res = a + b
    elif op == 1:
        res = a - b
    elif op == 2:
        res = a * b
    elif op == 3:
        with np.errstate(divide="ignore", invalid="ignore"):
            res = a / b
        q = truncate_div
    elif op == 4:
        res = np.maximum(a, 0.0)
    elif op == 5:
        res = np.minimum(np.maximum(a, 0.0), 6.0)
    elif op in (6, 7, 8, 9):
        res = a
    else:
        raise ValueError(f"op_code {op}")
    act = _ACT_OF_OP[op] if op in (6, 7, 8, 9) else act
    if act == 1:
        res = np.maximum(res, 0.0)
    elif act == 2:
        res = np.minimum(np.maximum(res, 0.0), 6.0)
    elif act >= 3:
        return act_values(act, q(res), alpha), host_quantize
    return res, q
