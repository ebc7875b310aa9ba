"""Per-node quantisation residuals on the device: the reference simulator's optional side output
``errors_out`` (inference-scheduler/src/codegen/_simulate.py:77-118 ``_residual_stats``, the
``_store_quant`` calls of :594-602, :620-765 and ``_matmul_exp`` :814-835).

For each kernel-bearing node (MatMul on either engine, a Conv without exponents, Pool, VectorOP)
the node's full-precision result is computed in float64 on the GPU from the same operand values
the HIP unit read, and compared with the value the unit wrote.  The full values are exact where
the reference's are (products of on-grid operands and their sums stay far inside 53 bits; the
pooling divide and the LP square root are the kernel's own fixed-point steps, exact in float64);
only DIV's quotient and the activation unit's transcendental functions round, as they do in the
reference's float64 numpy.  This is a report, not the hot path: the quantised values the graph
carries on are always the HIP units' outputs.
"""
from __future__ import annotations

import math
from collections import namedtuple
from typing import Optional

import torch

from . import units

ResidualStats = namedtuple("ResidualStats", ("abs_max", "nrmse", "sqnr_db"))

Q_MIN, Q_MAX = -128.0, 127.99609375             # ap_fixed<16,8>'s value range
_ACT_OF_OP = {units.OP_RELU: units.ACT_RELU, units.OP_RELU6: units.ACT_RELU6,
              6: units.ACT_LEAKY_RELU, 7: units.ACT_SILU, 8: units.ACT_GELU, 9: units.ACT_GELU_TANH}


def residual_stats(full: torch.Tensor, quant: torch.Tensor, eps: float = 1e-12) -> ResidualStats:
    """Summary of r = full - quant (_simulate.py:77-118): max |r|, ||r|| / ||full|| and
    20 log10(||full|| / ||r||).  An (almost) all-zero ``full`` gives (abs_max, 0, inf) when r is
    zero too, else (abs_max, inf, -inf)."""
    full = full.to(torch.float64).reshape(-1)
    r = full - quant.to(torch.float64).reshape(-1)
    abs_max = float(r.abs().max()) if r.numel() else 0.0
    norm_r = float(torch.linalg.vector_norm(r))
    norm_w = float(torch.linalg.vector_norm(full))
    if norm_w <= eps:
        return ResidualStats(abs_max, 0.0, math.inf) if norm_r <= eps else ResidualStats(abs_max, math.inf, -math.inf)
    sqnr = math.inf if norm_r <= eps else 20.0 * math.log10(norm_w / norm_r)
    return ResidualStats(abs_max, norm_r / norm_w, sqnr)


def truncate(x: torch.Tensor) -> torch.Tensor:
    """ApFixed.truncate (dtype.py:371-377): saturate, then floor at 2^-8."""
    return torch.floor(torch.clamp(x, Q_MIN, Q_MAX) * 256.0) / 256.0


def truncate_div(x: torch.Tensor) -> torch.Tensor:
    """ApFixed.truncate_div (dtype.py:379-383): saturate, then round toward zero at 2^-8."""
    return torch.trunc(torch.clamp(x, Q_MIN, Q_MAX) * 256.0) / 256.0


def conv_full(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], sh: int, sw: int, pt: int, pl: int,
              dh: int, dw: int, oh: int, ow: int, depthwise: bool) -> torch.Tensor:
    """The exact convolution of float64 values x [N][C][H][W] and w [M][C or 1][kh][kw] plus the
    bias (the reference's _conv2d_ref / _depthwise_conv2d_ref): one product per tap over the
    zero-padded input, summed in float64 (exact for on-grid operands)."""
    N, C, H, W = x.shape
    M, _, kh, kw = w.shape
    need_h = (oh - 1) * sh + (kh - 1) * dh + 1
    need_w = (ow - 1) * sw + (kw - 1) * dw + 1
    xp = x.new_zeros((N, C, max(need_h, pt + H), max(need_w, pl + W)))
    xp[:, :, pt:pt + H, pl:pl + W] = x
    y = x.new_zeros((N, M, oh, ow))
    for a in range(kh):
        for b in range(kw):
            xs = xp[:, :, a * dh:a * dh + (oh - 1) * sh + 1:sh, b * dw:b * dw + (ow - 1) * sw + 1:sw]
            if depthwise:
                y += xs * w[:, 0, a, b].reshape(1, -1, 1, 1)
            else:
                y += torch.matmul(w[:, :, a, b].contiguous(), xs.reshape(N, C, oh * ow)).reshape(N, M, oh, ow)
    if bias is not None:
        y += bias.reshape(1, -1, 1, 1)
    return y


def _trn(v: torch.Tensor, frac_bits: int) -> torch.Tensor:
    s = float(1 << frac_bits)
    return torch.floor(v * s) / s


def _trn_const(v: float, frac_bits: int) -> float:
    s = float(1 << frac_bits)
    return math.floor(v * s) / s


def poly_sqrt(acc: torch.Tensor) -> torch.Tensor:
    """The pooling unit's square root (the reference's _pool_poly_sqrt, _simulate.py:229-270):
    acc = m 4^k with m in [1, 4) held at 2^-16, a cubic in m with coefficients at 2^-15 and
    every Horner step floored at 2^-20, scaled by 2^k and floored at 2^-16; 0 where acc <= 0."""
    out = torch.zeros_like(acc)
    pos = acc > 0.0
    a = acc[pos]
    if a.numel() == 0:
        return out
    m, e = torch.frexp(a)                      # a = m 2^e, m in [0.5, 1)
    e = e.to(torch.int64)
    k = torch.div(e, 2, rounding_mode="floor")
    m = m * torch.exp2((e - 2 * k).to(torch.float64))
    bump = m < 1.0
    m = torch.where(bump, m * 4.0, m)
    k = torch.where(bump, k - 1, k)
    m = _trn(m, 16)
    c0, c1, c2, c3 = (_trn_const(c, 15) for c in (0.4434, 0.6432, -0.0943, 0.0077))
    t1 = _trn(c3 * m + c2, 20)
    t2 = _trn(t1 * m + c1, 20)
    s = _trn(t2 * m + c0, 20)
    out[pos] = _trn(s * torch.exp2(k.to(torch.float64)), 16)
    return out


def pool_full(x: torch.Tensor, ph: int, pw: int, sh: int, sw: int, pt: int, pl: int, dh: int, dw: int,
              oh: int, ow: int, pool_type: int, lp_order: int, count_include_pad: int) -> torch.Tensor:
    """The pooling unit's result before the store's floor (the reference's _pool2d_ref,
    _simulate.py:273-364): max of the taps inside the input; the sum times the divisor's
    reciprocal raw = round(2^23 / d) / 2^23 (d = the window, or the taps inside it); LP1 the sum
    of |x|, LP2 poly_sqrt of the sum of squares."""
    N, C, H, W = x.shape
    dev = x.device
    rows = torch.arange(oh, device=dev) * sh - pt
    cols = torch.arange(ow, device=dev) * sw - pl
    acc = (torch.full((N, C, oh, ow), -math.inf, dtype=torch.float64, device=dev) if pool_type == units.POOL_MAX
           else torch.zeros((N, C, oh, ow), dtype=torch.float64, device=dev))
    count = torch.zeros((oh, ow), dtype=torch.int64, device=dev)
    for a in range(ph):
        r = rows + a * dh
        r_in = (r >= 0) & (r < H)
        rc = r.clamp(0, H - 1)
        for b in range(pw):
            c = cols + b * dw
            valid = r_in[:, None] & ((c >= 0) & (c < W))[None, :]
            v = x[:, :, rc][:, :, :, c.clamp(0, W - 1)]
            if pool_type == units.POOL_MAX:
                acc = torch.where(valid, torch.maximum(acc, v), acc)
            elif pool_type == units.POOL_AVG:
                acc = acc + torch.where(valid, v, torch.zeros_like(v))
            else:
                t = v.abs() if lp_order == 1 else v * v
                acc = acc + torch.where(valid, t, torch.zeros_like(t))
            count += valid
    if pool_type == units.POOL_MAX:
        return acc
    if pool_type == units.POOL_AVG:
        d = torch.full_like(count, ph * pw) if count_include_pad else count.clamp(min=1)
        inv = (((1 << 23) + d // 2) // d).to(torch.float64) / float(1 << 23)
        return acc * inv
    return acc if lp_order == 1 else poly_sqrt(acc.clamp(min=0.0))


def act_values(act: int, x: torch.Tensor, alpha: int = 0) -> torch.Tensor:
    """The activation unit's unrounded result in double (vectorop_act.py:60-73)."""
    if act == units.ACT_LEAKY_RELU:
        return torch.where(x >= 0.0, x, x * ((alpha & 0xFFFF) / 65536.0))
    if act == units.ACT_SILU:
        return x / (1.0 + torch.exp(-x))
    if act == units.ACT_GELU:
        return x * (0.5 * (1.0 + torch.erf(x / math.sqrt(2.0))))
    if act == units.ACT_GELU_TANH:
        return x * (0.5 * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * (x * x * x)))))
    raise ValueError(f"act {act} is not an activation of the unit")


def vectorop_full(op: int, act: int, alpha: int, a: torch.Tensor, b: Optional[torch.Tensor]):
    """(full, rounding) of a VectorOP node (_simulate.py:721-765): the float64 op result on the
    broadcast operands, its fused RELU / RELU6 clamp; for an activation of the unit, the
    activation of the truncated op result with round-to-nearest as the rounding."""
    rnd = "floor"
    if op == units.OP_ADD:
        res = a + b
    elif op == units.OP_SUB:
        res = a - b
    elif op == units.OP_MUL:
        res = a * b
    elif op == units.OP_DIV:
        res, rnd = a / b, "trunc"
    elif op == units.OP_RELU:
        res = torch.clamp(a, min=0.0)
    elif op == units.OP_RELU6:
        res = torch.clamp(a, 0.0, 6.0)
    elif op in (6, 7, 8, 9):
        res = a
    else:
        raise ValueError(f"VectorOP op_code {op} has no residual model")
    act = _ACT_OF_OP.get(op, act) if op in (6, 7, 8, 9) else act
    if act == units.ACT_RELU:
        res = torch.clamp(res, min=0.0)
    elif act == units.ACT_RELU6:
        res = torch.clamp(res, 0.0, 6.0)
    elif act >= units.ACT_LEAKY_RELU:
        return act_values(act, truncate_div(res) if rnd == "trunc" else truncate(res), alpha), "nearest"
    return res, rnd


__all__ = ["ResidualStats", "residual_stats", "truncate", "truncate_div", "conv_full", "poly_sqrt", "pool_full",
           "act_values", "vectorop_full"]
