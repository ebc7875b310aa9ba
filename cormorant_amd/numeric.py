"""Weight encoding of the power-of-two numerics (inference-scheduler/src/numeric.py:199-307).

A MatMul or Conv whose activations carry power-of-two exponents reads its constant weight at
the exponent that puts every product on the output's accumulator grid: the kernels sum raw
int16 products exactly and write floor(acc / 2^F), so

    MatMul: f_w[i][j] = f_out[j] + F - f_in[i]                 (rank-1, per element)
    Conv:   f_w = f_y + F - f_x, per (out, in) channel pair    (depthwise: per channel)
            with the bias at f_y (the kernel seeds the accumulator with bias << F).

The weight is rounded half to even at its exponent and saturated to int16; ``data`` then
holds raw / 2^F (so the packers emit the raw lanes unchanged) and ``wexp`` the exponent.
Both functions mutate the graph's weight tensors in place and return
{tensor name: number of saturated elements}, as the reference's do.
"""
from __future__ import annotations

from typing import Dict, Iterable

import numpy as np

from .dtype import I16_HI, I16_LO, ApFixed16
from .graph import ConvNode, MatmulNode, TensorInfo


class NumericError(ValueError):
    """Inconsistent exponent metadata (numeric.py NumericError)."""


def _channels(t: TensorInfo, F: int, n: int) -> np.ndarray:
    e = np.asarray(F if t.exp is None else t.exp, np.int64).reshape(-1)
    if e.size == 1:
        return np.full(n, int(e[0]), np.int64)
    if e.size != n:
        raise NumericError(f"tensor '{t.onnx_name}': {e.size} exponents for {n} channels")
    return e


def _encode(data: np.ndarray, f: np.ndarray, F: int):
    """raw / 2^F (float32) of data rounded half to even at 2^-f and saturated; the count."""
    # scaling by 2^f is exact (ldexp), so this is round(data * 2^f) without the power array
    r = np.rint(np.ldexp(np.asarray(data, np.float64), np.asarray(f, np.int64)))
    n_sat = int(((r < I16_LO) | (r > I16_HI)).sum())
    return (np.clip(r, I16_LO, I16_HI) / float(1 << F)).astype(np.float32), n_sat


def encode_matmul_weights(nodes: Iterable, dtype: ApFixed16) -> Dict[str, int]:
    """Encode the constant B of every MatMul whose A, B or C has an exponent at the rank-1
    weight exponent (numeric.py:199-255).  A weight shared by MatMuls must see one exponent."""
    F = dtype.frac_bits
    done: Dict[str, np.ndarray] = {}
    sat: Dict[str, int] = {}
    for sn in nodes:
        if not isinstance(sn, MatmulNode):
            continue
        a, b = sn.inputs
        c = sn.output
        if a.exp is None and c.exp is None and b.exp is None:
            continue
        if b.data is None:
            raise NumericError(f"MatMul '{c.onnx_name}': exponents with a runtime B ('{b.onnx_name}')")
        if b.exp is not None:
            raise NumericError(f"weight '{b.onnx_name}': weight exponents are derived "
                               f"(f_w = f_out + {F} - f_in), not annotated")
        k, m = int(b.shape[-2]), int(b.shape[-1])
        wexp = np.add.outer(F - _channels(a, F, k), _channels(c, F, m))        # [K][M]
        if b.onnx_name in done:
            if not np.array_equal(done[b.onnx_name], wexp):
                raise NumericError(f"weight '{b.onnx_name}' read by MatMuls with different exponents")
            continue
        lo, hi = int(wexp.min()), int(wexp.max())
        etype = next(t for t in (np.int8, np.int16, np.int32, np.int64)
                     if np.iinfo(t).min <= lo and hi <= np.iinfo(t).max)
        w = np.asarray(b.data, np.float64).reshape(-1, k, m)
        data, n_sat = _encode(w, wexp[None], F)
        sat[b.onnx_name] = n_sat
        b.data = data.reshape(np.shape(b.data))
        b.wexp = wexp.astype(etype)
        done[b.onnx_name] = wexp
    return sat


def encode_conv_weights(nodes: Iterable, dtype: ApFixed16) -> Dict[str, int]:
    """Encode the weight and bias of every Conv whose input or output has an exponent
    (numeric.py:258-307): per-tensor f_w = f_y + F - f_x, or with per-channel exponents
    (chexp, axis 1) f_w[m][c] = f_y[m] + F - f_x[c] (depthwise f_w[m] = f_y[m] + F - f_x[m]);
    the bias at f_y."""
    F = dtype.frac_bits
    sat: Dict[str, int] = {}
    done: Dict[str, np.ndarray] = {}
    for sn in nodes:
        if not isinstance(sn, ConvNode):
            continue
        x, w, y = sn.inputs[0], sn.inputs[1], sn.output
        if x.exp is None and y.exp is None and x.chexp is None and y.chexp is None:
            continue
        if x.chexp is None and y.chexp is None:
            fx = int(np.asarray(F if x.exp is None else x.exp))
            fy = int(np.asarray(F if y.exp is None else y.exp))
            encoded = [(w, np.asarray(fy + F - fx, np.int64))]
            if sn.has_bias:
                encoded.append((sn.inputs[2], np.asarray(fy, np.int64)))
        else:
            fx = (np.asarray(x.chexp, np.int64) if x.chexp is not None
                  else np.full(sn.in_ch, F if x.exp is None else int(np.asarray(x.exp)), np.int64))
            fy = (np.asarray(y.chexp, np.int64) if y.chexp is not None
                  else np.full(sn.out_ch, F if y.exp is None else int(np.asarray(y.exp)), np.int64))
            fw = (fy + F - fx)[:, None] if sn.is_depthwise else np.add.outer(fy + F, -fx)
            encoded = [(w, fw.reshape(fw.shape + (1, 1)))]
            if sn.has_bias:
                encoded.append((sn.inputs[2], fy))
        for t, f in encoded:
            if t.onnx_name in done:
                if not np.array_equal(done[t.onnx_name], f):
                    raise NumericError(f"'{t.onnx_name}' read by Convs with different exponents")
                continue
            data, n_sat = _encode(np.asarray(t.data, np.float64).reshape(t.shape), f, F)
            sat[t.onnx_name] = n_sat
            t.data = data.reshape(np.shape(t.data))
            t.wexp = f.astype(np.int8) if (f.min() >= -128 and f.max() <= 127) else f
            done[t.onnx_name] = f
    return sat


__all__ = ["NumericError", "encode_matmul_weights", "encode_conv_weights"]
