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

import json
from typing import Dict, Iterable

import numpy as np

from .dtype import I16_HI, I16_LO, ApFixed16
from .graph import ConvNode, MatmulConvNode, MatmulNode, SchedulerError, TensorInfo


class NumericError(SchedulerError):
    """Inconsistent exponent metadata (numeric.py NumericError)."""


# ---------------------------------------------------------------- the axi.numeric annotations
# A model's numerics beyond the element type, the JSON object the reference reads from the
# ONNX metadata key "axi.numeric" (numeric.py:1-60): per-tensor or per-channel exponents
# (exp), per-channel Conv exponents (chexp), host-memory kinds (host), persistent states
# (state), group-major cache layouts (layout), the harness's fill of integer inputs
# (test_fill), int32 / float32 device kinds (dma) and MatMul engine pins (engine).
METADATA_KEY = "axi.numeric"
HOST_KINDS = ("f32", "i32", "i16")
DMA_KINDS = ("i32", "f32")
_SECTIONS = ("exp", "chexp", "host", "state", "test_fill", "layout", "dma", "engine")


def empty() -> dict:
    return {"exp": {}, "chexp": {}, "host": {}, "state": [], "test_fill": {}, "layout": {}, "dma": {}, "engine": {}}


def parse(text_or_dict) -> dict:
    """The annotations from their JSON text (or an already decoded dict); unknown sections are
    an error, missing ones empty (numeric.py:84-97, here without the ONNX container)."""
    d = json.loads(text_or_dict) if isinstance(text_or_dict, (str, bytes)) else dict(text_or_dict)
    unknown = set(d) - set(_SECTIONS) - {"version", "note"}
    if unknown:
        raise NumericError(f"{METADATA_KEY}: sections {sorted(unknown)} are not known")
    meta = empty()
    for k in _SECTIONS:
        if k in d:
            meta[k] = d[k]
    return meta


def to_metadata(meta: dict) -> str:
    """The JSON text of the annotations: version 1 and the non-empty sections (numeric.py:100-106)."""
    out = {"version": 1}
    out.update({k: v for k, v in meta.items() if v})
    return json.dumps(out, separators=(",", ":"))


def is_active(meta: dict) -> bool:
    return any(meta.get(k) for k in ("exp", "chexp", "host", "state", "dma"))


def _named(tensors: dict, name: str, section: str) -> TensorInfo:
    t = tensors.get(name)
    if t is None:
        raise NumericError(f"{METADATA_KEY}.{section}: no tensor '{name}' in the graph")
    return t


def apply(tensors: Dict[str, TensorInfo], meta: dict, dtype: ApFixed16) -> None:
    """Put the annotations on the tensors {name: TensorInfo} (numeric.py:113-193): host kinds
    (f32 -> float32 values, i32 -> host integers, i16 -> raw int16 at its exponent), int32 /
    float32 device kinds, exponents (an int or one per channel of the last axis, -30 .. 40),
    per-channel Conv exponents (4-D tensors without exp), states (their data the initial
    value), group-major layouts of 2-D states.  The element type must be 16-bit fixed point."""
    if is_active(meta) and getattr(dtype, "W", 0) != 16:
        raise NumericError(f"{METADATA_KEY} needs a 16-bit fixed-point element type")
    for name, kind in meta.get("host", {}).items():
        t = _named(tensors, name, "host")
        if kind not in HOST_KINDS:
            raise NumericError(f"host tensor '{name}': kind {kind!r} is none of {HOST_KINDS}")
        t.host = kind
        t.kind = {"f32": "f32", "i32": "host", "i16": "i16"}[kind]
    for name, kind in meta.get("dma", {}).items():
        t = _named(tensors, name, "dma")
        if kind not in DMA_KINDS:
            raise NumericError(f"device tensor '{name}': kind {kind!r} is none of {DMA_KINDS}")
        if t.host is not None:
            raise NumericError(f"tensor '{name}' has both a host and a device kind")
        t.kind = kind
    for name, e in meta.get("exp", {}).items():
        t = _named(tensors, name, "exp")
        if t.host in ("f32", "i32"):
            raise NumericError(f"tensor '{name}': a {t.host} host tensor takes no exponent")
        arr = np.asarray(e, np.int64)
        last = int(t.shape[-1]) if len(t.shape) else 1
        if arr.ndim > 1 or (arr.ndim == 1 and arr.size != last):
            raise NumericError(f"tensor '{name}': one exponent, or one per channel of the last axis ({last})")
        if (arr < -30).any() or (arr > 40).any():
            raise NumericError(f"tensor '{name}': exponent outside -30 .. 40")
        t.exp = arr.copy() if arr.ndim else int(arr)
    for name, e in meta.get("chexp", {}).items():
        t = _named(tensors, name, "chexp")
        arr = np.asarray(e, np.int64)
        if len(t.shape) != 4 or arr.ndim != 1 or arr.size != t.shape[1] or t.exp is not None or t.host:
            raise NumericError(f"tensor '{name}': chexp is one exponent per channel of a 4-D device tensor "
                               f"without exp")
        if (arr < -30).any() or (arr > 40).any():
            raise NumericError(f"tensor '{name}': exponent outside -30 .. 40")
        t.chexp = arr.copy()
    for name in meta.get("state", []):
        _named(tensors, name, "state").state = True
    for name in meta.get("test_fill", {}):
        _named(tensors, name, "test_fill")
    for name, e in meta.get("engine", {}).items():
        _named(tensors, name, "engine")
        if e not in ("conv", "matmul"):
            raise NumericError(f"engine of '{name}': \"conv\" or \"matmul\", not {e!r}")
    for name, gd in meta.get("layout", {}).items():
        t = _named(tensors, name, "layout")
        if len(gd) not in (2, 3):
            raise NumericError(f"layout of '{name}': [G, D] (or [G, D, K])")
        g, d = int(gd[0]), int(gd[1])
        if len(gd) == 3 and int(gd[2]) != 1:
            raise NumericError(f"layout of '{name}': interleaved V images (K > 1) are not supported")
        if not t.state or len(t.shape) != 2 or t.shape[1] != g * d or g < 1 or d < 1:
            raise NumericError(f"layout of '{name}': a group-major [G][R][D] layout takes a 2-D state [R][G D]")
        t.group_layout = (g, d)


def lower_engines(nodes: list, meta: dict) -> int:
    """MatMuls the annotations pin to the conv unit (engine "conv") become MatmulConvNodes, in
    place (matmul_lowering.py; kw 1, one output row).  Returns the count."""
    pins = meta.get("engine", {})
    n = 0
    for i, sn in enumerate(nodes):
        if isinstance(sn, MatmulNode) and pins.get(sn.output.onnx_name) == "conv":
            nodes[i] = MatmulConvNode(list(sn.inputs), sn.output)
            n += 1
    return n


def check(nodes: Iterable, dtype: ApFixed16) -> None:
    """Which nodes may touch annotated tensors (numeric.py:310-379): host tensors and states only
    the host / LLM ops and the row-ops and attention nodes that own them; per-channel Conv
    exponents only Convs; power-of-two exponents MatMuls (constant B), Convs (per-tensor
    exponents, constant weight and bias), copies that carry one exponent through (Transpose,
    Permute, Reshape with equal exponents), and the LLM-side nodes."""
    from .graph import (AttentionNode, AttnContractNode, KvWriteNode, LlmAttnConvNode, PermuteNode, ReshapeNode,
                        RowOpsNode, SoftmaxVopNode)
    from .host_ops import HostNode, LlmEmbedNode
    from .rowops_nodes import RoCallNode, RowOpsAdapter, TransposeRoNode
    llm = (HostNode, LlmEmbedNode, RowOpsAdapter, RoCallNode, RowOpsNode, LlmAttnConvNode, AttnContractNode,
           AttentionNode, KvWriteNode, SoftmaxVopNode)
    F = dtype.frac_bits
    for sn in nodes:
        label = f"{type(sn).__name__} '{sn.output.onnx_name}'"
        ts = [t for t in list(sn.inputs) + [sn.output] if t is not None]
        if isinstance(sn, llm) and not isinstance(sn, TransposeRoNode):
            continue
        if any(t.host is not None or t.kind == "host" or t.state for t in ts):
            raise NumericError(f"{label}: host tensors and states are read and written by the LLM ops only")
        if any(t.chexp is not None for t in ts) and not isinstance(sn, ConvNode):
            raise NumericError(f"{label}: per-channel Conv exponents are read and written by Convs only")
        if isinstance(sn, (MatmulNode, MatmulConvNode)):
            b = sn.inputs[1]
            if any(t.exp is not None for t in ts) and b.data is None and b.exp is None:
                raise NumericError(f"{label}: exponents with a runtime B that carries none")
            continue
        if isinstance(sn, ConvNode):
            x, w = sn.inputs[0], sn.inputs[1]
            bias = sn.inputs[2] if sn.has_bias else None
            if w.exp is not None or (bias is not None and bias.exp is not None):
                raise NumericError(f"{label}: weight and bias exponents are derived (f_w = f_y + {F} - f_x, the "
                                   f"bias at f_y), not annotated")
            scaled = any(t.exp is not None or t.chexp is not None for t in (x, sn.output))
            if scaled and (w.data is None or (bias is not None and bias.data is None)):
                raise NumericError(f"{label}: exponents need a constant weight and bias")
            for t in (x, sn.output):
                if t.exp is not None and np.ndim(t.exp) != 0:
                    raise NumericError(f"{label}: '{t.onnx_name}' takes one exponent (a Conv's channel axis is "
                                       f"not the last)")
            continue
        if isinstance(sn, (TransposeRoNode, PermuteNode)) and any(t.exp is not None for t in ts):
            es = {None if t.exp is None or np.ndim(t.exp) else int(np.asarray(t.exp)) for t in ts}
            if len(es) != 1 or None in es:
                raise NumericError(f"{label}: a copy's input and output carry one and the same exponent")
            continue
        if isinstance(sn, ReshapeNode):
            src, out = sn.inputs[0], sn.output
            if src.exp is not None or out.exp is not None:
                scalar = np.ndim(src.exp) == 0 and np.ndim(out.exp) == 0 and np.array_equal(
                    np.asarray(F if src.exp is None else src.exp), np.asarray(F if out.exp is None else out.exp))
                same_last = (len(src.shape) and len(out.shape) and src.shape[-1] == out.shape[-1]
                             and np.array_equal(src.exp_full(F), out.exp_full(F)))
                if not (scalar or same_last):
                    raise NumericError(f"{label}: '{src.onnx_name}' and '{out.onnx_name}' carry different exponents")
            continue
        if any(t.exp is not None for t in ts):
            raise NumericError(f"{label}: power-of-two exponents are taken by MatMuls, Convs, copies and the LLM "
                               f"ops only")


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
