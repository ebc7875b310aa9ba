"""The reference's host ops: the nodes its boards run on the CPU (inference-scheduler/src/
host_nodes.py, llm_nodes.py), with the reference's per-node contract ``reference(ins, dtype)``
(float64 values in, float64 values out, states updated in place; _simulate.py:667-690).

The arithmetic is libcormo_host.so (include/cormorant_host.h): IEEE double with glibc's exp /
erf / tanh in the reference's operation order, written back with round half to even -- bit for
bit what the reference's Python (whose ``math`` module is the same glibc) computes.  The
simulator hands these nodes host copies of their inputs and puts the results back on the
device.

LlmEmbedNode is the one LLM op that moves data only; it runs on the GPU (cm_embed_rows).
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from .graph import KernelNode, SchedulerError, TensorInfo

HERE = os.path.dirname(os.path.abspath(__file__))
HOST_LIB_PATH = os.path.join(HERE, "libcormo_host.so")

_P = ctypes.c_void_p
_U64, _U32, _I32, _D = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_double


class CmhAttnArgs(ctypes.Structure):
    """cmh_attn_args of include/cormorant_host.h."""
    _fields_ = [("q0", _P), ("k0", _P), ("v", _P), ("ck", _P), ("cv", _P), ("f_ck", _P), ("f_cv", _P),
                ("cos", _P), ("sin", _P), ("out", _P), ("f_out", _P), ("scale", _D),
                ("T", _U32), ("H", _U32), ("KV", _U32), ("HD", _U32), ("C", _U32), ("pos", _U32),
                ("n", ctypes.c_int64)]


HOST_SIGNATURES = {
    "cmh_abi_version": (_I32, []),
    "cmh_softmax": (_I32, [_P, _P, _U64, _U64]),
    "cmh_layernorm": (_I32, [_P, _P, _U64, _U64, _P, _P, _D, _I32]),
    "cmh_gelu": (_I32, [_P, _P, _U64, _I32, _D, _D, _I32]),
    "cmh_rmsnorm": (_I32, [_P, _P, _U64, _U32, _U32, _P, _D, _P]),
    "cmh_silu_mul": (_I32, [_P, _P, _P, _U64, _U32, _P, _P]),
    "cmh_resadd_f32": (_I32, [_P, _P, _P, _U64]),
    "cmh_to_f32": (_I32, [_P, _P, _U64]),
    "cmh_attention": (_I32, [ctypes.POINTER(CmhAttnArgs)]),
}

_host = None


def host_lib():
    """libcormo_host.so, loaded once; raises if it is not built (no fallback)."""
    global _host
    if _host is None:
        if not os.path.exists(HOST_LIB_PATH):
            raise RuntimeError(f"{HOST_LIB_PATH} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(HOST_LIB_PATH)
        for name, (res, args) in HOST_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _host = lib
    return _host


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _check(rc: int, what: str) -> None:
    if rc:
        raise ValueError(f"{what}: invalid arguments")


def _d(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, np.float64))


def _chan(t: TensorInfo, n: int, F: int = 8) -> np.ndarray:
    """int32 exponents of the last axis, n of them (a scalar broadcast)."""
    e = np.asarray(F if t.exp is None else t.exp, np.int64).reshape(-1)
    if e.size not in (1, n):
        raise SchedulerError(f"tensor '{t.onnx_name}': {e.size} exponents for rows of {n}")
    return np.ascontiguousarray(np.broadcast_to(e, (n,)), np.int32)


class HostNode:
    """A node the simulator runs on the host with ``reference(ins, dtype)``."""
    inputs: List[TensorInfo]
    output: TensorInfo

    def reference(self, ins, dtype):
        raise NotImplementedError


# ---------------------------------------------------------------- ONNX host ops (Q8.8)
@dataclass
class SoftmaxNode(HostNode):
    """ONNX Softmax over the last axis on the host (host_nodes.py:989-1041)."""
    inputs: List[TensorInfo]
    output: TensorInfo

    def reference(self, ins, dtype):
        n = int(self.inputs[0].shape[-1])
        x = _d(ins[0]).reshape(-1, n)
        y = np.empty(x.shape, np.int16)
        _check(host_lib().cmh_softmax(_ptr(x), _ptr(y), x.shape[0], n), "host softmax")
        return (y.astype(np.float64) / 256.0).reshape(self.output.shape)


@dataclass
class LayerNormNode(HostNode):
    """LayerNormalization over the last ``n`` elements on the host, ONNX or TF form
    (host_nodes.py:1049-1148); gamma / beta float32 constants or None."""
    inputs: List[TensorInfo]
    output: TensorInfo
    gamma: Optional[np.ndarray] = None
    beta: Optional[np.ndarray] = None
    eps: float = 1e-5
    tf_form: int = 0

    def reference(self, ins, dtype):
        n = int(self.inputs[0].shape[-1])
        x = _d(ins[0]).reshape(-1, n)
        g = None if self.gamma is None else np.ascontiguousarray(np.asarray(self.gamma, np.float32).reshape(-1))
        b = None if self.beta is None else np.ascontiguousarray(np.asarray(self.beta, np.float32).reshape(-1))
        for v, nm in ((g, "gamma"), (b, "beta")):
            if v is not None and v.size != n:
                raise SchedulerError(f"LayerNormalization: {nm} has {v.size} elements, expected {n}")
        y = np.empty(x.shape, np.int16)
        _check(host_lib().cmh_layernorm(_ptr(x), _ptr(y), x.shape[0], n, _ptr(g), _ptr(b), float(self.eps),
                                        int(self.tf_form)), "host layernorm")
        return (y.astype(np.float64) / 256.0).reshape(self.output.shape)


@dataclass
class TransposeNode(HostNode):
    """ONNX Transpose on the host (host_nodes.py:1254-1330): a bit move, output[i] =
    input[i permuted by ``perm``]; values and exponents unchanged."""
    inputs: List[TensorInfo]
    output: TensorInfo
    perm: Sequence[int] = ()

    def __post_init__(self):
        x = self.inputs[0]
        self.perm = [int(p) for p in (self.perm if len(self.perm) else range(len(x.shape) - 1, -1, -1))]
        if sorted(self.perm) != list(range(len(x.shape))) or list(self.output.shape) != [x.shape[p] for p in self.perm]:
            raise SchedulerError(f"Transpose '{self.output.onnx_name}': perm {self.perm} of {list(x.shape)}")

    def reference(self, ins, dtype):
        x = np.asarray(ins[0], np.float64).reshape(self.inputs[0].shape)
        return np.ascontiguousarray(x.transpose(self.perm)).reshape(self.output.shape)


GELU_C1 = 0.044715
GELU_C2 = math.sqrt(2.0 / math.pi)
SQRT2 = math.sqrt(2.0)


@dataclass
class GeluNode(HostNode):
    """GELU on the host (host_nodes.py:1158-1245): ``approximate`` "tanh" x (0.5 (1 + tanh(c2 (x +
    c1 x^3)))), "none" x (0.5 (1 + erf(x / k))) (x k with div 0)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    approximate: str = "none"
    c1: float = GELU_C1
    c2: float = GELU_C2
    k: float = SQRT2
    div: int = 1

    def reference(self, ins, dtype):
        x = _d(ins[0]).reshape(-1)
        y = np.empty(x.shape, np.int16)
        tanh = self.approximate == "tanh"
        p1, p2 = (self.c1, self.c2) if tanh else (self.k, float(self.div))
        _check(host_lib().cmh_gelu(_ptr(x), _ptr(y), x.size, int(tanh), float(p1), float(p2), int(self.div)),
               "host gelu")
        return (y.astype(np.float64) / 256.0).reshape(self.output.shape)


# ---------------------------------------------------------------- the LLM host ops
@dataclass
class LlmRMSNormNode(HostNode):
    """y = (h r) gamma, r = 1 / sqrt(sum(h^2) / n + eps) per row of gamma's n, at the output's
    per-channel exponents (llm_nodes.py:618-688); h float32 (the float residual) or int16."""
    inputs: List[TensorInfo]
    output: TensorInfo
    gamma: np.ndarray = None
    eps: float = 1e-5
    F: int = 8

    def reference(self, ins, dtype):
        g = np.ascontiguousarray(np.asarray(self.gamma, np.float32).reshape(-1))
        n, W = g.size, int(self.inputs[0].shape[-1])
        if W % n:
            raise SchedulerError(f"RMSNorm '{self.output.onnx_name}': rows of {W} are not rows of {n}")
        h = _d(ins[0]).reshape(-1, n)
        y = np.empty(h.shape, np.int16)
        fo = _chan(self.output, W, self.F)
        _check(host_lib().cmh_rmsnorm(_ptr(h), _ptr(y), h.shape[0], n, W, _ptr(g), float(self.eps), _ptr(fo)),
               "host rmsnorm")
        return (y.reshape(-1, W).astype(np.float64) / np.power(2.0, fo.astype(np.float64))).reshape(self.output.shape)


@dataclass
class LlmSiluMulNode(HostNode):
    """a = silu(g) u, silu tabulated over g's raw int16 per gate exponent, at the output's
    exponents (llm_nodes.py:694-751)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    F: int = 8

    def reference(self, ins, dtype):
        n = int(self.inputs[0].shape[-1])
        g, u = _d(ins[0]).reshape(-1, n), _d(ins[1]).reshape(-1, n)
        y = np.empty(g.shape, np.int16)
        fg, fo = _chan(self.inputs[0], n, self.F), _chan(self.output, n, self.F)
        _check(host_lib().cmh_silu_mul(_ptr(g), _ptr(u), _ptr(y), g.shape[0], n, _ptr(fg), _ptr(fo)), "host silu_mul")
        return (y.astype(np.float64) / np.power(2.0, fo.astype(np.float64))).reshape(self.output.shape)


@dataclass
class LlmResAddNode(HostNode):
    """y = float32(h + d): the float residual stream's add (llm_nodes.py:576-609)."""
    inputs: List[TensorInfo]
    output: TensorInfo

    def reference(self, ins, dtype):
        h, d = _d(ins[0]).reshape(-1), _d(ins[1]).reshape(-1)
        y = np.empty(h.size, np.float32)
        _check(host_lib().cmh_resadd_f32(_ptr(h), _ptr(d), _ptr(y), h.size), "host resadd")
        return y.astype(np.float64).reshape(self.output.shape)


@dataclass
class LlmDequantNode(HostNode):
    """y = float32(raw 2^-f[c]), e.g. the logits for the caller (llm_nodes.py:1722-1749)."""
    inputs: List[TensorInfo]
    output: TensorInfo

    def reference(self, ins, dtype):
        x = _d(ins[0]).reshape(-1)
        y = np.empty(x.size, np.float32)
        _check(host_lib().cmh_to_f32(_ptr(x), _ptr(y), x.size), "host dequant")
        return y.astype(np.float64).reshape(self.output.shape)


@dataclass
class LlmToHostNode(LlmDequantNode):
    """A float32 device tensor handed to the caller's host buffer (llm_nodes.py:1752-1780)."""


@dataclass
class LlmAttentionNode(HostNode):
    """Causal GQA attention over the KV caches on the host, the xattn policy (llm_nodes.py:794-955):
    inputs [q0 [T][H HD], k0 [T][KV HD], v [T][KV HD], pos, n (optional), cache_k, cache_v] --
    the caches logical [C][KV HD], stored group-major, states written in place; the output
    [T][H HD] at its per-channel exponents.  cos / sin: float32 [C][HD / 2]."""
    inputs: List[TensorInfo]
    output: TensorInfo
    heads: int = 1
    kv_heads: int = 1
    head_dim: int = 8
    cos: np.ndarray = None
    sin: np.ndarray = None
    F: int = 8

    def __post_init__(self):
        H, KV, HD = self.heads, self.kv_heads, self.head_dim
        what = f"LlmAttention '{self.output.onnx_name}'"
        if len(self.inputs) not in (6, 7):
            raise SchedulerError(f"{what}: inputs q0, k0, v, pos, [n], cache_k, cache_v")
        q0, ck = self.inputs[0], self.inputs[-2]
        if HD % 8 or H % KV:
            raise SchedulerError(f"{what}: head_dim % 8 and heads % kv_heads")
        self.C = int(ck.shape[0])
        self.T = q0.numel // (H * HD)
        self.cos = np.ascontiguousarray(np.asarray(self.cos, np.float32))
        self.sin = np.ascontiguousarray(np.asarray(self.sin, np.float32))
        if self.cos.shape != (self.C, HD // 2) or self.sin.shape != self.cos.shape:
            raise SchedulerError(f"{what}: cos / sin must be [{self.C}][{HD // 2}]")
        for t in (self.inputs[-2], self.inputs[-1]):
            if list(t.shape) != [self.C, KV * HD] or t.group_layout != (KV, HD) or not t.state:
                raise SchedulerError(f"{what}: '{t.onnx_name}' must be a state [{self.C}][{KV * HD}] stored "
                                     f"group-major")
        if self.output.numel != q0.numel:
            raise SchedulerError(f"{what}: output numel")

    @property
    def has_n(self) -> bool:
        return len(self.inputs) == 7

    def reference(self, ins, dtype):
        """ins: float64 values; the cache arrays (logical [C][KV HD]) are updated in place."""
        H, KV, HD, C, T = self.heads, self.kv_heads, self.head_dim, self.C, self.T
        q0t, k0t, vt, ckt, cvt = self.inputs[0], self.inputs[1], self.inputs[2], self.inputs[-2], self.inputs[-1]
        pos = int(np.asarray(ins[3]).reshape(-1)[0])
        n = int(np.asarray(ins[4]).reshape(-1)[0]) if self.has_n else T
        f_ck, f_cv = _chan(ckt, KV * HD, self.F), _chan(cvt, KV * HD, self.F)
        ck, cv = ins[-2], ins[-1]
        # the caches as the raw group-major lanes the host op keeps
        ckr = np.ascontiguousarray(np.rint(np.asarray(ck, np.float64).reshape(C, KV, HD)
                                           * np.power(2.0, f_ck.reshape(KV, HD))).transpose(1, 0, 2), np.int16)
        cvr = np.ascontiguousarray(np.rint(np.asarray(cv, np.float64).reshape(C, KV, HD)
                                           * np.power(2.0, f_cv.reshape(KV, HD))).transpose(1, 0, 2), np.int16)
        q0, k0, v = _d(ins[0]), _d(ins[1]), _d(ins[2])
        f_out = _chan(self.output, H * HD, self.F)
        out = np.empty(T * H * HD, np.int16)
        a = CmhAttnArgs(q0=_ptr(q0), k0=_ptr(k0), v=_ptr(v), ck=_ptr(ckr), cv=_ptr(cvr), f_ck=_ptr(f_ck),
                        f_cv=_ptr(f_cv), cos=_ptr(self.cos), sin=_ptr(self.sin), out=_ptr(out), f_out=_ptr(f_out),
                        scale=1.0 / math.sqrt(HD), T=T, H=H, KV=KV, HD=HD, C=C, pos=pos, n=n)
        _check(host_lib().cmh_attention(ctypes.byref(a)), "host attention")
        ck[...] = (ckr.transpose(1, 0, 2).reshape(C, KV * HD) / np.power(2.0, f_ck.astype(np.float64))).reshape(ck.shape)
        cv[...] = (cvr.transpose(1, 0, 2).reshape(C, KV * HD) / np.power(2.0, f_cv.astype(np.float64))).reshape(cv.shape)
        return (out.reshape(T, H * HD).astype(np.float64) / np.power(2.0, f_out.astype(np.float64))).reshape(
            self.output.shape)


# ---------------------------------------------------------------- the embedding (on the GPU)
@dataclass
class LlmEmbedNode(KernelNode):
    """h[t] = table[clamp(ids[t], 0, rows - 1)] (llm_nodes.py:466-570): ids an int32 tensor, the
    table float32 [rows][d]; the output the int32 residual (kind "i32": each row's values rounded
    half to even at the residual's exponent and saturated, _res32 :297-303) or float32 rows
    (kind "f32"), times ``scale`` first (a float32 product) when it is not 1.  The rows the
    gather copies are the output's own lanes, built once on the host from the constant table
    (int16 where every raw fits, the reference's res32_table), so the GPU gather is exact."""
    inputs: List[TensorInfo]
    output: TensorInfo
    table: np.ndarray = None
    scale: float = 1.0
    F: int = 8
    _image: Optional[np.ndarray] = field(default=None, init=False, repr=False)

    def __post_init__(self):
        ids, y = self.inputs[0], self.output
        tab = np.asarray(self.table, np.float32)
        what = f"LlmEmbed '{y.onnx_name}'"
        if tab.ndim != 2:
            raise SchedulerError(f"{what}: the table must be [rows][d]")
        self.rows, self.d = int(tab.shape[0]), int(tab.shape[1])
        if y.numel != ids.numel * self.d or int(y.shape[-1]) != self.d:
            raise SchedulerError(f"{what}: output [{ids.numel}][{self.d}]")
        if y.kind not in ("i32", "f32") or ids.kind not in ("i32", "host"):
            raise SchedulerError(f"{what}: int32 ids (device or host) into the int32 residual or float32 rows")
        if self.d % 4:
            raise SchedulerError(f"{what}: rows of a multiple of 4 lanes")
        if float(np.float32(self.scale)) != float(self.scale) or not self.scale > 0:
            raise SchedulerError(f"{what}: the scale must be a positive float32")
        self.table = tab

    def image(self) -> np.ndarray:
        """The output lanes of every table row: int16 / int32 raws of the residual, or float32."""
        if self._image is None:
            v = self.table if self.scale == 1.0 else (self.table * np.float32(self.scale)).astype(np.float32)
            if self.output.kind == "f32":
                self._image = np.ascontiguousarray(v, np.float32)
            else:
                f = np.broadcast_to(np.asarray(self.F if self.output.exp is None else self.output.exp,
                                               np.float64).reshape(-1), (self.d,))
                if (f != f[0]).any():
                    raise SchedulerError(f"LlmEmbed '{self.output.onnx_name}': the residual at one exponent")
                raw = np.clip(np.rint(v.astype(np.float64) * 2.0 ** f[0]), -2147483648.0, 2147483647.0)
                small = (raw >= -32768).all() and (raw <= 32767).all()
                self._image = np.ascontiguousarray(raw.astype(np.int16 if small else np.int32))
        return self._image


__all__ = ["HostNode", "SoftmaxNode", "LayerNormNode", "GeluNode", "LlmRMSNormNode", "LlmSiluMulNode",
           "LlmResAddNode", "LlmDequantNode", "LlmToHostNode", "LlmAttentionNode", "LlmEmbedNode", "host_lib",
           "HOST_SIGNATURES"]
