"""The front end's node choice: a graph described op by op becomes this simulator's nodes by the
reference's rules (OnnxGraph's node resolution, inference-scheduler/src/graph.py:817-856).

The reference reads an ONNX model; here (no ``onnx`` dependency) a graph arrives as a list of
``OpDesc`` -- op type, input and output tensor names, attributes, domain -- over a registry of
``TensorInfo`` (the tensors after ``numeric.apply``: shapes, exponents, weights, states), plus
the platform's unit flags (``Platform``: platforms/<platform>.json kernels.*).  The choice per op:

* the custom-domain ops (``LLM_DOMAIN``) through their factories, with the row-ops unit's
  overrides taking the ops it runs when the platform has the unit (graph.py:822-831,
  rowops_nodes.LLM_OVERRIDES / VIT_OVERRIDES);
* Gelu / LeakyRelu / Silu: the VectorOP activation unit, or for Gelu the host op where the unit
  cannot run it (vectorop_act.from_onnx, vectorop_act.py:146-171);
* Softmax: the softmax unit's row mode, or the host op (smx_nodes.from_onnx_softmax,
  smx_nodes.py:190-204, softmax_ineligible :173-187);
* LayerNormalization: the row-ops NORM, or the host op (rowops_nodes.from_onnx_layernorm
  :240-257, layernorm_ineligible :211-237);
* Transpose: the row-ops COPY / TRANSPOSE, or the host copy (from_onnx_transpose :353-370);
* the host ops (host_nodes.HOST_OP_FACTORIES, host_nodes.py:1723-1734), MatMul, Conv, the
  pooling ops, the reshape family, and the VectorOP ops (Add / Sub / Mul / Div / Relu and Clip,
  which maps to RELU6 only for bounds (0, 6): nodes.py:422-441); anything else is an error
  naming the supported ops.

Then, as the reference's constructor does, the unary activations fold into the VectorOP nodes
producing their inputs (``graph.fuse_activations``, graph.py:1005-1069).

The custom-domain ops this build takes are the ones its node kinds cover: LlmEmbed,
LlmRMSNorm, LlmResAdd, LlmSiluMul, LlmDequant, LlmToHost, LlmAttention (the host attention),
VitLayerNorm, VitResAdd, VitGelu; the prefill attention chain on the units (LlmAttnPrep on the
row-ops unit, LlmAttnScores / LlmAttnPV, LlmAttnSoftmax under the vsmx policy, LlmAttnMerge;
llama.py:329-402), LlmSelectRow, and the encoder template's VitAttnPrep (rowops) and
VitAttnSoftmax (vsmx; vit.py:564-630); and two ops of this build's own that stand for the
reference's attention chains, which it runs as one fused node each: ``VitAttention`` (VitAttnPrep,
LlmAttnScores, VitAttnSoftmax on the unit, LlmAttnPV, LlmAttnMerge: vit.py:19-32 -> AttentionNode)
and ``LlmDecodeAttention`` (LlmAttnPrep's RoPE and cache-row writes, the scores, LlmAttnSoftmax,
P.V: llm_nodes.py:1012-1030, rowops_nodes.py:893-1236 -> DecodePrepNode + DecodeAttentionNode).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from functools import lru_cache
from typing import Any, Callable, Dict, List, Optional, Sequence

import numpy as np

from . import units
from .graph import (KEY_QUANTUM, AttentionNode, AttnMergeNode, AttnSoftmaxNode, ConvNode, DecodeAttentionNode, Graph,
                    LlmAttnConvNode, MatmulNode, PoolNode, ReshapeNode, ScheduledNode, SchedulerError, SelectRowNode,
                    SoftmaxVopNode, TensorInfo, conv_out, fuse_activations, softmax_regs)
from .host_ops import (GeluNode, LayerNormNode, LlmAttentionNode, LlmDequantNode, LlmEmbedNode, LlmResAddNode,
                       LlmRMSNormNode, LlmSiluMulNode, LlmToHostNode, SoftmaxNode, TransposeNode)
from .rowops_nodes import (N_MAX, P1_BITS, AttnPrepRoNode, DecodePrepNode, DequantRoNode, VitAttnPrepRoNode, LayerNorm32RoNode, LayerNormRoNode,
                           ResAddBiasRoNode, ResAddRoNode, RMSNormRoNode, SiluMulRoNode, TransposeRoNode, beta_bits,
                           collapse, gamma_scale, transpose_job)

LLM_DOMAIN = "axi.llm"
Q88 = "ap_fixed<16,8>"
ALIGN_ELEMS = 8                 # 16-byte runs of int16 (nodes.py _ALIGN_ELEMS)
SMX_MAX_ROW = 2048              # the softmax unit's row buffer (vectorop_smx.MAX_ROW)


@dataclass
class OpDesc:
    """One op of a graph: what an ONNX NodeProto carries for the node choice."""
    op_type: str
    inputs: Sequence[str]
    outputs: Sequence[str]
    attrs: Dict[str, Any] = field(default_factory=dict)
    domain: str = ""
    name: str = ""

    @property
    def label(self) -> str:
        return self.name or self.op_type


@dataclass(frozen=True)
class Platform:
    """The platform's unit flags: VectorOPKernel's activation unit (kernels.vectorop.activations,
    AXI_VECTOROP_ACTIVATIONS), its softmax unit (kernels.vectorop.softmax, AXI_VECTOROP_SOFTMAX)
    and the row-ops unit (kernels.rowops.unit, AXI_ROWOPS)."""
    activations: bool = True
    softmax: bool = True
    rowops: bool = True


class _Ctx:
    def __init__(self, tensors: Dict[str, TensorInfo], platform: Platform, dtype: str):
        self.tensors, self.platform, self.dtype = tensors, platform, dtype

    def t(self, name: str, op: OpDesc) -> TensorInfo:
        if name not in self.tensors:
            raise SchedulerError(f"Tensor '{name}' of node '{op.label}' was not found in the graph.")
        return self.tensors[name]

    def ins(self, op: OpDesc) -> List[TensorInfo]:
        return [self.t(n, op) for n in op.inputs if n]

    def out(self, op: OpDesc) -> TensorInfo:
        return self.t(op.outputs[0], op)


def _plain_q88(t: TensorInfo) -> bool:
    """A Q8.8 tensor in device memory: no exponent annotation, not host memory, not a state."""
    return t.exp is None and t.wexp is None and t.chexp is None and t.host is None and not t.state and t.kind == "i16"


# ---------------------------------------------------------------- VectorOP ops (nodes.py:164-175, 395-441)
_VECTOROP = {"Add": (units.OP_ADD, 2), "Sub": (units.OP_SUB, 2), "Mul": (units.OP_MUL, 2), "Div": (units.OP_DIV, 2),
             "Relu": (units.OP_RELU, 1), "Clip": (units.OP_RELU6, 1)}


def _clip_bounds(op: OpDesc, ins: List[TensorInfo]):
    """Clip's (min, max): the attributes (opset < 11) or the constant inputs 2 and 3."""
    mn, mx = op.attrs.get("min"), op.attrs.get("max")
    if mn is None and len(ins) > 1 and ins[1].data is not None:
        mn = float(np.asarray(ins[1].data).reshape(-1)[0])
    if mx is None and len(ins) > 2 and ins[2].data is not None:
        mx = float(np.asarray(ins[2].data).reshape(-1)[0])
    return mn, mx


def _vectorop(op: OpDesc, ctx: _Ctx):
    code, arity = _VECTOROP[op.op_type]
    ins = ctx.ins(op)
    if op.op_type == "Clip":
        mn, mx = _clip_bounds(op, ins)
        if mn != 0.0 or mx != 6.0:
            raise SchedulerError(f"Clip node '{op.label}' has bounds (min={mn}, max={mx}). "
                                 f"Only Clip(0, 6) maps to VECTOROP_RELU6.")
        ins = ins[:1]
    if len(ins) != arity:
        kind = "Binary" if arity == 2 else "Unary"
        raise SchedulerError(f"{kind} op '{op.op_type}' in node '{op.label}' requires {arity} inputs, got {len(ins)}.")
    return ScheduledNode(ins, ctx.out(op), code)


# ---------------------------------------------------------------- the activation unit (vectorop_act.py:117-171)
ACT_OPS = ("Gelu", "LeakyRelu", "Silu")
ALPHA_ONE = 1 << 16


def _act_ineligible(op: OpDesc, ctx: _Ctx) -> Optional[str]:
    """Why the op cannot run on the activation unit, or None."""
    if not ctx.platform.activations:
        return "the platform's VectorOPKernel has no activation unit"
    if ctx.dtype != Q88:
        return f"the activation unit computes in {Q88}, not {ctx.dtype}"
    for t in (ctx.t(op.inputs[0], op), ctx.out(op)):
        if t.exp is not None or t.host is not None:
            return f"tensor '{t.onnx_name}' is not a plain Q8.8 DMA tensor (exponent / host memory)"
    return None


def _gelu_host(op: OpDesc, ctx: _Ctx) -> GeluNode:
    a = op.attrs
    return GeluNode([ctx.t(op.inputs[0], op)], ctx.out(op), approximate=str(a.get("approximate", "none")),
                    **{k: a[k] for k in ("c1", "c2", "k", "div") if k in a})


def gelu_act(host: GeluNode, dtype: str = Q88) -> Optional[int]:
    """ACT_GELU / ACT_GELU_TANH when the host op computes the unit's function on every Q8.8 input,
    else None (vectorop_act.gelu_act: the host op's values over all 65 536 inputs against the
    unit's table)."""
    if dtype != Q88:
        return None
    act = units.ACT_GELU_TANH if host.approximate == "tanh" else units.ACT_GELU
    return act if _gelu_matches(act, host.approximate, host.c1, host.c2, host.k, host.div) else None


@lru_cache(maxsize=None)
def _gelu_matches(act: int, approximate: str, c1: float, c2: float, k: float, div: int) -> bool:
    """Whether the host GELU with these constants equals the unit's table on all 65 536 inputs."""
    x = TensorInfo("x", [65536])
    probe = GeluNode([x], TensorInfo("y", [65536]), approximate=approximate, c1=c1, c2=c2, k=k, div=div)
    got = np.round(np.asarray(probe.reference([np.arange(-32768, 32768, dtype=np.float64) / 256.0], Q88)) * 256.0)
    return bool(np.array_equal(got, units.host_act_table(act).astype(np.float64)))


def leaky_alpha(alpha: float, label: str) -> int:
    """The alpha register of a LeakyRelu slope: round(alpha 2^16), 0 <= alpha < 1."""
    q = int(round(float(alpha) * ALPHA_ONE))
    if not (0.0 <= float(alpha) and q < ALPHA_ONE):
        raise SchedulerError(f"LeakyRelu node '{label}': alpha={alpha} -- VectorOPKernel takes a slope "
                             f"0 <= alpha < 1 (quantised to 2^-16).")
    return q


def _act(op: OpDesc, ctx: _Ctx):
    why = _act_ineligible(op, ctx)
    x, y = ctx.t(op.inputs[0], op), ctx.out(op)
    if op.op_type == "Gelu":
        host = _gelu_host(op, ctx)
        act = None if why else gelu_act(host, ctx.dtype)
        if act is None:
            return host
        return ScheduledNode([x], y, units.OP_GELU_TANH if act == units.ACT_GELU_TANH else units.OP_GELU)
    if why:
        raise SchedulerError(f"{op.op_type} node '{op.label}' needs VectorOPKernel's activation unit: {why}.")
    if op.op_type == "LeakyRelu":
        return ScheduledNode([x], y, units.OP_LEAKY_RELU, alpha=leaky_alpha(op.attrs.get("alpha", 0.01), op.label))
    return ScheduledNode([x], y, units.OP_SILU)


# ---------------------------------------------------------------- Softmax (smx_nodes.py:173-204)
def _rows_n(t: TensorInfo):
    n = int(t.shape[-1]) if len(t.shape) else 1
    return t.numel // max(n, 1), n


def softmax_ineligible(x: TensorInfo, y: TensorInfo, platform: Platform, dtype: str) -> Optional[str]:
    if not platform.softmax:
        return "the platform's VectorOPKernel has no softmax unit"
    if dtype != Q88:
        return f"the softmax unit reads {Q88}, not {dtype}"
    for t in (x, y):
        if not _plain_q88(t):
            return f"tensor '{t.onnx_name}' is not a plain Q8.8 DMA tensor"
    rows, n = _rows_n(x)
    if n > SMX_MAX_ROW:
        return f"rows of {n} elements (the unit buffers {SMX_MAX_ROW})"
    if rows > 1 and n % ALIGN_ELEMS:
        return f"rows of {n} elements are not 16-byte aligned"
    return None


def _softmax(op: OpDesc, ctx: _Ctx):
    x, y = ctx.t(op.inputs[0], op), ctx.out(op)
    axis = int(op.attrs.get("axis", -1))
    if axis not in (-1, len(x.shape) - 1):
        raise SchedulerError(f"Softmax node '{op.label}': axis {axis} (the last axis only)")
    if softmax_ineligible(x, y, ctx.platform, ctx.dtype) is not None:
        return SoftmaxNode([x], y)
    cm, cfg = softmax_regs(8, 1.0, 8)
    return SoftmaxVopNode([x], y, cm=cm, cfg=cfg)


# ---------------------------------------------------------------- LayerNormalization (rowops_nodes.py:211-257)
def _ln_params(op: OpDesc, ctx: _Ctx, n: int):
    ins = ctx.ins(op)
    gamma = op.attrs.get("gamma", ins[1].data if len(ins) > 1 and ins[1].data is not None else None)
    beta = op.attrs.get("beta", ins[2].data if len(ins) > 2 and ins[2].data is not None else None)
    gamma = np.ones(n) if gamma is None else np.asarray(gamma, np.float64).reshape(-1)
    beta = np.zeros(n) if beta is None else np.asarray(beta, np.float64).reshape(-1)
    return gamma, beta, float(op.attrs.get("epsilon", 1e-5))


def layernorm_ineligible(x: TensorInfo, y: TensorInfo, gamma, beta, eps: float, platform: Platform,
                         dtype: str) -> Optional[str]:
    if not platform.rowops:
        return "the platform has no row-ops unit"
    if dtype != Q88:
        return f"the unit's LayerNorm reads {Q88}, not {dtype}"
    for t in (x, y):
        if not _plain_q88(t):
            return f"tensor '{t.onnx_name}' is not a plain Q8.8 DMA tensor"
    rows, n = _rows_n(x)
    if n > N_MAX:
        return f"rows of {n} elements (the unit takes {N_MAX})"
    if rows > 1 and n % ALIGN_ELEMS:
        return f"rows of {n} elements are not 16-byte aligned"
    if not (np.isfinite(gamma).all() and np.isfinite(beta).all()):
        return "gamma / beta are not finite"
    g = gamma_scale(gamma)
    if g + 4 > 63 or P1_BITS + g - 8 > 63:
        return f"gamma's exponent 2^-{g} is beyond the unit's shifts"
    bb = beta_bits(beta)
    if (np.abs(np.rint(beta * 2.0 ** bb)) >= 2 ** 21).any() or P1_BITS + g - bb > 63:
        return "beta beyond the parameter block's int22"
    e = eps * n * n * 2.0 ** 16
    if not 0 <= e < 2.0 ** 63:
        return f"eps {eps} (E = eps n^2 2^16 beyond 63 bits)"
    return None


def _layernorm(op: OpDesc, ctx: _Ctx):
    x, y = ctx.t(op.inputs[0], op), ctx.out(op)
    n = int(x.shape[-1])
    if int(op.attrs.get("axis", -1)) not in (-1, len(x.shape) - 1):
        raise SchedulerError(f"LayerNormalization node '{op.label}': the last axis only")
    gamma, beta, eps = _ln_params(op, ctx, n)
    if layernorm_ineligible(x, y, gamma, beta, eps, ctx.platform, ctx.dtype) is not None:
        return LayerNormNode([x], y, gamma=gamma, beta=beta, eps=eps)
    return LayerNormRoNode([x], y, gamma=gamma, beta=beta, eps=eps)


# ---------------------------------------------------------------- Transpose (rowops_nodes.py:326-370)
def _transpose(op: OpDesc, ctx: _Ctx):
    x, y = ctx.t(op.inputs[0], op), ctx.out(op)
    perm = list(op.attrs.get("perm", range(len(x.shape) - 1, -1, -1)))
    host = TransposeNode([x], y, perm=perm)
    if (not ctx.platform.rowops or x.kind != "i16" or y.kind != "i16" or x.host is not None or y.host is not None
            or x.state or y.state):
        return host
    st = [int(np.prod(x.shape[i + 1:])) for i in range(len(x.shape))]
    dims, sstr = collapse([int(x.shape[p]) for p in perm], [st[p] for p in perm])
    if transpose_job(dims, sstr) is None:
        return host
    return TransposeRoNode([x], y, perm=perm)


# ---------------------------------------------------------------- MatMul, Conv, pools, reshapes
def _matmul(op: OpDesc, ctx: _Ctx):
    a, b = ctx.ins(op)[:2]
    y = ctx.out(op)
    if len(a.shape) < 2 or len(b.shape) < 2 or int(a.shape[-1]) != int(b.shape[-2]):
        raise SchedulerError(f"MatMul node '{op.label}': A {list(a.shape)} x B {list(b.shape)}")
    n, k, m = int(a.shape[-2]), int(a.shape[-1]), int(b.shape[-1])
    batch = max(a.numel // (n * k), b.numel // (k * m))
    if y.numel != batch * n * m:
        raise SchedulerError(f"MatMul node '{op.label}': output {list(y.shape)} for A {list(a.shape)} x "
                             f"B {list(b.shape)}")
    return MatmulNode([a, b], y)


def _pads4(op: OpDesc, nd: int = 2):
    p = list(op.attrs.get("pads", [0] * (2 * nd)))
    if op.attrs.get("auto_pad", "NOTSET") not in ("NOTSET", "VALID"):
        raise SchedulerError(f"node '{op.label}': auto_pad {op.attrs['auto_pad']} (explicit pads only)")
    return p[0], p[1], p[2], p[3]


def _conv(op: OpDesc, ctx: _Ctx):
    ins = ctx.ins(op)
    x, w, y = ins[0], ins[1], ctx.out(op)
    sh, sw = op.attrs.get("strides", [1, 1])
    dh, dw = op.attrs.get("dilations", [1, 1])
    pt, pl, pb, pr = _pads4(op)
    group = int(op.attrs.get("group", 1))
    C, M = int(x.shape[1]), int(w.shape[0])
    depthwise = group > 1
    if depthwise and not (group == C == M and int(w.shape[1]) == 1):
        raise SchedulerError(f"Conv node '{op.label}': group {group} (1, or depthwise with group = channels)")
    kh, kw = int(w.shape[2]), int(w.shape[3])
    oh, ow = conv_out(int(x.shape[2]), kh, sh, pt, pb, dh), conv_out(int(x.shape[3]), kw, sw, pl, pr, dw)
    if list(y.shape) != [int(x.shape[0]), M, oh, ow]:
        raise SchedulerError(f"Conv node '{op.label}': output {list(y.shape)}, expected {[int(x.shape[0]), M, oh, ow]}")
    return ConvNode(ins[:3], y, stride_h=int(sh), stride_w=int(sw), pad_top=int(pt), pad_left=int(pl),
                    dilation_h=int(dh), dilation_w=int(dw), is_depthwise=depthwise)


_POOLS = {"MaxPool": units.POOL_MAX, "AveragePool": units.POOL_AVG, "LpPool": units.POOL_LP,
          "GlobalMaxPool": units.POOL_MAX, "GlobalAveragePool": units.POOL_AVG, "GlobalLpPool": units.POOL_LP}


def _pool(op: OpDesc, ctx: _Ctx):
    x, y = ctx.t(op.inputs[0], op), ctx.out(op)
    kind = _POOLS[op.op_type]
    lp = int(op.attrs.get("p", 2))
    if op.op_type.startswith("Global"):
        H, W = int(x.shape[2]), int(x.shape[3])
        return PoolNode([x], y, kind, H, W, 1, 1, lp_order=lp)
    kh, kw = op.attrs["kernel_shape"]
    sh, sw = op.attrs.get("strides", [1, 1])
    dh, dw = op.attrs.get("dilations", [1, 1])
    pt, pl, _pb, _pr = _pads4(op)
    if int(op.attrs.get("ceil_mode", 0)):
        raise SchedulerError(f"{op.op_type} node '{op.label}': ceil_mode 1")
    return PoolNode([x], y, kind, int(kh), int(kw), int(sh), int(sw), int(pt), int(pl), int(dh), int(dw), lp,
                    int(op.attrs.get("count_include_pad", 0)))


RESHAPE_OPS = frozenset({"Reshape", "Squeeze", "Unsqueeze", "Dropout", "Flatten", "Identity"})


def _reshape(op: OpDesc, ctx: _Ctx):
    x, y = ctx.t(op.inputs[0], op), ctx.out(op)
    if x.numel != y.numel:
        raise SchedulerError(f"{op.op_type} node '{op.label}': {x.numel} elements into {y.numel}")
    return ReshapeNode([x], y)


# host ops of host_nodes.HOST_OP_FACTORIES that this build does not run
_HOST_NOT_BUILT = frozenset({"Slice", "Concat", "Resize", "Gather", "OneHot", "Cast"})


def _host_not_built(op: OpDesc, ctx: _Ctx):
    raise SchedulerError(f"Node '{op.label}': {op.op_type} is a host op of the reference that this build does not run")


# ---------------------------------------------------------------- the custom-domain ops
def _need_rowops(op: OpDesc, ctx: _Ctx, what: str):
    if not ctx.platform.rowops:
        raise SchedulerError(f"{op.op_type} node '{op.label}': {what} needs the row-ops unit")


def _llm_embed(op, ctx):
    return LlmEmbedNode([ctx.t(op.inputs[0], op)], ctx.out(op), table=op.attrs["table"],
                        scale=float(op.attrs.get("scale", 1.0)))


def _llm_rmsnorm(op, ctx):
    h, y = ctx.t(op.inputs[0], op), ctx.out(op)
    gamma, eps = op.attrs["gamma"], float(op.attrs.get("eps", 1e-5))
    if ctx.platform.rowops and h.kind == "i32":
        return RMSNormRoNode([h], y, gamma=gamma, eps=eps)
    return LlmRMSNormNode([h], y, gamma=gamma, eps=eps)


def _llm_resadd(op, ctx):
    h, d = ctx.ins(op)[:2]
    y = ctx.out(op)
    bias = op.attrs.get("bias")
    if ctx.platform.rowops and y.kind == "i32":
        return ResAddRoNode([h, d], y) if bias is None else ResAddBiasRoNode([h, d], y, bias=bias)
    if bias is not None:
        raise SchedulerError(f"{op.op_type} node '{op.label}': a bias needs the row-ops unit")
    return LlmResAddNode([h, d], y)


def _llm_silu_mul(op, ctx):
    g, u = ctx.ins(op)[:2]
    if ctx.platform.rowops:
        return SiluMulRoNode([g, u], ctx.out(op))
    return LlmSiluMulNode([g, u], ctx.out(op))


def _llm_dequant(op, ctx):
    x, y = ctx.t(op.inputs[0], op), ctx.out(op)
    if ctx.platform.rowops and y.kind == "f32":
        return DequantRoNode([x], y)
    return (LlmToHostNode if op.op_type == "LlmToHost" else LlmDequantNode)([x], y)


def _llm_attention(op, ctx):
    a = op.attrs
    return LlmAttentionNode(ctx.ins(op), ctx.out(op), heads=int(a["heads"]), kv_heads=int(a["kv_heads"]),
                            head_dim=int(a["head_dim"]), cos=a["cos"], sin=a["sin"])


def _vit_layernorm(op, ctx):
    _need_rowops(op, ctx, "the int32 residual's LayerNorm")
    return LayerNorm32RoNode([ctx.t(op.inputs[0], op)], ctx.out(op), gamma=op.attrs["gamma"], beta=op.attrs["beta"],
                             eps=float(op.attrs.get("eps", 1e-6)))


def _vit_gelu(op, ctx):
    """VitGelu(f, b): GELU of f + b on the activation unit (the act fused into the ADD's call,
    vit.py _gelu_vop_rows) where f and the output are plain Q8.8."""
    ins = ctx.ins(op)
    why = _act_ineligible(op, ctx)
    if why:
        raise SchedulerError(f"VitGelu node '{op.label}' needs VectorOPKernel's activation unit: {why}.")
    if len(ins) == 1:
        return ScheduledNode(ins, ctx.out(op), units.OP_GELU)
    return ScheduledNode(ins[:2], ctx.out(op), units.OP_ADD, act=units.ACT_GELU)


def _vit_attention(op, ctx):
    if not ctx.platform.softmax:
        raise SchedulerError(f"VitAttention node '{op.label}': the keys-major softmax needs VectorOPKernel's "
                             f"softmax unit")
    a = op.attrs
    return AttentionNode([ctx.t(op.inputs[0], op)], ctx.out(op), batch=int(a["batch"]), seq=int(a["seq"]),
                         heads=int(a["heads"]), head_dim=int(a["head_dim"]), q_off=int(a["q_off"]),
                         k_off=int(a["k_off"]), v_off=int(a["v_off"]), cm=int(a["cm"]), cfg=int(a["cfg"]))


def _llm_decode_attention(op, ctx):
    """inputs [q, k, v, K cache, V cache] (the caches [B][KV][C][HD] group-major), outputs
    [q after RoPE, o]: DecodePrepNode then DecodeAttentionNode."""
    if not (ctx.platform.rowops and ctx.platform.softmax):
        raise SchedulerError(f"LlmDecodeAttention node '{op.label}': needs the row-ops and softmax units")
    a = op.attrs
    q, k, v, kc, vc = ctx.ins(op)[:5]
    qr, o = ctx.t(op.outputs[0], op), ctx.t(op.outputs[1], op)
    pos_t = ctx.tensors.get(a["pos_t"]) if a.get("pos_t") else None
    H, KV, HD = int(a["heads"]), int(a["kv_heads"]), int(a["head_dim"])
    prep = DecodePrepNode([q, k, v, kc, vc], qr, heads=H, kv_heads=KV, head_dim=HD, cos=a["cos"], sin=a["sin"],
                          pos=int(a["pos"]), pos_t=pos_t)
    att = DecodeAttentionNode([qr, kc, vc], o, heads=H, kv_heads=KV, head_dim=HD, cm=int(a["cm"]), cfg=int(a["cfg"]),
                              mask=int(a["pos"]) + 1, mask_t=pos_t, mask_add=1)
    return [prep, att]


def _heads(op):
    a = op.attrs
    H, KV, HD = int(a["num_heads"]), int(a["num_kv_heads"]), int(a["head_dim"])
    return H, KV, HD, H // KV


def _llm_attn_prep(op, ctx):
    """LlmAttnPrep [q0, k0, v, pos, n, K cache, V cache] -> qx on the row-ops unit (the rowops
    policy, rowops_nodes.py:1134-1219); the host prep is not built."""
    _need_rowops(op, ctx, "the attention prep (the host LlmAttnPrep is not built)")
    a = op.attrs
    H, KV, HD, _ = _heads(op)
    ins = [ctx.t(n, op) for n in op.inputs if n]
    return AttnPrepRoNode(ins, ctx.out(op), heads=H, kv_heads=KV, head_dim=HD, fq=np.asarray(a["q_exp"], np.int64),
                          cos=a["cos"], sin=a["sin"], key_quantum=int(a.get("key_quantum", KEY_QUANTUM)))


def _llm_attn_conv(op, ctx):
    """LlmAttnScores [K cache, qx, pos, n] -> s_g, LlmAttnPV [P_g, V cache, pos, n] -> o_g
    (llm_nodes.py:1183-1425): one KV group's contraction on the conv unit over the runtime keys."""
    H, KV, HD, G = _heads(op)
    ins = [ctx.t(n, op) for n in op.inputs if n]
    qk = op.op_type == "LlmAttnScores"
    cache = ins[0] if qk else ins[1]
    T = (ins[1].shape[-1] if qk else ins[0].shape[0]) // G
    return LlmAttnConvNode(ins, ctx.out(op), kind="qk" if qk else "pv", group=int(op.attrs["group"]), T=int(T), H=H,
                           KV=KV, HD=HD, C=int(cache.shape[0]), Q=int(op.attrs.get("key_quantum", KEY_QUANTUM)),
                           static=len(ins) == 2, has_n=len(ins) != 3)


def _vit_attn_prep(op, ctx):
    """VitAttnPrep [q0, k0, v, K cache, V cache] -> qx with rowops = 1 (rowops_nodes.py:1596-1712):
    VitAttnPrepRoNode; the biases bq / bk / bv and the columns ``cols`` are attributes here.  The
    host VitAttnPrep, RoPE and the key rows are not built."""
    a = op.attrs
    if not (ctx.platform.rowops and int(a.get("rowops", 0))):
        raise SchedulerError(f"VitAttnPrep node '{op.label}': runs on the row-ops unit (rowops = 1); the host "
                             f"prep is not built")
    if int(a.get("rope", 0)):
        raise SchedulerError(f"VitAttnPrep node '{op.label}': the 3-D RoPE variant is not built")
    ins = [ctx.t(n, op) for n in op.inputs]
    return VitAttnPrepRoNode(ins, ctx.out(op), heads=int(a["num_heads"]), head_dim=int(a["head_dim"]),
                             fq=np.asarray(a["q_exp"]), fk=np.asarray(a["k_exp"]), fv=np.asarray(a["v_exp"]),
                             bq=a.get("bq"), bk=a.get("bk"), bv=a.get("bv"), cols=tuple(a.get("cols", (0, 0, 0))),
                             query_major=bool(int(a.get("query_major", 0))))


def _vit_attn_softmax(op, ctx):
    """VitAttnSoftmax [s] -> P with vsmx = 1: the static column-mode call on the softmax unit
    (smx_nodes.py:206-248); the host softmax and the row splits (``cols``) are not built."""
    a = op.attrs
    if not (ctx.platform.softmax and int(a.get("vsmx", 0))):
        raise SchedulerError(f"VitAttnSoftmax node '{op.label}': runs on VectorOPKernel's softmax unit (vsmx = 1); "
                             f"the host softmax is not built")
    if "cols" in a or int(a.get("query_major", 0)):
        raise SchedulerError(f"VitAttnSoftmax node '{op.label}': row splits / query-major scores are not built")
    s = ctx.t(op.inputs[0], op)
    C, T = (int(d) for d in s.shape)
    scale = float(a.get("logit_scale", 1.0 / np.sqrt(int(a["head_dim"]))))
    cm, cfg = softmax_regs(int(np.asarray(a["s_exp"]).reshape(-1)[0]), scale, int(np.asarray(a["p_exp"]).reshape(-1)[0]))
    return AttnSoftmaxNode([s], ctx.out(op), T=T, G=1, C=C, cm=cm, cfg=cfg, causal=False)


def _llm_attn_softmax(op, ctx):
    """LlmAttnSoftmax [s_g, pos, n] -> P_g with vsmx = 1 on the softmax unit (smx_nodes.py:284-324);
    the host p12 softmax is not built."""
    a = op.attrs
    if not (ctx.platform.softmax and int(a.get("vsmx", 0))):
        raise SchedulerError(f"LlmAttnSoftmax node '{op.label}': runs on VectorOPKernel's softmax unit (vsmx = 1); "
                             f"the host p12 softmax is not built")
    if int(a.get("window", 0)):
        raise SchedulerError(f"LlmAttnSoftmax node '{op.label}': a sliding window is the host softmax's (not built)")
    H, KV, HD, G = _heads(op)
    ins = [ctx.t(n, op) for n in op.inputs if n]
    C, GT = (int(d) for d in ins[0].shape)
    scale = float(a.get("logit_scale", 1.0 / np.sqrt(HD)))
    fs = np.broadcast_to(np.asarray(a["s_exp"], np.int64).reshape(-1), (G,))
    fp = np.broadcast_to(np.asarray(a["p_exp"], np.int64).reshape(-1), (G,))
    regs = [softmax_regs(int(fs[h]), scale, int(fp[h])) for h in range(G)]
    cm, cfg = (regs[0] if len(set(regs)) == 1 else ([r[0] for r in regs], [r[1] for r in regs]))
    if int(a.get("causal", 1)) == 2:
        raise SchedulerError(f"LlmAttnSoftmax node '{op.label}': the prefix-LM mask (causal 2) is not built")
    return AttnSoftmaxNode(ins, ctx.out(op), T=GT // G, G=G, C=C, Q=int(a.get("key_quantum", KEY_QUANTUM)),
                           group=int(a["group"]), cm=cm, cfg=cfg, causal=int(a.get("causal", 1)) == 1)


def _llm_attn_merge(op, ctx):
    H, KV, HD, G = _heads(op)
    ins = ctx.ins(op)
    return AttnMergeNode(ins, ctx.out(op), T=ins[0].numel // (G * HD), H=H, KV=KV, HD=HD)


def _llm_select_row(op, ctx):
    return SelectRowNode(ctx.ins(op)[:2], ctx.out(op))


LLM_FACTORIES: Dict[str, Callable] = {
    "LlmEmbed": _llm_embed, "LlmRMSNorm": _llm_rmsnorm, "LlmResAdd": _llm_resadd, "LlmSiluMul": _llm_silu_mul,
    "LlmDequant": _llm_dequant, "LlmToHost": _llm_dequant, "LlmAttention": _llm_attention,
    "VitLayerNorm": _vit_layernorm, "VitResAdd": _llm_resadd, "VitGelu": _vit_gelu, "VitAttention": _vit_attention,
    "LlmDecodeAttention": _llm_decode_attention, "LlmAttnPrep": _llm_attn_prep, "LlmAttnScores": _llm_attn_conv,
    "LlmAttnPV": _llm_attn_conv, "LlmAttnSoftmax": _llm_attn_softmax, "LlmAttnMerge": _llm_attn_merge,
    "LlmSelectRow": _llm_select_row, "VitAttnPrep": _vit_attn_prep, "VitAttnSoftmax": _vit_attn_softmax,
}
SUPPORTED = sorted(set(_VECTOROP) | set(ACT_OPS) | {"Softmax", "LayerNormalization", "Transpose", "MatMul", "Conv"}
                   | set(_POOLS) | RESHAPE_OPS)


def node_for(op: OpDesc, ctx: _Ctx):
    """The scheduled node (or nodes) of one op, by graph.py:817-856's order of rules."""
    if op.domain == LLM_DOMAIN:
        if op.op_type not in LLM_FACTORIES:
            raise SchedulerError(f"Node '{op.label}': unknown {LLM_DOMAIN} op '{op.op_type}' "
                                 f"(known: {sorted(LLM_FACTORIES)})")
        return LLM_FACTORIES[op.op_type](op, ctx)
    if op.op_type in ACT_OPS:
        return _act(op, ctx)
    if op.op_type == "Softmax":
        return _softmax(op, ctx)
    if op.op_type == "LayerNormalization":
        return _layernorm(op, ctx)
    if op.op_type == "Transpose":
        return _transpose(op, ctx)
    if op.op_type in _HOST_NOT_BUILT:
        return _host_not_built(op, ctx)
    if op.op_type == "MatMul":
        return _matmul(op, ctx)
    if op.op_type == "Conv":
        return _conv(op, ctx)
    if op.op_type in _POOLS:
        return _pool(op, ctx)
    if op.op_type in RESHAPE_OPS:
        return _reshape(op, ctx)
    if op.op_type in _VECTOROP:
        return _vectorop(op, ctx)
    raise SchedulerError(f"Node '{op.label}' (op_type='{op.op_type}') is not supported.\nSupported ops: {SUPPORTED}")


def build_graph(ops: Sequence[OpDesc], tensors: Dict[str, TensorInfo], inputs: Sequence[str],
                outputs: Sequence[str], platform: Platform = Platform(), dtype: str = Q88,
                fuse_act: bool = True) -> Graph:
    """The simulator graph of ``ops`` (in topological order) over the tensor registry: each op's
    node by ``node_for``; with exponent annotations the constant MatMul weights encoded at their
    rank-1 exponents (numeric.encode_matmul_weights); then the activation fusion.  ``inputs`` /
    ``outputs`` name the graph's input and output tensors."""
    ctx = _Ctx(dict(tensors), platform, dtype)
    nodes: List[object] = []
    for op in ops:
        sn = node_for(op, ctx)
        nodes.extend(sn if isinstance(sn, list) else [sn])
    g = Graph(nodes, input_tensors=[ctx.t(n, OpDesc("input", [], [n])) for n in inputs],
              output_tensors=[ctx.t(n, OpDesc("output", [], [n])) for n in outputs])
    if any(t.exp is not None or t.chexp is not None for t in ctx.tensors.values()):
        # the pow2 MatMuls' constant weights at their rank-1 exponents (graph.py:861-863)
        from .dtype import AP_FIXED_16_8
        from .numeric import encode_matmul_weights
        encode_matmul_weights(g.nodes, AP_FIXED_16_8)
    if fuse_act:
        fuse_activations(g)
    return g


__all__ = ["LLM_DOMAIN", "OpDesc", "Platform", "build_graph", "node_for", "gelu_act", "leaky_alpha",
           "softmax_ineligible", "layernorm_ineligible", "SUPPORTED"]
