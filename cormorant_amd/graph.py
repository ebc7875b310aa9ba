"""Graph IR of the simulator: tensors and the node kinds the reference's ``_forward_pass``
dispatches on (inference-scheduler/src/codegen/_simulate.py:617-765).

The reference builds these nodes from ONNX (graph.py, nodes.py); here they are built
directly (no ONNX dependency).  Field names follow the reference's ScheduledNode / MatmulNode
/ ConvNode / PoolNode / ReshapeNode (nodes.py:311-584, 632-1067, 1154, 1770-2140) so that a
node of either carries the same geometry.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from .units import (ACT_NONE, OP_ADD, OP_DIV, OP_MUL, OP_RELU, OP_RELU6, OP_SOFTMAX,
                    OP_SOFTMAX_T, OP_SUB, POOL_AVG, POOL_LP, POOL_MAX)


class SchedulerError(ValueError):
    """A node whose geometry the units cannot run (the reference's SchedulerError)."""


class KernelNode:
    """A node the HIP units compute.  ``reference(ins, dtype)`` gives its output values for the
    input values ``ins`` (one per input, in order; a constant input's entry is ignored and the
    tensor's own data used) by running the node alone through the units: the per-node
    contract of the reference's LlmKernelNode / HostNode (llm_nodes.py:1172-1181,
    _simulate.py:667-690), so a node can be checked or swapped one at a time without its
    graph.  ``host`` ({name: value}) gives the runtime host tensors a node reads besides its
    inputs (a runtime position ``pos_t``, a softmax's ``mask_t``)."""

    def reference(self, ins, dtype=None, host=None):
        from .simulate import node_reference
        return node_reference(self, ins, dtype, host=host)


@dataclass
class TensorInfo:
    """A tensor of the graph (tensor.py TensorInfo): logical shape; ``exp`` the power-of-two
    exponent (None: the element type's F, i.e. Q8.8), scalar or per channel of the last
    axis; ``data`` the float64 values of a weight (quantized when the graph is simulated,
    _simulate.py:531-539); ``wexp`` a weight's rank-1 exponent [k][m] (numeric.py:199-255)."""
    onnx_name: str
    shape: Sequence[int]
    exp: Optional[object] = None
    data: Optional[np.ndarray] = None
    wexp: Optional[np.ndarray] = None
    kind: str = "i16"                 # "i16", "i32" (row-ops residual), "f32" (dequant output)
    raw: bool = False                 # ``data`` holds raw lanes of ``kind`` (a table), not values
    chexp: Optional[np.ndarray] = None        # per-channel exponents of axis 1 (NCHW), tensor.py
    group_layout: Optional[tuple] = None      # (KV, HD): a [C][KV * HD] cache stored group-major
    state: bool = False               # a persistent state (a KV cache): updated in place, kept across passes
    host: Optional[str] = None        # the reference's host-memory annotation ("f32", "i32", "i16"), if any

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape)) if len(self.shape) else 1

    def exp_full(self, F: int) -> np.ndarray:
        return np.asarray(F if self.exp is None else self.exp, np.int64)


@dataclass
class ScheduledNode(KernelNode):
    """A VectorOP call (nodes.py:311-584): op_code 0..9, fused act, LeakyReLU alpha."""
    inputs: List[TensorInfo]
    output: TensorInfo
    op_code: int
    act: int = ACT_NONE
    alpha: int = 0

    @property
    def arity(self) -> int:
        return 2 if self.op_code < OP_RELU else 1

    @property
    def fusable_act(self) -> Optional[int]:
        """The act register value this unary node would become in its producer (RELU -> act 1,
        RELU6 -> 2, the activation unit's ops LeakyReLU / SiLU / GELU / GELU-tanh -> 3 .. 6;
        nodes.py:347-353), else None."""
        return _ACT_FOR_OP.get(self.op_code) if self.arity == 1 else None


ACTIVATION_OPS = frozenset({6, 7, 8, 9})          # LeakyReLU, SiLU, GELU, GELU-tanh (nodes.py:156)
_ACT_FOR_OP = {OP_RELU: 1, OP_RELU6: 2, 6: 3, 7: 4, 8: 5, 9: 6}


def fuse_activations(graph: "Graph") -> int:
    """Fold each unary activation into the VectorOP node producing its input (the reference's
    OnnxGraph._fuse_activations, graph.py:1005-1058): when the producer is a VectorOP with no act
    yet and is not itself an activation op, the intermediate is not a graph output, the
    activation is its only reader and keeps its element count, the producer writes the
    activation's output with ``act`` set and the activation node goes.  Returns the count."""
    nodes = graph.nodes
    readers: Dict[str, List[int]] = {}
    for i, sn in enumerate(nodes):
        for t in sn.inputs:
            if t is not None:
                readers.setdefault(t.onnx_name, []).append(i)
    producer = {sn.output.onnx_name: i for i, sn in enumerate(nodes)}
    outputs = {t.onnx_name for t in graph.output_tensors}
    gone = set()
    for i, sn in enumerate(nodes):
        if not isinstance(sn, ScheduledNode) or sn.fusable_act is None:
            continue
        src = sn.inputs[0]
        j = producer.get(src.onnx_name)
        if j is None:
            continue
        prod = nodes[j]
        if (not isinstance(prod, ScheduledNode) or prod.act != ACT_NONE or prod.op_code in ACTIVATION_OPS
                or src.onnx_name in outputs or readers.get(src.onnx_name, []) != [i]
                or src.numel != sn.output.numel):
            continue
        prod.act, prod.alpha, prod.output = sn.fusable_act, sn.alpha, sn.output
        producer[sn.output.onnx_name] = j
        gone.add(i)
    if gone:
        graph.nodes = [sn for i, sn in enumerate(nodes) if i not in gone]
    return len(gone)


@dataclass
class MatmulNode(KernelNode):
    """C = A x B (nodes.py:632-955): A [..., n, k], B [k, m] (shared) or [..., k, m]."""
    inputs: List[TensorInfo]
    output: TensorInfo


@dataclass
class MatmulConvNode(KernelNode):
    """One MatMul C [.., n, m] = A [.., n, k] . B [.., k, m] run on the conv unit with the operands'
    roles swapped (nodes.py:1627-1786, matmul_lowering.py): a 1 x kw conv of stride (1, kw), no
    pad, out_ch n, in_ch k / kw, output out_h x out_w = m, weight = A (row-major [n][k] is the
    packed tile-major weight when k % (16 kw) == 0), x = B in conv_lowered_b_image's layout (kw
    1: B itself; kw > 1: a constant B re-laid once), y = C row-major.  The result is
    MatmulNode's bit for bit (the simulator treats both alike, _simulate.py:620-633).

    Batch (matmul_lowering._batch_mode, :123-143): A shared and B batched -> the conv's batch;
    B shared and A batched -> the batch folded into the rows (out_ch = batch n); both batched ->
    one call per item."""
    inputs: List[TensorInfo]
    output: TensorInfo
    kw: int = 1
    out_w: int = 0               # 0: m (one output row)

    def __post_init__(self):
        a, b = self.inputs
        n, k = int(a.shape[-2]), int(a.shape[-1])
        m = int(b.shape[-1])
        what = f"MatMul-on-conv '{self.output.onnx_name}'"
        if int(b.shape[-2]) != k:
            raise SchedulerError(f"{what}: A [.., {n}, {k}] x B {list(b.shape)}")
        ab = int(np.prod(a.shape[:-2])) if len(a.shape) > 2 else 1
        bb = int(np.prod(b.shape[:-2])) if len(b.shape) > 2 else 1
        batch = max(ab, bb)
        if ab not in (1, batch) or bb not in (1, batch):
            raise SchedulerError(f"{what}: batch dimensions do not broadcast")
        if n < 2 or k % 16 or m % 8:
            raise SchedulerError(f"{what}: needs n >= 2, k % 16 == 0 and m % 8 == 0 (n {n}, k {k}, m {m})")
        kw = int(self.kw)
        if not 1 <= kw <= 7 or k % (16 * kw):
            raise SchedulerError(f"{what}: kw {kw} (1 .. 7, k a multiple of 16 kw)")
        if kw > 1 and b.data is None:
            raise SchedulerError(f"{what}: kw > 1 re-lays a constant B only")
        self.out_w = int(self.out_w) or m
        if m % self.out_w:
            raise SchedulerError(f"{what}: out_w {self.out_w} does not divide m {m}")
        self.n, self.k, self.m, self.batch = n, k, m, batch
        self.out_h = m // self.out_w
        self.a_batch_stride = n * k if ab > 1 else 0
        self.b_batch_stride = k * m if bb > 1 else 0
        self.c_batch_stride = n * m
        if batch == 1:
            self.conv_n, self.conv_batch, self.calls = n, 1, 1
        elif ab == 1:                              # shared weights: the conv's batch
            self.conv_n, self.conv_batch, self.calls = n, batch, 1
        elif bb == 1:                              # the batch folds into the rows
            self.conv_n, self.conv_batch, self.calls = batch * n, 1, 1
        else:                                      # one call per item
            self.conv_n, self.conv_batch, self.calls = n, 1, batch
        if self.output.numel != batch * n * m:
            raise SchedulerError(f"{what}: output numel")

    @property
    def in_ch(self) -> int:
        return self.k // self.kw

    @property
    def in_h(self) -> int:
        return self.out_h

    @property
    def in_w(self) -> int:
        return self.kw * self.out_w


@dataclass
class ConvNode(KernelNode):
    """NCHW Conv (nodes.py:1154): inputs x, w [M][C or 1][kh][kw], optional bias [M]."""
    inputs: List[TensorInfo]
    output: TensorInfo
    stride_h: int = 1
    stride_w: int = 1
    pad_top: int = 0
    pad_left: int = 0
    dilation_h: int = 1
    dilation_w: int = 1
    is_depthwise: bool = False

    has_bias = property(lambda self: len(self.inputs) > 2 and self.inputs[2] is not None)
    batch = property(lambda self: self.inputs[0].shape[0])
    in_ch = property(lambda self: self.inputs[0].shape[1])
    in_h = property(lambda self: self.inputs[0].shape[2])
    in_w = property(lambda self: self.inputs[0].shape[3])
    out_ch = property(lambda self: self.output.shape[1])
    out_h = property(lambda self: self.output.shape[2])
    out_w = property(lambda self: self.output.shape[3])
    kh = property(lambda self: self.inputs[1].shape[2])
    kw = property(lambda self: self.inputs[1].shape[3])


@dataclass
class PoolNode(KernelNode):
    """NCHW pooling (nodes.py:1770-2140)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    pool_type: int = POOL_MAX
    pool_h: int = 2
    pool_w: int = 2
    stride_h: int = 2
    stride_w: int = 2
    pad_top: int = 0
    pad_left: int = 0
    dil_h: int = 1
    dil_w: int = 1
    lp_order: int = 2
    count_include_pad: int = 0


@dataclass
class ReshapeNode(KernelNode):
    inputs: List[TensorInfo]
    output: TensorInfo


@dataclass
class SoftmaxVopNode(KernelNode):
    """The softmax unit (smx_nodes.py:121-386).  Row mode: softmax over the last axis of
    [rows, n].  Column mode (``keys_major``): input s[keys][queries], output P[queries][keys].
    ``cm`` / ``cfg`` / ``mask`` are the smx registers (vectorop_smx.scale_regs and
    causal_valid, mask None: every element valid -- ONNX Softmax's row mode,
    smx_nodes.py:190-204); the output exponent is cfg's f_p."""
    inputs: List[TensorInfo]
    output: TensorInfo
    cm: int = 12102203
    cfg: int = 0x0813
    mask: Optional[int] = None
    keys_major: bool = False
    mask_t: Optional[TensorInfo] = None      # a runtime mask: the host value of this tensor + mask_add
    mask_add: int = 0

    def mask_reg(self, n: int, host: Optional[int] = None) -> int:
        """The mask register: a runtime one (host + mask_add, the valid keys of a decode step at
        position host), the static one, or every element valid."""
        if self.mask_t is not None:
            if host is None:
                raise SchedulerError(f"softmax '{self.output.onnx_name}': the runtime mask needs its host value")
            return int(host) + self.mask_add
        return n if self.mask is None else self.mask


@dataclass
class DecodeAttentionNode(KernelNode):
    """One decode step's attention over the KV caches, fused: for every KV group (b, g) the
    group's G = heads / kv_heads query rows of q [B][heads hd] against cache rows [C][hd] of
    kc / vc [B][kv_heads][C][hd],
        s = sat16(wrap32(q K^T) >> 8),  P = the softmax unit's row mode over s (valid keys from
        the mask register),  o = sat16(wrap32(P V) >> 8),
    o [B][heads hd] -- the chain the unfused graph runs as two AttnContractNodes around a
    SoftmaxVopNode (LlmAttnConvNode's contractions, llm_nodes.py:1183-1425, and the row-mode
    softmax, vectorop_smx.py:50-66), with s and P never leaving the workgroup.  ``cm`` / ``cfg``
    / ``mask`` / ``mask_t`` / ``mask_add`` as SoftmaxVopNode's; the softmax's rows are the
    (b, g, i) in order.  q, kc and o at exponents with f_o = f_p + f_v - 8 (f_p cfg's)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    heads: int = 1
    kv_heads: int = 1
    head_dim: int = 64
    cm: int = 12102203
    cfg: int = 0x0813
    mask: Optional[int] = None
    mask_t: Optional[TensorInfo] = None
    mask_add: int = 0

    def mask_reg(self, n: int, host: Optional[int] = None) -> int:
        if self.mask_t is not None:
            if host is None:
                raise SchedulerError(f"decode attention '{self.output.onnx_name}': the runtime mask needs its host value")
            return int(host) + self.mask_add
        return n if self.mask is None else self.mask

    @property
    def group(self) -> int:
        return self.heads // self.kv_heads

    @staticmethod
    def supports(head_dim: int, ctx: int, group: int) -> bool:
        """The fused kernel's geometry: head dim 32 or 64, a cache of a multiple of 64 rows (up
        to 8192), at most 8 queries per KV group."""
        return head_dim in (32, 64) and ctx % 64 == 0 and 0 < ctx <= 8192 and 0 < group <= 8


def softmax_regs(f_s: int, sigma: float, f_p: int):
    """(smx_cm, smx_cfg) of scores at 2^-f_s with logit scale ``sigma`` and P at 2^-f_p
    (vectorop_smx.scale_regs + smx_nodes.regs, vectorop_smx.py:37-47, smx_nodes.py:64-76):
    Cm 2^-Cs = log2(e) sigma 2^-f_s 2^12 with Cm a 24-bit mantissa; cfg = Cs | f_p << 8."""
    c = math.log2(math.e) * float(sigma) * 2.0 ** (-float(f_s)) * 4096.0
    cs = 23 - math.floor(math.log2(c))
    cm = int(round(c * 2.0 ** cs))
    if cm >= 1 << 24:                          # rounding reached the next power of two
        cm, cs = cm >> 1, cs - 1
    if not 0 <= cs <= 63 or not 0 <= int(f_p) <= 31:
        raise SchedulerError(f"softmax registers out of range: f_s {f_s}, sigma {sigma}, f_p {f_p}")
    return cm, cs | (int(f_p) << 8)


@dataclass
class PermuteNode(KernelNode):
    """A data move between layouts (the attention's head split / merge, VitAttnPrep /
    LlmAttnMerge): output[i0][i1][i2][i3] = input_flat[offset + sum_k i_k strides[k]], the
    output's shape ``dims``; values and exponents move unchanged."""
    inputs: List[TensorInfo]
    output: TensorInfo
    dims: Tuple[int, int, int, int] = (1, 1, 1, 1)
    strides: Tuple[int, int, int, int] = (0, 0, 0, 1)
    offset: int = 0

    def gather_index(self) -> np.ndarray:
        """Flat input index of every output element, in output order."""
        idx = np.full(self.dims, self.offset, np.int64)
        for k, (d, st) in enumerate(zip(self.dims, self.strides)):
            shape = [1, 1, 1, 1]
            shape[k] = d
            idx = idx + (np.arange(d, dtype=np.int64) * st).reshape(shape)
        return idx.reshape(-1)


@dataclass
class RowOpsNode(KernelNode):
    """One row-ops job (ROWOPS_RTL_KERNEL.md 1.2) over whole tensors: A (and B) and C are
    [rows, n] raw tensors, the parameter block a uint8 array of 16-byte entries.  The
    higher-level row-ops node kinds (LayerNorm, RMSNorm, residual add, SiLU x up, RoPE,
    dequant; rowops_nodes.py) reduce to this job with their parameter blocks."""
    inputs: List[TensorInfo]
    output: TensorInfo
    op: int
    params: np.ndarray = field(default_factory=lambda: np.zeros(16, np.uint8))
    eps: int = 0
    aux: int = 0
    bq_sh: int = 0
    win_lo: int = 0
    win_hi: int = 0xFFFFFFFF


KEY_QUANTUM = 16


def attn_keys(pos: int, n: int, T: int, C: int, q: int = KEY_QUANTUM):
    """(valid rows n, keys) of a prefill-attention call: n clamped to 0 <= n <= T and
    pos + n <= C; the kernels run over keys = roundup(pos + n, q), at least q, at most C
    (llm_nodes.py:960-968)."""
    n = max(0, min(int(n), T, C - int(pos))) if int(pos) < C else 0
    k = -(-(int(pos) + n) // q) * q
    return n, max(q, min(k, C))


@dataclass
class LlmAttnConvNode(KernelNode):
    """One attention contraction of KV group ``group`` with a runtime key count
    (llm_nodes.py:1183-1425, reference() :1407-1425):
      kind "qk": s_g[j][p] = sum_d K_g[j][d] qx_g[d][p] for the cache rows j < keys,
                 inputs [K cache [C][KV HD] (group-major), qx [KV][HD][G T], pos, n],
                 output [C][G T] (rows >= keys zero);
      kind "pv": o_g[p][d] = sum_{j < keys} P_g[p][j] V_g[j][d],
                 inputs [P_g [G T][C], V cache [C][KV HD] (group-major), pos, n],
                 output [G T][HD].
    Raw integer sums, int32 wrap, floor(/ 2^8), saturated (_kernel_out :995-1001).
    ``static``: no pos / n, keys = C."""
    inputs: List[TensorInfo]
    output: TensorInfo
    kind: str = "qk"
    group: int = 0
    T: int = 1
    H: int = 1
    KV: int = 1
    HD: int = 16
    C: int = 16
    Q: int = KEY_QUANTUM
    static: bool = False
    has_n: bool = True

    @property
    def G(self) -> int:
        return self.H // self.KV


SMX_MAX_KEYS = 1024        # the softmax unit's column mode: keys per query column (vectorop_smx.py:34)


@dataclass
class AttnSoftmaxNode(KernelNode):
    """The prefill attention's softmax of KV group ``group`` on the softmax unit (LlmAttnSoftmax
    under the vsmx policy, smx_nodes.py:284-338): scores s_g [C][G T] (raw, keys-major, rows j <
    keys valid) -> P_g [G T][C] (raw at cfg's f_p), keys = roundup(pos + n, Q) (attn_keys).
    Column h' T + t (head h' of the group, query row t) is the unit's column-mode softmax over
    the keys j < min(keys, pos + 1 + t) (``causal``: the mask register valid0 = pos + 1 with
    period T) or j < max(min(keys, pos + n), 1) (not causal: an encoder's valid frames); P is 0
    at j >= keys.  ``cm`` / ``cfg``: the registers of softmax_regs, one pair for the group or one
    per head.  inputs [s_g, pos (host), n (host, optional: n = T)], or [s_g] alone (``static``: an
    encoder's VitAttnSoftmax, smx_nodes.py:206-248 -- pos 0, n = T, keys = C)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    T: int = 16
    G: int = 1
    C: int = 16
    Q: int = KEY_QUANTUM
    group: int = 0
    cm: object = 12102203
    cfg: object = 0x0813
    causal: bool = True

    def __post_init__(self):
        what = f"attention softmax '{self.output.onnx_name}'"
        if len(self.inputs) not in (1, 2, 3):
            raise SchedulerError(f"{what}: inputs scores, [pos, [n]]")
        s = self.inputs[0]
        GT = self.G * self.T
        if list(s.shape) != [self.C, GT] or list(self.output.shape) != [GT, self.C]:
            raise SchedulerError(f"{what}: scores [{self.C}][{GT}] -> P [{GT}][{self.C}]")
        if self.T % 16 or self.C % self.Q or self.Q % KEY_QUANTUM or not 0 < self.C <= SMX_MAX_KEYS:
            raise SchedulerError(f"{what}: query rows a multiple of 16, cache rows a multiple of the key "
                                 f"quantum and at most {SMX_MAX_KEYS}")
        if any(t.kind != "host" for t in self.inputs[1:]):
            raise SchedulerError(f"{what}: pos / n are host tensors")
        if self.static and self.C != -(-self.T // self.Q) * self.Q:
            raise SchedulerError(f"{what}: a static call has every key valid: C = roundup(T, {self.Q})")
        if any(np.asarray(r).size not in (1, self.G) for r in (self.cm, self.cfg)):
            raise SchedulerError(f"{what}: cm / cfg one pair, or one per head of the group")

    @property
    def has_n(self) -> bool:
        return len(self.inputs) == 3

    @property
    def static(self) -> bool:
        return len(self.inputs) == 1

    def pos_n(self, host) -> Tuple[int, int]:
        """(pos, n) of a call: the host values of the pos / n inputs (``host``: tensor -> int),
        n = T without its input, (0, T) for a static call."""
        if self.static:
            return 0, self.T
        return int(host(self.inputs[1])), int(host(self.inputs[2])) if self.has_n else self.T

    def regs(self) -> List[Tuple[int, int]]:
        """(cm, cfg) of each head of the group."""
        cm = np.broadcast_to(np.asarray(self.cm, np.int64).reshape(-1), (self.G,))
        cfg = np.broadcast_to(np.asarray(self.cfg, np.int64).reshape(-1), (self.G,))
        return [(int(a), int(b)) for a, b in zip(cm, cfg)]

    def mask_reg(self, pos: int, n: int, keys: int) -> int:
        """The softmax unit's mask register for this call: valid0 | period << 16."""
        if self.causal:
            return (int(pos) + 1) | (self.T << 16)
        return max(min(keys, int(pos) + int(n)), 1)


@dataclass
class AttnMergeNode(KernelNode):
    """LlmAttnMerge (llm_nodes.py:1560-1600, reference() :1660-1675): the P.V outputs o_g
    [G T][HD] of the KV groups, in group order, into pv [T][H HD] in head order,
    pv[t][(g G + h') HD + d] = o_g[h' T + t][d]; raw values move unchanged (pv's exponent is
    f_p + f_v - 8)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    T: int = 1
    H: int = 1
    KV: int = 1
    HD: int = 16

    def __post_init__(self):
        G = self.H // self.KV
        if len(self.inputs) != self.KV or any(t.numel != G * self.T * self.HD for t in self.inputs) \
                or self.output.numel != self.T * self.H * self.HD:
            raise SchedulerError(f"attention merge '{self.output.onnx_name}': {self.KV} inputs "
                                 f"[{G * self.T}][{self.HD}] -> [{self.T}][{self.H * self.HD}]")


@dataclass
class SelectRowNode(KernelNode):
    """LlmSelectRow (llm_nodes.py:1681-1718): y = h[n - 1] with n clamped to [1, rows], the last
    valid row of a padded prefill, written into its output (a state the head entry reads).
    inputs [h [rows][width], n (host)]; the output one row of h's kind and exponent."""
    inputs: List[TensorInfo]
    output: TensorInfo

    def __post_init__(self):
        h = self.inputs[0]
        if len(self.inputs) != 2 or self.inputs[1].kind != "host" or self.output.kind != h.kind \
                or self.output.numel != int(h.shape[-1]):
            raise SchedulerError(f"select row '{self.output.onnx_name}': inputs h, n (host); one row of h out")

    @property
    def rows(self) -> int:
        return self.inputs[0].numel // int(self.inputs[0].shape[-1])


@dataclass(frozen=True)
class HeadView:
    """Per-head blocks of a token-major tensor [batch seq][ld] as the slices [batch heads][seq]
    [width] of a contraction: slice b heads + h is rows b seq .. b seq + seq - 1, columns
    col + h width .. col + (h + 1) width - 1 (the q / K / V rows VitAttnPrep copies out of
    the fused projection, and the rows LlmAttnMerge copies o back into; vit.py:19-32), read
    or written in place."""
    col: int
    heads: int
    width: int
    seq: int

    def strides(self, ld: int) -> Tuple[int, int, int, int]:
        """(offset, row stride, slice stride over sequences, slice stride over heads) in elements."""
        return self.col, ld, self.seq * ld, self.width

    def gather(self, x: np.ndarray) -> np.ndarray:
        """[batch seq][ld] -> [batch heads][seq][width]."""
        ld = x.shape[-1]
        x = x.reshape(-1, self.seq, ld)[:, :, self.col:self.col + self.heads * self.width]
        return x.reshape(-1, self.seq, self.heads, self.width).transpose(0, 2, 1, 3).reshape(-1, self.seq, self.width)

    def scatter(self, y: np.ndarray, ld: int) -> np.ndarray:
        """[batch heads][seq][width] -> [batch seq][ld] (col 0, heads width == ld: every element)."""
        if self.col != 0 or self.heads * self.width != ld:
            raise ValueError("an output head view covers its tensor's rows")
        y = y.reshape(-1, self.heads, self.seq, self.width).transpose(0, 2, 1, 3)
        return y.reshape(-1, ld)


@dataclass
class AttnContractNode(KernelNode):
    """The attention contractions of ``batch`` (sequence, head) pairs with every key valid:
    out[i] = sat16(floor(wrap32(A[i] . B[i]) / 2^8)) for the raw int16 operands A [batch][n][k]
    and B [batch][k][m], the math of LlmAttnConvNode (q.K^T with A = K rows, B = the q image;
    P.V with A = P, B = V rows; llm_nodes.py:995-1001, 1407-1425) over static keys, one call
    for all pairs.  Output exponent f_a + f_b - 8 (score_exp / pv_exp, graph_builder.py:197-208).
    ``b_trans``: B given as [batch][m][k] (out = A . B^T), e.g. q rows against a K cache's rows,
    the scores then query-major.  ``a_view`` / ``b_view`` / ``c_view``: the operand (B as
    given, i.e. [batch][m][k] with ``b_trans``) or the output as a HeadView of a token-major
    tensor instead of a [batch][rows][cols] tensor of its own."""
    inputs: List[TensorInfo]
    output: TensorInfo
    b_trans: bool = False
    a_view: Optional[HeadView] = None
    b_view: Optional[HeadView] = None
    c_view: Optional[HeadView] = None

    def operand_shape(self, i: int) -> Tuple[int, int, int]:
        """[slices][rows][cols] of input ``i`` (0: A, 1: B as given) or 2: the output."""
        t = self.output if i == 2 else self.inputs[i]
        v = (self.a_view, self.b_view, self.c_view)[i]
        if v is None:
            if len(t.shape) != 3:
                raise SchedulerError(f"attention contraction '{self.output.onnx_name}': operand {i} not 3-d")
            return tuple(int(d) for d in t.shape)
        if len(t.shape) != 2 or int(t.shape[0]) % v.seq or v.col + v.heads * v.width > int(t.shape[1]):
            raise SchedulerError(f"attention contraction '{self.output.onnx_name}': head view outside its tensor")
        return int(t.shape[0]) // v.seq * v.heads, v.seq, v.width


@dataclass
class AttentionNode(KernelNode):
    """An encoder layer's attention as one node: for each of ``batch`` sequences of ``seq``
    tokens and each head, Q / K / V from the fused projection ``inputs[0]`` [batch seq][ld]
    (columns q_off / k_off / v_off + head_dim h), the scores s = K . Q^T keys-major at
    f_q + f_k - 8, P = the softmax unit's keys-major call with ``cm`` / ``cfg`` (every key
    valid), o = P . V at f_p + f_v - 8, merged into the output rows [batch seq][heads head_dim]:
    exactly the reference's chain VitAttnPrep, the q.K^T contraction, VitAttnSoftmaxVopNode,
    P.V and the merge (vit.py:19-32; llm_nodes.py:995-1001, 1407-1425; smx_nodes.py:121-248)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    batch: int = 1
    seq: int = 64
    heads: int = 1
    head_dim: int = 64
    q_off: int = 0
    k_off: int = 0
    v_off: int = 0
    cm: int = 12102203
    cfg: int = 0x0813


@dataclass
class KvWriteNode(KernelNode):
    """The step's K or V rows into the KV caches: x [B][KV * HD] (row b = sequence b's new
    row) -> cache [B][KV][C][HD] (each sequence's cache group-major) at row ``pos``, the
    cache written in place and returned as the output (the cache row writes of
    LlmAttnPrep / AttnPrepRoNode, llm_nodes.py:1012-1030 and :1155-1159).  The row is
    copied raw: x and the cache share one exponent."""
    inputs: List[TensorInfo]
    output: TensorInfo
    pos: int = 0
    pos_t: Optional[TensorInfo] = None       # a runtime position: this host tensor's value

    def position(self, host: Optional[int] = None) -> int:
        if self.pos_t is not None:
            if host is None:
                raise SchedulerError(f"KV write '{self.output.onnx_name}': the runtime position needs its host value")
            return int(host)
        return self.pos


@dataclass
class Graph:
    """Nodes in topological order plus the graph's inputs, outputs and weights."""
    nodes: List[object] = field(default_factory=list)
    input_tensors: List[TensorInfo] = field(default_factory=list)
    output_tensors: List[TensorInfo] = field(default_factory=list)

    @property
    def state_tensors(self) -> List[TensorInfo]:
        """The persistent states the nodes read and update in place (numeric.py states; the
        reference's Graph.state_tensors), in first-use order."""
        seen, out = set(), []
        for t in list(self.input_tensors) + [u for n in self.nodes for u in list(n.inputs) + [n.output]]:
            if t is not None and t.state and t.onnx_name not in seen:
                seen.add(t.onnx_name)
                out.append(t)
        return out

    @property
    def weight_tensors(self) -> List[TensorInfo]:
        seen, out = set(), []
        for n in self.nodes:
            for t in n.inputs:
                if t is not None and t.data is not None and t.onnx_name not in seen:
                    seen.add(t.onnx_name)
                    out.append(t)
        return out


def conv_out(size: int, k: int, stride: int, pad_lo: int, pad_hi: int, dil: int = 1) -> int:
    return (size + pad_lo + pad_hi - dil * (k - 1) - 1) // stride + 1


__all__ = ["SchedulerError", "KernelNode", "TensorInfo", "HeadView", "ScheduledNode", "MatmulNode", "MatmulConvNode", "ConvNode", "PoolNode",
           "ReshapeNode", "SoftmaxVopNode", "DecodeAttentionNode", "RowOpsNode", "LlmAttnConvNode", "KvWriteNode", "AttentionNode", "attn_keys",
           "AttnSoftmaxNode", "AttnMergeNode", "SelectRowNode", "KEY_QUANTUM", "SMX_MAX_KEYS",
           "Graph", "conv_out", "OP_ADD", "OP_SUB",
           "OP_MUL", "OP_DIV", "OP_RELU", "OP_RELU6", "OP_SOFTMAX", "OP_SOFTMAX_T", "POOL_MAX",
           "POOL_AVG", "POOL_LP"]
