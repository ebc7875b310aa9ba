"""Row-ops node adapters: the reference's RowOps nodes (inference-scheduler/src/rowops_nodes.py)
as jobs of the GPU row-ops unit.

Each adapter takes what the reference's factory takes -- the tensors with their exponents
and the float parameters (gamma, beta, eps, bias, the RoPE tables) -- derives the job
constants and the 16-byte-per-column parameter block exactly as the reference's scheduler
does (rowops_spec.py norm_params / gamma_scale / beta_bits / bias_bits / bias_params /
param_block), checks the same eligibility rules (SchedulerError), and lowers to one or
more ``RoJob``s that ``Simulator`` runs with ``units.rowops`` over raw device tensors.
The arithmetic itself is the unit's (cm_rowops), so an adapter's output is the
reference's ``reference()`` of the node bit for bit.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from .graph import KernelNode, SchedulerError, TensorInfo, attn_keys
from .units import (F_B_EN, F_NORM_LN, F_P_BCAST, F_RELU, RO_ADDX, RO_COPY, RO_DEQUANT, RO_MULACT,
                    RO_NORM, RO_ROPE, RO_XPOSE)

# the unit's fixed-point constants (rowops_spec.py:44-49, 316-320)
P1_BITS = 24          # the normalised value at 2^-24
BQ_BITS = 20          # beta as an int22 at 2^-20
ROPE_BITS = 23        # cos / sin as int24 at 2^-23
SILU_BITS = 20        # silu(g) at 2^-20
G_BITS = 14           # the gate at 2^-14 inside the unit
N_MAX = 4096          # elements per row
K_I16, K_I32, K_F32 = 0, 1, 2
BIAS_EXTRA = 8        # a COPY with a bias sums 8 bits below the finer grid (rowops_spec.py:160)
I32_HI = 2 ** 31 - 1
NO_WINDOW = 0xFFFFFFFF
QIMAGE_R = 8          # the q image's TRANSPOSE tiles: 8 query rows -> 16-byte granules (rowops_nodes.py:703)
KEY_QUANTUM = 16      # the attention's key count quantum (llm_nodes.KEY_QUANTUM)


# ---------------------------------------------------------------- job constants
def opword(op: int, ak: int = K_I16, bk: int = K_I16, ck: int = K_I16, b_en=False, p_bcast=False,
           relu=False, ln=False) -> int:
    """The op register: [3:0] op, [5:4] / [7:6] / [9:8] the A / B / C kinds, then the flags
    (rowops_spec.py:569-576)."""
    return (op | (ak << 4) | (bk << 6) | (ck << 8) | (F_B_EN if b_en else 0) | (F_P_BCAST if p_bcast else 0)
            | (F_RELU if relu else 0) | (F_NORM_LN if ln else 0))


def gamma_scale(gamma) -> int:
    """g such that the largest |gamma| * 2^g lies in [2^30, 2^31) (rowops_spec.py:124-130)."""
    m = float(np.max(np.abs(np.asarray(gamma, np.float64)))) if np.size(gamma) else 0.0
    return 0 if m == 0.0 else 30 - math.floor(math.log2(m))


def beta_bits(beta) -> int:
    """The finest scale 2^-bb (bb <= 20) at which round(beta * 2^bb) fits an int22
    (rowops_spec.py:133-144)."""
    if beta is None:
        return BQ_BITS
    m = float(np.max(np.abs(np.asarray(beta, np.float64)))) if np.size(beta) else 0.0
    bb = BQ_BITS
    while bb > 0 and abs(round(m * 2.0 ** bb)) >= 1 << 21:
        bb -= 1
    return bb


def bias_bits(bias, f: int) -> int:
    """A residual bias' scale: the sum's exponent, coarser only where beta_bits needs it
    (rowops_spec.py:147-151)."""
    return min(int(f), beta_bits(bias))


def quant_bias(bias, f: int) -> np.ndarray:
    """The bias values as the unit adds them at 2^-f: rounded once at 2^-bias_bits
    (rowops_spec.py:154-157)."""
    bb = bias_bits(bias, f)
    return np.rint(np.asarray(bias, np.float64) * 2.0 ** bb) / 2.0 ** bb


def bias_exp(bias, f_x, f_out, extra: int = BIAS_EXTRA) -> np.ndarray:
    """Per column, the exponent a COPY with a bias sums at: max(f_x, f_out) + extra, at most
    24, lowered where round(bias * 2^fp) would leave the int22, never below max(f_x, f_out)
    (rowops_spec.py:163-183)."""
    bias = np.asarray(bias, np.float64).reshape(-1)
    n = bias.size
    lo = np.maximum(np.broadcast_to(np.asarray(f_x, np.int64), (n,)),
                    np.broadcast_to(np.asarray(f_out, np.int64), (n,)))
    fp = np.minimum(lo + extra, 24)
    for _ in range(64):
        over = np.abs(np.rint(bias * np.power(2.0, fp.astype(np.float64)))) > (1 << 21) - 1
        if not over.any():
            break
        fp = np.where(over, fp - 1, fp)
    if (fp < lo).any():
        raise SchedulerError("bias_exp: a bias too large for the int22 parameter at the output's grid")
    return fp


def bias_params(bias, f_x, f_out):
    """(Bq' [n], sh_a [n], sh_c [n]) of a COPY with a bias at fp = bias_exp
    (rowops_spec.py:186-196)."""
    fp = bias_exp(bias, f_x, f_out)
    n = fp.size
    bq = np.rint(np.asarray(bias, np.float64).reshape(-1) * np.power(2.0, fp.astype(np.float64))).astype(np.int64)
    return (bq, fp - np.broadcast_to(np.asarray(f_x, np.int64), (n,)),
            fp - np.broadcast_to(np.asarray(f_out, np.int64), (n,)))


def norm_params(gamma, n: int, eps: float, f_in: int, beta=None, rms: bool = False):
    """(G int32 [n], g, Bq [n] or None, E): gamma (times sqrt(n) for RMSNorm) at 2^-g, eps as
    the eps register (eps n^2 2^(2 f_in) for LayerNorm, eps n 2^(2 f_in) for RMSNorm), and
    beta at the 2^-(24 + g) scale of the product, i.e. round(beta 2^bb) << (24 + g - bb)
    (rowops_spec.py:199-219)."""
    gamma = np.asarray(gamma, np.float64)
    gs = gamma * math.sqrt(n) if rms else gamma
    g = gamma_scale(gs)
    G = np.rint(gs * 2.0 ** g).astype(np.int64)
    if rms:
        return G, g, None, int(round(eps * n * 2.0 ** (2 * f_in)))
    E = int(round(eps * n * n * 2.0 ** (2 * f_in)))
    if beta is None:
        return G, g, None, E
    bb = beta_bits(beta)
    Bq = np.rint(np.asarray(beta, np.float64) * 2.0 ** bb).astype(np.int64) << (P1_BITS + g - bb)
    return G, g, Bq, E


def param_block(G, Bq, sh_a, sh_b, sh_c) -> np.ndarray:
    """The parameter block of the columns as bytes: per column a 16-byte entry of int32 G,
    int32 Bq' (an int22, sign-extended), u8 sh_a, sh_b, sh_c and zeros
    (ROWOPS_RTL_KERNEL.md 1.3; rowops_spec.py:579-601).  Scalars broadcast."""
    G = np.asarray(G, np.int64).reshape(-1)
    n = G.size
    cols = [np.broadcast_to(np.asarray(0 if v is None else v, np.int64), (n,)) for v in (Bq, sh_a, sh_b, sh_c)]
    Bq, sa, sb, sc = cols
    if (np.abs(G) > I32_HI).any() or (Bq < -(1 << 21)).any() or (Bq >= 1 << 21).any():
        raise SchedulerError("param_block: G beyond int32 or Bq' beyond int22")
    sh = np.stack([sa, sb, sc])
    if (sh < 0).any() or (sh > 63).any():
        raise SchedulerError("param_block: a shift outside 0..63")
    img = np.zeros((n, 16), np.uint8)
    img[:, 0:4] = (G & 0xFFFFFFFF).astype("<u4").view(np.uint8).reshape(n, 4)
    img[:, 4:8] = (Bq & 0xFFFFFFFF).astype("<u4").view(np.uint8).reshape(n, 4)
    img[:, 8], img[:, 9], img[:, 10] = sa, sb, sc
    return img.reshape(-1)


def pblock(G, Bq, sh_a, sh_b, sh_c, n: int):
    """(block, bcast): one entry with P_BCAST when every column's fields agree, else n
    entries (rowops_nodes.py:377-384)."""
    cols = [np.broadcast_to(np.asarray(0 if v is None else v, np.int64), (n,)) for v in (G, Bq, sh_a, sh_b, sh_c)]
    bcast = all(bool((c == c[0]).all()) for c in cols)
    if bcast:
        cols = [c[:1] for c in cols]
    return param_block(*cols), bcast


def rope_tables_raw(cos, sin):
    """int24 at 2^-23 of the cos / sin tables (rowops_spec.py:267-271)."""
    return (np.rint(np.asarray(cos, np.float64) * 2.0 ** ROPE_BITS).astype(np.int64),
            np.rint(np.asarray(sin, np.float64) * 2.0 ** ROPE_BITS).astype(np.int64))


def rope_table(cos, sin) -> np.ndarray:
    """The table a ROPE job streams as B: per position 2 HD int32, cos[0..HD) then
    sin[0..HD), the float32 [C][HD/2] tables repeated over both halves
    (rowops_nodes.py rope_raw_tensor)."""
    cos = np.asarray(cos, np.float32)
    sin = np.asarray(sin, np.float32)
    cr, sr = rope_tables_raw(np.concatenate([cos, cos], 1).astype(np.float64),
                             np.concatenate([sin, sin], 1).astype(np.float64))
    return np.ascontiguousarray(np.concatenate([cr, sr], axis=1).astype(np.int32))


# ---------------------------------------------------------------- jobs
@dataclass
class RoJob:
    """One RowOpsKernel job over the rows of the node's tensors: columns [col0, col0 + n)
    of A, C (and B, unless ``b_row0`` selects table rows), the op word, the parameter
    block and the eps / aux / bq_sh registers."""
    op: int
    params: np.ndarray
    n: int
    col0: int = 0
    eps: int = 0
    aux: int = 0
    bq_sh: int = 0
    b_row0: Optional[int] = None     # B is a table: job row t reads table row b_row0 + t
    b_same: bool = False             # ... or every job row reads table row b_row0 (B row stride 0)


def _exps(t: TensorInfo, F: int, n: int) -> np.ndarray:
    """Per-column exponents of the last axis (a scalar exponent broadcast)."""
    e = np.asarray(F if t.exp is None else t.exp, np.int64).reshape(-1)
    if e.size == 1:
        return np.full(n, int(e[0]), np.int64)
    if e.size != n:
        raise SchedulerError(f"tensor '{t.onnx_name}': {e.size} exponents for rows of {n}")
    return e


def _require(cond, what: str, msg: str):
    if not cond:
        raise SchedulerError(f"{what}: {msg}")


class RowOpsAdapter(KernelNode):
    """Base of the adapters: ``inputs`` / ``output`` tensors and ``jobs()``."""
    inputs: List[TensorInfo]
    output: TensorInfo

    def jobs(self) -> List[RoJob]:
        raise NotImplementedError

    @property
    def n(self) -> int:
        return int(self.inputs[0].shape[-1])

    @property
    def rows(self) -> int:
        return self.inputs[0].numel // self.n


# ---------------------------------------------------------------- adapters
@dataclass
class LayerNormRoNode(RowOpsAdapter):
    """ONNX LayerNormalization of Q8.8 rows on the unit (rowops_nodes.py:161-262): NORM with
    NORM_LN, gamma at 2^-g, beta as Bq' at 2^-bb, eps as E = eps n^2 2^16."""
    inputs: List[TensorInfo]
    output: TensorInfo
    gamma: Optional[np.ndarray] = None
    beta: Optional[np.ndarray] = None
    eps: float = 1e-5
    F: int = 8

    def __post_init__(self):
        n, what = self.n, f"LayerNormalization '{self.output.onnx_name}'"
        for t in (self.inputs[0], self.output):
            _require(t.exp is None and t.kind == "i16", what, f"'{t.onnx_name}' is not a plain Q8.8 tensor")
        _require(n <= N_MAX, what, f"rows of {n} elements (the unit takes {N_MAX})")
        self.gamma = np.ones(n) if self.gamma is None else np.asarray(self.gamma, np.float64).reshape(-1)
        self.beta = np.zeros(n) if self.beta is None else np.asarray(self.beta, np.float64).reshape(-1)
        _require(np.isfinite(self.gamma).all() and np.isfinite(self.beta).all(), what, "gamma / beta are not finite")
        G, g, _bq, E = norm_params(self.gamma, n, self.eps, self.F, beta=self.beta)
        _require(g + 4 <= 63 and P1_BITS + g - 8 <= 63, what, f"gamma's exponent 2^-{g} beyond the shifts")
        bb = beta_bits(self.beta)
        bqp = np.rint(self.beta * 2.0 ** bb).astype(np.int64)
        _require((np.abs(bqp) < 2 ** 21).all() and P1_BITS + g - bb <= 63, what, "beta beyond the int22")
        _require(0 <= E < 2 ** 63, what, f"eps {self.eps} beyond the eps register")
        self.g, self.bb, self.E = int(g), int(bb), int(E)
        self._params = param_block(G, bqp, 0, 0, P1_BITS + g - self.F)

    def jobs(self):
        return [RoJob(opword(RO_NORM, ln=True), self._params, self.n, eps=self.E, bq_sh=P1_BITS + self.g - self.bb)]


@dataclass
class LayerNorm32RoNode(RowOpsAdapter):
    """A LayerNorm of the int32 residual at 2^-fr into int16 at per-channel exponents
    (rowops_nodes.py:1282-1412, _layernorm32)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    gamma: np.ndarray = None
    beta: np.ndarray = None
    eps: float = 1e-6
    F: int = 8

    def __post_init__(self):
        h, y = self.inputs[0], self.output
        n, what = self.n, f"LayerNorm32 '{y.onnx_name}'"
        fr = _exps(h, self.F, n)
        _require(h.kind == "i32" and (fr == fr[0]).all(), what, "h: the int32 residual at one exponent")
        _require(y.kind == "i16" and y.numel == h.numel and y.shape[-1] == n, what, "output: int16 of h's shape")
        gamma = np.asarray(self.gamma, np.float64).reshape(-1)
        beta = np.asarray(self.beta, np.float64).reshape(-1)
        _require(gamma.size == n and beta.size == n and np.isfinite(gamma).all() and np.isfinite(beta).all(),
                 what, "gamma / beta [n]")
        G, g, _bq, E = norm_params(gamma, n, self.eps, int(fr[0]), beta=beta)
        bb = beta_bits(beta)
        bq = np.rint(beta * 2.0 ** bb).astype(np.int64)
        sh_c = P1_BITS + g - _exps(y, self.F, n)
        _require((sh_c >= 0).all() and (sh_c <= 63).all() and 0 <= P1_BITS + g - bb <= 63, what,
                 f"gamma's exponent 2^-{g} beyond the shifts")
        _require(0 <= E < 2 ** 63, what, f"eps {self.eps} beyond the eps register")
        _require(n <= N_MAX, what, f"rows of {n} beyond {N_MAX}")
        self.fr, self.g, self.bb, self.E = int(fr[0]), int(g), int(bb), int(E)
        self._params, self.bcast = pblock(G, bq, 0, 0, sh_c, n)

    def jobs(self):
        return [RoJob(opword(RO_NORM, K_I32, K_I16, K_I16, p_bcast=self.bcast, ln=True), self._params, self.n,
                      eps=self.E, bq_sh=P1_BITS + self.g - self.bb)]


@dataclass
class RMSNormRoNode(RowOpsAdapter):
    """LlmRMSNorm of an int32 tensor at 2^-fr into int16 at per-channel exponents, rows of
    gamma's length (rowops_nodes.py:449-496, from_llm_rmsnorm :617-649)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    gamma: np.ndarray = None
    eps: float = 1e-5
    F: int = 8

    @property
    def n(self) -> int:
        return int(np.asarray(self.gamma).size)

    def __post_init__(self):
        h, y = self.inputs[0], self.output
        self.gamma = np.asarray(self.gamma, np.float64).reshape(-1)
        n, W, what = self.n, int(h.shape[-1]), f"RMSNorm '{y.onnx_name}'"
        fr = _exps(h, self.F, W)
        _require(h.kind == "i32" and (fr == fr[0]).all(), what, "h: an int32 tensor at one exponent")
        _require(y.kind == "i16" and y.numel == h.numel and y.shape[-1] == W, what, "output: int16 of h's shape")
        _require(W % n == 0 and n <= N_MAX, what, "gamma size")
        G, g, _b, E = norm_params(self.gamma, n, self.eps, int(fr[0]), rms=True)
        fo = _exps(y, self.F, W)
        _require((fo.reshape(-1, n) == fo[:n]).all(), what, "output exponents: one per channel of a head")
        sh_c = P1_BITS + g - fo[:n]
        _require((sh_c >= 0).all() and (sh_c <= 63).all(), what, f"gamma's exponent 2^-{g} beyond the shifts")
        _require(0 <= E < 2 ** 63, what, f"eps {self.eps} beyond the eps register")
        self.fr, self.g, self.E = int(fr[0]), int(g), int(E)
        self._params, self.bcast = pblock(G, 0, 0, 0, sh_c, n)

    def jobs(self):
        return [RoJob(opword(RO_NORM, K_I32, K_I16, K_I16, p_bcast=self.bcast), self._params, self.n, eps=self.E)]


@dataclass
class ResAddRoNode(RowOpsAdapter):
    """LlmResAdd: h1 = sat32(h + (d << (fr - f_d))), the int32 residual plus the int16 delta at
    its per-channel exponents, one ADDX job (rowops_nodes.py:401-447, from_llm_resadd)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    F: int = 8

    def __post_init__(self):
        h, d, y = self.inputs[0], self.inputs[1], self.output
        n, what = self.n, f"ResAdd '{y.onnx_name}'"
        fr = _exps(h, self.F, n)
        _require(h.kind == "i32" and (fr == fr[0]).all() and y.kind == "i32"
                 and (_exps(y, self.F, n) == fr[0]).all(), what, "h and the output: the int32 residual at one exponent")
        _require(d.kind == "i16" and d.shape[-1] == n and d.numel == h.numel == y.numel, what,
                 "delta: int16 of the residual's shape")
        fd = _exps(d, self.F, n)
        _require((fd <= fr[0]).all() and (fr[0] - fd <= 63).all(), what, "delta exponents beyond the residual's")
        _require(n <= N_MAX, what, f"rows of {n} beyond {N_MAX}")
        self.fr = int(fr[0])
        self._params, self.bcast = pblock(0, 0, 0, self.fr - fd, 0, n)

    def jobs(self):
        return [RoJob(opword(RO_ADDX, K_I32, K_I16, K_I32, b_en=True, p_bcast=self.bcast), self._params, self.n)]


@dataclass
class ResAddBiasRoNode(RowOpsAdapter):
    """A residual add with a per-channel bias (VitResAdd): h1 = sat32(h + (d << (fr - f_d)) +
    (Bq' << (fr - bb))), Bq' = round(bias 2^bb), bb = bias_bits(bias, fr); h int16 or int32
    at one exponent (rowops_nodes.py:1237-1280, _resadd_bias)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    bias: np.ndarray = None
    F: int = 8

    def __post_init__(self):
        h, d, y = self.inputs[0], self.inputs[1], self.output
        n, what = self.n, f"ResAddBias '{y.onnx_name}'"
        fr = _exps(y, self.F, n)
        fa = _exps(h, self.F, n)
        _require(y.kind == "i32" and (fr == fr[0]).all(), what, "the output: the int32 residual at one exponent")
        _require(h.kind == "i16" or (fa == fa[0]).all(), what, "an int32 h at one exponent")
        _require(d.kind == "i16" and d.shape[-1] == n and d.numel == h.numel == y.numel, what, "shapes")
        fd = _exps(d, self.F, n)
        fr = int(fr[0])
        _require((fa <= fr).all() and (fd <= fr).all() and (fr - fa <= 63).all() and (fr - fd <= 63).all(), what,
                 f"exponents beyond the residual's 2^-{fr}")
        bias = np.asarray(self.bias, np.float64).reshape(-1)
        _require(bias.size == n and np.isfinite(bias).all(), what, "bias [n]")
        self.fr, self.bb, self.a32 = fr, bias_bits(bias, fr), h.kind == "i32"
        bq = np.rint(bias * 2.0 ** self.bb).astype(np.int64)
        self._params, self.bcast = pblock(0, bq, fr - fa, fr - fd, 0, n)

    def jobs(self):
        op = opword(RO_ADDX, K_I32 if self.a32 else K_I16, K_I16, K_I32, b_en=True, p_bcast=self.bcast)
        return [RoJob(op, self._params, self.n, bq_sh=self.fr - self.bb)]


@dataclass
class WidenRoNode(RowOpsAdapter):
    """LlmWiden: int16 at per-channel exponents -> int32 at one exponent fy >= each, exact
    (one COPY, A << (fy - f[c]); rowops_nodes.py:498-539, from_llm_widen)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    F: int = 8

    def __post_init__(self):
        x, y = self.inputs[0], self.output
        n, what = self.n, f"Widen '{y.onnx_name}'"
        _require(x.kind == "i16" and y.kind == "i32" and y.numel == x.numel and y.shape[-1] == n, what, "shapes")
        fx, fy = _exps(x, self.F, n), _exps(y, self.F, n)
        _require((fy == fy[0]).all() and (fx <= fy[0]).all() and (fy[0] - fx <= 16).all(), what,
                 "one output exponent, at most 16 finer than each input's")
        self._params, self.bcast = pblock(0, 0, fy[0] - fx, 0, 0, n)

    def jobs(self):
        return [RoJob(opword(RO_COPY, K_I16, K_I16, K_I32, p_bcast=self.bcast), self._params, self.n)]


@dataclass
class SiluMulRoNode(RowOpsAdapter):
    """LlmSiluMul: a = silu(g) * u, g int16 at per-channel exponents <= 14, u and a at theirs,
    one MULACT job (rowops_nodes.py:540-563, from_llm_silu_mul)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    F: int = 8

    def __post_init__(self):
        g, u, y = self.inputs[0], self.inputs[1], self.output
        n, what = self.n, f"SiluMul '{y.onnx_name}'"
        for t in (g, u, y):
            _require(t.kind == "i16" and t.shape[-1] == n and t.numel == g.numel, what, "int16 tensors of one shape")
        fg, fu, fa = (_exps(t, self.F, n) for t in (g, u, y))
        _require((fg <= G_BITS).all(), what, f"gate exponents above {G_BITS}")
        sh_c = SILU_BITS + fu - fa
        _require((sh_c >= 0).all() and (sh_c <= 63).all(), what, "up / output exponents beyond the shifts")
        _require(n <= N_MAX, what, f"rows of {n} beyond {N_MAX}")
        self._params, self.bcast = pblock(0, 0, G_BITS - fg, 0, sh_c, n)

    def jobs(self):
        return [RoJob(opword(RO_MULACT, b_en=True, p_bcast=self.bcast), self._params, self.n)]


@dataclass
class DequantRoNode(RowOpsAdapter):
    """LlmDequant: int16 at per-channel exponents (or the int32 residual) -> float32
    raw * 2^-f[c], round to nearest even (exact below 2^24).  A single row longer than the
    unit's 4096 (the logits) runs as one job per contiguous chunk, each with the parameter
    block of its columns (rowops_nodes.py:2501-2612, from_llm_dequant)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    F: int = 8
    align_elems: int = 8

    def __post_init__(self):
        x, y = self.inputs[0], self.output
        n, what = self.n, f"Dequant '{y.onnx_name}'"
        _require(x.kind in ("i16", "i32") and y.kind == "f32" and y.numel == x.numel and y.shape[-1] == n, what,
                 "shapes / kinds")
        f = _exps(x, self.F, n)
        _require((f >= 0).all() and (f <= 63).all(), what, "exponents beyond the shifts")
        self.a32 = x.kind == "i32"
        if n <= N_MAX:
            pb, bc = pblock(0, 0, 0, 0, f, n)
            self._chunks = [(0, n, pb, bc)]
            return
        _require(x.numel == n, what, f"a row of {n} (> {N_MAX}): one row")
        nc = next((d for d in range(N_MAX, 0, -1) if n % d == 0 and d % self.align_elems == 0), 0)
        _require(nc > 0, what, f"a row of {n} has no divisor <= {N_MAX} that is a multiple of {self.align_elems}")
        self._chunks = [(k * nc, nc) + pblock(0, 0, 0, 0, f[k * nc:(k + 1) * nc], nc) for k in range(n // nc)]

    def jobs(self):
        ak = K_I32 if self.a32 else K_I16
        return [RoJob(opword(RO_DEQUANT, ak, K_I16, K_F32, p_bcast=bc), pb, nc, col0=c0)
                for c0, nc, pb, bc in self._chunks]


@dataclass
class BiasCopyRoNode(RowOpsAdapter):
    """A COPY with a per-column bias (the vision / TTS bias adds): y = sat16(rne((x << (fp -
    f_x)) + round(bias 2^fp), fp - f_out)), then ReLU with ``relu`` -- rowops_spec.bias_round
    (rowops_spec.py:199-208) with fp = bias_exp."""
    inputs: List[TensorInfo]
    output: TensorInfo
    bias: np.ndarray = None
    relu: bool = False
    F: int = 8

    def __post_init__(self):
        x, y = self.inputs[0], self.output
        n, what = self.n, f"BiasCopy '{y.onnx_name}'"
        _require(x.kind == "i16" and y.kind == "i16" and y.numel == x.numel and y.shape[-1] == n, what, "shapes")
        bias = np.asarray(self.bias, np.float64).reshape(-1)
        _require(bias.size == n and n <= N_MAX, what, "bias [n], rows of at most 4096")
        bq, sa, sc = bias_params(bias, _exps(x, self.F, n), _exps(y, self.F, n))
        self._params, self.bcast = pblock(0, bq, sa, 0, sc, n)

    def jobs(self):
        return [RoJob(opword(RO_COPY, relu=self.relu, p_bcast=self.bcast), self._params, self.n)]


@dataclass
class RopeRoNode(RowOpsAdapter):
    """Rotate-half RoPE of [T][nh * HD] rows (q or k) at per-head exponents into int16 at the
    output's per-head exponents, position pos + t for row t -- one ROPE job with the cos / sin
    table as B (rowops_spec.rope; the RoPE jobs of AttnPrepRoNode, rowops_nodes.py:1008-1014
    and from_llm_attn_prep's rope_params :1181-1191).  ``table`` is the float32 [C][HD/2]
    cos / sin pair.  ``same_pos``: every row at position pos (the rows of a batch of
    sequences decoding at one position; the job's B row stride 0)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    heads: int = 1
    head_dim: int = 16
    cos: np.ndarray = None
    sin: np.ndarray = None
    pos: int = 0
    F: int = 8
    same_pos: bool = False
    pos_t: Optional[TensorInfo] = None       # a runtime position (this host tensor's value) for pos
    table: Optional[TensorInfo] = field(default=None, init=False)

    def __post_init__(self):
        x, y = self.inputs[0], self.output
        nh, HD = self.heads, self.head_dim
        n, what = self.n, f"RoPE '{y.onnx_name}'"
        _require(n == nh * HD and HD % 2 == 0 and n <= N_MAX, what, f"rows of {nh} x {HD}")
        _require(x.kind == "i16" and y.kind == "i16" and y.numel == x.numel and y.shape[-1] == n, what, "shapes")
        fx = _exps(x, self.F, n).reshape(nh, HD)
        fo = _exps(y, self.F, n).reshape(nh, HD)
        half = HD // 2
        frot = np.concatenate([fx[:, half:], fx[:, :half]], axis=1)
        fp = np.maximum(fx, frot)
        sa, sb, sc = fp - fx, fp - frot, fp + ROPE_BITS - fo
        _require((sa <= 63).all() and (sb <= 63).all() and (sc >= 0).all() and (sc <= 63).all(), what,
                 "RoPE exponents beyond the shifts")
        tab = rope_table(self.cos, self.sin)
        self._span = 1 if self.same_pos else self.rows
        _require(tab.shape[1] == 2 * HD and 0 <= self.pos and self.pos + self._span <= tab.shape[0], what,
                 "cos / sin tables [C][HD/2] covering the rows' positions")
        self.table = TensorInfo(f"{y.onnx_name}__rope_table", list(tab.shape), data=tab, kind="i32", raw=True)
        self._params, self.bcast = pblock(0, 0, sa.reshape(-1), sb.reshape(-1), sc.reshape(-1), n)

    def jobs(self, pos: Optional[int] = None):
        """The job at the static position, or at ``pos`` (the runtime position's host value)."""
        p = self.pos if pos is None else int(pos)
        if self.pos_t is not None and pos is None:
            raise SchedulerError(f"RoPE '{self.output.onnx_name}': the runtime position needs its host value")
        if not 0 <= p or p + self._span > self.table.shape[0]:
            raise SchedulerError(f"RoPE '{self.output.onnx_name}': position {p} past the cos / sin tables")
        return [RoJob(opword(RO_ROPE, K_I16, K_I32, K_I16, b_en=True, p_bcast=self.bcast), self._params, self.n,
                      aux=self.head_dim, b_row0=p, b_same=self.same_pos)]


# ---------------------------------------------------------------- register-level job lists
@dataclass
class DecodePrepNode(KernelNode):
    """A decode step's attention prep, fused: RoPE of q [B][heads hd] into the output qr and of
    k [B][kv_heads hd] straight into the K cache rows at the step's position, v's rows into the V
    cache rows -- the two RopeRoNodes (same_pos) and the two KvWriteNodes of the unfused step, the
    same jobs' arithmetic (their parameter blocks and table row) in one launch.  inputs: q, k, v,
    kc, vc (caches [B][kv_heads][C][hd], written in place; k's RoPE output at kc's exponents and
    v at vc's); ``pos`` or the runtime ``pos_t``."""
    inputs: List[TensorInfo]
    output: TensorInfo
    heads: int = 1
    kv_heads: int = 1
    head_dim: int = 64
    cos: np.ndarray = None
    sin: np.ndarray = None
    pos: int = 0
    pos_t: Optional[TensorInfo] = None
    F: int = 8

    def __post_init__(self):
        q, k, v, kc, vc = self.inputs[:5]
        B, KV, C, HD = (int(x) for x in kc.shape)
        what = f"decode prep '{self.output.onnx_name}'"
        _require(list(vc.shape) == [B, KV, C, HD] and KV == self.kv_heads and HD == self.head_dim
                 and list(q.shape) == [B, self.heads * HD] and list(k.shape) == [B, KV * HD]
                 and list(v.shape) == [B, KV * HD] and list(self.output.shape) == list(q.shape), what, "shapes")
        _require(HD % 16 == 0 and HD <= 128, what, "a head dim of a multiple of 16 up to 128")
        fk, fv = np.asarray(_exps(kc, self.F, 1)).reshape(-1), np.asarray(_exps(vc, self.F, 1)).reshape(-1)
        _require((fk == fk[0]).all() and (fv == fv[0]).all(), what, "the caches at one exponent each")
        _require((_exps(v, self.F, KV * HD) == fv[0]).all(), what, "v at the V cache's exponent")
        self.rope_q = RopeRoNode([q], self.output, heads=self.heads, head_dim=HD, cos=self.cos, sin=self.sin,
                                 pos=self.pos, F=self.F, same_pos=True, pos_t=self.pos_t)
        kr = TensorInfo(self.output.onnx_name + "__k_rope", [B, KV * HD], exp=int(fk[0]))
        self.rope_k = RopeRoNode([k], kr, heads=KV, head_dim=HD, cos=self.cos, sin=self.sin, pos=self.pos, F=self.F,
                                 same_pos=True, pos_t=self.pos_t)

    def position(self, host: Optional[int] = None) -> int:
        if self.pos_t is not None:
            if host is None:
                raise SchedulerError(f"decode prep '{self.output.onnx_name}': the runtime position needs its host value")
            return int(host)
        return self.pos


@dataclass
class RoCall:
    """One run_rowops call (rowops_nodes.py:143-151): the register block, each stream's buffer
    named -- a graph tensor's onnx_name, or a staging buffer of the node ("node:<key>") -- with
    its byte offset; ``p`` the parameter block bytes (None: the job reads none)."""
    a: Optional[str]
    a_off: int
    b: Optional[str]
    b_off: int
    c: str
    c_off: int
    p: Optional[np.ndarray]
    op: int
    n: int
    rows: int
    blocks: int
    a_s1: int
    a_s2: int
    b_s1: int
    b_s2: int
    c_s1: int
    c_s2: int
    eps: int = 0
    aux: int = 0
    bq_sh: int = 0
    win_lo: int = 0
    win_hi: int = NO_WINDOW


class RoCallNode(KernelNode):
    """Base of the nodes that lower to explicit unit calls over named buffers: ``staging()``
    the node's own buffers {key: bytes} (zero at creation, kept from call to call like the
    reference's DMA states), ``tables()`` constant buffers {key: raw lanes}, ``calls(host)``
    the jobs in order for the runtime host values {onnx_name: int} (pos, n)."""
    inputs: List[TensorInfo]
    output: TensorInfo

    def staging(self):
        return {}

    def tables(self):
        return {}

    def calls(self, host) -> List[RoCall]:
        raise NotImplementedError

    def host_inputs(self) -> List[TensorInfo]:
        return [t for t in self.inputs if t is not None and t.kind == "host"]


ZERO_PARAMS = param_block(0, 0, 0, 0, 0)        # one broadcast entry: COPY as an exact copy


def collapse(dims: Sequence[int], sstr: Sequence[int]):
    """Adjacent output dims that are adjacent in the source merged, size-1 dims dropped, left-
    padded to 5 dims (host_nodes._collapse, host_nodes.py:129-148)."""
    d, st = [], []
    for di, si in zip(dims, sstr):
        if di == 1:
            continue
        if d and st[-1] == si * di:
            d[-1] *= di
            st[-1] = si
        else:
            d.append(int(di))
            st.append(int(si))
    if not d:
        d, st = [1], [1]
    if len(d) > 5:
        raise SchedulerError(f"transpose: {len(d)} non-mergeable dimensions (max 5)")
    pad = 5 - len(d)
    return [1] * pad + d, [0] * pad + st


def transpose_job(dims: Sequence[int], sstr: Sequence[int], elem_bytes: int = 2):
    """The unit job of a collapsed transpose, or None where the unit cannot run it
    (rowops_nodes.transpose_job, rowops_nodes.py:337-366): (kind, n, rows, blocks, strides
    (a_s1, a_s2, b_s1, b_s2, c_s1, c_s2) in bytes).  [D2][D1][n] from source strides
    [n, D2 n, 1] is one COPY of n-element rows; [B][L][M] from strides [sB, 1, sM] one
    TRANSPOSE of 8-row tiles into granules at the output's row stride."""
    d = [(int(a), int(b)) for a, b in zip(dims, sstr) if a != 1]
    if elem_bytes != 2 or not d or len(d) > 3:
        return None
    al = 16 // elem_bytes
    if d[-1][1] == 1:
        if len(d) == 1:
            return None
        if len(d) == 2:
            d = [(1, 0)] + d
        (D2, s2), (D1, s1), (n, _) = d
        if n % al or s1 % al or s2 % al or n > N_MAX:
            return None
        return ("copy", n, D1, D2, (s1 * elem_bytes, s2 * elem_bytes, 0, 0, n * elem_bytes, D1 * n * elem_bytes))
    if len(d) == 2:
        d = [(1, 0)] + d
    (B, sB), (L, sL), (M, sM) = d
    if sL != 1 or M % QIMAGE_R or sM % al or sB % al or L > 1024:
        return None
    return ("xpose", L, M // QIMAGE_R, B, (QIMAGE_R * sM * elem_bytes, sB * elem_bytes, sM * elem_bytes,
                                           M * elem_bytes, QIMAGE_R * elem_bytes, L * M * elem_bytes))


@dataclass
class TransposeRoNode(RoCallNode):
    """An ONNX Transpose of an int16 tensor as one unit job, a bit copy (rowops_nodes.py:265-335,
    from_onnx_transpose :369-387): the output dims collapsed against the input's row-major
    strides (host TransposeNode, host_nodes.py:1265-1292), then a COPY (the outer axes swapped,
    rows kept: head split / merge) or a TRANSPOSE (K^T).  Other shapes raise SchedulerError
    (the reference keeps them on the host)."""
    inputs: List[TensorInfo]
    output: TensorInfo
    perm: Sequence[int] = ()

    def __post_init__(self):
        x, y = self.inputs[0], self.output
        rank = len(x.shape)
        what = f"Transpose '{y.onnx_name}'"
        self.perm = [int(p) for p in (self.perm if len(self.perm) else range(rank - 1, -1, -1))]
        _require(sorted(self.perm) == list(range(rank)), what, f"bad perm {self.perm}")
        _require(list(y.shape) == [x.shape[p] for p in self.perm], what, "output shape")
        _require(x.kind == "i16" and y.kind == "i16", what, "int16 tensors")
        st = [int(np.prod(x.shape[i + 1:])) for i in range(rank)]
        self.dims, self.sstr = collapse([int(x.shape[p]) for p in self.perm], [st[p] for p in self.perm])
        job = transpose_job(self.dims, self.sstr)
        _require(job is not None, what, f"collapsed dims {self.dims} / strides {self.sstr}: not a unit job")
        self.kind, self.n_, self.rows_, self.blocks, self.strides = job

    def calls(self, host=None):
        x, y = self.inputs[0].onnx_name, self.output.onnx_name
        s = self.strides
        if self.kind == "copy":
            return [RoCall(x, 0, None, 0, y, 0, ZERO_PARAMS, opword(RO_COPY, p_bcast=True), self.n_, self.rows_,
                           self.blocks, s[0], s[1], s[2], s[3], s[4], s[5])]
        return [RoCall(x, 0, None, 0, y, 0, None, opword(RO_XPOSE), self.n_, self.rows_, self.blocks, s[0], s[1],
                       s[2], s[3], s[4], s[5], aux=QIMAGE_R)]


@dataclass
class AttnPrepRoNode(RoCallNode):
    """LlmAttnPrep on the unit (rowops_nodes.py:893-1236, from_llm_attn_prep :1134-1219): for
    one sequence's rows t < n at positions pos + t -- RoPE of q0 into the q staging rows at the
    per-head exponents ``fq`` and of k0 at the K cache's, v re-rounded where the V cache's
    exponents differ, the q.K^T x image qx [KV][HD][G T] (x_g[d][h' T + t] = q[t][g G + h'][d])
    by TRANSPOSE, and the k / v rows into the group-major caches [KV][C][HD] in place.

    inputs [q0 [T][H HD], k0 [T][KV HD], v [T][KV HD], pos (host), n (host, optional: a
    decode step has n = T = 1), cache_k, cache_v]; the output qx holds raw integers (the
    contraction's input image, llm_nodes.py:1015), i.e. a tensor at exponent 0.  The q staging rows are
    zeroed each call, so qx's columns t >= n are 0.  The V cache without interleave (the
    reference's group_kw 1); head_dim 16 .. 128, T a multiple of 8 or one row with at most 8
    heads per group."""
    inputs: List[TensorInfo]
    output: TensorInfo
    heads: int = 1
    kv_heads: int = 1
    head_dim: int = 16
    fq: Optional[np.ndarray] = None
    cos: Optional[np.ndarray] = None
    sin: Optional[np.ndarray] = None
    key_quantum: int = KEY_QUANTUM
    F: int = 8

    @property
    def has_n(self) -> bool:
        return len(self.inputs) == 7

    def __post_init__(self):
        H, KV, HD = self.heads, self.kv_heads, self.head_dim
        what = f"AttnPrep '{self.output.onnx_name}'"
        _require(len(self.inputs) in (6, 7), what, "inputs q0, k0, v, pos, [n], cache_k, cache_v")
        q0, k0, v, pos = self.inputs[:4]
        ck, cv = self.inputs[-2], self.inputs[-1]
        _require(H % KV == 0, what, "heads a multiple of the KV heads")
        G = H // KV
        T = q0.numel // (H * HD)
        _require(self.has_n or T == 1, what, "n may be left out only in a decode step (one row)")
        _require(HD % 16 == 0 and 16 <= HD <= 128, what, f"head_dim {HD}: 16 .. 128, a multiple of 16")
        _require(H * HD <= N_MAX and KV * HD <= N_MAX, what, f"rows beyond {N_MAX}")
        _require(T % QIMAGE_R == 0 or (T == 1 and G <= QIMAGE_R), what,
                 f"rows {T} % {QIMAGE_R}, or one row with at most {QIMAGE_R} heads per group")
        C = int(ck.shape[0])
        _require(C % self.key_quantum == 0, what, "cache rows a multiple of the key quantum")
        _require(q0.numel == T * H * HD and k0.numel == T * KV * HD and v.numel == k0.numel, what, "q / k / v shapes")
        _require(list(self.output.shape) == [KV, HD, G * T], what, f"qx must be [{KV}][{HD}][{G * T}]")
        _require(self.output.exp is not None and (np.asarray(self.output.exp) == 0).all(), what,
                 "qx holds raw integers: exponent 0")
        for t, nm in ((q0, "q0"), (k0, "k0"), (v, "v"), (self.output, "qx")):
            _require(t.kind == "i16", what, f"{nm}: an int16 tensor")
        _require(pos.kind == "host" and (not self.has_n or self.inputs[4].kind == "host"), what,
                 "pos / n: host tensors")
        for t, nm in ((ck, "cache_k"), (cv, "cache_v")):
            _require(t.kind == "i16" and t.group_layout == (KV, HD) and list(t.shape) == [C, KV * HD], what,
                     f"{nm}: logical [{C}][{KV * HD}], stored group-major [{KV}][{C}][{HD}]")
        self.T, self.G, self.C = T, G, C
        self.fq = np.asarray(self.fq, np.int64).reshape(-1)
        _require(self.fq.size == H, what, "q_exp: one exponent per head")
        cos = np.asarray(self.cos, np.float32)
        sin = np.asarray(self.sin, np.float32)
        _require(cos.shape == (C, HD // 2) and sin.shape == cos.shape, what, f"cos / sin [{C}][{HD // 2}]")
        self._table = rope_table(cos, sin)                                   # [C][2 HD] int32

        def rope_params(t, nh, f_out):
            fx = _exps(t, self.F, nh * HD).reshape(nh, HD)
            half = HD // 2
            frot = np.concatenate([fx[:, half:], fx[:, :half]], axis=1)
            fp = np.maximum(fx, frot)
            fo = np.broadcast_to(np.asarray(f_out, np.int64).reshape(nh, -1), (nh, HD))
            sa, sb, sc = fp - fx, fp - frot, fp + ROPE_BITS - fo
            _require((sa >= 0).all() and (sa <= 63).all() and (sb <= 63).all() and (sc >= 0).all()
                     and (sc <= 63).all(), what, "RoPE exponents beyond the shifts")
            return sa.reshape(-1), sb.reshape(-1), sc.reshape(-1)

        fkc = _exps(ck, self.F, KV * HD).reshape(KV, HD)
        _require((fkc == fkc[:, :1]).all(), what, "the K cache's exponent must be one per KV head")
        self._pq, self._pq_bc = pblock(0, 0, *rope_params(q0, H, self.fq), H * HD)
        self._pk, self._pk_bc = pblock(0, 0, *rope_params(k0, KV, fkc[:, 0]), KV * HD)
        fv, fvc = _exps(v, self.F, KV * HD), _exps(cv, self.F, KV * HD)
        self.v_direct = bool((fv == fvc).all())
        if not self.v_direct:
            sa_v, sc_v = np.maximum(fvc - fv, 0), np.maximum(fv - fvc, 0)
            _require((sa_v <= 63).all() and (sc_v <= 63).all(), what, "v / V cache exponents beyond the shifts")
            self._pv, self._pv_bc = pblock(0, 0, sa_v, 0, sc_v, KV * HD)

    def staging(self):
        T, nq, nk = self.T, self.heads * self.head_dim, self.kv_heads * self.head_dim
        st = {"qs": T * nq * 2, "ks": T * nk * 2}
        if not self.v_direct:
            st["vs"] = T * nk * 2
        return st

    def tables(self):
        return {"rope": self._table}

    def calls(self, host):
        """The jobs of AttnPrepRoNode._jobs (rowops_nodes.py:997-1047) for this call's pos / n."""
        T, KV, HD, C, G = self.T, self.kv_heads, self.head_dim, self.C, self.G
        nq, nk = self.heads * HD, KV * HD
        q0, k0, v, pos_t = (t.onnx_name for t in self.inputs[:4])
        ck, cv, qx = self.inputs[-2].onnx_name, self.inputs[-1].onnx_name, self.output.onnx_name
        pos = int(host[pos_t])
        n_in = int(host[self.inputs[4].onnx_name]) if self.has_n else T
        n, _keys = attn_keys(pos, n_in, T, C, self.key_quantum)
        sq, sk, sv = nq * 2, nk * 2, nk * 2                  # the inputs' row strides (contiguous rows)
        sqs, sks = nq * 2, nk * 2
        copy0 = opword(RO_COPY, p_bcast=True)
        rope = opword(RO_ROPE, K_I16, K_I32, K_I16, b_en=True)
        jobs = [RoCall("node:qs", 0, None, 0, "node:qs", 0, ZERO_PARAMS, copy0, nq, T, 1, sqs, 0, 0, 0, sqs, 0,
                       win_lo=0, win_hi=0)]                 # the staging rows zeroed: rows >= n stay 0
        if n > 0:
            bo = pos * 8 * HD                                # the table row of position pos
            jobs.append(RoCall(q0, 0, "node:rope", bo, "node:qs", 0, self._pq, rope | (F_P_BCAST if self._pq_bc else 0),
                               nq, n, 1, sq, 0, 8 * HD, 0, sqs, 0, aux=HD))
            jobs.append(RoCall(k0, 0, "node:rope", bo, "node:ks", 0, self._pk, rope | (F_P_BCAST if self._pk_bc else 0),
                               nk, n, 1, sk, 0, 8 * HD, 0, sks, 0, aux=HD))
            if self.v_direct:
                vsrc, svs = v, sv
            else:
                vsrc, svs = "node:vs", sks
                jobs.append(RoCall(v, 0, None, 0, "node:vs", 0, self._pv, opword(RO_COPY, p_bcast=self._pv_bc), nk,
                                   n, 1, sv, 0, 0, 0, sks, 0))
        xpose = opword(RO_XPOSE)
        if T == 1:                                           # the group's heads as the tile's rows
            jobs.append(RoCall("node:qs", 0, None, 0, qx, 0, None, xpose, HD, 1, KV, 0, G * HD * 2, HD * 2, 2 * G,
                               0, HD * G * 2, aux=G))
        else:
            for g in range(KV):
                jobs.append(RoCall("node:qs", g * G * HD * 2, None, 0, qx, g * HD * G * T * 2, None, xpose, HD,
                                   T // QIMAGE_R, G, QIMAGE_R * sqs, HD * 2, sqs, 2 * G * T, 2 * QIMAGE_R, 2 * T,
                                   aux=QIMAGE_R))
        if n > 0:
            co = pos * HD * 2
            jobs.append(RoCall("node:ks", 0, None, 0, ck, co, ZERO_PARAMS, copy0, HD, n, KV, sks, HD * 2, 0, 0,
                               HD * 2, C * HD * 2))
            jobs.append(RoCall(vsrc, 0, None, 0, cv, co, ZERO_PARAMS, copy0, HD, n, KV, svs, HD * 2, 0, 0,
                               HD * 2, C * HD * 2))
        return jobs


@dataclass
class VitAttnPrepRoNode(RoCallNode):
    """VitAttnPrep on the unit (rowops_nodes.py:1415-1593, from_vit_attn_prep :1596-1712): an
    encoder's attention prep with every key valid (T = C rows, position 0, static jobs) --

      * q0 + bq rounded at the per-head exponents ``fq`` into the staging rows, then one
        TRANSPOSE (8-row tiles, the heads as blocks) into the q.K^T image qx [H][HD][T];
      * per head, k0 + bk at that head's exponent ``fk`` straight into the K cache rows;
      * v + bv at the V cache's exponents ``fv`` (per column) into staging, then one COPY into
        the V cache rows (the heads as blocks).

    Each add is a COPY with a bias (rowops_spec.bias_round: sat16(rne_shr((x << (fp - f_x)) +
    round(b 2^fp), fp - f_out)), the bias rounded once at 2^-fp); no bias rounds x alone.  The
    caches are raw states (exponent 0) stored group-major [H][C][HD]; qx holds raw integers.
    ``query_major``: q and k swap roles (k takes the image path, q the cache rows), so the
    scores come out query-major.

    inputs [q0, k0, v, cache_k, cache_v]: q0 / k0 / v rows of T, each read from column ``cols[i]``
    of its tensor's rows (one fused projection [T][3 D] may serve all three).  The V cache
    without interleave (the reference's group_kw 1); head_dim a multiple of 16, T a multiple
    of 8."""
    inputs: List[TensorInfo]
    output: TensorInfo
    heads: int = 1
    head_dim: int = 16
    fq: Optional[np.ndarray] = None
    fk: Optional[np.ndarray] = None
    fv: Optional[np.ndarray] = None
    bq: Optional[np.ndarray] = None
    bk: Optional[np.ndarray] = None
    bv: Optional[np.ndarray] = None
    cols: tuple = (0, 0, 0)
    query_major: bool = False
    F: int = 8

    def __post_init__(self):
        H, HD = self.heads, self.head_dim
        D = H * HD
        what = f"VitAttnPrep '{self.output.onnx_name}'"
        _require(len(self.inputs) == 5, what, "inputs q0, k0, v, cache_k, cache_v")
        ck, cv = self.inputs[3], self.inputs[4]
        _require(HD % 16 == 0 and 16 <= HD <= 1024 and D <= N_MAX, what, f"head_dim {HD}: a multiple of 16")
        C = int(ck.shape[0])
        self.T = T = C
        _require(T % QIMAGE_R == 0, what, f"rows {T} % {QIMAGE_R} (the q image's tiles)")
        for i, (t, nm) in enumerate(zip(self.inputs[:3], ("q0", "k0", "v"))):
            w = int(t.shape[-1])
            _require(t.kind == "i16" and t.numel == T * w and 0 <= self.cols[i] and self.cols[i] + D <= w
                     and self.cols[i] % 8 == 0 and w % 8 == 0, what,
                     f"{nm}: int16 rows of {T} holding {D} columns from column {self.cols[i]} (16-byte aligned)")
        for t, nm in ((ck, "cache_k"), (cv, "cache_v")):
            _require(t.kind == "i16" and t.state and t.group_layout == (H, HD) and list(t.shape) == [T, D]
                     and (np.asarray(0 if t.exp is None else t.exp) == 0).all(), what,
                     f"{nm}: a raw state (exponent 0), logical [{T}][{D}] stored group-major [{H}][{T}][{HD}]")
        _require(list(self.output.shape) == [H, HD, T] and self.output.kind == "i16"
                 and (np.asarray(0 if self.output.exp is None else self.output.exp) == 0).all(), what,
                 f"qx: raw integers [{H}][{HD}][{T}]")
        fq = np.broadcast_to(np.asarray(self.fq, np.int64).reshape(-1), (H,))
        fk = np.broadcast_to(np.asarray(self.fk, np.int64).reshape(-1), (H,))
        self.fq, self.fk = fq.copy(), fk.copy()
        self.fv = np.broadcast_to(np.asarray(self.fv, np.int64).reshape(-1), (D,)).copy()
        zero = np.zeros(D)
        bq, bk, bv = (zero if b is None else np.asarray(b, np.float64).reshape(-1) for b in (self.bq, self.bk, self.bv))
        _require(bq.size == D and bk.size == D and bv.size == D, what, f"biases of {D} columns")
        q0, k0 = self.inputs[0], self.inputs[1]
        cq, ckc = self.cols[0], self.cols[1]
        if self.query_major:             # k the image path, q the cache rows
            q0, k0, bq, bk, fq, fk, cq, ckc = k0, q0, bk, bq, fk, fq, ckc, cq
        self._img, self._rows = (q0, cq), (k0, ckc)

        def params(x, col, bias, f_out):
            fx = _exps(x, self.F, int(x.shape[-1]))[col:col + D]
            try:
                b, sa, sc = bias_params(bias, fx, f_out)
            except SchedulerError as e:
                raise SchedulerError(f"{what}: {e}") from None
            _require((sa >= 0).all() and (sa <= 63).all() and (sc >= 0).all() and (sc <= 63).all(), what,
                     "exponents beyond the shifts")
            return b, sa, sc

        b, sa, sc = params(q0, cq, bq, np.repeat(fq, HD))
        self._pq, self._pq_bc = pblock(0, b, sa, 0, sc, D)
        b, sa, sc = params(k0, ckc, bk, np.repeat(fk, HD))
        self._pk = [param_block(np.zeros(HD, np.int64), b[h * HD:(h + 1) * HD], sa[h * HD:(h + 1) * HD], 0,
                                sc[h * HD:(h + 1) * HD]) for h in range(H)]
        b, sa, sc = params(self.inputs[2], self.cols[2], bv, self.fv)
        self._pv, self._pv_bc = pblock(0, b, sa, 0, sc, D)

    def staging(self):
        D2 = self.heads * self.head_dim * 2
        return {"qs": self.T * D2, "vs": self.T * D2}

    def calls(self, host):
        T, H, HD = self.T, self.heads, self.head_dim
        D = H * HD
        SQ = D * 2
        (img, ci), (rows_t, cr), v = self._img, self._rows, self.inputs[2]
        stride = lambda t: int(t.shape[-1]) * 2                                   # noqa: E731
        ck, cv, qx = self.inputs[3].onnx_name, self.inputs[4].onnx_name, self.output.onnx_name
        jobs = [RoCall(img.onnx_name, ci * 2, None, 0, "node:qs", 0, self._pq, opword(RO_COPY, p_bcast=self._pq_bc),
                       D, T, 1, stride(img), 0, 0, 0, SQ, 0),
                RoCall("node:qs", 0, None, 0, qx, 0, None, opword(RO_XPOSE), HD, T // QIMAGE_R, H, QIMAGE_R * SQ,
                       HD * 2, SQ, 2 * T, 2 * QIMAGE_R, HD * T * 2, aux=QIMAGE_R)]
        for h in range(H):
            jobs.append(RoCall(rows_t.onnx_name, (cr + h * HD) * 2, None, 0, ck, h * T * HD * 2, self._pk[h],
                               opword(RO_COPY), HD, T, 1, stride(rows_t), 0, 0, 0, HD * 2, 0))
        jobs.append(RoCall(v.onnx_name, self.cols[2] * 2, None, 0, "node:vs", 0, self._pv,
                           opword(RO_COPY, p_bcast=self._pv_bc), D, T, 1, stride(v), 0, 0, 0, SQ, 0))
        jobs.append(RoCall("node:vs", 0, None, 0, cv, 0, ZERO_PARAMS, opword(RO_COPY, p_bcast=True), HD, T, H, SQ,
                           HD * 2, 0, 0, HD * 2, T * HD * 2))
        return jobs


ADAPTERS = (LayerNormRoNode, LayerNorm32RoNode, RMSNormRoNode, ResAddRoNode, ResAddBiasRoNode, WidenRoNode,
            SiluMulRoNode, DequantRoNode, BiasCopyRoNode, RopeRoNode)

__all__ = ["RoJob", "RowOpsAdapter", "RoCall", "RoCallNode", "TransposeRoNode", "AttnPrepRoNode", "VitAttnPrepRoNode",
           "collapse",
           "transpose_job", "opword", "gamma_scale", "beta_bits", "bias_bits", "quant_bias", "bias_exp",
           "bias_params", "norm_params", "param_block", "pblock", "rope_tables_raw", "rope_table"] + \
          [c.__name__ for c in ADAPTERS]
