"""Graph builders for the benchmark workloads, with seeded synthetic weights.

small_cnn -- batch 1, Q8.8 throughout: Conv 3x3 1->8 pad 1 + bias -> ReLU -> MaxPool 2x2 ->
Conv 3x3 8->16 pad 1 + bias -> ReLU -> MaxPool 2x2 -> flatten 784 -> MatMul 784x10 -> Add
bias -> Softmax (row mode, regs(8, 1.0, 8)).  Weights U(+-0.25), biases U(+-0.1); the
input U[0, 1).  The node kinds are the reference's mapping of this network
(ConvNode, ScheduledNode RELU, PoolNode MAX, ReshapeNode, MatmulNode, ScheduledNode ADD,
SoftmaxVopNode; _simulate.py:617-765).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import units
from .graph import (AttentionNode, AttnContractNode, ConvNode, DecodeAttentionNode, Graph, HeadView, MatmulNode,
                    PoolNode, ReshapeNode, ScheduledNode, SoftmaxVopNode, TensorInfo, conv_out, softmax_regs)
from .host_ops import LlmEmbedNode
from .rowops_nodes import LayerNorm32RoNode, ResAddBiasRoNode


def small_cnn(seed: int = 0, as_ops: bool = False):
    """(graph, inputs): the small CNN and one seeded input image.  ``as_ops``: instead of the
    graph, (ops, tensors, inputs, outputs) -- the network as the reference's ONNX ops for the
    front end (frontend.build_graph), over the same seeded tensors."""
    rng = np.random.default_rng(seed)
    T = TensorInfo
    x = T("input", [1, 1, 28, 28])
    w1 = T("conv1.w", [8, 1, 3, 3], data=rng.uniform(-0.25, 0.25, (8, 1, 3, 3)))
    b1 = T("conv1.b", [8], data=rng.uniform(-0.1, 0.1, 8))
    c1 = T("conv1", [1, 8, 28, 28])
    r1 = T("relu1", [1, 8, 28, 28])
    p1 = T("pool1", [1, 8, 14, 14])
    w2 = T("conv2.w", [16, 8, 3, 3], data=rng.uniform(-0.25, 0.25, (16, 8, 3, 3)))
    b2 = T("conv2.b", [16], data=rng.uniform(-0.1, 0.1, 16))
    c2 = T("conv2", [1, 16, 14, 14])
    r2 = T("relu2", [1, 16, 14, 14])
    p2 = T("pool2", [1, 16, 7, 7])
    fl = T("flat", [1, 784])
    wf = T("fc.w", [784, 10], data=rng.uniform(-0.25, 0.25, (784, 10)))
    mm = T("fc", [1, 10])
    bf = T("fc.b", [10], data=rng.uniform(-0.1, 0.1, 10))
    ad = T("logits", [1, 10])
    sm = T("probs", [1, 10])
    nodes = [
        ConvNode([x, w1, b1], c1, pad_top=1, pad_left=1),
        ScheduledNode([c1], r1, units.OP_RELU),
        PoolNode([r1], p1, units.POOL_MAX, 2, 2, 2, 2),
        ConvNode([p1, w2, b2], c2, pad_top=1, pad_left=1),
        ScheduledNode([c2], r2, units.OP_RELU),
        PoolNode([r2], p2, units.POOL_MAX, 2, 2, 2, 2),
        ReshapeNode([p2], fl),
        MatmulNode([fl, wf], mm),
        ScheduledNode([mm, bf], ad, units.OP_ADD),
        SoftmaxVopNode([ad], sm),
    ]
    g = Graph(nodes, input_tensors=[x], output_tensors=[sm])
    inputs = {"input": np.round(rng.uniform(0.0, 1.0, (1, 1, 28, 28)) * 256) / 256}
    if as_ops:
        from .frontend import OpDesc as O
        ops = [O("Conv", ["input", "conv1.w", "conv1.b"], ["conv1"], {"pads": [1, 1, 1, 1]}),
               O("Relu", ["conv1"], ["relu1"]),
               O("MaxPool", ["relu1"], ["pool1"], {"kernel_shape": [2, 2], "strides": [2, 2]}),
               O("Conv", ["pool1", "conv2.w", "conv2.b"], ["conv2"], {"pads": [1, 1, 1, 1]}),
               O("Relu", ["conv2"], ["relu2"]),
               O("MaxPool", ["relu2"], ["pool2"], {"kernel_shape": [2, 2], "strides": [2, 2]}),
               O("Flatten", ["pool2"], ["flat"]),
               O("MatMul", ["flat", "fc.w"], ["fc"]),
               O("Add", ["fc", "fc.b"], ["logits"]),
               O("Softmax", ["logits"], ["probs"], {"axis": -1})]
        return (ops, {t.onnx_name: t for t in [x, w1, b1, c1, r1, p1, w2, b2, c2, r2, p2, fl, wf, mm, bf, ad, sm]},
                ["input"], ["probs"]), inputs
    return g, inputs


# ---------------------------------------------------------------- MobileNetV2-style CNN
# (expansion t, output channels c, repeats n, first stride s) of the 17 inverted residual blocks
MOBILENET_V2_BLOCKS = ((1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1),
                       (6, 160, 3, 2), (6, 320, 1, 1))


def mobilenet_v2(batch: int = 32, res: int = 224, seed: int = 0, classes: int = 1000, as_ops: bool = False):
    """(graph, inputs, macs): MobileNetV2 1.0 in Q8.8, NCHW, batch ``batch`` at ``res`` x ``res``.

    Stem Conv 3x3 s2 3->32 pad 1 + RELU6; the 17 inverted residual blocks (1x1 expand x t +
    RELU6 where t > 1, depthwise 3x3 stride s pad 1 + RELU6, 1x1 project, residual ADD where
    stride 1 and the channels match); Conv 1x1 320->1280 + RELU6; global AVG pool over the
    final plane; flatten; MatMul 1280 x ``classes``.  The node kinds are the reference's
    mapping of these ONNX ops (Conv -> ConvNode, Clip(0, 6) -> VectorOP RELU6, Add -> VectorOP
    ADD, GlobalAveragePool -> PoolNode AVG, Flatten -> ReshapeNode, MatMul -> MatmulNode;
    graph.py:1005-1069, _simulate.py:617-765).  Convolutions carry no bias (a folded
    batch-norm's bias is a plain VectorOP ADD in the reference's mapping, left out here).

    He-normal weights (std sqrt(2 / fan_in)), the input U[0, 1); every tensor Q8.8.  Weights
    come from their own generator, so a smaller batch of the same seed is the leading images
    of a larger one.  ``macs`` counts the convolutions' and the classifier's multiply-adds.
    ``as_ops``: (ops, tensors, inputs, outputs) -- the reference's ONNX ops (Conv, Clip(0, 6),
    Add, GlobalAveragePool, Flatten, MatMul) over the same tensors -- in place of the graph."""
    from .frontend import OpDesc
    T = TensorInfo
    rng_in = np.random.default_rng([seed, 0])
    x_val = np.round(rng_in.random((batch, 3, res, res)) * 256) / 256
    rng = np.random.default_rng([seed, 1])
    nodes, macs, ops, reg = [], [0], [], {}
    x_t = T("input", [batch, 3, res, res])
    reg["input"] = x_t
    cur = x_t
    count = [0]

    def op(kind, ins, out, **attrs):
        for t in list(ins) + [out]:
            reg[t.onnx_name] = t
        ops.append(OpDesc(kind, [t.onnx_name for t in ins], [out.onnx_name], attrs))

    def name(tag):
        count[0] += 1
        return f"n{count[0]}.{tag}"

    def conv(x, cout, k, stride, depthwise=False):
        cin, h, w = x.shape[1], x.shape[2], x.shape[3]
        pad = k // 2
        oh, ow = conv_out(h, k, stride, pad, pad), conv_out(w, k, stride, pad, pad)
        fan_in = (1 if depthwise else cin) * k * k
        wt = T(name("w"), [cout, 1 if depthwise else cin, k, k],
               data=rng.standard_normal((cout, 1 if depthwise else cin, k, k)) * math.sqrt(2.0 / fan_in))
        y = T(name("conv"), [batch, cout, oh, ow])
        nodes.append(ConvNode([x, wt], y, stride_h=stride, stride_w=stride, pad_top=pad, pad_left=pad,
                              is_depthwise=depthwise))
        op("Conv", [x, wt], y, strides=[stride, stride], pads=[pad] * 4, group=cout if depthwise else 1)
        macs[0] += batch * cout * oh * ow * fan_in
        return y

    def relu6(x):
        y = T(name("relu6"), list(x.shape))
        nodes.append(ScheduledNode([x], y, units.OP_RELU6))
        op("Clip", [x], y, min=0.0, max=6.0)
        return y

    cur = relu6(conv(cur, 32, 3, 2))
    for t, c, n, s in MOBILENET_V2_BLOCKS:
        for i in range(n):
            stride = s if i == 0 else 1
            inp = cur
            h = inp
            if t != 1:
                h = relu6(conv(h, inp.shape[1] * t, 1, 1))
            h = relu6(conv(h, h.shape[1], 3, stride, depthwise=True))
            h = conv(h, c, 1, 1)
            if stride == 1 and inp.shape[1] == c:
                y = T(name("add"), list(h.shape))
                nodes.append(ScheduledNode([h, inp], y, units.OP_ADD))
                op("Add", [h, inp], y)
                h = y
            cur = h
    cur = relu6(conv(cur, 1280, 1, 1))
    pooled = T("pool", [batch, 1280, 1, 1])
    nodes.append(PoolNode([cur], pooled, units.POOL_AVG, cur.shape[2], cur.shape[3], 1, 1))
    op("GlobalAveragePool", [cur], pooled)
    flat = T("flat", [batch, 1280])
    nodes.append(ReshapeNode([pooled], flat))
    op("Flatten", [pooled], flat)
    wf = T("fc.w", [1280, classes], data=rng.standard_normal((1280, classes)) * math.sqrt(2.0 / 1280))
    logits = T("logits", [batch, classes])
    nodes.append(MatmulNode([flat, wf], logits))
    op("MatMul", [flat, wf], logits)
    macs[0] += batch * 1280 * classes
    if as_ops:
        return (ops, reg, ["input"], ["logits"]), {"input": x_val}, macs[0]
    return Graph(nodes, input_tensors=[x_t], output_tensors=[logits]), {"input": x_val}, macs[0]


# ---------------------------------------------------------------- BERT-base-shaped encoder
RES_BITS = 15        # the int32 residual's exponent (graph_builder.py:35)
F_Q88 = 8            # the element grid of Q8.8 tensors (the activation unit's input)


def _fit_exp(maxabs: float, margin: float = 1.25, lo: int = -8, hi: int = 24) -> int:
    """The largest f with maxabs * margin * 2^f <= 32767 (a per-tensor pow2 exponent)."""
    if maxabs <= 0:
        return hi
    return int(max(lo, min(hi, math.floor(math.log2(32767.0 / (maxabs * margin))))))


def _gelu(x):
    return x * 0.5 * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))


def _layer_norm(h, gamma, beta, eps):
    mu = h.mean(axis=-1, keepdims=True)
    var = ((h - mu) ** 2).mean(axis=-1, keepdims=True)
    return (h - mu) / np.sqrt(var + eps) * gamma + beta


@dataclass
class BertShape:
    layers: int = 12
    batch: int = 8
    seq: int = 384
    d: int = 768
    heads: int = 12
    ff: int = 3072
    vocab: int = 30522
    eps: float = 1e-12

    @property
    def hd(self) -> int:
        return self.d // self.heads

    def macs(self) -> int:
        """Multiply-accumulates of one forward: the linears and the attention contractions."""
        rows = self.batch * self.seq
        lin = rows * (3 * self.d * self.d + self.d * self.d + 2 * self.d * self.ff)
        att = 2 * self.batch * self.heads * self.seq * self.seq * self.hd
        return self.layers * (lin + att)

    def linear_macs(self) -> int:
        """Multiply-accumulates of the linears alone (the plane GEMM's share of a forward)."""
        return self.layers * self.batch * self.seq * (4 * self.d * self.d + 2 * self.d * self.ff)


def bert_encoder(shape: BertShape = BertShape(), seed: int = 0, calib_seqs: int = 1, fused_attention: bool = True,
                 as_ops: bool = False, prep_attention: bool = False):
    """(graph, inputs, exps): the BERT-base-shaped encoder in per-tensor power-of-two numerics.

    Token ids U{0 .. vocab-1} (the graph's input) and embedding rows N(0, 1), gathered on the
    GPU into the int32 residual at 2^-15 (LlmEmbedNode); per layer, in the arrangement of the
    reference's encoder template (vit.py:19-32):

        x  = LayerNorm32(h)                          row-ops NORM, int32 -> int16
        qkv = x . Wqkv                               MatMul (pow2, int32 wrap)
        s  = K . q^T   [B H][keys][queries]          batched MatMul, K and q rows per head read in
                                                     place from qkv (q as B^T), f_s = f_q + f_k - 8
        P  = softmax over keys (column mode)         VectorOP softmax, logit scale 1/sqrt(hd)
        o  = P . V     [B H][queries][hd]            batched MatMul, V rows read in place, o written
                                                     per head into its columns of om, f_o = f_p + f_v - 8
        h1 = ResAddBias(h, om . Wo, bo)              MatMul, row-ops ADDX
        x2 = LayerNorm32(h1);  f = x2 . W1  (at 2^-8)
        a  = GELU(f + b1)                            VectorOP ADD with the GELU act
        h  = ResAddBias(h1, a . W2, b2)

    Weights N(0, 0.02), biases N(0, 0.02), LayerNorm gamma N(1, 0.02), beta N(0, 0.02).
    Exponents: a float64 run of the first ``calib_seqs`` sequences gives each tensor's
    largest |value|, and each tensor takes the largest exponent that keeps it below 32767
    with a 1.25 margin; the contractions' output exponents follow from their operands', the
    q / v exponents are lowered where the scores or P.V would not fit.  ``exps`` records them.
    ``fused_attention`` (default): the head split, q.K^T, the softmax, P.V and the merge as
    one AttentionNode (the same arithmetic in one call, cm_attention on MFMA); False: node by
    node, the contractions on the plane GEMM reading and writing per-head views in place.
    ``prep_attention`` (one sequence): the reference's own chain of the encoder template instead
    (vit.py:564-630) -- VitAttnPrep on the row-ops unit (VitAttnPrepRoNode: q into the q.K^T
    image, k / v into the K / V caches, raw states [T][D] group-major shared by the layers), per
    head q.K^T (LlmAttnConvNode, static keys), the column-mode softmax (AttnSoftmaxNode, static)
    and P.V, and LlmAttnMerge -- the same integers as the fused node.
    ``as_ops`` (the fused or the prep attention): (ops, tensors, inputs, outputs) in place of the
    graph -- the encoder as the reference's ops (LlmEmbed, VitLayerNorm, MatMul, the attention
    chain as VitAttention or as VitAttnPrep / LlmAttnScores / VitAttnSoftmax / LlmAttnPV /
    LlmAttnMerge, VitResAdd, Add + Gelu) for the front end, weights not yet encoded.
    """
    from .frontend import LLM_DOMAIN, OpDesc
    from .numeric import encode_matmul_weights
    from .dtype import AP_FIXED_16_8

    S = shape
    # ids / embeddings and weights from their own generators: a smaller batch of the same seed
    # is the leading sequences of a larger one, with the same weights and exponents
    rng_in = np.random.default_rng([seed, 0])
    emb = rng_in.standard_normal((S.vocab, S.d), dtype=np.float32)
    ids = rng_in.integers(0, S.vocab, (S.batch, S.seq))
    h0 = emb[ids[:calib_seqs]].astype(np.float64).reshape(-1, S.d)
    h0 = np.round(h0 * 2.0 ** RES_BITS) / 2.0 ** RES_BITS
    rng = np.random.default_rng([seed, 1])
    norm = lambda *sh: (rng.standard_normal(sh, dtype=np.float32) * 0.02)       # noqa: E731
    Ls = []
    for _ in range(S.layers):
        Ls.append(dict(g1=1.0 + norm(S.d).astype(np.float64), be1=norm(S.d).astype(np.float64),
                       wqkv=norm(S.d, 3 * S.d), wo=norm(S.d, S.d), bo=norm(S.d).astype(np.float64),
                       g2=1.0 + norm(S.d).astype(np.float64), be2=norm(S.d).astype(np.float64),
                       w1=norm(S.d, S.ff), b1=norm(S.ff).astype(np.float64), w2=norm(S.ff, S.d),
                       b2=norm(S.d).astype(np.float64)))

    # ---- calibration: a float64 forward of the first sequences, the largest |value| per tensor
    H, hd, T = S.heads, S.hd, S.seq
    cal = []
    h = h0[:calib_seqs * T]
    for L in Ls:
        m = {}
        x = _layer_norm(h, L["g1"], L["be1"], S.eps)
        qkv = x @ L["wqkv"].astype(np.float64)
        q, k, v = qkv[:, :S.d], qkv[:, S.d:2 * S.d], qkv[:, 2 * S.d:]
        m.update(x1=np.abs(x).max(), q=np.abs(q).max(), k=np.abs(k).max(), v=np.abs(v).max())
        qh = q.reshape(-1, T, H, hd).transpose(0, 2, 1, 3)
        kh = k.reshape(-1, T, H, hd).transpose(0, 2, 1, 3)
        vh = v.reshape(-1, T, H, hd).transpose(0, 2, 1, 3)
        s = kh @ qh.transpose(0, 1, 3, 2)                       # [b][h][keys][queries]
        p = np.exp((s - s.max(axis=2, keepdims=True)) / math.sqrt(hd))
        p = p / p.sum(axis=2, keepdims=True)
        o = p.transpose(0, 1, 3, 2) @ vh                        # [b][h][queries][hd]
        m.update(s=np.abs(s).max(), o=np.abs(o).max())
        om = o.transpose(0, 2, 1, 3).reshape(-1, S.d)
        ao = om @ L["wo"].astype(np.float64)
        h1 = h + ao + L["bo"]
        x2 = _layer_norm(h1, L["g2"], L["be2"], S.eps)
        f = x2 @ L["w1"].astype(np.float64)
        a = _gelu(f + L["b1"])
        dd = a @ L["w2"].astype(np.float64)
        h = h1 + dd + L["b2"]
        m.update(ao=np.abs(ao).max(), x2=np.abs(x2).max(), f=np.abs(f + L["b1"]).max(), dd=np.abs(dd).max())
        cal.append(m)

    exps = []
    for m in cal:
        e = {key: _fit_exp(val) for key, val in m.items()}
        e["p"] = 14                                             # P <= 1: 2^14 fits int16
        # scores s at f_q + f_k - 8: lower the larger of q / k until s fits
        while e["q"] + e["k"] - F_Q88 > e["s"]:
            if e["q"] >= e["k"]:
                e["q"] -= 1
            else:
                e["k"] -= 1
        e["s"] = e["q"] + e["k"] - F_Q88
        # P.V at f_p + f_v - 8 must fit: v no finer than the output allows
        e["v"] = min(e["v"], e["o"] - e["p"] + F_Q88)
        e["o"] = e["p"] + e["v"] - F_Q88
        e["f"] = F_Q88                                          # the act unit's grid
        e["ao"] = min(e["ao"], RES_BITS)                        # residual deltas: no finer than 2^-15
        e["dd"] = min(e["dd"], RES_BITS)
        exps.append(e)

    # ---- the integer graph: the token ids in, their embedding rows gathered into the int32
    # residual at 2^-15 (LlmEmbedNode, the host op the reference runs before the encoder)
    T_ = TensorInfo
    rows, D = S.batch * S.seq, S.d
    BH = S.batch * H
    ids_t = T_("ids", [rows], exp=0, kind="i32")
    h_in = T_("h0", [rows, D], exp=RES_BITS, kind="i32")
    nodes = [LlmEmbedNode([ids_t], h_in, table=emb)]
    ops, reg = [], {"ids": ids_t}
    if as_ops and not (fused_attention or prep_attention):
        raise ValueError("bert_encoder: the op list describes the fused (VitAttention) or the prep attention")
    if prep_attention:
        from .graph import AttnMergeNode, AttnSoftmaxNode, LlmAttnConvNode
        from .rowops_nodes import VitAttnPrepRoNode
        if S.batch != 1 or T % 16:
            raise ValueError("bert_encoder: the prep attention takes one sequence of a multiple of 16 tokens")
        # the K / V caches: raw states [T][D] stored group-major [H][T][hd], shared by the layers
        kc_t = T_("vit.kc", [T, D], exp=0, group_layout=(H, hd), state=True)
        vc_t = T_("vit.vc", [T, D], exp=0, group_layout=(H, hd), state=True)

    def op(kind, ins, out, domain="", **attrs):
        for t in list(ins) + [out]:
            reg[t.onnx_name] = t
        ops.append(OpDesc(kind, [t.onnx_name for t in ins], [out.onnx_name], attrs, domain))

    op("LlmEmbed", [ids_t], h_in, LLM_DOMAIN, table=emb)
    hcur = h_in
    for li, (L, e) in enumerate(zip(Ls, exps)):
        p = f"l{li}."
        x1 = T_(p + "x1", [rows, D], exp=e["x1"])
        nodes.append(LayerNorm32RoNode([hcur], x1, gamma=L["g1"], beta=L["be1"], eps=S.eps))
        op("VitLayerNorm", [hcur], x1, LLM_DOMAIN, gamma=L["g1"], beta=L["be1"], eps=S.eps)
        wqkv = T_(p + "wqkv", [D, 3 * D], data=L["wqkv"])
        qkv = T_(p + "qkv", [rows, 3 * D], exp=np.repeat([e["q"], e["k"], e["v"]], D))
        nodes.append(MatmulNode([x1, wqkv], qkv))
        op("MatMul", [x1, wqkv], qkv)
        ld = 3 * D
        cmr, cfg = softmax_regs(e["s"], 1.0 / math.sqrt(hd), e["p"])
        om = T_(p + "om", [rows, D], exp=e["o"])
        if prep_attention:
            qx = T_(p + "qx", [H, hd, T], exp=0)
            nodes.append(VitAttnPrepRoNode([qkv, qkv, qkv, kc_t, vc_t], qx, heads=H, head_dim=hd, fq=e["q"], fk=e["k"],
                                           fv=e["v"], cols=(0, D, 2 * D)))
            op("VitAttnPrep", [qkv, qkv, qkv, kc_t, vc_t], qx, LLM_DOMAIN, num_heads=H, head_dim=hd, q_exp=[e["q"]] * H,
               k_exp=[e["k"]] * H, v_exp=[e["v"]] * D, cols=(0, D, 2 * D), rowops=1)
            geo = dict(T=T, H=H, KV=H, HD=hd, C=T, static=True)
            heads_attrs = dict(num_heads=H, num_kv_heads=H, head_dim=hd)
            outs = []
            for hh in range(H):
                st = T_(p + f"s{hh}", [T, T], exp=0)
                nodes.append(LlmAttnConvNode([kc_t, qx], st, kind="qk", group=hh, **geo))
                op("LlmAttnScores", [kc_t, qx], st, LLM_DOMAIN, group=hh, **heads_attrs)
                pt = T_(p + f"p{hh}", [T, T], exp=0)
                nodes.append(AttnSoftmaxNode([st], pt, T=T, G=1, C=T, cm=cmr, cfg=cfg, causal=False))
                op("VitAttnSoftmax", [st], pt, LLM_DOMAIN, head_dim=hd, s_exp=[e["s"]], p_exp=[e["p"]], vsmx=1)
                ot = T_(p + f"o{hh}", [T, hd], exp=0)
                nodes.append(LlmAttnConvNode([pt, vc_t], ot, kind="pv", group=hh, **geo))
                op("LlmAttnPV", [pt, vc_t], ot, LLM_DOMAIN, group=hh, **heads_attrs)
                outs.append(ot)
            nodes.append(AttnMergeNode(outs, om, T=T, H=H, KV=H, HD=hd))
            ops.append(OpDesc("LlmAttnMerge", [t.onnx_name for t in outs], [om.onnx_name], heads_attrs, LLM_DOMAIN))
            reg[om.onnx_name] = om
        elif fused_attention:
            nodes.append(AttentionNode([qkv], om, batch=S.batch, seq=T, heads=H, head_dim=hd, q_off=0, k_off=D,
                                       v_off=2 * D, cm=cmr, cfg=cfg))
            op("VitAttention", [qkv], om, LLM_DOMAIN, batch=S.batch, seq=T, heads=H, head_dim=hd, q_off=0, k_off=D,
               v_off=2 * D, cm=cmr, cfg=cfg)
        else:
            # the per-head q / K / V rows read in place from qkv, o written in place into om
            hv = lambda col: HeadView(col, H, hd, T)                                 # noqa: E731
            # s[j][i] = K[j] . Q[i]: the q rows as the transposed B image (no q transpose)
            sc = T_(p + "s", [BH, T, T], exp=e["s"])
            nodes.append(AttnContractNode([qkv, qkv], sc, b_trans=True, a_view=hv(D), b_view=hv(0)))
            pr = T_(p + "P", [BH, T, T], exp=e["p"])
            nodes.append(SoftmaxVopNode([sc], pr, cm=cmr, cfg=cfg, keys_major=True))
            nodes.append(AttnContractNode([pr, qkv], om, b_view=hv(2 * D), c_view=hv(0)))
        wo = T_(p + "wo", [D, D], data=L["wo"])
        ao = T_(p + "ao", [rows, D], exp=e["ao"])
        nodes.append(MatmulNode([om, wo], ao))
        op("MatMul", [om, wo], ao)
        h1 = T_(p + "h1", [rows, D], exp=RES_BITS, kind="i32")
        nodes.append(ResAddBiasRoNode([hcur, ao], h1, bias=L["bo"]))
        op("VitResAdd", [hcur, ao], h1, LLM_DOMAIN, bias=L["bo"])
        x2 = T_(p + "x2", [rows, D], exp=e["x2"])
        nodes.append(LayerNorm32RoNode([h1], x2, gamma=L["g2"], beta=L["be2"], eps=S.eps))
        op("VitLayerNorm", [h1], x2, LLM_DOMAIN, gamma=L["g2"], beta=L["be2"], eps=S.eps)
        w1 = T_(p + "w1", [D, S.ff], data=L["w1"])
        # FFN1's output, the bias and the GELU run in the element type itself (Q8.8: no annotation)
        f = T_(p + "f", [rows, S.ff])
        nodes.append(MatmulNode([x2, w1], f))
        op("MatMul", [x2, w1], f)
        b1 = T_(p + "b1", [S.ff], data=L["b1"])
        a = T_(p + "a", [rows, S.ff])
        nodes.append(ScheduledNode([f, b1], a, units.OP_ADD, act=units.ACT_GELU))
        fb = T_(p + "fb", [rows, S.ff])
        op("Add", [f, b1], fb)
        op("Gelu", [fb], a)
        w2 = T_(p + "w2", [S.ff, D], data=L["w2"])
        dd = T_(p + "dd", [rows, D], exp=e["dd"])
        nodes.append(MatmulNode([a, w2], dd))
        op("MatMul", [a, w2], dd)
        hn = T_(p + "h", [rows, D], exp=RES_BITS, kind="i32")
        nodes.append(ResAddBiasRoNode([h1, dd], hn, bias=L["b2"]))
        op("VitResAdd", [h1, dd], hn, LLM_DOMAIN, bias=L["b2"])
        hcur = hn
    feeds = {"ids": ids.reshape(-1).astype(np.float64)}
    if as_ops:
        return (ops, reg, ["ids"], [hcur.onnx_name]), feeds, exps
    g = Graph(nodes, input_tensors=[ids_t], output_tensors=[hcur])
    encode_matmul_weights(g.nodes, AP_FIXED_16_8)
    return g, feeds, exps


# ---------------------------------------------------------------- SmolLM2-360M-shaped decode step
@dataclass
class LlamaShape:
    """A Llama-architecture decoder (SmolLM2-360M's by default: config.json of the checkpoint
    the reference's llama.py front end reads) and the decode step's batch / cache."""
    layers: int = 32
    batch: int = 16
    d: int = 960
    heads: int = 15
    kv: int = 5
    hd: int = 64
    ff: int = 2560
    vocab: int = 49152
    ctx: int = 1024
    theta: float = 100000.0
    eps: float = 1e-5

    @property
    def group(self) -> int:
        return self.heads // self.kv

    def macs(self, keys: int = None) -> int:
        """Multiply-accumulates of one step: the linears (q, k, v, o, gate, up, down and the
        tied head) for every sequence, and q.K^T / P.V over ``keys`` cache rows."""
        keys = self.ctx if keys is None else keys
        D, A, K = self.d, self.heads * self.hd, self.kv * self.hd
        lin = self.layers * (D * A + 2 * D * K + A * D + 3 * D * self.ff) + D * self.vocab
        att = self.layers * 2 * self.heads * keys * self.hd
        return self.batch * (lin + att)

    def weight_bytes(self) -> int:
        D, A, K = self.d, self.heads * self.hd, self.kv * self.hd
        return 2 * (self.layers * (D * A + 2 * D * K + A * D + 3 * D * self.ff) + D * self.vocab)


def rope_half_tables(theta: float, hd: int, n: int):
    """float32 cos / sin [n][hd/2] as the reference's rope.half_tables (rope.py:51-58,
    133-146): inv_j = float32(1 / theta^(2j/hd)) from float64, a = float32(float32(pos) * inv_j),
    cos = float32(cos(double(a)))."""
    inv = np.array([1.0 / (theta ** (2 * j / hd)) for j in range(hd // 2)], np.float64).astype(np.float32)
    ang = (np.arange(n, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    c = np.cos(ang.astype(np.float64)).astype(np.float32)
    s = np.sin(ang.astype(np.float64)).astype(np.float32)
    return c, s


def _rms(h, gamma, eps):
    return h / np.sqrt((h * h).mean(axis=-1, keepdims=True) + eps) * gamma


def _rope_f(x, heads, hd, cos, sin):
    """Rotate-half RoPE of rows [T][heads * hd] at one position (cos / sin [hd / 2])."""
    x = x.reshape(-1, heads, hd)
    half = hd // 2
    x1, x2 = x[..., :half], x[..., half:]
    c, s = cos.astype(np.float64), sin.astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1).reshape(-1, heads * hd)


KV_SIGMA = 0.6       # std of the synthetic cache rows: about a projection's (sqrt(960) x 0.02)


def smollm2_weights(shape: LlamaShape = LlamaShape(), seed: int = 0):
    """The synthetic float32 weights of ``shape`` (the decode step's ``weights``): the tied
    embedding [vocab][d], per layer the linears (wq [d][heads hd], wk / wv [d][kv hd], wo,
    wg / wu [d][ff], wd [ff][d]) N(0, 0.02) and the RMSNorm gammas 1 + N(0, 0.02), the final
    gamma."""
    S = shape
    A, KD = S.heads * S.hd, S.kv * S.hd
    rng = np.random.default_rng([seed, 1])
    nrm = lambda *sh: rng.standard_normal(sh, dtype=np.float32) * np.float32(0.02)     # noqa: E731
    emb = nrm(S.vocab, S.d)
    Ls = [dict(g1=1.0 + nrm(S.d).astype(np.float64), wq=nrm(S.d, A), wk=nrm(S.d, KD), wv=nrm(S.d, KD),
               wo=nrm(A, S.d), g2=1.0 + nrm(S.d).astype(np.float64), wg=nrm(S.d, S.ff), wu=nrm(S.d, S.ff),
               wd=nrm(S.ff, S.d))
          for _ in range(S.layers)]
    gf = 1.0 + nrm(S.d).astype(np.float64)
    return emb, Ls, gf


def smollm2_decode(shape: LlamaShape = LlamaShape(), seed: int = 0, calib_seqs: int = 1, weights=None,
                   runtime_pos: bool = False, fused_attention: bool = True, as_ops: bool = False):
    """(graph, inputs, exps): one greedy decode step of ``shape.batch`` sequences, each at cache
    position ctx - 1 (the cache full after the step's row: every cache row is a key), pow2
    numerics on the units as the reference's llama.py front end lays out a layer with the
    row-ops policy (llama.py:140-400, ``rowops`` + ``drope``):

        x  = RMSNorm(h)                    row-ops NORM, int32 residual at 2^-15 -> int16
        q, k, v = x Wq, x Wk, x Wv         MatMul (pow2, int32 wrap)
        q, k = RoPE(q), RoPE(k)            row-ops ROPE at position pos
        cache rows pos <- k, v             the attention prep's cache writes
        s  = q_g . K_cache^T               batched contraction per (sequence, group), query-major
        P  = softmax over keys             VectorOP softmax (row mode), keys <= pos
        o  = P . V_cache                   batched contraction
        h1 = ResAdd(h, o Wo)               row-ops ADDX
        x2 = RMSNorm(h1); m = SiluMul(x2 Wg, x2 Wu); h = ResAdd(h1, m Wd)
    then RMSNorm, the tied head (x E^T) and Dequant to float32 logits.

    Synthetic data (no checkpoint): the tied embedding, every linear N(0, 0.02), RMSNorm
    gammas 1 + N(0, 0.02); the step's token ids (the graph's input) gathered on the GPU from the
    tied embedding into the int32 residual (LlmEmbedNode); the cache
    rows before ``pos`` N(0, KV_SIGMA) in place of a prefill; every draw is per sequence, so a
    smaller batch of the same seed is the leading sequences of a larger one.  Exponents from a
    float64 run of the step over the first ``calib_seqs`` sequences (``_fit_exp``), with the
    pow2 rules: f_s = f_q + f_k - 8 (q / k lowered until
    s fits), P at 2^-14, f_o = f_p + f_v - 8, deltas at <= 2^-15, the gate at <= 2^-14, and
    every weight's exponent f_out + 8 - f_in at least 10.  ``weights``: smollm2_weights(shape,
    seed) made once for several builds (they depend on the shape's sizes, not its batch).

    ``runtime_pos``: the step's position is a host input "pos" (RoPE's table row, the cache row
    written, the softmax's valid keys pos + 1) and the KV caches are persistent states, so one
    graph runs successive decode steps over the same caches (_forward_pass with ``states``);
    the inputs then carry "pos" = ctx - 1 and the caches' prefill as the states' first values.

    ``fused_attention``: the RoPE of q / k and the cache row writes as one DecodePrepNode, and
    q.K^T, the softmax and P.V as one DecodeAttentionNode (the same arithmetic; the RoPE'd k rows,
    s and P not materialized) where the kernels take the geometry; otherwise the RoPE and KV-write
    nodes, the two contractions and the softmax node.

    ``as_ops`` (with the fused attention): (ops, tensors, inputs, outputs) in place of the graph --
    the step as the reference's LLM ops (LlmEmbed, LlmRMSNorm, MatMul, the attention prep and
    chain as LlmDecodeAttention, LlmResAdd, LlmSiluMul, LlmDequant) for the front end."""
    from .frontend import LLM_DOMAIN, OpDesc
    from .dtype import AP_FIXED_16_8
    from .numeric import encode_matmul_weights
    from .rowops_nodes import DecodePrepNode, DequantRoNode, RMSNormRoNode, ResAddRoNode, RopeRoNode, SiluMulRoNode
    from .graph import KvWriteNode

    S = shape
    if S.ctx % 16 or S.heads % S.kv or S.hd % 16:
        raise ValueError("ctx and head_dim multiples of 16, heads a multiple of the KV heads")
    pos = S.ctx - 1
    B, D, H, KV, HD, G = S.batch, S.d, S.heads, S.kv, S.hd, S.group
    A, KD = H * HD, KV * HD
    keys = S.ctx
    emb, Ls, gf = smollm2_weights(S, seed) if weights is None else weights
    rng_in = np.random.default_rng([seed, 0])
    ids = rng_in.integers(0, S.vocab, B * 64)[::64]            # sequence b's id: one draw per sequence slot
    h0 = np.round(emb[ids].astype(np.float64) * 2.0 ** RES_BITS) / 2.0 ** RES_BITS
    cos, sin = rope_half_tables(S.theta, HD, S.ctx)

    def cache_rows(layer, which):
        """[B][KV][ctx][HD] float values of the synthetic rows before pos (zeros after)."""
        c = np.zeros((B, KV, S.ctx, HD), np.float32)
        for b in range(B):
            r = np.random.default_rng([seed, 2, layer, which, b])
            c[b, :, :pos, :] = r.standard_normal((KV, pos, HD), dtype=np.float32) * np.float32(KV_SIGMA)
        return c

    # ---- calibration: the step in float64 over the first sequences
    cb = max(1, min(calib_seqs, B))
    cal, caches = [], []
    h = h0[:cb]
    for li, L in enumerate(Ls):
        m = {}
        x = _rms(h, L["g1"], S.eps)
        q = x @ L["wq"].astype(np.float64)
        k = x @ L["wk"].astype(np.float64)
        v = x @ L["wv"].astype(np.float64)
        qr = _rope_f(q, H, HD, cos[pos], sin[pos])
        kr = _rope_f(k, KV, HD, cos[pos], sin[pos])
        kc, vc = cache_rows(li, 0), cache_rows(li, 1)
        caches.append((kc, vc))
        kc, vc = kc[:cb], vc[:cb]
        kfull, vfull = kc.copy(), vc.copy()
        kfull[:, :, pos, :] = kr.reshape(cb, KV, HD)
        vfull[:, :, pos, :] = v.reshape(cb, KV, HD)
        qh = qr.reshape(cb, KV, G, HD)
        s = np.einsum("bgjd,bgpd->bgjp", kfull[:, :, :pos + 1], qh)            # [B][KV][keys][G]
        p = np.exp((s - s.max(axis=2, keepdims=True)) / math.sqrt(HD))
        p = p / p.sum(axis=2, keepdims=True)
        o = np.einsum("bgjp,bgjd->bgpd", p, vfull[:, :, :pos + 1]).reshape(cb, A)
        a = o @ L["wo"].astype(np.float64)
        h1 = h + a
        x2 = _rms(h1, L["g2"], S.eps)
        gt = x2 @ L["wg"].astype(np.float64)
        up = x2 @ L["wu"].astype(np.float64)
        mm = gt / (1.0 + np.exp(-gt)) * up
        dd = mm @ L["wd"].astype(np.float64)
        h = h1 + dd
        m.update(x=np.abs(x).max(), q=max(np.abs(q).max(), np.abs(qr).max()),
                 k=max(np.abs(k).max(), np.abs(kr).max(), np.abs(kc).max()),
                 v=max(np.abs(v).max(), np.abs(vc).max()), s=np.abs(s).max(), o=np.abs(o).max(), a=np.abs(a).max(),
                 x2=np.abs(x2).max(), g=np.abs(gt).max(), u=np.abs(up).max(), m=np.abs(mm).max(),
                 d=np.abs(dd).max())
        cal.append(m)
    xf = _rms(h, gf, S.eps)
    logits = xf @ emb.T.astype(np.float64)
    fin = dict(xf=_fit_exp(np.abs(xf).max()), logits=_fit_exp(np.abs(logits).max()))

    # the largest exponents that fit, lowered where a rule ties them: a weight's rank-1
    # exponent f_out + 8 - f_in kept >= W_MIN (N(0, 0.02) weights then keep >= 5 bits)
    W_MIN = 10
    exps = []
    for m in cal:
        f = {key: _fit_exp(val) for key, val in m.items()}
        e = {"p": 14, "q": f["q"], "k": f["k"]}
        while e["q"] + e["k"] - F_Q88 > f["s"]:                 # s = K . q at f_q + f_k - 8
            if e["q"] >= e["k"]:
                e["q"] -= 1
            else:
                e["k"] -= 1
        e["s"] = e["q"] + e["k"] - F_Q88
        e["a"] = min(f["a"], RES_BITS)                          # residual deltas at <= 2^-15
        e["v"] = min(f["v"], f["o"] - e["p"] + F_Q88, e["a"] + F_Q88 - W_MIN - e["p"] + F_Q88)
        e["o"] = e["p"] + e["v"] - F_Q88                        # o = P . V at f_p + f_v - 8
        e["x"] = min(f["x"], e["q"] + F_Q88 - W_MIN, e["k"] + F_Q88 - W_MIN, e["v"] + F_Q88 - W_MIN)
        e["g"] = min(f["g"], 14)                                # the gate at <= 2^-14 (MULACT)
        e["u"] = f["u"]
        e["d"] = min(f["d"], RES_BITS)
        e["m"] = min(f["m"], e["d"] + F_Q88 - W_MIN)
        e["x2"] = min(f["x2"], e["g"] + F_Q88 - W_MIN, e["u"] + F_Q88 - W_MIN)
        exps.append(e)
    fin["xf"] = min(fin["xf"], fin["logits"] + F_Q88 - W_MIN)
    exps.append(fin)

    # ---- the integer graph
    T_ = TensorInfo
    nodes, ops, reg = [], [], {}
    if as_ops and not (fused_attention and DecodeAttentionNode.supports(HD, S.ctx, G) and HD % 16 == 0):
        raise ValueError("smollm2_decode: the op list describes the fused decode attention")

    def op(kind, ins, outs, domain="", **attrs):
        outs = outs if isinstance(outs, list) else [outs]
        for t in list(ins) + outs:
            reg[t.onnx_name] = t
        ops.append(OpDesc(kind, [t.onnx_name for t in ins], [t.onnx_name for t in outs], attrs, domain))

    ids_t = T_("ids", [B], exp=0, kind="i32")
    h_in = T_("h0", [B, D], exp=RES_BITS, kind="i32")
    nodes.append(LlmEmbedNode([ids_t], h_in, table=emb))
    op("LlmEmbed", [ids_t], h_in, LLM_DOMAIN, table=emb)
    inputs = {"ids": ids.astype(np.float64)}
    pos_t = T_("pos", [1], kind="host") if runtime_pos else None
    if runtime_pos:
        inputs["pos"] = np.array([pos], np.float64)
    cache_ts = []
    hcur = h_in
    for li, (L, e) in enumerate(zip(Ls, exps)):
        p = f"l{li}."
        kc_t = T_(p + "kc", [B, KV, S.ctx, HD], exp=e["k"], state=runtime_pos)
        vc_t = T_(p + "vc", [B, KV, S.ctx, HD], exp=e["v"], state=runtime_pos)
        cache_ts += [kc_t, vc_t]
        kc, vc = caches[li]
        inputs[kc_t.onnx_name] = np.round(kc.astype(np.float64) * 2.0 ** e["k"]) / 2.0 ** e["k"]
        inputs[vc_t.onnx_name] = np.round(vc.astype(np.float64) * 2.0 ** e["v"]) / 2.0 ** e["v"]
        x = T_(p + "x", [B, D], exp=e["x"])
        nodes.append(RMSNormRoNode([hcur], x, gamma=L["g1"], eps=S.eps))
        op("LlmRMSNorm", [hcur], x, LLM_DOMAIN, gamma=L["g1"], eps=S.eps)
        q = T_(p + "q", [B, A], exp=e["q"])
        nodes.append(MatmulNode([x, T_(p + "wq", [D, A], data=L["wq"])], q))
        op("MatMul", nodes[-1].inputs, q)
        k = T_(p + "k", [B, KD], exp=e["k"])
        nodes.append(MatmulNode([x, T_(p + "wk", [D, KD], data=L["wk"])], k))
        op("MatMul", nodes[-1].inputs, k)
        v = T_(p + "v", [B, KD], exp=e["v"])
        nodes.append(MatmulNode([x, T_(p + "wv", [D, KD], data=L["wv"])], v))
        op("MatMul", nodes[-1].inputs, v)
        qr = T_(p + "qr", [B, A], exp=e["q"])
        cmr, cfg = softmax_regs(e["s"], 1.0 / math.sqrt(HD), e["p"])
        om = T_(p + "om", [B, A], exp=e["o"])
        if fused_attention and DecodeAttentionNode.supports(HD, S.ctx, G) and HD % 16 == 0:
            # RoPE of q and k with the cache rows written in one launch, then the attention
            nodes.append(DecodePrepNode([q, k, v, kc_t, vc_t], qr, heads=H, kv_heads=KV, head_dim=HD, cos=cos,
                                        sin=sin, pos=pos, pos_t=pos_t))
            nodes.append(DecodeAttentionNode([qr, kc_t, vc_t], om, heads=H, kv_heads=KV, head_dim=HD, cm=cmr, cfg=cfg,
                                             mask=pos + 1, mask_t=pos_t, mask_add=1))
            op("LlmDecodeAttention", [q, k, v, kc_t, vc_t], [qr, om], LLM_DOMAIN, heads=H, kv_heads=KV, head_dim=HD,
               cos=cos, sin=sin, pos=pos, pos_t=pos_t.onnx_name if pos_t is not None else None, cm=cmr, cfg=cfg)
        else:
            nodes.append(RopeRoNode([q], qr, heads=H, head_dim=HD, cos=cos, sin=sin, pos=pos, same_pos=True,
                                    pos_t=pos_t))
            kr = T_(p + "kr", [B, KD], exp=e["k"])
            nodes.append(RopeRoNode([k], kr, heads=KV, head_dim=HD, cos=cos, sin=sin, pos=pos, same_pos=True,
                                    pos_t=pos_t))
            kc2 = T_(p + "kc1", [B, KV, S.ctx, HD], exp=e["k"])
            nodes.append(KvWriteNode([kr, kc_t], kc2, pos=pos, pos_t=pos_t))
            vc2 = T_(p + "vc1", [B, KV, S.ctx, HD], exp=e["v"])
            nodes.append(KvWriteNode([v, vc_t], vc2, pos=pos, pos_t=pos_t))
            _decode_attention_unfused(nodes, T_, p, e, qr, kc2, vc2, om, B, KV, G, HD, keys, S.ctx, cmr, cfg, pos,
                                      pos_t)
        a = T_(p + "a", [B, D], exp=e["a"])
        nodes.append(MatmulNode([om, T_(p + "wo", [A, D], data=L["wo"])], a))
        op("MatMul", nodes[-1].inputs, a)
        h1 = T_(p + "h1", [B, D], exp=RES_BITS, kind="i32")
        nodes.append(ResAddRoNode([hcur, a], h1))
        op("LlmResAdd", [hcur, a], h1, LLM_DOMAIN)
        x2 = T_(p + "x2", [B, D], exp=e["x2"])
        nodes.append(RMSNormRoNode([h1], x2, gamma=L["g2"], eps=S.eps))
        op("LlmRMSNorm", [h1], x2, LLM_DOMAIN, gamma=L["g2"], eps=S.eps)
        gt = T_(p + "g", [B, S.ff], exp=e["g"])
        nodes.append(MatmulNode([x2, T_(p + "wg", [D, S.ff], data=L["wg"])], gt))
        op("MatMul", nodes[-1].inputs, gt)
        up = T_(p + "u", [B, S.ff], exp=e["u"])
        nodes.append(MatmulNode([x2, T_(p + "wu", [D, S.ff], data=L["wu"])], up))
        op("MatMul", nodes[-1].inputs, up)
        mm = T_(p + "m", [B, S.ff], exp=e["m"])
        nodes.append(SiluMulRoNode([gt, up], mm))
        op("LlmSiluMul", [gt, up], mm, LLM_DOMAIN)
        dd = T_(p + "d", [B, D], exp=e["d"])
        nodes.append(MatmulNode([mm, T_(p + "wd", [S.ff, D], data=L["wd"])], dd))
        op("MatMul", nodes[-1].inputs, dd)
        hn = T_(p + "h", [B, D], exp=RES_BITS, kind="i32")
        nodes.append(ResAddRoNode([h1, dd], hn))
        op("LlmResAdd", [h1, dd], hn, LLM_DOMAIN)
        hcur = hn
    xf = T_("xf", [B, D], exp=fin["xf"])
    nodes.append(RMSNormRoNode([hcur], xf, gamma=gf, eps=S.eps))
    op("LlmRMSNorm", [hcur], xf, LLM_DOMAIN, gamma=gf, eps=S.eps)
    lq = T_("logits_q", [B, S.vocab], exp=fin["logits"])
    nodes.append(MatmulNode([xf, T_("w.lm_head", [D, S.vocab], data=np.ascontiguousarray(emb.T))], lq))
    op("MatMul", nodes[-1].inputs, lq)
    # the dequant's jobs take rows of at most 4096: the logits as [B * vocab / chunk][chunk]
    chunk = next(c for c in range(4096, 0, -8) if S.vocab % c == 0)
    lr = T_("logits_rows", [B * S.vocab // chunk, chunk], exp=fin["logits"])
    nodes.append(ReshapeNode([lq], lr))
    op("Reshape", [lq], lr)
    lf = T_("logits_f32", [B * S.vocab // chunk, chunk], kind="f32")
    nodes.append(DequantRoNode([lr], lf))
    op("LlmDequant", [lr], lf, LLM_DOMAIN)
    lo = T_("logits", [B, S.vocab], kind="f32")
    nodes.append(ReshapeNode([lf], lo))
    op("Reshape", [lf], lo)
    graph_inputs = [ids_t] + ([pos_t] if runtime_pos else []) + cache_ts
    if as_ops:
        for t in graph_inputs:
            reg[t.onnx_name] = t
        return (ops, reg, [t.onnx_name for t in graph_inputs], [lo.onnx_name]), inputs, exps
    g = Graph(nodes, input_tensors=graph_inputs, output_tensors=[lo])
    encode_matmul_weights(g.nodes, AP_FIXED_16_8)
    return g, inputs, exps

def smollm2_prefill(shape: LlamaShape, T: int, exps, weights, with_head: bool = False, as_ops: bool = False):
    """The prefill_T entry of one sequence (llama.py:28-33; the layers :404-450 with the FPGA
    prefill attention :329-402; the entry :465-497): ids [T] (int32), pos and n (host) -> every
    layer's KV cache rows pos .. pos + n - 1 written in place, and the state ``h_last`` = the
    residual's row n - 1 after the last layer (LlmSelectRow).  Rows t >= n are computed but
    write nothing the caches or h_last keep.  ``with_head``: also that row's float32 logits
    (the prefill_T_logits entry).

    The numerics and weights are the decode step's (``exps`` and ``weights`` as smollm2_decode
    returns and takes them), and the caches are the decode graph's, one sequence of them: the
    states ``l<i>.kc`` / ``l<i>.vc`` hold logical [C][KV HD] stored group-major [KV][C][HD],
    byte for byte sequence b's slice of the decode graph's [B][KV][C][HD] caches (prefill_cache
    / decode_cache convert the float64 values).  A layer: RMSNorm; the q / k / v MatMuls; the
    attention prep on the row-ops unit (AttnPrepRoNode: RoPE of q / k at positions pos + t, the
    q.K^T image, the cache rows); per KV group q.K^T (LlmAttnConvNode) over keys = roundup(pos
    + n, 16), the causal column-mode softmax (AttnSoftmaxNode) and P.V; the merge; the o MatMul,
    ResAdd, RMSNorm, gate / up, SiluMul, down, ResAdd.  T a multiple of 16, ctx at most 1024
    (the softmax unit's column mode).

    ``as_ops``: (ops, tensors, inputs, outputs) in place of the graph -- the entry as the
    reference's LLM ops (LlmEmbed, LlmRMSNorm, MatMul, LlmAttnPrep, LlmAttnScores, LlmAttnSoftmax
    with vsmx, LlmAttnPV, LlmAttnMerge, LlmResAdd, LlmSiluMul, LlmSelectRow) for the front end."""
    from .dtype import AP_FIXED_16_8
    from .frontend import LLM_DOMAIN, OpDesc
    from .graph import AttnMergeNode, AttnSoftmaxNode, LlmAttnConvNode, SelectRowNode, SMX_MAX_KEYS
    from .numeric import encode_matmul_weights
    from .rowops_nodes import AttnPrepRoNode, DequantRoNode, RMSNormRoNode, ResAddRoNode, SiluMulRoNode

    S = shape
    if T % 16 or S.ctx % 16 or S.ctx > SMX_MAX_KEYS or S.heads % S.kv or S.hd % 16:
        raise ValueError(f"prefill: T a multiple of 16, ctx a multiple of 16 up to {SMX_MAX_KEYS}, heads a multiple "
                         "of the KV heads, head_dim a multiple of 16")
    D, H, KV, HD, G, C = S.d, S.heads, S.kv, S.hd, S.group, S.ctx
    A, KD = H * HD, KV * HD
    emb, Ls, gf = weights
    cos, sin = rope_half_tables(S.theta, HD, C)
    T_ = TensorInfo
    nodes, ops, reg = [], [], {}

    def add(node, kind, domain=LLM_DOMAIN, outs=None, **attrs):
        nodes.append(node)
        ins = [t for t in node.inputs if t is not None]
        outs = [node.output] if outs is None else outs
        for t in ins + outs:
            reg[t.onnx_name] = t
        ops.append(OpDesc(kind, [t.onnx_name for t in ins], [t.onnx_name for t in outs], attrs, domain))

    ids_t = T_("ids", [T], exp=0, kind="i32")
    pos_t = T_("pos", [1], kind="host")
    n_t = T_("n", [1], kind="host")
    h0 = T_("h0", [T, D], exp=RES_BITS, kind="i32")
    add(LlmEmbedNode([ids_t], h0, table=emb), "LlmEmbed", table=emb)
    hcur = h0
    heads = dict(num_heads=H, num_kv_heads=KV, head_dim=HD)
    for li, (L, e) in enumerate(zip(Ls, exps)):
        p = f"l{li}."
        kc_t = T_(p + "kc", [C, KD], exp=e["k"], group_layout=(KV, HD), state=True)
        vc_t = T_(p + "vc", [C, KD], exp=e["v"], group_layout=(KV, HD), state=True)
        x = T_(p + "x", [T, D], exp=e["x"])
        add(RMSNormRoNode([hcur], x, gamma=L["g1"], eps=S.eps), "LlmRMSNorm", gamma=L["g1"], eps=S.eps)
        q0 = T_(p + "q", [T, A], exp=e["q"])
        add(MatmulNode([x, T_(p + "wq", [D, A], data=L["wq"])], q0), "MatMul", domain="")
        k0 = T_(p + "k", [T, KD], exp=e["k"])
        add(MatmulNode([x, T_(p + "wk", [D, KD], data=L["wk"])], k0), "MatMul", domain="")
        v = T_(p + "v", [T, KD], exp=e["v"])
        add(MatmulNode([x, T_(p + "wv", [D, KD], data=L["wv"])], v), "MatMul", domain="")
        qx = T_(p + "qx", [KV, HD, G * T], exp=0)
        fq = np.full(H, e["q"])
        add(AttnPrepRoNode([q0, k0, v, pos_t, n_t, kc_t, vc_t], qx, heads=H, kv_heads=KV, head_dim=HD, fq=fq,
                           cos=cos, sin=sin), "LlmAttnPrep", q_exp=fq, cos=cos, sin=sin, rowops=1, **heads)
        cmr, cfg = softmax_regs(e["s"], 1.0 / math.sqrt(HD), e["p"])
        geo = dict(T=T, H=H, KV=KV, HD=HD, C=C)
        outs = []
        for grp in range(KV):
            s = T_(p + f"s{grp}", [C, G * T], exp=0)
            add(LlmAttnConvNode([kc_t, qx, pos_t, n_t], s, kind="qk", group=grp, **geo), "LlmAttnScores", group=grp,
                **heads)
            pg = T_(p + f"p{grp}", [G * T, C], exp=0)
            add(AttnSoftmaxNode([s, pos_t, n_t], pg, T=T, G=G, C=C, group=grp, cm=cmr, cfg=cfg), "LlmAttnSoftmax",
                group=grp, s_exp=[e["s"]] * G, p_exp=[e["p"]] * G, vsmx=1, **heads)
            og = T_(p + f"o{grp}", [G * T, HD], exp=0)
            add(LlmAttnConvNode([pg, vc_t, pos_t, n_t], og, kind="pv", group=grp, **geo), "LlmAttnPV", group=grp,
                **heads)
            outs.append(og)
        om = T_(p + "om", [T, A], exp=e["o"])
        add(AttnMergeNode(outs, om, T=T, H=H, KV=KV, HD=HD), "LlmAttnMerge", **heads)
        a = T_(p + "a", [T, D], exp=e["a"])
        add(MatmulNode([om, T_(p + "wo", [A, D], data=L["wo"])], a), "MatMul", domain="")
        h1 = T_(p + "h1", [T, D], exp=RES_BITS, kind="i32")
        add(ResAddRoNode([hcur, a], h1), "LlmResAdd")
        x2 = T_(p + "x2", [T, D], exp=e["x2"])
        add(RMSNormRoNode([h1], x2, gamma=L["g2"], eps=S.eps), "LlmRMSNorm", gamma=L["g2"], eps=S.eps)
        gt = T_(p + "g", [T, S.ff], exp=e["g"])
        add(MatmulNode([x2, T_(p + "wg", [D, S.ff], data=L["wg"])], gt), "MatMul", domain="")
        up = T_(p + "u", [T, S.ff], exp=e["u"])
        add(MatmulNode([x2, T_(p + "wu", [D, S.ff], data=L["wu"])], up), "MatMul", domain="")
        mm = T_(p + "m", [T, S.ff], exp=e["m"])
        add(SiluMulRoNode([gt, up], mm), "LlmSiluMul")
        dd = T_(p + "d", [T, D], exp=e["d"])
        add(MatmulNode([mm, T_(p + "wd", [S.ff, D], data=L["wd"])], dd), "MatMul", domain="")
        hn = T_(p + "h", [T, D], exp=RES_BITS, kind="i32")
        add(ResAddRoNode([h1, dd], hn), "LlmResAdd")
        hcur = hn
    h_last = T_("h_last", [1, D], exp=RES_BITS, kind="i32", state=True)
    add(SelectRowNode([hcur, n_t], h_last), "LlmSelectRow")
    outputs = [h_last]
    if with_head:
        fin = exps[-1]
        xf = T_("xf", [1, D], exp=fin["xf"])
        add(RMSNormRoNode([h_last], xf, gamma=gf, eps=S.eps), "LlmRMSNorm", gamma=gf, eps=S.eps)
        lq = T_("logits_q", [1, S.vocab], exp=fin["logits"])
        add(MatmulNode([xf, T_("w.lm_head", [D, S.vocab], data=np.ascontiguousarray(emb.T))], lq), "MatMul",
            domain="")
        chunk = next(c for c in range(4096, 0, -8) if S.vocab % c == 0)
        lr = T_("logits_rows", [S.vocab // chunk, chunk], exp=fin["logits"])
        add(ReshapeNode([lq], lr), "Reshape", domain="")
        lf = T_("logits_f32", [S.vocab // chunk, chunk], kind="f32")
        add(DequantRoNode([lr], lf), "LlmDequant")
        lo = T_("logits", [1, S.vocab], kind="f32")
        add(ReshapeNode([lf], lo), "Reshape", domain="")
        outputs.append(lo)
    graph_inputs = [ids_t, pos_t, n_t]
    if as_ops:
        return ops, reg, [t.onnx_name for t in graph_inputs], [t.onnx_name for t in outputs]
    g = Graph(nodes, input_tensors=graph_inputs, output_tensors=outputs)
    encode_matmul_weights(g.nodes, AP_FIXED_16_8)
    return g


def prefill_cache(decode_cache: np.ndarray, b: int) -> np.ndarray:
    """Sequence b's rows of a decode graph's cache values [B][KV][C][HD] as the prefill entry's
    logical [C][KV HD] (a copy)."""
    _, KV, C, HD = decode_cache.shape
    return np.ascontiguousarray(decode_cache[b].transpose(1, 0, 2)).reshape(C, KV * HD)


def decode_cache(prefill_cache_values: np.ndarray, out: np.ndarray, b: int) -> None:
    """The prefill entry's cache values [C][KV HD] into sequence b of a decode graph's [B][KV][C][HD]."""
    _, KV, C, HD = out.shape
    out[b] = np.asarray(prefill_cache_values).reshape(C, KV, HD).transpose(1, 0, 2)


def _decode_attention_unfused(nodes, T_, p, e, qr, kc2, vc2, om, B, KV, G, HD, keys, ctx, cmr, cfg, pos, pos_t):
    """A decode layer's attention as the reference's nodes: per (sequence, group) the group's G
    query rows against the cache's K rows, the scores query-major s[b g][h'][j] (the unit's
    column mode takes query blocks of 16, so the G queries of a decode step go through its row
    mode: VitAttnSoftmax's query_major calls, smx_nodes.py:250-253), the softmax, P.V."""
    qrows = T_(p + "qrows", [B * KV, G, HD], exp=e["q"])
    nodes.append(ReshapeNode([qr], qrows))
    kview = T_(p + "kc1v", [B * KV, ctx, HD], exp=e["k"])
    nodes.append(ReshapeNode([kc2], kview))
    st = T_(p + "s", [B * KV, G, keys], exp=e["s"])
    nodes.append(AttnContractNode([qrows, kview], st, b_trans=True))
    pr = T_(p + "P", [B * KV, G, keys], exp=e["p"])
    nodes.append(SoftmaxVopNode([st], pr, cm=cmr, cfg=cfg, mask=pos + 1, mask_t=pos_t, mask_add=1))
    vview = T_(p + "vc1v", [B * KV, ctx, HD], exp=e["v"])
    nodes.append(ReshapeNode([vc2], vview))
    o = T_(p + "o", [B * KV, G, HD], exp=e["o"])
    nodes.append(AttnContractNode([pr, vview], o))
    nodes.append(ReshapeNode([o], om))

