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
from .graph import (AttnContractNode, ConvNode, Graph, MatmulNode, PermuteNode, PoolNode, ReshapeNode, ScheduledNode,
                    SoftmaxVopNode, TensorInfo, conv_out, softmax_regs)
from .rowops_nodes import LayerNorm32RoNode, ResAddBiasRoNode


def small_cnn(seed: int = 0):
    """(graph, inputs): the small CNN and one seeded input image."""
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
    return g, inputs


# ---------------------------------------------------------------- MobileNetV2-style CNN
# (expansion t, output channels c, repeats n, first stride s) of the 17 inverted residual blocks
MOBILENET_V2_BLOCKS = ((1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1),
                       (6, 160, 3, 2), (6, 320, 1, 1))


def mobilenet_v2(batch: int = 32, res: int = 224, seed: int = 0, classes: int = 1000):
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
    of a larger one.  ``macs`` counts the convolutions' and the classifier's multiply-adds."""
    T = TensorInfo
    rng_in = np.random.default_rng([seed, 0])
    x_val = np.round(rng_in.random((batch, 3, res, res)) * 256) / 256
    rng = np.random.default_rng([seed, 1])
    nodes, macs = [], [0]
    x_t = T("input", [batch, 3, res, res])
    cur = x_t
    count = [0]

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
        macs[0] += batch * cout * oh * ow * fan_in
        return y

    def relu6(x):
        y = T(name("relu6"), list(x.shape))
        nodes.append(ScheduledNode([x], y, units.OP_RELU6))
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
                h = y
            cur = h
    cur = relu6(conv(cur, 1280, 1, 1))
    pooled = T("pool", [batch, 1280, 1, 1])
    nodes.append(PoolNode([cur], pooled, units.POOL_AVG, cur.shape[2], cur.shape[3], 1, 1))
    flat = T("flat", [batch, 1280])
    nodes.append(ReshapeNode([pooled], flat))
    wf = T("fc.w", [1280, classes], data=rng.standard_normal((1280, classes)) * math.sqrt(2.0 / 1280))
    logits = T("logits", [batch, classes])
    nodes.append(MatmulNode([flat, wf], logits))
    macs[0] += batch * 1280 * classes
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


def bert_encoder(shape: BertShape = BertShape(), seed: int = 0, calib_seqs: int = 1):
    """(graph, inputs, exps): the BERT-base-shaped encoder in per-tensor power-of-two numerics.

    Token ids U{0 .. vocab-1} and embedding rows N(0, 1) (the embedding lookup is the host
    op whose result, the int32 residual at 2^-15, is the graph's input); per layer, in the
    arrangement of the reference's encoder template (vit.py:19-32):

        x  = LayerNorm32(h)                          row-ops NORM, int32 -> int16
        qkv = x . Wqkv                               MatMul (pow2, int32 wrap)
        q^T, K, V per head                           Permute (the head split)
        s  = K . q^T   [B H][keys][queries]          batched MatMul, f_s = f_q + f_k - 8
        P  = softmax over keys (column mode)         VectorOP softmax, logit scale 1/sqrt(hd)
        o  = P . V     [B H][queries][hd]            batched MatMul, f_o = f_p + f_v - 8
        h1 = ResAddBias(h, merge(o) . Wo, bo)        Permute, MatMul, row-ops ADDX
        x2 = LayerNorm32(h1);  f = x2 . W1  (at 2^-8)
        a  = GELU(f + b1)                            VectorOP ADD with the GELU act
        h  = ResAddBias(h1, a . W2, b2)

    Weights N(0, 0.02), biases N(0, 0.02), LayerNorm gamma N(1, 0.02), beta N(0, 0.02).
    Exponents: a float64 run of the first ``calib_seqs`` sequences gives each tensor's
    largest |value|, and each tensor takes the largest exponent that keeps it below 32767
    with a 1.25 margin; the contractions' output exponents follow from their operands', the
    q / v exponents are lowered where the scores or P.V would not fit.  ``exps`` records them.
    """
    from .numeric import encode_matmul_weights
    from .dtype import AP_FIXED_16_8

    S = shape
    # ids / embeddings and weights from their own generators: a smaller batch of the same seed
    # is the leading sequences of a larger one, with the same weights and exponents
    rng_in = np.random.default_rng([seed, 0])
    emb = rng_in.standard_normal((S.vocab, S.d), dtype=np.float32)
    ids = rng_in.integers(0, S.vocab, (S.batch, S.seq))
    h0 = emb[ids].astype(np.float64).reshape(S.batch * S.seq, S.d)
    del emb
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

    # ---- the integer graph
    T_ = TensorInfo
    rows, D = S.batch * S.seq, S.d
    BH = S.batch * H
    nodes = []
    h_in = T_("h0", [rows, D], exp=RES_BITS, kind="i32")
    hcur = h_in
    for li, (L, e) in enumerate(zip(Ls, exps)):
        p = f"l{li}."
        x1 = T_(p + "x1", [rows, D], exp=e["x1"])
        nodes.append(LayerNorm32RoNode([hcur], x1, gamma=L["g1"], beta=L["be1"], eps=S.eps))
        wqkv = T_(p + "wqkv", [D, 3 * D], data=L["wqkv"])
        qkv = T_(p + "qkv", [rows, 3 * D], exp=np.repeat([e["q"], e["k"], e["v"]], D))
        nodes.append(MatmulNode([x1, wqkv], qkv))
        ld = 3 * D
        qT = T_(p + "qT", [BH, hd, T], exp=e["q"])
        kh = T_(p + "kh", [BH, T, hd], exp=e["k"])
        vh = T_(p + "vh", [BH, T, hd], exp=e["v"])
        nodes.append(PermuteNode([qkv], qT, dims=(S.batch, H, hd, T), strides=(T * ld, hd, 1, ld), offset=0))
        nodes.append(PermuteNode([qkv], kh, dims=(S.batch, H, T, hd), strides=(T * ld, hd, ld, 1), offset=D))
        nodes.append(PermuteNode([qkv], vh, dims=(S.batch, H, T, hd), strides=(T * ld, hd, ld, 1), offset=2 * D))
        sc = T_(p + "s", [BH, T, T], exp=e["s"])
        nodes.append(AttnContractNode([kh, qT], sc))
        cmr, cfg = softmax_regs(e["s"], 1.0 / math.sqrt(hd), e["p"])
        pr = T_(p + "P", [BH, T, T], exp=e["p"])
        nodes.append(SoftmaxVopNode([sc], pr, cm=cmr, cfg=cfg, keys_major=True))
        o = T_(p + "o", [BH, T, hd], exp=e["o"])
        nodes.append(AttnContractNode([pr, vh], o))
        om = T_(p + "om", [rows, D], exp=e["o"])
        nodes.append(PermuteNode([o], om, dims=(S.batch, T, H, hd), strides=(H * T * hd, hd, T * hd, 1)))
        wo = T_(p + "wo", [D, D], data=L["wo"])
        ao = T_(p + "ao", [rows, D], exp=e["ao"])
        nodes.append(MatmulNode([om, wo], ao))
        h1 = T_(p + "h1", [rows, D], exp=RES_BITS, kind="i32")
        nodes.append(ResAddBiasRoNode([hcur, ao], h1, bias=L["bo"]))
        x2 = T_(p + "x2", [rows, D], exp=e["x2"])
        nodes.append(LayerNorm32RoNode([h1], x2, gamma=L["g2"], beta=L["be2"], eps=S.eps))
        w1 = T_(p + "w1", [D, S.ff], data=L["w1"])
        f = T_(p + "f", [rows, S.ff], exp=F_Q88)
        nodes.append(MatmulNode([x2, w1], f))
        b1 = T_(p + "b1", [S.ff], data=L["b1"])
        a = T_(p + "a", [rows, S.ff], exp=F_Q88)
        nodes.append(ScheduledNode([f, b1], a, units.OP_ADD, act=units.ACT_GELU))
        w2 = T_(p + "w2", [S.ff, D], data=L["w2"])
        dd = T_(p + "dd", [rows, D], exp=e["dd"])
        nodes.append(MatmulNode([a, w2], dd))
        hn = T_(p + "h", [rows, D], exp=RES_BITS, kind="i32")
        nodes.append(ResAddBiasRoNode([h1, dd], hn, bias=L["b2"]))
        hcur = hn
    g = Graph(nodes, input_tensors=[h_in], output_tensors=[hcur])
    encode_matmul_weights(g.nodes, AP_FIXED_16_8)
    return g, {"h0": h0}, exps
