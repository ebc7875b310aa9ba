"""Graphs with power-of-two numerics on the GPU against the value-domain restatement of the
reference simulator (oracle_graph): encoded MatMul / Conv weights (numeric.py), the int32
wrap, the prefill-attention contractions with a runtime key count, and a decoder-style chain
of row-ops adapters around a MatMul."""
import numpy as np
import pytest

from cormorant_amd import rowops_nodes as rn
from cormorant_amd.dtype import AP_FIXED_16_8 as DT
from cormorant_amd.graph import ConvNode, Graph, LlmAttnConvNode, MatmulNode, TensorInfo
from cormorant_amd.numeric import encode_conv_weights, encode_matmul_weights
from cormorant_amd.simulate import Simulator
from oracle import graph_sim as oracle_graph
from oracle.attn_prep import clamp_n

pytestmark = pytest.mark.gpu


def on_grid(rng, shape, exp, scale=1.0, lo=-32768, hi=32767):
    e = np.asarray(exp, np.float64)
    raw = np.clip(np.round(rng.normal(0, scale, shape) * 2.0 ** e), lo, hi)
    return raw / 2.0 ** e


def check(graph, inputs):
    got = Simulator(graph).simulate(inputs)
    want = oracle_graph.forward(graph, inputs)
    for t in graph.output_tensors:
        np.testing.assert_array_equal(got[t.onnx_name], want[t.onnx_name], err_msg=t.onnx_name)
    return got


@pytest.mark.parametrize("wrap_big", [False, True])
def test_pow2_matmul(wrap_big):
    rng = np.random.default_rng(11 + wrap_big)
    T, K, M = 6, 256 if wrap_big else 96, 40
    fa = np.full(K, 14) if wrap_big else rng.integers(8, 13, K)
    fo = np.full(M, 14) if wrap_big else rng.integers(6, 11, M)
    a = TensorInfo("a", [T, K], exp=fa)
    w = TensorInfo("w", [K, M], data=rng.normal(0, 40.0 if wrap_big else 0.05, (K, M)))
    c = TensorInfo("c", [T, M], exp=fo)
    g = Graph(nodes=[MatmulNode([a, w], c)], input_tensors=[a], output_tensors=[c])
    encode_matmul_weights(g.nodes, DT)
    x = on_grid(rng, (T, K), fa, 1.9 if wrap_big else 1.0)
    got = check(g, {"a": x})
    if wrap_big:                               # the sums do wrap: some outputs differ from the saturated ones
        acc = (x * 2.0 ** fa) @ (np.asarray(w.data) * 256.0)
        assert (np.abs(acc) >= 2.0 ** 31).any()


@pytest.mark.parametrize("dw", [False, True])
def test_pow2_conv_per_channel(dw):
    rng = np.random.default_rng(13 + dw)
    C, M, H = (8, 8, 9) if dw else (5, 12, 9)
    fx, fy = rng.integers(8, 12, C), rng.integers(6, 10, M)
    x = TensorInfo("x", [2, C, H, H], chexp=fx)
    w = TensorInfo("w", [M, 1 if dw else C, 3, 3], data=rng.normal(0, 0.3, (M, 1 if dw else C, 3, 3)))
    b = TensorInfo("b", [M], data=rng.normal(0, 0.5, M))
    y = TensorInfo("y", [2, M, H, H], chexp=fy)
    g = Graph(nodes=[ConvNode([x, w, b], y, pad_top=1, pad_left=1, is_depthwise=dw)], input_tensors=[x],
              output_tensors=[y])
    encode_conv_weights(g.nodes, DT)
    check(g, {"x": on_grid(rng, (2, C, H, H), fx.reshape(1, -1, 1, 1))})


@pytest.mark.parametrize("pos,n", [(5, 8), (0, 3), (50, 8), (64, 8)])
def test_attention_contractions(pos, n):
    rng = np.random.default_rng(17 + pos)
    KV, H, HD, T, C = 2, 4, 16, 8, 64
    G = H // KV
    fk = np.repeat(rng.integers(9, 12, KV), HD)
    kc = TensorInfo("kc", [C, KV * HD], exp=fk, group_layout=(KV, HD))
    vc = TensorInfo("vc", [C, KV * HD], exp=np.repeat(rng.integers(9, 12, KV), HD), group_layout=(KV, HD))
    qx = TensorInfo("qx", [KV, HD, G * T], exp=0)
    tp, tn = TensorInfo("pos", [1], kind="host"), TensorInfo("n", [1], kind="host")
    nodes, outs = [], []
    for grp in range(KV):
        s = TensorInfo(f"s{grp}", [C, G * T], exp=0)
        p = TensorInfo(f"p{grp}", [G * T, C], exp=0)
        o = TensorInfo(f"o{grp}", [G * T, HD], exp=0)
        geo = dict(group=grp, T=T, H=H, KV=KV, HD=HD, C=C)
        nodes += [LlmAttnConvNode([kc, qx, tp, tn], s, kind="qk", **geo),
                  LlmAttnConvNode([p, vc, tp, tn], o, kind="pv", **geo)]
        outs += [s, o]
    prob_inputs = {f"p{grp}": rng.integers(0, 4096, (G * T, C)).astype(np.float64) for grp in range(KV)}
    g = Graph(nodes=nodes, input_tensors=[kc, vc, qx, tp, tn] + [TensorInfo(k, [G * T, C], exp=0) for k in prob_inputs],
              output_tensors=outs)
    inputs = {"kc": on_grid(rng, (C, KV * HD), fk, 8.0), "vc": on_grid(rng, (C, KV * HD), vc.exp, 8.0),
              "qx": rng.integers(-32768, 32768, (KV, HD, G * T)).astype(np.float64),
              "pos": np.array([pos]), "n": np.array([n]), **prob_inputs}
    got = check(g, inputs)
    keys = clamp_n(pos, n, T, C)[1]
    assert (got["s0"][keys:] == 0).all()


def test_decoder_chain():
    """h (int32 residual) -> RMSNorm -> MatMul (pow2) -> ResAdd -> Dequant."""
    rng = np.random.default_rng(19)
    T, D, M, fr = 8, 64, 64, 15
    fy = rng.integers(9, 12, D)
    fd = rng.integers(9, 13, M)
    h = TensorInfo("h", [T, D], exp=fr, kind="i32")
    y = TensorInfo("y", [T, D], exp=fy)
    w = TensorInfo("w", [D, M], data=rng.normal(0, 0.1, (D, M)))
    d = TensorInfo("d", [T, M], exp=fd)
    h1 = TensorInfo("h1", [T, M], exp=fr, kind="i32")
    out = TensorInfo("out", [T, M], kind="f32")
    nodes = [rn.RMSNormRoNode([h], y, gamma=rng.uniform(0.5, 1.5, D), eps=1e-5), MatmulNode([y, w], d),
             rn.ResAddRoNode([h, d], h1), rn.DequantRoNode([h1], out)]
    g = Graph(nodes=nodes, input_tensors=[h], output_tensors=[h1, out])
    encode_matmul_weights(g.nodes, DT)
    check(g, {"h": np.round(rng.normal(0, 3.0, (T, D)) * 2.0 ** fr) / 2.0 ** fr})
