"""The host ops inside simulator graphs on the GPU, against the oracle, every tensor bit for bit:
a decode layer on the reference's host-attention path (the token-id embedding gathered on the
GPU into the float residual; RMSNorm, the attention with its KV caches as states, SiLU x up,
the residual adds and the dequant on the host; the pow2 MatMuls on the GPU units) over several
positions with the states carried from step to step; the ONNX host ops (LayerNorm, GELU,
Softmax) around a Q8.8 MatMul; and the embedding into the int32 residual."""
import numpy as np
import pytest

from cormorant_amd.dtype import AP_FIXED_16_8
from cormorant_amd.graph import Graph, MatmulNode, TensorInfo as T
from cormorant_amd.host_ops import (GeluNode, LayerNormNode, LlmAttentionNode, LlmDequantNode, LlmEmbedNode,
                                    LlmResAddNode, LlmRMSNormNode, LlmSiluMulNode, SoftmaxNode)
from cormorant_amd.models import rope_half_tables
from cormorant_amd.numeric import encode_matmul_weights
from cormorant_amd.rowops_nodes import LayerNorm32RoNode
from cormorant_amd.simulate import Simulator
from oracle import graph_sim

pytestmark = pytest.mark.gpu


def _host_decode_layer(d=64, H=4, KV=2, HD=16, ff=128, vocab=300, C=32, seed=0):
    rng = np.random.default_rng(seed)
    w = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)   # noqa: E731
    emb = rng.standard_normal((vocab, d)).astype(np.float32) * np.float32(0.5)
    cos, sin = rope_half_tables(10000.0, HD, C)
    A, K = H * HD, KV * HD
    nodes = []
    ids = T("ids", [1], exp=0, kind="i32")
    h = T("h", [1, d], kind="f32")
    nodes.append(LlmEmbedNode([ids], h, table=emb))
    x = T("x", [1, d], exp=12)
    nodes.append(LlmRMSNormNode([h], x, gamma=1.0 + w(d), eps=1e-5))
    q, k, v = T("q", [1, A], exp=12), T("k", [1, K], exp=12), T("v", [1, K], exp=11)
    for out, n_out in ((q, A), (k, K), (v, K)):
        nodes.append(MatmulNode([x, T("w" + out.onnx_name, [d, n_out], data=w(d, n_out) * 20)], out))
    pos = T("pos", [1], kind="host")
    ck = T("ck", [C, K], exp=11, group_layout=(KV, HD), state=True)
    cv = T("cv", [C, K], exp=10, group_layout=(KV, HD), state=True)
    o = T("o", [1, A], exp=12)
    nodes.append(LlmAttentionNode([q, k, v, pos, ck, cv], o, heads=H, kv_heads=KV, head_dim=HD, cos=cos, sin=sin))
    a = T("a", [1, d], exp=13)
    nodes.append(MatmulNode([o, T("wo", [A, d], data=w(A, d) * 20)], a))
    h1 = T("h1", [1, d], kind="f32")
    nodes.append(LlmResAddNode([h, a], h1))
    x2 = T("x2", [1, d], exp=12)
    nodes.append(LlmRMSNormNode([h1], x2, gamma=1.0 + w(d), eps=1e-5))
    g, u = T("g", [1, ff], exp=12), T("u", [1, ff], exp=12)
    nodes.append(MatmulNode([x2, T("wg", [d, ff], data=w(d, ff) * 20)], g))
    nodes.append(MatmulNode([x2, T("wu", [d, ff], data=w(d, ff) * 20)], u))
    m = T("m", [1, ff], exp=12)
    nodes.append(LlmSiluMulNode([g, u], m))
    dd = T("dd", [1, d], exp=13)
    nodes.append(MatmulNode([m, T("wd", [ff, d], data=w(ff, d) * 20)], dd))
    h2 = T("h2", [1, d], kind="f32")
    nodes.append(LlmResAddNode([h1, dd], h2))
    xf = T("xf", [1, d], exp=12)
    nodes.append(LlmRMSNormNode([h2], xf, gamma=1.0 + w(d), eps=1e-5))
    lq = T("lq", [1, vocab], exp=10)
    nodes.append(MatmulNode([xf, T("head", [d, vocab], data=np.ascontiguousarray(emb.T) * 0.05)], lq))
    lo = T("logits", [1, vocab], kind="f32")
    nodes.append(LlmDequantNode([lq], lo))
    gr = Graph(nodes, input_tensors=[ids, pos], output_tensors=[lo])
    encode_matmul_weights(gr.nodes, AP_FIXED_16_8)
    states = {"ck": rng.integers(-2000, 2000, (C, K)) / 2.0 ** 11, "cv": rng.integers(-2000, 2000, (C, K)) / 2.0 ** 10}
    return gr, states


def test_host_attention_decode_steps():
    g, states = _host_decode_layer()
    sim = Simulator(g)
    st_gpu = {k: v.copy() for k, v in states.items()}
    st_ref = {k: v.copy() for k, v in states.items()}
    for step, (tok, p) in enumerate(((17, 5), (250, 6), (3, 7), (-4, 31))):
        feeds = {"ids": np.array([tok]), "pos": np.array([p])}
        print(f"host decode step {step}: id {tok} at {p}", flush=True)
        got = sim._forward_pass(feeds, states=st_gpu)
        want = graph_sim.forward(g, feeds, states=st_ref)
        for name, v in got.items():
            np.testing.assert_array_equal(v, np.asarray(want[name]).reshape(v.shape), err_msg=f"step {step}: {name}")
        for k in states:
            np.testing.assert_array_equal(st_gpu[k], st_ref[k], err_msg=k)
    assert not np.array_equal(st_gpu["ck"], states["ck"])


def test_onnx_host_ops_around_a_matmul():
    rng = np.random.default_rng(4)
    x = T("x", [8, 96])
    y1 = T("ln", [8, 96])
    wt = T("w", [96, 64], data=rng.uniform(-0.25, 0.25, (96, 64)))
    y2 = T("mm", [8, 64])
    y3 = T("gelu", [8, 64])
    y4 = T("tanh", [8, 64])
    y5 = T("sm", [8, 64])
    nodes = [LayerNormNode([x], y1, gamma=(1 + 0.1 * rng.standard_normal(96)).astype(np.float32),
                           beta=(0.1 * rng.standard_normal(96)).astype(np.float32), eps=1e-5),
             MatmulNode([y1, wt], y2), GeluNode([y2], y3), GeluNode([y3], y4, approximate="tanh"),
             SoftmaxNode([y4], y5)]
    g = Graph(nodes, input_tensors=[x], output_tensors=[y5])
    xv = rng.integers(-3000, 3000, (8, 96)) / 256.0
    got = Simulator(g)._forward_pass({"x": xv})
    want = graph_sim.forward(g, {"x": xv})
    for name, v in got.items():
        np.testing.assert_array_equal(v, want[name].reshape(v.shape), err_msg=name)


def test_embedding_into_the_int32_residual():
    """Token ids (clamped into the table) -> the int32 residual at 2^-15 -> LayerNorm32 on the unit."""
    rng = np.random.default_rng(6)
    tab = rng.standard_normal((1000, 256)).astype(np.float32)
    ids = T("ids", [64], exp=0, kind="i32")
    h = T("h", [64, 256], exp=15, kind="i32")
    x = T("x", [64, 256], exp=12)
    g = Graph([LlmEmbedNode([ids], h, table=tab),
               LayerNorm32RoNode([h], x, gamma=np.ones(256), beta=np.zeros(256), eps=1e-6)],
              input_tensors=[ids], output_tensors=[x])
    idv = rng.integers(-5, 1005, 64)
    got = Simulator(g)._forward_pass({"ids": idv})
    want = graph_sim.forward(g, {"ids": idv})
    for name in ("h", "x"):
        np.testing.assert_array_equal(got[name], want[name].reshape(got[name].shape), err_msg=name)
