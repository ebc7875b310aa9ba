"""Residual statistics on the GPU (Simulator.compute_quant_errors / _forward_pass(errors_out=...),
the reference's _simulate.py:77-118, 409-422, 594-602) against the oracle's restatement over
the same ramp inputs: the same nodes recorded, abs_max equal and the norms' ratios equal to
float64 rounding."""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _compare(got, want):
    assert set(got) == set(want), (sorted(set(got) ^ set(want)))
    for name, w in want.items():
        g = got[name]
        for gv, wv, what in zip(g, w, ("abs_max", "nrmse", "sqnr_db")):
            if math.isinf(wv) or math.isnan(wv):
                assert gv == wv or (math.isnan(gv) and math.isnan(wv)), (name, what, gv, wv)
            else:
                assert gv == pytest.approx(wv, rel=1e-9, abs=1e-15), (name, what, gv, wv)


def _check(g, inputs=None):
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as oracle_graph
    sim = Simulator(g)
    if inputs is None:
        got = sim.compute_quant_errors()
        inputs = sim._build_ramp_inputs()
    else:
        got = {}
        sim._forward_pass(inputs, errors_out=got)
    want = {}
    oracle_graph.forward(g, inputs, errors_out=want)
    _compare(got, want)
    return got


def test_small_cnn_ramp(torch_gpu):
    from cormorant_amd import models
    g, _ = models.small_cnn(0)
    got = _check(g)
    assert len(got) >= 6
    # truncation at 2^-8: every unsaturated residual is below one step
    assert all(s.abs_max < 1.0 / 256 or s.abs_max > 1.0 for s in got.values())


def test_small_cnn_seeded_input(torch_gpu):
    from cormorant_amd import models
    g, inputs = models.small_cnn(3)
    _check(g, inputs)


def test_units_mix(torch_gpu):
    """Every kind of node that records: convs (bias / none, depthwise, stride, dilation), the
    three pools (count_include_pad both ways, LP1 / LP2), VectorOP ops with RELU / RELU6 and the
    activation unit, a batched MatMul; a reshape that records nothing."""
    from cormorant_amd import graph as G
    rng = np.random.default_rng(11)

    def w(name, shape, lo=-1.0, hi=1.0):
        return G.TensorInfo(name, shape, data=rng.uniform(lo, hi, shape))

    x = G.TensorInfo("x", [2, 4, 12, 12])
    c1 = G.TensorInfo("c1", [2, 8, 12, 12])
    c2 = G.TensorInfo("c2", [2, 8, 6, 6])
    c3 = G.TensorInfo("c3", [2, 8, 8, 8])
    p1 = G.TensorInfo("p1", [2, 8, 3, 3])
    p2 = G.TensorInfo("p2", [2, 8, 3, 3])
    p3 = G.TensorInfo("p3", [2, 8, 6, 6])
    p4 = G.TensorInfo("p4", [2, 8, 4, 4])
    v1 = G.TensorInfo("v1", [2, 8, 3, 3])
    v2 = G.TensorInfo("v2", [2, 8, 3, 3])
    v3 = G.TensorInfo("v3", [2, 8, 3, 3])
    v4 = G.TensorInfo("v4", [2, 8, 3, 3])
    r = G.TensorInfo("r", [2, 8, 9])
    m = G.TensorInfo("m", [2, 8, 5])
    nodes = [
        G.ConvNode([x, w("w1", [8, 4, 3, 3], -0.25, 0.25), w("b1", [8])], c1, pad_top=1, pad_left=1),
        G.ConvNode([c1, w("w2", [8, 1, 3, 3])], c2, stride_h=2, stride_w=2, pad_top=1, pad_left=1,
                   is_depthwise=True),
        G.ConvNode([c1, w("w3", [8, 8, 3, 3], -0.1, 0.1)], c3, dilation_h=2, dilation_w=2),
        G.PoolNode([c2], p1, G.POOL_MAX, 2, 2, 2, 2),
        G.PoolNode([c2], p2, G.POOL_AVG, 3, 3, 2, 2, 1, 1, count_include_pad=0),
        G.PoolNode([c2], p3, G.POOL_AVG, 3, 3, 1, 1, 1, 1, count_include_pad=1),
        G.PoolNode([c3], p4, G.POOL_LP, 3, 3, 2, 2, 1, 1, lp_order=2),
        G.ScheduledNode([p1, p2], v1, G.OP_MUL, act=2),
        G.ScheduledNode([v1, w("d", [3, 3], 0.5, 2.0)], v2, G.OP_DIV),
        G.ScheduledNode([v2, p1], v3, G.OP_SUB, act=5),
        G.ScheduledNode([v3], v4, 7),
        G.ReshapeNode([v4], r),
        G.MatmulNode([r, w("w4", [9, 5])], m),
    ]
    g = G.Graph(nodes, [x], [m, p3, p4])
    got = _check(g)
    assert "r" not in got and {"c1", "c2", "c3", "p1", "p2", "p3", "p4", "v1", "v2", "v3", "v4", "m"} <= set(got)
    inputs = {"x": np.round(rng.uniform(-3, 3, (2, 4, 12, 12)) * 256) / 256}
    _check(g, inputs)


def test_mobilenet_v2_small(torch_gpu):
    from cormorant_amd import models
    g, inputs, _ = models.mobilenet_v2(batch=2, res=32, seed=1)
    _check(g, inputs)


def test_bert_small_pow2(torch_gpu):
    """Power-of-two MatMuls (the reference's _matmul_exp residual, :814-835) and the GELU unit."""
    from cormorant_amd import models
    shape = models.BertShape(layers=1, batch=1, seq=64, d=128, heads=2, ff=256, vocab=300)
    g, inputs, _ = models.bert_encoder(shape, seed=2)
    got = _check(g, inputs)
    assert any(s.abs_max > 0 for s in got.values())
