"""VitAttnPrep on the row-ops unit (VitAttnPrepRoNode, the reference's rowops_nodes.py:1415-1712)
and the encoder template's attention chain on the HIP units, against the oracle."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.parametrize("fused_qkv,query_major,bias", [(False, False, True), (True, False, False),
                                                        (False, True, True), (True, True, True)])
def test_vit_attn_prep_node(torch_gpu, fused_qkv, query_major, bias):
    from cormorant_amd.graph import Graph, TensorInfo
    from cormorant_amd.rowops_nodes import VitAttnPrepRoNode
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as og
    rng = np.random.default_rng(int(fused_qkv) * 4 + int(query_major) * 2 + int(bias))
    T, H, HD = 32, 3, 32
    D = H * HD
    fx = rng.integers(8, 12, 3 * D)                              # per-column exponents of the projections
    kc = TensorInfo("kc", [T, D], exp=0, group_layout=(H, HD), state=True)
    vc = TensorInfo("vc", [T, D], exp=0, group_layout=(H, HD), state=True)
    qx = TensorInfo("qx", [H, HD, T], exp=0)
    if fused_qkv:
        qkv = TensorInfo("qkv", [T, 3 * D], exp=fx)
        srcs, cols, ins = [qkv, qkv, qkv], (0, D, 2 * D), [qkv]
        feeds = {"qkv": np.round(rng.normal(0, 4, (T, 3 * D)) * 2.0 ** fx) / 2.0 ** fx}
    else:
        srcs = [TensorInfo(n, [T, D], exp=fx[i * D:(i + 1) * D]) for i, n in enumerate(("q", "k", "v"))]
        cols, ins = (0, 0, 0), srcs
        feeds = {t.onnx_name: np.round(rng.normal(0, 4, (T, D)) * 2.0 ** t.exp) / 2.0 ** t.exp for t in srcs}
    b = (lambda: rng.normal(0, 0.5, D)) if bias else (lambda: None)
    node = VitAttnPrepRoNode(srcs + [kc, vc], qx, heads=H, head_dim=HD, fq=rng.integers(7, 11, H),
                             fk=rng.integers(7, 11, H), fv=rng.integers(7, 11, D), bq=b(), bk=b(), bv=b(),
                             cols=cols, query_major=query_major)
    g = Graph([node], ins, [qx])
    sim = Simulator(g)
    st_g = sim.initial_states()
    st_o = {k: v.copy() for k, v in st_g.items()}
    got = sim._forward_pass(feeds, states=st_g)
    want = og.forward(g, feeds, states=st_o)
    np.testing.assert_array_equal(got["qx"], want["qx"])
    for k in st_o:
        np.testing.assert_array_equal(st_g[k], st_o[k], err_msg=k)
    assert np.abs(st_g["kc"]).max() > 0 and np.abs(got["qx"]).max() > 0


def test_encoder_prep_chain(torch_gpu):
    """The encoder with the reference's own attention chain (one sequence of 64 tokens, 2 layers):
    every tensor equals the oracle's, and the output equals the fused attention's on the GPU."""
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as og
    S = models.BertShape(layers=2, batch=1, seq=64, d=128, heads=2, ff=256, vocab=300)
    gp, inputs, _ = models.bert_encoder(S, seed=5, prep_attention=True)
    gf, _, _ = models.bert_encoder(S, seed=5)
    got = Simulator(gp)._forward_pass(inputs)
    want = og.forward(gp, inputs)
    for name in want:
        if name in got:
            np.testing.assert_array_equal(np.asarray(got[name]).reshape(-1), np.asarray(want[name]).reshape(-1),
                                          err_msg=name)
    out = gp.output_tensors[0].onnx_name
    np.testing.assert_array_equal(Simulator(gf).simulate(inputs)[out], got[out])
