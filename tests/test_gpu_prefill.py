"""The prefill_T entry on the HIP units (the reference's llama.py:28-33, 329-450, 465-497)
against the oracle's forward pass: a 64-row prefill of every sequence into the decode graph's KV
caches, then two decode steps over them; the one-row prefill equal to the decode step; the
attention softmax's per-head and non-causal forms."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _shape(batch):
    from cormorant_amd import models
    return models.LlamaShape(layers=2, batch=batch, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=128)


def _assert_same(got, want, names=None):
    for name in (want if names is None else names):
        if name in got:
            np.testing.assert_array_equal(np.asarray(got[name]).reshape(-1), np.asarray(want[name]).reshape(-1),
                                          err_msg=name)


def test_prefill_64_rows_then_two_decode_steps(torch_gpu):
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as og
    S = _shape(2)
    w = models.smollm2_weights(S, 1)
    g, _, exps = models.smollm2_decode(S, seed=1, weights=w, runtime_pos=True)
    pg = models.smollm2_prefill(S, 64, exps, w, with_head=True)
    sim_d = Simulator(g)
    sim_p = Simulator(pg, share=sim_d)
    dec_g = {t.onnx_name: np.zeros(t.shape) for t in g.state_tensors}
    dec_o = {k: v.copy() for k, v in dec_g.items()}
    rng = np.random.default_rng(21)
    n = 60
    for b in range(S.batch):
        print(f"prefill sequence {b}: T 64, pos 0, n {n}", flush=True)
        feeds = {"ids": rng.integers(0, S.vocab, 64).astype(np.float64), "pos": np.array([0]), "n": np.array([n])}
        ps_g = {k: models.prefill_cache(v, b) for k, v in dec_g.items()}
        ps_g["h_last"] = np.zeros((1, S.d))
        ps_o = {k: v.copy() for k, v in ps_g.items()}
        got = sim_p._forward_pass(feeds, states=ps_g)
        want = og.forward(pg, feeds, states=ps_o)
        _assert_same(got, want)
        for k in ps_o:
            np.testing.assert_array_equal(ps_g[k], ps_o[k], err_msg=k)
        assert (ps_g["l1.kc"][:n] != 0).any() and (ps_g["l1.kc"][n:] == 0).all()
        for k in dec_g:
            models.decode_cache(ps_g[k], dec_g[k], b)
            models.decode_cache(ps_o[k], dec_o[k], b)
    for step in range(2):
        print(f"decode step {step} at position {n + step}", flush=True)
        feeds = {"ids": rng.integers(0, S.vocab, S.batch).astype(np.float64), "pos": np.array([n + step])}
        got = sim_d._forward_pass(feeds, states=dec_g)
        want = og.forward(g, feeds, states=dec_o)
        _assert_same(got, want, ["logits"])
        for k in dec_o:
            np.testing.assert_array_equal(dec_g[k], dec_o[k], err_msg=k)


def test_one_row_prefill_is_the_decode_step(torch_gpu):
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator
    S = _shape(1)
    w = models.smollm2_weights(S, 2)
    g, _, exps = models.smollm2_decode(S, seed=2, weights=w, runtime_pos=True)
    pg = models.smollm2_prefill(S, 32, exps, w)
    p1 = models.smollm2_prefill(S, 16, exps, w, with_head=True)
    sim_d = Simulator(g)
    sim_p, sim_1 = Simulator(pg, share=sim_d), Simulator(p1, share=sim_d)
    rng = np.random.default_rng(4)
    st = {t.onnx_name: np.zeros(t.shape) for t in pg.state_tensors}
    sim_p._forward_pass({"ids": rng.integers(0, S.vocab, 32).astype(float), "pos": np.array([0]),
                         "n": np.array([32])}, states=st)
    dec = {t.onnx_name: np.zeros(t.shape) for t in g.state_tensors}
    for k in dec:
        models.decode_cache(st[k], dec[k], 0)
    x = int(rng.integers(0, S.vocab))
    ids = np.concatenate([[x], rng.integers(0, S.vocab, 15)]).astype(float)
    v1 = sim_1._forward_pass({"ids": ids, "pos": np.array([32]), "n": np.array([1])}, states=st)
    vd = sim_d._forward_pass({"ids": np.array([float(x)]), "pos": np.array([32])}, states=dec)
    np.testing.assert_array_equal(v1["logits"].reshape(-1), vd["logits"].reshape(-1))
    for k in dec:
        np.testing.assert_array_equal(models.prefill_cache(dec[k], 0), st[k], err_msg=k)


@pytest.mark.parametrize("causal,per_head,pos,n", [(True, False, 0, 32), (True, True, 37, 20), (False, False, 11, 7),
                                                   (True, False, 100, 32), (False, True, 0, 1)])
def test_attention_softmax_node(torch_gpu, causal, per_head, pos, n):
    from cormorant_amd import graph as G
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as og
    T, Gq, C = 32, 3, 128
    rng = np.random.default_rng(pos + n)
    s = G.TensorInfo("s", [C, Gq * T], exp=0)
    tp, tn = G.TensorInfo("pos", [1], kind="host"), G.TensorInfo("n", [1], kind="host")
    p = G.TensorInfo("p", [Gq * T, C], exp=0)
    regs = [G.softmax_regs(f, 0.125, 14) for f in (9, 10, 11)]
    cm = [r[0] for r in regs] if per_head else regs[1][0]
    cfg = [r[1] for r in regs] if per_head else regs[1][1]
    g = G.Graph([G.AttnSoftmaxNode([s, tp, tn], p, T=T, G=Gq, C=C, cm=cm, cfg=cfg, causal=causal)], [s, tp, tn], [p])
    feeds = {"s": rng.integers(-3000, 3000, (C, Gq * T)).astype(np.float64), "pos": np.array([pos]),
             "n": np.array([n])}
    got = Simulator(g).simulate(feeds)["p"]
    want = og.forward(g, feeds)["p"]
    np.testing.assert_array_equal(got, want)
    keys = G.attn_keys(pos, n, T, C)[1]
    assert (got[:, keys:] == 0).all() and (got[:, :keys] > 0).any()
