"""The prefill_T entry (the reference's llama.py:28-33, 329-450, 465-497) on the oracle: its
attention softmax pinned by closed forms of the causal mask (smx_nodes.py:326-338), the whole
entry pinned to the decode step (one valid row at position p is that step, bit for bit, caches
included), and its caches against a float64 causal prefill."""
import math

import numpy as np
import pytest

from cormorant_amd import graph as G
from cormorant_amd import models
from oracle import graph_sim as og

SMALL = models.LlamaShape(layers=2, batch=1, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=128)


@pytest.fixture(scope="module")
def built():
    w = models.smollm2_weights(SMALL, 0)
    g, _, exps = models.smollm2_decode(SMALL, weights=w, runtime_pos=True)
    return w, g, exps


def _softmax_graph(T, Gq, C, causal=True, cm=None, cfg=None):
    s = G.TensorInfo("s", [C, Gq * T], exp=0)
    pos, n = G.TensorInfo("pos", [1], kind="host"), G.TensorInfo("n", [1], kind="host")
    p = G.TensorInfo("p", [Gq * T, C], exp=0)
    cm_, cfg_ = G.softmax_regs(10, 0.125, 14)
    node = G.AttnSoftmaxNode([s, pos, n], p, T=T, G=Gq, C=C, cm=cm_ if cm is None else cm,
                             cfg=cfg_ if cfg is None else cfg, causal=causal)
    return G.Graph([node], [s, pos, n], [p])


@pytest.mark.parametrize("pos,n", [(0, 16), (0, 5), (7, 16), (40, 3), (120, 16)])
def test_softmax_causal_closed_form(pos, n):
    """Equal scores: row t of every head spreads 2^14 evenly over its pos + 1 + t keys (the
    unit rounds each share alike), nothing past them and nothing at or past keys =
    roundup(pos + n, 16)."""
    T, Gq, C = 16, 2, 128
    g = _softmax_graph(T, Gq, C)
    P = og.forward(g, {"s": np.zeros((C, Gq * T)), "pos": np.array([pos]), "n": np.array([n])})["p"]
    n_c, keys = G.attn_keys(pos, n, T, C)
    for h in range(Gq):
        for t in range(T):
            row = P[h * T + t]
            v = min(keys, pos + 1 + t)
            assert (row[v:] == 0).all()
            assert (row[:v] == row[0]).all() and row[0] > 0
            assert abs(row[0] * v - 2 ** 14) <= v              # each share 2^14 / v, rounded
    assert (P[:, keys:] == 0).all()


def test_softmax_not_causal_closed_form():
    T, C, pos, n = 16, 64, 5, 9
    g = _softmax_graph(T, 1, C, causal=False)
    P = og.forward(g, {"s": np.zeros((C, T)), "pos": np.array([pos]), "n": np.array([n])})["p"]
    assert (P[:, :pos + n] == P[0, 0]).all() and (P[:, pos + n:] == 0).all()


def test_softmax_node_contract():
    with pytest.raises(G.SchedulerError):
        _softmax_graph(8, 1, 64)                    # query rows in blocks of 16
    with pytest.raises(G.SchedulerError):
        _softmax_graph(16, 1, 2048)                 # the unit's column mode takes 1024 keys
    with pytest.raises(G.SchedulerError):
        _softmax_graph(16, 2, 64, cm=[1, 2, 3])     # registers: one pair or one per head


def test_cache_views_round_trip():
    rng = np.random.default_rng(0)
    dec = rng.normal(size=(3, 2, 16, 8))
    pc = models.prefill_cache(dec, 1)
    assert pc.shape == (16, 16)
    # logical [C][KV HD]: row j, group g's columns are K_g[j]
    np.testing.assert_array_equal(pc[5, 8:16], dec[1, 1, 5])
    out = np.zeros_like(dec)
    models.decode_cache(pc, out, 2)
    np.testing.assert_array_equal(out[2], dec[1])


def test_prefill_one_row_is_the_decode_step(built):
    """A 16-row prefill with n = 1 at position 40 over a cache filled by a 64-row prefill equals
    the decode step at position 40 on the same cache: the logits, the new cache row of every
    layer and the residual row, bit for bit."""
    w, g, exps = built
    pg = models.smollm2_prefill(SMALL, 64, exps, w)
    p1 = models.smollm2_prefill(SMALL, 16, exps, w, with_head=True)
    rng = np.random.default_rng(3)
    st = {t.onnx_name: np.zeros(t.shape) for t in pg.state_tensors}
    og.forward(pg, {"ids": rng.integers(0, SMALL.vocab, 64).astype(float), "pos": np.array([0]),
                    "n": np.array([40])}, states=st)
    assert (st["l0.kc"][:40] != 0).any() and (st["l0.kc"][40:] == 0).all()
    dec = {t.onnx_name: np.zeros(t.shape) for t in g.state_tensors}
    for k in dec:
        models.decode_cache(st[k], dec[k], 0)
    x = int(rng.integers(0, SMALL.vocab))
    ids = np.concatenate([[x], rng.integers(0, SMALL.vocab, 15)]).astype(float)
    v1 = og.forward(p1, {"ids": ids, "pos": np.array([40]), "n": np.array([1])}, states=st)
    vd = og.forward(g, {"ids": np.array([float(x)]), "pos": np.array([40])}, states=dec)
    np.testing.assert_array_equal(v1["logits"].reshape(-1), vd["logits"].reshape(-1))
    np.testing.assert_array_equal(st["h_last"].reshape(-1), vd["l1.h"].reshape(-1))
    for k in dec:
        np.testing.assert_array_equal(models.prefill_cache(dec[k], 0), st[k])


def test_prefill_cache_rows_follow_float(built):
    """Layer 0's K cache rows are RoPE(RMSNorm(embedding) Wk) at their positions to within the
    cache's rounding and the projection's fixed-point error; rows past pos + n stay as they were."""
    w, _, exps = built
    emb, Ls, _ = w
    T, n, pos = 32, 29, 3
    pg = models.smollm2_prefill(SMALL, T, exps, w)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, SMALL.vocab, T)
    st = {t.onnx_name: np.zeros(t.shape) for t in pg.state_tensors}
    og.forward(pg, {"ids": ids.astype(float), "pos": np.array([pos]), "n": np.array([n])}, states=st)
    H, KV, HD = SMALL.heads, SMALL.kv, SMALL.hd
    cos, sin = models.rope_half_tables(SMALL.theta, HD, SMALL.ctx)
    x = models._rms(emb[ids].astype(np.float64), Ls[0]["g1"], SMALL.eps)
    k = x @ Ls[0]["wk"].astype(np.float64)
    kr = np.concatenate([models._rope_f(k[t:t + 1], KV, HD, cos[pos + t], sin[pos + t]) for t in range(n)])
    got = st["l0.kc"][pos:pos + n]
    assert np.abs(got - kr).max() < 0.03 * np.abs(kr).max()
    assert (st["l0.kc"][:pos] == 0).all() and (st["l0.kc"][pos + n:] == 0).all()


def test_prefill_contract(built):
    w, _, exps = built
    with pytest.raises(ValueError):
        models.smollm2_prefill(SMALL, 24, exps, w)                       # T a multiple of 16
    big = models.LlamaShape(layers=1, batch=1, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=2048)
    with pytest.raises(ValueError):
        models.smollm2_prefill(big, 16, exps, w)                          # the unit's 1024 keys
