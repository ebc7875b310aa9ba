"""The row-ops unit's attention prep (AttnPrepRoNode: RoPE of q / k, the V re-round, the q.K^T x
image by TRANSPOSE, the cache rows written in place) and its Transpose node (TransposeRoNode:
head split as one COPY, K^T as one TRANSPOSE) on the GPU, against the oracle's restatement of
the reference's reference() (oracle/attn_prep.py): prefill rows (8-row tiles) with a partial
n, a decode step (one row, the group's heads as the tile), v at the V cache's exponents or
re-rounded, and several calls in a row over the same states."""
import math

import numpy as np
import pytest

from cormorant_amd.graph import Graph, TensorInfo
from cormorant_amd.models import rope_half_tables
from cormorant_amd.rowops_nodes import AttnPrepRoNode, TransposeRoNode
from cormorant_amd.simulate import Simulator
from oracle import graph_sim

pytestmark = pytest.mark.gpu


def _grid(rng, shape, f, lim=12000):
    """Values on the 2^-f grid (per channel of the last axis), raws within +-lim."""
    r = rng.integers(-lim, lim, shape)
    return r / np.power(2.0, np.asarray(f, np.float64))


def _prep_graph(T, H, KV, HD, C, with_n, v_direct, seed):
    rng = np.random.default_rng(seed)
    G = H // KV
    fq0 = np.repeat(rng.integers(9, 13, H), HD)                  # per head
    fk0 = np.repeat(rng.integers(9, 13, KV), HD)
    fv = np.repeat(rng.integers(9, 13, KV), HD)
    fkc = np.repeat(rng.integers(8, 12, KV), HD)                 # one per KV head
    fvc = fv.copy() if v_direct else np.repeat(rng.integers(7, 14, KV), HD)
    fq = rng.integers(8, 12, H)
    cos, sin = rope_half_tables(10000.0, HD, C)
    Ti = TensorInfo
    q0 = Ti("q0", [T, H * HD], exp=fq0)
    k0 = Ti("k0", [T, KV * HD], exp=fk0)
    v = Ti("v", [T, KV * HD], exp=fv)
    pos = Ti("pos", [1], kind="host")
    n = Ti("n", [1], kind="host")
    ck = Ti("ck", [C, KV * HD], exp=fkc, group_layout=(KV, HD), state=True)
    cv = Ti("cv", [C, KV * HD], exp=fvc, group_layout=(KV, HD), state=True)
    qx = Ti("qx", [KV, HD, G * T], exp=0)
    ins = [q0, k0, v, pos] + ([n] if with_n else []) + [ck, cv]
    node = AttnPrepRoNode(ins, qx, heads=H, kv_heads=KV, head_dim=HD, fq=fq, cos=cos, sin=sin)
    g = Graph([node], input_tensors=[t for t in ins if not t.state], output_tensors=[qx])

    def feeds(p, nv):
        f = {"q0": _grid(rng, (T, H * HD), fq0), "k0": _grid(rng, (T, KV * HD), fk0),
             "v": _grid(rng, (T, KV * HD), fv), "pos": np.array([p])}
        if with_n:
            f["n"] = np.array([nv])
        return f

    states = {"ck": _grid(rng, (C, KV * HD), fkc), "cv": _grid(rng, (C, KV * HD), fvc)}
    return g, feeds, states, node


@pytest.mark.parametrize("T,H,KV,HD,C,with_n,v_direct,steps", [
    (8, 4, 2, 32, 64, True, False, [(5, 6), (11, 8), (60, 8)]),     # prefill: partial n, clamped at C
    (16, 6, 3, 64, 128, True, True, [(0, 16), (16, 13)]),
    (1, 6, 2, 64, 128, False, False, [(77, 1), (78, 1), (127, 1)]),  # decode steps, G = 3
    (1, 15, 5, 64, 1024, False, True, [(1023, 1)]),                   # SmolLM2's heads at the last row
])
def test_attn_prep_steps(T, H, KV, HD, C, with_n, v_direct, steps):
    g, feeds, states, node = _prep_graph(T, H, KV, HD, C, with_n, v_direct, seed=T * 100 + H)
    assert node.v_direct == v_direct
    sim = Simulator(g)
    st_gpu = {k: v.copy() for k, v in states.items()}
    st_ref = {k: v.copy() for k, v in states.items()}
    for p, nv in steps:
        f = feeds(p, nv)
        print(f"attn prep T={T} H={H} KV={KV} HD={HD} C={C}: pos {p} n {nv}", flush=True)
        got = sim._forward_pass(f, states=st_gpu)
        want = graph_sim.forward(g, f, states=st_ref)
        np.testing.assert_array_equal(got["qx"], want["qx"].reshape(got["qx"].shape))
        for k in ("ck", "cv"):
            np.testing.assert_array_equal(st_gpu[k], st_ref[k], err_msg=k)
            np.testing.assert_array_equal(got[k], st_ref[k], err_msg=k)
    assert not np.array_equal(st_gpu["ck"], states["ck"]), "the K cache was not written"


@pytest.mark.parametrize("shape,perm,kind", [
    ((16, 3, 64), (1, 0, 2), "copy"),              # head split [T][H][HD] -> [H][T][HD]
    ((12, 384, 64), (1, 0, 2), "copy"),            # head merge of BERT's 12 heads
    ((1, 16, 3, 64), (0, 2, 1, 3), "copy"),        # with a unit batch axis
    ((6, 24, 64), (0, 2, 1), "xpose"),             # K^T per (sequence, head)
    ((40, 96), (1, 0), "xpose"),
])
def test_transpose_on_the_unit(shape, perm, kind):
    rng = np.random.default_rng(len(shape) + sum(perm))
    x = TensorInfo("x", list(shape), exp=10)
    y = TensorInfo("y", [shape[p] for p in perm], exp=10)
    node = TransposeRoNode([x], y, perm=perm)
    assert node.kind == kind
    g = Graph([node], input_tensors=[x], output_tensors=[y])
    xv = rng.integers(-32768, 32768, shape) / 1024.0
    got = Simulator(g).simulate({"x": xv})["y"]
    np.testing.assert_array_equal(got, graph_sim.forward(g, {"x": xv})["y"].reshape(got.shape))
    np.testing.assert_array_equal(got, np.transpose(xv, perm))
