"""The SmolLM2-shaped decode step on the GPU (Simulator) against the value-domain
restatement of the reference simulator (oracle_graph), every tensor bit for bit: RMSNorm,
RoPE at the step's position, the residual adds and SiLU x up on row-ops, the pow2 linears and
the tied head, the KV-cache row writes, the batched q.K^T / P.V contractions over the whole
cache, the row-mode softmax and the float32 dequant of the logits."""
import numpy as np
import pytest

from cormorant_amd import models
from cormorant_amd.simulate import Simulator
from oracle import graph_sim as oracle_graph

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,seed", [
    (models.LlamaShape(layers=2, batch=3, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=64), 1),
    (models.LlamaShape(layers=1, batch=2, vocab=4096, ctx=256), 2),
    # the configuration's own step: 16 sequences (the 16-row skinny products and the grouped
    # q / k / v and gate / up launches), 1024-row caches, the 49152-column tied head
    (models.LlamaShape(layers=1, batch=16), 5),
    # the whole 32-layer stack at full width (two sequences, a 4096-row head, 256-row caches)
    (models.LlamaShape(layers=32, batch=2, vocab=4096, ctx=256), 7),
])
def test_decode_step_every_tensor(shape, seed):
    g, inputs, _ = models.smollm2_decode(shape, seed=seed)
    assert any(type(n).__name__ == "DecodeAttentionNode" for n in g.nodes)
    got = Simulator(g)._forward_pass(inputs)
    want = oracle_graph.forward(g, inputs)
    for name, v in got.items():
        np.testing.assert_array_equal(v, want[name].reshape(v.shape), err_msg=name)


@pytest.mark.parametrize("shape,seed", [
    (models.LlamaShape(layers=2, batch=3, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=64), 1),
    (models.LlamaShape(layers=1, batch=16), 5),
])
def test_decode_step_unfused_attention(shape, seed):
    """The same step with the attention as the two contractions around the softmax node (s and
    P materialized and compared too)."""
    g, inputs, _ = models.smollm2_decode(shape, seed=seed, fused_attention=False)
    got = Simulator(g)._forward_pass(inputs)
    want = oracle_graph.forward(g, inputs)
    for name, v in got.items():
        np.testing.assert_array_equal(v, want[name].reshape(v.shape), err_msg=name)


def test_decode_steps_over_states():
    """Successive decode steps of one graph with a runtime position: each step's K / V rows land
    in the caches (persistent states, updated in place), and the next step reads them; every
    tensor and the caches after every step against the oracle run over its own states."""
    shape = models.LlamaShape(layers=2, batch=3, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=64)
    g, inputs, _ = models.smollm2_decode(shape, seed=7, runtime_pos=True)
    sim = Simulator(g)
    names = [t.onnx_name for t in g.state_tensors]
    assert len(names) == 2 * shape.layers
    st_gpu = {nm: np.array(inputs[nm], np.float64) for nm in names}
    st_ref = {nm: np.array(inputs[nm], np.float64) for nm in names}
    rng = np.random.default_rng(8)
    for pos in (40, 41, 42, 63):
        feeds = {"ids": rng.integers(0, shape.vocab, shape.batch).astype(np.float64), "pos": np.array([pos])}
        print(f"decode step at {pos}", flush=True)
        got = Simulator._forward_pass(sim, feeds, states=st_gpu)
        want = oracle_graph.forward(g, feeds, states=st_ref)
        for name, v in got.items():
            np.testing.assert_array_equal(v, np.asarray(want[name]).reshape(v.shape), err_msg=f"pos {pos}: {name}")
        for nm in names:
            np.testing.assert_array_equal(st_gpu[nm], st_ref[nm], err_msg=f"pos {pos}: state {nm}")
    # the rows written are the steps' positions
    k0 = st_gpu[names[0]]
    assert not np.array_equal(k0[:, :, 40:43], np.asarray(inputs[names[0]])[:, :, 40:43])
