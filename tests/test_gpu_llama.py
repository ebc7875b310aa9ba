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
])
def test_decode_step_every_tensor(shape, seed):
    g, inputs, _ = models.smollm2_decode(shape, seed=seed)
    got = Simulator(g)._forward_pass(inputs)
    want = oracle_graph.forward(g, inputs)
    for name, v in got.items():
        np.testing.assert_array_equal(v, want[name].reshape(v.shape), err_msg=name)
