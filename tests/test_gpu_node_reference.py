"""The per-node reference(ins, dtype) contract on the GPU: each graph run node at a time, every
node through its own ``reference`` (a one-node run of the units; host ops through their C++
host arithmetic) on the values its predecessors produced, equals the whole graph's pass tensor
for tensor, persistent states included (the reference's _forward_pass calling
sn.reference(ins, dtype) per LlmKernelNode / HostNode, _simulate.py:667-690)."""
import numpy as np
import pytest

from cormorant_amd import models
from cormorant_amd.dtype import AP_FIXED_16_8 as DT
from cormorant_amd.simulate import Simulator

pytestmark = pytest.mark.gpu

TINY_BERT = models.BertShape(layers=1, batch=1, seq=64, d=128, heads=2, ff=256, vocab=500)
TINY_LLAMA = models.LlamaShape(layers=2, batch=2, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=64)


def node_at_a_time(g, inputs):
    """Every node's reference() in graph order over a value table seeded by the inputs and the
    states' initial values; in-place state writers update the state's entry."""
    sim = Simulator(g)
    vals = {k: np.asarray(v, np.float64) for k, v in sim.initial_states().items()}
    vals.update({k: np.asarray(v) for k, v in inputs.items()})
    for sn in g.nodes:
        ins = [None if t is None else vals.get(t.onnx_name) for t in sn.inputs]
        vals[sn.output.onnx_name] = np.asarray(sn.reference(ins, DT, host=vals))
    return vals


@pytest.mark.parametrize("label,build", [
    ("small CNN", lambda: models.small_cnn(1)[:2]),
    ("MobileNetV2 32x32", lambda: models.mobilenet_v2(batch=1, res=32, seed=1)[:2]),
    ("encoder layer, fused attention", lambda: models.bert_encoder(TINY_BERT, seed=1)[:2]),
    ("encoder layer, unit contractions", lambda: models.bert_encoder(TINY_BERT, seed=2, fused_attention=False)[:2]),
    ("decode step, runtime position and states", lambda: models.smollm2_decode(TINY_LLAMA, seed=3,
                                                                                 runtime_pos=True)[:2]),
])
def test_node_at_a_time_equals_the_graph(label, build):
    g, inputs = build()
    states = Simulator(g).initial_states()
    whole = Simulator(g)._forward_pass(inputs, states=states)
    per_node = node_at_a_time(g, inputs)
    assert len(g.nodes) > 3
    for name, v in whole.items():
        np.testing.assert_array_equal(np.asarray(per_node[name]).reshape(v.shape), v, err_msg=f"{label}: {name}")


def test_reference_refuses_a_missing_input():
    g, _ = models.small_cnn(1)[:2]
    sn = next(n for n in g.nodes if n.inputs[0].data is None)
    with pytest.raises(ValueError, match="no value"):
        sn.reference([None] * len(sn.inputs), DT)
    with pytest.raises(ValueError, match="values for"):
        sn.reference([], DT)
    g, inputs = models.smollm2_decode(TINY_LLAMA, seed=3, runtime_pos=True)[:2]
    sn = next(n for n in g.nodes if getattr(n, "pos_t", None) is not None and n.pos_t not in n.inputs)
    with pytest.raises(ValueError, match="needs its value in host"):
        sn.reference([inputs.get(t.onnx_name, np.zeros(t.shape)) for t in sn.inputs], DT)
