"""The row-ops node adapters on the GPU (through Simulator), bit for bit against the
reference's rowops_spec outputs and the reference nodes' closed forms (rowops_node_cases)."""
import numpy as np
import pytest
import torch

from cormorant_amd.graph import Graph
from cormorant_amd.simulate import Simulator
from rowops_node_cases import CASES, same

pytestmark = pytest.mark.gpu
_NP = {"i16": np.int16, "i32": np.int32, "f32": np.float32}


def run(node, raw_inputs):
    """One adapter node through the Simulator: raw numpy inputs (by tensor) -> raw output."""
    g = Graph(nodes=[node], input_tensors=list(node.inputs), output_tensors=[node.output])
    sim = Simulator(g)
    dev = {t.onnx_name: torch.from_numpy(np.ascontiguousarray(x.astype(_NP[t.kind]).reshape(-1))).cuda()
           for t, x in raw_inputs}
    out = sim.forward_raw(dev)[node.output.onnx_name]
    return out.cpu().numpy().reshape(node.output.shape)


@pytest.mark.parametrize("name,build", CASES, ids=[c[0] for c in CASES])
def test_adapter(name, build):
    node, ins, want = build()
    got = run(node, ins)
    assert same(got, want.reshape(got.shape)), name
