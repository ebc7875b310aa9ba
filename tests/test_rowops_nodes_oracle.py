"""The row-ops node adapters' jobs run through the oracle on the CPU (the Simulator's
row re-layout restated), against the reference's rowops_spec outputs and the reference
nodes' closed forms: pins the parameter derivation and the job registers without a GPU."""
import numpy as np
import pytest

from oracle.graph_sim import run_adapter
from rowops_node_cases import CASES, same



def run_oracle(oracle_lib, node, raw_inputs):
    vals = {t.onnx_name: x for t, x in raw_inputs}
    return run_adapter(node, lambda t: vals[t.onnx_name])


@pytest.mark.parametrize("name,build", CASES, ids=[c[0] for c in CASES])
def test_adapter_through_the_oracle(oracle_lib, name, build):
    node, ins, want = build()
    got = run_oracle(oracle_lib, node, ins)
    assert same(got, want.reshape(got.shape)), name
