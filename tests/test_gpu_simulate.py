"""Graph-level parity: cormorant_amd.simulate.Simulator (every node on the HIP units) against
the value-domain restatement of the reference's _forward_pass (oracle/graph_sim.py)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_small_cnn_matches_reference_forward(torch_gpu, seed):
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as oracle_graph
    g, inputs = models.small_cnn(seed)
    sim = Simulator(g)
    got = sim._forward_pass(inputs)
    want = oracle_graph.forward(g, inputs)
    for name in want:
        if name in got:
            np.testing.assert_array_equal(got[name], want[name], err_msg=name)
    out = sim.simulate(inputs)["probs"]
    np.testing.assert_array_equal(out, want["probs"])
    assert abs(out.sum() - 1.0) < 0.05          # a softmax over 10 classes at 2^-8


def test_matmul_node_batched_broadcast_b(torch_gpu):
    """MatMul with A [3, 5, 70] and a shared weight B [70, 33] (packed once)."""
    from cormorant_amd import graph as G
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as oracle_graph
    rng = np.random.default_rng(4)
    a = G.TensorInfo("a", [3, 5, 70])
    w = G.TensorInfo("w", [70, 33], data=rng.uniform(-2, 2, (70, 33)))
    c = G.TensorInfo("c", [3, 5, 33])
    g = G.Graph([G.MatmulNode([a, w], c)], [a], [c])
    inputs = {"a": np.round(rng.uniform(-4, 4, (3, 5, 70)) * 256) / 256}
    np.testing.assert_array_equal(Simulator(g).simulate(inputs)["c"], oracle_graph.forward(g, inputs)["c"])


def test_vectorop_broadcast_bias_unaligned(torch_gpu):
    """ADD of a bias [10] onto [6, 10] (a chunk that is not a whole 8-lane word) and onto
    [4, 16] (one that is): both broadcast paths."""
    from cormorant_amd import graph as G
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim as oracle_graph
    rng = np.random.default_rng(5)
    for rows, n in ((6, 10), (4, 16)):
        x = G.TensorInfo("x", [rows, n])
        b = G.TensorInfo("b", [n], data=rng.uniform(-1, 1, n))
        y = G.TensorInfo("y", [rows, n])
        g = G.Graph([G.ScheduledNode([x, b], y, G.OP_ADD, act=1)], [x], [y])
        inputs = {"x": np.round(rng.uniform(-2, 2, (rows, n)) * 256) / 256}
        np.testing.assert_array_equal(Simulator(g).simulate(inputs)["y"], oracle_graph.forward(g, inputs)["y"])


def test_expected_dat_of_the_small_cnn():
    """generate_expected_dat: the ramp-input simulation's output as the little-endian storage
    lanes, decoded back equal to the oracle's forward over the same ramp inputs."""
    import numpy as np
    from cormorant_amd import models
    from cormorant_amd.dtype import AP_FIXED_16_8
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim
    g, _ = models.small_cnn(0)
    sim = Simulator(g)
    ramp = sim._build_ramp_inputs()
    assert ramp["input"].reshape(-1)[5] == 5 / 256
    out = g.output_tensors[0]
    dat = sim.generate_expected_dat(out)
    got = np.frombuffer(dat, "<u2").view(np.int16) / 256.0
    want = graph_sim.forward(g, ramp)[out.onnx_name].reshape(-1)
    np.testing.assert_array_equal(got, want)
    assert dat == AP_FIXED_16_8.dat_bytes(want)
