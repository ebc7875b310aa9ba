"""MobileNetV2 (Q8.8) on the GPU (Simulator) against the value-domain restatement of the
reference simulator (oracle_graph), every tensor bit for bit: the stem and pointwise
convolutions on the plane GEMM, the depthwise 3x3 kernels at strides 1 and 2, RELU6 and the
residual ADD on VectorOP, the global average pool and the classifier MatMul."""
import numpy as np
import pytest

from cormorant_amd import models
from cormorant_amd.simulate import Simulator
from oracle import graph_sim as oracle_graph

pytestmark = pytest.mark.gpu


# (32, 224): the configuration's own batch -- the 1x1 convolutions fold 32 images into their
# GEMM columns (up to 401 408 lines), every image compared
@pytest.mark.parametrize("batch,res,seed", [(1, 32, 0), (2, 64, 1), (1, 224, 2), (32, 224, 5)])
def test_mobilenet_every_tensor(batch, res, seed):
    g, inputs, _ = models.mobilenet_v2(batch=batch, res=res, seed=seed)
    got = Simulator(g)._forward_pass(inputs)
    want = oracle_graph.forward(g, inputs)
    for name, v in got.items():
        np.testing.assert_array_equal(v, want[name].reshape(v.shape), err_msg=name)


def test_mobilenet_batch_prefix():
    """A smaller batch of the same seed is the leading images of a larger one."""
    g2, in2, _ = models.mobilenet_v2(batch=2, res=32, seed=3)
    g1, in1, _ = models.mobilenet_v2(batch=1, res=32, seed=3)
    np.testing.assert_array_equal(in2["input"][:1], in1["input"])
