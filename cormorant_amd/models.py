"""Graph builders for the benchmark workloads, with seeded synthetic weights.

small_cnn -- batch 1, Q8.8 throughout: Conv 3x3 1->8 pad 1 + bias -> ReLU -> MaxPool 2x2 ->
Conv 3x3 8->16 pad 1 + bias -> ReLU -> MaxPool 2x2 -> flatten 784 -> MatMul 784x10 -> Add
bias -> Softmax (row mode, regs(8, 1.0, 8)).  Weights U(+-0.25), biases U(+-0.1); the
input U[0, 1).  The node kinds are the reference's mapping of this network
(ConvNode, ScheduledNode RELU, PoolNode MAX, ReshapeNode, MatmulNode, ScheduledNode ADD,
SoftmaxVopNode; _simulate.py:617-765).
"""
from __future__ import annotations

import numpy as np

from . import units
from .graph import (ConvNode, Graph, MatmulNode, PoolNode, ReshapeNode, ScheduledNode,
                    SoftmaxVopNode, TensorInfo)


def small_cnn(seed: int = 0):
    """(graph, inputs): the small CNN and one seeded input image."""
    rng = np.random.default_rng(seed)
    T = TensorInfo
    x = T("input", [1, 1, 28, 28])
    w1 = T("conv1.w", [8, 1, 3, 3], data=rng.uniform(-0.25, 0.25, (8, 1, 3, 3)))
    b1 = T("conv1.b", [8], data=rng.uniform(-0.1, 0.1, 8))
    c1 = T("conv1", [1, 8, 28, 28])
    r1 = T("relu1", [1, 8, 28, 28])
    p1 = T("pool1", [1, 8, 14, 14])
    w2 = T("conv2.w", [16, 8, 3, 3], data=rng.uniform(-0.25, 0.25, (16, 8, 3, 3)))
    b2 = T("conv2.b", [16], data=rng.uniform(-0.1, 0.1, 16))
    c2 = T("conv2", [1, 16, 14, 14])
    r2 = T("relu2", [1, 16, 14, 14])
    p2 = T("pool2", [1, 16, 7, 7])
    fl = T("flat", [1, 784])
    wf = T("fc.w", [784, 10], data=rng.uniform(-0.25, 0.25, (784, 10)))
    mm = T("fc", [1, 10])
    bf = T("fc.b", [10], data=rng.uniform(-0.1, 0.1, 10))
    ad = T("logits", [1, 10])
    sm = T("probs", [1, 10])
    nodes = [
        ConvNode([x, w1, b1], c1, pad_top=1, pad_left=1),
        ScheduledNode([c1], r1, units.OP_RELU),
        PoolNode([r1], p1, units.POOL_MAX, 2, 2, 2, 2),
        ConvNode([p1, w2, b2], c2, pad_top=1, pad_left=1),
        ScheduledNode([c2], r2, units.OP_RELU),
        PoolNode([r2], p2, units.POOL_MAX, 2, 2, 2, 2),
        ReshapeNode([p2], fl),
        MatmulNode([fl, wf], mm),
        ScheduledNode([mm, bf], ad, units.OP_ADD),
        SoftmaxVopNode([ad], sm),
    ]
    g = Graph(nodes, input_tensors=[x], output_tensors=[sm])
    inputs = {"input": np.round(rng.uniform(0.0, 1.0, (1, 1, 28, 28)) * 256) / 256}
    return g, inputs
