"""cormorant_amd -- the fixed-point simulator's five units (VectorOP, Matmul, Conv, Pooling,
RowOps) as hand-written gfx950 HIP kernels behind a C ABI (include/cormorant_hip.h), with a
Python mirror of the reference simulator's API on top.

``units``  the register-level calls on device tensors (one per unit);
``dtype``  the value <-> raw conversions of the reference's DataType;
``graph``  nodes, graphs and ``Simulator.simulate`` (the reference's per-node dispatch).
"""
from . import units  # noqa: F401

__all__ = ["units"]
