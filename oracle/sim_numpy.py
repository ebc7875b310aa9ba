"""TEST INFRASTRUCTURE ONLY: the reference simulator's own CPU algorithm for the Matmul unit,
restated with numpy -- the CPU baseline that bench.py times.

The reference's Q8.8 MatMul branch (inference-scheduler/src/codegen/_simulate.py:620-633)
holds values as float64 (raw * 2^-8), multiplies with ``np.matmul`` (BLAS dgemm; the sums
of on-grid products are exact) and writes ``ApFixed.truncate`` (dtype.py:371-377): clip to
the Q8.8 range, floor at 2^-8.  B is the logical [k][m] matrix (the packed image is a DDR
layout only, nodes.py:606-628).
"""
import numpy as np

Q_MIN, Q_MAX = -128.0, 127.99609375


def unpack_b(bp: np.ndarray, k: int, m: int) -> np.ndarray:
    """The logical B [k][m] of a packed 32-column tile image (MatmulKernel.h:91-113)."""
    mp = (m + 31) // 32 * 32
    t = np.asarray(bp).reshape(mp // 32, k, 32)
    return t.transpose(1, 0, 2).reshape(k, mp)[:, :m]


def matmul_q88(a_raw: np.ndarray, b_raw: np.ndarray) -> np.ndarray:
    """Raw int16 C of the simulator's Q8.8 MatMul for raw int16 A [.., n, k] and B [k, m]."""
    a = np.asarray(a_raw, np.float64) / 256.0
    b = np.asarray(b_raw, np.float64) / 256.0
    full = np.matmul(a, b)
    q = np.floor(np.clip(full, Q_MIN, Q_MAX) * 256.0)
    return q.astype(np.int16)
