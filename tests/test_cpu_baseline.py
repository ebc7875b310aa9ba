"""The numpy restatement of the reference simulator's MatMul (the CPU baseline bench.py
times) agrees with the C oracle, including saturation; bench.py refuses more than one GPU."""
import subprocess
import sys

import numpy as np

from oracle import sim_numpy


def test_sim_numpy_matches_oracle(oracle_lib):
    rng = np.random.default_rng(5)
    n, k, m = 9, 300, 70
    a = rng.integers(-32768, 32768, (n, k)).astype(np.int16)
    b = rng.integers(-32768, 32768, (k, m)).astype(np.int16)
    want = oracle_lib.matmul(a.reshape(-1), b.reshape(-1), n, k, m).reshape(n, m)
    got = sim_numpy.matmul_q88(a, b)
    np.testing.assert_array_equal(got, want)
    assert (np.abs(want.astype(np.int64)) == 32767).any() or (want == -32768).any()


def test_unpack_b_inverts_packing():
    rng = np.random.default_rng(6)
    k, m = 37, 70
    b = rng.integers(-100, 100, (k, m)).astype(np.int16)
    mp = 96
    bp = np.zeros((mp // 32) * k * 32, np.int16)
    for j in range(m):
        bp[((j // 32) * k + np.arange(k)) * 32 + j % 32] = b[:, j]
    np.testing.assert_array_equal(sim_numpy.unpack_b(bp, k, m), b)


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
