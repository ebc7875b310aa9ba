"""cm_matmul_noalloc (the matmul entry point that allocates nothing) against cm_matmul, bit for
bit, through the C ABI: the plane GEMM (Q8.8 saturate, batched A, packed B), the wrap-mode
split over k (partials in the scratch) and the skinny path (split-k partials in the scratch),
each as two calls in a row, the second smaller, so the second reads a scratch the first left
behind; and a call past the scratch maximum refused."""
import numpy as np
import pytest
import torch

from cormorant_amd import units as U
from tests.gpu_util import POISON16, host

pytestmark = pytest.mark.gpu

TAIL = 16


def _operands(rng, n, k, m, batch, a_bs, b_packed):
    a = torch.from_numpy(rng.integers(-32768, 32768, (batch - 1) * a_bs + n * k + TAIL).astype(np.int16)).cuda()
    b = torch.from_numpy(rng.integers(-32768, 32768, U.matmul_b_extent(k, m, b_packed, 0) + TAIL)
                         .astype(np.int16)).cuda()
    return a, b


def _both(a, b, n, k, m, batch, a_bs, b_packed, wrap32):
    total = batch * n * m + TAIL
    want = torch.full((total,), int(POISON16), dtype=torch.int16, device="cuda")
    got = torch.full((total,), int(POISON16), dtype=torch.int16, device="cuda")
    U.matmul(a, b, want, n, k, m, batch=batch, a_bs=a_bs, b_packed=b_packed, wrap32=wrap32)
    U.matmul_noalloc(a, b, got, n, k, m, batch=batch, a_bs=a_bs, b_packed=b_packed, wrap32=wrap32)
    return host(got), host(want)


# (n, k, m, batch, a_bs per n*k, b_packed, wrap32) of the first call and the smaller second
CASES = {
    "plane_gemm_q88": [(512, 2048, 1024, 2, 1, 1, False), (96, 320, 160, 1, 0, 0, False)],
    "wrap_split_k": [(128, 2048, 256, 1, 0, 0, True), (64, 1024, 128, 1, 0, 1, True)],
    "skinny_split_k": [(16, 960, 2560, 1, 0, 2, True), (3, 256, 64, 1, 0, 0, True)],
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_noalloc_matches_matmul_twice(case):
    U.init()
    rng = np.random.default_rng(len(case))
    for n, k, m, batch, abs_f, b_packed, wrap32 in CASES[case]:
        print(f"noalloc {case}: n={n} k={k} m={m} batch={batch} b_packed={b_packed} wrap32={wrap32}", flush=True)
        a_bs = abs_f * n * k
        a, b = _operands(rng, n, k, m, batch, a_bs, b_packed)
        got, want = _both(a, b, n, k, m, batch, a_bs, b_packed, wrap32)
        np.testing.assert_array_equal(got, want)
        assert (got[batch * n * m:] == POISON16).all(), "a write past the output"


def test_noalloc_refuses_past_its_maximum():
    U.init()
    n = k = m = 4096                      # planes of A and B: 64 MiB, plus their line sums
    a = torch.zeros(n * k, dtype=torch.int16, device="cuda")
    b = torch.zeros(k * m, dtype=torch.int16, device="cuda")
    c = torch.full((n * m,), int(POISON16), dtype=torch.int16, device="cuda")
    with pytest.raises(ValueError, match="no-allocation maximum"):
        U.matmul_noalloc(a, b, c, n, k, m)
    assert (host(c) == POISON16).all(), "a refused call wrote its output"
