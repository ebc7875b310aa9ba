"""The row-ops oracle (cm_oracle.c) against the reference's own row-ops oracle
(kernels/rowops_rtl/tb/verilator/rowops_ref.h, built into oracle/_ref by oracle/Makefile)
on seeded random jobs of every op, and on the 43 fixtures.  CPU only; skipped where the
reference checkout was not available to build _ref."""
import ctypes
import os

import numpy as np
import pytest

from golden_io import RO_COLS, arr, cases
from rowops_cases import RO_CASES, make_job

REF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                   "librowops_ref.so")


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    lib = ctypes.CDLL(REF)
    U64, U32, P = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p
    lib.ref_rowops.argtypes = [P, U64, P, U64, P, U64, P, U64] + [U32] * 10 + [ctypes.c_longlong] + [U32] * 4
    lib.ref_rowops.restype = ctypes.c_int
    return lib


def run_ref(lib, a, b, c, p, r):
    ptr = lambda x: x.ctypes.data if x is not None and len(x) else None
    ln = lambda x: len(x) if x is not None else 0
    lib.ref_rowops_reset()
    rc = lib.ref_rowops(ptr(a), ln(a), ptr(b), ln(b), c.ctypes.data, len(c), ptr(p), ln(p), r["op"], r["n"],
                        r["c1"], r["c2"], r["a_s1"], r["a_s2"], r["b_s1"], r["b_s2"], r["c_s1"], r["c_s2"],
                        r["eps"], r["aux"], r["bq_sh"], r.get("win_lo", 0), r.get("win_hi", 0xFFFFFFFF))
    assert rc == 0


@pytest.mark.parametrize("case", RO_CASES, ids=lambda c: c[0])
def test_random_jobs_match_the_reference_oracle(ref, oracle_lib, case):
    a, b, p, c_len, r = make_job(case)
    mine = np.full(c_len, 0xDE, np.uint8)
    oracle_lib.rowops_reset_params()
    oracle_lib.rowops(a, b, mine, p, r["op"], r["n"], r["c1"], r["c2"], r["a_s1"], r["a_s2"], r["b_s1"],
                      r["b_s2"], r["c_s1"], r["c_s2"], r["eps"], r["aux"], r["bq_sh"])
    theirs = np.full(c_len, 0xDE, np.uint8)
    run_ref(ref, a, b, theirs, p, r)
    np.testing.assert_array_equal(mine, theirs)


def test_fixtures_through_the_reference_oracle(ref):
    """The reference oracle itself reproduces the fixtures (so the shim passes registers right)."""
    for t in cases("rowops", RO_COLS):
        a, b, p, c = (arr("rowops", t["idx"], x) for x in "abpc")
        got = np.full(len(c), 0xDE, np.uint8)
        run_ref(ref, a, b, got, p, t)
        np.testing.assert_array_equal(got, c, err_msg=t["label"])
