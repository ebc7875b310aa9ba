"""The oracle's row-ops adapter path (oracle/rowops_adapt.py: its own restatement of the
specification's job constants, then the C oracle's job) against the vectors the reference's
rowops_spec wrote (tests/golden/rowops_spec.npz): norm_params / gamma_scale / beta_bits,
bias_params and quant_bias.  The adapter path end to end (these constants through the C
oracle's job) is checked over the reference's layer_norm / rms_norm / silu_mul / rope / bias
outputs in test_rowops_nodes_oracle.py."""
import numpy as np
import pytest

from oracle import rowops_adapt as ra
from tests.golden_io import load

SPEC = load("rowops_spec")


@pytest.mark.parametrize("i", range(int(SPEC["np_count"][0])))
def test_norm_params(i):
    p = f"np{i}_"
    n, f_in, rms, g, E, bb, gs = (int(v) for v in SPEC[p + "meta"])
    gamma, beta, eps = SPEC[p + "gamma"], SPEC[p + "beta"], float(SPEC[p + "eps"][0])
    G, g2, Bq, E2 = ra.norm_params(gamma, n, eps, f_in, beta=None if rms else beta, rms=bool(rms))
    assert (g2, E2, ra.beta_bits(beta), ra.gamma_scale(gamma)) == (g, E, bb, gs)
    np.testing.assert_array_equal(G, SPEC[p + "G"])
    np.testing.assert_array_equal(np.zeros(0, np.int64) if Bq is None else Bq, SPEC[p + "Bq"])


@pytest.mark.parametrize("i", range(int(SPEC["bias_count"][0])))
def test_bias_params(i):
    p = f"bias{i}_"
    bq, sa, sc = ra.bias_params(SPEC[p + "bias"], SPEC[p + "fx"], SPEC[p + "fo"])
    np.testing.assert_array_equal(bq, SPEC[p + "bq"])
    np.testing.assert_array_equal(sa, SPEC[p + "sa"])
    np.testing.assert_array_equal(sc, SPEC[p + "sc"])


@pytest.mark.parametrize("i", range(int(SPEC["qb_count"][0])))
def test_quant_bias_bits(i):
    p = f"qb{i}_"
    bias, fr = SPEC[p + "bias"], int(SPEC[p + "fr"][0])
    bb = ra.bias_bits(bias, fr)
    assert bb == int(SPEC[p + "bb"][0])
    np.testing.assert_array_equal(np.rint(bias * 2.0 ** bb) / 2.0 ** bb, SPEC[p + "q"])
