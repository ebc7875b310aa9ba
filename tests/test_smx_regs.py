"""The softmax unit's registers and integer softmax pinned by vectors of the reference's own
vectorop_smx.py (tests/golden/smx_regs.npz, written by tests/golden/make_smx_regs_vectors.py):
graph.softmax_regs -- the derivation BERT's and the decoders' attention use -- against
scale_regs over 480 (f_s, sigma) pairs, and the oracle's row-mode softmax (and the unit's, on
the GPU) against softmax_raw on seeded rows with per-row valid lengths."""
import os

import numpy as np
import pytest

from cormorant_amd.graph import softmax_regs
from oracle import cm

V = np.load(os.path.join(os.path.dirname(__file__), "golden", "smx_regs.npz"))


@pytest.mark.parametrize("f_p", [8, 14, 15])
def test_softmax_regs_equal_the_reference_scale_regs(f_p):
    for f_s, sigma, cm_ref, cs_ref in zip(V["regs_fs"], V["regs_sigma"], V["regs_cm"], V["regs_cs"]):
        got = softmax_regs(int(f_s), float(sigma), f_p)
        assert got == (int(cm_ref), int(cs_ref) | (f_p << 8)), (f_s, sigma)


def _cases():
    return range(int(V["sm_count"][0]))


@pytest.mark.parametrize("i", _cases())
def test_oracle_softmax_equals_softmax_raw(i):
    x, valid, want = V[f"sm{i}_x"], V[f"sm{i}_valid"], V[f"sm{i}_p"]
    c_m, c_s, f_p = (int(v) for v in V[f"sm{i}_regs"])
    rows, n = x.shape
    n8 = (n + 7) & ~7
    for r in range(rows):
        xr = np.zeros(n8, np.int16)
        xr[:n] = x[r]
        got = cm.vectorop(xr, None, n8, n, 10, 1, n8, n8, 0, 0, c_m, c_s | (f_p << 8), int(valid[r]))[:n]
        np.testing.assert_array_equal(got.astype(np.int64), want[r], err_msg=f"row {r}")


@pytest.mark.gpu
@pytest.mark.parametrize("i", _cases())
def test_unit_softmax_equals_softmax_raw(i):
    import torch
    from cormorant_amd import units
    units.init()
    x, valid, want = V[f"sm{i}_x"], V[f"sm{i}_valid"], V[f"sm{i}_p"]
    c_m, c_s, f_p = (int(v) for v in V[f"sm{i}_regs"])
    rows, n = x.shape
    n8 = (n + 7) & ~7
    for r in range(rows):
        xr = np.zeros(n8, np.int16)
        xr[:n] = x[r]
        y = torch.full((n8,), 0x5A5A, dtype=torch.int16, device="cuda")
        units.vectorop(torch.from_numpy(xr).cuda(), None, y, n, units.OP_SOFTMAX, outer=1, a_inc=n8, b_inc=n8,
                       smx_cm=c_m, smx_cfg=c_s | (f_p << 8), smx_mask=int(valid[r]))
        np.testing.assert_array_equal(y.cpu().numpy()[:n].astype(np.int64), want[r], err_msg=f"row {r}")
