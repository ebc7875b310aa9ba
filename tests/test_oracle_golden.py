"""The oracle against every known-answer fixture the reference holds for the five units
(hw/test_data, converted to tests/golden/*.npz) and against the ROM text tables.

These pin the oracle before it is trusted as the checker of the HIP library.  CPU only."""
import json

import numpy as np
import pytest

from golden_io import (CONV_COLS, MM_COLS, POOL_COLS, RO_COLS, VEC_COLS, arr, cases,
                       chain_jobs, load)

VEC = cases("vecop", VEC_COLS)
MM = cases("matmul", MM_COLS)
CONV = cases("conv", CONV_COLS)
POOL = cases("pool", POOL_COLS)
RO = cases("rowops", RO_COLS)


def vec_c_len(t, fixture_len):
    size, outer = t["size"], t["outer"]
    padded = (size + 7) & ~7
    if t["op"] == 10:
        need = (outer - 1) * t["b_inc"] + padded
    elif t["op"] == 11:
        need = max(((outer & ~15) - 1) * t["b_inc"] + padded, 0)
    else:
        need = (outer - 1) * (t["a_inc"] + t["b_inc"]) + padded
    return max(need, fixture_len)


@pytest.mark.parametrize("t", VEC, ids=lambda t: f"{t['idx']}-{t['label']}")
def test_vecop_fixture(oracle_lib, t):
    a, b, c = arr("vecop", t["idx"], "a"), arr("vecop", t["idx"], "b"), arr("vecop", t["idx"], "c")
    got = oracle_lib.vectorop(a, b if b is not None and len(b) else None, vec_c_len(t, len(c)),
                              t["size"], t["op"], t["outer"], t["a_inc"], t["b_inc"], t["act"],
                              t["alpha"], t["smx_cm"], t["smx_cfg"], t["smx_mask"])
    np.testing.assert_array_equal(got[:len(c)], c)


@pytest.mark.parametrize("t", MM, ids=lambda t: f"{t['idx']}-{t['label']}")
def test_matmul_fixture(oracle_lib, t):
    a, b, c = (arr("matmul", t["idx"], x) for x in "abc")
    got = oracle_lib.matmul(a, b, t["n"], t["k"], t["m"], t["batch"], t["a_stride"],
                            t["b_stride"], t["n"] * t["m"], t["b_packed"], t["gemv_kw"])
    np.testing.assert_array_equal(got, c)


@pytest.mark.parametrize("t", CONV, ids=lambda t: f"{t['idx']}-{t['label']}")
def test_conv_fixture(oracle_lib, t):
    x, w, b, y = (arr("conv", t["idx"], n) for n in ("x", "w", "b", "y"))
    got = oracle_lib.conv(x, w, b if b is not None and len(b) else None, len(y), t["batch"],
                          t["in_ch"], t["in_h"], t["in_w"], t["out_ch"], t["out_h"], t["out_w"],
                          t["kh"], t["kw"], t["stride_h"], t["stride_w"], t["dilation_h"],
                          t["dilation_w"], t["pad_top"], t["pad_left"], t["has_bias"],
                          t["is_depthwise"])
    np.testing.assert_array_equal(got, y)


@pytest.mark.parametrize("t", [t for t in CONV if t["y_cs"] or t["y_cn"]],
                         ids=lambda t: f"{t['idx']}-{t['label']}")
def test_conv_y_pattern(oracle_lib, t):
    """The y channel pattern scatters the dense planes (ConvKernel.h:250-258)."""
    x, w, y = (arr("conv", t["idx"], n) for n in ("x", "w", "y"))
    plane = t["out_h"] * t["out_w"]
    cs = t["y_cs"] or plane
    cn = t["y_cn"] or t["out_ch"]
    span = max((c % cn) * cs + (c // cn) * t["y_gs"] for c in range(t["out_ch"])) + plane
    got = oracle_lib.conv(x, w, None, span, 1, t["in_ch"], t["in_h"], t["in_w"], t["out_ch"],
                          t["out_h"], t["out_w"], t["kh"], t["kw"], t["stride_h"], t["stride_w"],
                          t["dilation_h"], t["dilation_w"], t["pad_top"], t["pad_left"], 0, 0,
                          t["y_cs"], t["y_cn"], t["y_gs"])
    for c in range(t["out_ch"]):
        off = (c % cn) * cs + (c // cn) * t["y_gs"]
        np.testing.assert_array_equal(got[off:off + plane], y[c * plane:(c + 1) * plane])


@pytest.mark.parametrize("t", POOL, ids=lambda t: f"{t['idx']}-{t['label']}")
def test_pool_fixture(oracle_lib, t):
    x, y = arr("pool", t["idx"], "x"), arr("pool", t["idx"], "y")
    got = oracle_lib.pool(x, t["N"], t["C"], t["H"], t["W"], t["out_h"], t["out_w"], t["pool_h"],
                          t["pool_w"], t["stride_h"], t["stride_w"], t["pad_top"], t["pad_left"],
                          t["dil_h"], t["dil_w"], t["pool_type"], t["lp_order"],
                          t["count_include_pad"])
    np.testing.assert_array_equal(got, y)


def _ro_images(t):
    a = arr("rowops", t["idx"], "a")
    b = arr("rowops", t["idx"], "b")
    p = arr("rowops", t["idx"], "p")
    c = arr("rowops", t["idx"], "c")
    return a, b, p, c


@pytest.mark.parametrize("t", RO, ids=lambda t: f"{t['idx']}-{t['label']}")
def test_rowops_fixture(oracle_lib, t):
    a, b, p, c_want = _ro_images(t)
    c = np.full(len(c_want), 0xDE, np.uint8)
    oracle_lib.rowops_reset_params()
    oracle_lib.rowops(a, b, c, p, t["op"], t["n"], t["c1"], t["c2"], t["a_s1"], t["a_s2"],
                      t["b_s1"], t["b_s2"], t["c_s1"], t["c_s2"], t["eps"], t["aux"], t["bq_sh"],
                      t["win_lo"], t["win_hi"])
    np.testing.assert_array_equal(c, c_want)


@pytest.mark.parametrize("cid", sorted({j["chain"] for j in chain_jobs()}))
def test_rowops_chain_fixture(oracle_lib, cid):
    d = load("rowops")
    seg = d[f"chain{cid}_mem"].copy()
    want = d[f"chain{cid}_out"]
    oracle_lib.rowops_reset_params()
    for j in [j for j in chain_jobs() if j["chain"] == cid]:
        a = seg[j["a"]:]
        b = seg[j["b"]:]
        p = seg[j["p"]:]
        c = seg[j["c"]:]
        oracle_lib.rowops(a, b, c, p, j["op"], j["n"], j["c1"], j["c2"], j["a_s1"], j["a_s2"],
                          j["b_s1"], j["b_s2"], j["c_s1"], j["c_s2"], j["eps"], j["aux"],
                          j["bq_sh"], j["win_lo"], j["win_hi"])
    np.testing.assert_array_equal(seg, want)


def test_rowops_table_image(oracle_lib):
    """The 64 KiB TLOAD image (rowops_spec.table_image) equals tables.hex."""
    np.testing.assert_array_equal(oracle_lib.rowops_table_image(), load("rowops")["tables"])


def test_act_tables_equal_the_rom(oracle_lib):
    """SiLU / GELU / GELU-tanh over all 65 536 Q8.8 inputs equal the RTL ROM text
    (vo_act_rom.sv: f(x) = max(x, 0) - rom[BASE + |x|] for |x| < LEN), the check of the
    reference's test_activations.py:96-110."""
    d = load("roms")
    rom = d["act_rom"].astype(np.int64)
    seg = json.loads(str(d["act_segments"]))
    raw = np.arange(-32768, 32768, dtype=np.int64)
    for name, act in (("SILU", 4), ("GELU", 5), ("GELU_TANH", 6)):
        base, n = seg[name]
        t = np.abs(raw)
        m = np.where(t < n, rom[base + np.minimum(t, n - 1)], 0)
        np.testing.assert_array_equal(oracle_lib.act_table(act), np.maximum(raw, 0) - m,
                                      err_msg=name)


def test_smx_table_equals_the_rom(oracle_lib):
    np.testing.assert_array_equal(oracle_lib.smx_table(), load("roms")["smx_tab"])
