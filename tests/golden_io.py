"""Loaders for the committed golden fixtures (tests/golden/*.npz, converted from the
reference's hw/test_data by tests/golden/make_fixtures.py)."""
import functools
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

VEC_COLS = ("idx", "size", "op", "outer", "a_inc", "b_inc", "act", "alpha", "smx_cm",
            "smx_cfg", "smx_mask", "label")
MM_COLS = ("idx", "n", "k", "m", "batch", "a_stride", "b_stride", "b_packed", "gemv_kw", "label")
CONV_COLS = ("idx", "batch", "in_ch", "in_h", "in_w", "out_ch", "out_h", "out_w", "kh", "kw",
             "stride_h", "stride_w", "dilation_h", "dilation_w", "pad_top", "pad_left",
             "has_bias", "is_depthwise", "y_cs", "y_cn", "y_gs", "label")
POOL_COLS = ("idx", "N", "C", "H", "W", "out_h", "out_w", "pool_h", "pool_w", "stride_h",
             "stride_w", "pad_top", "pad_left", "dil_h", "dil_w", "pool_type", "lp_order",
             "count_include_pad", "label")
RO_COLS = ("idx", "op", "n", "c1", "c2", "a_s1", "a_s2", "b_s1", "b_s2", "c_s1", "c_s2", "eps",
           "aux", "bq_sh", "win_lo", "win_hi", "label")
CHAIN_COLS = ("chain", "job", "op", "n", "c1", "c2", "a", "a_s1", "a_s2", "b", "b_s1", "b_s2",
              "c", "c_s1", "c_s2", "p", "eps", "aux", "bq_sh", "win_lo", "win_hi", "label")


@functools.lru_cache(maxsize=None)
def load(unit):
    return np.load(os.path.join(GOLDEN, f"{unit}.npz"))


def cases(unit, cols):
    d = load(unit)
    return [dict(zip(cols, r)) for r in json.loads(str(d["manifest"]))]


def chain_jobs():
    d = load("rowops")
    return [dict(zip(CHAIN_COLS, r)) for r in json.loads(str(d["chain_manifest"]))]


def arr(unit, idx, name):
    d = load(unit)
    key = f"c{idx}_{name}"
    return d[key] if key in d else None
