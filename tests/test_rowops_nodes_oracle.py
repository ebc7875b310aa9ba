"""The row-ops node adapter cases on the CPU, against the reference's rowops_spec outputs and
the reference nodes' closed forms: (1) the graph-level oracle's own adapter path
(oracle/rowops_adapt.py: its restated job constants through the C oracle's job), (2) the
product adapters' job lists (parameters and registers as the GPU receives them) through the
same C oracle job with the Simulator's row re-layout."""
import numpy as np
import pytest

from oracle import cm
from oracle import rowops_adapt
from rowops_node_cases import CASES, same

_NP = {"i16": np.int16, "i32": np.int32, "f32": np.float32}
_KB = {"i16": 2, "i32": 4, "f32": 4}


def _exp(t, n):
    return np.broadcast_to(np.asarray(8 if t.exp is None else t.exp, np.float64).reshape(-1), (n,))


def _rows16(x2d, kind):
    """[rows][n] lanes as a byte image whose rows start at 16-byte multiples."""
    rows, n = x2d.shape
    s1 = (_KB[kind] * n + 15) & ~15
    img = np.zeros((rows, s1), np.uint8)
    img[:, :_KB[kind] * n] = np.ascontiguousarray(x2d.astype(_NP[kind])).view(np.uint8).reshape(rows, -1)
    return img.reshape(-1), s1


def product_jobs(node, raw_of):
    """The product adapter's jobs through the C oracle: raw output lanes."""
    at, ot = node.inputs[0], node.output
    bt = getattr(node, "table", None) or (node.inputs[1] if len(node.inputs) > 1 else None)
    jobs = node.jobs()
    width = max(j.col0 + j.n for j in jobs)
    rows = at.numel // width
    a2d = np.asarray(raw_of(at)).reshape(rows, width)
    out = np.zeros((rows, width), _NP[ot.kind])
    for j in jobs:
        a_img, a_s1 = _rows16(a2d[:, j.col0:j.col0 + j.n], at.kind)
        b_img, b_s1 = None, 0
        if bt is not None:
            if j.b_row0 is None:
                b2d = np.asarray(raw_of(bt)).reshape(rows, width)[:, j.col0:j.col0 + j.n]
            else:
                b2d = np.asarray(bt.data).reshape(-1, bt.shape[-1])[j.b_row0:j.b_row0 + (1 if j.b_same else rows)]
            b_img, b_s1 = _rows16(b2d, bt.kind)
            if j.b_same:
                b_s1 = 0
        c_img, c_s1 = _rows16(np.zeros((rows, j.n), _NP[ot.kind]), ot.kind)
        cm.rowops_reset_params()
        cm.rowops(a_img, b_img, c_img, j.params, j.op, j.n, rows, 1, a_s1, 0, b_s1, 0, c_s1, 0, j.eps, j.aux,
                  j.bq_sh)
        out[:, j.col0:j.col0 + j.n] = c_img.reshape(rows, c_s1)[:, :_KB[ot.kind] * j.n].copy().view(_NP[ot.kind])
    return out


@pytest.mark.parametrize("name,build", CASES, ids=[c[0] for c in CASES])
def test_oracle_adapter(oracle_lib, name, build):
    node, ins, want = build()
    vals = [np.asarray(x, np.float64) / np.power(2.0, _exp(t, t.shape[-1]))[None, :]
            for t, x in ins]
    y = rowops_adapt.adapter(node, vals)
    ot = node.output
    got = y if ot.kind == "f32" else np.rint(y.reshape(-1, ot.shape[-1]) * np.power(2.0, _exp(ot, ot.shape[-1])))
    assert same(np.asarray(got).reshape(want.shape), want), name


@pytest.mark.parametrize("name,build", CASES, ids=[c[0] for c in CASES])
def test_product_jobs_through_the_oracle(oracle_lib, name, build):
    node, ins, want = build()
    vals = {t.onnx_name: x for t, x in ins}
    got = product_jobs(node, lambda t: vals[t.onnx_name])
    assert same(got, want.reshape(got.shape)), name
