"""The row-ops node adapters' jobs run through the oracle on the CPU (the Simulator's
row re-layout restated), against the reference's rowops_spec outputs and the reference
nodes' closed forms: pins the parameter derivation and the job registers without a GPU."""
import numpy as np
import pytest

from rowops_node_cases import CASES, same

_NP = {"i16": np.int16, "i32": np.int32, "f32": np.float32}
_KB = {"i16": 2, "i32": 4, "f32": 4}


def rows16(x2d, kind):
    rows, w = x2d.shape
    stride = (_KB[kind] * w + 15) & ~15
    img = np.zeros((rows, stride), np.uint8)
    img[:, :_KB[kind] * w] = np.ascontiguousarray(x2d.astype(_NP[kind])).view(np.uint8).reshape(rows, -1)
    return img.reshape(-1), stride


def run_oracle(oracle_lib, node, raw_inputs):
    vals = {t.onnx_name: x for t, x in raw_inputs}
    at, ot = node.inputs[0], node.output
    bt = getattr(node, "table", None) or (node.inputs[1] if len(node.inputs) > 1 else None)
    jobs = node.jobs()
    width = max(j.col0 + j.n for j in jobs)
    rows = at.numel // width
    a2d = np.asarray(vals[at.onnx_name]).reshape(rows, width)
    out = np.zeros((rows, width), _NP[ot.kind])
    for j in jobs:
        a_img, a_s1 = rows16(a2d[:, j.col0:j.col0 + j.n], at.kind)
        b_img, b_s1 = None, 0
        if bt is not None:
            if j.b_row0 is None:
                b2d = np.asarray(vals[bt.onnx_name]).reshape(rows, width)[:, j.col0:j.col0 + j.n]
            else:
                b2d = np.asarray(bt.data).reshape(-1, bt.shape[-1])[j.b_row0:j.b_row0 + rows]
            b_img, b_s1 = rows16(b2d, bt.kind)
        c_img, c_s1 = rows16(np.zeros((rows, j.n), _NP[ot.kind]), ot.kind)
        oracle_lib.rowops_reset_params()
        oracle_lib.rowops(a_img, b_img, c_img, j.params, j.op, j.n, rows, 1, a_s1, 0, b_s1, 0, c_s1, 0,
                          j.eps, j.aux, j.bq_sh)
        c = c_img.reshape(rows, c_s1)[:, :_KB[ot.kind] * j.n].copy().view(_NP[ot.kind])
        out[:, j.col0:j.col0 + j.n] = c
    return out


@pytest.mark.parametrize("name,build", CASES, ids=[c[0] for c in CASES])
def test_adapter_through_the_oracle(oracle_lib, name, build):
    node, ins, want = build()
    got = run_oracle(oracle_lib, node, ins)
    assert same(got, want.reshape(got.shape)), name
