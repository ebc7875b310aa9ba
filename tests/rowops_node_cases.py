"""The row-ops node adapter cases: each builds (node, raw inputs, expected raw output) from
the reference's rowops_spec outputs (tests/golden/rowops_spec.npz) or, where the reference
node's reference() is a closed form (ResAdd, ResAddBias, Widen, Dequant), from that form.
Run on the GPU by test_gpu_rowops_nodes.py and through the oracle by
test_rowops_nodes_oracle.py."""
import os

import numpy as np

from cormorant_amd import rowops_nodes as rn
from cormorant_amd.graph import TensorInfo

GOLD = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rowops_spec.npz"))


def T(name, shape, kind="i16", exp=None):
    return TensorInfo(name, list(shape), exp=exp, kind=kind)


def layer_norm(i):
    x, gamma, beta = GOLD[f"ln{i}_x"], GOLD[f"ln{i}_gamma"], GOLD[f"ln{i}_beta"]
    eps, fx, fout = float(GOLD[f"ln{i}_eps"][0]), int(GOLD[f"ln{i}_fx"][0]), GOLD[f"ln{i}_fout"]
    rows, n = x.shape
    if int(GOLD[f"ln{i}_kind"][0]) == 0:
        xt, yt = T("x", [rows, n]), T("y", [rows, n])
        node = rn.LayerNormRoNode([xt], yt, gamma=gamma, beta=beta, eps=eps)
    else:
        xt, yt = T("h", [rows, n], "i32", fx), T("y", [rows, n], exp=fout)
        node = rn.LayerNorm32RoNode([xt], yt, gamma=gamma, beta=beta, eps=eps)
    return node, [(xt, x)], GOLD[f"ln{i}_y"]


def rms_norm(i):
    h, gamma, fr, fout = GOLD[f"rms{i}_h"], GOLD[f"rms{i}_gamma"], int(GOLD[f"rms{i}_fr"][0]), GOLD[f"rms{i}_fout"]
    rows, n = h.shape
    ht, yt = T("h", [rows, n], "i32", fr), T("y", [rows, n], exp=fout)
    node = rn.RMSNormRoNode([ht], yt, gamma=gamma, eps=float(GOLD[f"rms{i}_eps"][0]))
    return node, [(ht, h)], GOLD[f"rms{i}_y"]


def rms_norm_over_heads():
    """gamma of one head's length over a row of several heads (a q / k norm)."""
    h, gamma, fr, fout = GOLD["rms0_h"], GOLD["rms0_gamma"], int(GOLD["rms0_fr"][0]), GOLD["rms0_fout"]
    rows, n = h.shape
    ht = T("h", [1, rows * n], "i32", fr)
    yt = T("y", [1, rows * n], exp=np.tile(fout, rows))
    node = rn.RMSNormRoNode([ht], yt, gamma=gamma, eps=float(GOLD["rms0_eps"][0]))
    return node, [(ht, h.reshape(1, -1))], GOLD["rms0_y"].reshape(1, -1)


def silu_mul(i):
    g, u = GOLD[f"silu{i}_g"], GOLD[f"silu{i}_u"]
    rows, n = g.shape
    gt, ut = T("g", [rows, n], exp=GOLD[f"silu{i}_fg"]), T("u", [rows, n], exp=GOLD[f"silu{i}_fu"])
    yt = T("y", [rows, n], exp=GOLD[f"silu{i}_fa"])
    return rn.SiluMulRoNode([gt, ut], yt), [(gt, g), (ut, u)], GOLD[f"silu{i}_y"]


def rope(i):
    x = GOLD[f"rope{i}_x"]
    Tn, nh, HD = x.shape
    fx, fo = GOLD[f"rope{i}_fx"], GOLD[f"rope{i}_fo"]
    xt = T("x", [Tn, nh * HD], exp=np.repeat(fx, HD))
    yt = T("y", [Tn, nh * HD], exp=np.repeat(fo, HD))
    node = rn.RopeRoNode([xt], yt, heads=nh, head_dim=HD, cos=GOLD[f"rope{i}_cos"], sin=GOLD[f"rope{i}_sin"],
                         pos=int(GOLD[f"rope{i}_pos"][0]))
    return node, [(xt, x.reshape(Tn, -1))], GOLD[f"rope{i}_y"].reshape(Tn, -1)


def bias_copy(i):
    x = GOLD[f"bias{i}_x"]
    rows, n = x.shape
    xt, yt = T("x", [rows, n], exp=GOLD[f"bias{i}_fx"]), T("y", [rows, n], exp=GOLD[f"bias{i}_fo"])
    node = rn.BiasCopyRoNode([xt], yt, bias=GOLD[f"bias{i}_bias"], relu=bool(GOLD[f"bias{i}_relu"][0]))
    return node, [(xt, x)], GOLD[f"bias{i}_y"]


def res_add():
    """h1 = sat32(h + d << (fr - f_d)) (rowops_nodes.py:421-425: rint((h + d) 2^fr), clipped)."""
    rng = np.random.default_rng(7)
    rows, n, fr = 6, 96, 15
    h = rng.integers(-2 ** 31, 2 ** 31, (rows, n), dtype=np.int64)
    h[0, :4] = [2 ** 31 - 1, -2 ** 31, 2 ** 31 - 5, -2 ** 31 + 5]
    fd = rng.integers(6, 16, n)
    d = rng.integers(-32768, 32768, (rows, n), dtype=np.int64)
    d[0, :4] = [32767, -32768, 32767, -32768]
    ht, dt, yt = T("h", [rows, n], "i32", fr), T("d", [rows, n], exp=fd), T("y", [rows, n], "i32", fr)
    want = np.clip(h + (d << (fr - fd)[None, :]), -2 ** 31, 2 ** 31 - 1)
    return rn.ResAddRoNode([ht, dt], yt), [(ht, h), (dt, d)], want


def res_add_bias(a32):
    """sat32(rint((h + d + quant_bias(bias, fr)) 2^fr)) (rowops_nodes.py:1258-1263), in integers;
    the integer form equals the reference's value form (checked here)."""
    rng = np.random.default_rng(8 + a32)
    rows, n, fr = 4, 64, 15
    fa = np.full(n, fr if a32 else 10)
    h = (rng.integers(-2 ** 30, 2 ** 30, (rows, n)) if a32 else rng.integers(-32768, 32768, (rows, n))).astype(np.int64)
    fd = rng.integers(6, 16, n)
    d = rng.integers(-32768, 32768, (rows, n), dtype=np.int64)
    bias = rng.uniform(-3, 3, n)
    ht = T("h", [rows, n], "i32" if a32 else "i16", fr if a32 else fa)
    dt, yt = T("d", [rows, n], exp=fd), T("y", [rows, n], "i32", fr)
    bb = rn.bias_bits(bias, fr)
    bq = np.rint(bias * 2.0 ** bb).astype(np.int64)
    want = np.clip((h << (fr - fa)[None, :]) + (d << (fr - fd)[None, :]) + (bq << (fr - bb))[None, :],
                   -2 ** 31, 2 ** 31 - 1)
    vals = h / 2.0 ** fa[None, :] + d / 2.0 ** fd[None, :] + rn.quant_bias(bias, fr)[None, :]
    assert np.array_equal(want, np.clip(np.rint(vals * 2.0 ** fr), -2 ** 31, 2 ** 31 - 1))
    return rn.ResAddBiasRoNode([ht, dt], yt, bias=bias), [(ht, h), (dt, d)], want


def widen():
    rng = np.random.default_rng(9)
    rows, n, fy = 3, 40, 16
    fx = rng.integers(0, 17, n)
    x = rng.integers(-32768, 32768, (rows, n), dtype=np.int64)
    xt, yt = T("x", [rows, n], exp=fx), T("y", [rows, n], "i32", fy)
    return rn.WidenRoNode([xt], yt), [(xt, x)], x << (fy - fx)[None, :]


def dequant(case):
    """float32(raw 2^-f[c]), round to nearest even (rowops_nodes.py:2539-2541)."""
    rng = np.random.default_rng({"i16": 10, "i32": 11, "logits": 12}[case])
    rows, n = (5, 72) if case != "logits" else (1, 49152)
    kind = "i32" if case == "i32" else "i16"
    f = rng.integers(0, 30, n)
    lim = 2 ** 31 if kind == "i32" else 32768
    x = rng.integers(-lim, lim, (rows, n), dtype=np.int64)
    xt, yt = T("x", [rows, n], kind, f), T("y", [rows, n], "f32")
    return rn.DequantRoNode([xt], yt), [(xt, x)], (x / np.power(2.0, f)[None, :]).astype(np.float32)


CASES = ([(f"layer_norm{i}", lambda i=i: layer_norm(i)) for i in range(int(GOLD["ln_count"][0]))]
         + [(f"rms_norm{i}", lambda i=i: rms_norm(i)) for i in range(int(GOLD["rms_count"][0]))]
         + [("rms_norm_heads", rms_norm_over_heads)]
         + [(f"silu_mul{i}", lambda i=i: silu_mul(i)) for i in range(int(GOLD["silu_count"][0]))]
         + [(f"rope{i}", lambda i=i: rope(i)) for i in range(int(GOLD["rope_count"][0]))]
         + [(f"bias_copy{i}", lambda i=i: bias_copy(i)) for i in range(int(GOLD["bias_count"][0]))]
         + [("res_add", res_add), ("res_add_bias_i32", lambda: res_add_bias(True)),
            ("res_add_bias_i16", lambda: res_add_bias(False)), ("widen", widen)]
         + [(f"dequant_{c}", lambda c=c: dequant(c)) for c in ("i16", "i32", "logits")])


def same(got, want):
    """Bit-exact comparison (float32 outputs compared as bits)."""
    got, want = np.asarray(got), np.asarray(want)
    if want.dtype == np.float32:
        return np.array_equal(got.astype(np.float32).view(np.uint32), want.view(np.uint32))
    return np.array_equal(got.astype(np.int64), want.astype(np.int64))
