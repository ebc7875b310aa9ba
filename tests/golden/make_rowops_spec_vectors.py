"""Writes tests/golden/rowops_spec.npz: input / output vectors of the reference's row-ops
integer specifications (inference-scheduler/src/rowops_spec.py) for the node adapters'
parameter derivation and arithmetic, which the hardware fixtures (hw/test_data, built from
ready parameter blocks) leave open: norm_params / gamma_scale / beta_bits (float gamma,
beta, eps -> the job constants), layer_norm (int16 and int32 rows), rms_norm, silu_mul,
rope, bias_round / bias_params and quant_bias.

Runs in the build container only (it loads the reference module by path; the module
imports math, functools, typing and numpy alone).  The npz holds data: seeded inputs and
the module's outputs.  Usage: python tests/golden/make_rowops_spec_vectors.py
"""
import importlib.util
import math
import os

import numpy as np

SPEC = "/root/reference/inference-scheduler/src/rowops_spec.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rowops_spec.npz")


def load_spec():
    spec = importlib.util.spec_from_file_location("ref_rowops_spec", SPEC)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    rs = load_spec()
    rng = np.random.default_rng(20260101)
    out = {}

    # ---- norm_params / gamma_scale / beta_bits over assorted gamma, beta, eps, n, f_in
    np_cases = []
    for i in range(24):
        n = int(rng.choice([8, 64, 96, 576, 768, 960]))
        gamma = rng.uniform(0.02, 6.0, n) * rng.choice([1e-3, 1.0, 30.0])
        beta = rng.uniform(-1, 1, n) * rng.choice([0.1, 1.5, 4.2, 40.0])
        eps = float(rng.choice([1e-12, 1e-6, 1e-5, 1e-3]))
        f_in = int(rng.choice([8, 12, 15, 16]))
        rms = bool(i % 2)
        G, g, Bq, E = rs.norm_params(gamma, n, eps, f_in, beta=None if rms else beta, rms=rms)
        np_cases.append(i)
        out[f"np{i}_gamma"], out[f"np{i}_beta"] = gamma, beta
        out[f"np{i}_meta"] = np.array([n, f_in, int(rms), g, E, rs.beta_bits(beta), rs.gamma_scale(gamma)],
                                      np.int64)
        out[f"np{i}_eps"] = np.array([eps])
        out[f"np{i}_G"] = G
        out[f"np{i}_Bq"] = np.zeros(0, np.int64) if Bq is None else Bq
    out["np_count"] = np.array([len(np_cases)])

    # ---- layer_norm: int16 rows at 2^-8 -> 2^-8 (LayerNormRoNode), and the int32 residual
    # at 2^-15 -> per-channel exponents (LayerNorm32RoNode)
    ln = []
    for i, (rows, n, kind) in enumerate([(6, 96, "i16"), (5, 64, "i16"), (4, 768, "i16"), (5, 64, "i32"),
                                         (3, 256, "i32"), (4, 32, "i16")]):
        gamma = rng.uniform(0.2, 2.0, n)
        beta = rng.uniform(-0.5, 0.5, n) * (8.0 if i == 4 else 1.0)
        eps = [1e-5, 1e-12, 1e-5, 1e-6, 1e-6, 1e-3][i]
        if kind == "i16":
            x = rng.standard_normal((rows, n)) * rng.choice([0.05, 1.0, 8.0], rows)[:, None] + 3.0
            x_raw = np.clip(np.rint(x * 256.0), -32768, 32767).astype(np.int64)
            if i == 5:
                x_raw[0] = 77                                       # a constant row: V = 0
            f_x, f_out = 8, np.full(n, 8, np.int64)
        else:
            x = rng.standard_normal((rows, n)) * rng.choice([0.01, 1.0, 40.0], rows)[:, None]
            x_raw = np.rint(x * 2.0 ** 15).astype(np.int64)
            f_x, f_out = 15, rng.integers(8, 13, n).astype(np.int64)
        y = rs.layer_norm(x_raw, f_x, gamma, beta, eps, f_out)
        out.update({f"ln{i}_x": x_raw, f"ln{i}_gamma": gamma, f"ln{i}_beta": beta, f"ln{i}_eps": np.array([eps]),
                    f"ln{i}_fx": np.array([f_x]), f"ln{i}_fout": f_out, f"ln{i}_y": y,
                    f"ln{i}_kind": np.array([0 if kind == "i16" else 1])})
        ln.append(i)
    out["ln_count"] = np.array([len(ln)])

    # ---- rms_norm: the int32 residual at 2^-fr -> per-channel exponents
    for i, (rows, n, fr) in enumerate([(5, 64, 15), (4, 960, 15), (3, 32, 12)]):
        gamma = rng.uniform(0.05, 4.0, n)
        h = rng.standard_normal((rows, n)) * rng.choice([0.01, 1.0, 40.0], rows)[:, None]
        h[0, 3] = 25000.0 / 2 ** (15 - fr) if rows > 0 else 0.0
        h_raw = np.clip(np.rint(h * 2.0 ** fr), -2 ** 31, 2 ** 31 - 1).astype(np.int64)
        f_out = rng.integers(8, 13, n).astype(np.int64)
        eps = [1e-5, 1e-5, 1e-6][i]
        y = rs.rms_norm(h_raw, fr, gamma, eps, f_out)
        out.update({f"rms{i}_h": h_raw, f"rms{i}_gamma": gamma, f"rms{i}_eps": np.array([eps]),
                    f"rms{i}_fr": np.array([fr]), f"rms{i}_fout": f_out, f"rms{i}_y": y})
    out["rms_count"] = np.array([3])

    # ---- silu_mul: gate at per-channel exponents <= 14, up and output at theirs
    for i, (rows, n) in enumerate([(4, 64), (3, 256)]):
        fg = rng.integers(6, 15, n).astype(np.int64)
        fu = rng.integers(6, 13, n).astype(np.int64)
        fa = rng.integers(6, 13, n).astype(np.int64)
        g = rng.integers(-32768, 32768, (rows, n)).astype(np.int64)
        u = rng.integers(-32768, 32768, (rows, n)).astype(np.int64)
        y = rs.silu_mul(g, fg, u, fu, fa)
        out.update({f"silu{i}_g": g, f"silu{i}_u": u, f"silu{i}_fg": fg, f"silu{i}_fu": fu, f"silu{i}_fa": fa,
                    f"silu{i}_y": y})
    out["silu_count"] = np.array([2])

    # ---- rope: rotate-half over heads, cos / sin rows of positions pos .. pos + T
    for i, (T, nh, HD, C, pos) in enumerate([(4, 3, 16, 32, 5), (2, 5, 64, 64, 40)]):
        theta = 1e5 if i else 1e4
        inv = 1.0 / theta ** (np.arange(0, HD, 2, dtype=np.float64) / HD)
        ang = np.arange(C, dtype=np.float64)[:, None] * inv[None, :]
        cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        cr, sr = rs.rope_tables_raw(np.concatenate([cos, cos], 1).astype(np.float64),
                                    np.concatenate([sin, sin], 1).astype(np.float64))
        fx = rng.integers(6, 13, nh).astype(np.int64)
        fo = rng.integers(6, 13, nh).astype(np.int64)
        x = rng.integers(-32768, 32768, (T, nh, HD)).astype(np.int64)
        y = rs.rope(x, np.repeat(fx[:, None], HD, 1), cr[pos:pos + T], sr[pos:pos + T], fo)
        out.update({f"rope{i}_x": x, f"rope{i}_cos": cos, f"rope{i}_sin": sin, f"rope{i}_cr": cr, f"rope{i}_sr": sr,
                    f"rope{i}_fx": fx, f"rope{i}_fo": fo, f"rope{i}_pos": np.array([pos]), f"rope{i}_y": y})
    out["rope_count"] = np.array([2])

    # ---- bias_round (a COPY with a per-column bias), bias_params, quant_bias / bias_bits
    for i, (rows, n, relu) in enumerate([(4, 32, False), (3, 64, True)]):
        fx = rng.integers(6, 13, n).astype(np.int64)
        fo = rng.integers(6, 13, n).astype(np.int64)
        bias = rng.uniform(-3, 3, n) * (10.0 if i else 1.0)
        x = rng.integers(-32768, 32768, (rows, n)).astype(np.int64)
        y = rs.bias_round(x, fx, bias, fo, relu=relu)
        bq, sa, sc = rs.bias_params(bias, fx, fo)
        out.update({f"bias{i}_x": x, f"bias{i}_fx": fx, f"bias{i}_fo": fo, f"bias{i}_bias": bias,
                    f"bias{i}_relu": np.array([int(relu)]), f"bias{i}_y": y, f"bias{i}_bq": bq, f"bias{i}_sa": sa,
                    f"bias{i}_sc": sc})
    out["bias_count"] = np.array([2])
    for i in range(6):
        bias = rng.uniform(-1, 1, 48) * [0.5, 3.0, 9.0, 100.0, 1e-3, 2.0][i]
        fr = [15, 15, 12, 15, 8, 20][i]
        out[f"qb{i}_bias"], out[f"qb{i}_fr"] = bias, np.array([fr])
        out[f"qb{i}_bb"] = np.array([rs.bias_bits(bias, fr)])
        out[f"qb{i}_q"] = rs.quant_bias(bias, fr)
    out["qb_count"] = np.array([6])

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
