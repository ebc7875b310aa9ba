"""Writes tests/golden/smx_regs.npz: input / output vectors of the reference's softmax-unit
register derivation and integer softmax (inference-scheduler/src/vectorop_smx.py: scale_regs
:37-47, softmax_raw :50-66) that the hardware fixtures (11 softmax cases at fixed registers)
leave open: (Cm, Cs) over a grid of score exponents f_s and logit scales sigma, and P for
seeded rows at several register pairs, valid lengths and output exponents.

Runs in the build container only (it loads the reference module by path; the module imports
math, typing and numpy alone).  The npz holds data: the grid and the module's outputs.
Usage: python tests/golden/make_smx_regs_vectors.py
"""
import importlib.util
import math
import os

import numpy as np

SPEC = "/root/reference/inference-scheduler/src/vectorop_smx.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "smx_regs.npz")


def load_spec():
    spec = importlib.util.spec_from_file_location("ref_vectorop_smx", SPEC)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    smx = load_spec()
    out = {}
    # (f_s, sigma) over score exponents -8 .. 31 and the scales of attention heads 16 .. 128,
    # 1.0 (ONNX Softmax), and a few arbitrary ones; those Cs leaves out of range are skipped
    sigmas = [1.0, 0.5, 0.125, 0.37, 1.0 / math.sqrt(16), 1.0 / math.sqrt(32), 1.0 / math.sqrt(64),
              1.0 / math.sqrt(80), 1.0 / math.sqrt(96), 1.0 / math.sqrt(128), 2.0, 0.0123]
    grid = []
    for f_s in range(-8, 32):
        for sigma in sigmas:
            try:
                cm, cs = smx.scale_regs(f_s, sigma)
            except ValueError:
                continue
            grid.append((f_s, sigma, cm, cs))
    out["regs_fs"] = np.array([g[0] for g in grid], np.int64)
    out["regs_sigma"] = np.array([g[1] for g in grid], np.float64)
    out["regs_cm"] = np.array([g[2] for g in grid], np.int64)
    out["regs_cs"] = np.array([g[3] for g in grid], np.int64)

    # softmax_raw: seeded int16 rows [rows][n] at several registers, valid lengths, f_p
    rng = np.random.default_rng(20261202)
    cases = []
    for i, (rows, n, f_s, sigma, f_p, spread) in enumerate([
            (6, 64, 8, 1.0, 8, 2000), (5, 384, 11, 1.0 / 8, 14, 20000), (4, 96, 4, 0.37, 15, 300),
            (7, 1000, 13, 1.0 / math.sqrt(64), 14, 30000), (3, 16, 0, 1.0, 12, 40), (4, 2048, 9, 0.5, 13, 8000)]):
        cm, cs = smx.scale_regs(f_s, sigma)
        x = rng.integers(-spread, spread, (rows, n)).astype(np.int64)
        valid = rng.integers(0, n + 1, rows)
        valid[0] = n
        p = smx.softmax_raw(x, valid, cm, cs, f_p)
        out[f"sm{i}_x"], out[f"sm{i}_valid"], out[f"sm{i}_p"] = x.astype(np.int16), valid.astype(np.int64), p
        out[f"sm{i}_regs"] = np.array([cm, cs, f_p], np.int64)
        cases.append(i)
    out["sm_count"] = np.array([len(cases)])
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(grid)} register pairs, {len(cases)} softmax cases")


if __name__ == "__main__":
    main()
