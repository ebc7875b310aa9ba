#!/usr/bin/env python3
"""Throughput of the Matmul unit on one MI355X: the batched int16 Q8.8 MatMul of the
reference's MatmulKernel (A 4 x 512 x 4096, B 4096 x 4096 in packed 32-column tiles shared
by the batch, round-to-nearest inputs, floor + saturate outputs), bit-exact with the
reference simulator.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

A step is one cm_matmul call over the whole batch with inputs resident in HBM.  Prints one
JSON line: GMAC/s (int16 multiply-accumulates per second), the roofline of the dominant
kernel (the plane GEMM on i8 MFMA: 4 byte products of 2 ops per int16 MAC, against the
5.0 POP/s dense i8 peak), and the CPU baseline: the reference simulator's own algorithm
(float64 BLAS matmul + floor/clip, restated in oracle/sim_numpy.py) timed on the host cores
on one batch slice, whose output must equal the GPU's bit for bit.
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

N, K, M, BATCH = 512, 4096, 4096, 4
MACS = N * K * M * BATCH
I8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA, 5.0 POP/s
GEMM_KERNEL = "gemm_planes_kernel"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_planes_kernel_matmul_512x4096x4096x4_traffic.md")


def quantize_q88(v):
    """ApFixed.quantize (dtype.py:367-369): clip to [-128, 127.996], round half to even."""
    import numpy as np
    return np.round(np.clip(v, -128.0, 127.99609375) * 256.0).astype(np.int16)


def make_inputs(seed: int):
    import numpy as np
    rng = np.random.default_rng(seed)
    a = quantize_q88(np.clip(rng.standard_normal((BATCH, N, K)), -8.0, 8.0))
    b = quantize_q88(rng.normal(0.0, 0.05, (K, M)))
    # packed tile-major image: Bp[(mt * K + kk) * 32 + m1] = B[kk][mt * 32 + m1]
    bp = np.ascontiguousarray(b.reshape(K, M // 32, 32).transpose(1, 0, 2)).reshape(-1)
    return a, b, bp


def read_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 --pmc summary, if any."""
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def cpu_baseline(a, b, min_seconds: float = 10.0):
    """The reference simulator's Q8.8 MatMul (np.matmul float64 + truncate) over the whole
    batch, repeated on this host's cores until at least `min_seconds` have passed; returns
    (GMAC/s, BLAS threads, seconds, repetitions, output)."""
    from oracle import sim_numpy
    try:
        from threadpoolctl import threadpool_info
        threads = max((i.get("num_threads", 1) for i in threadpool_info()
                       if i.get("user_api") == "blas"), default=1)
    except Exception:
        threads = os.cpu_count() or 1
    reps, t0 = 0, time.perf_counter()
    while True:
        out = sim_numpy.matmul_q88(a, b)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    return MACS * reps / dt / 1e9, threads, dt, reps, out


CAL_ELEMS = 128 << 20          # 256 MiB of int16


def calibrate(units, torch):
    """A plain copy of known size for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE: RELU
    (VectorOP op 4) over non-negative values reads 256 MiB and writes 256 MiB."""
    x = torch.arange(CAL_ELEMS, device="cuda", dtype=torch.int32).remainder_(30000).to(torch.int16)
    y = torch.empty_like(x)
    units.init()
    for _ in range(3):
        units.vectorop(x, None, y, CAL_ELEMS, units.OP_RELU)
    torch.cuda.synchronize()
    assert torch.equal(x, y)
    print(json.dumps({"calibration": "vectorop_kernel RELU", "bytes_read": CAL_ELEMS * 2,
                      "bytes_written": CAL_ELEMS * 2, "launches": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the default warmup outlasts the power controller's first response to the load (the
    # clock dips for some tens of steps, then settles), so the timed steps see its steady state
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate", action="store_true",
                    help="run only the copy used to scale HBM counters: a RELU over 256 MiB of "
                         "non-negative int16 (reads and writes exactly 256 MiB each)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the units run on a single MI355X here; "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from cormorant_amd import _lib, units

    if args.calibrate:
        calibrate(units, torch)
        return
    a, b, bp = make_inputs(args.seed)
    dev = torch.device("cuda:0")
    da = torch.from_numpy(a.reshape(-1)).to(dev)
    dbp = torch.from_numpy(bp).to(dev)
    dc = torch.empty(BATCH * N * M, dtype=torch.int16, device=dev)
    units.init()

    def step():
        units.matmul(da, dbp, dc, N, K, M, batch=BATCH, a_bs=N * K, b_bs=0, c_bs=N * M,
                     b_packed=1)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    _lib.timing_reset()
    _lib.timing_select(GEMM_KERNEL)     # events around the GEMM launches only
    _lib.timing_enable(True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    _lib.timing_select("")
    ms = start.elapsed_time(stop) / args.steps
    gemm_ms, gemm_n = _lib.timing_read(GEMM_KERNEL)
    gemm_avg_ms = gemm_ms / max(gemm_n, 1)
    _lib.timing_reset()

    achieved = 8.0 * MACS / (gemm_avg_ms * 1e-3) / 1e12        # i8 TOP/s of the GEMM kernel
    traffic = read_traffic()
    result = {
        "metric": "bit-exact fixed-point GMAC/s + inferences/s (BERT-base L384) vs CPU simulator",
        "value": round(MACS / (ms * 1e-3) / 1e9, 1),
        "unit": "GMAC/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16",
        "data": f"synthetic (seed {args.seed}): A N(0,1) clipped to +-8, B N(0,0.05), Q8.8 RNE",
        "config": {"workload": "MatmulKernel int16 Q8.8 batched x4: A 4x512x4096, B 4096x4096 "
                               "packed 32-column tiles shared by the batch, no bias",
                   "n": N, "k": K, "m": M, "batch": BATCH, "b_packed": 1, "wrap32": 0},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": I8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / I8_PEAK_TOPS, 4),
                     "traffic": traffic, "kernel": GEMM_KERNEL,
                     "kernel_ms": round(gemm_avg_ms, 4),
                     "ops_per_launch": 8 * MACS},
    }

    # full-size bit-exact check of the whole output against the reference's CPU algorithm
    if not args.no_cpu_baseline:
        gmacs, threads, dt, reps, cref = cpu_baseline(a, b)
        got = dc.cpu().numpy().reshape(BATCH, N, M)
        result["cpu_baseline"] = {"value": round(gmacs, 2), "unit": "GMAC/s", "cores": threads,
                                  "kind": "port",
                                  "sample": f"the whole step ({BATCH}x{N}x{K}x{M}) {reps} times in "
                                            f"{dt:.1f} s: float64 np.matmul + clip/floor as "
                                            "_simulate.py:620-633"}
        result["parity"] = ("output bit-exact vs the CPU simulator algorithm"
                            if np.array_equal(got, cref) else "MISMATCH vs the CPU simulator algorithm")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
