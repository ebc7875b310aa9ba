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
BERT_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_planes_kernel_bert_base_l384_traffic.md")


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


def read_traffic(path=TRAFFIC_FILE, key="traffic_bytes_per_launch"):
    """HBM bytes of the GEMM from a committed rocprofv3 --pmc summary, if any."""
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(key + r":\s*([0-9.eE+]+)", text)
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


HBM_PEAK_GBS = 8000.0


def hbm_kernels(torch, units, reps: int = 20):
    """The HBM-bound units at shapes of the reference's configurations, each a workload of
    tens of MB: algorithmic bytes (each tensor once; 2 B int16, 4 B int32 / float32) over the
    mean time of ``reps`` back-to-back launches.  One JSON line per workload."""
    import numpy as np
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    i16 = lambda n, lo=-32768, hi=32768: torch.randint(lo, hi, (n,), dtype=torch.int16, device=dev, generator=g)  # noqa: E731
    i32 = lambda n, lo=-2 ** 30, hi=2 ** 30: torch.randint(lo, hi, (n,), dtype=torch.int32, device=dev, generator=g)  # noqa: E731
    u8 = lambda t: t.view(torch.uint8)   # noqa: E731
    lines = []

    def run(name, shape, nbytes, fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        us = s.elapsed_time(e) / reps * 1e3
        gbs = nbytes / (us * 1e-6) / 1e9
        line = {"kernel": name, "shape": shape, "bytes": int(nbytes), "us": round(us, 2), "GB/s": round(gbs, 1),
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
        print(json.dumps(line), flush=True)
        lines.append(line)

    units.init()
    # element-wise VectorOP: one run of the whole tensor
    def elementwise(name, shape, op, binary, act=0):
        n = int(np.prod(shape))
        a, b, c = i16(n), i16(n) if binary else None, torch.empty(n, dtype=torch.int16, device=dev)
        run(name, shape, (6 if binary else 4) * n, lambda: units.vectorop(a, b, c, n, op, act=act))
    elementwise("vectorop_kernel RELU6 (MobileNetV2 expand output)", [32, 96, 112, 112], units.OP_RELU6, False)
    elementwise("vectorop_kernel ADD (MobileNetV2 residual)", [32, 144, 56, 56], units.OP_ADD, True)
    elementwise("vectorop_kernel GELU erf (BERT FFN)", [3072, 3072], units.OP_GELU, False)
    # softmax: keys-major (BERT attention, 96 heads of 384 keys x 384 queries) and row mode
    heads, keys, q = 96, 384, 384
    x = i16(heads * keys * q, -2000, 2000)
    y = torch.empty(heads * q * keys, dtype=torch.int16, device=dev)
    run("softmax_cols_kernel (BERT, 96 heads)", [heads, keys, q], 4 * heads * keys * q,
        lambda: units.softmax(x, y, keys, units.OP_SOFTMAX_T, q, q, keys, 12102203, 0x0813, keys, batch=heads,
                              a_bs=keys * q, c_bs=q * keys))
    rows = heads * q
    run("softmax_rows_kernel (BERT row mode)", [rows, keys], 4 * rows * keys,
        lambda: units.vectorop(x, None, y, keys, units.OP_SOFTMAX, outer=rows, a_inc=keys, b_inc=keys,
                               smx_cm=12102203, smx_cfg=0x0813, smx_mask=keys))
    # pooling
    N, C, H = 32, 64, 112
    xp, yp = i16(N * C * H * H), torch.empty(N * C * (H // 2) ** 2, dtype=torch.int16, device=dev)
    run("pool_kernel MAX 2x2 s2", [N, C, H, H], 2 * N * C * H * H + 2 * N * C * (H // 2) ** 2,
        lambda: units.pool(xp, yp, N, C, H, H, H // 2, H // 2, 2, 2, 2, 2))
    N, C, H = 32, 1280, 7
    xg, yg = i16(N * C * H * H), torch.empty(N * C, dtype=torch.int16, device=dev)
    run("pool_global_kernel AVG (MobileNetV2 head)", [N, C, H, H], 2 * N * C * H * H + 2 * N * C,
        lambda: units.pool(xg, yg, N, C, H, H, 1, 1, H, H, 1, 1, pool_type=units.POOL_AVG))
    # depthwise 3x3 conv (MobileNetV2 block)
    N, C, H = 32, 144, 56
    xd, yd = i16(N * C * H * H, -2048, 2048), torch.empty(N * C * H * H, dtype=torch.int16, device=dev)
    wd = i16(units.conv_weight_numel(C, C, 3, 3, True), -512, 512)
    bd = i16(C, -512, 512)
    run("conv_dw_kernel 3x3 s1 (MobileNetV2)", [N, C, H, H], 4 * N * C * H * H,
        lambda: units.conv(xd, wd, bd, yd, N, C, H, H, C, H, H, 3, 3, pad_top=1, pad_left=1, has_bias=1,
                           is_depthwise=1))
    # row-ops jobs on contiguous rows (one broadcast parameter entry)
    p0 = torch.zeros(16, dtype=torch.uint8, device=dev)
    def rowjob(name, rows, n, op, ak, ck, bk=None, aux=0, nbytes=None, rope_hd=0, a32_range=2 ** 30, per_col=False):
        kb = {units.K_I16: 2, units.K_I32: 4, units.K_F32: 4}
        a = i32(rows * n, -a32_range, a32_range) if ak == units.K_I32 else i16(rows * n, -4096, 4096)
        b, b_s1 = None, 0
        if rope_hd:                       # one cos / sin position row (2 HD int32) per row
            b, b_s1 = i32(rows * 2 * rope_hd, -2 ** 23, 2 ** 23), 8 * rope_hd
        elif bk is not None:
            b = i32(rows * n) if bk == units.K_I32 else i16(rows * n, -4096, 4096)
            b_s1 = kb[bk] * n
        c = torch.empty(rows * n * kb[ck], dtype=torch.uint8, device=dev)
        opw = op | (ak << 4) | ((bk or 0) << 6) | (ck << 8) | (units.F_B_EN if bk is not None else 0)
        p = torch.zeros(16 * n, dtype=torch.uint8, device=dev) if per_col else p0
        opw |= 0 if per_col else units.F_P_BCAST
        run(name, [rows, n], nbytes, lambda: units.rowops(u8(a), u8(b) if b is not None else None, c, p, opw, n,
                                                           rows, 1, kb[ak] * n, 0, b_s1, 0, kb[ck] * n, 0, 1 << 20,
                                                           aux, 0))
    # norm inputs in a residual stream's range (|x| < 2^20, 32 at 2^-15)
    rowjob("ro_norm_kernel LayerNorm i32->i16 (BERT)", 3072 * 8, 768, units.RO_NORM | units.F_NORM_LN, units.K_I32,
           units.K_I16, nbytes=6 * 3072 * 8 * 768, a32_range=2 ** 20)
    rowjob("ro_norm_kernel LayerNorm i32->i16 (BERT, one forward's 3072 rows, per-column G / B)", 3072, 768,
           units.RO_NORM | units.F_NORM_LN, units.K_I32, units.K_I16, nbytes=6 * 3072 * 768, a32_range=2 ** 20,
           per_col=True)
    rowjob("ro_norm_kernel RMSNorm i32->i16 (SmolLM2 rows)", 16384, 960, units.RO_NORM, units.K_I32, units.K_I16,
           nbytes=6 * 16384 * 960, a32_range=2 ** 20)
    rowjob("ro_stream_kernel ADDX i32+i16->i32", 3072 * 8, 768, units.RO_ADDX, units.K_I32, units.K_I32,
           bk=units.K_I16, nbytes=10 * 3072 * 8 * 768)
    rowjob("ro_stream_kernel ADDX i32+i16->i32 (BERT residual, 3072 rows, per-column bias)", 3072, 768, units.RO_ADDX,
           units.K_I32, units.K_I32, bk=units.K_I16, nbytes=10 * 3072 * 768, per_col=True)
    rowjob("ro_stream_kernel MULACT (SiLU x up)", 8192, 2560, units.RO_MULACT, units.K_I16, units.K_I16,
           bk=units.K_I16, nbytes=6 * 8192 * 2560)
    rowjob("ro_stream_kernel DEQUANT i16->f32 (logits)", 4096, 4096, units.RO_DEQUANT, units.K_I16, units.K_F32,
           nbytes=6 * 4096 * 4096)
    rowjob("ro_stream_kernel ROPE (SmolLM2 q, HD 64)", 16384, 960, units.RO_ROPE, units.K_I16, units.K_I16,
           bk=units.K_I32, aux=64, rope_hd=64, nbytes=4 * 16384 * 960 + 8 * 64 * 16384)
    return lines


# ---------------------------------------------------------------- graph workloads
GRAPH_KERNELS = ("gemm_planes_kernel", "split_rows_kernel", "split_cols_kernel", "split_kernel",
                 "softmax_cols_kernel", "softmax_rows_kernel", "ro_norm_kernel", "ro_stream_kernel",
                 "vectorop_kernel", "permute_words_kernel", "permute_tile_kernel", "conv_dw_kernel",
                 "conv_dw3_kernel", "conv_dw3v_kernel", "pool_kernel", "pool_global_kernel", "pool2x2_kernel",
                 "softmax_long_kernel", "smx_etab_kernel", "copy_elems_kernel", "permute_elems_kernel",
                 "split_fold_kernel", "split_fold_lds_kernel", "skinny_wrap_kernel", "skinny_reduce_kernel",
                 "skinny_planes_kernel", "skinny_mulact_kernel", "decode_attn_kernel", "decode_prep_kernel",
                 "attention_kernel", "embed_rows_kernel", "ro_fold_kernel",
                 "ro_tload_kernel", "ro_xpose_kernel", "conv_small_kernel")


TIMED_REPLAYS = 10      # replays of the instrumented graph whose per-launch events are read


def run_graph(args, torch, sim, feeds, out_name, each=()):
    """Warm the simulator up, capture the forward as a HIP graph and time ``args.steps``
    replays after ``args.warmup`` (the step time).  Then capture the same forward a second time
    with a HIP event pair around every kernel launch -- on a stream under capture the pairs are
    event-record nodes of the graph, re-recorded by each replay -- and read them after each of
    TIMED_REPLAYS replays, each run right after three replays of the plain graph so that the GPU
    is in the same loaded state as in the timed region.  Returns (ms per step, {kernel: {ms per
    step (mean over the instrumented replays), launches per step}}, the output tensor); with
    ``each``, per_kernel[name]["each"] for those kernels: every launch's mean ms, in launch order."""
    from cormorant_amd import _lib
    keep = [out_name]                         # the step's result; intermediates only the GEMMs read stay unwritten
    for _ in range(2):                        # weights, packed images, tables, workspace
        sim.forward_raw(feeds, keep=keep)
    torch.cuda.synchronize()
    # one timed eager forward creates the event pairs the instrumented capture reuses (no event is
    # created while a stream is being captured)
    _lib.timing_reset()
    _lib.timing_select("")
    _lib.timing_enable(True)
    sim.forward_raw(feeds, keep=keep)
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    _lib.timing_reset()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sim.forward_raw(feeds, keep=keep)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    hg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(hg):
        out = sim.forward_raw(feeds, keep=keep)[out_name]
    for _ in range(args.warmup):
        hg.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        hg.replay()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps

    # the instrumented graph: the same launches, each between two event-record nodes
    hg_t = torch.cuda.CUDAGraph()
    _lib.timing_enable(True)
    try:
        with torch.cuda.graph(hg_t):
            sim.forward_raw(feeds, keep=keep)
    finally:
        _lib.timing_enable(False)
    acc, acc_each = {}, {}
    for _ in range(TIMED_REPLAYS):
        for _ in range(3):
            hg.replay()
        hg_t.replay()
        torch.cuda.synchronize()
        for k in GRAPH_KERNELS:
            ms_k, n_k = _lib.timing_read(k)
            if n_k:
                a = acc.setdefault(k, [0.0, n_k])
                a[0] += ms_k
        for k in each:
            e = _lib.timing_read_each(k)
            a = acc_each.setdefault(k, [0.0] * len(e))
            for i, v in enumerate(e):
                a[i] += v
    _lib.timing_reset()
    del hg_t
    per_kernel = {k: {"ms": round(v[0] / TIMED_REPLAYS, 4), "launches": v[1]} for k, v in acc.items()}
    for k, v in acc_each.items():
        per_kernel.setdefault(k, {"ms": 0.0, "launches": 0})["each"] = [x / TIMED_REPLAYS for x in v]
    return ms, per_kernel, out


def step_fields(args, ms):
    return {"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int16"}


def gemm_roofline(per_kernel, macs):
    gemm_ms = per_kernel.get(GEMM_KERNEL, {}).get("ms", float("nan"))
    achieved = 8.0 * macs / (gemm_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": I8_PEAK_TOPS, "unit": "TFLOP/s",
            "frac": round(achieved / I8_PEAK_TOPS, 4), "traffic": None, "kernel": GEMM_KERNEL,
            "kernel_ms_per_step": gemm_ms, "ops_per_step": 8 * macs}


def cnn_roofline(g, per_kernel):
    """The small CNN's dominant kernel, the two few-tap convolutions (conv_small_kernel, on the
    VALU), against HBM: their algorithmic bytes (input, weights, output once at int16) over
    their summed launch time.  At batch 1 every launch is latency-bound."""
    byt = 0
    for sn in g.nodes:
        if type(sn).__name__ == "ConvNode":
            byt += 2 * (sn.batch * sn.in_ch * sn.in_h * sn.in_w + sn.out_ch * sn.in_ch * sn.kh * sn.kw
                        + sn.batch * sn.out_ch * sn.out_h * sn.out_w)
    t_ms = per_kernel.get("conv_small_kernel", {}).get("ms", float("nan"))
    gbs = byt / (t_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 6), "traffic": None, "kernel": "conv_small_kernel",
            "kernel_ms_per_step": t_ms, "bytes_per_step": byt,
            "note": "latency-bound: two launches over 26 KB of tensors; the fraction is not meaningful"}


def cores():
    return len(os.sched_getaffinity(0))


def finish(result, ok=None):
    """Print the JSON line; exit 1 when the parity check ran and found a mismatch (the line
    then carries "MISMATCH" and no figure of it may be used)."""
    print(json.dumps(result), flush=True)
    if ok is False:
        print("bench.py: the GPU output differs from the CPU simulator algorithm", file=sys.stderr, flush=True)
        sys.exit(1)


# ---------------------------------------------------------------- BERT-base L384 encoder forward
def bert_bench(args, torch, np):
    """One step = one forward of the 12-layer encoder over the batch of 8 x 384 tokens, the
    int32 residual input resident on the GPU, replayed as a captured HIP graph."""
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator

    shape = models.BertShape()
    t0 = time.time()
    g, inputs, exps = models.bert_encoder(shape, seed=args.seed)
    build_s = time.time() - t0
    sim = Simulator(g)
    out_name = g.output_tensors[0].onnx_name
    feeds = {name: sim._to_device(sim._tensor(name), v) for name, v in inputs.items()}
    ms, per_kernel, out = run_graph(args, torch, sim, feeds, out_name)
    macs = shape.macs()
    result = {
        "metric": "bit-exact fixed-point GMAC/s + inferences/s (BERT-base L384) vs CPU simulator",
        "value": round(macs / (ms * 1e-3) / 1e9, 1),
        "unit": "GMAC/s",
        "inferences_per_s": round(shape.batch / (ms * 1e-3), 1),
        **step_fields(args, ms),
        "data": f"synthetic (seed {args.seed}): token ids U(0, 30522) (the step's input, gathered on the GPU), "
                "embedding rows N(0,1), weights / "
                "biases N(0,0.02), LayerNorm gamma N(1,0.02), beta N(0,0.02); per-tensor pow2 exponents "
                "from a float64 calibration of the first sequence",
        "config": {"workload": "BERT-base-shaped encoder forward: 12 layers, batch 8, sequence 384, hidden "
                               "768, 12 heads x 64, FFN 3072 GELU(erf), pre-LN on an int32 residual at 2^-15",
                   "layers": shape.layers, "batch": shape.batch, "seq": shape.seq, "hidden": shape.d,
                   "heads": shape.heads, "ffn": shape.ff, "macs_per_step": macs},
        "roofline": gemm_roofline(per_kernel, shape.linear_macs()),
        "kernels_ms_per_step": per_kernel,
        "graph_build_s": round(build_s, 1),
    }
    # the second kernel: the fused attention, against its algorithmic contractions only (q.K^T and
    # P.V, 2 x 384^2 x 64 MAC per (sequence, head); the softmax's VALU work is not counted)
    att_macs = shape.macs() - shape.linear_macs()
    att_ms = per_kernel.get("attention_kernel", {}).get("ms", float("nan"))
    result["attention_roofline"] = {"bound": "mfma", "kernel": "attention_kernel", "kernel_ms_per_step": att_ms,
                                    "ops_per_step": 8 * att_macs,
                                    "achieved": round(8.0 * att_macs / (att_ms * 1e-3) / 1e12, 1),
                                    "peak": I8_PEAK_TOPS, "unit": "TFLOP/s",
                                    "frac": round(8.0 * att_macs / (att_ms * 1e-3) / 1e12 / I8_PEAK_TOPS, 4)}
    # the GEMM launches' HBM bytes per forward, from the committed --pmc summary
    result["roofline"]["traffic"] = read_traffic(BERT_TRAFFIC_FILE, "traffic_bytes_per_step")
    ok = None
    if not args.no_cpu_baseline:
        from oracle import graph_sim
        # parity: the whole step on the CPU (float64 BLAS contractions, the C oracle's units)
        t1 = time.time()
        full = graph_sim.forward(g, inputs)
        dt_full = time.time() - t1
        got = sim._to_values(sim._tensor(out_name), out)
        ok = bool(np.array_equal(got, full[out_name].reshape(got.shape)))
        # the CPU baselines on layer 0 (every layer has the same shapes and work): the same seed's
        # one-layer encoder is the first layer of the twelve, checked against the step's tensor
        g1, in1, _ = models.bert_encoder(models.BertShape(layers=1), seed=args.seed)
        layer_macs = macs // shape.layers
        cpu = {}
        for algo in ("ref", "oracle"):
            t1 = time.time()
            v1 = graph_sim.forward(g1, in1, algo=algo)
            cpu[algo] = time.time() - t1
            ok = ok and bool(np.array_equal(v1[g1.output_tensors[0].onnx_name], full["l0.h"]))
        result["cpu_baseline"] = {
            "label": "cpu_sim_ref", "value": round(layer_macs / cpu["ref"] / 1e9, 3), "unit": "GMAC/s",
            "cores": cores(), "kind": "port", "extrapolated": True,
            "sample": f"layer 0 of 12 over the whole batch ({shape.batch} x {shape.seq} tokens, "
                      f"{layer_macs / 1e9:.2f} GMAC) in {cpu['ref']:.1f} s, the per-layer rate standing for the "
                      "12 identical layers: the reference simulator's algorithms restated -- float64 BLAS "
                      "contractions, per-row LayerNorm in Python integers (rowops_spec.py:249-282), GELU by "
                      "np.vectorize(math.erf) per element (host_nodes.py:156-162), the integer softmax"}
        result["cpu_ref"] = {
            "label": "cpu_ref", "value": round(layer_macs / cpu["oracle"] / 1e9, 3), "unit": "GMAC/s",
            "cores": cores(), "kind": "port", "extrapolated": True,
            "sample": f"layer 0 of 12 over the whole batch in {cpu['oracle']:.1f} s: the C oracle "
                      "(oracle/cm_oracle.c, OpenMP over output rows) for every contraction and unit"}
        result["parity"] = (f"all {shape.batch} sequences' outputs bit-exact vs the CPU simulator algorithm "
                            f"(the whole step in {dt_full:.1f} s); layer 0 bit-exact under both CPU baselines"
                            if ok else "MISMATCH vs the CPU simulator algorithm")
    finish(result, ok)


# ---------------------------------------------------------------- MobileNetV2, batch 32
def conv_macs(sn) -> int:
    return sn.batch * sn.out_ch * sn.out_h * sn.out_w * sn.kh * sn.kw * (1 if sn.is_depthwise else sn.in_ch)


def conv_pointwise(sn) -> bool:
    return (sn.kh == sn.kw == sn.stride_h == sn.stride_w == 1 and sn.pad_top == sn.pad_left == 0
            and (sn.in_h, sn.in_w) == (sn.out_h, sn.out_w))


def conv_on_gemm(sn) -> bool:
    """A convolution the library runs on the plane GEMM (not depthwise, not a few-tap one)."""
    from cormorant_amd import units
    return not sn.is_depthwise and not units.conv_small(sn.in_ch, sn.kh, sn.kw, sn.out_ch, sn.batch)


def matmul_on_skinny(sn) -> bool:
    """A saturating MatMul of a constant weight and at most 32 rows, which the simulator runs as
    saturating skinny products (skinny_planes_kernel, 16 rows a launch)."""
    a, b = sn.inputs
    return (b.data is not None and len(a.shape) == 2 and len(b.shape) == 2 and int(a.shape[-2]) <= 32
            and int(a.shape[-1]) % 8 == 0 and a.exp is None and b.exp is None and b.wexp is None)


def write_conv_roofline(path, g, per_kernel, batch, ms):
    """A markdown table of every convolution and product launch of one forward against its own
    roofline: the GEMM launches (and the fold split before each folded 1x1) against
    max(i8-MFMA time, HBM time) of their algorithmic work and bytes, the few-tap convolutions
    (VALU) against their HBM time.  Algorithmic bytes: each operand once at int16, the output
    once.  The i-th GEMM / fold / few-tap launch is the i-th node of the graph that makes one."""
    gemm = per_kernel.get("gemm_planes_kernel", {}).get("each", [])
    fold = per_kernel.get("split_fold_kernel", {}).get("each", [])
    small = per_kernel.get("conv_small_kernel", {}).get("each", [])
    skinny = per_kernel.get("skinny_planes_kernel", {}).get("each", [])
    gi = fi = si = ki = 0
    rows = []
    for sn in g.nodes:
        kind = type(sn).__name__
        if kind == "ConvNode" and not sn.is_depthwise:
            n = sn.batch * sn.out_h * sn.out_w
            k = sn.in_ch * sn.kh * sn.kw
            byt = 2 * (sn.out_ch * k + sn.batch * sn.in_ch * sn.in_h * sn.in_w + sn.out_ch * n)
            shape = f"{sn.in_ch}x{sn.in_h}x{sn.in_w} -> {sn.out_ch}, {sn.kh}x{sn.kw} s{sn.stride_h}"
            if conv_on_gemm(sn):
                split_us = None
                if conv_pointwise(sn):
                    split_us = fold[fi] * 1e3 if fi < len(fold) else float("nan")
                    fi += 1
                us = gemm[gi] * 1e3 if gi < len(gemm) else float("nan")
                gi += 1
                rows.append((sn.output.onnx_name, shape, "gemm_planes_kernel", us, conv_macs(sn), byt, split_us))
            else:
                us = small[si] * 1e3 if si < len(small) else float("nan")
                si += 1
                rows.append((sn.output.onnx_name, shape, "conv_small_kernel", us, conv_macs(sn), byt, None))
        elif kind == "MatmulNode":
            a, b = sn.inputs
            n, kk, m = int(a.shape[-2]), int(a.shape[-1]), int(b.shape[-1])
            if matmul_on_skinny(sn):
                launches = (n + 15) // 16
                us = sum(skinny[ki:ki + launches]) * 1e3 if ki + launches <= len(skinny) else float("nan")
                ki += launches
                kern = "skinny_planes_kernel" if launches == 1 else f"skinny_planes_kernel x {launches}"
            else:
                us = gemm[gi] * 1e3 if gi < len(gemm) else float("nan")
                gi += 1
                kern = "gemm_planes_kernel"
            rows.append((sn.output.onnx_name, f"{n}x{kk} . {kk}x{m}", kern, us, n * kk * m,
                         2 * (n * kk + kk * m + n * m), None))
    tot_us = tot_bound = 0.0
    lines = [f"| output | shape (batch {batch}) | kernel | us | G MAC | MB | MFMA-bound us | HBM-bound us | "
             "of roofline | fold split us (HBM-bound us) |", "|---|---|---|---|---|---|---|---|---|---|"]
    for name, shape, kern, us, macs, byt, split_us in rows:
        t_mfma = 8.0 * macs / (I8_PEAK_TOPS * 1e12) * 1e6 if kern.startswith(("gemm", "skinny")) else 0.0
        t_hbm = byt / (HBM_PEAK_GBS * 1e9) * 1e6
        bound = max(t_mfma, t_hbm)
        split = ""
        if split_us is not None:
            # the split reads the int16 input and writes its two byte planes (as many bytes)
            s_hbm = 2.0 * sn_bytes_in(g, name) / (HBM_PEAK_GBS * 1e9) * 1e6
            split = f"{split_us:.1f} ({s_hbm:.2f})"
            tot_us += split_us
            tot_bound += s_hbm
        tot_us += us
        tot_bound += bound
        lines.append(f"| {name} | {shape} | {kern} | {us:.1f} | {macs / 1e9:.3f} | {byt / 1e6:.1f} | "
                     f"{t_mfma:.2f} | {t_hbm:.2f} | {bound / us:.2f} | {split} |")
    lines.append(f"\nThese launches, with the fold splits: {tot_us:.1f} us of the {ms * 1e3:.1f} us step; their "
                 f"rooflines sum to {tot_bound:.1f} us ({tot_bound / tot_us:.2f} of their time).")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def sn_bytes_in(g, out_name) -> int:
    """Bytes of the int16 input of the convolution writing ``out_name``."""
    sn = next(n for n in g.nodes if n.output.onnx_name == out_name)
    return 2 * sn.batch * sn.in_ch * sn.in_h * sn.in_w


def mobilenet_bench(args, torch, np):
    """One step = one forward of MobileNetV2 1.0 over 32 images of 3 x 224 x 224 (Q8.8), the
    input resident on the GPU, replayed as a captured HIP graph."""
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator

    batch = 32
    g, inputs, macs = models.mobilenet_v2(batch=batch, seed=args.seed)
    sim = Simulator(g)
    out_name = g.output_tensors[0].onnx_name
    x = sim._to_device(sim._tensor("input"), inputs["input"])
    each = (("gemm_planes_kernel", "split_fold_kernel", "conv_small_kernel", "skinny_planes_kernel")
            if args.per_launch else ())
    ms, per_kernel, out = run_graph(args, torch, sim, {"input": x}, out_name, each=each)
    if args.per_launch:
        write_conv_roofline(args.per_launch, g, per_kernel, batch, ms)
        for k in each:
            per_kernel.get(k, {}).pop("each", None)
    result = {
        "metric": "bit-exact fixed-point images/s (MobileNetV2 batch 32, 224x224, Q8.8)",
        "value": round(batch / (ms * 1e-3), 1),
        "unit": "images/s",
        "gmacs_per_s": round(macs / (ms * 1e-3) / 1e9, 1),
        **step_fields(args, ms),
        "data": f"synthetic (seed {args.seed}): input U[0,1), He-normal weights, every tensor Q8.8 (RNE, saturated)",
        "config": {"workload": "MobileNetV2 1.0 forward, batch 32 x 3 x 224 x 224, 17 inverted residual blocks, "
                               "1x1 320->1280, global average pool, 1280x1000 classifier",
                   "batch": batch, "res": 224, "macs_per_step": macs},
        "kernels_ms_per_step": per_kernel,
    }
    # the GEMM's share of the MACs: the standard / pointwise convolutions it runs (the few-tap
    # convolutions run on the VALU, the classifier on the skinny products)
    off_mfma = sum(conv_macs(sn) for sn in g.nodes if type(sn).__name__ == "ConvNode" and not conv_on_gemm(sn))
    off_mfma += sum(int(sn.inputs[0].shape[-2]) * int(sn.inputs[0].shape[-1]) * int(sn.inputs[1].shape[-1])
                    for sn in g.nodes if type(sn).__name__ == "MatmulNode" and matmul_on_skinny(sn))
    result["roofline"] = gemm_roofline(per_kernel, macs - off_mfma)
    result["roofline"]["macs_on_mfma"] = macs - off_mfma
    ok = None
    if not args.no_cpu_baseline:
        from oracle import graph_sim
        t1 = time.time()
        want = graph_sim.forward(g, inputs)[out_name]
        dt = time.time() - t1
        got = sim._to_values(sim._tensor(out_name), out)
        ok = bool(np.array_equal(got, want.reshape(got.shape)))
        result["cpu_baseline"] = {"value": round(batch / dt, 2), "unit": "images/s", "cores": cores(),
                                  "kind": "port",
                                  "sample": f"the whole step ({batch} images, {macs / 1e9:.2f} G MAC) in {dt:.1f} s: "
                                            "the reference simulator's algorithms restated (float64 per-tap "
                                            "contractions, the C oracle's pooling / VectorOP)"}
        result["parity"] = (f"all {batch} images' logits bit-exact vs the CPU simulator algorithm"
                            if ok else "MISMATCH vs the CPU simulator algorithm")
    finish(result, ok)


# ---------------------------------------------------------------- SmolLM2-360M decode, batch 16
def smollm2_bench(args, torch, np):
    """One step = one greedy decode step of 16 sequences at cache position 1023 (every one of
    the 1024 cache rows a key): 32 layers and the tied head, the residual and the 64 KV caches
    resident on the GPU, replayed as a captured HIP graph (the step's cache row writes
    rewrite the same rows each replay).  Before it (untimed), the prefill entry fills each
    sequence's cache rows 0 .. 1022 from 1023 random token ids: one 1024-row prefill call per
    sequence, writing in place into that sequence's slice of the decode graph's caches."""
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator

    shape = models.LlamaShape()
    t0 = time.time()
    weights = models.smollm2_weights(shape, seed=args.seed)
    g, inputs, exps = models.smollm2_decode(shape, seed=args.seed, weights=weights)
    pg = models.smollm2_prefill(shape, shape.ctx, exps, weights)
    build_s = time.time() - t0
    sim = Simulator(g)
    out_name = g.output_tensors[0].onnx_name
    feeds = {name: sim._to_device(sim._tensor(name), v) for name, v in inputs.items()}
    # the caches prefilled from random token ids (rows 0 .. pos - 1 of every sequence)
    pos = shape.ctx - 1
    sim_p = Simulator(pg, share=sim)
    rng = np.random.default_rng([args.seed, 7])
    h_last = torch.zeros((1, shape.d), dtype=torch.int32, device="cuda")
    caches = [t.onnx_name for t in pg.state_tensors if t.onnx_name != "h_last"]
    torch.cuda.synchronize()
    t1 = time.time()
    for b in range(shape.batch):
        ids = rng.integers(0, shape.vocab, shape.ctx)
        pf = {"ids": sim_p._to_device(sim_p._tensor("ids"), ids.astype(np.float64)), "pos": np.array([0]),
              "n": np.array([pos]), "h_last": h_last}
        pf.update({name: feeds[name].view(shape.batch, -1)[b] for name in caches})
        sim_p.forward_raw(pf, keep=["h_last"] + caches)
    torch.cuda.synchronize()
    prefill_s = time.time() - t1
    sat = sum(int((feeds[name].abs() >= 32767).sum()) for name in caches)
    filled = len(caches) * shape.batch * shape.kv * pos * shape.hd
    for name in caches:                      # the oracle's decode step reads the same caches
        inputs[name] = sim._to_values(sim._tensor(name), feeds[name])
    ms, per_kernel, out = run_graph(args, torch, sim, feeds, out_name)
    macs = shape.macs()
    kv_bytes = shape.layers * 2 * shape.batch * shape.kv * shape.ctx * shape.hd * 2
    step_bytes = shape.weight_bytes() + kv_bytes
    # the linears (7 per layer and the tied head) run as skinny_planes_kernel launches and, for
    # gate / up with the SiLU gate, skinny_mulact_kernel launches; together they read every
    # weight's byte planes once: 2 bytes per weight, the column sums aside
    sk_bytes = shape.weight_bytes()
    sk_ms = sum(per_kernel.get(k, {}).get("ms", 0.0) for k in ("skinny_planes_kernel", "skinny_mulact_kernel"))
    sk_ms = sk_ms or float("nan")
    # the decode attention reads each layer's K and V cache rows once
    da_ms = per_kernel.get("decode_attn_kernel", {}).get("ms", 0.0) or float("nan")
    result = {
        "metric": "bit-exact fixed-point tokens/s (SmolLM2-360M-shaped decode, batch 16, 1024-row KV cache)",
        "value": round(shape.batch / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "gmacs_per_s": round(macs / (ms * 1e-3) / 1e9, 1),
        "step_hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        **step_fields(args, ms),
        "data": f"synthetic (seed {args.seed}): tied embedding and linears N(0,0.02), RMSNorm gammas "
                "1+N(0,0.02), the step's residual = embedding rows of random ids; every sequence's cache "
                "rows 0 .. 1022 written by the prefill entry over 1023 random token ids (untimed); "
                "per-tensor pow2 exponents from a float64 run of sequence 0",
        "prefill": {"entry": f"prefill_{shape.ctx}", "calls": shape.batch, "rows_per_call": pos, "s": round(prefill_s, 3),
                    "tokens_per_s": round(shape.batch * pos / prefill_s, 1),
                    "cache_saturated_frac": round(sat / filled, 6),
                    "note": "eager calls (not graph replays), timed with the host clock around all 16"},
        "config": {"workload": "SmolLM2-360M-shaped greedy decode step: 32 layers, d 960, 15 q / 5 KV heads x "
                               "64, FFN 2560 SiLU-gated, RoPE theta 1e5, tied head 49152, batch 16 sequences "
                               "at position 1023 of a 1024-row KV cache",
                   "layers": shape.layers, "batch": shape.batch, "hidden": shape.d, "heads": shape.heads,
                   "kv_heads": shape.kv, "ffn": shape.ff, "vocab": shape.vocab, "ctx": shape.ctx,
                   "macs_per_step": macs, "weight_bytes": shape.weight_bytes(), "kv_bytes": kv_bytes},
        "roofline": {"bound": "hbm", "achieved": round(sk_bytes / (sk_ms * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(sk_bytes / (sk_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "skinny_planes_kernel", "kernels": ["skinny_planes_kernel", "skinny_mulact_kernel"],
                     "kernel_ms_per_step": sk_ms, "bytes_per_step": sk_bytes,
                     "note": "the linears (7 per layer and the tied head: skinny_planes_kernel and the gate / up "
                             "launches of skinny_mulact_kernel) against their algorithmic bytes: every int16 "
                             "weight once (its two byte planes)"},
        "attention_roofline": {"bound": "hbm", "kernel": "decode_attn_kernel", "kernel_ms_per_step": da_ms,
                               "bytes_per_step": kv_bytes,
                               "achieved": round(kv_bytes / (da_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                               "unit": "GB/s", "frac": round(kv_bytes / (da_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                               "note": "every layer's K and V cache rows once"},
        "kernels_ms_per_step": per_kernel,
        "graph_build_s": round(build_s, 1),
    }
    ok = None
    if not args.no_cpu_baseline:
        from oracle import graph_sim
        t1 = time.time()
        want = graph_sim.forward(g, inputs)[out_name]
        dt = time.time() - t1
        got = sim._to_values(sim._tensor(out_name), out)
        ok = bool(np.array_equal(got, want.reshape(got.shape)))
        result["cpu_baseline"] = {"value": round(shape.batch / dt, 3), "unit": "tokens/s", "cores": cores(),
                                  "kind": "port",
                                  "sample": f"the whole step ({shape.batch} sequences, {macs / 1e9:.2f} GMAC) in "
                                            f"{dt:.1f} s: the reference simulator's algorithms restated (float64 "
                                            "BLAS contractions, the C oracle's row-ops / softmax)"}
        result["parity"] = (f"all {shape.batch} sequences' logits bit-exact vs the CPU simulator algorithm"
                            if ok else "MISMATCH vs the CPU simulator algorithm")
    finish(result, ok)


# ---------------------------------------------------------------- small CNN, batch 1
def cnn_bench(args, torch, np):
    """One step = one forward of the small CNN (batch 1, 28 x 28, Q8.8): latency-bound, so
    the figure is inferences/s of the replayed graph."""
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator

    g, inputs = models.small_cnn(args.seed)
    macs = 290080
    sim = Simulator(g)
    out_name = g.output_tensors[0].onnx_name
    x = sim._to_device(sim._tensor("input"), inputs["input"])
    ms, per_kernel, out = run_graph(args, torch, sim, {"input": x}, out_name)
    result = {
        "metric": "bit-exact fixed-point inferences/s (small CNN, batch 1, Q8.8)",
        "value": round(1.0 / (ms * 1e-3), 1),
        "unit": "inferences/s",
        "us_per_inference": round(ms * 1e3, 2),
        **step_fields(args, ms),
        "data": f"synthetic (seed {args.seed}): input U[0,1), weights U(+-0.25), biases U(+-0.1), Q8.8",
        "config": {"workload": "small CNN forward, batch 1: Conv3x3 1->8 + RELU + MaxPool, Conv3x3 8->16 + RELU "
                               "+ MaxPool, MatMul 784x10 + bias, Softmax", "batch": 1, "macs_per_step": macs},
        "roofline": cnn_roofline(g, per_kernel),
        "kernels_ms_per_step": per_kernel,
    }
    ok = None
    if not args.no_cpu_baseline:
        from oracle import graph_sim
        reps, t1 = 0, time.time()
        while reps == 0 or time.time() - t1 < 10.0:
            want = graph_sim.forward(g, inputs)[out_name]
            reps += 1
        dt = (time.time() - t1) / reps
        got = sim._to_values(sim._tensor(out_name), out)
        ok = bool(np.array_equal(got, want.reshape(got.shape)))
        result["cpu_baseline"] = {"value": round(1.0 / dt, 1), "unit": "inferences/s", "cores": cores(),
                                  "kind": "port",
                                  "sample": f"the whole forward {reps} times in {dt * reps:.1f} s"}
        result["parity"] = ("output bit-exact vs the CPU simulator algorithm"
                            if ok else "MISMATCH vs the CPU simulator algorithm")
    finish(result, ok)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the default warmup outlasts the power controller's first response to the load (the
    # clock dips for some tens of steps, then settles), so the timed steps see its steady state
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--per-launch", default="",
                    help="(--config mobilenet) write a markdown table of every convolution / product launch "
                         "against its roofline to this path")
    ap.add_argument("--hbm", action="store_true",
                    help="measure the HBM-bound units (VectorOP, softmax, pooling, depthwise conv, "
                         "row-ops) against the 8 TB/s roofline instead of the matmul step")
    ap.add_argument("--config", default="bert", choices=["bert", "matmul", "mobilenet", "cnn", "smollm2"],
                    help="bert: the BERT-base L384 encoder forward of 8 sequences (the headline metric); "
                         "matmul: the batched Q8.8 MatMul 4 x 512 x 4096 x 4096; mobilenet: MobileNetV2 "
                         "at batch 32; cnn: the small CNN at batch 1; smollm2: a SmolLM2-360M-shaped "
                         "decode step of 16 sequences")
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
    if args.hbm:
        hbm_kernels(torch, units)
        return
    if args.config == "bert":
        bert_bench(args, torch, np)
        return
    if args.config == "mobilenet":
        mobilenet_bench(args, torch, np)
        return
    if args.config == "cnn":
        cnn_bench(args, torch, np)
        return
    if args.config == "smollm2":
        smollm2_bench(args, torch, np)
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
        "metric": "bit-exact fixed-point GMAC/s (Q8.8 MatMul 4x512x4096x4096) vs CPU simulator",
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
    ok = None
    if not args.no_cpu_baseline:
        gmacs, threads, dt, reps, cref = cpu_baseline(a, b)
        got = dc.cpu().numpy().reshape(BATCH, N, M)
        result["cpu_baseline"] = {"value": round(gmacs, 2), "unit": "GMAC/s", "cores": threads,
                                  "kind": "port",
                                  "sample": f"the whole step ({BATCH}x{N}x{K}x{M}) {reps} times in "
                                            f"{dt:.1f} s: float64 np.matmul + clip/floor as "
                                            "_simulate.py:620-633"}
        ok = bool(np.array_equal(got, cref))
        result["parity"] = ("output bit-exact vs the CPU simulator algorithm"
                            if ok else "MISMATCH vs the CPU simulator algorithm")
    finish(result, ok)


if __name__ == "__main__":
    main()
