"""Seeded random row-ops jobs (byte images + registers) shared by the GPU parity test and
the oracle-vs-reference-oracle test."""
import numpy as np

def _params(rng, n, g_lo=0, g_hi=1 << 31, bq=1 << 21, sh=(0, 63), sb=(0, 63), sc=(0, 63)):
    p = np.zeros((n, 16), np.uint8)
    p[:, 0:4] = rng.integers(g_lo, g_hi, n).astype(np.int64).astype(np.uint32).view(np.uint8).reshape(n, 4)
    p[:, 4:8] = rng.integers(-bq, bq, n).astype(np.int32).view(np.uint8).reshape(n, 4)
    p[:, 8] = rng.integers(sh[0], sh[1] + 1, n)
    p[:, 9] = rng.integers(sb[0], sb[1] + 1, n)
    p[:, 10] = rng.integers(sc[0], sc[1] + 1, n)
    return p.reshape(-1)


RO_CASES = [  # label, op word, n, rows, blocks, kinds (a, b, c bytes), param ranges, aux, eps, bq_sh
    ("copy_i16", 1 | (1 << 12), 300, 5, 2),
    ("addx_i32_i16_i32", 2 | (1 << 4) | (1 << 8) | (1 << 12), 768, 6, 1),
    ("addx_relu_bcast", 2 | (1 << 12) | (1 << 13) | (1 << 15), 100, 4, 3),
    ("copy_scale", 1 | (1 << 17), 257, 3, 1),
    ("dequant_i32", 3 | (1 << 4) | (2 << 8), 333, 4, 1),
    ("mulact", 4 | (1 << 12), 2560, 3, 1),
    ("gate", 10 | (1 << 12), 500, 3, 1),
    ("norm_rms_i32", 5 | (1 << 4), 960, 5, 1),
    ("norm_ln_i16", 5 | (1 << 16), 768, 7, 1),
    ("norm_ln_i32_4096", 5 | (1 << 4) | (1 << 16), 4096, 2, 1),
    ("rope_hd64", 6 | (2 << 6), 320, 4, 1),
    # rows of whole 8-element units (the 16-byte kernels): COPY from int32, ADDX with an int32 B,
    # the scale flag (128-bit path), broadcast parameters with relu, LN / RMS over 8 .. 2048 lanes
    ("copy_i32_i16_u8", 1 | (1 << 4) | (1 << 12), 256, 3, 2),
    ("addx_i16_i32_i32_u8", 2 | (1 << 6) | (1 << 8) | (1 << 12), 512, 4, 2),
    ("copy_scale_u8", 1 | (1 << 17), 264, 3, 1),
    ("addx_relu_bcast_u8", 2 | (1 << 12) | (1 << 13) | (1 << 15), 104, 4, 3),
    ("norm_ln_i16_64", 5 | (1 << 16), 64, 9, 1),
    ("norm_rms_i16_2048", 5, 2048, 3, 1),
    # rows past 1024 elements over more rows than compute units: the workgroup-per-row kernel
    # taking rows in turn
    ("norm_ln_i32_4096_rows", 5 | (1 << 4) | (1 << 16), 4096, 150, 3),
    ("norm_rms_i16_1536_rows", 5, 1536, 400, 2),
    # broadcast parameters on the workgroup-per-row kernel, one and two units a lane: each lane
    # decodes the one entry it reads
    ("norm_ln_i32_4096_bcast", 5 | (1 << 4) | (1 << 13) | (1 << 16), 4096, 3, 2),
    ("norm_rms_i16_2560_bcast", 5 | (1 << 13), 2560, 5, 1),
    ("norm_rms_i32_1280_bcast", 5 | (1 << 4) | (1 << 13), 1280, 7, 1),
    # two units a lane over at least twelve rows per compute unit (3072 on 256): a workgroup of
    # twelve wavefronts per compute unit
    ("norm_ln_i32_768_many_rows", 5 | (1 << 4) | (1 << 16), 768, 1031, 3),
    ("norm_rms_i16_1000_many_rows", 5, 1000, 3100, 1),
    # the 16-byte unit kernel of DEQUANT / MULACT / GATE / ROPE: shifts on both sides of its 64-bit
    # bounds (sa, sb <= 23, sc <= 61), extreme int16 operands, RoPE tables past 2^23
    ("dequant_i16_u8", 3 | (2 << 8), 512, 4, 2),
    ("mulact_u8", 4 | (1 << 12), 2560, 3, 2),
    ("mulact_u8_wide", 4 | (1 << 12), 512, 4, 1),
    ("gate_u8", 10 | (1 << 12), 512, 3, 2),
    ("rope_hd64_u8", 6 | (1 << 6), 320, 4, 2),
    ("rope_hd32_u8_wide", 6 | (1 << 6), 256, 3, 1),
]

# parameter / operand ranges of the cases above that differ from their op's defaults
_WIDE = {"dequant_i16_u8": dict(sc=(0, 63)), "mulact_u8_wide": dict(sh=(15, 40), sc=(20, 63)),
         "gate_u8": dict(sh=(0, 30), sb=(0, 30), sc=(20, 63)), "rope_hd32_u8_wide": dict(sh=(18, 30), sb=(18, 30), sc=(20, 63))}




def make_job(case):
    """(a, b, p, c_len, regs) of one random job; regs = the register values after the images."""
    label, op, n, c1, c2 = case
    rng = np.random.default_rng(len(label) * 1000 + n)
    code = op & 15
    ak, bk, ck = (op >> 4) & 3, (op >> 6) & 3, (op >> 8) & 3
    kb = lambda kd: 2 if kd == 0 else 4
    if code == 3:
        ck = 2
    a_s1 = (kb(ak) * n + 15) & ~15
    b_s1 = (8 * 64 + 15) & ~15 if code == 6 else (kb(bk) * n + 15) & ~15
    c_s1 = ((kb(ck) * n + 15) & ~15) + 16
    a_s2, b_s2, c_s2 = a_s1 * c1 + 32, b_s1 * c1 + 16, c_s1 * c1 + 48
    lim_a = 1 << 20 if ak == 1 else 1 << 15
    a = np.zeros(a_s2 * c2, np.uint8)
    b = np.zeros(b_s2 * c2, np.uint8)
    for i2 in range(c2):
        for i1 in range(c1):
            off = i2 * a_s2 + i1 * a_s1
            vals = rng.integers(-lim_a, lim_a, n).astype(np.int16 if ak == 0 else np.int32)
            if label.endswith("_u8") or "_u8_" in label:
                vals[:2] = [-lim_a, lim_a - 1]
            a[off:off + kb(ak) * n] = vals.view(np.uint8)
            boff = i2 * b_s2 + i1 * b_s1
            if code == 6:
                tb = 1 << 25 if "wide" in label else 1 << 23
                cs = rng.integers(-tb, tb, 128).astype(np.int32)
                cs[:4] = [1 << 23, -(1 << 23), tb - 1, -tb]
                b[boff:boff + 512] = cs.view(np.uint8)
            else:
                bv = rng.integers(-32768, 32768, n).astype(np.int16 if bk == 0 else np.int32)
                b[boff:boff + kb(bk) * n] = bv.view(np.uint8)
    eps, aux, bq_sh = 0, 0, 0
    if code == 5:
        p = _params(rng, n, 1 << 29, 1 << 31, 1 << 20, sc=(30, 45))
        eps, bq_sh = int(rng.integers(0, 1 << 20)), 20
    elif code == 6:
        aux = 32 if "hd32" in label else 64
        p = _params(rng, n, **_WIDE.get(label, dict(sh=(0, 2), sb=(0, 2), sc=(20, 26))))
    elif code == 4:
        p = _params(rng, n, **_WIDE.get(label, dict(sh=(0, 6), sc=(14, 30))))
    elif code == 10:
        p = _params(rng, n, **_WIDE.get(label, dict(sh=(0, 5), sb=(0, 5), sc=(30, 40))))
    elif code == 3:
        p = _params(rng, n, **_WIDE.get(label, dict(sc=(0, 30))))
    elif op & (1 << 17):
        p = _params(rng, n, 0, 1 << 25, 1 << 10, sh=(0, 4), sb=(0, 4), sc=(10, 30))
    else:
        p = _params(rng, n, sh=(0, 12), sb=(0, 12), sc=(0, 16))
        bq_sh = 3
    regs = dict(op=op, n=n, c1=c1, c2=c2, a_s1=a_s1, a_s2=a_s2, b_s1=b_s1, b_s2=b_s2, c_s1=c_s1,
                c_s2=c_s2, eps=eps, aux=aux, bq_sh=bq_sh)
    return a, b, p, c_s2 * c2, regs
