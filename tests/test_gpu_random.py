"""Seeded random parity of every unit against the oracle, beyond the fixtures: full-range
int16 operands (saturation, the int32 wrap of the power-of-two path), all B images, odd
geometries, DIV by zero, masked softmax, every row-ops op; outputs poisoned first so that
a stray or missing write shows."""
import numpy as np
import pytest

from gpu_util import POISON16, dev16, dev8, host, poisoned16
from rowops_cases import RO_CASES, make_job

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def U():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cormorant_amd import units
    units.init()
    return units


def rint16(rng, n, lo=-32768, hi=32768):
    return rng.integers(lo, hi, n).astype(np.int16)


def pack_b(b, k, m):
    mp = (m + 31) // 32 * 32
    p = np.zeros((k, mp), np.int16)
    p[:, :m] = b.reshape(k, m)
    return np.ascontiguousarray(p.reshape(k, mp // 32, 32).transpose(1, 0, 2)).reshape(-1)


def gemv_image(b, k, m, kw):
    """matmul_gemv_index (MatmulKernel.h:148-154)."""
    b = b.reshape(k, m)
    if kw == 1:
        return b.reshape(-1).copy()
    img = np.zeros(k * m, np.int16)
    for kk in range(k):
        c = (kk // (16 * kw)) * 16 + kk % 16
        j = (kk // 16) % kw
        img[(c * m + np.arange(m)) * kw + j] = b[kk]
    return img


MM_CASES = [  # n, k, m, batch, a_bs_mode, b_bs_mode, layout, kw, full_range, wrap
    (1, 1, 1, 1, 1, 1, "row", 0, True, False),
    (37, 300, 70, 1, 1, 1, "row", 0, True, False),
    (37, 300, 70, 1, 1, 1, "row", 0, True, True),
    (130, 520, 200, 3, 1, 0, "packed", 0, False, False),
    (130, 520, 200, 3, 0, 1, "packed", 0, True, True),
    (5, 256, 96, 2, 1, 1, "gemv", 2, False, False),
    (3, 512, 64, 1, 1, 1, "gemv", 4, True, True),
    (2, 256, 40, 2, 1, 0, "gemv", 8, False, False),
    (16, 960, 136, 1, 1, 1, "gemv", 1, False, False),
    (256, 4096, 128, 1, 1, 1, "packed", 0, True, False),
    (200, 13, 333, 2, 1, 1, "row", 0, True, True),
    (9, 8192, 17, 1, 1, 1, "packed", 0, True, False),      # last k of the int32 recombination
    (9, 9000, 17, 1, 1, 1, "packed", 0, True, False),      # int64 recombination
    (3, 32768, 5, 1, 1, 1, "row", 0, True, False),
    (3, 32768, 5, 1, 1, 1, "row", 0, True, True),
    # wrap32 with at most 32 rows: the skinny path (v_dot2 over pairs of k, k split over the grid)
    (1, 960, 960, 1, 1, 1, "packed", 0, True, True),
    (16, 2560, 960, 1, 1, 1, "row", 0, True, True),
    (3, 1024, 64, 80, 1, 1, "row", 0, True, True),
    (32, 4096, 256, 2, 1, 0, "packed", 0, True, True),
    (16, 32768, 64, 1, 1, 1, "row", 0, True, True),
    (5, 2, 32, 1, 1, 1, "packed", 0, True, True),
    (17, 96, 2, 3, 0, 1, "row", 0, True, True),
    (9, 200, 640, 1, 1, 1, "row", 0, False, True),
    # the transposed image [m][k] (b_packed 2): skinny (wrap, <= 32 rows) and plane paths
    (3, 64, 1024, 80, 1, 1, "trans", 0, True, True),
    (16, 960, 320, 2, 1, 0, "trans", 0, True, True),
    (40, 72, 100, 3, 1, 1, "trans", 0, True, True),
    (64, 256, 96, 2, 1, 1, "trans", 0, True, False),
    (7, 100, 33, 1, 1, 1, "trans", 0, False, False),
    (5, 70, 64, 2, 1, 1, "trans", 0, True, True),
    (32, 136, 258, 2, 0, 1, "trans", 0, True, True),
    (2, 8, 2, 1, 1, 1, "trans", 0, True, True),
    # rows of at most 256 k through the short-row split (kp 64 / 128 / 192 / 256), both operands
    (100, 64, 96, 2, 1, 1, "row", 0, True, False),
    (70, 184, 40, 2, 1, 1, "trans", 0, True, True),
    (48, 120, 136, 3, 1, 1, "trans", 0, False, False),
    (33, 256, 64, 2, 1, 0, "row", 0, True, True),
    (130, 192, 72, 1, 1, 1, "trans", 0, True, False),
    # wrap products of few output tiles split over k (int32 partials, the last slice of a tile
    # to arrive adds the others and stores the tile)
    (512, 1024, 256, 1, 1, 1, "row", 0, True, True),
    (300, 2048, 200, 2, 1, 1, "row", 0, True, True),
    (200, 1280, 96, 1, 1, 1, "packed", 0, True, True),
    (64, 4096, 64, 1, 1, 1, "row", 0, True, True),
    (129, 1536, 130, 1, 1, 1, "trans", 0, False, True),
    (96, 1536, 40, 3, 1, 0, "row", 0, True, True),
    # saturating products of few output tiles (one workgroup per tile over all of k):
    # MobileNetV2's classifier at batch 32, ragged tiles, K past 8192 (the int64 recombination)
    (32, 1280, 1000, 1, 1, 1, "packed", 0, True, False),
    (160, 960, 300, 2, 1, 1, "row", 0, True, False),
    (100, 12288, 130, 1, 1, 1, "trans", 0, True, False),
    (70, 600, 33, 3, 1, 0, "row", 0, False, False),
    # wrap products of one slice at sizes past the split over k: BERT's output projection,
    # ragged rows and columns, the packed and transposed images
    (3072, 768, 768, 1, 1, 1, "row", 0, True, True),
    (1024, 2048, 640, 1, 1, 1, "packed", 0, True, True),
    (1000, 1024, 1000, 1, 1, 1, "row", 0, True, True),
    (640, 4096, 1000, 1, 1, 1, "trans", 0, True, True),
]


@pytest.mark.parametrize("k", [1, 8192, 8193, 32768])
@pytest.mark.parametrize("wrap", [False, True])
def test_matmul_extreme_operands(U, oracle_lib, k, wrap):
    """Rows and columns of the int16 extremes: the largest |sum| each recombination path meets."""
    n, m = 4, 6
    a = np.empty((n, k), np.int16)
    a[0], a[1], a[2], a[3] = -32768, 32767, -32768, 32767
    a[3, ::2] = -32768
    b = np.empty((k, m), np.int16)
    b[:, 0], b[:, 1], b[:, 2], b[:, 3], b[:, 4], b[:, 5] = -32768, 32767, -32768, 32767, 1, -1
    b[1::2, 2] = 32767
    b[::3, 5] = 0
    a, b = a.reshape(-1), b.reshape(-1)
    want = oracle_lib.matmul(a, b, n, k, m, 1, 0, 0, n * m, 0, 0, wrap)
    c = poisoned16(n * m + 8)
    U.matmul(dev16(a), dev16(b), c, n, k, m, 1, 0, 0, n * m, 0, 0, wrap)
    got = host(c)
    np.testing.assert_array_equal(got[:n * m], want)
    assert (got[n * m:] == POISON16).all()


@pytest.mark.parametrize("case", MM_CASES, ids=lambda c: "n%d_k%d_m%d_b%d_%s%d_%s" % (
    c[0], c[1], c[2], c[3], c[6], c[7], "wrap" if c[9] else "sat"))
def test_matmul_random(U, oracle_lib, case):
    n, k, m, batch, am, bm, layout, kw, full, wrap = case
    rng = np.random.default_rng(n * 7 + k + m)
    lim = 32768 if full else 2048
    a_bs, b_bs = (n * k if am else 0), (k * m if bm else 0)
    a = rint16(rng, max(batch - 1, 0) * a_bs + n * k, -lim, lim)
    bl = [rint16(rng, k * m, -lim, lim) for _ in range(batch if bm else 1)]
    if layout == "packed":
        imgs = [pack_b(x, k, m) for x in bl]
    elif layout == "gemv":
        imgs = [gemv_image(x, k, m, kw) for x in bl]
    elif layout == "trans":
        imgs = [np.ascontiguousarray(x.reshape(k, m).T).reshape(-1) for x in bl]
    else:
        imgs = bl
    img_len = len(imgs[0])
    b = np.concatenate(imgs)
    b_bs_img = img_len if bm else 0
    bp = {"packed": 1, "trans": 2}.get(layout, 0)
    want = oracle_lib.matmul(a, b, n, k, m, batch, a_bs, b_bs_img, n * m, bp, kw if layout == "gemv" else 0, wrap)
    if layout == "trans":      # the oracle's transposed image against the row-major product
        ref = oracle_lib.matmul(a, np.concatenate(bl), n, k, m, batch, a_bs, k * m if bm else 0, n * m, 0, 0, wrap)
        np.testing.assert_array_equal(want, ref)
    c = poisoned16(batch * n * m + 8)
    U.matmul(dev16(a), dev16(b), c, n, k, m, batch, a_bs, b_bs_img, n * m, bp, kw if layout == "gemv" else 0, wrap)
    got = host(c)
    np.testing.assert_array_equal(got[:batch * n * m], want)
    assert (got[batch * n * m:] == POISON16).all()


@pytest.mark.parametrize("wrap", [True, False])
def test_matmul_split_calls_in_turn(U, oracle_lib, wrap):
    """Products split over k, finished by the last slice of each tile to arrive (its arrival
    count reset for the next call): shapes of different tile and slice counts called in turn,
    each call with new operands, every output against the oracle.  The saturating products of
    the same shapes (and of MobileNetV2's few-tile shapes) run unsplit in turn between them."""
    rng = np.random.default_rng(11)
    shapes = [(300, 2048, 200, 2), (64, 4096, 64, 1), (512, 1024, 256, 1), (300, 2048, 200, 2), (96, 1536, 40, 3)]
    if not wrap:
        shapes += [(32, 1280, 1000, 1), (160, 960, 160, 1), (64, 4096, 64, 1)]
    for rep in range(2):
        for n, k, m, batch in shapes:
            a = rint16(rng, batch * n * k, -32768, 32768)
            b = rint16(rng, batch * k * m, -32768, 32768)
            want = oracle_lib.matmul(a, b, n, k, m, batch, n * k, k * m, n * m, 0, 0, wrap)
            c = poisoned16(batch * n * m + 8)
            U.matmul(dev16(a), dev16(b), c, n, k, m, batch, n * k, k * m, n * m, 0, 0, wrap)
            got = host(c)
            np.testing.assert_array_equal(got[:batch * n * m], want, err_msg=f"rep {rep} shape {(n, k, m, batch)}")
            assert (got[batch * n * m:] == POISON16).all()


@pytest.mark.parametrize("case", [c for c in MM_CASES if c[0] * c[1] * c[2] <= 2 ** 22], ids=lambda c: "n%d_k%d_m%d_b%d_%s%d_%s" % (
    c[0], c[1], c[2], c[3], c[6], c[7], "wrap" if c[9] else "sat"))
def test_matmul_planes_equals_matmul(U, case):
    """B split once (cm_matmul_split_b) then cm_matmul_planes: the same output as cm_matmul,
    shared and per-slice B, every B image, reused for a second A."""
    n, k, m, batch, am, bm, layout, kw, full, wrap = case
    rng = np.random.default_rng(n + k + m + 3)
    lim = 32768 if full else 2048
    a_bs = n * k if am else 0
    bl = [rint16(rng, k * m, -lim, lim) for _ in range(batch if bm else 1)]
    imgs = [pack_b(x, k, m) for x in bl] if layout == "packed" else (
        [gemv_image(x, k, m, kw) for x in bl] if layout == "gemv" else bl)
    b = dev16(np.concatenate(imgs))
    slices = batch if bm else 1
    b_bs = len(imgs[0]) if bm else 0
    planes = U.matmul_b_planes(b, k, m, slices, b_bs, int(layout == "packed"), kw if layout == "gemv" else 0)
    for rep in range(2):
        a = dev16(rint16(rng, max(batch - 1, 0) * a_bs + n * k, -lim, lim))
        want = poisoned16(batch * n * m + 8)
        U.matmul(a, b, want, n, k, m, batch, a_bs, b_bs, n * m, int(layout == "packed"),
                 kw if layout == "gemv" else 0, wrap)
        got = poisoned16(batch * n * m + 8)
        U.matmul_planes(a, planes, got, n, k, m, batch, a_bs, slices, n * m, wrap)
        np.testing.assert_array_equal(host(got), host(want))


STRIDED_CASES = [  # B, T, H, hd, ld, a (col or None), b (col or None), b_trans, c (ldc or None), full, wrap
    (2, 64, 3, 64, 576, 192, 0, True, None, True, True),       # K . q^T from a fused projection
    (2, 64, 3, 64, 576, None, 384, False, 192, True, True),    # P . V into the merged rows
    (1, 384, 2, 64, 384, None, 256, False, 136, False, True),  # 384 keys; o rows wider than the heads
    (3, 40, 2, 24, 160, 16, 112, True, None, True, False),     # ragged rows, saturating
    (2, 72, 1, 32, 48, 8, None, False, 40, True, True),        # one head, padded rows
]


@pytest.mark.parametrize("case", STRIDED_CASES, ids=lambda c: "B%d_T%d_H%d_hd%d_%s_%s_%s" % (
    c[0], c[1], c[2], c[3], "av" if c[5] is not None else "a", ("btv" if c[7] else "bv") if c[6] is not None else "b",
    "cv" if c[8] else "c"))
def test_matmul_strided_random(U, oracle_lib, case):
    """cm_matmul_strided against cm_matmul's oracle on the gathered operands: per-head rows
    read in place from a token-major tensor (A, B and B^T), the output written per head into
    the columns of token-major rows (the columns between left untouched), or plain slices."""
    from cormorant_amd.graph import HeadView
    B, T, H, hd, ld, acol, bcol, btr, ldc, full, wrap = case
    rng = np.random.default_rng(B * 1000 + T * 10 + hd)
    lim = 32768 if full else 2048
    x = rint16(rng, B * T * ld, -lim, lim).reshape(B * T, ld)
    BH = B * H
    # the logical contraction: A [BH][n][k], B [BH][k][m]
    if acol is not None:                       # A = per-head rows of x: n = T, k = hd
        n, k = T, hd
        av = HeadView(acol, H, hd, T)
        a_log, a_src, a_view = av.gather(x), x.reshape(-1), av.strides(ld)
    else:                                      # A = plain [BH][T][T] (probabilities)
        n, k = T, T
        a_log = rint16(rng, BH * T * T, -lim, lim).reshape(BH, T, T)
        a_src, a_view = a_log.reshape(-1), (0, T, H * T * T, T * T)
    if bcol is not None:
        bv = HeadView(bcol, H, hd, T)
        g = bv.gather(x)                       # [BH][T][hd]
        b_log = g.transpose(0, 2, 1) if btr else g
        b_src, b_view = x.reshape(-1), bv.strides(ld)
    else:
        b_log = rint16(rng, BH * k * hd, -lim, lim).reshape(BH, k, hd)
        b_src, b_view = b_log.reshape(-1), (0, hd, H * k * hd, k * hd)
    m = b_log.shape[2]
    assert b_log.shape[1] == k
    want = oracle_lib.matmul(np.ascontiguousarray(a_log).reshape(-1), np.ascontiguousarray(b_log).reshape(-1),
                             n, k, m, BH, n * k, k * m, n * m, 0, 0, wrap).reshape(BH, n, m)
    if ldc is None:
        c_len, c_view = BH * n * m, (0, m, H * n * m, n * m)
        full_want = want.reshape(-1)
    else:
        c_len, c_view = B * T * ldc, (0, ldc, T * ldc, m)
        full_want = np.full(c_len, POISON16, np.int16)
        for bt in range(BH):
            for i in range(n):
                base = (bt // H) * T * ldc + (bt % H) * m + i * ldc
                full_want[base:base + m] = want[bt, i]
    c = poisoned16(c_len + 8)
    U.matmul_strided(dev16(a_src), dev16(b_src), c, n, k, m, BH, H, a_view, b_view, c_view, b_trans=btr, wrap32=wrap)
    got = host(c)
    np.testing.assert_array_equal(got[:c_len], full_want)
    assert (got[c_len:] == POISON16).all()


@pytest.mark.parametrize("n,k,ms,bp", [
    (16, 960, (960, 320, 320), 2),       # SmolLM2's q / k / v
    (16, 960, (2560, 2560), 2),          # gate / up
    (3, 64, (130, 64, 2, 66), 2),        # one k slice (no reduce), ragged column blocks
    (32, 2560, (96, 512), 0),            # row-major B, 40 k slices
    (9, 200, (64, 32, 160), 1),          # packed B
])
def test_matmul_skinny_multi(U, oracle_lib, n, k, ms, bp):
    """cm_matmul_skinny_multi against the oracle's products one by one (and the outputs'
    neighbours untouched): full-range operands, the int32 wrap."""
    rng = np.random.default_rng(n + k + len(ms) + bp)
    a = rint16(rng, n * k)
    bl = [rint16(rng, k * m) for m in ms]
    imgs = [pack_b(x, k, m) if bp == 1 else (np.ascontiguousarray(x.reshape(k, m).T).reshape(-1) if bp == 2 else x)
            for x, m in zip(bl, ms)]
    wants = [oracle_lib.matmul(a, x, n, k, m, 1, 0, 0, n * m, 0, 0, True) for x, m in zip(bl, ms)]
    outs = [poisoned16(n * m + 8) for m in ms]
    U.matmul_skinny_multi(dev16(a), n, k, [dev16(x) for x in imgs], outs, list(ms), b_packed=bp)
    for got, want, m in zip(outs, wants, ms):
        g = host(got)
        np.testing.assert_array_equal(g[:n * m], want)
        assert (g[n * m:] == POISON16).all()


@pytest.mark.parametrize("n,k,ms", [
    (16, 960, (960, 320, 320)),          # SmolLM2's q / k / v
    (16, 960, (2560, 2560)),             # gate / up
    (16, 2560, (960,)),                  # down: 40 k steps over 8 wavefronts
    (16, 960, (49152,)),                 # the tied head
    (1, 8, (1, 33, 64, 7)),              # one k group, ragged columns
    (5, 200, (31, 100)),                 # k past a step, rows short of 16
    (16, 4104, (40,)),                   # several chunks per wavefront, k past a slab
])
def test_matmul_skinny_planes(U, oracle_lib, n, k, ms):
    """cm_matmul_skinny_planes against the oracle's products one by one (the outputs'
    neighbours untouched): full-range operands, the int32 wrap, B from its split image."""
    rng = np.random.default_rng(n + 3 * k + len(ms))
    a = rint16(rng, n * k)
    bl = [rint16(rng, k * m) for m in ms]
    planes = [U.matmul_b_planes(dev16(x), k, m) for x, m in zip(bl, ms)]
    wants = [oracle_lib.matmul(a, x, n, k, m, 1, 0, 0, n * m, 0, 0, True) for x, m in zip(bl, ms)]
    outs = [poisoned16(n * m + 8) for m in ms]
    U.matmul_skinny_planes(dev16(a), n, k, planes, outs, list(ms))
    for got, want, m in zip(outs, wants, ms):
        g = host(got)
        np.testing.assert_array_equal(g[:n * m], want)
        assert (g[n * m:] == POISON16).all()


@pytest.mark.parametrize("n,k,ms,full", [
    (16, 1280, (1000,), False),          # MobileNetV2's classifier, half its batch
    (1, 784, (10,), True),               # a small CNN's classifier
    (16, 960, (2560, 2560), True),       # two products, two blocks a workgroup
    (5, 200, (31, 100), True),           # k past a step, rows short of 16
    (3, 32768, (17,), True),             # the longest k: every limb sum at its bound
    (16, 4104, (40, 600), False),        # several chunks per wavefront, k past a slab
])
def test_matmul_skinny_planes_sat(U, oracle_lib, n, k, ms, full):
    """cm_matmul_skinny_planes_sat against the oracle's saturating products (the outputs'
    neighbours untouched): sums far past int32, B from its split image."""
    rng = np.random.default_rng(n + 5 * k + len(ms))
    lim = 32768 if full else 2048
    a = rint16(rng, n * k, -lim, lim)
    bl = [rint16(rng, k * m, -lim, lim) for m in ms]
    planes = [U.matmul_b_planes(dev16(x), k, m) for x, m in zip(bl, ms)]
    wants = [oracle_lib.matmul(a, x, n, k, m, 1, 0, 0, n * m, 0, 0, False) for x, m in zip(bl, ms)]
    outs = [poisoned16(n * m + 8) for m in ms]
    U.matmul_skinny_planes(dev16(a), n, k, planes, outs, list(ms), wrap32=False)
    for got, want, m in zip(outs, wants, ms):
        g = host(got)
        np.testing.assert_array_equal(g[:n * m], want)
        assert (g[n * m:] == POISON16).all()


def test_matmul_skinny_planes_sat_extremes(U, oracle_lib):
    """Rows and columns of the int16 extremes through the saturating skinny products: the
    largest |sum| (2^30 k) each side of the saturation."""
    n, k = 4, 32768
    a = np.empty((n, k), np.int16)
    a[0], a[1], a[2], a[3] = -32768, 32767, -32768, 32767
    a[3, ::2] = -32768
    b = np.empty((k, 6), np.int16)
    b[:, 0], b[:, 1], b[:, 2], b[:, 3], b[:, 4], b[:, 5] = -32768, 32767, -32768, 32767, 1, -1
    b[1::2, 2] = 32767
    b[::3, 5] = 0
    a, b = a.reshape(-1), b.reshape(-1)
    want = oracle_lib.matmul(a, b, n, k, 6, 1, 0, 0, n * 6, 0, 0, False)
    c = poisoned16(n * 6 + 8)
    U.matmul_skinny_planes(dev16(a), n, k, [U.matmul_b_planes(dev16(b), k, 6)], [c], [6], wrap32=False)
    got = host(c)
    np.testing.assert_array_equal(got[:n * 6], want)
    assert (got[n * 6:] == POISON16).all()


@pytest.mark.parametrize("n,k,m,kind", [
    (16, 960, 960, "resadd"),            # SmolLM2's o projection and residual add (int32 x and out)
    (16, 2560, 960, "resadd"),           # the down projection
    (5, 200, 72, "copy_relu"),           # an int16 COPY with bias, shifts, ReLU (per-column block)
    (1, 8, 24, "scale"),                 # F_SCALE, int16 x, int32 out, broadcast block
])
def test_matmul_skinny_planes_output_job(U, oracle_lib, n, k, m, kind):
    """cm_matmul_skinny_planes_addx equals cm_matmul_skinny_planes followed by the cm_rowops job
    on its output (both outputs), for the residual add and other COPY / ADDX jobs."""
    import torch
    from cormorant_amd import rowops_nodes as rn
    rng = np.random.default_rng(n + k + m)
    a = rint16(rng, n * k)
    b = rint16(rng, k * m)
    planes = U.matmul_b_planes(dev16(b), k, m)
    if kind == "resadd":
        ak, ck = rn.K_I32, rn.K_I32
        blk, bc = rn.pblock(0, 0, 0, rng.integers(0, 10, m), 0, m)
        op = rn.opword(rn.RO_ADDX, ak, rn.K_I16, ck, b_en=True, p_bcast=bc)
        bq_sh = 0
    elif kind == "copy_relu":
        ak, ck = rn.K_I16, rn.K_I16
        blk, bc = rn.pblock(0, rng.integers(-2 ** 21, 2 ** 21, m), rng.integers(0, 4, m), rng.integers(0, 4, m),
                            rng.integers(0, 6, m), m)
        op = rn.opword(rn.RO_ADDX, ak, rn.K_I16, ck, b_en=True, p_bcast=bc, relu=True)
        bq_sh = 3
    else:
        ak, ck = rn.K_I16, rn.K_I32
        blk, bc = rn.pblock(12345, 7, 2, 1, 9, m)
        op = rn.opword(rn.RO_ADDX, ak, rn.K_I16, ck, b_en=True, p_bcast=bc) | U.F_SCALE
        bq_sh = 5
    xb = 2 if ak == rn.K_I16 else 4
    cb = 2 if ck == rn.K_I16 else 4
    x = torch.from_numpy(rng.integers(-2 ** (8 * xb - 2), 2 ** (8 * xb - 2), n * m).astype(np.int16 if xb == 2 else np.int32)).cuda()
    p = torch.from_numpy(np.ascontiguousarray(blk, np.uint8)).cuda()
    c = poisoned16(n * m + 8)
    out = torch.full((n * m * cb + 16,), 0x5A, dtype=torch.uint8, device="cuda")
    U.matmul_skinny_planes_addx(dev16(a), n, k, planes, c, m, x, p, op, out, bq_sh=bq_sh)
    c2 = poisoned16(n * m + 8)
    U.matmul_skinny_planes(dev16(a), n, k, [planes], [c2], [m])
    out2 = torch.full((n * m * cb + 16,), 0x5A, dtype=torch.uint8, device="cuda")
    U.rowops(x.view(torch.uint8), c2.view(torch.uint8), out2, p, op, m, n, 1, m * xb, 0, m * 2, 0, m * cb, 0,
             bq_sh=bq_sh)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(c), host(c2))
    np.testing.assert_array_equal(out.cpu().numpy(), out2.cpu().numpy())
    np.testing.assert_array_equal(host(c2)[:n * m], oracle_lib.matmul(a, b, n, k, m, 1, 0, 0, n * m, 0, 0, True))


@pytest.mark.parametrize("n,k,m,kind", [
    (16, 960, 2560, "silu"),             # SmolLM2's gate / up and its SiLU gate
    (16, 960, 2560, "wide"),             # shifts past the 64-bit bounds (the 128-bit element rule)
    (5, 200, 72, "bcast"),               # rows short of 16, columns short of a block, one entry
    (1, 8, 24, "silu"),                  # one k group
    (16, 4104, 200, "silu"),             # k past four slabs of column sums
    (16, 64, 4096, "silu"),              # the unit's longest row
])
def test_matmul_skinny_planes_mulact(U, oracle_lib, n, k, m, kind):
    """cm_matmul_skinny_planes_mulact equals cm_matmul_skinny_planes of gate and up followed by
    the cm_rowops MULACT job over their outputs (all three outputs, neighbours untouched)."""
    import torch
    from cormorant_amd import rowops_nodes as rn
    rng = np.random.default_rng(7 * n + k + m)
    a = rint16(rng, n * k)
    bg, bu = rint16(rng, k * m), rint16(rng, k * m)
    pg, pu = U.matmul_b_planes(dev16(bg), k, m), U.matmul_b_planes(dev16(bu), k, m)
    if kind == "silu":
        blk, bc = rn.pblock(0, 0, rng.integers(0, 15, m), 0, rng.integers(10, 31, m), m)
    elif kind == "wide":
        blk, bc = rn.pblock(0, 0, rng.integers(15, 41, m), 0, rng.integers(20, 64, m), m)
    else:
        blk, bc = rn.pblock(0, 0, 6, 0, 17, m)
    op = rn.opword(rn.RO_MULACT, b_en=True, p_bcast=bc)
    p = torch.from_numpy(np.ascontiguousarray(blk, np.uint8)).cuda()
    cg, cu, out = poisoned16(n * m + 8), poisoned16(n * m + 8), poisoned16(n * m + 8)
    U.matmul_skinny_planes_mulact(dev16(a), n, k, pg, pu, cg, cu, m, p, op, out)
    cg2, cu2, out2 = poisoned16(n * m + 8), poisoned16(n * m + 8), poisoned16(n * m + 8)
    U.matmul_skinny_planes(dev16(a), n, k, [pg, pu], [cg2, cu2], [m, m])
    U.rowops(cg2.view(torch.uint8), cu2.view(torch.uint8), out2.view(torch.uint8), p, op, m, n, 1, m * 2, 0, m * 2, 0,
             m * 2, 0)
    torch.cuda.synchronize()
    for got, want in ((cg, cg2), (cu, cu2), (out, out2)):
        np.testing.assert_array_equal(host(got), host(want))
    assert (host(out)[n * m:] == POISON16).all()
    np.testing.assert_array_equal(host(cg2)[:n * m], oracle_lib.matmul(a, bg, n, k, m, 1, 0, 0, n * m, 0, 0, True))
    np.testing.assert_array_equal(host(cu2)[:n * m], oracle_lib.matmul(a, bu, n, k, m, 1, 0, 0, n * m, 0, 0, True))


@pytest.mark.parametrize("groups,G,C,mask,regs,lim", [
    (80, 3, 1024, 1024, 2, 3000),        # SmolLM2's step: 16 sequences x 5 groups, every cache row a key
    (10, 3, 1024, 700, 1, 3000),         # keys past the valid count
    (4, 8, 2048, (100 | (3 << 16)), 3, 32768),   # a periodic mask (per-row valid counts), full range
    (7, 1, 64, 0, 0, 32768),             # no valid key: P = 0, o = 0
    (3, 5, 128, 128, 1, 32768),
    (300, 2, 192, 150, 2, 3000),         # more groups than CUs
    (2, 4, 8192, 8000, 1, 3000),         # the longest cache
])
def test_decode_attention(U, oracle_lib, groups, G, C, mask, regs, lim):
    """cm_decode_attention against the oracle's chain per group: s = q K^T (int32 wrap), the
    row-mode softmax (op 10, the softmax row index bg G + i), o = P V."""
    rng = np.random.default_rng(groups + G + C)
    smx_cm, smx_cfg = _attention_regs()[regs]
    q = rng.integers(-lim, lim, (groups, G, 64)).astype(np.int16)
    kc = rng.integers(-lim, lim, (groups, C, 64)).astype(np.int16)
    vc = rng.integers(-32768, 32768, (groups, C, 64)).astype(np.int16)
    s = np.stack([oracle_lib.matmul(q[b].reshape(-1), np.ascontiguousarray(kc[b].T).reshape(-1), G, 64, C, 1, 0, 0,
                                    G * C, 0, 0, True).reshape(G, C) for b in range(groups)])
    p = oracle_lib.vectorop(s.reshape(-1), None, groups * G * C, C, 10, groups * G, C, C, 0, 0, smx_cm, smx_cfg,
                            mask).reshape(groups, G, C)
    want = np.stack([oracle_lib.matmul(p[b].reshape(-1), vc[b].reshape(-1), G, C, 64, 1, 0, 0, G * 64, 0, 0,
                                       True).reshape(G, 64) for b in range(groups)])
    o = poisoned16(groups * G * 64 + 8)
    U.decode_attention(dev16(q.reshape(-1)), dev16(kc.reshape(-1)), dev16(vc.reshape(-1)), o, groups, G, C, smx_cm,
                       smx_cfg, mask)
    got = host(o)
    np.testing.assert_array_equal(got[:groups * G * 64].reshape(groups, G, 64), want)
    assert (got[groups * G * 64:] == POISON16).all()


def _attention_regs():
    from cormorant_amd.graph import softmax_regs
    return [(12102203, 0x0813), softmax_regs(9, 0.125, 15), softmax_regs(12, 0.125, 14), softmax_regs(6, 1.0, 14)]


@pytest.mark.parametrize("B,T,H,regs,lim", [
    (2, 64, 2, 0, 32768),        # full-range q / k / v, the small CNN's register pair
    (1, 128, 3, 1, 32768),       # P at 2^-15: P up to 32767
    (2, 384, 2, 2, 3000),        # BERT-like scores
    (1, 256, 1, 3, 32768),
    (1, 384, 1, 1, 32768),
])
def test_attention_random(U, oracle_lib, B, T, H, regs, lim):
    """cm_attention against the oracle's chain per (sequence, head): s = K . Q^T (int32 wrap,
    keys-major), the keys-major softmax (op 11), o = P . V; Q / K / V at their column offsets
    of wider rows, o into wider merged rows whose other columns stay untouched."""
    cm, cfg = _attention_regs()[regs]
    rng = np.random.default_rng(T * 10 + H + regs)
    hd, D = 64, 64 * H
    ld, o_ld = 3 * D + 8, D + 16
    q_off, k_off, v_off = 8, 8 + D, 8 + 2 * D
    x = rint16(rng, B * T * ld, -lim, lim).reshape(B * T, ld)
    want = np.full((B * T, o_ld), POISON16, np.int16)
    for b in range(B):
        rows = x[b * T:(b + 1) * T]
        for h in range(H):
            Q = rows[:, q_off + hd * h:q_off + hd * (h + 1)]
            K = rows[:, k_off + hd * h:k_off + hd * (h + 1)]
            V = rows[:, v_off + hd * h:v_off + hd * (h + 1)]
            s = oracle_lib.matmul(np.ascontiguousarray(K).ravel(), np.ascontiguousarray(Q.T).ravel(), T, hd, T,
                                  1, 0, 0, T * T, 0, 0, True)
            p = oracle_lib.vectorop(s, None, T * T, T, 11, T, T, T, 0, 0, cm, cfg, T)
            o = oracle_lib.matmul(p, np.ascontiguousarray(V).ravel(), T, T, hd, 1, 0, 0, T * hd, 0, 0, True)
            want[b * T:(b + 1) * T, hd * h:hd * (h + 1)] = o.reshape(T, hd)
    out = poisoned16(B * T * o_ld)
    U.attention(dev16(x.ravel()), out, B, T, H, hd, ld, q_off, k_off, v_off, o_ld, cm, cfg)
    np.testing.assert_array_equal(host(out).reshape(B * T, o_ld), want)


def test_matmul_q88_saturates_where_int32_would_wrap(U, oracle_lib):
    """acc = 16 * 32767^2 exceeds int32: the Q8.8 path saturates the true sum, the
    power-of-two path wraps it (_simulate.py:620-633 vs 814-835; test_numeric.py:148-184)."""
    k = 16
    a = np.full(k, 32767, np.int16)
    b = np.full(k, 32767, np.int16)
    for wrap, expect in ((False, 32767), (True, None)):
        c = poisoned16(8)
        U.matmul(dev16(a), dev16(b), c, 1, k, 1, wrap32=wrap)
        got = int(host(c)[0])
        acc = 16 * 32767 * 32767
        if expect is None:
            w = (acc + 2 ** 31) % 2 ** 32 - 2 ** 31
            expect = max(-32768, min(32767, w >> 8))
        assert got == expect


def test_matmul_c2_shape_against_numpy_float64(U):
    """The C2 workload shape (4 x 512 x 4096 x 4096, shared packed B) against the reference's
    own CPU algorithm (float64 np.matmul + clip/floor), every output."""
    import bench
    from oracle import sim_numpy
    a, b, bp = bench.make_inputs(7)
    c = poisoned16(4 * 512 * 4096)
    U.matmul(dev16(a.reshape(-1)), dev16(bp), c, 512, 4096, 4096, 4, 512 * 4096, 0, 512 * 4096, 1, 0, False)
    np.testing.assert_array_equal(host(c).reshape(4, 512, 4096), sim_numpy.matmul_q88(a, b))


CONV_CASES = [  # batch, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, bias, dwise, full, wrap
    (2, 3, 31, 29, 17, 7, 7, 2, 2, 1, 1, 3, 3, 3, 3, 1, 0, False, False),
    (1, 21, 12, 13, 40, 3, 3, 1, 1, 2, 2, 2, 2, 2, 2, 1, 0, True, False),
    (3, 40, 9, 9, 33, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, True, True),
    (1, 64, 14, 14, 64, 3, 3, 2, 1, 1, 1, 1, 0, 1, 2, 1, 0, False, False),
    (2, 24, 15, 17, 24, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, True, False),
    (1, 16, 20, 20, 16, 5, 5, 2, 2, 1, 1, 2, 2, 2, 2, 0, 1, True, True),
    (32, 3, 16, 16, 32, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 1, 0, False, False),
    # depthwise 3x3 strips: int32 sums (small operands, wrap) and int64 (full range), s1 / s2,
    # asymmetric pads, strips cut by the plane's last rows
    (2, 24, 15, 17, 24, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, False, False),
    (2, 24, 15, 17, 24, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, True, False),
    (3, 8, 9, 33, 8, 3, 3, 1, 1, 1, 1, 0, 2, 1, 0, 1, 1, False, True),
    (3, 8, 9, 33, 8, 3, 3, 1, 1, 1, 1, 0, 2, 1, 0, 1, 1, True, True),
    (1, 32, 56, 56, 32, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, False, False),
    (2, 16, 112, 112, 16, 3, 3, 2, 2, 1, 1, 0, 0, 1, 1, 0, 1, False, False),
    (4, 40, 7, 7, 40, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, False, False),
    # depthwise 3x3 s1 on rows of 8k columns (16-byte words, v_dot2 pairs): left pads 0 / 1 / 2,
    # strips cut by the plane's end, int64 sums (full range) and wrap
    (2, 16, 13, 24, 16, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, False, False),
    (1, 8, 10, 16, 8, 3, 3, 1, 1, 1, 1, 0, 0, 0, 2, 0, 1, False, True),
    (1, 8, 12, 16, 8, 3, 3, 1, 1, 1, 1, 2, 2, 0, 0, 1, 1, True, False),
    (1, 8, 20, 56, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, True, False),
    (2, 8, 9, 32, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, True, True),
    # 1x1 stride 1 unpadded: the images folded into the GEMM's columns (even / odd planes,
    # line groups across images, 1280 rows, two k slabs), and 1x1 convs that do not fold
    (32, 24, 14, 14, 144, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, False, False),
    (5, 96, 7, 7, 160, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, True, False),
    (2, 320, 8, 8, 1280, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, False, True),
    (2, 1100, 4, 6, 40, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, True, False),
    (3, 16, 33, 35, 24, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, False, False),
    (2, 16, 9, 9, 24, 1, 1, 2, 2, 1, 1, 0, 0, 0, 0, 1, 0, False, False),
    (2, 16, 9, 9, 24, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, False, False),
    # folded 1x1 with 2^16 lines and more (the LDS-tiled split): an even and an odd plane (the
    # first two run on the VALU as few-tap convolutions, the other two on the GEMM)
    (4, 24, 128, 128, 40, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, False, False),
    (3, 20, 151, 149, 24, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, True, False),
    (4, 96, 128, 128, 160, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, False, False),
    (3, 100, 151, 149, 130, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, True, False),
    # few taps (at most 16 channels, 80 taps): straight on the VALU -- MobileNetV2's stem, the
    # small CNN's first layer, 7x7 over one channel with asymmetric pads (int64 sums), dilation
    # and wrap with 33 output channels, a wide plane, exactly 80 taps, 64 taps full range wrapped
    (4, 3, 224, 224, 32, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 1, 0, False, False),
    (2, 1, 28, 28, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, False, False),
    (1, 1, 20, 23, 20, 7, 7, 1, 2, 1, 1, 3, 2, 3, 4, 1, 0, True, False),
    (3, 8, 15, 14, 33, 3, 3, 2, 1, 2, 1, 2, 1, 0, 2, 1, 0, False, True),
    (1, 4, 9, 300, 5, 1, 3, 1, 3, 1, 2, 0, 2, 0, 2, 1, 0, True, False),
    (2, 5, 11, 11, 16, 4, 4, 3, 3, 1, 1, 0, 0, 1, 1, 0, 0, False, False),
    (2, 16, 12, 12, 7, 2, 2, 2, 2, 1, 1, 0, 0, 0, 0, 1, 0, True, True),
    # 1x1 over several 16-channel tiles of the packed weights (a last tile of 8 and of 16 lanes)
    (2, 32, 20, 20, 16, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, False, False),
    (3, 40, 9, 10, 50, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, True, False),
    (1, 80, 7, 7, 130, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, True, True),
    (2, 20, 9, 9, 24, 2, 2, 1, 1, 1, 1, 1, 0, 0, 1, 1, 0, False, False),
    # GEMM convolutions of few output tiles and long k: MobileNetV2's 7 x 7 960 -> 160 (folded),
    # 3 x 3 over 128 channels (im2col) at full range, 1100 channels wrapped
    (4, 960, 7, 7, 160, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0, False, False),
    (2, 128, 8, 8, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, True, False),
    (2, 1100, 7, 7, 320, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, True, True),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: "b%d_c%d_%dx%d_m%d_k%dx%d_s%d%d%s%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], c[7], c[8], "_dw" if c[16] else "", "_wrap" if c[18] else ""))
def test_conv_random(U, oracle_lib, case):
    from cormorant_amd.packing import conv_bias_image, conv_weight_image
    (bt, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, has_b, dwise, full, wrap) = case
    rng = np.random.default_rng(C * 31 + M)
    lim = 32768 if full else 1024
    oh = (H + pt + pb - dh * (kh - 1) - 1) // sh + 1
    ow = (W + pl + pr - dw * (kw - 1) - 1) // sw + 1
    x = rint16(rng, bt * C * H * W, -lim, lim)
    w = conv_weight_image(rint16(rng, M * (1 if dwise else C) * kh * kw, -lim, lim).reshape(
        M, 1 if dwise else C, kh, kw), bool(dwise))
    bias = conv_bias_image(rint16(rng, M, -lim, lim))
    want = oracle_lib.conv(x, w, bias if has_b else None, bt * M * oh * ow, bt, C, H, W, M, oh, ow, kh, kw,
                           sh, sw, dh, dw, pt, pl, has_b, dwise, wrap32=wrap)
    y = poisoned16(bt * M * oh * ow + 8)
    U.conv(dev16(x), dev16(w), dev16(bias), y, bt, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, has_b,
           dwise, wrap32=wrap)
    got = host(y)
    np.testing.assert_array_equal(got[:bt * M * oh * ow], want)
    assert (got[bt * M * oh * ow:] == POISON16).all()


@pytest.mark.parametrize("case", [c for c in CONV_CASES if not c[16]], ids=lambda c: "b%d_c%d_%dx%d_m%d_k%dx%d_s%d%d" % (
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], c[7], c[8]))
def test_conv_planes_equals_conv(U, case):
    """Weights split once (cm_conv_split_w) then cm_conv_planes: the same output as cm_conv,
    for two inputs through the same planes."""
    from cormorant_amd.packing import conv_bias_image, conv_weight_image
    (bt, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, has_b, dwise, full, wrap) = case
    rng = np.random.default_rng(C * 17 + M)
    lim = 32768 if full else 1024
    oh = (H + pt + pb - dh * (kh - 1) - 1) // sh + 1
    ow = (W + pl + pr - dw * (kw - 1) - 1) // sw + 1
    w = dev16(conv_weight_image(rint16(rng, M * C * kh * kw, -lim, lim).reshape(M, C, kh, kw), False))
    bias = dev16(conv_bias_image(rint16(rng, M, -lim, lim)))
    planes = U.conv_w_planes(w, M, C, kh, kw)
    for rep in range(2):
        x = dev16(rint16(rng, bt * C * H * W, -lim, lim))
        want = poisoned16(bt * M * oh * ow + 8)
        U.conv(x, w, bias, want, bt, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, has_b, 0, wrap32=wrap)
        got = poisoned16(bt * M * oh * ow + 8)
        U.conv_planes(x, planes, bias, got, bt, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, has_b,
                      wrap32=wrap)
        np.testing.assert_array_equal(host(got), host(want))


@pytest.mark.parametrize("op", range(10))
@pytest.mark.parametrize("act", range(7))
def test_vectorop_all_ops_and_acts(U, oracle_lib, op, act):
    rng = np.random.default_rng(op * 10 + act)
    size, outer = 1000, 3
    a = rint16(rng, size * outer + 8)
    b = rint16(rng, size * outer + 8)
    if op == 3:
        b[::7] = 0                       # DIV by zero: the simulator's +-inf / NaN rules
        a[::14] = 0
    alpha = int(rng.integers(0, 1 << 32))
    a_inc = b_inc = 1000
    c_len = (outer - 1) * 2000 + 1000
    want = np.full(c_len + 8, 0x5A5A, np.int16)
    oracle_lib.vectorop(a, b, c_len + 8, size, op, outer, a_inc, b_inc, act, alpha, c=want)
    c = poisoned16(c_len + 8)
    U.vectorop(dev16(a), dev16(b), c, size, op, outer, a_inc, b_inc, act, alpha)
    np.testing.assert_array_equal(host(c), want)


def test_vectorop_large_and_broadcast(U, oracle_lib):
    rng = np.random.default_rng(11)
    n = 3_000_001
    a, b = rint16(rng, n + 7), rint16(rng, n + 7)
    want = oracle_lib.vectorop(a, b, n + 7, n, 2, act=5)
    c = poisoned16(n + 7)
    U.vectorop(dev16(a), dev16(b), c, n, 2, act=5)
    np.testing.assert_array_equal(host(c), want)
    # b repeats (b_inc 0) over 400 runs of 4096
    a = rint16(rng, 400 * 4096)
    b = rint16(rng, 4096)
    want = oracle_lib.vectorop(a, b, 400 * 4096, 4096, 0, 400, 4096, 0, 1)
    c = poisoned16(400 * 4096)
    U.vectorop(dev16(a), dev16(b), c, 4096, 0, 400, 4096, 0, 1)
    np.testing.assert_array_equal(host(c), want)


@pytest.mark.parametrize("n,rows,mask,cfg", [(384, 40, 384, 0x0813), (2048, 3, 2048, 0x0F0C),
                                             (1, 9, 1, 0x0813), (1000, 17, 37 | (16 << 16), 0x0A11),
                                             (5000, 2, 4000, 0x0813)])
def test_softmax_rows_random(U, oracle_lib, n, rows, mask, cfg):
    rng = np.random.default_rng(n + rows)
    n8 = (n + 7) & ~7
    a = rint16(rng, rows * n8, -3000, 3000)
    want = np.full(rows * n8 + 8, 0x5A5A, np.int16)
    oracle_lib.vectorop(a, None, rows * n8 + 8, n, 10, rows, n8, n8, 0, 0, 12102203, cfg, mask, c=want)
    c = poisoned16(rows * n8 + 8)
    U.vectorop(dev16(a), None, c, n, 10, rows, n8, n8, smx_cm=12102203, smx_cfg=cfg, smx_mask=mask)
    np.testing.assert_array_equal(host(c), want)


@pytest.mark.parametrize("keys,queries,mask", [(384, 384, 384), (1024, 64, 1024), (37, 16, 37),
                                               (96, 50, 1 | (96 << 16)), (200, 48, 100 | (3 << 16))])
def test_softmax_cols_random(U, oracle_lib, keys, queries, mask):
    rng = np.random.default_rng(keys + queries)
    k8 = (keys + 7) & ~7
    a = rint16(rng, keys * queries, -4000, 4000)
    c_len = queries * k8 + 8
    want = np.full(c_len, 0x5A5A, np.int16)
    oracle_lib.vectorop(a, None, c_len, keys, 11, queries, queries, k8, 0, 0, 12102203, 0x0C1A, mask, c=want)
    c = poisoned16(c_len)
    U.vectorop(dev16(a), None, c, keys, 11, queries, queries, k8, smx_cm=12102203, smx_cfg=0x0C1A,
               smx_mask=mask)
    np.testing.assert_array_equal(host(c), want)


@pytest.mark.parametrize("op,size,outer,mask,batch", [
    (11, 384, 384, 384, 5), (11, 1024, 64, 1024, 3), (11, 96, 48, 1 | (96 << 16), 4), (11, 37, 16, 37, 2),
    (10, 384, 96, 384, 6), (10, 2048, 8, 2048, 3), (10, 2056, 5, 2056, 2), (10, 100, 33, 1 | (100 << 16), 4)])
def test_softmax_batched(U, oracle_lib, op, size, outer, mask, batch):
    """cm_softmax over `batch` matrices at strides = one VectorOP softmax call per matrix
    (rows longer than 2048 take the re-reading path)."""
    rng = np.random.default_rng(size * 7 + outer + batch)
    s8 = (size + 7) & ~7
    if op == 11:
        a_inc, c_inc, na, nc = outer, s8, size * outer, (outer & ~15) * s8
    else:
        a_inc, c_inc, na, nc = s8, s8, outer * s8, outer * s8
    a_bs, c_bs = na + 8, nc + 16                     # strided matrices with gaps
    a = rint16(rng, batch * a_bs, -4000, 4000)
    want = np.full(batch * c_bs + 8, 0x5A5A, np.int16)
    for i in range(batch):
        part = np.full(c_bs, 0x5A5A, np.int16)
        oracle_lib.vectorop(a[i * a_bs:i * a_bs + na], None, c_bs, size, op, outer, a_inc, c_inc, 0, 0, 12102203,
                            0x0C1A, mask, c=part)
        want[i * c_bs:(i + 1) * c_bs] = part
    c = poisoned16(batch * c_bs + 8)
    U.softmax(dev16(a), c, size, op, outer, a_inc, c_inc, 12102203, 0x0C1A, mask, batch=batch, a_bs=a_bs, c_bs=c_bs)
    np.testing.assert_array_equal(host(c), want)


# (Cm, cfg): the exponential's scale Cm / 2^Cs decides where e vanishes (dlim, the least
# max - x with (d Cm) >> Cs >= 17 * 4096) and so whether e is tabulated per d (dlim up to
# 16383) or computed from the 4096-entry table: Cm 17410 / 17409 at Cs = 12 put dlim at
# 16383 and 16384; Cm = 0 never decays; Cs = 46 / 47 straddle the host's shortcut for huge
# shifts; f_p = 31 (cfg 0x1Fxx) lets e R 2^(f_p - 40) + 1/2 reach 2^31 before saturating.
SMX_PARAMS = [(12102203, 0x0813), (0, 0x0813), (1, 0x0000), (0xFFFFFF, 0x0F00), (0xFFFFFF, 0x003F),
              (17410, 0x0F0C), (17409, 0x0F0C), (3, 0x1F2E), (3, 0x1F2F), (12102203, 0x1F13)]


def _smx_scores(rng, n):
    a = rint16(rng, n)
    a[: n // 7] = rng.choice(np.array([-32768, 32767, 0, -1], np.int16), n // 7)
    return a


@pytest.mark.parametrize("cm,cfg", SMX_PARAMS)
@pytest.mark.parametrize("n", [1, 129, 384, 1000, 1025])
def test_softmax_rows_params(U, oracle_lib, cm, cfg, n):
    """Row mode over the exponential's parameter range and every row length form (1..8
    words per lane of a 16-lane row, and the three-pass form past 1024), full-range scores
    (max - x up to 65535), one row of equal scores, a causal valid count."""
    rows, n8 = 37, (n + 7) & ~7
    rng = np.random.default_rng(cm + cfg + n)
    a = _smx_scores(rng, rows * n8)
    a[:n8] = -32768
    for mask in (n, 1 | (min(n, 40) << 16)):
        want = np.full(rows * n8 + 8, 0x5A5A, np.int16)
        oracle_lib.vectorop(a, None, rows * n8 + 8, n, 10, rows, n8, n8, 0, 0, cm, cfg, mask, c=want)
        c = poisoned16(rows * n8 + 8)
        U.vectorop(dev16(a), None, c, n, 10, rows, n8, n8, smx_cm=cm, smx_cfg=cfg, smx_mask=mask)
        np.testing.assert_array_equal(host(c), want, err_msg=f"mask {mask:#x}")


@pytest.mark.parametrize("cm,cfg", SMX_PARAMS)
@pytest.mark.parametrize("keys,queries", [(37, 48), (384, 80), (1024, 64)])
def test_softmax_cols_params(U, oracle_lib, cm, cfg, keys, queries):
    """Column mode over the same parameters; 1024 keys with the largest tabulated e leaves
    room in LDS for narrower query tiles only."""
    rng = np.random.default_rng(cm + cfg + keys)
    k8 = (keys + 7) & ~7
    a = _smx_scores(rng, keys * queries)
    c_len = queries * k8 + 8
    for mask in (keys, 3 | (min(keys, 20) << 16)):
        want = np.full(c_len, 0x5A5A, np.int16)
        oracle_lib.vectorop(a, None, c_len, keys, 11, queries, queries, k8, 0, 0, cm, cfg, mask, c=want)
        c = poisoned16(c_len)
        U.vectorop(dev16(a), None, c, keys, 11, queries, queries, k8, smx_cm=cm, smx_cfg=cfg, smx_mask=mask)
        np.testing.assert_array_equal(host(c), want, err_msg=f"mask {mask:#x}")


POOL_CASES = [  # N, C, H, W, ph, pw, sh, sw, pt, pl, pb, pr, dh, dw, type, lp, cip
    (2, 5, 17, 19, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 0, 2, 0),
    (1, 7, 13, 11, 3, 2, 1, 2, 1, 0, 1, 1, 2, 1, 1, 2, 0),
    (1, 7, 13, 11, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 1, 2, 1),
    (2, 3, 9, 9, 2, 2, 2, 2, 0, 0, 0, 0, 1, 1, 2, 1, 0),
    (2, 3, 9, 9, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 2, 2, 0),
    (32, 64, 7, 7, 7, 7, 1, 1, 0, 0, 0, 0, 1, 1, 1, 2, 0),
    (4, 32, 6, 6, 6, 6, 1, 1, 0, 0, 0, 0, 1, 1, 0, 2, 0),
    (3, 16, 5, 5, 5, 5, 1, 1, 0, 0, 0, 0, 1, 1, 2, 2, 0),
    (2, 7, 9, 9, 9, 9, 1, 1, 0, 0, 0, 0, 1, 1, 1, 2, 0),       # global, plane above 64
    # MAX / AVG 2x2 s2 on rows of 16k columns (16-byte words); odd heights drop the last row
    (2, 5, 8, 32, 2, 2, 2, 2, 0, 0, 0, 0, 1, 1, 0, 2, 0),
    (2, 5, 9, 32, 2, 2, 2, 2, 0, 0, 0, 0, 1, 1, 1, 2, 1),
    (1, 3, 16, 112, 2, 2, 2, 2, 0, 0, 0, 0, 1, 1, 1, 2, 0),
    (1, 3, 16, 112, 2, 2, 2, 2, 0, 0, 0, 0, 1, 1, 0, 2, 0),
]


@pytest.mark.parametrize("case", POOL_CASES)
def test_pool_random(U, oracle_lib, case):
    N, C, H, W, ph, pw, sh, sw, pt, pl, pb, pr, dh, dw, typ, lp, cip = case
    rng = np.random.default_rng(H * W + typ)
    oh = (H + pt + pb - dh * (ph - 1) - 1) // sh + 1
    ow = (W + pl + pr - dw * (pw - 1) - 1) // sw + 1
    x = rint16(rng, N * C * H * W)
    want = oracle_lib.pool(x, N, C, H, W, oh, ow, ph, pw, sh, sw, pt, pl, dh, dw, typ, lp, cip)
    y = poisoned16(N * C * oh * ow + 8)
    U.pool(dev16(x), y, N, C, H, W, oh, ow, ph, pw, sh, sw, pt, pl, dh, dw, typ, lp, cip)
    got = host(y)
    np.testing.assert_array_equal(got[:N * C * oh * ow], want)
    assert (got[N * C * oh * ow:] == POISON16).all()


@pytest.mark.parametrize("n,rows,ln,bcast,lim,bq_sh", [
    (768, 37, True, False, 1 << 20, 12),       # BERT's residual add + LayerNorm32
    (768, 3100, True, False, 1 << 20, 12),     # BERT's rows and more: twelve wavefronts per workgroup
    (960, 9, False, False, 1 << 20, 0),        # SmolLM2's residual add + RMSNorm
    (64, 70, True, True, 1 << 30, 40),         # broadcast parameters, values past the 64-bit bounds
    (4096, 3, True, False, 1 << 24, 20),
    (256, 5, True, False, 1 << 16, 45),        # bq_sh past 40: the NORM's general kernel
])
def test_rowops_addx_norm_jobs(U, oracle_lib, n, rows, ln, bcast, lim, bq_sh):
    """An ADDX job (int32 + int16 -> int32) and the NORM of its output as one job list
    (rowops_jobs, cm_rowops_chain) against the oracle running the two jobs in turn: both
    outputs, and the parameter RAM a later P_KEEP job reads."""
    from rowops_cases import _params
    rng = np.random.default_rng(n + rows + bq_sh)
    a = rng.integers(-lim, lim, n * rows).astype(np.int32).view(np.uint8)
    b = rng.integers(-32768, 32768, n * rows).astype(np.int16).view(np.uint8)
    ent = 1 if bcast else n
    pa = _params(rng, ent, sh=(0, 20), sb=(0, 20), sc=(0, 30))
    pn = _params(rng, ent, g_lo=-(1 << 20), g_hi=1 << 20, sc=(20, 50))
    op_a = 2 | (1 << 4) | (1 << 8) | (1 << 12) | ((1 << 13) if bcast else 0)
    op_n = 5 | (1 << 4) | ((1 << 16) if ln else 0) | ((1 << 13) if bcast else 0)
    eps = int(rng.integers(0, 1 << 20))
    h_want = np.full(4 * n * rows, 0xDE, np.uint8)
    x_want = np.full(2 * n * rows, 0xDE, np.uint8)
    k_want = np.full(2 * n * rows, 0xDE, np.uint8)
    oracle_lib.rowops_reset_params()
    oracle_lib.rowops(a, b, h_want, pa, op_a, n, rows, 1, 4 * n, 0, 2 * n, 0, 4 * n, 0, 0, 0, 0)
    oracle_lib.rowops(h_want, None, x_want, pn, op_n, n, rows, 1, 4 * n, 0, 0, 0, 2 * n, 0, eps, 0, bq_sh)
    decoy = _params(rng, ent)              # what a P_KEEP job must not read
    oracle_lib.rowops(h_want, None, k_want, decoy, op_n | (1 << 14), n, rows, 1, 4 * n, 0, 0, 0, 2 * n, 0, eps, 0,
                      bq_sh)
    ad, bd, pad, pnd = dev8(a), dev8(b), dev8(pa), dev8(pn)
    hd, xd, kd = (dev8(np.full(m, 0xDE, np.uint8)) for m in (4 * n * rows, 2 * n * rows, 2 * n * rows))
    common = dict(c1=rows, c2=1, a_s2=0, b_s2=0, c_s2=0, aux=0, win_lo=0, win_hi=0xFFFFFFFF)
    U.rowops_jobs([dict(a=ad, b=bd, c=hd, p=pad, op=op_a, n=n, a_s1=4 * n, b_s1=2 * n, c_s1=4 * n, eps=0,
                        bq_sh=0, **common),
                   dict(a=hd, b=None, c=xd, p=pnd, op=op_n, n=n, a_s1=4 * n, b_s1=0, c_s1=2 * n, eps=eps,
                        bq_sh=bq_sh, **common)])
    U.rowops(hd, None, kd, dev8(decoy), op_n | (1 << 14), n, rows, 1, 4 * n, 0, 0, 0, 2 * n, 0, eps, 0, bq_sh)
    np.testing.assert_array_equal(host(hd), h_want)
    np.testing.assert_array_equal(host(xd), x_want)
    np.testing.assert_array_equal(host(kd), k_want)


@pytest.mark.parametrize("case", RO_CASES, ids=lambda c: c[0])
def test_rowops_random(U, oracle_lib, case):
    a, b, p, c_len, r = make_job(case)
    want = np.full(c_len, 0xDE, np.uint8)
    oracle_lib.rowops_reset_params()
    oracle_lib.rowops(a, b, want, p, r["op"], r["n"], r["c1"], r["c2"], r["a_s1"], r["a_s2"], r["b_s1"],
                      r["b_s2"], r["c_s1"], r["c_s2"], r["eps"], r["aux"], r["bq_sh"])
    cd = dev8(np.full(c_len, 0xDE, np.uint8))
    U.rowops(dev8(a), dev8(b), cd, dev8(p), r["op"], r["n"], r["c1"], r["c2"], r["a_s1"], r["a_s2"], r["b_s1"],
             r["b_s2"], r["c_s1"], r["c_s2"], r["eps"], r["aux"], r["bq_sh"])
    np.testing.assert_array_equal(host(cd), want)


def test_table_init_round_trip(U, oracle_lib):
    """cm_act_table_init / cm_rowops_tables_init: the library's own tables in give the same
    results; a changed SiLU entry shows in the VectorOP output; a table without the unit's
    form is refused and leaves the tables as they were."""
    full = np.stack([U.host_act_table(a) for a in (4, 5, 6)])
    img = U.host_rowops_table_image()
    x = np.arange(-2048, 2048, dtype=np.int16)
    def silu(xs):                                      # ADD of zeros with the SiLU act register
        c = poisoned16(len(xs) + 8)
        U.vectorop(dev16(xs), dev16(np.zeros(len(xs), np.int16)), c, len(xs), U.OP_ADD, act=4)
        return host(c)[:len(xs)]
    before = silu(x)
    try:
        U.act_table_init(full)
        U.rowops_tables_init(img)
        np.testing.assert_array_equal(silu(x), before)
        changed = full.copy()
        d1 = -int(changed[0][32768 - 1])                  # SiLU(-1) = -d[1], SiLU(1) = 1 - d[1]
        d1n = d1 + 1 if d1 < 255 else d1 - 1
        changed[0][32768 - 1], changed[0][32768 + 1] = -d1n, 1 - d1n
        U.act_table_init(changed)
        got = silu(x)
        want = before.copy()
        want[2048 - 1], want[2048 + 1] = -d1n, 1 - d1n
        np.testing.assert_array_equal(got, want)
        bad = full.copy()
        bad[1][32768 - 5] = 3                             # GELU(-5) = +3: no byte d[5]
        with pytest.raises(ValueError):
            U.act_table_init(bad)
        np.testing.assert_array_equal(silu(x), got)       # unchanged by the refused call
        U.act_table_init(full)
    finally:                                         # the library's own tables for every later test
        U.act_table_init(full)
        U.rowops_tables_init(img)
    np.testing.assert_array_equal(silu(x), before)


def test_rowops_table_entry_reaches_norm(U, monkeypatch):
    """A changed rsqrt entry installed by cm_rowops_tables_init shows in a NORM's output: RMSNorm
    rows whose D falls on the changed entry take it (exactly the reference algorithm with that
    table: oracle/sim_ref.rms_norm over the patched table), the other rows do not change, and the
    library's own image restores the results."""
    from oracle import rowops_adapt as ra
    from oracle import sim_ref
    rng = np.random.default_rng(44)
    n, rows, f_h, f_out = 64, 12, 15, 11
    h = rng.integers(-2 ** 20, 2 ** 20, (rows, n)).astype(np.int64)
    gamma = 1.0 + 0.05 * rng.standard_normal(n)
    G, g, _b, E = ra.norm_params(gamma, n, 1e-5, f_h, rms=True)

    def index(D):
        d = D.bit_length() - 32
        d += d & 1
        return (D >> d if d >= 0 else D << -d) >> 19

    idx = [index(int((h[r] * h[r]).sum()) + E) for r in range(rows)]
    target = idx[0]
    img = U.host_rowops_table_image()
    changed = img.copy()
    words = changed[32768:].view(np.uint32)
    words[target] = words[target] - (1 << 26)      # a 1.5 % error in the Newton step's start
    table = sim_ref._rsqrt_table()
    patched = list(table)
    patched[target] = int(words[target])
    op = U.RO_NORM | (U.K_I32 << 4) | (U.K_I16 << 8)
    p = dev8(ra._params(n, G, 0, 0, 0, ra.P1_BITS + g - f_out))

    def norm_rows():
        c = dev8(np.full(rows * n * 2, 0xDE, np.uint8))
        U.rowops(dev8(h.astype(np.int32).view(np.uint8).reshape(-1)), None, c, p, op, n, rows, 1, 4 * n, 0, 0, 0,
                 2 * n, 0, E, 0, 0)
        return host(c).view(np.int16).reshape(rows, n).astype(np.int64)

    want_default = sim_ref.rms_norm(h, f_h, gamma, 1e-5, f_out)
    monkeypatch.setattr(sim_ref, "_rsqrt_table", lambda: patched)
    want_changed = sim_ref.rms_norm(h, f_h, gamma, 1e-5, f_out)
    monkeypatch.undo()
    hit = np.array([i == target for i in idx])
    assert (want_changed[hit] != want_default[hit]).any() and (want_changed[~hit] == want_default[~hit]).all()
    np.testing.assert_array_equal(norm_rows(), want_default)
    try:
        U.rowops_tables_init(changed)
        np.testing.assert_array_equal(norm_rows(), want_changed)
    finally:
        U.rowops_tables_init(img)
    np.testing.assert_array_equal(norm_rows(), want_default)
