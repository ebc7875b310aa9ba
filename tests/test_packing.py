"""The host-side weight images (cormorant_amd.packing) against the reference's fixture images."""
import numpy as np

from cormorant_amd.packing import conv_bias_image, conv_weight_image, pack_matmul_b
from golden_io import CONV_COLS, MM_COLS, arr, cases


def test_pack_matmul_b_matches_the_packed_fixtures():
    """Packed and row-major fixtures of the same shape pair up through pack_matmul_b."""
    n_checked = 0
    for t in cases("matmul", MM_COLS):
        if not t["b_packed"] or t["batch"] != 1:
            continue
        k, m = t["k"], t["m"]
        bp = arr("matmul", t["idx"], "b")
        mp = (m + 31) // 32 * 32
        logical = bp[:(mp // 32) * k * 32].reshape(mp // 32, k, 32).transpose(1, 0, 2).reshape(k, mp)[:, :m]
        np.testing.assert_array_equal(pack_matmul_b(logical), bp[:len(pack_matmul_b(logical))])
        n_checked += 1
    assert n_checked >= 6


def _unpack_conv(w, M, C, kh, kw, dwise):
    if dwise:
        stride = (kh * kw + 7) & ~7
        return w[:M * stride].reshape(M, stride)[:, :kh * kw].reshape(M, 1, kh, kw)
    tiles = (C + 15) // 16
    rem = C - (tiles - 1) * 16
    last = 8 if rem <= 8 else 16
    per_m = kh * kw * ((tiles - 1) * 16 + last)
    W = w[:M * per_m].reshape(M, per_m)
    out = np.zeros((M, C, kh, kw), np.int16)
    for c in range(C):
        tt, lane = divmod(c, 16)
        lanes = last if tt + 1 == tiles else 16
        for a in range(kh):
            for b in range(kw):
                out[:, c, a, b] = W[:, tt * kh * kw * 16 + (a * kw + b) * lanes + lane]
    return out


def test_conv_weight_image_round_trips_every_fixture():
    for t in cases("conv", CONV_COLS):
        w = arr("conv", t["idx"], "w")
        M, C, kh, kw, dw = t["out_ch"], t["in_ch"], t["kh"], t["kw"], bool(t["is_depthwise"])
        img = conv_weight_image(_unpack_conv(w, M, C, kh, kw, dw), dw)
        assert len(img) == len(w), t["label"]
        np.testing.assert_array_equal(img, w, err_msg=t["label"])
        if t["has_bias"]:
            b = arr("conv", t["idx"], "b")
            np.testing.assert_array_equal(conv_bias_image(b[:M]), b[:len(conv_bias_image(b[:M]))])
