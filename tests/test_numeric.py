"""Weight encoding (cormorant_amd.numeric; numeric.py:199-307 of the reference) pinned by what
it must guarantee: every product of an output column on that column's accumulator grid (the
invariant _simulate.py:821-827 checks), the weight within half an LSB of its float value
where it does not saturate, the saturation count, the conv / depthwise / bias exponents, the
errors; and the runtime key count of the prefill attention (llm_nodes.py:960-968)."""
import numpy as np
import pytest

from cormorant_amd.dtype import AP_FIXED_16_8 as DT
from cormorant_amd.graph import ConvNode, MatmulNode, TensorInfo, attn_keys
from cormorant_amd.numeric import NumericError, encode_conv_weights, encode_matmul_weights
from oracle import graph_sim as oracle_graph

F = 8


def _mm(rng, k=48, m=20, t=6, scale=0.3, fa=None, fo=None, name="w"):
    a = TensorInfo("a", [t, k], exp=rng.integers(8, 13, k) if fa is None else fa)
    w = TensorInfo(name, [k, m], data=rng.normal(0, scale, (k, m)))
    c = TensorInfo("c", [t, m], exp=rng.integers(6, 11, m) if fo is None else fo)
    return MatmulNode([a, w], c)


def test_matmul_weights_land_on_the_output_grid():
    rng = np.random.default_rng(1)
    sn = _mm(rng)
    w0 = np.array(sn.inputs[1].data, copy=True)
    sat = encode_matmul_weights([sn], DT)
    a, w, c = sn.inputs[0], sn.inputs[1], sn.output
    fa, fo = np.asarray(a.exp), np.asarray(c.exp)
    assert (fa[:, None] + w.wexp == fo[None, :] + F).all()                  # products on 2^-(f_out + F)
    raw = np.asarray(w.data, np.float64) * 2.0 ** F
    assert np.array_equal(raw, np.round(raw)) and raw.min() >= -32768 and raw.max() <= 32767
    val = raw * 2.0 ** -w.wexp
    ok = np.abs(raw) < 32767
    assert (np.abs(val - w0)[ok] <= 2.0 ** (-w.wexp[ok] - 1)).all()       # round to nearest
    r = np.round(w0 * 2.0 ** w.wexp)
    assert sat["w"] == int(((r < -32768) | (r > 32767)).sum())


def test_matmul_saturation_count():
    rng = np.random.default_rng(2)
    sn = _mm(rng, k=8, m=4, fa=np.full(8, 8), fo=np.full(4, 8))            # wexp = 8: |w| < 128
    w = sn.inputs[1]
    w.data = np.full((8, 4), 0.5)
    w.data[0, 0], w.data[1, 1], w.data[2, 2] = 200.0, -300.0, 32767.5 / 256   # the tie rounds to 32768: saturates
    sat = encode_matmul_weights([sn], DT)
    assert sat["w"] == 3
    raw = np.asarray(w.data) * 256
    assert raw[0, 0] == 32767 and raw[1, 1] == -32768 and raw[2, 2] == 32767


def test_encoded_matmul_simulates_close_to_the_float_product():
    """A sign or index mistake in f_w shows as a large error here."""
    rng = np.random.default_rng(3)
    sn = _mm(rng, k=64, m=16, t=5, scale=0.05)
    w0 = np.array(sn.inputs[1].data, copy=True)
    encode_matmul_weights([sn], DT)
    a, c = sn.inputs[0], sn.output
    x = np.round(rng.normal(0, 1.0, (5, 64)) * 2.0 ** a.exp) / 2.0 ** a.exp
    y = oracle_graph.forward(type("G", (), {"nodes": [sn]})(), {"a": x})["c"]
    exact = x @ w0
    bound = np.abs(x) @ (2.0 ** (-sn.inputs[1].wexp - 1.0)) + 2.0 ** -np.asarray(c.exp, np.float64)[None, :]
    assert (np.abs(y - exact) <= bound + 1e-12).all()


def test_matmul_encoding_errors():
    rng = np.random.default_rng(4)
    sn1, sn2 = _mm(rng), _mm(rng)
    sn2.inputs[1] = sn1.inputs[1]                                           # one weight, two exponent sets
    with pytest.raises(NumericError):
        encode_matmul_weights([sn1, sn2], DT)
    sn = _mm(rng)
    sn.inputs[1].data = None
    with pytest.raises(NumericError):
        encode_matmul_weights([sn], DT)
    sn = _mm(rng)
    sn.inputs[1].exp = 9
    with pytest.raises(NumericError):
        encode_matmul_weights([sn], DT)
    plain = MatmulNode([TensorInfo("a", [2, 4]), TensorInfo("w", [4, 3], data=np.ones((4, 3)))], TensorInfo("c", [2, 3]))
    assert encode_matmul_weights([plain], DT) == {} and plain.inputs[1].wexp is None


def _conv(rng, dw=False, chx=None, chy=None, ex=None, ey=None, bias=True):
    C, M = (6, 6) if dw else (5, 7)
    x = TensorInfo("x", [1, C, 6, 6], exp=ex, chexp=chx)
    w = TensorInfo("w", [M, 1 if dw else C, 3, 3], data=rng.normal(0, 0.2, (M, 1 if dw else C, 3, 3)))
    b = TensorInfo("b", [M], data=rng.normal(0, 0.5, M)) if bias else None
    y = TensorInfo("y", [1, M, 6, 6], exp=ey, chexp=chy)
    return ConvNode([x, w] + ([b] if bias else []), y, pad_top=1, pad_left=1, is_depthwise=dw)


def test_conv_weight_exponents():
    rng = np.random.default_rng(5)
    sn = _conv(rng, ex=10, ey=7)
    encode_conv_weights([sn], DT)
    assert int(sn.inputs[1].wexp) == 7 + F - 10 and int(sn.inputs[2].wexp) == 7
    fx, fy = rng.integers(8, 12, 5), rng.integers(6, 10, 7)
    sn = _conv(rng, chx=fx, chy=fy)
    encode_conv_weights([sn], DT)
    assert np.array_equal(sn.inputs[1].wexp.reshape(7, 5), fy[:, None] + F - fx[None, :])
    assert np.array_equal(sn.inputs[2].wexp, fy)
    fx, fy = rng.integers(8, 12, 6), rng.integers(6, 10, 6)
    sn = _conv(rng, dw=True, chx=fx, chy=fy)
    encode_conv_weights([sn], DT)
    assert np.array_equal(sn.inputs[1].wexp.reshape(6), fy + F - fx)
    plain = _conv(rng)
    assert encode_conv_weights([plain], DT) == {} and plain.inputs[1].wexp is None


def test_attn_keys_known_answers():
    assert attn_keys(0, 5, 8, 64, 16) == (5, 16)
    assert attn_keys(13, 8, 8, 64, 16) == (8, 32)
    assert attn_keys(60, 8, 8, 64, 16) == (4, 64)          # n clamped to the cache
    assert attn_keys(64, 8, 8, 64, 16) == (0, 64)          # pos past the cache: no rows, keys <= C
    assert attn_keys(3, 20, 8, 64, 16) == (8, 16)          # n clamped to T
    assert attn_keys(0, 0, 8, 64, 16) == (0, 16)           # at least one quantum
    assert attn_keys(5, -3, 8, 64, 16) == (0, 16)
