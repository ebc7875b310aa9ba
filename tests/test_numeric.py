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


# ---------------------------------------------------------------- annotations, checks, fusion
def test_annotations_parse_apply_round_trip():
    from cormorant_amd.dtype import AP_FIXED_16_8
    from cormorant_amd.graph import TensorInfo as T
    from cormorant_amd.numeric import apply, empty, is_active, parse, to_metadata
    meta = parse('{"version": 1, "exp": {"q": 11, "k": [9, 10, 11, 12]}, "host": {"h": "f32", "pos": "i32"}, '
                 '"state": ["kc"], "layout": {"kc": [2, 8]}, "dma": {"r": "i32"}, "engine": {"q": "conv"}}')
    assert is_active(meta) and not is_active(empty())
    assert parse(to_metadata(meta)) == meta
    ts = {n: T(n, s) for n, s in (("q", [4, 16]), ("k", [2, 4]), ("h", [1, 16]), ("pos", [1]), ("kc", [32, 16]),
                                 ("r", [4, 16]))}
    apply(ts, meta, AP_FIXED_16_8)
    assert ts["q"].exp == 11 and list(ts["k"].exp) == [9, 10, 11, 12]
    assert ts["h"].kind == "f32" and ts["h"].host == "f32" and ts["pos"].kind == "host"
    assert ts["kc"].state and ts["kc"].group_layout == (2, 8) and ts["r"].kind == "i32"


@pytest.mark.parametrize("meta,msg", [
    ('{"host": {"q": "f64"}}', "kind"),
    ('{"exp": {"q": [1, 2]}}', "last axis"),
    ('{"exp": {"q": 50}}', "outside"),
    ('{"host": {"q": "f32"}, "exp": {"q": 8}}', "host tensor"),
    ('{"chexp": {"q": [8, 8, 8, 8]}}', "4-D"),
    ('{"layout": {"q": [2, 8]}}', "2-D state"),
    ('{"exp": {"nope": 8}}', "no tensor"),
    ('{"bogus": 1}', "not known"),
])
def test_annotation_errors(meta, msg):
    from cormorant_amd.dtype import AP_FIXED_16_8
    from cormorant_amd.graph import TensorInfo as T
    from cormorant_amd.numeric import NumericError, apply, parse
    with pytest.raises(NumericError, match=msg):
        apply({"q": T("q", [4, 16])}, parse(meta), AP_FIXED_16_8)


def test_check_accepts_the_workload_graphs_and_refuses_misplaced_numerics():
    from cormorant_amd import models, units
    from cormorant_amd.dtype import AP_FIXED_16_8
    from cormorant_amd.graph import ConvNode, ScheduledNode, TensorInfo as T
    from cormorant_amd.numeric import NumericError, check
    g, _, _ = models.bert_encoder(models.BertShape(layers=1, batch=1, seq=64, d=64, heads=1, ff=128, vocab=50))
    check(g.nodes, AP_FIXED_16_8)
    g, _, _ = models.smollm2_decode(models.LlamaShape(layers=1, batch=2, d=64, heads=4, kv=2, hd=16, ff=128,
                                                      vocab=64, ctx=32), runtime_pos=True)
    check(g.nodes, AP_FIXED_16_8)
    check(models.small_cnn(0)[0].nodes, AP_FIXED_16_8)
    with pytest.raises(NumericError, match="power-of-two"):
        check([ScheduledNode([T("a", [8], exp=10), T("b", [8], exp=10)], T("c", [8], exp=10), units.OP_ADD)],
              AP_FIXED_16_8)
    with pytest.raises(NumericError, match="states"):
        check([ScheduledNode([T("a", [8], state=True)], T("c", [8]), units.OP_RELU)], AP_FIXED_16_8)
    with pytest.raises(NumericError, match="derived"):
        check([ConvNode([T("x", [1, 1, 4, 4], exp=10), T("w", [1, 1, 1, 1], exp=3, data=np.ones((1, 1, 1, 1)))],
                        T("y", [1, 1, 4, 4], exp=10))], AP_FIXED_16_8)


def test_fuse_activations_rules():
    from cormorant_amd import units
    from cormorant_amd.graph import Graph, MatmulNode, ScheduledNode, TensorInfo as T, fuse_activations
    a, b = T("a", [16]), T("b", [16])
    s, r = T("s", [16]), T("r", [16])
    m, g_ = T("m", [16]), T("g", [16])
    x, out2 = T("x", [16]), T("o2", [16])
    w = T("w", [16, 16], data=np.zeros((16, 16)))
    mm, mr = T("mm", [1, 16]), T("mr", [1, 16])
    nodes = [ScheduledNode([a, b], s, units.OP_ADD), ScheduledNode([s], r, units.OP_RELU),       # fused
             ScheduledNode([a, b], m, units.OP_MUL), ScheduledNode([m], g_, units.OP_GELU),       # fused
             ScheduledNode([a, b], x, units.OP_SUB), ScheduledNode([x], out2, units.OP_RELU6),   # x is read twice
             ScheduledNode([x, x], T("x2", [16]), units.OP_ADD),
             MatmulNode([T("a2", [1, 16]), w], mm), ScheduledNode([mm], mr, units.OP_RELU)]       # not a VectorOP
    g = Graph(nodes, input_tensors=[a, b], output_tensors=[r, g_, out2, mr])
    assert fuse_activations(g) == 2
    assert [type(n).__name__ for n in g.nodes].count("ScheduledNode") == 6
    assert g.nodes[0].output is r and g.nodes[0].act == units.ACT_RELU
    assert g.nodes[1].output is g_ and g.nodes[1].act == units.ACT_GELU


def test_engine_pins_lower_matmuls_to_the_conv_unit():
    from cormorant_amd.graph import MatmulConvNode, MatmulNode, TensorInfo as T
    from cormorant_amd.numeric import lower_engines, parse
    nodes = [MatmulNode([T("a", [16, 64]), T("b", [64, 40], data=np.zeros((64, 40)))], T("c", [16, 40])),
             MatmulNode([T("a", [16, 64]), T("b2", [64, 40], data=np.zeros((64, 40)))], T("d", [16, 40]))]
    assert lower_engines(nodes, parse('{"engine": {"c": "conv", "d": "matmul"}}')) == 1
    assert isinstance(nodes[0], MatmulConvNode) and isinstance(nodes[1], MatmulNode)
