"""The front end's node choice (cormorant_amd/frontend.py, the reference's graph.py:817-856 and its
unit-or-host rules): the five workloads described op by op build the same nodes as their
hand-built graphs, and every fallback to a host op fires where the reference's does."""
import dataclasses

import numpy as np
import pytest

from cormorant_amd import frontend, models, units
from cormorant_amd.frontend import LLM_DOMAIN, OpDesc, Platform, build_graph
from cormorant_amd.graph import SchedulerError, TensorInfo


def _same_value(a, b):
    if isinstance(a, TensorInfo) or isinstance(b, TensorInfo):
        return (a is None) == (b is None) and (a is None or a.onnx_name == b.onnx_name)
    if isinstance(a, np.ndarray) or isinstance(b, np.ndarray):
        return np.array_equal(np.asarray(a), np.asarray(b))
    if isinstance(a, (list, tuple)) and isinstance(b, (list, tuple)):
        return len(a) == len(b) and all(_same_value(x, y) for x, y in zip(a, b))
    return a == b


def assert_same_graph(g1, g2):
    assert len(g1.nodes) == len(g2.nodes)
    for i, (a, b) in enumerate(zip(g1.nodes, g2.nodes)):
        assert type(a) is type(b), f"node {i}: {type(a).__name__} vs {type(b).__name__}"
        for f in dataclasses.fields(a):
            va, vb = getattr(a, f.name), getattr(b, f.name)
            assert _same_value(va, vb), f"node {i} ({type(a).__name__}) field {f.name}"
        for ta, tb in zip(list(a.inputs) + [a.output], list(b.inputs) + [b.output]):
            if ta is None:
                continue
            assert ta.onnx_name == tb.onnx_name and list(ta.shape) == list(tb.shape)
            assert _same_value(ta.exp, tb.exp) and ta.kind == tb.kind
            assert _same_value(ta.wexp, tb.wexp) and _same_value(ta.data, tb.data), ta.onnx_name
    assert [t.onnx_name for t in g1.input_tensors] == [t.onnx_name for t in g2.input_tensors]
    assert [t.onnx_name for t in g1.output_tensors] == [t.onnx_name for t in g2.output_tensors]


def test_small_cnn_from_ops():
    g, _ = models.small_cnn(3)
    (ops, tensors, ins, outs), _ = models.small_cnn(3, as_ops=True)
    assert_same_graph(build_graph(ops, tensors, ins, outs), g)


def test_mobilenet_v2_from_ops():
    g, _, _ = models.mobilenet_v2(batch=2, res=32, seed=1)
    (ops, tensors, ins, outs), _, _ = models.mobilenet_v2(batch=2, res=32, seed=1, as_ops=True)
    assert_same_graph(build_graph(ops, tensors, ins, outs), g)


def test_bert_encoder_from_ops():
    shape = models.BertShape(layers=2, batch=1, seq=64, d=128, heads=2, ff=256, vocab=300)
    g, _, _ = models.bert_encoder(shape, seed=4)
    (ops, tensors, ins, outs), _, _ = models.bert_encoder(shape, seed=4, as_ops=True)
    g2 = build_graph(ops, tensors, ins, outs)
    assert_same_graph(g2, g)
    # the FFN's Add and Gelu became one VectorOP node with the GELU act (graph.py:1005-1069)
    assert sum(type(n).__name__ == "ScheduledNode" and n.act == units.ACT_GELU for n in g2.nodes) == 2


@pytest.mark.parametrize("runtime_pos", [False, True])
def test_smollm2_decode_from_ops(runtime_pos):
    shape = models.LlamaShape(layers=2, batch=2, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=64)
    g, _, _ = models.smollm2_decode(shape, seed=2, runtime_pos=runtime_pos)
    (ops, tensors, ins, outs), _, _ = models.smollm2_decode(shape, seed=2, runtime_pos=runtime_pos, as_ops=True)
    assert_same_graph(build_graph(ops, tensors, ins, outs), g)


@pytest.mark.parametrize("with_head", [False, True])
def test_smollm2_prefill_from_ops(with_head):
    """The prefill entry's op list (LlmAttnPrep, LlmAttnScores, LlmAttnSoftmax vsmx, LlmAttnPV,
    LlmAttnMerge, LlmSelectRow among the usual ops) builds the hand-built graph."""
    shape = models.LlamaShape(layers=2, batch=1, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=128)
    w = models.smollm2_weights(shape, 3)
    _, _, exps = models.smollm2_decode(shape, seed=3, weights=w, runtime_pos=True)
    g = models.smollm2_prefill(shape, 32, exps, w, with_head=with_head)
    ops, tensors, ins, outs = models.smollm2_prefill(shape, 32, exps, w, with_head=with_head, as_ops=True)
    assert_same_graph(build_graph(ops, tensors, ins, outs), g)


def test_prefill_attention_ops_refused_off_the_units():
    """The host forms of the prefill chain are not built: LlmAttnPrep without the row-ops unit,
    LlmAttnSoftmax without vsmx or the softmax unit, the prefix-LM mask."""
    shape = models.LlamaShape(layers=1, batch=1, d=128, heads=4, kv=2, hd=32, ff=256, vocab=512, ctx=128)
    w = models.smollm2_weights(shape, 3)
    _, _, exps = models.smollm2_decode(shape, seed=3, weights=w, runtime_pos=True)
    ops, tensors, ins, outs = models.smollm2_prefill(shape, 16, exps, w, as_ops=True)
    prep = next(o for o in ops if o.op_type == "LlmAttnPrep")
    smx = next(o for o in ops if o.op_type == "LlmAttnSoftmax")
    with pytest.raises(SchedulerError, match="row-ops"):
        _one(prep, tensors, Platform(rowops=False))
    with pytest.raises(SchedulerError, match="vsmx"):
        _one(smx, tensors, Platform(softmax=False))
    host = frontend.OpDesc(smx.op_type, smx.inputs, smx.outputs, {**smx.attrs, "vsmx": 0}, smx.domain)
    with pytest.raises(SchedulerError, match="p12"):
        _one(host, tensors)
    prefix = frontend.OpDesc(smx.op_type, smx.inputs, smx.outputs, {**smx.attrs, "causal": 2}, smx.domain)
    with pytest.raises(SchedulerError, match="prefix"):
        _one(prefix, tensors)
    enc = frontend.OpDesc(smx.op_type, smx.inputs, smx.outputs, {**smx.attrs, "causal": 0}, smx.domain)
    assert _one(enc, tensors).causal is False


# ---------------------------------------------------------------- the unit-or-host rules
def _t(name, shape, **kw):
    return TensorInfo(name, list(shape), **kw)


def _one(op, tensors, platform=Platform()):
    return frontend.node_for(op, frontend._Ctx(tensors, platform, frontend.Q88))


def _kind(sn):
    return type(sn).__name__


def test_softmax_unit_or_host():
    T = {"x": _t("x", [4, 64]), "y": _t("y", [4, 64])}
    sn = _one(OpDesc("Softmax", ["x"], ["y"]), T)
    assert _kind(sn) == "SoftmaxVopNode" and (sn.cm, sn.cfg) == (12102203, 0x0813)
    assert _kind(_one(OpDesc("Softmax", ["x"], ["y"]), T, Platform(softmax=False))) == "SoftmaxNode"
    # exponent-annotated tensors, rows beyond the unit's buffer, unaligned rows: the host op
    P = {"x": _t("x", [4, 64], exp=10), "y": _t("y", [4, 64])}
    assert _kind(_one(OpDesc("Softmax", ["x"], ["y"]), P)) == "SoftmaxNode"
    L = {"x": _t("x", [2, 2056]), "y": _t("y", [2, 2056])}
    assert _kind(_one(OpDesc("Softmax", ["x"], ["y"]), L)) == "SoftmaxNode"
    U = {"x": _t("x", [3, 10]), "y": _t("y", [3, 10])}
    assert _kind(_one(OpDesc("Softmax", ["x"], ["y"]), U)) == "SoftmaxNode"
    # one row of 10 (the small CNN's logits) stays on the unit
    O = {"x": _t("x", [1, 10]), "y": _t("y", [1, 10])}
    assert _kind(_one(OpDesc("Softmax", ["x"], ["y"]), O)) == "SoftmaxVopNode"


def test_layernorm_unit_or_host():
    rng = np.random.default_rng(0)
    n = 96
    g, b = 1 + 0.1 * rng.standard_normal(n), 0.1 * rng.standard_normal(n)
    T = {"x": _t("x", [8, n]), "y": _t("y", [8, n])}
    op = OpDesc("LayerNormalization", ["x"], ["y"], {"gamma": g, "beta": b, "epsilon": 1e-5})
    assert _kind(_one(op, T)) == "LayerNormRoNode"
    assert _kind(_one(op, T, Platform(rowops=False))) == "LayerNormNode"
    assert _kind(_one(op, {"x": _t("x", [8, n], exp=12), "y": _t("y", [8, n])})) == "LayerNormNode"
    assert _kind(_one(OpDesc("LayerNormalization", ["x"], ["y"], {"gamma": np.ones(4104), "beta": np.zeros(4104)}),
                      {"x": _t("x", [2, 4104]), "y": _t("y", [2, 4104])})) == "LayerNormNode"
    assert _kind(_one(OpDesc("LayerNormalization", ["x"], ["y"], {"gamma": np.ones(12), "beta": np.zeros(12)}),
                      {"x": _t("x", [3, 12]), "y": _t("y", [3, 12])})) == "LayerNormNode"
    big = OpDesc("LayerNormalization", ["x"], ["y"], {"gamma": g, "beta": np.full(n, 1e9)})
    assert _kind(_one(big, T)) == "LayerNormNode"
    nan = OpDesc("LayerNormalization", ["x"], ["y"], {"gamma": np.full(n, np.nan), "beta": b})
    assert _kind(_one(nan, T)) == "LayerNormNode"


def test_activation_unit_or_host():
    T = {"x": _t("x", [64]), "y": _t("y", [64])}
    assert _one(OpDesc("Gelu", ["x"], ["y"]), T).op_code == units.OP_GELU
    assert _one(OpDesc("Gelu", ["x"], ["y"], {"approximate": "tanh"}), T).op_code == units.OP_GELU_TANH
    # a GELU whose constants differ from the unit's function stays on the host
    assert _kind(_one(OpDesc("Gelu", ["x"], ["y"], {"approximate": "tanh", "c1": 0.05}), T)) == "GeluNode"
    assert _kind(_one(OpDesc("Gelu", ["x"], ["y"]), T, Platform(activations=False))) == "GeluNode"
    assert _kind(_one(OpDesc("Gelu", ["x"], ["y"]), {"x": _t("x", [64], exp=9), "y": _t("y", [64])})) == "GeluNode"
    assert _one(OpDesc("Silu", ["x"], ["y"]), T).op_code == units.OP_SILU
    lr = _one(OpDesc("LeakyRelu", ["x"], ["y"], {"alpha": 0.1}), T)
    assert lr.op_code == units.OP_LEAKY_RELU and lr.alpha == round(0.1 * 65536)
    assert _one(OpDesc("LeakyRelu", ["x"], ["y"]), T).alpha == round(0.01 * 65536)       # ONNX's default slope
    with pytest.raises(SchedulerError):
        _one(OpDesc("LeakyRelu", ["x"], ["y"], {"alpha": 1.5}), T)
    for op in ("Silu", "LeakyRelu"):          # no host fallback for these: the unit or an error
        with pytest.raises(SchedulerError):
            _one(OpDesc(op, ["x"], ["y"]), T, Platform(activations=False))


def test_clip_maps_to_relu6_only():
    T = {"x": _t("x", [16]), "y": _t("y", [16]), "lo": _t("lo", [1], data=np.zeros(1)),
         "hi": _t("hi", [1], data=np.full(1, 6.0)), "one": _t("one", [1], data=np.ones(1))}
    assert _one(OpDesc("Clip", ["x"], ["y"], {"min": 0.0, "max": 6.0}), T).op_code == units.OP_RELU6
    sn = _one(OpDesc("Clip", ["x", "lo", "hi"], ["y"]), T)            # opset 11: bounds as constant inputs
    assert sn.op_code == units.OP_RELU6 and [t.onnx_name for t in sn.inputs] == ["x"]
    with pytest.raises(SchedulerError, match="Only Clip"):
        _one(OpDesc("Clip", ["x", "lo", "one"], ["y"]), T)
    with pytest.raises(SchedulerError):
        _one(OpDesc("Add", ["x"], ["y"]), T)                          # a binary op with one input


def test_transpose_unit_or_host():
    T = {"x": _t("x", [1, 16, 4, 32]), "y": _t("y", [1, 4, 16, 32])}
    op = OpDesc("Transpose", ["x"], ["y"], {"perm": [0, 2, 1, 3]})   # a head split: one COPY job
    assert _kind(_one(op, T)) == "TransposeRoNode"
    assert _kind(_one(op, T, Platform(rowops=False))) == "TransposeNode"
    K = {"x": _t("x", [64, 32]), "y": _t("y", [32, 64])}              # K^T: one TRANSPOSE job
    assert _kind(_one(OpDesc("Transpose", ["x"], ["y"]), K)) == "TransposeRoNode"
    B2 = {"x": _t("x", [2, 16, 4, 32]), "y": _t("y", [2, 4, 16, 32])}  # four dims that do not merge
    assert _kind(_one(op, B2)) == "TransposeNode"
    O = {"x": _t("x", [2, 5, 3]), "y": _t("y", [3, 5, 2])}
    assert _kind(_one(OpDesc("Transpose", ["x"], ["y"]), O)) == "TransposeNode"   # not a unit job


def test_llm_ops_take_the_rowops_unit_where_present():
    T = {"h": _t("h", [2, 64], exp=15, kind="i32"), "x": _t("x", [2, 64], exp=10),
         "d": _t("d", [2, 64], exp=12), "h1": _t("h1", [2, 64], exp=15, kind="i32")}
    rms = OpDesc("LlmRMSNorm", ["h"], ["x"], {"gamma": np.ones(64)}, LLM_DOMAIN)
    assert _kind(_one(rms, T)) == "RMSNormRoNode"
    assert _kind(_one(rms, T, Platform(rowops=False))) == "LlmRMSNormNode"
    add = OpDesc("LlmResAdd", ["h", "d"], ["h1"], {}, LLM_DOMAIN)
    assert _kind(_one(add, T)) == "ResAddRoNode"
    assert _kind(_one(add, T, Platform(rowops=False))) == "LlmResAddNode"
    with pytest.raises(SchedulerError, match="row-ops"):
        _one(OpDesc("VitLayerNorm", ["h"], ["x"], {"gamma": np.ones(64), "beta": np.zeros(64)}, LLM_DOMAIN), T,
             Platform(rowops=False))


def test_unsupported_ops_are_errors():
    T = {"x": _t("x", [4]), "y": _t("y", [4])}
    with pytest.raises(SchedulerError, match="not supported"):
        _one(OpDesc("Erf", ["x"], ["y"]), T)
    with pytest.raises(SchedulerError, match="unknown"):
        _one(OpDesc("LlmFoo", ["x"], ["y"], {}, LLM_DOMAIN), T)
    with pytest.raises(SchedulerError, match="host op"):
        _one(OpDesc("Gather", ["x"], ["y"]), T)
    with pytest.raises(SchedulerError, match="not found"):
        _one(OpDesc("Relu", ["z"], ["y"]), T)


def test_frontend_graph_simulates_like_the_hand_built_one():
    """The front end's small CNN through the CPU checker gives the hand-built graph's values."""
    from oracle import graph_sim
    g, inputs = models.small_cnn(5)
    (ops, tensors, ins, outs), _ = models.small_cnn(5, as_ops=True)
    a = graph_sim.forward(g, inputs)
    b = graph_sim.forward(build_graph(ops, tensors, ins, outs), inputs)
    assert np.array_equal(a["probs"], b["probs"])
