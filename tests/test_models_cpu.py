"""Graph builders on the CPU: the MobileNetV2 structure and its multiply-add count."""
from cormorant_amd import models
from cormorant_amd.graph import ConvNode, ScheduledNode


def test_mobilenet_v2_structure():
    g, inputs, macs = models.mobilenet_v2(batch=32, res=224)
    convs = [n for n in g.nodes if isinstance(n, ConvNode)]
    assert len(convs) == 52                      # stem + 17 blocks (16 with an expand) x 3 - 1 + head
    assert sum(n.is_depthwise for n in convs) == 17
    adds = [n for n in g.nodes if isinstance(n, ScheduledNode) and n.op_code == 0]
    assert len(adds) == 10                       # stride-1 blocks with matching channels
    assert macs == 32 * 300_774_272              # MobileNetV2 1.0 at 224: 300.8 M MAC per image
    assert g.output_tensors[0].shape == [32, 1000]
    assert inputs["input"].shape == (32, 3, 224, 224)


def test_smollm2_step_work():
    """SmolLM2-360M: 361 758 720 MAC per token in the linears and the tied head, 1.007 G MAC
    of attention for 16 sequences over 1024 keys, 723.5 MB of int16 weights."""
    s = models.LlamaShape()
    assert s.macs(keys=0) == 16 * 361_758_720
    assert s.macs() - s.macs(keys=0) == 16 * 32 * 2 * 15 * 1024 * 64
    assert s.weight_bytes() == 2 * 361_758_720


def test_smollm2_small_graph():
    from cormorant_amd.graph import KvWriteNode, SoftmaxVopNode
    g, inputs, exps = models.smollm2_decode(models.LlamaShape(layers=2, batch=2, d=64, heads=4, kv=2, hd=16,
                                                              ff=128, vocab=256, ctx=32), seed=3)
    assert sum(isinstance(n, KvWriteNode) for n in g.nodes) == 4
    smx = [n for n in g.nodes if isinstance(n, SoftmaxVopNode)]
    assert len(smx) == 2 and all(n.mask == 32 for n in smx)
    for e in exps[:-1]:
        assert e["s"] == e["q"] + e["k"] - 8 and e["o"] == e["p"] + e["v"] - 8
        assert e["a"] <= 15 and e["d"] <= 15 and e["g"] <= 14
    assert set(inputs) == {"ids"} | {f"l{i}.{c}" for i in range(2) for c in ("kc", "vc")}
