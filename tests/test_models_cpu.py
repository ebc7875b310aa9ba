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
