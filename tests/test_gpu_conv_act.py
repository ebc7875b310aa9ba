"""A convolution with the RELU / RELU6 that follows it fused (cm_conv_act, cm_conv_planes_act)
against the oracle's two unit calls -- the convolution, then VectorOP op 4 / 5 on its raw
output -- on every conv path (the folded 1x1 GEMM, im2col, the three depthwise kernels), with
full-range operands so that both bounds bite; and MobileNetV2's forward with only its logits
kept (every conv + RELU6 pair fused) against the oracle's graph."""
import numpy as np
import pytest

from gpu_util import POISON16, dev16, host, poisoned16
from test_gpu_random import CONV_CASES, rint16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def U():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cormorant_amd import units
    units.init()
    return units


@pytest.mark.parametrize("act", [1, 2])
@pytest.mark.parametrize("case", [c for c in CONV_CASES if not c[18]], ids=lambda c: "b%d_c%d_%dx%d_m%d_k%dx%d_s%d%d%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], c[7], c[8], "_dw" if c[16] else ""))
def test_conv_act_equals_conv_then_vectorop(U, oracle_lib, case, act):
    from cormorant_amd.packing import conv_bias_image, conv_weight_image
    (bt, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, has_b, dwise, full, wrap) = case
    rng = np.random.default_rng(C * 13 + M + act)
    lim = 32768 if full else 1024
    oh = (H + pt + pb - dh * (kh - 1) - 1) // sh + 1
    ow = (W + pl + pr - dw * (kw - 1) - 1) // sw + 1
    n = bt * M * oh * ow
    x = rint16(rng, bt * C * H * W, -lim, lim)
    w = conv_weight_image(rint16(rng, M * (1 if dwise else C) * kh * kw, -lim, lim).reshape(
        M, 1 if dwise else C, kh, kw), bool(dwise))
    bias = conv_bias_image(rint16(rng, M, -lim, lim))
    conv = oracle_lib.conv(x, w, bias if has_b else None, n, bt, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl,
                           has_b, dwise)
    want = oracle_lib.vectorop(conv, None, (n + 7) & ~7, n, 4 if act == 1 else 5)[:n]
    assert (want == 0).any() and (want != conv).any()        # the activation changes the output
    y = poisoned16(n + 8)
    U.conv(dev16(x), dev16(w), dev16(bias), y, bt, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, has_b, dwise,
           act=act)
    got = host(y)
    np.testing.assert_array_equal(got[:n], want)
    assert (got[n:] == POISON16).all()
    if not dwise:
        planes = U.conv_w_planes(dev16(w), M, C, kh, kw)
        y2 = poisoned16(n + 8)
        U.conv_planes(dev16(x), planes, dev16(bias), y2, bt, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl,
                      has_b, act=act)
        np.testing.assert_array_equal(host(y2)[:n], want)


def test_conv_act_refuses_other_acts(U):
    x, w = dev16(np.zeros(64, np.int16)), dev16(np.zeros(16 * 9, np.int16))
    with pytest.raises(ValueError):
        U.conv(x, w, None, poisoned16(64), 1, 1, 8, 8, 1, 8, 8, 3, 3, pad_top=1, pad_left=1, is_depthwise=1, act=3)


@pytest.mark.parametrize("batch,res,seed", [(2, 32, 0), (4, 64, 1)])
def test_mobilenet_logits_with_fused_relu6(batch, res, seed):
    """forward_raw keeping the logits alone runs every conv + RELU6 pair as one call; the logits
    equal the oracle's graph, and the fused pairs' intermediates are never written."""
    from cormorant_amd import models
    from cormorant_amd.simulate import Simulator
    from oracle import graph_sim
    g, inputs, _ = models.mobilenet_v2(batch=batch, res=res, seed=seed)
    sim = Simulator(g)
    feeds = {"input": sim._to_device(sim._tensor("input"), inputs["input"])}
    raw = sim.forward_raw(feeds, keep=["logits"])
    fused = [sn for i, sn in enumerate(g.nodes[:-1]) if sim._conv_act_fusable(sn, g.nodes[i + 1])]
    assert len(fused) == 35
    assert all(sn.output.onnx_name not in raw for sn in fused)
    got = sim._to_values(sim._tensor("logits"), raw["logits"])
    want = graph_sim.forward(g, inputs)["logits"]
    np.testing.assert_array_equal(got, want.reshape(got.shape))
