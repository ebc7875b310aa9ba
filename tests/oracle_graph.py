"""A CPU forward pass of a cormorant_amd Graph that restates the reference simulator's
``_forward_pass`` (inference-scheduler/src/codegen/_simulate.py:541-769) in the value domain
with numpy float64, the way the reference computes: np.matmul / per-tap conv sums (exact for
on-grid operands), then ``truncate`` (clip + floor).  Pooling, the activation unit, softmax
and row-ops use the C oracle on raw lanes.  Test infrastructure only: the graph-level check
of cormorant_amd.simulate.Simulator.
"""
import numpy as np

from cormorant_amd import graph as G
from cormorant_amd.dtype import AP_FIXED_16_8 as DT
from oracle import cm


def _conv_int(x, w, sh, sw, pt, pl, dh, dw, oh, ow, dwise):
    """_conv2d_int (_simulate.py:198-220): exact per-tap sums of float64 integers."""
    N, C, H, W = x.shape
    kh, kw = w.shape[2], w.shape[3]
    need_h = (oh - 1) * sh + (kh - 1) * dh + 1
    need_w = (ow - 1) * sw + (kw - 1) * dw + 1
    xp = np.zeros((N, C, max(need_h, pt + H), max(need_w, pl + W)))
    xp[:, :, pt:pt + H, pl:pl + W] = x
    y = np.zeros((N, w.shape[0], oh, ow))
    for a in range(kh):
        for b in range(kw):
            xs = xp[:, :, a * dh:a * dh + (oh - 1) * sh + 1:sh, b * dw:b * dw + (ow - 1) * sw + 1:sw]
            if dwise:
                y += xs * w[:, 0, a, b][None, :, None, None]
            else:
                y += np.einsum("nchw,mc->nmhw", xs, w[:, :, a, b], optimize=True)
    return y


def _weight(t):
    return DT.quantize(np.asarray(t.data, np.float64).reshape(t.shape))


def forward(graph, inputs):
    vals = {k: np.asarray(v, np.float64) for k, v in inputs.items()}
    get = lambda t: vals[t.onnx_name] if t.onnx_name in vals else _weight(t)
    for sn in graph.nodes:
        out = sn.output
        if isinstance(sn, G.MatmulNode):
            a, b = get(sn.inputs[0]), get(sn.inputs[1])
            vals[out.onnx_name] = DT.truncate(np.matmul(a, b)).reshape(out.shape)
        elif isinstance(sn, G.ConvNode):
            x, w = get(sn.inputs[0]), get(sn.inputs[1])
            acc = _conv_int(x * 256, w * 256, sn.stride_h, sn.stride_w, sn.pad_top, sn.pad_left,
                            sn.dilation_h, sn.dilation_w, sn.out_h, sn.out_w, sn.is_depthwise) / 65536.0
            if sn.has_bias:
                acc = acc + get(sn.inputs[2]).reshape(1, -1, 1, 1)
            vals[out.onnx_name] = DT.truncate(acc).reshape(out.shape)
        elif isinstance(sn, G.ReshapeNode):
            vals[out.onnx_name] = get(sn.inputs[0]).reshape(out.shape)
        elif isinstance(sn, G.PoolNode):
            xt = sn.inputs[0]
            raw = DT.to_raw(get(xt)).reshape(-1)
            y = cm.pool(raw, xt.shape[0], xt.shape[1], xt.shape[2], xt.shape[3], out.shape[2],
                        out.shape[3], sn.pool_h, sn.pool_w, sn.stride_h, sn.stride_w, sn.pad_top,
                        sn.pad_left, sn.dil_h, sn.dil_w, sn.pool_type, sn.lp_order, sn.count_include_pad)
            vals[out.onnx_name] = DT.from_raw(y).reshape(out.shape)
        elif isinstance(sn, G.SoftmaxVopNode):
            x = DT.to_raw(get(sn.inputs[0]))
            n = x.shape[-1]
            rows = x.size // n
            n8 = (n + 7) & ~7
            xr = np.zeros((rows, n8), np.int16)
            xr[:, :n] = x.reshape(rows, n)
            c = cm.vectorop(xr.reshape(-1), None, rows * n8, n, 10, rows, n8, n8, 0, 0, sn.cm, sn.cfg, sn.mask_reg(n))
            fp = (sn.cfg >> 8) & 31
            vals[out.onnx_name] = (c.reshape(rows, n8)[:, :n].astype(np.float64) / 2.0 ** fp).reshape(out.shape)
        elif isinstance(sn, G.ScheduledNode):
            # numpy broadcasting of the logical arrays (_simulate.py:721-765), on raw lanes
            full = lambda t: np.broadcast_to(get(t).reshape([1] * (len(out.shape) - len(t.shape)) + list(t.shape)),
                                             out.shape)
            ar = DT.to_raw(full(sn.inputs[0])).reshape(-1)
            br = DT.to_raw(full(sn.inputs[1])).reshape(-1) if sn.arity == 2 else None
            n = ar.size
            c = cm.vectorop(ar, br, (n + 7) & ~7, n, sn.op_code, 1, 0, 0, sn.act, sn.alpha)
            vals[out.onnx_name] = DT.from_raw(c[:n]).reshape(out.shape)
        else:
            raise NotImplementedError(type(sn).__name__)
    return vals
