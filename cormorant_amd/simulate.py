"""The fixed-point simulator on the GPU: ``Simulator(graph).simulate(inputs)`` is the
reference's ``CodeGenerator.simulate`` (inference-scheduler/src/codegen/_simulate.py:382-403)
and ``_forward_pass`` its per-node dispatch (:541-769), with every node run by the HIP units.

Values cross the API as float64 arrays (value = raw * 2^-f, exact), as in the reference.
Inside, each tensor is a raw int16 (int32 / float32 for row-ops kinds) torch tensor on the
device with its exponent, so a graph runs from node to node without leaving HBM; the
conversion happens once at the graph's inputs, weights and returned tensors.
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional

import numpy as np
import torch

from . import residuals, units
from .dtype import AP_FIXED_16_8, ApFixed16
from .graph import (AttentionNode, AttnContractNode, AttnMergeNode, AttnSoftmaxNode, ConvNode, DecodeAttentionNode, Graph,
                    KvWriteNode, LlmAttnConvNode, MatmulConvNode, SelectRowNode,
                    MatmulNode, PermuteNode, PoolNode, ReshapeNode, RowOpsNode, ScheduledNode, SchedulerError, SoftmaxVopNode,
                    TensorInfo, attn_keys)
from .packing import conv_bias_image, conv_lowered_b_image, conv_weight_image, pack_matmul_b
from .host_ops import HostNode, LlmEmbedNode
from .rowops_nodes import DecodePrepNode, RoCallNode, RoJob, RowOpsAdapter

def node_reference(node, ins, dtype: Optional[ApFixed16] = None, device: str = "cuda",
                   host: Optional[Dict[str, np.ndarray]] = None) -> np.ndarray:
    """The output values of ``node`` alone for the input values ``ins`` (one per node input,
    in order), computed by the HIP units: a one-node graph through ``Simulator._forward_pass``.
    The per-node form of the reference's ``reference(ins, dtype)`` (_simulate.py:667-690).  A
    constant input (a tensor with ``data`` that is not a state) reads its own data, as in the
    graph; a state input whose value is a float64 array is updated in place (the node's write
    into the persistent state), any other value seeds the state.  ``host`` holds the values of
    runtime host tensors the node reads outside its inputs (``pos_t``, ``mask_t``)."""
    if len(ins) != len(node.inputs):
        raise ValueError(f"{type(node).__name__}.reference: {len(ins)} values for {len(node.inputs)} inputs")
    feeds: Dict[str, np.ndarray] = {}
    states: Dict[str, np.ndarray] = {}
    graph_in = []
    for t, v in zip(node.inputs, ins):
        if t is None or t.onnx_name in feeds or t.onnx_name in states or (t.data is not None and not t.state):
            continue
        if v is None:
            raise ValueError(f"{type(node).__name__}.reference: no value for input '{t.onnx_name}'")
        if t.state and isinstance(v, np.ndarray) and v.dtype == np.float64 and v.size == t.numel:
            states[t.onnx_name] = v              # updated in place, as the graph's state
        else:
            feeds[t.onnx_name] = np.asarray(v)
        graph_in.append(t)
    for field_name, t in vars(node).items():      # runtime host tensors outside the inputs
        if isinstance(t, TensorInfo) and t.kind == "host" and t is not node.output and t.onnx_name not in feeds:
            if host is None or t.onnx_name not in host:
                raise ValueError(f"{type(node).__name__}.reference: the runtime tensor '{t.onnx_name}' "
                                 f"({field_name}) needs its value in host")
            feeds[t.onnx_name] = np.asarray(host[t.onnx_name])
            graph_in.append(t)
    g = Graph(nodes=[node], input_tensors=graph_in, output_tensors=[node.output])
    out = node.output.onnx_name
    sim = Simulator(g, dtype or AP_FIXED_16_8, device)
    return sim._forward_pass(feeds, states={**sim.initial_states(), **states}, keep=[out])[out]


_TORCH = {"i16": torch.int16, "i32": torch.int32, "f32": torch.float32}
_NP = {"i16": np.int16, "i32": np.int32, "f32": np.float32}
_KB = {"i16": 2, "i32": 4, "f32": 4}


def _pad8(n: int) -> int:
    return (n + 7) & ~7


class Simulator:
    """Forward-simulates ``graph`` with the HIP units on ``device``."""

    def __init__(self, graph: Graph, dtype: ApFixed16 = AP_FIXED_16_8, device: str = "cuda",
                 share: Optional["Simulator"] = None):
        """``share``: another entry of the same model (a prefill and a decode graph over one set of
        weights): its device copies of the weights and their packed images are used, not uploaded
        again -- the entries of a reference project read the same initializers by name."""
        self._graph = graph
        self._dtype = dtype
        self.device = torch.device(device)
        self._weights: Dict[str, torch.Tensor] = {} if share is None else share._weights    # raw device weights
        self._images: Dict[str, torch.Tensor] = {} if share is None else share._images      # packed weight images
        self._infos: Dict[str, TensorInfo] = {}
        self._params: Dict[int, list] = {}                # row-ops parameter blocks on the device
        self._staging: Dict[tuple, torch.Tensor] = {}     # row-ops nodes' staging buffers
        self._plan = None                                  # MatMuls fed byte planes by their A's producer
        self._keep = None                                  # forward_raw's keep (None: every tensor)
        self._planes_only_names = None                     # tensors only plane-path MatMuls read
        self._errors = None                                # residual statistics being collected
        for t in graph.input_tensors + graph.output_tensors:
            self._infos[t.onnx_name] = t
        # the fused launches that apply a row-ops job inside another unit leave the device's
        # parameter RAM as it was; a graph with a P_KEEP job (which reads that RAM) runs every
        # row-ops job on the unit itself instead
        self._ram_free = not any(isinstance(sn, RowOpsNode) and (sn.op & units.F_P_KEEP) for sn in graph.nodes)
        for sn in graph.nodes:
            for t in list(sn.inputs) + [sn.output]:
                if t is not None:
                    self._infos.setdefault(t.onnx_name, t)
        units.init()

    # ------------------------------------------------------------------ public API
    def simulate(self, inputs: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
        """float64 inputs (on their grids) -> float64 graph outputs (_simulate.py:382-403)."""
        arrays = self._forward_pass(inputs, keep=[t.onnx_name for t in self._graph.output_tensors])
        return {t.onnx_name: arrays[t.onnx_name] for t in self._graph.output_tensors}

    def initial_states(self) -> Dict[str, np.ndarray]:
        """Fresh float64 values of the graph's persistent states: a state's ``data``, else 0
        (the reference's initial_states)."""
        out = {}
        for t in self._graph.state_tensors:
            v = np.zeros(t.shape) if t.data is None else np.asarray(t.data, np.float64).reshape(t.shape)
            out[t.onnx_name] = v.copy()
        return out

    def _forward_pass(self, input_arrays: Dict[str, np.ndarray], errors_out=None, states=None,
                      keep: Optional[Iterable[str]] = None) -> Dict[str, np.ndarray]:
        """Run every node; returns float64 values of every tensor visited, or only ``keep`` and
        the states (the reference's lean mode, _simulate.py:541-592).  ``states`` ({name:
        float64 array}, default fresh initial_states()) are the persistent state tensors: the
        nodes update them in place on the device and the caller's arrays receive the new values,
        so a caller can run several passes over the same states (_simulate.py:573-577,
        609-611).  Inputs may also carry a state's value (it then replaces the array's).
        ``errors_out`` (a dict) receives {output name: ResidualStats} of every MatMul, Conv
        without exponents, Pool and VectorOP node (_simulate.py:594-602): each node then runs
        in its own launch, so that its output exists to compare."""
        st_names = [t.onnx_name for t in self._graph.state_tensors]
        if states is None:
            states = self.initial_states()
        missing = [nm for nm in st_names if nm not in states and nm not in input_arrays]
        if missing:
            raise KeyError(f"states {missing} have no value")
        feeds = {nm: self._to_device(self._tensor(nm), states[nm]) for nm in st_names if nm not in input_arrays}
        feeds.update({name: self._to_device(self._tensor(name), v) for name, v in input_arrays.items()})
        self._errors = errors_out
        try:
            raw = self.forward_raw(feeds, keep=None if keep is None else set(keep) | set(st_names))
        finally:
            self._errors = None
        for nm in st_names:                      # the states as the pass left them, in place
            if nm in states:
                states[nm][...] = self._to_values(self._tensor(nm), feeds[nm]).reshape(np.shape(states[nm]))
        # (names with '#' are a producer's byte planes for a MatMul, not graph tensors)
        wanted = {nm for nm in raw if "#" not in nm} if keep is None else set(keep) | set(st_names)
        return {name: self._to_values(self._tensor(name), t) for name, t in raw.items() if name in wanted}

    def forward_raw(self, raw_inputs: Dict[str, torch.Tensor],
                    keep: Optional[Iterable[str]] = None) -> Dict[str, torch.Tensor]:
        """The device-resident path: raw input tensors in, raw tensors of every node out.  With
        ``keep`` (the names the caller reads; the graph's outputs and states are always kept) a
        tensor that only plane-path MatMuls read, as the byte planes its producer writes, is not
        written at all and is absent from the result."""
        self._keep = None if keep is None else set(keep)
        raw: Dict[str, torch.Tensor] = dict(raw_inputs)
        nodes = self._graph.nodes
        fuse = self._errors is None                 # residual statistics read every node's own output
        i = 0
        while i < len(nodes):
            sn = nodes[i]
            i += 1
            if not fuse:
                self._dispatch(sn, raw)
                self._record_residuals(sn, raw)
                continue
            if self._skinny_single(sn):
                # the skinny MatMuls that follow on the same A: one launch for up to 4
                group = [sn]
                while (i < len(nodes) and len(group) < 4 and self._skinny_single(nodes[i])
                       and nodes[i].inputs[0].onnx_name == sn.inputs[0].onnx_name):
                    group.append(nodes[i])
                    i += 1
                if len(group) > 1:
                    if i < len(nodes) and self._mulact_fusable(group, nodes[i]):
                        # gate / up and the SiLU gate over their outputs: one launch
                        self._matmul_mulact(group, nodes[i], raw)
                        i += 1
                        continue
                    self._matmul_group(group, raw)
                    continue
            if i < len(nodes) and self._output_job_fusable(sn, nodes[i]):
                # a decode linear and the row-ops job on its output (the residual add): one launch
                self._matmul_output_job(sn, nodes[i], raw)
                i += 1
                continue
            if i < len(nodes) and self._addx_norm_fusable(sn, nodes[i]):
                # a residual add and the LayerNorm of its output: one launch, both outputs kept
                self._addx_norm(sn, nodes[i], raw)
                i += 1
                continue
            if i < len(nodes) and self._conv_act_fusable(sn, nodes[i]):
                # a convolution and the RELU / RELU6 of its output: one launch, the activated output alone
                act = units.ACT_RELU if nodes[i].op_code == units.OP_RELU else units.ACT_RELU6
                raw[nodes[i].output.onnx_name] = self._conv(sn, raw, act=act, out_t=nodes[i].output)
                i += 1
                continue
            if self._planes_out(sn) is not None and self._planes_node(sn, raw):
                continue
            if i < len(nodes) and self._prep_attention_fusable(sn, nodes[i]):
                # the decode prep and the attention of its outputs: one launch
                self._prep_attention(sn, nodes[i], raw)
                i += 1
                continue
            self._dispatch(sn, raw)
        return raw

    def _dispatch(self, sn, raw: Dict[str, torch.Tensor]) -> None:
        """Run one node on its unit, its output into ``raw``."""
        if isinstance(sn, MatmulNode):
            raw[sn.output.onnx_name] = self._matmul(sn, raw)
        elif isinstance(sn, LlmEmbedNode):
            raw[sn.output.onnx_name] = self._embed(sn, raw)
        elif isinstance(sn, HostNode):
            raw[sn.output.onnx_name] = self._host_node(sn, raw)
        elif isinstance(sn, MatmulConvNode):
            raw[sn.output.onnx_name] = self._matmul_conv(sn, raw)
        elif isinstance(sn, ConvNode):
            raw[sn.output.onnx_name] = self._conv(sn, raw)
        elif isinstance(sn, ReshapeNode):
            raw[sn.output.onnx_name] = self._get(sn.inputs[0], raw)
        elif isinstance(sn, PoolNode):
            raw[sn.output.onnx_name] = self._pool(sn, raw)
        elif isinstance(sn, SoftmaxVopNode):
            raw[sn.output.onnx_name] = self._softmax(sn, raw)
        elif isinstance(sn, RowOpsNode):
            raw[sn.output.onnx_name] = self._rowops(sn, raw)
        elif isinstance(sn, RowOpsAdapter):
            raw[sn.output.onnx_name] = self._adapter(sn, raw)
        elif isinstance(sn, RoCallNode):
            raw[sn.output.onnx_name] = self._ro_calls(sn, raw)
        elif isinstance(sn, LlmAttnConvNode):
            raw[sn.output.onnx_name] = self._attn_conv(sn, raw)
        elif isinstance(sn, AttnSoftmaxNode):
            raw[sn.output.onnx_name] = self._attn_softmax(sn, raw)
        elif isinstance(sn, AttnMergeNode):
            raw[sn.output.onnx_name] = self._attn_merge(sn, raw)
        elif isinstance(sn, SelectRowNode):
            raw[sn.output.onnx_name] = self._select_row(sn, raw)
        elif isinstance(sn, PermuteNode):
            raw[sn.output.onnx_name] = self._permute(sn, raw)
        elif isinstance(sn, AttnContractNode):
            raw[sn.output.onnx_name] = self._attn_contract(sn, raw)
        elif isinstance(sn, KvWriteNode):
            raw[sn.output.onnx_name] = self._kv_write(sn, raw)
        elif isinstance(sn, DecodeAttentionNode):
            raw[sn.output.onnx_name] = self._decode_attention(sn, raw)
        elif isinstance(sn, DecodePrepNode):
            raw[sn.output.onnx_name] = self._decode_prep(sn, raw)
        elif isinstance(sn, AttentionNode):
            raw[sn.output.onnx_name] = self._attention(sn, raw)
        elif isinstance(sn, ScheduledNode):
            raw[sn.output.onnx_name] = self._vectorop(sn, raw)
        else:
            raise SchedulerError(f"_forward_pass: unsupported node {type(sn).__name__}")

    # ------------------------------------------------------------------ expected outputs on disk
    def _build_ramp_inputs(self) -> Dict[str, np.ndarray]:
        """The inputs the reference's generated test writes into the buffers (_simulate.py:423-504):
        an exponent tensor the ramp p[i] = (int16) i at its exponent(s); an integer tensor (ids)
        i % R with R the smallest embedding table that reads it (else 2); a float32 host tensor
        (i % 17 - 8) / 4; a host integer i % 2; a Q8.8 tensor the ramp at 2^-8."""
        out = {}
        dt = self._dtype
        readers = {}
        for sn in self._graph.nodes:
            if isinstance(sn, LlmEmbedNode):
                name = sn.inputs[0].onnx_name
                readers[name] = min(readers.get(name, sn.rows), sn.rows)
        for t in self._graph.input_tensors:
            idx = np.arange(t.numel, dtype=np.int64)
            if t.kind == "f32":
                v = ((idx % 17) - 8).astype(np.float64) * 0.25
            elif t.kind == "host" or (t.kind == "i32" and t.onnx_name in readers):
                v = (idx % max(1, min(readers.get(t.onnx_name, 2), 32767))).astype(np.float64)
            elif t.exp is not None:
                e = np.broadcast_to(np.asarray(t.exp, np.float64).reshape(-1), (t.shape[-1],) if len(t.shape) else (1,))
                v = dt.ramp_to_float_exp(idx, np.tile(e, t.numel // e.size))
            else:
                v = dt.ramp_to_float(idx)
            out[t.onnx_name] = v.reshape(t.shape)
        return out

    def _simulate(self) -> Dict[str, np.ndarray]:
        """The forward pass with the ramp inputs (_simulate.py:506-525)."""
        return self._forward_pass(self._build_ramp_inputs())

    def compute_quant_errors(self) -> Dict[str, "residuals.ResidualStats"]:
        """{output name: ResidualStats(abs_max, nrmse, sqnr_db)} of every MatMul, Conv without
        exponents, Pool and VectorOP node over the ramp inputs (_simulate.py:409-422)."""
        errors: Dict[str, residuals.ResidualStats] = {}
        self._forward_pass(self._build_ramp_inputs(), errors_out=errors)
        return errors

    # ------------------------------------------------------------------ residual statistics
    def _dev_values(self, t: TensorInfo, r: torch.Tensor) -> torch.Tensor:
        """float64 values of a raw device tensor, on the device, in the tensor's logical shape: a
        weight with a rank-1 exponent at raw * 2^-wexp (the value the reference's forward pass
        holds for it, _simulate.py:531-539), others at their own exponent(s)."""
        v = r.to(torch.float64)
        if t.kind == "f32":
            return v.reshape(t.shape)
        if t.group_layout is not None:
            KV, HD = t.group_layout
            v = v.reshape(KV, -1, HD).transpose(0, 1)
        v = v.reshape(t.shape)
        e = np.asarray(t.wexp, np.float64) if t.wexp is not None else np.asarray(self._exp_b(t), np.float64)
        return v * torch.as_tensor(np.power(2.0, -e), dtype=torch.float64, device=self.device)

    def _record_residuals(self, sn, raw: Dict[str, torch.Tensor]) -> None:
        """The node's ResidualStats into the collected statistics (_simulate.py:594-602, 620-765,
        814-835): its full-precision result in float64 on the device against the value its unit
        wrote.  Conv with exponents, reshapes, host and row-ops nodes record none, as in the
        reference."""
        ot = sn.output
        if isinstance(sn, (MatmulNode, MatmulConvNode)):
            at, bt = sn.inputs[0], sn.inputs[1]
            full = torch.matmul(self._dev_values(at, self._get(at, raw)), self._dev_values(bt, self._get(bt, raw)))
        elif isinstance(sn, ConvNode):
            if any(t is not None and (t.exp is not None or t.wexp is not None or t.chexp is not None)
                   for t in (sn.inputs[0], sn.inputs[1], ot)):
                return
            x = self._dev_values(sn.inputs[0], self._get(sn.inputs[0], raw))
            w = self._dev_values(sn.inputs[1], self._get(sn.inputs[1], raw))
            bias = self._dev_values(sn.inputs[2], self._get(sn.inputs[2], raw)) if sn.has_bias else None
            full = residuals.conv_full(x, w, bias, sn.stride_h, sn.stride_w, sn.pad_top, sn.pad_left, sn.dilation_h,
                                       sn.dilation_w, sn.out_h, sn.out_w, sn.is_depthwise)
        elif isinstance(sn, PoolNode):
            x = self._dev_values(sn.inputs[0], self._get(sn.inputs[0], raw))
            full = residuals.pool_full(x, sn.pool_h, sn.pool_w, sn.stride_h, sn.stride_w, sn.pad_top, sn.pad_left,
                                       sn.dil_h, sn.dil_w, int(ot.shape[2]), int(ot.shape[3]), sn.pool_type,
                                       sn.lp_order, sn.count_include_pad)
        elif type(sn) is ScheduledNode:
            a = self._dev_values(sn.inputs[0], self._get(sn.inputs[0], raw))
            b = self._dev_values(sn.inputs[1], self._get(sn.inputs[1], raw)) if sn.arity == 2 else None
            full, _ = residuals.vectorop_full(sn.op_code, sn.act, sn.alpha, a, b)
        else:
            return
        quant = self._dev_values(ot, raw[ot.onnx_name][:ot.numel])
        self._errors[ot.onnx_name] = residuals.residual_stats(full.reshape(ot.shape), quant)

    def _expected_storage(self, name: str, logical: np.ndarray) -> np.ndarray:
        """A tensor's values as the buffer lanes the board writes (_simulate.py:841-891): float32
        for a float32 tensor, int32 for the int32 residual, else the uint16 storage at the
        tensor's exponent(s) (integer tensors: their raw integers); contiguous (this simulator
        keeps no broadcast strides)."""
        t = self._tensor(name)
        flat = np.asarray(logical, np.float64).reshape(-1)
        if t.kind == "f32":
            return flat.astype(np.float32)
        if t.kind == "i32":
            e = np.asarray(0 if t.exp is None else t.exp, np.float64).reshape(-1)
            e = np.tile(e, flat.size // e.size) if e.size > 1 else e
            return np.clip(np.rint(flat * np.power(2.0, e)), -2 ** 31, 2 ** 31 - 1).astype(np.int32)
        if t.kind == "host":
            return flat.astype(np.int32)
        if t.exp is not None:
            e = np.asarray(t.exp, np.float64).reshape(-1)
            e = np.tile(e, flat.size // e.size) if e.size > 1 else e
            return self._dtype.exp_to_storage(flat, e)
        return self._dtype.float_to_storage(flat)

    def _emit_expected_c(self, c_name: str, storage_buf: np.ndarray) -> str:
        """``static const uint16_t expected_<c_name>[N]`` eight literals a row (_simulate.py:893-915)."""
        buf = np.asarray(storage_buf).reshape(-1)
        rows = ["    " + ", ".join(self._dtype.format_literal(v) for v in buf[i:i + 8]) for i in range(0, len(buf), 8)]
        inner = ",\n".join(rows)
        return f"static const uint16_t expected_{c_name}[{len(buf)}] = {{\n{inner}\n}};\n"

    def generate_expected_dat(self, tensor: TensorInfo) -> bytes:
        """The little-endian bytes of expected/<name>.dat: the tensor's ramp-input simulation as
        the storage lanes (_simulate.py:950-964)."""
        sim = self._simulate()
        buf = self._expected_storage(tensor.onnx_name, sim[tensor.onnx_name])
        return buf.astype(buf.dtype.newbyteorder("<")).tobytes()

    # ------------------------------------------------------------------ conversions
    def _tensor(self, name: str) -> TensorInfo:
        return self._infos[name]

    def _exp(self, t: TensorInfo):
        return self._dtype.frac_bits if t.exp is None else t.exp

    def _exp_b(self, t: TensorInfo):
        """The exponents broadcastable over the tensor: per channel of axis 1 (chexp), else
        scalar or per channel of the last axis."""
        if t.chexp is not None:
            return np.asarray(t.chexp, np.int64).reshape((1, -1) + (1,) * (len(t.shape) - 2))
        return self._exp(t)

    @staticmethod
    def _group_major(t: TensorInfo, logical: np.ndarray) -> np.ndarray:
        KV, HD = t.group_layout
        return np.ascontiguousarray(logical.reshape(-1, KV, HD).transpose(1, 0, 2))

    def _to_device(self, t: TensorInfo, values: np.ndarray):
        v = np.asarray(values, np.float64).reshape(t.shape)
        if t.kind == "host":                              # a host scalar / array (pos, n)
            return np.asarray(values).reshape(t.shape).astype(np.int64)
        if t.kind == "f32":
            r = v.astype(np.float32)
        elif t.kind == "i32":
            s = np.power(2.0, np.asarray(self._exp_b(t), np.float64))
            r = np.clip(np.round(v * s), -2 ** 31, 2 ** 31 - 1).astype(np.int32)
        else:
            r = self._dtype.to_raw(v, self._exp_b(t))
        if t.group_layout is not None:
            r = self._group_major(t, r)
        return torch.from_numpy(np.ascontiguousarray(r)).to(self.device)

    def _to_values(self, t: TensorInfo, raw) -> np.ndarray:
        if t.kind == "host":
            return np.asarray(raw, np.float64).reshape(t.shape)
        r = raw.detach().cpu().numpy()
        if t.group_layout is not None:
            KV, HD = t.group_layout
            r = r.reshape(KV, -1, HD).transpose(1, 0, 2)
        r = r.reshape(t.shape)
        if t.kind == "f32":
            return r.astype(np.float64)
        return self._dtype.from_raw(r, self._exp_b(t))

    def _get(self, t: TensorInfo, raw: Dict[str, torch.Tensor]) -> torch.Tensor:
        if t.onnx_name in raw:
            return raw[t.onnx_name]
        if t.data is None:
            raise KeyError(f"tensor '{t.onnx_name}' has no value (not an input, weight or node output)")
        w = self._weights.get(t.onnx_name)
        if w is None and t.raw:
            w = self._upload(np.asarray(t.data).astype(_NP[t.kind]))
            self._weights[t.onnx_name] = w
        if w is None:
            # a weight as the kernels read it (_simulate.py:531-539): quantized to the element
            # type's grid; with a rank-1 exponent the stored data is raw / 2^F, so its raw lanes
            # are the Q8.8 raw; otherwise the raw at the tensor's own exponent
            q = self._dtype.quantize(np.asarray(t.data, np.float64).reshape(t.shape))
            r = self._dtype.to_raw(q) if t.wexp is not None else self._dtype.to_raw(q, self._exp(t))
            w = self._upload(r)
            self._weights[t.onnx_name] = w
        return w

    def _upload(self, arr: np.ndarray) -> torch.Tensor:
        """A weight on the device in a buffer whose last 8-lane word is whole (zero lanes past
        the data), so that the VectorOP unit reads it in place (_padded)."""
        src = torch.from_numpy(np.ascontiguousarray(arr))
        buf = torch.zeros(_pad8(src.numel()), dtype=src.dtype, device=self.device)
        buf[:src.numel()].copy_(src.reshape(-1))
        return buf[:src.numel()].view(src.shape)

    def _new(self, t: TensorInfo, numel: Optional[int] = None) -> torch.Tensor:
        """An output buffer of `numel` lanes (the tensor's by default) with room for its last
        8-lane word, which the VectorOP unit reads whole (_padded)."""
        n = t.numel if numel is None else numel
        return torch.empty(_pad8(n), dtype=_TORCH[t.kind], device=self.device)[:n]

    @staticmethod
    def _padded(x: torch.Tensor, rows: int, n: int, n_pad: int) -> torch.Tensor:
        """Rows of n lanes at a stride of n_pad (the VectorOP unit's 8-lane words).  One row
        whose buffer holds the lanes past n (every _new / _upload buffer) is read in place: the
        unit's results in lanes below n do not depend on the lanes past it (element-wise ops;
        the softmax counts at most n valid scores), and its own lanes past n are not read back."""
        if n == n_pad:
            return x.reshape(-1).contiguous()
        if rows == 1 and x.is_contiguous() and x.dim() >= 1:
            lanes = x.untyped_storage().nbytes() // x.element_size()
            if x.storage_offset() + n_pad <= lanes:
                return torch.as_strided(x, (n_pad,), (1,), x.storage_offset())
        out = torch.zeros((rows, n_pad), dtype=x.dtype, device=x.device)
        out[:, :n] = x.reshape(rows, n)
        return out.reshape(-1)

    # ------------------------------------------------------------------ units
    def _pow2(self, *ts: TensorInfo) -> bool:
        return any(t is not None and (t.exp is not None or t.wexp is not None) for t in ts)

    def _matmul(self, sn: MatmulNode, raw) -> torch.Tensor:
        at, bt, ot = sn.inputs[0], sn.inputs[1], sn.output
        use = self._plan_planes()[0].get(id(sn))
        if use is not None and at.onnx_name + "#planes" in raw:
            # A's producer wrote its byte planes: only B's (split once) remain
            self._check_exponents(at, bt, ot)
            n, k, m = int(at.shape[-2]), int(at.shape[-1]), int(bt.shape[-1])
            c = self._new(ot, n * m)
            units.matmul_aplanes(raw[at.onnx_name + "#planes"], use[1], self._shared_b_planes(bt, self._get(bt, raw)),
                                 c, n, k, m, wrap32=self._pow2(at, bt, ot))
            return c
        a, b = self._get(at, raw), self._get(bt, raw)
        n, k = at.shape[-2], at.shape[-1]
        m = bt.shape[-1]
        if bt.shape[-2] != k:
            raise SchedulerError(f"MatMul: A [.., {n}, {k}] x B {list(bt.shape)}")
        a_batch = int(np.prod(at.shape[:-2])) if len(at.shape) > 2 else 1
        b_batch = int(np.prod(bt.shape[:-2])) if len(bt.shape) > 2 else 1
        batch = max(a_batch, b_batch)
        if a_batch not in (1, batch) or b_batch not in (1, batch):
            raise SchedulerError("MatMul: batch dimensions do not broadcast")
        wrap = self._pow2(at, bt, ot)
        if wrap:
            self._check_exponents(at, bt, ot)
        c = self._new(ot, batch * n * m)
        if bt.data is not None and b_batch == 1 and batch == 1 and wrap and n <= 16 and k % 8 == 0:
            # a decode-sized product: MFMA over the weight's split image, one launch
            units.matmul_skinny_planes(a.reshape(-1).contiguous(), n, k, [self._row_planes(bt, b, k, m)], [c], [m])
            return c
        if bt.data is not None and b_batch == 1 and batch == 1 and not wrap and n <= 32 and k % 8 == 0:
            # a classifier at a small batch: the saturating skinny products, 16 rows a launch
            af, planes = a.reshape(-1).contiguous(), self._row_planes(bt, b, k, m)
            for r0 in range(0, n, 16):
                rows = min(16, n - r0)
                units.matmul_skinny_planes(af[r0 * k:], rows, k, [planes], [c[r0 * m:]], [m], wrap32=False)
            return c
        if bt.data is not None and b_batch == 1 and wrap and n <= 32 and m % 2 == 0 and k % 8 == 0:
            # a decode-sized product: the library's skinny path reads the weight itself, kept
            # as its transposed image [m][k] (each column's k contiguous)
            units.matmul(a.reshape(-1).contiguous(), self._trans_image(bt, b, k, m), c, n, k, m, batch=batch,
                         a_bs=n * k if a_batch > 1 else 0, b_bs=0, c_bs=n * m, b_packed=2, wrap32=True)
            return c
        if bt.data is not None and b_batch == 1:
            # a shared weight: the packed image (the scheduler's packing), split once
            planes = self._shared_b_planes(bt, b)
            units.matmul_planes(a.reshape(-1).contiguous(), planes, c, n, k, m, batch=batch,
                                a_bs=n * k if a_batch > 1 else 0, c_bs=n * m, wrap32=wrap)
        else:
            units.matmul(a.reshape(-1).contiguous(), b.reshape(-1).contiguous(), c, n, k, m, batch=batch,
                         a_bs=n * k if a_batch > 1 else 0, b_bs=k * m if b_batch > 1 else 0,
                         c_bs=n * m, wrap32=wrap)
        return c

    def _shared_b_planes(self, bt: TensorInfo, b: torch.Tensor) -> torch.Tensor:
        """A constant 2-d weight's split image, from its packed image (the scheduler's packing), built once."""
        planes = self._images.get(bt.onnx_name)
        if planes is None:
            k, m = int(bt.shape[-2]), int(bt.shape[-1])
            img = torch.from_numpy(pack_matmul_b(b.cpu().numpy().reshape(k, m))).to(self.device)
            planes = units.matmul_b_planes(img, k, m, b_packed=1)
            self._images[bt.onnx_name] = planes
        return planes

    # ------------------------------------------------------------------ operands split by their producers
    def _plan_planes(self):
        """({id(MatMul): (A's name, partial sums)}, {A's name: (n, k, partial sums)}): the
        MatMuls of a constant 2-d weight on the plane path (not the skinny products) whose A,
        n x k with k a multiple of 64, comes from a node that can write A's byte planes as it
        writes A -- a whole-row NORM job, a VectorOP over rows of k, the fused attention."""
        if self._plan is not None:
            return self._plan
        prod = {sn.output.onnx_name: sn for sn in self._graph.nodes if getattr(sn, "output", None) is not None}
        consumers, producers = {}, {}
        for sn in self._graph.nodes:
            if not isinstance(sn, MatmulNode):
                continue
            at, bt, ot = sn.inputs[0], sn.inputs[1], sn.output
            if bt.data is None or len(bt.shape) != 2 or len(at.shape) != 2 or int(bt.shape[0]) != int(at.shape[1]):
                continue
            n, k = int(at.shape[0]), int(at.shape[1])
            if k % 64 or at.kind != "i16" or (self._pow2(at, bt, ot) and n <= 32):
                continue
            nsum = self._planes_sums(prod.get(at.onnx_name), n, k)
            if nsum is None or producers.get(at.onnx_name, (n, k, nsum)) != (n, k, nsum):
                continue
            consumers[id(sn)] = (at.onnx_name, nsum)
            producers[at.onnx_name] = (n, k, nsum)
        self._plan = (consumers, producers)
        return self._plan

    def _planes_sums(self, p, n: int, k: int) -> Optional[int]:
        """The partial row sums `p` would write with the planes of its n x k output, or None
        where it cannot write them."""
        if p is None:
            return None
        ot = p.output
        if isinstance(p, RowOpsAdapter) and getattr(p, "pos_t", None) is None:
            jobs = p.jobs()
            if (len(jobs) == 1 and jobs[0].op & 15 == units.RO_NORM and jobs[0].col0 == 0 and jobs[0].n == k
                    and jobs[0].b_row0 is None and not jobs[0].op & (1 << 14) and (jobs[0].op >> 8) & 3 == 0
                    and ot.kind == "i16" and p.inputs[0].numel == n * k and self._rows_whole(p, k)):
                return (k + 1023) // 1024
            return None
        if isinstance(p, AttentionNode):
            cols = p.heads * p.head_dim
            ok = (p.head_dim == 64 and p.seq in (64, 128, 256, 384) and cols == k and p.batch * p.seq == n
                  and int(p.inputs[0].shape[-1]) % 8 == 0 and p.q_off % 8 == 0 and p.k_off % 8 == 0
                  and p.v_off % 8 == 0 and p.heads <= 64)
            return p.heads if ok else None
        if isinstance(p, ScheduledNode) and p.op_code <= 9 and ot.numel == n * k and k <= 32768:
            if p.arity == 1:
                return (k + 1023) // 1024 if p.inputs[0].numel == n * k else None
            na, nb = p.inputs[0].numel, p.inputs[1].numel
            if max(na, nb) == n * k and min(na, nb) == k and n > 1:
                return (k + 1023) // 1024
        return None

    def _planes_out(self, sn) -> Optional[tuple]:
        """(n, k, partial sums) of the planes ``sn`` writes with its output, or None."""
        out = getattr(sn, "output", None)
        if out is None or isinstance(sn, MatmulNode):
            return None
        return self._plan_planes()[1].get(out.onnx_name)

    def _planes_only(self, name: str) -> bool:
        """True if forward_raw may leave ``name`` unwritten: the caller does not keep it, it is
        no graph output or state, and every node reading it is a MatMul on the plane path."""
        if self._keep is None or name in self._keep:
            return False
        if self._planes_only_names is None:
            plan = self._plan_planes()[0]
            readers: Dict[str, list] = {}
            for sn in self._graph.nodes:
                for t in getattr(sn, "inputs", []) or []:
                    if t is not None:
                        readers.setdefault(t.onnx_name, []).append(sn)
            fixed = {t.onnx_name for t in self._graph.output_tensors} | {t.onnx_name for t in self._graph.state_tensors}
            self._planes_only_names = {
                nm for nm, rs in readers.items()
                if nm not in fixed and all(id(r) in plan and plan[id(r)][0] == nm and r.inputs[0].onnx_name == nm
                                          and all(t is None or t.onnx_name != nm for t in r.inputs[1:]) for r in rs)}
        return name in self._planes_only_names

    def _planes_node(self, sn, raw) -> bool:
        """Run ``sn`` with the byte planes of its output as well (raw[name + '#planes']); False
        if it runs the plain way after all."""
        n, k, nsum = self._planes_out(sn)
        name = sn.output.onnx_name
        planes = units.a_planes(n, k, nsum, self.device)
        if isinstance(sn, RowOpsAdapter):
            at, ot = sn.inputs[0], sn.output
            a2d = self._get(at, raw).reshape(n, k)
            out = None if self._planes_only(name) else torch.empty((n, k), dtype=_TORCH[ot.kind], device=self.device)
            params = self._params.get(id(sn))
            if params is None:
                params = [torch.from_numpy(np.ascontiguousarray(sn.jobs()[0].params, np.uint8)).to(self.device)]
                self._params[id(sn)] = params
            units.rowops_jobs([self._whole_row_job(sn, a2d, None, out, params[0])], planes=planes)
            if out is not None:
                raw[name] = out.reshape(-1)
        elif isinstance(sn, AttentionNode):
            # o itself only where something besides the output projection's planes reads it
            self._attention(sn, raw, planes=planes, write_o=not self._planes_only(name))
            if self._attention_out is not None:
                raw[name] = self._attention_out
        else:
            a = self._get(sn.inputs[0], raw).reshape(-1).contiguous()
            # the int16 output only where something besides the plane-path MatMuls reads it
            c = None if self._planes_only(name) else self._new(sn.output, n * k)
            if sn.arity == 1:
                units.vectorop_planes(a, None, c, k, sn.op_code, n, k, 0, planes, act=sn.act, alpha=sn.alpha)
            else:
                b = self._get(sn.inputs[1], raw).reshape(-1).contiguous()
                a_inc, b_inc = (k, 0) if a.numel() == n * k else (0, k)
                units.vectorop_planes(a, b, c, k, sn.op_code, n, a_inc, b_inc, planes, act=sn.act, alpha=sn.alpha)
            if c is not None:
                raw[name] = c
        raw[name + "#planes"] = planes
        return True

    def _addx_norm_fusable(self, sn, nxt) -> bool:
        """``sn`` is a one-job COPY / ADDX adapter over whole rows writing int32 and ``nxt`` a
        one-job NORM adapter over the same whole rows reading that output: one chain call
        (cm_rowops_chain runs the pair as one launch)."""
        if not (isinstance(sn, RowOpsAdapter) and isinstance(nxt, RowOpsAdapter) and len(sn.inputs) == 2
                and len(nxt.inputs) == 1 and nxt.inputs[0].onnx_name == sn.output.onnx_name):
            return False
        if getattr(sn, "pos_t", None) is not None or getattr(nxt, "pos_t", None) is not None:
            return False
        ja, jn = sn.jobs(), nxt.jobs()
        if len(ja) != 1 or len(jn) != 1:
            return False
        ja, jn = ja[0], jn[0]
        width = sn.n
        return (ja.op & 15 in (units.RO_COPY, units.RO_ADDX) and jn.op & 15 == units.RO_NORM and ja.col0 == 0
                and jn.col0 == 0 and ja.n == width and jn.n == width and ja.b_row0 is None and jn.b_row0 is None
                and sn.output.kind == "i32" and sn.inputs[1].kind == "i16" and sn.inputs[0].kind in ("i16", "i32")
                and self._rows_whole(sn, width) and self._rows_whole(nxt, width) and width % 8 == 0
                and sn.inputs[0].numel == sn.output.numel == nxt.output.numel)

    def _addx_norm(self, sn: RowOpsAdapter, nxt: RowOpsAdapter, raw) -> None:
        """The residual add and the NORM of its output as one chain (and the NORM's byte planes
        when a MatMul takes its output as A)."""
        width = sn.n
        rows = sn.output.numel // width
        pl = self._planes_out(nxt)
        jobs = []
        for node in (sn, nxt):
            params = self._params.get(id(node))
            if params is None:
                params = [torch.from_numpy(np.ascontiguousarray(node.jobs()[0].params, np.uint8)).to(self.device)]
                self._params[id(node)] = params
            a2d = (self._get(node.inputs[0], raw) if node is sn else out1).reshape(rows, width)
            b_all = self._get(node.inputs[1], raw) if len(node.inputs) > 1 else None
            # the NORM's rows only where something besides the next MatMul's planes reads them
            skip = node is nxt and pl is not None and self._planes_only(node.output.onnx_name)
            out = None if skip else torch.empty((rows, width), dtype=_TORCH[node.output.kind], device=self.device)
            jobs.append(self._whole_row_job(node, a2d, b_all, out, params[0]))
            if node is sn:
                out1 = out
            if out is not None:
                raw[node.output.onnx_name] = out.reshape(-1)
        planes = units.a_planes(*pl, self.device) if pl is not None else None
        units.rowops_jobs(jobs, planes=planes)
        if planes is not None:
            raw[nxt.output.onnx_name + "#planes"] = planes

    def _embed(self, sn: LlmEmbedNode, raw) -> torch.Tensor:
        """The embedding rows gathered on the device from the output-lane image of the table."""
        key = f"{id(sn)}#embed"
        img = self._images.get(key)
        if img is None:
            img = torch.from_numpy(sn.image()).to(self.device)
            self._images[key] = img
        ids = self._get(sn.inputs[0], raw)
        if not isinstance(ids, torch.Tensor):                 # host ids (an i32 host tensor)
            ids = torch.from_numpy(np.asarray(ids, np.int64).reshape(-1).astype(np.int32)).to(self.device)
        ids = ids.reshape(-1).contiguous()
        out = self._new(sn.output)
        units.embed_rows(img, ids, out, sn.rows, sn.d)
        return out

    def _host_node(self, sn: HostNode, raw) -> torch.Tensor:
        """A host op (host_ops): host copies of its inputs' values, the node's reference(), the
        result (and every state it updated in place) back on the device."""
        ins = []
        for t in sn.inputs:
            v = self._get(t, raw)
            ins.append(np.asarray(v) if t.kind == "host" else self._to_values(t, v))
        y = sn.reference(ins, self._dtype)
        for t, v in zip(sn.inputs, ins):
            if t.state:
                dev = self._get(t, raw)
                dev.copy_(self._to_device(t, v).reshape(dev.shape))
        return self._to_device(sn.output, y).reshape(-1)

    def _matmul_conv(self, sn: MatmulConvNode, raw) -> torch.Tensor:
        """A MatMul on the conv unit (nodes.py:1712-1756): weight = A's rows, x = B's conv image,
        one call, or one per batch item when both operands are batched."""
        at, bt, ot = sn.inputs[0], sn.inputs[1], sn.output
        wrap = self._pow2(at, bt, ot)
        if wrap:
            self._check_exponents(at, bt, ot)
        a = self._get(at, raw).reshape(-1).contiguous()
        b = self._get(bt, raw).reshape(-1)
        if sn.kw > 1:                              # a constant B re-laid once
            key = f"{bt.onnx_name}#conv_kw{sn.kw}"
            img = self._images.get(key)
            if img is None:
                img = torch.from_numpy(conv_lowered_b_image(b.cpu().numpy(), sn.k, sn.m, sn.kw)).to(self.device)
                self._images[key] = img
        else:
            img = b.contiguous()
        c = self._new(ot)
        per = 1 if sn.calls > 1 else 0
        for i in range(sn.calls):
            units.conv(img[i * per * sn.b_batch_stride:], a[i * per * sn.a_batch_stride:], None,
                       c[i * per * sn.c_batch_stride:], sn.conv_batch, sn.in_ch, sn.in_h, sn.in_w, sn.conv_n,
                       sn.out_h, sn.out_w, 1, sn.kw, 1, sn.kw, wrap32=wrap)
        return c

    def _skinny_planes_ok(self, sn) -> bool:
        """A MatMul the skinny plane kernel takes: a constant 2-d pow2 weight, one slice of A of
        at most 16 rows, k a multiple of 8."""
        if not isinstance(sn, MatmulNode):
            return False
        at, bt, ot = sn.inputs[0], sn.inputs[1], sn.output
        if bt.data is None or len(at.shape) > 2 or len(bt.shape) != 2 or bt.shape[0] != at.shape[-1]:
            return False
        return self._pow2(at, bt, ot) and int(at.shape[-2]) <= 16 and int(at.shape[-1]) % 8 == 0

    def _output_job_fusable(self, sn, nxt) -> bool:
        """``nxt`` is a one-job COPY / ADDX adapter over whole rows whose B is the skinny
        MatMul ``sn``'s output (and whose A is another tensor): the pair runs as one launch."""
        if not self._ram_free:
            return False
        if not (self._skinny_planes_ok(sn) and isinstance(nxt, RowOpsAdapter) and len(nxt.inputs) == 2
                and getattr(nxt, "pos_t", None) is None and getattr(nxt, "table", None) is None):
            return False
        xt, bt, ot = nxt.inputs[0], nxt.inputs[1], nxt.output
        n, m = int(sn.inputs[0].shape[-2]), int(sn.inputs[1].shape[-1])
        if bt.onnx_name != sn.output.onnx_name or xt.onnx_name == sn.output.onnx_name:
            return False
        if xt.kind not in ("i16", "i32") or ot.kind not in ("i16", "i32") or xt.numel != n * m or ot.numel != n * m:
            return False
        jobs = nxt.jobs()
        if len(jobs) != 1:
            return False
        j = jobs[0]
        code = j.op & 15
        return (j.col0 == 0 and j.n == m and j.b_row0 is None and code in (units.RO_COPY, units.RO_ADDX)
                and (j.op >> 6) & 3 == 0 and not (j.op & (1 << 14)))

    def _matmul_output_job(self, sn: MatmulNode, nxt: RowOpsAdapter, raw) -> None:
        """The skinny MatMul and its output's row-ops job in one launch; both outputs kept."""
        at, bt, ot = sn.inputs[0], sn.inputs[1], sn.output
        self._check_exponents(at, bt, ot)
        n, k, m = int(at.shape[-2]), int(at.shape[-1]), int(bt.shape[-1])
        a = self._get(at, raw).reshape(-1).contiguous()
        c = self._new(ot, n * m)
        j = nxt.jobs()[0]
        params = self._params.get(id(nxt))
        if params is None:
            params = [torch.from_numpy(np.ascontiguousarray(j.params, np.uint8)).to(self.device)]
            self._params[id(nxt)] = params
        x = self._get(nxt.inputs[0], raw).reshape(-1).contiguous()
        out = self._new(nxt.output)
        units.matmul_skinny_planes_addx(a, n, k, self._row_planes(bt, self._get(bt, raw), k, m), c, m, x, params[0],
                                        j.op, out, bq_sh=j.bq_sh)
        raw[ot.onnx_name] = c
        raw[nxt.output.onnx_name] = out

    def _row_planes(self, bt: TensorInfo, b: torch.Tensor, k: int, m: int) -> torch.Tensor:
        """A weight's split image (byte planes and column sums) from its row-major lanes, built once."""
        img = self._images.get(bt.onnx_name + "#planes")
        if img is None:
            img = units.matmul_b_planes(b.reshape(-1).contiguous(), k, m)
            self._images[bt.onnx_name + "#planes"] = img
        return img

    def _trans_image(self, bt: TensorInfo, b: torch.Tensor, k: int, m: int) -> torch.Tensor:
        """A weight's transposed image [m][k], built once."""
        img = self._images.get(bt.onnx_name + "#trans")
        if img is None:
            wt = np.ascontiguousarray(b.cpu().numpy().reshape(k, m).T)
            img = torch.from_numpy(wt).to(self.device)
            self._images[bt.onnx_name + "#trans"] = img
        return img

    def _skinny_single(self, sn) -> bool:
        """A MatMul of one slice the skinny path takes: a constant pow2 weight, at most 32 rows."""
        if not isinstance(sn, MatmulNode):
            return False
        at, bt, ot = sn.inputs[0], sn.inputs[1], sn.output
        if bt.data is None or len(at.shape) > 2 or len(bt.shape) > 2 or bt.shape[-2] != at.shape[-1]:
            return False
        n, k, m = int(at.shape[-2]), int(at.shape[-1]), int(bt.shape[-1])
        return self._pow2(at, bt, ot) and n <= 32 and m % 2 == 0 and k % 8 == 0

    def _matmul_group(self, group, raw) -> None:
        """Consecutive skinny MatMuls of the same A (q / k / v, gate / up) in one launch, each
        output as _matmul would give it."""
        at = group[0].inputs[0]
        a = self._get(at, raw).reshape(-1).contiguous()
        n, k = int(at.shape[-2]), int(at.shape[-1])
        planes = n <= 16
        bs, cs, ms = [], [], []
        for sn in group:
            bt, ot = sn.inputs[1], sn.output
            self._check_exponents(at, bt, ot)
            m = int(bt.shape[-1])
            b = self._get(bt, raw)
            bs.append(self._row_planes(bt, b, k, m) if planes else self._trans_image(bt, b, k, m))
            cs.append(self._new(ot, n * m))
            ms.append(m)
        if planes:
            units.matmul_skinny_planes(a, n, k, bs, cs, ms)
        else:
            units.matmul_skinny_multi(a, n, k, bs, cs, ms, b_packed=2)
        for sn, c in zip(group, cs):
            raw[sn.output.onnx_name] = c

    def _mulact_fusable(self, group, nxt) -> bool:
        """``nxt`` is a one-job MULACT adapter over whole rows of the two skinny plane products
        in ``group`` (gate first, then up, m columns each): the three run as one launch."""
        if not self._ram_free:
            return False
        if len(group) != 2 or not isinstance(nxt, RowOpsAdapter) or len(nxt.inputs) != 2:
            return False
        if getattr(nxt, "pos_t", None) is not None or getattr(nxt, "table", None) is not None:
            return False
        if not all(self._skinny_planes_ok(sn) for sn in group):
            return False
        g, u = group
        n, m = int(g.inputs[0].shape[-2]), int(g.inputs[1].shape[-1])
        if int(u.inputs[1].shape[-1]) != m or nxt.output.kind != "i16" or nxt.output.numel != n * m:
            return False
        if nxt.inputs[0].onnx_name != g.output.onnx_name or nxt.inputs[1].onnx_name != u.output.onnx_name:
            return False
        jobs = nxt.jobs()
        if len(jobs) != 1:
            return False
        j = jobs[0]
        return (j.op & 15 == units.RO_MULACT and j.col0 == 0 and j.n == m and j.b_row0 is None
                and (j.op >> 4) & 63 == 0 and not (j.op & units.F_P_KEEP) and bool(j.op & units.F_B_EN))

    def _matmul_mulact(self, group, nxt: RowOpsAdapter, raw) -> None:
        """The gate and up products and the MULACT job over them in one launch; all outputs kept."""
        g, u = group
        at = g.inputs[0]
        n, k, m = int(at.shape[-2]), int(at.shape[-1]), int(g.inputs[1].shape[-1])
        for sn in group:
            self._check_exponents(at, sn.inputs[1], sn.output)
        a = self._get(at, raw).reshape(-1).contiguous()
        bs = [self._row_planes(sn.inputs[1], self._get(sn.inputs[1], raw), k, m) for sn in group]
        cg, cu = self._new(g.output, n * m), self._new(u.output, n * m)
        j = nxt.jobs()[0]
        params = self._params.get(id(nxt))
        if params is None:
            params = [torch.from_numpy(np.ascontiguousarray(j.params, np.uint8)).to(self.device)]
            self._params[id(nxt)] = params
        out = self._new(nxt.output)
        units.matmul_skinny_planes_mulact(a, n, k, bs[0], bs[1], cg, cu, m, params[0], j.op, out)
        raw[g.output.onnx_name] = cg
        raw[u.output.onnx_name] = cu
        raw[nxt.output.onnx_name] = out

    def _check_exponents(self, at: TensorInfo, bt: TensorInfo, ot: TensorInfo) -> None:
        """Every product of column j must sit at 2^-(f_out[j] + F) (_simulate.py:821-827)."""
        F = self._dtype.frac_bits
        k, m = bt.shape[-2], bt.shape[-1]
        fa = np.broadcast_to(at.exp_full(F).reshape(-1) if np.ndim(at.exp_full(F)) else at.exp_full(F), (k,))
        fw = np.broadcast_to(bt.wexp if bt.wexp is not None else bt.exp_full(F), (k, m))
        fo = np.broadcast_to(ot.exp_full(F), (m,))
        if not np.array_equal(fa[:, None] + fw, np.broadcast_to(fo[None, :] + F, (k, m))):
            raise ValueError("MatMul: exponents are inconsistent (accumulator not on the 2^-(f_out+F) grid)")

    def _reader_counts(self) -> Dict[str, int]:
        """How many nodes read each tensor."""
        if getattr(self, "_readers_n", None) is None:
            n: Dict[str, int] = {}
            for sn in self._graph.nodes:
                for t in getattr(sn, "inputs", []) or []:
                    if t is not None:
                        n[t.onnx_name] = n.get(t.onnx_name, 0) + 1
            self._readers_n = n
        return self._readers_n

    def _conv_act_fusable(self, sn, nxt) -> bool:
        """``sn`` a Q8.8 convolution whose output only ``nxt``, a unary RELU / RELU6 VectorOP of
        plain Q8.8 tensors without an act of its own, reads, and which the caller does not keep:
        the convolution applies the activation as it stores (cm_conv_act) and writes ``nxt``'s
        output alone -- the two unit calls' result, with the intermediate never written."""
        if not (isinstance(sn, ConvNode) and isinstance(nxt, ScheduledNode) and nxt.arity == 1
                and nxt.op_code in (units.OP_RELU, units.OP_RELU6) and nxt.act == units.ACT_NONE):
            return False
        ct = sn.output
        if self._keep is None or ct.onnx_name in self._keep or nxt.inputs[0].onnx_name != ct.onnx_name:
            return False
        if nxt.output.numel != ct.numel or self._pow2(*sn.inputs[:2], ct) or self._planes_out(nxt) is not None:
            return False
        for t in (ct, nxt.output):
            if t.exp is not None or t.chexp is not None or t.kind != "i16" or t.state:
                return False
        fixed = {t.onnx_name for t in self._graph.output_tensors}
        return ct.onnx_name not in fixed and self._reader_counts().get(ct.onnx_name, 0) == 1

    def _conv(self, sn: ConvNode, raw, act: int = 0, out_t=None) -> torch.Tensor:
        """The convolution; with ``act`` (RELU / RELU6) the activated result, stored as ``out_t``."""
        xt, wt, ot = sn.inputs[0], sn.inputs[1], sn.output
        bias_t = sn.inputs[2] if sn.has_bias else None
        x = self._get(xt, raw)
        img = self._images.get(wt.onnx_name)
        if img is None:
            w = self._get(wt, raw).cpu().numpy().reshape(wt.shape)
            img = torch.from_numpy(conv_weight_image(w, sn.is_depthwise)).to(self.device)
            if not sn.is_depthwise and wt.data is not None and not units.conv_small(sn.in_ch, sn.kh, sn.kw, sn.out_ch, sn.batch):
                # a constant weight of a standard convolution on the GEMM: its operand split once
                img = units.conv_w_planes(img, sn.out_ch, sn.in_ch, sn.kh, sn.kw)
            self._images[wt.onnx_name] = img
        bias = None
        if bias_t is not None:
            key = bias_t.onnx_name + "#bias"
            bias = self._images.get(key)
            if bias is None:
                bias = torch.from_numpy(conv_bias_image(self._get(bias_t, raw).cpu().numpy())).to(self.device)
                self._images[key] = bias
        y = self._new(ot if out_t is None else out_t)
        if img.dtype == torch.uint8:
            units.conv_planes(x.reshape(-1).contiguous(), img, bias, y, sn.batch, sn.in_ch, sn.in_h, sn.in_w,
                              sn.out_ch, sn.out_h, sn.out_w, sn.kh, sn.kw, sn.stride_h, sn.stride_w, sn.dilation_h,
                              sn.dilation_w, sn.pad_top, sn.pad_left, int(bias is not None),
                              wrap32=self._pow2(xt, wt, ot), act=act)
            return y
        units.conv(x.reshape(-1).contiguous(), img, bias, y, sn.batch, sn.in_ch, sn.in_h, sn.in_w, sn.out_ch,
                   sn.out_h, sn.out_w, sn.kh, sn.kw, sn.stride_h, sn.stride_w, sn.dilation_h, sn.dilation_w,
                   sn.pad_top, sn.pad_left, int(bias is not None), int(sn.is_depthwise),
                   wrap32=self._pow2(xt, wt, ot), act=act)
        return y

    def _pool(self, sn: PoolNode, raw) -> torch.Tensor:
        xt, ot = sn.inputs[0], sn.output
        y = self._new(ot)
        units.pool(self._get(xt, raw).reshape(-1).contiguous(), y, xt.shape[0], xt.shape[1], xt.shape[2],
                   xt.shape[3], ot.shape[2], ot.shape[3], sn.pool_h, sn.pool_w, sn.stride_h, sn.stride_w,
                   sn.pad_top, sn.pad_left, sn.dil_h, sn.dil_w, sn.pool_type, sn.lp_order,
                   sn.count_include_pad)
        return y

    def _vectorop(self, sn: ScheduledNode, raw) -> torch.Tensor:
        """_simulate.py:721-765: both operands at the element type's grid; a smaller operand
        repeats over leading blocks (nodes.py:226-303)."""
        ot = sn.output
        a = self._get(sn.inputs[0], raw).reshape(-1)
        total = ot.numel
        c = self._new(ot, _pad8(total))
        if sn.arity == 1:
            if a.numel() != total:
                raise SchedulerError("unary VectorOP: input and output sizes differ")
            units.vectorop(self._padded(a, 1, total, _pad8(total)), None, c, total, sn.op_code,
                           act=sn.act, alpha=sn.alpha)
            return c[:total]
        b = self._get(sn.inputs[1], raw).reshape(-1)
        na, nb = a.numel(), b.numel()
        if total % na or total % nb or max(na, nb) != total:
            raise SchedulerError(f"VectorOP: operands of {na} and {nb} elements onto {total}")
        small = min(na, nb)
        if small == total:
            units.vectorop(self._padded(a, 1, total, _pad8(total)), self._padded(b, 1, total, _pad8(total)),
                           c, total, sn.op_code, act=sn.act, alpha=sn.alpha)
            return c[:total]
        outer = total // small
        if small % 8 == 0:
            # broadcast through the registers: the repeated operand has increment 0
            a_inc, b_inc = (small, 0) if na == total else (0, small)
            units.vectorop(a.contiguous(), b.contiguous(), c, small, sn.op_code, outer=outer, a_inc=a_inc,
                           b_inc=b_inc, act=sn.act, alpha=sn.alpha)
            return c[:total]
        # a chunk that is not a whole number of 8-lane words: repeat it in memory
        if na < total:
            a = a.repeat(outer)
        else:
            b = b.repeat(outer)
        units.vectorop(self._padded(a, 1, total, _pad8(total)), self._padded(b, 1, total, _pad8(total)), c,
                       total, sn.op_code, act=sn.act, alpha=sn.alpha)
        return c[:total]

    def _softmax(self, sn: SoftmaxVopNode, raw) -> torch.Tensor:
        xt, ot = sn.inputs[0], sn.output
        x = self._get(xt, raw)
        if not sn.keys_major:
            n = xt.shape[-1]
            rows = xt.numel // n
            np8 = _pad8(n)
            c = torch.empty(rows * np8, dtype=torch.int16, device=self.device)
            units.vectorop(self._padded(x, rows, n, np8), None, c, n, units.OP_SOFTMAX, outer=rows, a_inc=np8,
                           b_inc=np8, smx_cm=sn.cm, smx_cfg=sn.cfg,
                           smx_mask=sn.mask_reg(n, self._host_int(sn.mask_t, raw)))
            return c.reshape(rows, np8)[:, :n].reshape(-1).contiguous()
        keys, queries = xt.shape[-2], xt.shape[-1]
        heads = xt.numel // (keys * queries)
        if queries % 16:
            raise SchedulerError("keys-major softmax: the query count must be a multiple of 16")
        kp = _pad8(keys)
        out = torch.empty(heads * queries * kp, dtype=torch.int16, device=self.device)
        units.softmax(x.reshape(-1).contiguous(), out, keys, units.OP_SOFTMAX_T, queries, queries, kp, sn.cm, sn.cfg,
                      sn.mask_reg(keys, self._host_int(sn.mask_t, raw)), batch=heads, a_bs=keys * queries,
                      c_bs=queries * kp)
        return out.reshape(heads * queries, kp)[:, :keys].reshape(-1).contiguous()

    def _rowops(self, sn: RowOpsNode, raw) -> torch.Tensor:
        """One job over [rows, n] tensors; rows are re-laid at 16-byte strides."""
        at, ot = sn.inputs[0], sn.output
        bt = sn.inputs[1] if len(sn.inputs) > 1 else None
        n = at.shape[-1]
        rows = at.numel // n
        kb = {"i16": 2, "i32": 4, "f32": 4}

        def rowbuf(t: Optional[TensorInfo], x: Optional[torch.Tensor], width: int):
            stride = (kb[t.kind] * width + 15) & ~15
            per = stride // kb[t.kind]
            buf = torch.zeros(rows * per, dtype=_TORCH[t.kind], device=self.device)
            if x is not None:
                buf.view(rows, per)[:, :width] = x.reshape(rows, width)
            return buf, stride, per

        a_buf, a_s1, _ = rowbuf(at, self._get(at, raw), n)
        b_buf, b_s1 = None, 0
        if bt is not None:
            b_buf, b_s1, _ = rowbuf(bt, self._get(bt, raw), bt.shape[-1])
        c_buf, c_s1, c_per = rowbuf(ot, None, ot.shape[-1])
        p = torch.from_numpy(np.ascontiguousarray(sn.params, np.uint8)).to(self.device)
        as_u8 = lambda t: t.view(torch.uint8) if t is not None else None
        units.rowops(as_u8(a_buf), as_u8(b_buf), as_u8(c_buf), p, sn.op, n, rows, 1, a_s1, 0, b_s1, 0,
                     c_s1, 0, sn.eps, sn.aux, sn.bq_sh, sn.win_lo, sn.win_hi)
        return c_buf.view(rows, c_per)[:, :ot.shape[-1]].reshape(-1).contiguous()

    def _attn_conv(self, sn: LlmAttnConvNode, raw) -> torch.Tensor:
        """q.K^T / P.V of one KV group over keys = roundup(pos + n, Q) keys: a raw int16
        matmul with the int32-wrap output rule on the group-major caches."""
        if sn.static:
            keys = sn.C
        else:
            pos = int(np.asarray(self._get(sn.inputs[2], raw)).reshape(-1)[0])
            n = int(np.asarray(self._get(sn.inputs[3], raw)).reshape(-1)[0]) if sn.has_n else sn.T
            keys = attn_keys(pos, n, sn.T, sn.C, sn.Q)[1]
        g, HD, GT, C = sn.group, sn.HD, sn.G * sn.T, sn.C
        w, x = sn.inputs[0], sn.inputs[1]
        if sn.kind == "qk":
            if w.group_layout != (sn.KV, HD):
                raise SchedulerError("q.K^T: the K cache must be stored group-major")
            kc = self._get(w, raw).reshape(sn.KV, C, HD)[g, :keys]
            qx = self._get(x, raw).reshape(sn.KV, HD, GT)[g]
            out = torch.zeros((C, GT), dtype=torch.int16, device=self.device)
            units.matmul(kc.reshape(-1), qx.reshape(-1).contiguous(), out.reshape(-1), keys, HD, GT, wrap32=True)
            return out.reshape(-1)
        if x.group_layout != (sn.KV, HD):
            raise SchedulerError("P.V: the V cache must be stored group-major")
        p = self._get(w, raw).reshape(GT, C)[:, :keys].contiguous()
        vc = self._get(x, raw).reshape(sn.KV, C, HD)[g, :keys]
        out = torch.empty(GT * HD, dtype=torch.int16, device=self.device)
        units.matmul(p.reshape(-1), vc.reshape(-1), out, GT, keys, HD, wrap32=True)
        return out

    def _attn_softmax(self, sn: AttnSoftmaxNode, raw) -> torch.Tensor:
        """The prefill softmax of one KV group over keys = roundup(pos + n, Q): one column-mode
        call over the group's G T query columns (the mask's period T restarts the causal valid
        length at each head), or one call per head where their registers differ; P is zero past
        the keys."""
        T, C = sn.T, sn.C
        GT = sn.G * T
        pos, n_in = sn.pos_n(lambda t: self._host_int(t, raw))
        n, keys = attn_keys(pos, n_in, T, C, sn.Q)
        s = self._get(sn.inputs[0], raw).reshape(-1)
        out = torch.zeros(GT * C, dtype=torch.int16, device=self.device)
        mask = sn.mask_reg(pos, n, keys)
        regs = sn.regs()
        if len(set(regs)) == 1:
            units.softmax(s, out, keys, units.OP_SOFTMAX_T, GT, GT, C, regs[0][0], regs[0][1], mask)
        else:
            for h, (cm_h, cfg_h) in enumerate(regs):
                units.softmax(s[h * T:], out[h * T * C:], keys, units.OP_SOFTMAX_T, T, GT, C, cm_h, cfg_h, mask)
        return out

    def _attn_merge(self, sn: AttnMergeNode, raw) -> torch.Tensor:
        """Each group's P.V rows [G T][HD] copied into their heads' columns of pv [T][H HD]."""
        T, H, HD = sn.T, sn.H, sn.HD
        G = H // sn.KV
        out = self._new(sn.output)
        for g, t in enumerate(sn.inputs):
            units.copy16(self._get(t, raw).reshape(-1), out[g * G * HD:], (1, G, T, HD), (0, T * HD, HD, 1),
                         (0, HD, H * HD, 1))
        return out

    def _select_row(self, sn: SelectRowNode, raw) -> torch.Tensor:
        """Row n - 1 of h (n clamped to 1 .. rows) into the output, in place where it is a state."""
        h, ot = sn.inputs[0], sn.output
        w = int(h.shape[-1])
        r = min(max(self._host_int(sn.inputs[1], raw), 1), sn.rows) - 1
        x = self._get(h, raw).reshape(-1)
        out = raw.get(ot.onnx_name)
        if out is None:
            out = self._new(ot)
        lanes = x.element_size() // 2                   # int16 lanes per element
        units.copy16(x.view(torch.int16)[r * w * lanes:], out.reshape(-1).view(torch.int16), (1, 1, 1, w * lanes),
                     (0, 0, 0, 1), (0, 0, 0, 1))
        return out

    def _attn_contract(self, sn: AttnContractNode, raw) -> torch.Tensor:
        at, bt, ot = sn.inputs[0], sn.inputs[1], sn.output
        batch, n, k = sn.operand_shape(0)
        b3 = sn.operand_shape(1)
        kb, mb = (2, 1) if sn.b_trans else (1, 2)
        m = b3[mb]
        if b3[0] != batch or b3[kb] != k or sn.operand_shape(2) != (batch, n, m):
            raise SchedulerError(f"attention contraction '{ot.onnx_name}': [b][n][k] x [b][k][m] -> [b][n][m]")
        fa, fb, fo = (self._view_exp(t, v, ot) for t, v in ((at, sn.a_view), (bt, sn.b_view), (ot, sn.c_view)))
        if fo != fa + fb - self._dtype.frac_bits:
            raise SchedulerError(f"attention contraction '{ot.onnx_name}': output exponent is not f_a + f_b - 8")
        a, b = self._get(at, raw).reshape(-1), self._get(bt, raw).reshape(-1)
        c = self._new(ot)
        if sn.a_view is None and sn.b_view is None and sn.c_view is None:
            units.matmul(a.contiguous(), b.contiguous(), c, n, k, m, batch=batch, a_bs=n * k, b_bs=k * m,
                         c_bs=n * m, b_packed=2 if sn.b_trans else 0, wrap32=True)
            return c
        inner = next(v.heads for v in (sn.a_view, sn.b_view, sn.c_view) if v is not None)
        def view(t, v, rows, cols):
            if v is None:
                return (0, cols, inner * rows * cols, rows * cols)   # slice bt at bt rows cols
            if v.heads != inner:
                raise SchedulerError(f"attention contraction '{ot.onnx_name}': head views of different head counts")
            return v.strides(int(t.shape[-1]))
        units.matmul_strided(a, b, c, n, k, m, batch, inner, view(at, sn.a_view, n, k),
                             view(bt, sn.b_view, *((m, k) if sn.b_trans else (k, m))), view(ot, sn.c_view, n, m),
                             b_trans=sn.b_trans, wrap32=True)
        return c

    def _view_exp(self, t: TensorInfo, v, ot: TensorInfo) -> int:
        """The one exponent of a contraction operand: the tensor's, or a head view's columns'."""
        e = np.asarray(self._exp(t)).reshape(-1)
        if v is not None and e.size > 1:
            e = np.broadcast_to(e, (int(t.shape[-1]),))[v.col:v.col + v.heads * v.width]
        if e.size == 0 or (e != e[0]).any():
            raise SchedulerError(f"attention contraction '{ot.onnx_name}': operand '{t.onnx_name}' at one exponent")
        return int(e[0])

    def _permute(self, sn: PermuteNode, raw) -> torch.Tensor:
        xt, ot = sn.inputs[0], sn.output
        if xt.kind != "i16" or ot.kind != "i16" or int(np.prod(sn.dims)) != ot.numel:
            raise SchedulerError(f"Permute '{ot.onnx_name}': int16 tensors, dims covering the output")
        x = self._get(xt, raw).reshape(-1)
        out = self._new(ot)
        units.permute16(x[int(sn.offset):], out, sn.dims, sn.strides)
        return out

    @staticmethod
    def _rows_whole(sn: RowOpsAdapter, width: int) -> bool:
        """Every tensor of the adapter has rows of whole 16-byte words."""
        ts = [sn.inputs[0], sn.output] + ([sn.inputs[1]] if len(sn.inputs) > 1 else [])
        if getattr(sn, "table", None) is not None:
            return False
        return all((width * _KB[t.kind]) % 16 == 0 and int(t.shape[-1]) == width for t in ts)

    def _rows16(self, x2d: torch.Tensor, kind: str):
        """[rows][w] lanes re-laid at a 16-byte row stride: (buffer, stride bytes, lanes per row)."""
        rows, w = x2d.shape
        per = ((_KB[kind] * w + 15) & ~15) // _KB[kind]
        buf = torch.zeros((rows, per), dtype=_TORCH[kind], device=self.device)
        buf[:, :w] = x2d
        return buf, per * _KB[kind], per

    def _attention(self, sn: AttentionNode, raw, planes: Optional[torch.Tensor] = None,
                   write_o: bool = True) -> Optional[torch.Tensor]:
        """An encoder layer's attention: one cm_attention call (with ``planes``, cm_attention_planes:
        o's byte planes as well, and with ``write_o`` False the planes alone: None returned), or
        (shapes it does not take) the head split, the two contractions and the softmax unit
        call by call."""
        xt, ot = sn.inputs[0], sn.output
        B, T, H, hd = sn.batch, sn.seq, sn.heads, sn.head_dim
        ld, cols = int(xt.shape[-1]), sn.heads * sn.head_dim
        if list(xt.shape) != [B * T, ld] or list(ot.shape) != [B * T, cols]:
            raise SchedulerError(f"attention '{ot.onnx_name}': qkv [{B * T}][ld] -> o [{B * T}][{cols}]")
        fx = np.broadcast_to(np.asarray(self._exp(xt)).reshape(-1), (ld,))
        f = {}
        for key, off in (("q", sn.q_off), ("k", sn.k_off), ("v", sn.v_off)):
            e = fx[off:off + cols]
            if e.size != cols or (e != e[0]).any():
                raise SchedulerError(f"attention '{ot.onnx_name}': {key} columns at one exponent")
            f[key] = int(e[0])
        fo = np.asarray(self._exp(ot)).reshape(-1)
        fp = (sn.cfg >> 8) & 31
        if fo.size != 1 or int(fo[0]) != fp + f["v"] - self._dtype.frac_bits:
            raise SchedulerError(f"attention '{ot.onnx_name}': output exponent is not f_p + f_v - 8")
        x = self._get(xt, raw).reshape(-1)
        o = self._new(ot) if write_o or planes is None else None
        if (hd == 64 and T in (64, 128, 256, 384) and ld % 8 == 0 and cols % 8 == 0
                and sn.q_off % 8 == 0 and sn.k_off % 8 == 0 and sn.v_off % 8 == 0):
            if planes is not None:
                units.attention_planes(x, o, B, T, H, hd, ld, sn.q_off, sn.k_off, sn.v_off, sn.cm, sn.cfg, planes)
                self._attention_out = o
                return o
            units.attention(x, o, B, T, H, hd, ld, sn.q_off, sn.k_off, sn.v_off, cols, sn.cm, sn.cfg)
            return o
        if planes is not None:
            raise SchedulerError(f"attention '{ot.onnx_name}': no planes for this shape")
        if T % 16:
            raise SchedulerError(f"attention '{ot.onnx_name}': the keys-major softmax takes query blocks of 16")
        BH, dev = B * H, self.device
        qT = torch.empty(BH * hd * T, dtype=torch.int16, device=dev)
        kh = torch.empty(BH * T * hd, dtype=torch.int16, device=dev)
        vh = torch.empty(BH * T * hd, dtype=torch.int16, device=dev)
        units.permute16(x[sn.q_off:], qT, (B, H, hd, T), (T * ld, hd, 1, ld))
        units.permute16(x[sn.k_off:], kh, (B, H, T, hd), (T * ld, hd, ld, 1))
        units.permute16(x[sn.v_off:], vh, (B, H, T, hd), (T * ld, hd, ld, 1))
        sc = torch.empty(BH * T * T, dtype=torch.int16, device=dev)
        units.matmul(kh, qT, sc, T, hd, T, batch=BH, a_bs=T * hd, b_bs=hd * T, c_bs=T * T, wrap32=True)
        kp = _pad8(T)
        pr = torch.empty(BH * T * kp, dtype=torch.int16, device=dev)
        units.softmax(sc, pr, T, units.OP_SOFTMAX_T, T, T, kp, sn.cm, sn.cfg, T, batch=BH, a_bs=T * T, c_bs=T * kp)
        oh = torch.empty(BH * T * hd, dtype=torch.int16, device=dev)
        units.matmul(pr, vh, oh, T, T, hd, batch=BH, a_bs=T * kp, b_bs=T * hd, c_bs=T * hd, wrap32=True)
        units.permute16(oh, o, (B, T, H, hd), (H * T * hd, hd, T * hd, 1))
        return o

    def _decode_attention(self, sn: DecodeAttentionNode, raw) -> torch.Tensor:
        """q.K^T, the row-mode softmax and P.V of every KV group in one launch."""
        qt, kt, vt = sn.inputs[:3]
        ot = sn.output
        B, KV, C, HD = (int(v) for v in kt.shape)
        G = sn.group
        if (list(vt.shape) != [B, KV, C, HD] or sn.kv_heads != KV or sn.head_dim != HD or sn.heads != KV * G
                or list(qt.shape) != [B, sn.heads * HD] or list(ot.shape) != [B, sn.heads * HD]):
            raise SchedulerError(f"decode attention '{ot.onnx_name}': q {list(qt.shape)}, caches {list(kt.shape)}, "
                                 f"o {list(ot.shape)}")
        fq, fk, fv, fo = (np.asarray(self._exp_b(t)).reshape(-1) for t in (qt, kt, vt, ot))
        if any((e != e[0]).any() for e in (fq, fk, fv, fo)):
            raise SchedulerError(f"decode attention '{ot.onnx_name}': q, the caches and o at one exponent each")
        fp = (sn.cfg >> 8) & 31
        if int(fo[0]) != fp + int(fv[0]) - self._dtype.frac_bits:
            raise SchedulerError(f"decode attention '{ot.onnx_name}': the output exponent is not f_p + f_v - 8")
        o = self._new(ot)
        units.decode_attention(self._get(qt, raw).reshape(-1).contiguous(), self._get(kt, raw).reshape(-1),
                               self._get(vt, raw).reshape(-1), o, B * KV, G, C, sn.cm, sn.cfg,
                               sn.mask_reg(C, self._host_int(sn.mask_t, raw)), head_dim=HD)
        return o

    def _prep_attention_fusable(self, sn, nxt) -> bool:
        """``nxt`` is the decode attention of ``sn``'s outputs: q = the prep's qr, the caches the
        prep writes, their shapes the ones both calls take."""
        if not self._ram_free:
            return False
        if not (isinstance(sn, DecodePrepNode) and isinstance(nxt, DecodeAttentionNode)):
            return False
        q, k, v, kc, vc = sn.inputs[:5]
        qt, kt, vt = nxt.inputs[:3]
        if (qt.onnx_name != sn.output.onnx_name or kt.onnx_name != kc.onnx_name or vt.onnx_name != vc.onnx_name
                or nxt.kv_heads != sn.kv_heads or nxt.heads != sn.heads or nxt.head_dim != sn.head_dim):
            return False
        B, KV, C, HD = (int(x) for x in kc.shape)
        return HD in (32, 64) and C % 64 == 0 and C <= 8192 and sn.heads % KV == 0 and sn.heads // KV <= 8

    def _prep_attention(self, sn: DecodePrepNode, nxt: DecodeAttentionNode, raw) -> None:
        """The prep's RoPE / cache writes and the attention over them in one launch (both outputs
        kept, the caches updated in place); the checks of _decode_prep and _decode_attention."""
        q, k, v, kc, vc = sn.inputs[:5]
        B, KV, C, HD = (int(x) for x in kc.shape)
        pos = sn.position(self._host_int(sn.pos_t, raw))
        if not 0 <= pos < C:
            raise SchedulerError(f"decode prep '{sn.output.onnx_name}': position {pos} of {C} cache rows")
        ot = nxt.output
        fq, fk, fv, fo = (np.asarray(self._exp_b(t)).reshape(-1) for t in (nxt.inputs[0], nxt.inputs[1], nxt.inputs[2], ot))
        if any((e != e[0]).any() for e in (fq, fk, fv, fo)):
            raise SchedulerError(f"decode attention '{ot.onnx_name}': q, the caches and o at one exponent each")
        if int(fo[0]) != ((nxt.cfg >> 8) & 31) + int(fv[0]) - self._dtype.frac_bits:
            raise SchedulerError(f"decode attention '{ot.onnx_name}': the output exponent is not f_p + f_v - 8")
        jq, jk = sn.rope_q.jobs(pos=pos)[0], sn.rope_k.jobs(pos=pos)[0]
        params = self._params.get(id(sn))
        if params is None:
            params = [torch.from_numpy(np.ascontiguousarray(j.params, np.uint8)).to(self.device) for j in (jq, jk)]
            self._params[id(sn)] = params
        tab = self._get(sn.rope_q.table, raw).reshape(-1, 2 * HD)
        qr = self._new(sn.output)
        o = self._new(ot)
        units.decode_attention_prep(self._get(q, raw).reshape(-1).contiguous(), self._get(k, raw).reshape(-1).contiguous(),
                                    self._get(v, raw).reshape(-1).contiguous(), qr, self._get(kc, raw).reshape(-1),
                                    self._get(vc, raw).reshape(-1), o, B, sn.heads, KV, HD, C, pos, tab[jq.b_row0],
                                    params[0], jq.op, params[1], jk.op, nxt.cm, nxt.cfg,
                                    nxt.mask_reg(C, self._host_int(nxt.mask_t, raw)))
        raw[sn.output.onnx_name] = qr
        raw[ot.onnx_name] = o

    def _decode_prep(self, sn: DecodePrepNode, raw) -> torch.Tensor:
        """RoPE of q (into the output) and k (into the K cache rows) and the V cache rows, one launch."""
        q, k, v, kc, vc = sn.inputs[:5]
        B, KV, C, HD = (int(x) for x in kc.shape)
        pos = sn.position(self._host_int(sn.pos_t, raw))
        if not 0 <= pos < C:
            raise SchedulerError(f"decode prep '{sn.output.onnx_name}': position {pos} of {C} cache rows")
        jq, jk = sn.rope_q.jobs(pos=pos)[0], sn.rope_k.jobs(pos=pos)[0]
        params = self._params.get(id(sn))
        if params is None:
            params = [torch.from_numpy(np.ascontiguousarray(j.params, np.uint8)).to(self.device) for j in (jq, jk)]
            self._params[id(sn)] = params
        tab = self._get(sn.rope_q.table, raw).reshape(-1, 2 * HD)
        qr = self._new(sn.output)
        units.decode_prep(self._get(q, raw).reshape(-1).contiguous(), self._get(k, raw).reshape(-1).contiguous(),
                          self._get(v, raw).reshape(-1).contiguous(), qr, self._get(kc, raw).reshape(-1), C,
                          self._get(vc, raw).reshape(-1), B, sn.heads, KV, HD, pos, tab[jq.b_row0], params[0], jq.op,
                          params[1], jk.op)
        return qr

    def _kv_write(self, sn: KvWriteNode, raw) -> torch.Tensor:
        """Row ``pos`` of every sequence's group-major cache from the step's rows, in place."""
        xt, ct = sn.inputs[0], sn.inputs[1]
        B, KV, C, HD = (int(v) for v in ct.shape)
        pos = sn.position(self._host_int(sn.pos_t, raw))
        if list(xt.shape) != [B, KV * HD] or not 0 <= pos < C:
            raise SchedulerError(f"KV write: rows {list(xt.shape)} into a cache {list(ct.shape)} at {pos}")
        if not np.array_equal(np.broadcast_to(self._exp_b(xt), (KV * HD,)),
                              np.broadcast_to(np.asarray(self._exp_b(ct)).reshape(-1), (KV * HD,))):
            raise SchedulerError("KV write: the rows and the cache at different exponents")
        x = self._get(xt, raw).reshape(-1).contiguous()
        cache = self._get(ct, raw)
        units.copy16(x, cache.reshape(-1)[pos * HD:], (B, KV, HD, 1), (KV * HD, HD, 1, 0),
                     (KV * C * HD, C * HD, 1, 0))
        return cache

    def _ro_calls(self, sn: RoCallNode, raw) -> torch.Tensor:
        """A node's unit calls over named buffers: the graph's tensors (the states written in
        place), the node's staging buffers (zero at creation, kept across calls) and tables."""
        host = {t.onnx_name: int(np.asarray(self._get(t, raw)).reshape(-1)[0]) for t in sn.host_inputs()}
        out = self._new(sn.output)
        bufs = {sn.output.onnx_name: out.view(torch.uint8)}
        for t in sn.inputs:
            if t is not None and t.kind != "host":
                bufs[t.onnx_name] = self._get(t, raw).reshape(-1).view(torch.uint8)
        key = id(sn)
        for k, nbytes in sn.staging().items():
            b = self._staging.get((key, k))
            if b is None:
                b = torch.zeros(nbytes + 16, dtype=torch.uint8, device=self.device)
                self._staging[(key, k)] = b
            bufs["node:" + k] = b
        for k, lanes in sn.tables().items():
            b = self._images.get(f"{key}:{k}")
            if b is None:
                b = torch.from_numpy(np.ascontiguousarray(lanes).reshape(-1).view(np.uint8).copy()).to(self.device)
                self._images[f"{key}:{k}"] = b
            bufs["node:" + k] = b
        params = self._params.setdefault(key, {})
        for j in sn.calls(host):
            p = None
            if j.p is not None:
                pk = np.asarray(j.p, np.uint8).tobytes()
                p = params.get(pk)
                if p is None:
                    p = torch.from_numpy(np.frombuffer(pk, np.uint8).copy()).to(self.device)
                    params[pk] = p
            units.rowops(bufs[j.a] if j.a else None, bufs[j.b] if j.b else None, bufs[j.c], p, j.op, j.n, j.rows,
                         j.blocks, j.a_s1, j.a_s2, j.b_s1, j.b_s2, j.c_s1, j.c_s2, j.eps, j.aux, j.bq_sh, j.win_lo,
                         j.win_hi, a_off=j.a_off, b_off=j.b_off, c_off=j.c_off)
        return out

    def _whole_row_job(self, sn: RowOpsAdapter, a2d: torch.Tensor, b_all, out: torch.Tensor, p: torch.Tensor) -> dict:
        """The single job of a whole-row adapter as rowops_jobs() takes it."""
        at, ot = sn.inputs[0], sn.output
        bt = getattr(sn, "table", None) or (sn.inputs[1] if len(sn.inputs) > 1 else None)
        j = sn.jobs()[0]
        rows, width = a2d.shape
        u8 = lambda t: t.reshape(-1).view(torch.uint8) if t is not None else None   # noqa: E731
        b2d = b_all.reshape(rows, width).contiguous() if b_all is not None else None
        return dict(a=u8(a2d.contiguous()), b=u8(b2d), c=u8(out), p=p, op=j.op, n=j.n, c1=rows, c2=1,
                    a_s1=width * _KB[at.kind], a_s2=0, b_s1=width * _KB[bt.kind] if bt is not None else 0, b_s2=0,
                    c_s1=width * _KB[ot.kind], c_s2=0, eps=j.eps, aux=j.aux, bq_sh=j.bq_sh, win_lo=0,
                    win_hi=0xFFFFFFFF)

    def _host_int(self, t: Optional[TensorInfo], raw) -> Optional[int]:
        """The first value of a host tensor (a runtime position), or None."""
        return None if t is None else int(np.asarray(self._get(t, raw)).reshape(-1)[0])

    def _adapter(self, sn: RowOpsAdapter, raw) -> torch.Tensor:
        """A row-ops adapter: its jobs over row views of the tensors (rows of ``n`` = the job
        width; a job covers the columns [col0, col0 + n) of every row)."""
        at, ot = sn.inputs[0], sn.output
        bt = getattr(sn, "table", None) or (sn.inputs[1] if len(sn.inputs) > 1 else None)
        pos_t = getattr(sn, "pos_t", None)
        jobs = sn.jobs(pos=self._host_int(pos_t, raw)) if pos_t is not None else sn.jobs()
        width = max(j.col0 + j.n for j in jobs)
        rows = at.numel // width
        a2d = self._get(at, raw).reshape(rows, width)
        out = torch.empty((rows, width), dtype=_TORCH[ot.kind], device=self.device)
        b_all = self._get(bt, raw) if bt is not None else None
        u8 = lambda t: t.reshape(-1).view(torch.uint8) if t is not None else None   # noqa: E731
        params = self._params.get(id(sn))
        if params is None:
            params = [torch.from_numpy(np.ascontiguousarray(j.params, np.uint8)).to(self.device) for j in jobs]
            self._params[id(sn)] = params
        if len(jobs) == 1 and jobs[0].col0 == 0 and jobs[0].b_row0 is None and self._rows_whole(sn, width):
            # rows already whole 16-byte multiples: the jobs run on the tensors themselves
            units.rowops_jobs([self._whole_row_job(sn, a2d, b_all, out, params[0])])
            return out.reshape(-1)
        j0 = jobs[0]
        if (len(jobs) == 1 and j0.col0 == 0 and j0.b_row0 is not None and b_all is not None
                and all((width * _KB[t.kind]) % 16 == 0 and int(t.shape[-1]) == width for t in (at, ot))):
            # a table job (RoPE) over whole rows: A, C and the table rows in place
            tab = b_all.reshape(-1, int(bt.shape[-1]))
            tb = int(bt.shape[-1]) * _KB[bt.kind]
            n_tab = 1 if j0.b_same else rows
            if tb % 16 == 0 and j0.b_row0 + n_tab <= tab.shape[0]:
                units.rowops(u8(a2d.contiguous()), u8(tab[j0.b_row0:j0.b_row0 + n_tab]), u8(out), params[0], j0.op,
                             j0.n, rows, 1, width * _KB[at.kind], 0, 0 if j0.b_same else tb, 0,
                             width * _KB[ot.kind], 0, j0.eps, j0.aux, j0.bq_sh, 0, 0xFFFFFFFF)
                return out.reshape(-1)
        for ji, j in enumerate(jobs):
            a_buf, a_s1, _ = self._rows16(a2d[:, j.col0:j.col0 + j.n], at.kind)
            b_buf, b_s1 = None, 0
            if b_all is not None:
                if j.b_row0 is None:
                    b2d = b_all.reshape(rows, width)[:, j.col0:j.col0 + j.n]
                else:
                    tab = b_all.reshape(-1, int(bt.shape[-1]))
                    if j.b_row0 + (1 if j.b_same else rows) > tab.shape[0]:
                        raise SchedulerError("row-ops job: table rows past the table")
                    b2d = tab[j.b_row0:j.b_row0 + (1 if j.b_same else rows)]
                b_buf, b_s1, _ = self._rows16(b2d, bt.kind)
                if j.b_same:
                    b_s1 = 0
            c_buf, c_s1, c_per = self._rows16(torch.zeros((rows, j.n), dtype=_TORCH[ot.kind], device=self.device),
                                              ot.kind)
            units.rowops(u8(a_buf), u8(b_buf), u8(c_buf), params[ji], j.op, j.n, rows, 1, a_s1, 0, b_s1, 0, c_s1,
                         0, j.eps, j.aux, j.bq_sh, 0, 0xFFFFFFFF)
            out[:, j.col0:j.col0 + j.n] = c_buf[:, :j.n]
        return out.reshape(-1)


__all__ = ["Simulator"]
