"""The on-disk formats (the reference's weight / expected-output .dat files and C literals,
dtype.py:385-443, _simulate.py:841-964) on the CPU: closed forms of the storage encodings
(round half to even, saturation, two's complement, little-endian), the ramp fill's values, the
literal text, a .dat round trip, and the expected-storage layout of each tensor kind."""
import numpy as np

from cormorant_amd.dtype import AP_FIXED_16_8 as DT
from cormorant_amd.graph import Graph, ReshapeNode, TensorInfo as T


def test_dat_bytes_closed_form():
    v = np.array([0.0, 1 / 256, -1 / 256, 127.99609375, -128.0, 200.0, -300.0, 0.5 / 256, 1.5 / 256, -0.5 / 256])
    want = [0x0000, 0x0001, 0xFFFF, 0x7FFF, 0x8000, 0x7FFF, 0x8000, 0x0000, 0x0002, 0x0000]
    b = DT.dat_bytes(v)
    assert len(b) == 2 * v.size
    assert list(np.frombuffer(b, "<u2")) == want
    assert b[:4] == bytes([0, 0, 1, 0])                       # little-endian


def test_exp_storage_and_ramp():
    assert list(DT.exp_to_storage(np.array([1.0, -0.5, 3.0, 1e9]), np.array([12, 12, 14, 3]))) == \
        [4096, 0x10000 - 2048, 0x7FFF, 0x7FFF]
    pos = np.array([0, 1, 255, 256, 0x7FFF, 0x8000, 0xFFFF, 0x10001])
    np.testing.assert_array_equal(DT.ramp_to_float(pos) * 256, [0, 1, 255, 256, 32767, -32768, -1, 1])
    np.testing.assert_array_equal(DT.ramp_to_float_exp(pos, 4) * 16, [0, 1, 255, 256, 32767, -32768, -1, 1])
    assert DT.format_literal(0xABC) == "0x0ABC" and DT.format_literal(-1) == "0xFFFF"
    assert list(DT.int_to_storage(np.array([3.0, -2.0, 70000.0]))) == [3, 0xFFFE, 0x7FFF]


def test_dat_round_trip():
    rng = np.random.default_rng(0)
    v = rng.integers(-32768, 32768, 1000) / 256.0
    back = np.frombuffer(DT.dat_bytes(v), "<u2").view(np.int16) / 256.0
    np.testing.assert_array_equal(back, v)


def test_expected_storage_of_each_kind():
    """Through a graph of aliases (no GPU needed for the storage step): Q8.8, exponents per
    channel, the int32 residual and float32 values."""
    from cormorant_amd.simulate import Simulator
    q, e = T("q", [2, 4]), T("e", [2, 4], exp=np.array([8, 10, 12, 14]))
    r, f = T("r", [3], exp=15, kind="i32"), T("f", [2], kind="f32")
    g = Graph([ReshapeNode([q], T("q2", [8]))], input_tensors=[q, e, r, f], output_tensors=[])
    sim = Simulator.__new__(Simulator)                         # the storage encoders read no device state
    sim._graph, sim._dtype = g, DT
    sim._infos = {t.onnx_name: t for t in (q, e, r, f)}
    qv = np.array([[1.0, -1.0, 0.5, 127.99609375], [0, 0, 0, -128.0]])
    assert list(sim._expected_storage("q", qv)[:4]) == [256, 0x10000 - 256, 128, 0x7FFF]
    ev = np.array([[1.0, 1.0, 1.0, 1.0], [0, 0, 0, -1.0]])
    assert list(sim._expected_storage("e", ev)) == [256, 1024, 4096, 16384, 0, 0, 0, 0x10000 - 16384]
    rv = sim._expected_storage("r", np.array([1.0, -2.5, 3e-5]))
    assert rv.dtype == np.int32 and list(rv) == [32768, -81920, 1]
    fv = sim._expected_storage("f", np.array([0.1, -3.0]))
    assert fv.dtype == np.float32 and fv[0] == np.float32(0.1)
    text = sim._emit_expected_c("q", sim._expected_storage("q", qv))
    assert text.startswith("static const uint16_t expected_q[8] = {\n    0x0100, 0xFF00, 0x0080, 0x7FFF,")
    assert text.endswith("0x8000\n};\n")
