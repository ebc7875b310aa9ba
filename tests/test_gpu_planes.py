"""Operands split by their producers: the NORM job (alone and after the residual add it runs
with as one launch), the VectorOP over rows and the fused attention write the byte planes of
their int16 output for the MatMul that takes it as A (cm_matmul_aplanes).  Checked on the GPU:
the producer's own output is what the plain call writes, the planes and partial row sums are
the split of that output (x - 128 = 256 hi + lo), and the MatMul over them equals the MatMul of
the int16 output, bit for bit, in both output rules (Q8.8 saturation, pow2 int32 wrap); graphs
with such producers equal the oracle in every tensor."""
import numpy as np
import pytest
import torch

from cormorant_amd import rowops_nodes as rn
from cormorant_amd.graph import Graph, MatmulNode, ScheduledNode, TensorInfo
from cormorant_amd.simulate import Simulator
from gpu_util import dev16, host
from oracle import graph_sim as oracle_graph

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def U():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cormorant_amd import units
    units.init()
    return units


def split_ref(x2d: np.ndarray, groups: int):
    """hi / lo byte planes of int16 rows and the row sums over `groups` equal column groups."""
    x = x2d.astype(np.int32)
    hi = ((x >> 8) & 0xFF).astype(np.uint8)
    lo = ((x & 0xFF) ^ 0x80).astype(np.uint8)
    n, k = x.shape
    sums = x.reshape(n, groups, k // groups).sum(axis=2).T            # [groups][n]
    return hi, lo, sums


def split_ref_slabs(x2d: np.ndarray):
    """As split_ref with the sums per 1024 columns (the last slab possibly shorter)."""
    x = x2d.astype(np.int32)
    n, k = x.shape
    hi, lo, _ = split_ref(x2d, 1)
    sums = np.stack([x[:, s:s + 1024].sum(axis=1) for s in range(0, k, 1024)])
    return hi, lo, sums


def read_planes(planes: torch.Tensor, n: int, k: int, nsum: int):
    lines = (n + 255) // 256 * 256
    b = host(planes)
    hi = b[:lines * k].reshape(lines, k)[:n]
    lo = b[lines * k:2 * lines * k].reshape(lines, k)[:n]
    part = b[2 * lines * k:2 * lines * k + 4 * nsum * lines].view(np.int32).reshape(nsum, lines)[:, :n]
    return hi, lo, part


def check_matmul(U, planes, nsum, a16: torch.Tensor, n, k, seed):
    """matmul_aplanes over the producer's planes == matmul_planes over its int16 output."""
    rng = np.random.default_rng(seed)
    for m, wrap in ((384, True), (200, False)):
        w = rng.integers(-3000, 3000, (k, m)).astype(np.int16)
        from cormorant_amd.packing import pack_matmul_b
        bp = U.matmul_b_planes(torch.from_numpy(pack_matmul_b(w)).cuda(), k, m, b_packed=1)
        c1 = torch.empty(n * m, dtype=torch.int16, device="cuda")
        c2 = torch.empty(n * m, dtype=torch.int16, device="cuda")
        U.matmul_aplanes(planes, nsum, bp, c1, n, k, m, wrap32=wrap)
        U.matmul_planes(a16.reshape(-1).contiguous(), bp, c2, n, k, m, wrap32=wrap)
        np.testing.assert_array_equal(host(c1), host(c2), err_msg=f"m {m} wrap {wrap}")


def _ln32(rows, n, seed):
    rng = np.random.default_rng(seed)
    gamma = 1.0 + 0.05 * rng.standard_normal(n)
    beta = 0.05 * rng.standard_normal(n)
    ht = TensorInfo("h", [rows, n], exp=15, kind="i32")
    yt = TensorInfo("y", [rows, n], exp=11)
    return rn.LayerNorm32RoNode([ht], yt, gamma=gamma, beta=beta, eps=1e-6)


def _job(node, a, b, c, p):
    j = node.jobs()[0]
    u8 = lambda t: t.reshape(-1).view(torch.uint8) if t is not None else None   # noqa: E731
    kb = {"i16": 2, "i32": 4}
    n = node.n
    rows = node.output.numel // n
    return dict(a=u8(a), b=u8(b), c=u8(c), p=p, op=j.op, n=j.n, c1=rows, c2=1, a_s1=n * kb[node.inputs[0].kind],
                a_s2=0, b_s1=n * kb[node.inputs[1].kind] if b is not None else 0, b_s2=0,
                c_s1=n * kb[node.output.kind], c_s2=0, eps=j.eps, aux=j.aux, bq_sh=j.bq_sh)


def _params(node):
    return torch.from_numpy(np.ascontiguousarray(node.jobs()[0].params, np.uint8)).cuda()


@pytest.mark.parametrize("rows,n", [(300, 768), (64, 1088), (513, 2048), (3100, 768)])
def test_norm_planes(U, rows, n):
    """A NORM job's planes: the int16 rows as the plain job writes them, their split, and the
    MatMul over them."""
    node = _ln32(rows, n, rows + n)
    rng = np.random.default_rng(rows)
    h = torch.from_numpy(rng.integers(-2 ** 24, 2 ** 24, rows * n).astype(np.int32)).cuda()
    y0 = torch.empty(rows * n, dtype=torch.int16, device="cuda")
    y1 = torch.empty(rows * n, dtype=torch.int16, device="cuda")
    p = _params(node)
    U.rowops_jobs([_job(node, h, None, y0, p)])
    nsum = (n + 1023) // 1024
    planes = U.a_planes(rows, n, nsum, "cuda")
    U.rowops_jobs([_job(node, h, None, y1, p)], planes=planes)
    y = host(y1).reshape(rows, n)
    np.testing.assert_array_equal(y, host(y0).reshape(rows, n))
    hi, lo, part = read_planes(planes, rows, n, nsum)
    rhi, rlo, rsum = split_ref_slabs(y)
    np.testing.assert_array_equal(hi, rhi)
    np.testing.assert_array_equal(lo, rlo)
    np.testing.assert_array_equal(part, rsum)
    check_matmul(U, planes, nsum, y1, rows, n, rows)


@pytest.mark.parametrize("rows,n,a32,planes_on", [(300, 768, True, True), (300, 768, True, False),
                                                  (77, 1088, False, True), (3100, 768, True, True)])
def test_addx_norm_one_launch(U, rows, n, a32, planes_on):
    """The residual add and the NORM of its output as one chain call (one launch) write what
    the two jobs write one call at a time, and the NORM's planes."""
    rng = np.random.default_rng(n + rows)
    ht = TensorInfo("h", [rows, n], exp=15, kind="i32" if a32 else "i16")
    if not a32:
        ht = TensorInfo("h", [rows, n], exp=10)
    dt = TensorInfo("d", [rows, n], exp=12)
    h1t = TensorInfo("h1", [rows, n], exp=15, kind="i32")
    add = rn.ResAddBiasRoNode([ht, dt], h1t, bias=rng.uniform(-2, 2, n))
    ln = rn.LayerNorm32RoNode([h1t], TensorInfo("y", [rows, n], exp=11), gamma=1 + 0.05 * rng.standard_normal(n),
                              beta=0.05 * rng.standard_normal(n), eps=1e-6)
    h = (rng.integers(-2 ** 26, 2 ** 26, rows * n).astype(np.int32) if a32
         else rng.integers(-32768, 32768, rows * n).astype(np.int16))
    h = torch.from_numpy(h).cuda()
    d = dev16(rng.integers(-32768, 32768, rows * n), 0)
    pa, pn = _params(add), _params(ln)
    outs = []
    for fused in (False, True):
        h1 = torch.empty(rows * n, dtype=torch.int32, device="cuda")
        y = torch.empty(rows * n, dtype=torch.int16, device="cuda")
        ja, jn = _job(add, h, d, h1, pa), _job(ln, h1, None, y, pn)
        planes = None
        if fused:
            planes = U.a_planes(rows, n, (n + 1023) // 1024, "cuda") if planes_on else None
            U.rowops_jobs([ja, jn], planes=planes)
        else:
            U.rowops_jobs([ja])
            U.rowops_jobs([jn])
        outs.append((host(h1), host(y), planes, y))
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1], outs[0][1])
    if planes_on:
        nsum = (n + 1023) // 1024
        hi, lo, part = read_planes(outs[1][2], rows, n, nsum)
        rhi, rlo, rsum = split_ref_slabs(outs[1][1].reshape(rows, n))
        np.testing.assert_array_equal(hi, rhi)
        np.testing.assert_array_equal(lo, rlo)
        np.testing.assert_array_equal(part, rsum)
        check_matmul(U, outs[1][2], nsum, outs[1][3], rows, n, n)
        # the NORM's rows left unwritten (c None): the same residual sum and planes
        h1 = torch.empty(rows * n, dtype=torch.int32, device="cuda")
        p2 = U.a_planes(rows, n, nsum, "cuda")
        jn2 = dict(_job(ln, h1, None, outs[1][3], pn), c=None)
        U.rowops_jobs([_job(add, h, d, h1, pa), jn2], planes=p2)
        np.testing.assert_array_equal(host(h1), outs[0][0])
        hi2, lo2, part2 = read_planes(p2, rows, n, nsum)
        np.testing.assert_array_equal(hi2, rhi)
        np.testing.assert_array_equal(lo2, rlo)
        np.testing.assert_array_equal(part2, rsum)
        with pytest.raises(ValueError):                # a null output without planes is refused
            U.rowops_jobs([_job(add, h, d, h1, pa), jn2])


def test_null_outputs_refused_at_the_c_abi(U):
    """cm_rowops and cm_rowops_chain called directly (no Python checks in between): a job with
    work and a null c is CM_EINVAL for NORM, COPY, ADDX and TRANSPOSE, alone and in a chain
    without planes; nothing is launched for it."""
    import ctypes
    from cormorant_amd import _lib
    lib = _lib.lib()
    n, rows = 64, 4
    a = torch.zeros(rows * n, dtype=torch.int32, device="cuda")
    b = torch.zeros(rows * n, dtype=torch.int16, device="cuda")
    p = torch.zeros(16, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for code, bk in ((U.RO_NORM, None), (U.RO_COPY, None), (U.RO_ADDX, U.K_I16)):
        op = code | (U.K_I32 << 4) | ((bk or 0) << 6) | U.F_P_BCAST | (U.F_B_EN if bk is not None else 0)
        if code == U.RO_ADDX:
            op |= U.K_I32 << 8
        rc = lib.cm_rowops(a.data_ptr(), b.data_ptr() if bk is not None else None, None, p.data_ptr(), op, n, rows,
                           1, 4 * n, 0, 2 * n, 0, 4 * n, 0, 1 << 20, 0, 0, 0, 0xFFFFFFFF, stream)
        assert rc < 0, (code, rc)
        assert "null output" in lib.cm_last_error().decode()
        desc = _lib.CmRowopsDesc(a=a.data_ptr(), b=b.data_ptr() if bk is not None else 0, c=0, p=p.data_ptr(), op=op,
                            n=n, c1=rows, c2=1, a_s1=4 * n, b_s1=2 * n, c_s1=4 * n, eps=1 << 20, win_hi=0xFFFFFFFF)
        rc = lib.cm_rowops_chain(ctypes.byref(desc), 1, stream)
        assert rc < 0, (code, rc)
    xop = U.RO_XPOSE
    rc = lib.cm_rowops(b.data_ptr(), None, None, None, xop, 16, 1, 1, 2 * 64, 0, 0, 0, 2 * 16, 0, 0, 8, 0, 0,
                       0xFFFFFFFF, stream)
    assert rc < 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows,k,act,arity", [(300, 3072, 5, 2), (96, 1088, 0, 2), (130, 640, 2, 1)])
def test_vectorop_planes(U, rows, k, act, arity):
    """A VectorOP over rows of k (ADD of a broadcast bias row with GELU / no act; RELU6 alone):
    the plain call's output, its planes, the MatMul over them."""
    rng = np.random.default_rng(k + act)
    a = dev16(rng.integers(-6000, 6000, rows * k), 0)
    b = dev16(rng.integers(-600, 600, k), 0) if arity == 2 else None
    op = U.OP_ADD if arity == 2 else U.OP_RELU6
    c0 = torch.empty(rows * k, dtype=torch.int16, device="cuda")
    c1 = torch.empty(rows * k, dtype=torch.int16, device="cuda")
    if arity == 2:
        U.vectorop(a, b, c0, k, op, outer=rows, a_inc=k, b_inc=0, act=act)
    else:
        U.vectorop(a, None, c0, rows * k, op)
    nsum = (k + 1023) // 1024
    planes = U.a_planes(rows, k, nsum, "cuda")
    U.vectorop_planes(a, b, c1, k, op, rows, k, 0, planes, act=act)
    y = host(c1).reshape(rows, k)
    np.testing.assert_array_equal(y, host(c0).reshape(rows, k))
    hi, lo, part = read_planes(planes, rows, k, nsum)
    rhi, rlo, rsum = split_ref_slabs(y)
    np.testing.assert_array_equal(hi, rhi)
    np.testing.assert_array_equal(lo, rlo)
    np.testing.assert_array_equal(part, rsum)
    check_matmul(U, planes, nsum, c1, rows, k, k)
    # the planes alone (no int16 output): the same planes and sums
    p2 = U.a_planes(rows, k, nsum, "cuda")
    U.vectorop_planes(a, b, None, k, op, rows, k, 0, p2, act=act)
    hi2, lo2, part2 = read_planes(p2, rows, k, nsum)
    np.testing.assert_array_equal(hi2, rhi)
    np.testing.assert_array_equal(lo2, rlo)
    np.testing.assert_array_equal(part2, rsum)


@pytest.mark.parametrize("B,T,H", [(2, 128, 3), (1, 384, 12)])
def test_attention_planes(U, B, T, H):
    """The fused attention's o with its planes (per-head partial sums): o as cm_attention
    writes it, the split, the output projection over the planes."""
    from cormorant_amd.graph import softmax_regs
    rng = np.random.default_rng(T + H)
    hd, D = 64, 64 * H
    ld = 3 * D
    cm, cfg = softmax_regs(9, 0.125, 14)
    x = dev16(rng.integers(-3000, 3000, B * T * ld), 0)
    o0 = torch.empty(B * T * D, dtype=torch.int16, device="cuda")
    o1 = torch.empty(B * T * D, dtype=torch.int16, device="cuda")
    U.attention(x, o0, B, T, H, hd, ld, 0, D, 2 * D, D, cm, cfg)
    planes = U.a_planes(B * T, D, H, "cuda")
    U.attention_planes(x, o1, B, T, H, hd, ld, 0, D, 2 * D, cm, cfg, planes)
    y = host(o1).reshape(B * T, D)
    np.testing.assert_array_equal(y, host(o0).reshape(B * T, D))
    hi, lo, part = read_planes(planes, B * T, D, H)
    rhi, rlo, rsum = split_ref(y, H)
    np.testing.assert_array_equal(hi, rhi)
    np.testing.assert_array_equal(lo, rlo)
    np.testing.assert_array_equal(part, rsum)
    check_matmul(U, planes, H, o1, B * T, D, T)
    # the planes alone (no o): the same planes and sums
    p2 = U.a_planes(B * T, D, H, "cuda")
    U.attention_planes(x, None, B, T, H, hd, ld, 0, D, 2 * D, cm, cfg, p2)
    hi2, lo2, part2 = read_planes(p2, B * T, D, H)
    np.testing.assert_array_equal(hi2, rhi)
    np.testing.assert_array_equal(lo2, rlo)
    np.testing.assert_array_equal(part2, rsum)


def test_graph_with_split_producers(U):
    """A graph where every MatMul's A comes from a producer that writes its planes (the
    residual add + LayerNorm pair, the LayerNorm alone, a bias + GELU VectorOP), rows not a
    multiple of 256, k not a multiple of 1024: every tensor equals the oracle's."""
    rng = np.random.default_rng(11)
    rows, d, ff = 300, 320, 1088
    h0 = TensorInfo("h0", [rows, d], exp=15, kind="i32")
    dd = TensorInfo("dd", [rows, d], exp=12)
    h1 = TensorInfo("h1", [rows, d], exp=15, kind="i32")
    x1 = TensorInfo("x1", [rows, d], exp=11)
    x2 = TensorInfo("x2", [rows, d], exp=11)
    w1 = TensorInfo("w1", [d, ff], data=rng.standard_normal((d, ff)) * 0.02)
    f = TensorInfo("f", [rows, ff])
    b1 = TensorInfo("b1", [ff], data=rng.standard_normal(ff) * 0.1)
    a = TensorInfo("a", [rows, ff])
    w2 = TensorInfo("w2", [ff, d], data=rng.standard_normal((ff, d)) * 0.02)
    y = TensorInfo("y", [rows, d])
    wq = TensorInfo("wq", [d, 256], data=rng.standard_normal((d, 256)) * 0.02)
    q = TensorInfo("q", [rows, 256], exp=9)
    g1, be1 = 1 + 0.02 * rng.standard_normal(d), 0.02 * rng.standard_normal(d)
    nodes = [
        rn.LayerNorm32RoNode([h0], x1, gamma=g1, beta=be1, eps=1e-6),
        MatmulNode([x1, wq], q),
        rn.ResAddBiasRoNode([h0, dd], h1, bias=rng.uniform(-1, 1, d)),
        rn.LayerNorm32RoNode([h1], x2, gamma=g1, beta=be1, eps=1e-6),
        MatmulNode([x2, w1], f),
        ScheduledNode([f, b1], a, U.OP_ADD, act=U.ACT_GELU),
        MatmulNode([a, w2], y),
    ]
    from cormorant_amd.numeric import encode_matmul_weights
    from cormorant_amd.dtype import AP_FIXED_16_8
    g = Graph(nodes, input_tensors=[h0, dd], output_tensors=[y, q])
    encode_matmul_weights(g.nodes, AP_FIXED_16_8)
    inputs = {"h0": rng.integers(-2 ** 17, 2 ** 17, (rows, d)) / 2.0 ** 15,
              "dd": rng.integers(-3000, 3000, (rows, d)) / 2.0 ** 12}
    sim = Simulator(g)
    consumers, producers = sim._plan_planes()
    assert set(producers) == {"x1", "x2", "a"}, producers
    got = sim._forward_pass(inputs)
    want = oracle_graph.forward(g, inputs)
    for name, v in got.items():
        np.testing.assert_array_equal(v, want[name].reshape(v.shape), err_msg=name)
