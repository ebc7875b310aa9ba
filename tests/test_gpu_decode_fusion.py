"""The decode step's prep (RoPE of q / k, the KV cache rows) run by the attention workgroups
(cm_decode_attention_prep) against the two launches it replaces (cm_decode_prep, then
cm_decode_attention): qr, both caches and o bit for bit, at the first, a middle and the last
cache row, head dims 64 and 32, broadcast and per-column RoPE parameter blocks."""
import numpy as np
import pytest
import torch

from cormorant_amd import rowops_nodes as rn
from cormorant_amd.graph import TensorInfo, softmax_regs
from gpu_util import host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def U():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cormorant_amd import units
    units.init()
    return units


@pytest.mark.parametrize("B,H,KV,HD,C,pos,bcast", [(16, 15, 5, 64, 1024, 1023, True), (16, 15, 5, 64, 1024, 0, False),
                                                   (3, 8, 2, 32, 256, 130, False), (2, 6, 6, 64, 128, 77, True)])
def test_prep_then_attention(U, B, H, KV, HD, C, pos, bcast):
    rng = np.random.default_rng(B * 100 + C + pos)
    theta = 1e5
    inv = theta ** (-np.arange(0, HD, 2) / HD)
    ang = np.outer(np.arange(C), inv)
    cos, sin = np.cos(ang), np.sin(ang)
    qt = TensorInfo("q", [B, H * HD], exp=10)
    kt = TensorInfo("k", [B, KV * HD], exp=10)
    # RoPE jobs of the decode graph's nodes (same_pos: every row at one position)
    rq = rn.RopeRoNode([qt], TensorInfo("qr", [B, H * HD], exp=10), heads=H, head_dim=HD, cos=cos, sin=sin, pos=pos,
                       same_pos=True)
    rk = rn.RopeRoNode([kt], TensorInfo("kr", [B, KV * HD], exp=10), heads=KV, head_dim=HD, cos=cos, sin=sin,
                       pos=pos, same_pos=True)
    jq, jk = rq.jobs(pos=pos)[0], rk.jobs(pos=pos)[0]
    if not bcast:      # per-column blocks: the broadcast entry repeated (the same rule, column by column)
        jq.params = np.tile(jq.params[:16], H * HD) if jq.op & (1 << 13) else jq.params
        jk.params = np.tile(jk.params[:16], KV * HD) if jk.op & (1 << 13) else jk.params
        jq.op &= ~(1 << 13)
        jk.op &= ~(1 << 13)
    tab = torch.from_numpy(np.ascontiguousarray(rq.table.data, np.int32)).cuda().reshape(-1, 2 * HD)[jq.b_row0]
    pq = torch.from_numpy(np.ascontiguousarray(jq.params, np.uint8)).cuda()
    pk = torch.from_numpy(np.ascontiguousarray(jk.params, np.uint8)).cuda()
    q = torch.from_numpy(rng.integers(-3000, 3000, B * H * HD).astype(np.int16)).cuda()
    k = torch.from_numpy(rng.integers(-3000, 3000, B * KV * HD).astype(np.int16)).cuda()
    v = torch.from_numpy(rng.integers(-3000, 3000, B * KV * HD).astype(np.int16)).cuda()
    kc0 = torch.from_numpy(rng.integers(-3000, 3000, B * KV * C * HD).astype(np.int16)).cuda()
    vc0 = torch.from_numpy(rng.integers(-3000, 3000, B * KV * C * HD).astype(np.int16)).cuda()
    cm, cfg = softmax_regs(12, 1.0 / np.sqrt(HD), 14)
    mask = (pos + 1) | (0 << 16)                       # valid keys: rows 0 .. pos
    outs = []
    for fused in (False, True):
        kc, vc = kc0.clone(), vc0.clone()
        qr = torch.full((B * H * HD,), 0x5A5A, dtype=torch.int16, device="cuda")
        o = torch.full((B * H * HD,), 0x5A5A, dtype=torch.int16, device="cuda")
        if fused:
            U.decode_attention_prep(q, k, v, qr, kc, vc, o, B, H, KV, HD, C, pos, tab, pq, jq.op, pk, jk.op, cm, cfg, mask)
        else:
            U.decode_prep(q, k, v, qr, kc, C, vc, B, H, KV, HD, pos, tab, pq, jq.op, pk, jk.op)
            U.decode_attention(qr, kc, vc, o, B * KV, H // KV, C, cm, cfg, mask, head_dim=HD)
        outs.append([host(x) for x in (qr, kc, vc, o)])
    for name, a, b in zip(("qr", "kc", "vc", "o"), outs[1], outs[0]):
        np.testing.assert_array_equal(a, b, err_msg=name)
