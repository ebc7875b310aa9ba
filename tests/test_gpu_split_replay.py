"""The split-k product finished in place (each slice's int32 partials with agent-scope stores,
a per-tile arrival count, the last slice adds the others') replayed from a captured HIP graph:
an FFN2-shaped wrap-mode MatMul (3072 x 3072 x 768, split over k in three) 100 times, the output
poisoned by eager work between replays, every replay against the oracle, stopping at the first
mismatch.  The arrival counts are reset by each tile's last slice, so replays need no clearing."""
import numpy as np
import pytest

from oracle import cm

pytestmark = pytest.mark.gpu


def test_split_k_product_replays():
    import torch
    from cormorant_amd import units
    units.init()
    n, k, m = 3072, 3072, 768
    rng = np.random.default_rng(2026)
    a = rng.integers(-32768, 32768, n * k).astype(np.int16)
    b = rng.integers(-32768, 32768, k * m).astype(np.int16)
    want = torch.from_numpy(cm.matmul(a, b, n, k, m, wrap32=True).astype(np.int16)).cuda()
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    c = torch.empty(n * m, dtype=torch.int16, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        units.matmul(da, db, c, n, k, m, wrap32=True)       # workspace sized before the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(c, want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        units.matmul(da, db, c, n, k, m, wrap32=True)
    for r in range(100):
        c.fill_(0x5A5A)                                     # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(c, want):
            bad = int((c != want).sum())
            pytest.fail(f"replay {r}: {bad} outputs differ from the oracle")
