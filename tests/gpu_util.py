"""Helpers of the GPU parity tests: padded device copies and poison fills."""
import numpy as np
import torch

POISON16 = np.int16(0x5A5A)


def dev16(a, extra: int = 16) -> torch.Tensor:
    """A GPU int16 copy of ``a`` with ``extra`` zero lanes after it (whole-word reads past a
    run's end stay inside the tensor)."""
    a = np.asarray(a, np.int16).reshape(-1)
    t = torch.zeros(len(a) + extra, dtype=torch.int16, device="cuda")
    if len(a):
        t[:len(a)] = torch.from_numpy(a.copy()).cuda()
    return t


def dev8(a, extra: int = 0) -> torch.Tensor:
    a = np.asarray(a, np.uint8).reshape(-1)
    t = torch.zeros(len(a) + extra, dtype=torch.uint8, device="cuda")
    if len(a):
        t[:len(a)] = torch.from_numpy(a.copy()).cuda()
    return t


def poisoned16(n: int) -> torch.Tensor:
    return torch.full((n,), int(POISON16), dtype=torch.int16, device="cuda")


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()
