"""The units' weight images, built on the host once per weight (as the reference's scheduler
does when it emits a graph):

* matmul packed B -- ``Bp[((j // 32) * k + kk) * 32 + j % 32] = B[kk][j]``, m zero-padded to
  a multiple of 32 (MatmulKernel.h:91-113; nodes.py:606-628);
* conv weights -- ``[M][ceil(C/16)][kh][kw][lanes]`` with 16-lane input-channel tiles, the
  last one 8 lanes when at most 8 channels remain, unused lanes zero; depthwise
  ``[M][roundup(kh*kw, 8)]``; bias ``[roundup(M, 8)]`` (ConvKernel.h:136-159;
  nodes.py:1097-1150).
"""
from __future__ import annotations

import numpy as np


def pack_matmul_b(b: np.ndarray) -> np.ndarray:
    """Packed tile-major image of a raw int16 B [k][m]."""
    b = np.asarray(b, np.int16)
    k, m = b.shape
    mp = (m + 31) // 32 * 32
    pad = np.zeros((k, mp), np.int16)
    pad[:, :m] = b
    return np.ascontiguousarray(pad.reshape(k, mp // 32, 32).transpose(1, 0, 2)).reshape(-1)


def conv_weight_image(w: np.ndarray, depthwise: bool = False) -> np.ndarray:
    """Packed image of raw int16 conv weights w [M][C][kh][kw] ([M][1][kh][kw] depthwise)."""
    w = np.asarray(w, np.int16)
    M, C, kh, kw = w.shape
    if depthwise:
        stride = (kh * kw + 7) & ~7
        out = np.zeros((M, stride), np.int16)
        out[:, :kh * kw] = w.reshape(M, kh * kw)
        return out.reshape(-1)
    tiles = (C + 15) // 16
    rem = C - (tiles - 1) * 16
    last = 8 if rem <= 8 else 16
    per_m = kh * kw * ((tiles - 1) * 16 + last)
    out = np.zeros((M, per_m), np.int16)
    for t in range(tiles):
        lanes = last if t + 1 == tiles else 16
        c0, c1 = 16 * t, min(C, 16 * t + 16)
        blk = np.zeros((M, kh, kw, lanes), np.int16)
        blk[..., :c1 - c0] = w[:, c0:c1].transpose(0, 2, 3, 1)
        off = t * kh * kw * 16
        out[:, off:off + kh * kw * lanes] = blk.reshape(M, -1)
    return out.reshape(-1)


def conv_bias_image(bias: np.ndarray) -> np.ndarray:
    """Bias padded to a whole number of 8-lane words (ConvKernel.h:146)."""
    bias = np.asarray(bias, np.int16).reshape(-1)
    out = np.zeros((len(bias) + 7) & ~7, np.int16)
    out[:len(bias)] = bias
    return out
