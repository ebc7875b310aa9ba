"""The units' weight images, built on the host once per weight (as the reference's scheduler
does when it emits a graph):

* matmul packed B -- ``Bp[((j // 32) * k + kk) * 32 + j % 32] = B[kk][j]``, m zero-padded to
  a multiple of 32 (MatmulKernel.h:91-113; nodes.py:606-628);
* conv weights -- ``[M][ceil(C/16)][kh][kw][lanes]`` with 16-lane input-channel tiles, the
  last one 8 lanes when at most 8 channels remain, unused lanes zero; depthwise
  ``[M][roundup(kh*kw, 8)]``; bias ``[roundup(M, 8)]`` (ConvKernel.h:136-159;
  nodes.py:1097-1150);
* a MatMul lowered onto the conv unit -- B as the conv's x image (nodes.py:1592-1624).
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


CONV_TILE_IC = 16      # input channels per packed weight tile (ConvKernel.h)


def conv_lowered_k_index(c, j, kw: int):
    """K index of input channel c at kernel column j of a MatMul lowered onto the conv unit (1 x kw
    kernel, in_ch = K / kw): A's row read as the packed weight [N][K/(16 kw)][1][kw][16] puts
    channel c of column j at (c / 16) 16 kw + 16 j + c % 16 (nodes.py:1592-1599)."""
    t = CONV_TILE_IC
    return (c // t) * t * kw + j * t + c % t


def conv_lowered_b_image(b: np.ndarray, k: int, m: int, kw: int) -> np.ndarray:
    """The conv x image of a lowered MatMul's B [..., k, m] (one image per slice, concatenated):
    x[s][c][kw p + j] = B[s][conv_lowered_k_index(c, j)][p] for c < k / kw, so that a 1 x kw
    conv of stride (1, kw) over in_h x kw out_w reads B's column p at output position p; kw = 1
    is B itself (nodes.py:1601-1624)."""
    b3 = np.asarray(b).reshape(-1, k, m)
    if kw == 1:
        return np.ascontiguousarray(b3).reshape(-1)
    c = np.arange(k // kw)[:, None]
    j = np.arange(kw)[None, :]
    img = b3[:, conv_lowered_k_index(c, j, kw), :]           # [s][in_ch][kw][m]
    return np.ascontiguousarray(img.transpose(0, 1, 3, 2)).reshape(-1)
