"""Value <-> raw conversions of the reference's fixed-point element type (Q8.8 ap_fixed<16,8>
and power-of-two exponents), used at the edges of a simulated graph.

Mirrors inference-scheduler/src/dtype.py: ``quantize`` (clip, round half to even,
dtype.py:367-369), ``truncate`` (clip, floor, :371-377), ``truncate_div`` (clip, toward zero,
:379-383), ``host_quantize`` (NaN -> 0, then quantize, :214-219), ``quantize_exp`` /
``truncate_exp`` (:278-291) and the raw storage encodings (``float_to_storage`` :391-395,
``exp_to_storage``).
Inside the simulator every tensor is a raw int16 lane array on the device with an exponent
f (value = raw * 2^-f); the float64 values of the reference's API appear only here.
"""
from __future__ import annotations

import numpy as np

I16_LO, I16_HI = -32768, 32767


class ApFixed16:
    """ap_fixed<16, I>: 16-bit two's complement with F = 16 - I fraction bits."""

    def __init__(self, integer_bits: int = 8):
        self.W, self.I = 16, integer_bits
        self.F = 16 - integer_bits
        self.scale = float(1 << self.F)
        self.min_val = -float(1 << (integer_bits - 1))
        self.max_val = float(1 << (integer_bits - 1)) - 1.0 / self.scale

    name = property(lambda self: f"ap_fixed<16,{self.I}>")
    frac_bits = property(lambda self: self.F)
    raw_range = property(lambda self: (float(I16_LO), float(I16_HI)))

    # -- the reference's value-domain rules ---------------------------------------------
    def quantize(self, x) -> np.ndarray:
        """clip, then round half to even at 2^-F (dtype.py:367-369)."""
        c = np.clip(np.asarray(x, np.float64), self.min_val, self.max_val)
        return np.round(c * self.scale) / self.scale

    def truncate(self, x) -> np.ndarray:
        """clip, then floor at 2^-F: a kernel output (dtype.py:371-377)."""
        c = np.clip(np.asarray(x, np.float64), self.min_val, self.max_val)
        return np.floor(c * self.scale) / self.scale

    def truncate_div(self, x) -> np.ndarray:
        """clip, then toward zero at 2^-F: the DIV output (C integer division, dtype.py:379-383)."""
        c = np.clip(np.asarray(x, np.float64), self.min_val, self.max_val)
        return np.trunc(c * self.scale) / self.scale

    def host_quantize(self, x) -> np.ndarray:
        """What a host op writes back for a double result: NaN -> 0, then quantize
        (dtype.py:214-219, the generated C host_st())."""
        x = np.asarray(x, np.float64)
        return self.quantize(np.where(np.isnan(x), 0.0, x))

    def truncate_exp(self, x, f) -> np.ndarray:
        """floor at 2^-f, saturate: a kernel output at a power-of-two exponent (dtype.py:287-291)."""
        s = np.power(2.0, np.asarray(f, np.float64))
        return np.clip(np.floor(np.asarray(x, np.float64) * s), I16_LO, I16_HI) / s

    def float_to_storage(self, x) -> np.ndarray:
        """The uint16 storage lanes of values (clip, round half to even; dtype.py:391-395)."""
        c = np.clip(np.asarray(x, np.float64), self.min_val, self.max_val)
        return np.round(c * self.scale).astype(np.int16).view(np.uint16)

    def exp_to_storage(self, x, f) -> np.ndarray:
        """The uint16 storage lanes of values at 2^-f: round half to even, saturate
        (dtype.py:436-439)."""
        s = np.power(2.0, np.asarray(f, np.float64))
        r = np.clip(np.round(np.asarray(x, np.float64) * s), I16_LO, I16_HI)
        return r.astype(np.int16).view(np.uint16)

    def int_to_storage(self, x) -> np.ndarray:
        """The uint16 lanes of integer values (ids, masks): the raw integers themselves,
        truncated toward zero and saturated."""
        r = np.clip(np.trunc(np.asarray(x, np.float64)), I16_LO, I16_HI)
        return r.astype(np.int16).view(np.uint16)

    def dat_bytes(self, data) -> bytes:
        """The little-endian bytes of a .dat file: float_to_storage of the flattened values
        (dtype.py:397-400)."""
        return self.float_to_storage(np.asarray(data, np.float64).reshape(-1)).astype("<u2").tobytes()

    def ramp_to_float(self, positions) -> np.ndarray:
        """The value of the test harness's fill p[pos] = (Data_t)(pos & 0xFFFF) (dtype.py:385-389)."""
        raw = (np.asarray(positions, np.int64) & 0xFFFF).astype(np.uint16).view(np.int16)
        return raw.astype(np.float64) / self.scale

    def ramp_to_float_exp(self, positions, f) -> np.ndarray:
        """The ramp fill's value at 2^-f (dtype.py:441-443)."""
        raw = (np.asarray(positions, np.int64) & 0xFFFF).astype(np.uint16).view(np.int16)
        return raw.astype(np.float64) / np.power(2.0, np.asarray(f, np.float64))

    def format_literal(self, storage_val) -> str:
        """A storage lane as a C literal, 0x%04X (dtype.py:417-419)."""
        return f"0x{int(storage_val) & 0xFFFF:04X}"

    def quantize_exp(self, x, f) -> np.ndarray:
        """round half to even at 2^-f, saturate, NaN -> 0 (dtype.py:278-285)."""
        s = np.power(2.0, np.asarray(f, np.float64))
        x = np.asarray(x, np.float64)
        r = np.round(np.where(np.isnan(x), 0.0, x) * s)
        return np.clip(r, I16_LO, I16_HI) / s

    # -- raw lanes ------------------------------------------------------------------------
    def to_raw(self, values, f=None) -> np.ndarray:
        """Raw int16 of values on the 2^-f grid (f = F by default): rint(v * 2^f), saturated.
        Values off the grid are rounded half to even (float_to_storage / exp_to_storage)."""
        s = np.power(2.0, np.asarray(self.F if f is None else f, np.float64))
        r = np.round(np.asarray(values, np.float64) * s)
        return np.clip(r, I16_LO, I16_HI).astype(np.int16)

    def from_raw(self, raw, f=None) -> np.ndarray:
        """float64 values raw * 2^-f."""
        s = np.power(2.0, np.asarray(self.F if f is None else f, np.float64))
        return np.asarray(raw, np.float64) / s


AP_FIXED_16_8 = ApFixed16(8)
