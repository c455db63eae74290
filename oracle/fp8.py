"""OCP FP8 E4M3 ("e4m3fn") decoding and encoding for the fp8 KV-cache tests.

TEST INFRASTRUCTURE ONLY: imported by tests/ (and nothing under decode-kernel_amd/).

The reference caches fp16 only; an fp8 cache is this library's extension, so there is no
reference file to follow. The format is the OCP 8-bit Floating Point Specification
(OFP8, v1.0, 2023), E4M3 variant, restated from its definition:

  bit 7 sign, bits 6..3 exponent e (bias 7), bits 2..0 mantissa m;
  e == 0          -> subnormal  (-1)^s * (m / 8) * 2^-6     (smallest 2^-9)
  e == 15, m == 7 -> NaN (0x7F, 0xFF); there are no infinities
  otherwise       -> normal     (-1)^s * (1 + m / 8) * 2^(e - 7)  (largest 448)

The attention oracle runs on the dequantised cache: K = k_scale * decode(code),
V = v_scale * decode(code), per tensor.

Pinned by tests/test_oracle.py: known answers from the specification's table (0x38 = 1,
0x7E = 448, 0x08 = 2^-6, 0x01 = 2^-9, 0x80 = -0, 0x7F NaN), the count of finite values,
and all 256 codes against torch.float8_e4m3fn's own conversion; `encode` against torch's
float32 -> float8_e4m3fn rounding on a dense sweep including every midpoint.
"""
from __future__ import annotations

import numpy as np

MAX = 448.0


def decode(codes) -> np.ndarray:
    """float64 values of uint8 E4M3 codes (NaN for 0x7F / 0xFF)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = (c & 0x7).astype(np.float64)
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = sign * mag
    return np.where((e == 15) & ((c & 0x7) == 7), np.nan, val)


def _finite_table():
    codes = np.arange(0x7F, dtype=np.uint8)          # 0x00..0x7E: every non-negative finite
    return codes, decode(codes)


def encode(x) -> np.ndarray:
    """uint8 E4M3 codes of float values: round to nearest, ties to the even code; a
    magnitude that rounds above 448 becomes NaN (0x7F with the sign), as does NaN."""
    x = np.asarray(x, dtype=np.float64)
    codes, vals = _finite_table()
    a = np.abs(x)
    hi = np.searchsorted(vals, a, side="left").clip(1, len(vals) - 1)   # vals[hi] >= a
    lo = hi - 1
    d_lo, d_hi = a - vals[lo], vals[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (codes[hi] % 2 == 0))
    out = np.where(pick_hi, codes[hi], codes[lo]).astype(np.uint8)
    out = np.where(a <= vals[0], 0, out).astype(np.uint8)
    # above the largest value: 448 up to and including the midpoint 464 toward the next
    # (absent) step 480, whose code would be odd; NaN beyond
    over = a > MAX
    out = np.where(over & (a <= 464.0), 0x7E, out)
    out = np.where(over & (a > 464.0), 0x7F, out)
    out = np.where(np.isnan(x), 0x7F, out).astype(np.uint8)
    return out | np.where(np.signbit(x), 0x80, 0).astype(np.uint8)


def encode_saturating(x) -> np.ndarray:
    """encode() of x clamped to [-448, 448] (NaN stays NaN): the cache-write rounding."""
    return encode(np.clip(np.asarray(x, np.float64), -MAX, MAX))


def signed_rank(codes) -> np.ndarray:
    """Position of each finite code on the number line in code steps (+-0 -> 0), so two
    codes are neighbours iff their ranks differ by 1."""
    c = np.asarray(codes, np.uint8).astype(np.int64)
    return np.where(c & 0x80, -(c & 0x7F), c & 0x7F)


def dequantize(codes, scale: float) -> np.ndarray:
    """float32 scale * decode(codes), the values the kernel attends over."""
    return (decode(codes) * np.float64(scale)).astype(np.float32)
