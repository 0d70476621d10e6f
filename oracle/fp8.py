"""OCP fp8 e4m3fn quantisation at the bit level (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

The reference has no fp8 path (its README only names the Hadamard functions),
so the per-(b, h) absmax scheme is the build's own definition:

* ``amax = max |x|`` over one (b, h) slice of the rotated bf16 tensor,
* ``inv = fp32(448 / amax)`` (correctly rounded fp32 division; amax == 0
  gives ``inv = 1``), dequant scale ``sigma = fp32(amax / 448)``,
* ``x8 = e4m3(clamp(fp32(x * inv), -448, 448))`` with round-to-nearest-even.

e4m3fn: 1 sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities,
max finite 448, smallest subnormal 2^-9.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn byte, RNE, saturating at +-448; NaN -> 0x7f."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 31) & 1).astype(np.uint8)
    a = np.abs(x).astype(np.float64)
    out = np.zeros(x.shape, dtype=np.uint8)
    nan = np.isnan(x)
    a = np.where(nan, 0.0, np.minimum(a, E4M3_MAX))
    # exponent of the value in the e4m3 grid; subnormal range shares 2^-6's step
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.clip(e, -6, 8)
    step = np.exp2(e - 3)  # spacing of representable values in this binade
    q = a / step  # exact in fp64 for fp32 inputs
    fl = np.floor(q)
    frac = q - fl
    up = (frac > 0.5) | ((frac == 0.5) & (np.mod(fl, 2) == 1))
    m = fl + up  # integer multiple of step, may carry into the next binade
    val = m * step
    # re-derive exponent / mantissa from the rounded value
    with np.errstate(divide="ignore"):
        e2 = np.floor(np.log2(np.where(val > 0, val, 1.0)))
    sub = val < 2.0 ** -6
    exp_field = np.where(sub, 0, e2 + 7).astype(np.int64)
    mant = np.where(sub, np.round(val / 2.0 ** -9), np.round((val / np.exp2(e2) - 1.0) * 8)).astype(np.int64)
    mag = np.where(val == 0, 0, (exp_field << 3) | mant).astype(np.uint8)
    out = (sign << 7) | mag
    out = np.where(nan, np.uint8(0x7F), out).astype(np.uint8)
    return out


def e4m3_decode(b: np.ndarray) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return (s * val).astype(np.float32)


def quantize_per_head(x: np.ndarray):
    """``x`` fp32 ``[B, H, T, d]`` (bf16 values) -> ``(bytes, sigma [B, H])``."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=(2, 3)).astype(np.float32)
    safe = np.where(amax > 0, amax, np.float32(E4M3_MAX)).astype(np.float32)
    inv = (np.float32(E4M3_MAX) / safe).astype(np.float32)
    sigma = (safe / np.float32(E4M3_MAX)).astype(np.float32)
    y = (x * inv[:, :, None, None]).astype(np.float32)
    y = np.clip(y, -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3_encode(y), sigma
