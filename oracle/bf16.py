"""bfloat16 bit-pattern helpers (oracle; test infrastructure only).

Restates ``quant/q4nx.py:32-124`` (``to_bf16_u16``, ``bf16_to_f32``,
``bf16_floor``, ``bf16_ceil``, ``bf16_nextafter``) and the NumPy branch of
``host/weights.py:104-123`` (``f32_to_bf16_rtne``: same rounding, NaN -> 0x7FC0).

bf16 values travel as ``uint16`` bit patterns, as everywhere in the reference.

Pins:
* ``f32_to_bf16``: equals torch's float32->bfloat16 conversion (IEEE RNE) on
  every finite value of a dense sweep, plus the tie cases of
  ``quant/test_q4nx.py:521-531`` (1+2^-8 -> 0x3F80, 1+2^-7+2^-8 -> 0x3F82) and
  NaN -> 0x7FC0 (tests/test_oracle_bf16.py).
* ``bf16_floor``/``bf16_ceil``/``bf16_next_up``: brute force against the sorted
  set of all finite bf16 values (tests/test_oracle_bf16.py), plus the property
  checks of ``quant/test_q4nx.py:56-106``.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "f32_to_bf16",
    "bf16_to_f32",
    "bf16_round",
    "bf16_floor",
    "bf16_ceil",
    "bf16_next_up",
]


def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bits with round-to-nearest-even; every NaN becomes 0x7FC0.

    Follows ``quant/q4nx.py:32-44`` / ``host/weights.py:104-115``: add
    ``0x7FFF + lsb`` to the float32 bits and keep the high half.
    """
    a = np.ascontiguousarray(x, dtype=np.float32)
    bits = a.view(np.uint32)
    lsb = (bits >> np.uint32(16)) & np.uint32(1)
    out = ((bits + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        out[nan] = 0x7FC0
    return out


def bf16_to_f32(u16) -> np.ndarray:
    """bf16 bits -> float32 (exact: the bits become the high half). ``quant/q4nx.py:47-49``."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x) -> np.ndarray:
    """float32 values rounded (RNE) onto the bf16 grid. ``quant/q4nx.py:52-54``."""
    return bf16_to_f32(f32_to_bf16(x))


def _narrow_f64(x: np.ndarray, toward_pos: bool) -> np.ndarray:
    """float64 -> float32 rounded toward -inf (``toward_pos`` False) or +inf.

    ``quant/q4nx.py:61-64,87-90``: convert with RNE, then step one float32 ulp when
    the conversion went the wrong way.
    """
    f = x.astype(np.float32)
    if toward_pos:
        wrong = f.astype(np.float64) < x
        return np.where(wrong, np.nextafter(f, np.float32(np.inf)), f)
    wrong = f.astype(np.float64) > x
    return np.where(wrong, np.nextafter(f, np.float32(-np.inf)), f)


def _directed(x, toward_pos: bool):
    arr = np.asarray(x)
    scalar = arr.ndim == 0
    if arr.dtype == np.float64:
        f32 = _narrow_f64(arr, toward_pos)
    else:
        f32 = np.ascontiguousarray(arr, dtype=np.float32)
    f32 = np.atleast_1d(np.asarray(f32, dtype=np.float32))
    bits = f32.view(np.uint32)
    negative = (bits >> np.uint32(31)) == 1
    has_tail = (bits & np.uint32(0xFFFF)) != 0
    # Truncation of the low half moves toward zero; step away from zero when that
    # is the requested direction (positive for ceil, negative for floor).
    bump = has_tail & (~negative if toward_pos else negative)
    hi = (bits >> np.uint32(16)) + bump.astype(np.uint32)
    out = (hi.astype(np.uint32) << np.uint32(16)).view(np.float32).copy()
    nan = np.isnan(f32)
    if nan.any():
        out[nan] = np.nan
    out = out.reshape(np.shape(arr))
    return out.item() if scalar else out


def bf16_floor(x):
    """Greatest bf16 value <= x (float32 or float64 input). ``quant/q4nx.py:57-80``."""
    return _directed(x, toward_pos=False)


def bf16_ceil(x):
    """Smallest bf16 value >= x (float32 or float64 input). ``quant/q4nx.py:83-106``."""
    return _directed(x, toward_pos=True)


def bf16_next_up(x):
    """Next bf16 value toward +inf from an exact bf16 value. ``quant/q4nx.py:109-124``.

    -0 is treated as +0; the successor of 0 is the smallest positive subnormal
    (0x0001); negative values step toward zero, and -min_subnormal steps to +0.
    """
    arr = np.asarray(x, dtype=np.float32)
    scalar = arr.ndim == 0
    hi = (np.atleast_1d(arr).view(np.uint32) >> np.uint32(16)).astype(np.int64)
    hi = np.where(hi == 0x8000, 0, hi)
    neg = (hi & 0x8000) != 0
    nxt = np.where(hi == 0, 1, np.where(neg, np.where(hi == 0x8001, 0, hi - 1), hi + 1))
    out = (nxt.astype(np.uint32) << np.uint32(16)).view(np.float32).reshape(arr.shape)
    return out.item() if scalar else out
