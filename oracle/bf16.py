"""bfloat16 helpers on numpy uint16 bit patterns (test infrastructure).

numpy has no bfloat16 dtype, so bf16 tensors are carried as ``uint16`` bit
patterns.  Two roundings are provided:

* ``f32_to_bf16``: round-to-nearest-even from float32, the rounding every
  ``static_cast<bfloat>(float)`` in the reference's Metal kernels performs
  (``metal_runtime.py:267-336``).
* ``f64_to_bf16``: correctly rounded (nearest-even) from float64 with a single
  rounding.  Implemented via round-to-odd to float32 followed by RNE to bf16,
  which is exact because float32 carries more than bf16's 8 + 2 bits.
"""
from __future__ import annotations

import numpy as np


def bf16_to_f32(bits) -> np.ndarray:
    """Widen bf16 bit patterns to float32 values (exact)."""
    raw = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return raw.view(np.float32)


def f32_to_bf16(values) -> np.ndarray:
    """Round float32 values to bf16 bit patterns, nearest-even; NaN -> 0x7FC0."""
    arr = np.asarray(values, dtype=np.float32)
    f = np.ascontiguousarray(arr).reshape(arr.shape)
    u = f.view(np.uint32).astype(np.uint64)
    bias = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
    out = ((u + bias) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(f)
    if np.any(nan):
        out = np.where(nan, np.uint16(0x7FC0) | (((u >> np.uint64(16)) & np.uint64(0x8000)).astype(np.uint16)), out)
    return out.astype(np.uint16)


def _f64_to_f32_round_to_odd(values) -> np.ndarray:
    d = np.asarray(values, dtype=np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        t = d.astype(np.float32)
    # Step toward zero where RNE rounded away from zero (gives truncation).
    with np.errstate(invalid="ignore"):
        away = np.isfinite(d) & (np.abs(t.astype(np.float64)) > np.abs(d))
    bits = t.view(np.uint32).copy()
    bits = np.where(away, bits - np.uint32(1), bits)
    t = bits.view(np.float32)
    with np.errstate(invalid="ignore"):
        inexact = np.isfinite(d) & (t.astype(np.float64) != d)
    bits = np.where(inexact, bits | np.uint32(1), bits)
    return bits.view(np.float32)


def f64_to_bf16(values) -> np.ndarray:
    """Round float64 values to bf16 with a single nearest-even rounding."""
    return f32_to_bf16(_f64_to_f32_round_to_odd(values))


def round_bf16_f32(values) -> np.ndarray:
    """float32 values rounded through bf16 (RNE) and widened back."""
    return bf16_to_f32(f32_to_bf16(values))


def bf16_from_float(values) -> np.ndarray:
    """Convenience: any float array -> bf16 bits via float32 RNE."""
    return f32_to_bf16(np.asarray(values, dtype=np.float32))
