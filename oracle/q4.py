"""Affine 4-bit (Q4) packing, dequantisation and quantised matmuls (test infrastructure).

Semantics restated from the reference:

* nibble order: value ``k`` of a row lives in word ``k >> 3`` at bit offset
  ``4 * (k & 7)``, LSB first (``models/flashnext/metal_runtime.py:980``; the
  packer at ``models/flashnext/tests/unit/test_metal_runtime_g64.py:16-26``).
* dequant: ``w = scale[g] * q + bias[g]`` with ``g = k // group_size``
  (``metal_runtime.py:975-986``), scales/biases stored as bf16.
* QMV: ``y[t, o] = sum_g scale[o,g] * sum_i x_i q_i + bias[o,g] * sum_i x_i``
  accumulated in float and rounded once to the activation dtype
  (``metal_runtime.py:955-987``, the reference's ``_numpy_projection``).
* ``quantized_matmul`` / ``gather_qmm`` (MLX op semantics with
  ``transpose=True``) as used at ``models/flashnext/expert_cache.py:799-810``.
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16, f64_to_bf16


def pack_q4(q) -> np.ndarray:
    """Pack integers 0..15 along the last axis into uint32 words, LSB first.

    Restates the packer in ``tests/unit/test_metal_runtime_g64.py:16-26``.
    """
    q = np.asarray(q)
    if q.shape[-1] % 8:
        raise ValueError("last dimension must be a multiple of 8")
    words = q.shape[-1] // 8
    out = np.zeros(q.shape[:-1] + (words,), dtype=np.uint32)
    for k in range(8):
        out |= (q[..., k::8].astype(np.uint32) & np.uint32(15)) << np.uint32(4 * k)
    return out


def unpack_q4(words, count: int | None = None) -> np.ndarray:
    """Inverse of :func:`pack_q4`: ``q = (w[k >> 3] >> 4 (k & 7)) & 15``.

    Restates the unpack expression of ``metal_runtime.py:980``.
    """
    w = np.asarray(words, dtype=np.uint32)
    n = w.shape[-1] * 8 if count is None else int(count)
    out = np.empty(w.shape[:-1] + (w.shape[-1] * 8,), dtype=np.uint8)
    for k in range(8):
        out[..., k::8] = ((w >> np.uint32(4 * k)) & np.uint32(15)).astype(np.uint8)
    return out[..., :n]


def quantize_affine(weights, group_size: int = 32):
    """Quantise float weights to (packed uint32, bf16 scales, bf16 biases).

    Fixture generator only (not a reference function): per group
    ``bias = min``, ``scale = (max - min) / 15`` (both rounded to bf16) and
    ``q = clip(round((w - bias) / scale), 0, 15)``.  Parity never depends on
    how the packed tensors were made: both sides consume the same bytes.
    """
    w = np.asarray(weights, dtype=np.float32)
    if w.shape[-1] % group_size:
        raise ValueError("input width must be a multiple of group_size")
    groups = w.reshape(w.shape[:-1] + (w.shape[-1] // group_size, group_size))
    lo = groups.min(axis=-1)
    hi = groups.max(axis=-1)
    scale = np.maximum((hi - lo) / 15.0, 1e-8).astype(np.float32)
    scale_bits = f32_to_bf16(scale)
    bias_bits = f32_to_bf16(lo)
    s = bf16_to_f32(scale_bits)[..., None]
    b = bf16_to_f32(bias_bits)[..., None]
    q = np.clip(np.rint((groups - b) / s), 0, 15).astype(np.uint8)
    return pack_q4(q.reshape(w.shape)), scale_bits, bias_bits


def dequantize_f64(packed, scales, biases, group_size: int = 32) -> np.ndarray:
    """Exact dequantised values ``s*q + b`` as float64 (s, b given as bf16 bits)."""
    q = unpack_q4(packed).astype(np.float64)
    s = np.repeat(bf16_to_f32(scales).astype(np.float64), group_size, axis=-1)
    b = np.repeat(bf16_to_f32(biases).astype(np.float64), group_size, axis=-1)
    return s * q + b


def dequantize_bf16(packed, scales, biases, group_size: int = 32) -> np.ndarray:
    """Dequantised weights as bf16 bits: float32 ``s*q + b`` (one rounding) then RNE.

    ``s*q`` is exact in float32 (8-bit by 4-bit significands), so the float32
    sum has one rounding; this is the value MLX's affine dequantise produces
    in float before storing bf16.
    """
    q = unpack_q4(packed).astype(np.float32)
    s = np.repeat(bf16_to_f32(scales), group_size, axis=-1)
    b = np.repeat(bf16_to_f32(biases), group_size, axis=-1)
    return f32_to_bf16(s * q + b)


def qmv_f64(x, packed, scales, biases, group_size: int = 32) -> np.ndarray:
    """``x @ dequant(W).T`` accumulated in float64, before output rounding.

    ``x``: float array ``[T, K]``; ``packed``: ``[N, K/8]``.  Returns ``[T, N]``
    float64.  Restates ``_numpy_projection`` (``metal_runtime.py:955-987``):
    ``sum_g s*sum(x q) + b*sum(x)`` equals ``sum_k x_k (s q_k + b)`` exactly in
    real arithmetic; both are float64 here.
    """
    dense = dequantize_f64(packed, scales, biases, group_size)
    return np.asarray(x, dtype=np.float64) @ dense.T


def quantized_matmul(x_bits, packed, scales, biases, group_size: int = 32,
                     out="bf16"):
    """MLX ``quantized_matmul(x, w, s, b, transpose=True)`` on bf16 activations.

    Returns bf16 bits (``out="bf16"``) or float32 (``out="f32"``) of
    ``x @ dequant(w).T`` computed with float64 accumulation.
    """
    x = bf16_to_f32(x_bits)
    y = qmv_f64(x, packed, scales, biases, group_size)
    if out == "f32":
        return y.astype(np.float32)
    return f64_to_bf16(y)


class ExpertBank:
    """Per-expert Q4 projection bank ``[E, O, I/8]`` with a dequant cache."""

    def __init__(self, packed, scales, biases, group_size: int = 32):
        self.packed = np.asarray(packed, dtype=np.uint32)
        self.scales = np.asarray(scales, dtype=np.uint16)
        self.biases = np.asarray(biases, dtype=np.uint16)
        self.group_size = int(group_size)
        self._dense: dict[int, np.ndarray] = {}

    @property
    def out_width(self) -> int:
        return int(self.packed.shape[1])

    @property
    def in_width(self) -> int:
        return int(self.packed.shape[2]) * 8

    def dense(self, expert: int) -> np.ndarray:
        cached = self._dense.get(int(expert))
        if cached is None:
            cached = dequantize_f64(
                self.packed[expert], self.scales[expert], self.biases[expert],
                self.group_size,
            )
            self._dense[int(expert)] = cached
        return cached

    def dense_bf16(self, expert: int) -> np.ndarray:
        """Weights as bf16 MFMA tiles hold them: bf16(fma_f32(q, s, b)), as float64."""
        key = ("bf16", int(expert))
        cached = self._dense.get(key)
        if cached is None:
            q = unpack_q4(self.packed[expert]).astype(np.float64)
            s = np.repeat(bf16_to_f32(self.scales[expert]).astype(np.float64), self.group_size, axis=-1)
            b = np.repeat(bf16_to_f32(self.biases[expert]).astype(np.float64), self.group_size, axis=-1)
            # q*s + b is exact in float64 (4-bit q, 8-bit s, b aligned); one
            # rounding to float32 reproduces the fused multiply-add.
            cached = bf16_to_f32(f32_to_bf16((q * s + b).astype(np.float32))).astype(np.float64)
            self._dense[key] = cached
        return cached

    def project(self, x_f, expert: int, weights: str = "exact") -> np.ndarray:
        """float64 ``x @ W_e.T`` for rows ``x_f`` ``[n, I]``.

        ``weights="exact"`` uses the exact dequantized weights; ``"bf16"``
        uses them rounded to bf16 first (the grouped GEMM's MFMA tiles).
        """
        w = self.dense(expert) if weights == "exact" else self.dense_bf16(expert)
        return np.asarray(x_f, dtype=np.float64) @ w.T


def gather_qmm(x_bits, bank: ExpertBank, rhs_indices, weights: str = "exact") -> np.ndarray:
    """MLX ``gather_qmm(x, w, s, b, rhs_indices, transpose=True)`` for 2-D rows.

    ``x_bits``: bf16 ``[N, K]`` (one row per gathered product);
    ``rhs_indices``: ``[N]`` expert ids.  Returns bf16 ``[N, O]``, each row
    ``bf16(x_row . W_e)`` with the dot product in float64 over the exact
    dequantized weights (``weights="exact"``) or over the weights rounded to
    bf16 first (``"bf16"``, the MFMA tiles of the grouped GEMM).  Sorting the
    rows (``sorted_indices=True``) does not change any row's value.
    """
    x = bf16_to_f32(x_bits).astype(np.float64)
    idx = np.asarray(rhs_indices).reshape(-1)
    out = np.empty((idx.size, bank.out_width), dtype=np.float64)
    for e in np.unique(idx):
        rows = np.nonzero(idx == e)[0]
        out[rows] = bank.project(x[rows], int(e), weights)
    return f64_to_bf16(out)
