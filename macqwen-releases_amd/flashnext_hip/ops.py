"""MLX-compatible quantized operators on the gfx950 library.

``quantized_matmul`` and ``gather_qmm`` keep MLX's argument meaning for the
affine 4-bit format the reference uses (``transpose=True``, ``bits=4``,
``mode="affine"``; ``models/flashnext/expert_cache.py:799-810``,
``models/flashnext/loader.py:190-217``).  Every call runs a HIP kernel from
``libmqmoe.so``; there is no host fallback.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._tensors import act_dtype, half16, ptr, require_cuda, stream_handle, words32

SUPPORTED_GROUP_SIZES = (32, 64)


def _check_format(bits: int, group_size: int, mode: str, transpose: bool) -> None:
    if bits != 4:
        raise ValueError(f"only 4-bit weights are supported (got bits={bits})")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError(f"group_size must be one of {SUPPORTED_GROUP_SIZES}")
    if mode != "affine":
        raise ValueError(f"only affine quantization is supported (got {mode!r})")
    if not transpose:
        raise ValueError("only transpose=True (x @ w.T) is supported")


def unpack(words: torch.Tensor) -> torch.Tensor:
    """uint8 nibble values ``[..., 8*n]`` of packed words ``[..., n]``."""
    w = words32(words, "words")
    out = torch.empty(w.shape[:-1] + (w.shape[-1] * 8,), dtype=torch.uint8, device=w.device)
    lib = _lib.load()
    _lib.check(lib.mq_q4_unpack(ptr(w), ptr(out), w.numel(), stream_handle()), lib)
    return out


def dequantize(weight, scales, biases, group_size: int = 32, bits: int = 4) -> torch.Tensor:
    """``mx.dequantize`` for 2-D or 3-D packed weights -> bf16 ``[..., out, in]``."""
    _check_format(bits, group_size, "affine", True)
    w = words32(weight, "weight")
    s = half16(scales, "scales")
    b = half16(biases, "biases")
    cols = w.shape[-1] * 8
    rows = w.numel() // w.shape[-1]
    if s.shape[:-1] != w.shape[:-1] or s.shape[-1] * group_size != cols or b.shape != s.shape:
        raise ValueError("scales/biases do not match the packed weight shape")
    out = torch.empty(w.shape[:-1] + (cols,), dtype=torch.bfloat16, device=w.device)
    lib = _lib.load()
    _lib.check(lib.mq_q4_dequant(ptr(w), ptr(s), ptr(b), ptr(out), rows, cols, group_size,
                                 stream_handle()), lib)
    return out


def quantized_matmul(x, w, scales, biases, transpose: bool = True, group_size: int = 32,
                     bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """``mx.quantized_matmul(x, w, scales, biases, transpose=True)``: ``x @ dequant(w).T``."""
    _check_format(bits, group_size, mode, transpose)
    x = require_cuda(x, "x")
    dt = act_dtype(x)
    w = words32(w, "w")
    s = half16(scales, "scales")
    b = half16(biases, "biases")
    if w.dim() != 2:
        raise ValueError("w must be [out, in/8]")
    n, k = w.shape[0], w.shape[1] * 8
    if x.shape[-1] != k:
        raise ValueError(f"x width {x.shape[-1]} != weight input width {k}")
    if s.shape != (n, k // group_size) or b.shape != s.shape:
        raise ValueError("scales/biases do not match the packed weight shape")
    rows = int(math.prod(x.shape[:-1]))
    y = torch.empty(x.shape[:-1] + (n,), dtype=x.dtype, device=x.device)
    if rows == 0:
        return y
    lib = _lib.load()
    _lib.check(lib.mq_q4_qmv(ptr(x), dt, ptr(w), ptr(s), ptr(b), ptr(y), rows, n, k, group_size,
                             stream_handle()), lib)
    return y


def swiglu(gate, up, *, scalar: bool = False) -> torch.Tensor:
    """MLX ``swiglu(gate, up)`` with the fused Up epilogue's rounding points
    (``models/flashnext/metal_runtime.py:278-287, 895-907``): every step rounded
    to the input dtype.  ``scalar`` selects the per-element device sequence of
    the decode kernels instead of the four-at-a-time one of the grouped kernels
    (bit-identical)."""
    g = require_cuda(gate, "gate")
    u = require_cuda(up, "up")
    dt = act_dtype(g, "gate")
    if u.dtype != g.dtype or u.shape != g.shape:
        raise ValueError("gate and up must have the same shape and dtype")
    out = torch.empty_like(g)
    lib = _lib.load()
    _lib.check(lib.mq_swiglu(ptr(g), ptr(u), ptr(out), g.numel(), dt,
                             _lib.MQ_SWIGLU_SCALAR if scalar else 0, stream_handle()), lib)
    return out


def sigmoid(x) -> torch.Tensor:
    """``mx.sigmoid`` with every step of the sequence rounded to x's dtype
    (the shared-expert gate, ``models/flashnext/adaptive_topk.py:264``)."""
    x = require_cuda(x, "x")
    dt = act_dtype(x)
    out = torch.empty_like(x)
    lib = _lib.load()
    _lib.check(lib.mq_sigmoid(ptr(x), ptr(out), x.numel(), dt, stream_handle()), lib)
    return out


def dense_projection(weight, scales, biases) -> "_lib.MqProjection":
    """MqProjection over dense expert arrays ``[E, out, in/8]``."""
    p = _lib.MqProjection()
    p.weight, p.scales, p.biases = ptr(weight), ptr(scales), ptr(biases)
    return p


def gather_qmm(x, w, scales, biases, lhs_indices=None, rhs_indices=None, transpose: bool = True,
               group_size: int = 32, bits: int = 4, mode: str = "affine",
               sorted_indices: bool = False) -> torch.Tensor:
    """``mx.gather_qmm``: ``out[b] = x[lhs[b]] @ dequant(w[rhs[b]]).T``.

    ``x``: ``[*Bx, M, K]``; ``w``: ``[E, N, K/8]``; indices broadcast with the
    batch shape.  Returns ``[*B, M, N]`` in x's dtype.  ``sorted_indices`` is a
    scheduling hint that does not change any value.
    """
    _check_format(bits, group_size, mode, transpose)
    x = require_cuda(x, "x")
    dt = act_dtype(x)
    w = words32(w, "w")
    s = half16(scales, "scales")
    b = half16(biases, "biases")
    if w.dim() != 3:
        raise ValueError("w must be [experts, out, in/8]")
    experts, n, k = w.shape[0], w.shape[1], w.shape[2] * 8
    if x.dim() < 2 or x.shape[-1] != k:
        raise ValueError("x must be [..., M, K] with K matching the weights")
    m = x.shape[-2]
    bx = x.shape[:-2]
    if lhs_indices is not None:
        lhs = require_cuda(lhs_indices, "lhs_indices").to(torch.int64)
        flat_x = x.reshape(-1, m, k)
        x = flat_x[lhs.reshape(-1)].reshape(lhs.shape + (m, k))
        bx = lhs.shape
    if rhs_indices is None:
        rhs = torch.arange(experts, device=x.device)[: max(1, int(math.prod(bx)))].reshape(bx) \
            if len(bx) else torch.zeros((), dtype=torch.int64, device=x.device)
    else:
        rhs = require_cuda(rhs_indices, "rhs_indices")
    batch = torch.broadcast_shapes(tuple(bx), tuple(rhs.shape))
    xb = x.expand(batch + (m, k)).contiguous()
    rb = rhs.to(torch.int64).expand(batch).reshape(-1)
    if rb.numel() and (int(rb.min()) < 0 or int(rb.max()) >= experts):
        raise ValueError("rhs_indices contain an expert outside the weight bank")
    routes = rb.repeat_interleave(m).to(torch.int32).contiguous()
    pairs = routes.numel()
    out = torch.empty(batch + (m, n), dtype=x.dtype, device=x.device)
    if pairs == 0:
        return out
    proj = dense_projection(w, s, b)
    lib = _lib.load()
    _lib.check(lib.mq_gather_qmv(ptr(xb), dt, 1, proj, ptr(routes), ptr(out), pairs, 1, k, n,
                                 experts, group_size, stream_handle()), lib)
    return out
