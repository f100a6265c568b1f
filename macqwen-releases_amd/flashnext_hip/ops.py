"""MLX-compatible quantized operators on the gfx950 library.

``quantized_matmul`` and ``gather_qmm`` keep MLX's argument meaning for the
affine 4-bit format the reference uses (``transpose=True``, ``bits=4``,
``mode="affine"``; ``models/flashnext/expert_cache.py:799-810``,
``models/flashnext/loader.py:190-217``).  Every call runs a HIP kernel from
``libmqmoe.so``; there is no host fallback.
"""
from __future__ import annotations

import ctypes
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


def swiglu(gate, up, *, scalar: bool = False, table: bool = False) -> torch.Tensor:
    """MLX ``swiglu(gate, up)`` with the fused Up epilogue's rounding points
    (``models/flashnext/metal_runtime.py:278-287, 895-907``): every step rounded
    to the input dtype.  ``scalar`` selects the per-element device sequence of
    the decode kernels and ``table`` the grouped gate/up epilogue's sequence
    with the sigmoid looked up in a table, instead of the four-at-a-time one
    (all bit-identical)."""
    g = require_cuda(gate, "gate")
    u = require_cuda(up, "up")
    dt = act_dtype(g, "gate")
    if u.dtype != g.dtype or u.shape != g.shape:
        raise ValueError("gate and up must have the same shape and dtype")
    out = torch.empty_like(g)
    lib = _lib.load()
    flags = (_lib.MQ_SWIGLU_SCALAR if scalar else 0) | (_lib.MQ_SWIGLU_TABLE if table else 0)
    _lib.check(lib.mq_swiglu(ptr(g), ptr(u), ptr(out), g.numel(), dt, flags, stream_handle()), lib)
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


# Row count from which bf16 gather calls run as grouped MFMA GEMMs over rows
# sorted by expert; below it, each row is a GEMV.  The reference sorts from
# the same size (`indices.size >= 64`, models/flashnext/expert_cache.py:1793).
GROUPED_MIN_ROWS = 64


def gather_qmm(x, w, scales, biases, lhs_indices=None, rhs_indices=None, transpose: bool = True,
               group_size: int = 32, bits: int = 4, mode: str = "affine",
               sorted_indices: bool = False) -> torch.Tensor:
    """``mx.gather_qmm``: ``out[b] = x[lhs[b]] @ dequant(w[rhs[b]]).T``.

    ``x``: ``[*Bx, M, K]``; ``w``: ``[E, N, K/8]``.  As in MLX, ``lhs_indices``
    defaults to every batch of x and ``rhs_indices`` to every expert, and the
    two broadcast to the output batch.  Returns ``[*B, M, N]`` in x's dtype.
    ``sorted_indices`` is a scheduling hint that does not change any value.

    bf16 calls of at least ``GROUPED_MIN_ROWS`` rows with K a multiple of 128
    (the prefill / verify shape: x ``[T*k, 1, H]`` after the sort,
    models/flashnext/expert_cache.py:787-810, 1790-1806) run as one grouped
    MFMA GEMM (``mq_gather_qmm``); the rest run one GEMV per row
    (``mq_gather_qmv``).  Neither path copies x per row or waits for the
    device: an expert index outside the bank raises a device flag that
    ``check_device_errors()`` reports, and its row reads zero weights.
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
    if s.shape != (experts, n, k // group_size) or b.shape != s.shape:
        raise ValueError("scales/biases do not match the packed weight shape")
    dev = x.device
    m = x.shape[-2]
    bx = tuple(x.shape[:-2])
    x_batches = int(math.prod(bx))
    lhs = (torch.arange(x_batches, device=dev).reshape(bx) if lhs_indices is None
           else require_cuda(lhs_indices, "lhs_indices"))
    rhs = (torch.arange(experts, device=dev) if rhs_indices is None
           else require_cuda(rhs_indices, "rhs_indices"))
    batch = torch.broadcast_shapes(tuple(lhs.shape), tuple(rhs.shape))
    out = torch.empty(batch + (m, n), dtype=x.dtype, device=dev)
    rows = int(math.prod(batch)) * m
    if rows == 0:
        return out
    if rows >= 2 ** 31:
        raise ValueError("too many rows")
    # Route word of every output row (b, j): rhs[b], as int32 (an index
    # outside [0, experts) becomes a word that addresses nothing).
    routes = rhs.expand(batch).reshape(-1, 1).expand(-1, m).to(torch.int32).contiguous()
    # x row of every output row: lhs[b] * M + j, unless that is the identity.
    identity = lhs_indices is None and tuple(batch) == bx
    x_rows = None
    if not identity:
        x_rows = (lhs.expand(batch).reshape(-1, 1).to(torch.int64) * m
                  + torch.arange(m, device=dev)).to(torch.int32).reshape(-1)
    proj = dense_projection(w, s, b)
    lib = _lib.load()
    x2 = x.reshape(-1, k)
    if dt == _lib.MQ_BF16 and rows >= GROUPED_MIN_ROWS and k % 128 == 0 and n % 4 == 0:
        a = _lib.MqGatherArgs()
        a.x, a.x_rows, a.routes, a.out = ptr(x2), ptr(x_rows), ptr(routes), ptr(out)
        a.w = proj
        a.x_count, a.rows, a.in_width, a.out_width = x2.shape[0], rows, k, n
        a.expert_count, a.group_size = experts, group_size
        ws_bytes = int(lib.mq_gather_qmm_workspace_size(rows, experts))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
        _lib.check(lib.mq_gather_qmm(ctypes.byref(a), stream_handle()), lib)
        return out
    # GEMV per row: x is read as [tokens, in] with `slots` rows per token
    # when the rows of one x row are consecutive (the decode shape x
    # [T, 1, 1, H] against indices [T, k]); otherwise the rows are gathered.
    tokens, slots, xs = rows, 1, x2
    bxp = (1,) * (len(batch) - len(bx)) + bx
    if not identity:
        if m == 1 and lhs_indices is None and len(batch) and bxp[-1] == 1 and bxp[:-1] == tuple(batch[:-1]):
            tokens, slots = x_batches, batch[-1]
        else:
            xs = x2.index_select(0, x_rows.to(torch.int64))
    _lib.check(lib.mq_gather_qmv(ptr(xs), dt, 0, ctypes.byref(proj), ptr(routes), ptr(out), tokens, slots, k, n,
                                 experts, group_size, stream_handle()), lib)
    return out
