"""Small helpers that turn torch device tensors into C-ABI arguments."""
from __future__ import annotations

import torch

from . import _lib


def require_cuda(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor on the GPU")
    if not t.is_cuda:
        raise ValueError(f"{name} must live on the GPU (got {t.device})")
    return t.contiguous()


def act_dtype(t: torch.Tensor, name: str = "x") -> int:
    if t.dtype == torch.bfloat16:
        return _lib.MQ_BF16
    if t.dtype == torch.float32:
        return _lib.MQ_F32
    raise TypeError(f"{name} must be bfloat16 or float32 (got {t.dtype})")


def words32(t: torch.Tensor, name: str) -> torch.Tensor:
    """A 32-bit view (int32 storage) of uint32 / int32 / int64 word tensors."""
    t = require_cuda(t, name)
    if t.dtype in (torch.int32,):
        return t
    if t.dtype == getattr(torch, "uint32", None):
        return t.view(torch.int32)
    if t.dtype == torch.int64:
        if t.numel() and (int(t.min()) < -(2 ** 31) or int(t.max()) >= 2 ** 32):
            raise ValueError(f"{name} holds values outside 32 bits")
        return torch.where(t >= 2 ** 31, t - 2 ** 32, t).to(torch.int32).contiguous()
    raise TypeError(f"{name} must hold uint32 words (int32/uint32/int64 tensor), got {t.dtype}")


def half16(t: torch.Tensor, name: str) -> torch.Tensor:
    """bf16 metadata (scales/biases) as contiguous 16-bit storage."""
    t = require_cuda(t, name)
    if t.dtype == torch.bfloat16:
        return t
    if t.dtype in (torch.int16, getattr(torch, "uint16", None)):
        return t.view(torch.bfloat16)
    raise TypeError(f"{name} must be bfloat16 (got {t.dtype})")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(stream=None) -> int | None:
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream
