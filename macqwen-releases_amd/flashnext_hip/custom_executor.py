"""Executor plug-in for the reference's layer benchmark seam.

``models/flashnext/tests/bench/bench_runtime_layer.py --custom-executor
module:attr`` loads a module and looks for ``build_executor`` (then
``create_executor``, an executor class, ``execute``, ``run``; ``:85-101``),
calls the builder with the arguments its signature names out of the
benchmark's context (here ``packs``, ``group_size``, ``bits``, ``mode`` and
``activation``; ``:118-145, 383-408``), then calls the runner's ``execute``
the same way with ``x``, ``indices`` and ``scores`` (``:173-201``).  Its MLX arm is the
unsorted ``gather_qmm`` chain followed by the bf16 combine
``(y * scores[..., None]).sum(-2)`` (``:304-326``).

:func:`build_executor` returns a :class:`LayerRunner` with that contract on
gfx950: the packs go to HBM once, and every call runs the grouped path
(``mq_moe_grouped``: device sort, bf16 MFMA grouped GEMMs, SwiGLU, the bf16
generic combine), returning ``[..., hidden]`` with scores and
``[..., top_k, hidden]`` without.  The runner carries no ``last_path``: the
benchmark counts a runner without one as a native execution (``:205-211``).
"""
from __future__ import annotations

from typing import Any, Mapping

import numpy as np
import torch

from .grouped import GroupedMoE

PROJECTIONS = ("gate_proj", "up_proj", "down_proj")


def _device_tensor(value: Any, dtype: torch.dtype, name: str, device) -> torch.Tensor:
    """A contiguous device tensor with ``dtype`` storage from a torch tensor or
    a numpy array (bf16 given as uint16 bits or float32 values)."""
    if isinstance(value, torch.Tensor):
        t = value
    else:
        arr = np.asarray(value)
        if dtype == torch.bfloat16 and arr.dtype == np.uint16:
            t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16)
        elif dtype == torch.int32 and arr.dtype == np.uint32:
            t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int32))
        else:
            t = torch.from_numpy(np.ascontiguousarray(arr))
    if dtype == torch.int32 and t.dtype == getattr(torch, "uint32", None):
        t = t.view(torch.int32)
    if dtype == torch.bfloat16 and t.dtype in (torch.int16, getattr(torch, "uint16", None)):
        t = t.view(torch.bfloat16)
    if t.dtype != dtype:
        if dtype == torch.int32 or not t.is_floating_point():
            raise TypeError(f"{name} must hold {dtype} data (got {t.dtype})")
        t = t.to(dtype)
    return t.to(device).contiguous()


class LayerRunner:
    """One MoE layer's experts (all of ``packs``) behind ``execute(x, indices, scores)``."""

    def __init__(self, packs: Mapping[str, Any], group_size: int = 32, device="cuda"):
        self.device = torch.device(device)
        banks = []
        for proj in PROJECTIONS:
            if proj not in packs:
                raise ValueError(f"packs must hold {', '.join(PROJECTIONS)}")
            w, s, b = packs[proj]
            banks.append((_device_tensor(w, torch.int32, f"{proj}.weight", self.device),
                          _device_tensor(s, torch.bfloat16, f"{proj}.scales", self.device),
                          _device_tensor(b, torch.bfloat16, f"{proj}.biases", self.device)))
        gate, up, down = banks
        if gate[0].dim() != 3 or up[0].shape != gate[0].shape or down[0].dim() != 3:
            raise ValueError("packed weights must be [experts, out, in / 8] for gate, up and down")
        self.expert_count, self.inter = int(gate[0].shape[0]), int(gate[0].shape[1])
        self.hidden = int(down[0].shape[1])
        if gate[0].shape[2] * 8 != self.hidden or down[0].shape[2] * 8 != self.inter:
            raise ValueError("gate/up inputs must be the hidden width and down inputs the intermediate width")
        self.group_size = int(group_size)
        self._moe = GroupedMoE(gate, up, down, hidden=self.hidden, inter=self.inter,
                               expert_count=self.expert_count, group_size=self.group_size)

    def execute(self, x, indices, scores=None):
        """``x [..., hidden]``, ``indices [..., top_k]`` expert ids (same
        leading shape), optional ``scores [..., top_k]`` -> bf16
        ``[..., hidden]`` (combined) or ``[..., top_k, hidden]``."""
        xt = _device_tensor(x, torch.bfloat16, "x", self.device)
        it = indices if isinstance(indices, torch.Tensor) else torch.from_numpy(np.asarray(indices))
        lead = tuple(it.shape[:-1])
        top_k = int(it.shape[-1])
        if xt.shape[-1] != self.hidden or tuple(xt.shape[:-1]) != lead:
            raise ValueError(f"x must be [..., {self.hidden}] with the leading shape of indices {lead}")
        routes = it.reshape(-1, top_k).to(self.device)
        if routes.dtype not in (torch.int32, torch.int64) and routes.dtype != getattr(torch, "uint32", None):
            raise TypeError(f"indices must be integer expert ids (got {routes.dtype})")
        if routes.numel() and (int(routes.min()) < 0 or int(routes.max()) >= self.expert_count):
            raise ValueError(f"indices must lie in 0..{self.expert_count - 1}")
        x2 = xt.reshape(-1, self.hidden)
        if scores is None:
            _out, y = self._moe(x2, routes, combine=False)
            return y.reshape(*lead, top_k, self.hidden)
        sc = _device_tensor(scores, torch.bfloat16, "scores", self.device).reshape(-1, top_k)
        if sc.shape[0] != routes.shape[0]:
            raise ValueError("scores must have the shape of indices")
        out, _y = self._moe(x2, routes, sc)
        return out.reshape(*lead, self.hidden)

    run = execute
    __call__ = execute


def build_executor(packs: Mapping[str, Any], group_size: int = 32, bits: int = 4, mode: str = "affine",
                   activation: Any = None) -> LayerRunner:
    """The benchmark's builder: 4-bit affine packs at group 32 or 64 with the
    SwiGLU activation; raises ``ValueError`` for anything else."""
    if bits != 4 or mode != "affine":
        raise ValueError(f"only 4-bit affine packs are supported (got bits={bits}, mode={mode!r})")
    if group_size not in (32, 64):
        raise ValueError(f"group_size must be 32 or 64 (got {group_size})")
    name = activation if activation is None or isinstance(activation, str) else type(activation).__name__
    if name not in (None, "swiglu", "SwiGLU"):  # the benchmark passes an nn.SwiGLU instance
        raise ValueError(f"only the SwiGLU activation is supported (got {activation!r})")
    return LayerRunner(packs, group_size)
