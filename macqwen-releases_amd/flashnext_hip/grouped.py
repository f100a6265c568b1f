"""Prefill / speculative-verify grouped path (token-sorted grouped GEMMs).

The reference runs more than 8 tokens through ``StreamingSwitchGLU._one_pass``
/ ``_issue`` (``models/flashnext/expert_cache.py:1743-1810``): the
(token, slot) rows are sorted by expert (``build_plan`` ``:750-760``,
mlx-vlm ``_gather_sort``), three ``mx.gather_qmm(transpose=True, group 32,
bits 4, sorted_indices=True)`` calls and the SwiGLU run over the sorted rows,
the rows are unsorted, and ``_moe_call`` combines the slots in bf16
(``adaptive_topk.py:274-277``) and adds the gated shared expert.

:func:`grouped_moe` does the same in one C-ABI call (``mq_moe_grouped``): a
counting sort on the device, bf16 MFMA grouped GEMMs with the weights
dequantized in registers, and the bf16 combine.  The shared expert may be given
precomputed (``shared``) or as a dense single-expert bank
(``shared_expert``), which then runs as one more group over all tokens.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._tensors import half16, ptr, require_cuda, stream_handle
from .ops import dense_projection


def _proj(p) -> _lib.MqProjection:
    if isinstance(p, _lib.MqProjection):
        return p
    w, s, b = p
    return dense_projection(w, s, b)


class GroupedMoE:
    """Grouped expert MLP over a fixed set of projections.

    ``gate``, ``up``, ``down``: ``(weight, scales, biases)`` dense banks
    (``[E, out, in/8]`` int32 / bf16) or :class:`_lib.MqProjection` structs
    (pool or stream-pack addressing).  ``expert_count`` bounds plain route
    ids (the dense bank size); pool slot words are bounded by the pool.
    """

    def __init__(self, gate, up, down, *, hidden: int, inter: int, expert_count: int = 0,
                 group_size: int = 32, shared_expert=None):
        # The structs hold raw device pointers: keep the tensors they point to alive.
        self._keep = (gate, up, down, shared_expert)
        self.gate, self.up, self.down = _proj(gate), _proj(up), _proj(down)
        self.hidden, self.inter, self.group_size = int(hidden), int(inter), int(group_size)
        if expert_count == 0 and isinstance(gate, tuple):
            expert_count = int(gate[0].shape[0])
        self.expert_count = int(expert_count)
        self._shared = None
        if shared_expert is not None:
            self._shared = (_lib.MqProjection * 3)(*[_proj(p) for p in shared_expert])
        self._workspace = None
        self._lib = _lib.load()

    @property
    def route_keys(self) -> int:
        g = self.gate
        slots = g.pool_slots if g.pool else 0
        ids = g.stream_records if g.stream_pack else (self.expert_count if g.weight else 0)
        return int(slots + ids)

    def workspace_bytes(self, tokens: int, slots: int) -> int:
        return int(self._lib.mq_grouped_workspace_size(tokens, slots, self.hidden, self.inter, self.route_keys,
                                                       1 if self._shared is not None else 0))

    def __call__(self, x: torch.Tensor, routes: torch.Tensor, scores: torch.Tensor | None = None, *,
                 shared: torch.Tensor | None = None, shared_gate: torch.Tensor | None = None,
                 stream=None, combine: bool = True):
        """Returns ``(out [T, H] or None, y [T, K, H])`` in bf16."""
        x = half16(require_cuda(x, "x"), "x")
        if x.dtype != torch.bfloat16:
            raise TypeError("the grouped path takes bf16 activations")
        tokens, hidden = x.shape
        if hidden != self.hidden:
            raise ValueError(f"x width {hidden} != hidden {self.hidden}")
        routes = require_cuda(routes, "routes").to(torch.int32).contiguous()
        if routes.dim() != 2 or routes.shape[0] != tokens:
            raise ValueError("routes must be [tokens, slots]")
        slots = routes.shape[1]
        dev = x.device
        need = self.workspace_bytes(tokens, slots)
        if self._workspace is None or self._workspace.numel() < need or self._workspace.device != dev:
            self._workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        y = torch.empty((tokens, slots, hidden), dtype=torch.bfloat16, device=dev)
        out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=dev) if combine else None
        a = _lib.MqGroupedArgs()
        a.x = ptr(x)
        a.gate, a.up, a.down = self.gate, self.up, self.down
        a.routes = ptr(routes)
        keep = [routes]
        if scores is not None:
            scores = half16(require_cuda(scores, "scores").to(torch.bfloat16), "scores")
            keep.append(scores)
            a.scores = ptr(scores)
        if shared is not None:
            shared = half16(require_cuda(shared, "shared").to(torch.bfloat16), "shared")
            keep.append(shared)
            a.shared = ptr(shared)
        if self._shared is not None:
            a.shared_expert = ctypes.addressof(self._shared)
        if shared_gate is not None:
            shared_gate = half16(require_cuda(shared_gate, "shared_gate").to(torch.bfloat16).reshape(-1),
                                 "shared_gate")
            keep.append(shared_gate)
            a.shared_gate = ptr(shared_gate)
        a.out = ptr(out) if out is not None else None
        a.y = ptr(y)
        a.workspace = ptr(self._workspace)
        a.workspace_bytes = self._workspace.numel()
        a.tokens, a.slots, a.hidden, a.inter = tokens, slots, hidden, self.inter
        a.expert_count, a.group_size = self.expert_count, self.group_size
        _lib.check(self._lib.mq_moe_grouped(ctypes.byref(a), stream_handle(stream)), self._lib)
        if stream is not None:
            # Temporaries may be freed when this returns: tie their reuse to `stream`.
            for t in keep + [x, y] + ([out] if out is not None else []):
                t.record_stream(stream)
        return out, y


def grouped_moe(x, routes, scores, gate, up, down, *, hidden: int | None = None, inter: int | None = None,
                group_size: int = 32, shared_expert=None, shared=None, shared_gate=None, stream=None):
    """One-shot :class:`GroupedMoE` call over dense banks."""
    hidden = hidden if hidden is not None else x.shape[-1]
    inter = inter if inter is not None else gate[0].shape[1]
    g = GroupedMoE(gate, up, down, hidden=hidden, inter=inter, group_size=group_size, shared_expert=shared_expert)
    return g(x, routes, scores, shared=shared, shared_gate=shared_gate, stream=stream)
