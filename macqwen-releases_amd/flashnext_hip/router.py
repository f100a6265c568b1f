"""Router chain on gfx950: gate GEMV, softmax, top-k, renorm, keep/pad, slot words.

One call of :func:`route` replaces the reference's MLX chain in ``_moe_call``
(``models/flashnext/adaptive_topk.py:53-64, 75-261``; ``compiled.py:61-71``)
and the host-side slot encoding of ``_pool_pass``
(``models/flashnext/expert_cache.py:1694-1725``).  Everything stays on the
device: route words are produced by the kernel from a device slot table, so a
fully resident pool needs no host synchronisation per layer.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._tensors import half16, ptr, require_cuda, stream_handle, words32


@dataclass
class RouteResult:
    inds: torch.Tensor            # [T, k] int32 expert ids, score-descending
    scores: torch.Tensor          # [T, k] renormalised scores (bf16 or f32)
    scores_raw: torch.Tensor      # [T, k] bf16 softmax gates
    routes: torch.Tensor          # [T, k] int32 route words
    keeps: torch.Tensor           # [T] int32 active prefix
    logits: torch.Tensor | None   # [T, E] bf16
    shared_gate: torch.Tensor | None  # [T] bf16

    def width(self) -> int:
        """``max(keeps)``: the reference's truncated route width (host sync)."""
        return int(self.keeps.max())


def route(x: torch.Tensor, gate_w: torch.Tensor | None, top_k: int, *, threshold: float = 1.0,
          min_keep: int = 1, blend: float = 1.0, slot_table: torch.Tensor | None = None,
          shared_gate_w: torch.Tensor | None = None, logits: torch.Tensor | None = None,
          score_dtype: torch.dtype = torch.bfloat16, keep_logits: bool = True) -> RouteResult:
    """Route ``x [T, H]`` (bf16) through ``gate_w [E, H]`` (bf16)."""
    if logits is None:
        x = half16(x, "x")
        tokens, hidden = x.shape
        gate_w = half16(gate_w, "gate_w")
        experts = gate_w.shape[0]
        if gate_w.shape[1] != hidden:
            raise ValueError("gate_w must be [experts, hidden]")
    else:
        logits = half16(logits, "logits")
        tokens, experts = logits.shape
        hidden = 0 if x is None else x.shape[-1]
        if x is not None:
            x = half16(x, "x")
    dev = (x if x is not None else logits).device
    if score_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("score_dtype must be bfloat16 or float32")
    inds = torch.empty((tokens, top_k), dtype=torch.int32, device=dev)
    scores = torch.empty((tokens, top_k), dtype=score_dtype, device=dev)
    raw = torch.empty((tokens, top_k), dtype=torch.bfloat16, device=dev)
    routes = torch.empty((tokens, top_k), dtype=torch.int32, device=dev)
    keeps = torch.empty((tokens,), dtype=torch.int32, device=dev)
    logits_out = None
    if logits is None:  # the library allocates nothing: the logits need a buffer either way
        logits_out = torch.empty((tokens, experts), dtype=torch.bfloat16, device=dev)
    shared_gate = None
    if shared_gate_w is not None:
        shared_gate_w = half16(shared_gate_w, "shared_gate_w").reshape(-1)
        shared_gate = torch.empty((tokens,), dtype=torch.bfloat16, device=dev)
    table = words32(slot_table, "slot_table") if slot_table is not None else None

    a = _lib.MqRouteArgs()
    a.x = ptr(x)
    a.gate_w = ptr(gate_w) if logits is None else None
    a.logits_in = ptr(logits)
    a.shared_gate_w = ptr(shared_gate_w)
    a.slot_table = ptr(table)
    a.logits_out = ptr(logits_out)
    a.inds, a.scores = ptr(inds), ptr(scores)
    a.score_dtype = _lib.MQ_BF16 if score_dtype == torch.bfloat16 else _lib.MQ_F32
    a.scores_raw, a.routes, a.keeps = ptr(raw), ptr(routes), ptr(keeps)
    a.shared_gate = ptr(shared_gate)
    a.tokens, a.hidden, a.experts, a.top_k = tokens, hidden, experts, top_k
    a.threshold, a.min_keep, a.blend = float(threshold), int(min_keep), float(blend)
    lib = _lib.load()
    _lib.check(lib.mq_route_topk(a, stream_handle()), lib)
    return RouteResult(inds, scores, raw, routes, keeps, logits_out if keep_logits else None, shared_gate)
