"""The MoE block composition of ``_moe_call`` on gfx950.

``_moe_call`` (``models/flashnext/adaptive_topk.py:53-292``) runs the router,
renormalises, computes the shared expert and its sigmoid gate, then hands the
routed experts, scores and ``shared_y`` to the switch block whose executor
fuses the combine.  :class:`DecodeLayer` does the same with two C-ABI calls
into device-resident buffers (router kernel pair, then the fused expert
kernels with the shared expert in-kernel), so one decode step needs no host
synchronisation and can be captured in a HIP graph.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._tensors import ptr
from .layout import HEADER_SIZE, SlabLayout
from .ops import dense_projection


def pool_projection(pool: torch.Tensor, layout: SlabLayout, name: str) -> _lib.MqProjection:
    p = _lib.MqProjection()
    p.pool = ptr(pool)
    p.pool_header = HEADER_SIZE
    p.pool_stride = layout.record_stride
    p.off_weight = layout.offset(name, "weight")
    p.off_scales = layout.offset(name, "scales")
    p.off_biases = layout.offset(name, "biases")
    p.pool_slots = (pool.numel() * pool.element_size() - HEADER_SIZE) // layout.record_stride
    return p


@dataclass
class LayerWeights:
    """Device-resident weights of one MoE layer addressed through a slot pool."""

    layout: SlabLayout
    pool: torch.Tensor
    slot_table: torch.Tensor
    router_w: torch.Tensor
    shared_gate_w: torch.Tensor | None
    shared: tuple | None  # three (weight, scales, biases) dense single-expert banks


class DecodeLayer:
    """One MoE decode layer for a fixed token count, with preallocated buffers."""

    def __init__(self, weights: LayerWeights, tokens: int, top_k: int, *, threshold: float = 1.0,
                 min_keep: int = 1, blend: float = 1.0, device="cuda", x: torch.Tensor | None = None,
                 generic_combine: bool = False):
        """``x``: optional caller-owned bf16 ``[tokens, hidden]`` input buffer
        (e.g. a row of a larger staging tensor); allocated here when omitted.
        ``generic_combine``: combine the slots in the reference's generic bf16
        order (every score product rounded to bf16, ``MQ_DECODE_GENERIC_COMBINE``)
        instead of the fused executor's float32 order."""
        lay = weights.layout
        self.w = weights
        self.tokens, self.top_k = tokens, top_k
        self.hidden, self.inter = lay.hidden, lay.inter
        self.experts = weights.router_w.shape[0]
        dev = torch.device(device)
        bf = torch.bfloat16
        if x is None:
            x = torch.zeros((tokens, self.hidden), dtype=bf, device=dev)
        elif x.dtype != bf or tuple(x.shape) != (tokens, self.hidden) or not x.is_contiguous() or x.device != dev:
            raise ValueError(f"x must be a contiguous bf16 [{tokens}, {self.hidden}] tensor on {dev}")
        self.x = x
        self.logits = torch.empty((tokens, self.experts), dtype=bf, device=dev)
        self.inds = torch.empty((tokens, top_k), dtype=torch.int32, device=dev)
        self.scores = torch.empty((tokens, top_k), dtype=bf, device=dev)
        self.scores_raw = torch.empty((tokens, top_k), dtype=bf, device=dev)
        self.routes = torch.empty((tokens, top_k), dtype=torch.int32, device=dev)
        self.keeps = torch.empty((tokens,), dtype=torch.int32, device=dev)
        self.shared_gate = torch.empty((tokens,), dtype=bf, device=dev)
        has_shared = weights.shared is not None
        self.act = torch.empty((tokens * top_k + (tokens if has_shared else 0), self.inter), dtype=bf, device=dev)
        self.out = torch.empty((tokens, self.hidden), dtype=bf, device=dev)

        r = _lib.MqRouteArgs()
        r.x, r.gate_w, r.logits_in = ptr(self.x), ptr(weights.router_w), None
        r.shared_gate_w = ptr(weights.shared_gate_w) if has_shared else None
        r.slot_table = ptr(weights.slot_table)
        r.logits_out = ptr(self.logits)
        r.inds, r.scores, r.score_dtype = ptr(self.inds), ptr(self.scores), _lib.MQ_BF16
        r.scores_raw, r.routes, r.keeps = ptr(self.scores_raw), ptr(self.routes), ptr(self.keeps)
        r.shared_gate = ptr(self.shared_gate) if has_shared else None
        r.tokens, r.hidden, r.experts, r.top_k = tokens, self.hidden, self.experts, top_k
        r.threshold, r.min_keep, r.blend = float(threshold), int(min_keep), float(blend)
        self.route_args = r

        a = _lib.MqMoeArgs()
        a.x, a.x_dtype = ptr(self.x), _lib.MQ_BF16
        a.gate = pool_projection(weights.pool, lay, "gate_proj")
        a.up = pool_projection(weights.pool, lay, "up_proj")
        a.down = pool_projection(weights.pool, lay, "down_proj")
        a.routes, a.scores, a.score_dtype = ptr(self.routes), ptr(self.scores), _lib.MQ_BF16
        a.keeps = ptr(self.keeps) if threshold < 1.0 else None
        if has_shared:
            self._shared_projs = (_lib.MqProjection * 3)(*[dense_projection(*bank) for bank in weights.shared])
            import ctypes

            a.shared_expert = ctypes.addressof(self._shared_projs)
            a.shared_gate = ptr(self.shared_gate)
        a.out, a.act_out = ptr(self.out), ptr(self.act)
        a.tokens, a.slots, a.hidden, a.inter = tokens, top_k, self.hidden, self.inter
        a.expert_count, a.group_size = self.experts, lay.group_size
        a.flags = _lib.MQ_DECODE_GENERIC_COMBINE if generic_combine else 0
        self.moe_args = a
        self._lib = _lib.load()

    def launch(self, stream: int | None) -> None:
        """The whole layer on ``stream`` (a raw hipStream_t handle): router
        logits, gate/up with the top-k selection folded in, down + combine."""
        rc = self._lib.mq_moe_layer(self.route_args, self.moe_args, stream)
        if rc:
            _lib.check(rc, self._lib)

    def launch_unfused(self, stream) -> None:
        """Same layer as separate router (logits + select) and expert calls."""
        self.launch_router(stream)
        self.launch_experts(stream)

    def launch_router(self, stream):
        _lib.check(self._lib.mq_route_topk(self.route_args, stream), self._lib)

    def launch_experts(self, stream):
        _lib.check(self._lib.mq_moe_decode(self.moe_args, stream), self._lib)


class MoEBlock:
    """``_moe_call`` for any token count (``adaptive_topk.py:53-292``).

    Up to ``fused_max_tokens`` tokens (8, the bound under which the reference
    hands the scores to the fused executor, ``adaptive_topk.py:266-269``) the
    block runs a :class:`DecodeLayer` per token count: router, experts and the
    ordered float32 combine with ``shared_y`` in the down kernel.  Beyond it
    the reference sends the (token, slot) rows through ``switch_mlp(x, inds)``
    and combines them in bf16 as ``(y * scores).sum(-2) + shared_gate * shared``
    (``adaptive_topk.py:274-277``).  Here that is the routed decode layer
    again, with the generic bf16 combine (``MQ_DECODE_GENERIC_COMBINE``), up
    to ``routed_max_tokens`` tokens (64; at verify sizes it is 1.1-1.8x
    faster than the grouped GEMMs, whose tiles hold one or two rows per expert
    there), and the grouped path (sort + MFMA GEMMs + bf16 combine) beyond.
    At a keep threshold below 1 the dropped slots carry the row's first expert
    and score 0 on every path (``adaptive_topk.py:213-227``).

    ``last_path`` is ``"fused"``, ``"routed"`` or ``"grouped"`` after each call.
    """

    def __init__(self, weights: LayerWeights, top_k: int, *, threshold: float = 1.0, min_keep: int = 1,
                 blend: float = 1.0, fused_max_tokens: int = 8, routed_max_tokens: int = 64):
        from .grouped import GroupedMoE

        if not 0 <= fused_max_tokens <= 8:
            raise ValueError("fused_max_tokens must be in 0..8")
        if not (routed_max_tokens == 0 or fused_max_tokens <= routed_max_tokens <= 64):
            raise ValueError("routed_max_tokens must be 0 or in fused_max_tokens..64")
        self.w = weights
        self.top_k, self.threshold, self.min_keep, self.blend = int(top_k), float(threshold), int(min_keep), float(blend)
        self.fused_max_tokens = int(fused_max_tokens)
        self.routed_max_tokens = int(routed_max_tokens)
        self.device = weights.pool.device
        self.hidden, self.inter = weights.layout.hidden, weights.layout.inter
        self._layers: dict[int, DecodeLayer] = {}
        lay = weights.layout
        self._grouped = GroupedMoE(pool_projection(weights.pool, lay, "gate_proj"),
                                   pool_projection(weights.pool, lay, "up_proj"),
                                   pool_projection(weights.pool, lay, "down_proj"),
                                   hidden=lay.hidden, inter=lay.inter, group_size=lay.group_size,
                                   shared_expert=weights.shared)
        self._pool = weights.pool  # the projection structs hold its address
        self.last_path = None
        self.last_route = None

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """``x``: bf16 ``[T, hidden]`` on the block's device -> bf16 ``[T, hidden]``."""
        from .router import route

        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != self.hidden:
            raise ValueError(f"x must be bf16 [tokens, {self.hidden}]")
        if x.device != self.device:
            raise ValueError(f"x is on {x.device}, the block on {self.device}")
        tokens = int(x.shape[0])
        if tokens == 0:
            raise ValueError("x has no tokens")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        fused = tokens <= self.fused_max_tokens
        if fused or tokens <= self.routed_max_tokens:
            layer = self._layers.get(tokens)
            if layer is None:
                layer = DecodeLayer(self.w, tokens, self.top_k, threshold=self.threshold, min_keep=self.min_keep,
                                    blend=self.blend, device=self.device, generic_combine=not fused)
                self._layers[tokens] = layer
            layer.x.copy_(x)
            layer.launch(stream)
            self.last_path = "fused" if fused else "routed"
            self.last_route = layer
            return layer.out.clone()
        r = route(x, self.w.router_w, self.top_k, threshold=self.threshold, min_keep=self.min_keep,
                  blend=self.blend, slot_table=self.w.slot_table, shared_gate_w=self.w.shared_gate_w,
                  keep_logits=False)
        out, _y = self._grouped(x, r.routes, r.scores, shared_gate=r.shared_gate)
        self.last_path = "grouped"
        self.last_route = r
        return out
