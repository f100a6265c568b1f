"""Bounded decode MoE executor on gfx950: the drop-in for ``MetalMoEExecutor``.

Keeps the reference executor's constructor, ``execute`` signature, return
shapes, bounds, error types and observable state
(``models/flashnext/metal_runtime.py:422-932``).  Differences by design:

* the three Metal kernels become two HIP kernels (fused gate+up+SwiGLU, and
  down + score combine + shared epilogue) from ``libmqmoe.so``;
* there is no CPU/"reference" compute fallback: when the HIP library or a
  gfx950 device is unavailable, ``execute`` raises ``RuntimeError`` after
  argument validation (the reference silently ran numpy);
* the resident record pack works at any (hidden, intermediate, group) shape
  (the reference hard-codes 2560/640, ``metal_runtime.py:854-859``).
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any, Mapping, Sequence

import numpy as np
import torch

from . import _lib
from ._tensors import act_dtype, half16, ptr, require_cuda, stream_handle, words32
from .layout import HEADER_SIZE, make_layout
from .profiler import BoundaryProfiler

MAX_TOKENS = 8
MAX_EXPERTS = 512
MAX_TOP_K = 10
MAX_WIDTH = 16_384
GROUP_SIZE = 32
SUPPORTED_GROUP_SIZES = (32, 64)
BITS = 4


@dataclass(frozen=True)
class Q4G32Projection:
    """One projection's expert bank: uint32 nibble words ``[E, out, in/8]`` and
    bf16 group scales and biases ``[E, out, in/group]``."""

    weight: Any
    scales: Any
    biases: Any


@dataclass(frozen=True)
class HipCapabilities:
    """What the probe found (library, device, injected backend); readable as
    attributes or by key, like the reference's capability mapping."""

    available: bool
    supports_custom_moe: bool
    backend: str
    reason: str

    @property
    def custom_hip(self) -> bool:
        return self.supports_custom_moe

    def __getitem__(self, key: str) -> Any:
        return getattr(self, key)


def probe_capabilities(backend: Any = None) -> HipCapabilities:
    """Capability flags without launching a kernel.

    ``backend`` may be ``None``/``"hip"`` (probe the library and device),
    ``"reference"`` (report unavailable), or an object exposing
    ``available``/``supports_custom_moe`` (the reference's injection seam,
    ``metal_runtime.py:65-96``).
    """
    if backend == "reference":
        return HipCapabilities(False, False, "reference", "reference backend requested")
    if backend is not None and hasattr(backend, "available"):
        available = bool(getattr(backend, "available"))
        supports = bool(getattr(backend, "supports_custom_moe", False))
        reason = "injected backend capability"
        if not available:
            reason = "injected backend is unavailable"
        elif not supports:
            reason = "backend does not provide custom MoE"
        return HipCapabilities(available and supports, supports, "injected", reason)
    if backend not in (None, "hip"):
        return HipCapabilities(False, False, str(backend), "unknown backend")
    try:
        lib = _lib.load()
    except _lib.NativeUnavailable as exc:
        return HipCapabilities(False, False, "hip", str(exc))
    if not torch.cuda.is_available():
        return HipCapabilities(False, False, "hip", "no GPU visible to torch")
    if not lib.mq_available():
        return HipCapabilities(False, False, "hip", _lib.last_error(lib))
    return HipCapabilities(True, True, "hip", "gfx950 device detected")


def _as_projection(value: Any) -> Q4G32Projection:
    if isinstance(value, Q4G32Projection):
        return value
    if isinstance(value, Mapping):
        return Q4G32Projection(value["weight"], value["scales"], value["biases"])
    if isinstance(value, Sequence) and len(value) == 3:
        return Q4G32Projection(value[0], value[1], value[2])
    raise TypeError("projection must be (weight, scales, biases)")


def _shape(value: Any) -> tuple[int, ...]:
    return tuple(int(item) for item in value.shape)


def _validate_projection(projection: Q4G32Projection, expert_count, input_width: int,
                         output_width: int, group_size: int = GROUP_SIZE) -> None:
    """Shape and dtype checks of ``metal_runtime.py:115-142``."""
    weight_shape = _shape(projection.weight)
    scale_shape = _shape(projection.scales)
    bias_shape = _shape(projection.biases)
    count = weight_shape[0] if expert_count is None else expert_count
    expected_weight = (count, output_width, input_width // 8)
    expected_meta = (count, output_width, input_width // group_size)
    if weight_shape != expected_weight:
        raise ValueError(f"weight shape {weight_shape} != {expected_weight}")
    if scale_shape != expected_meta or bias_shape != expected_meta:
        raise ValueError(f"Q4/G{group_size} scales and biases have an invalid shape")
    dtype = getattr(projection.weight, "dtype", None)
    ok = dtype in (torch.int32, getattr(torch, "uint32", None), np.uint32, np.int32) or \
        str(dtype) in ("uint32", "int32")
    if not ok:
        raise TypeError("Q4 weights must use uint32 packed values")


def weighted_combine(expert_outputs: Any, routes: Any, scores: Any) -> Any:
    """``(selected * scores[..., None]).sum(-2)``, with ``routes`` selecting from
    ``[..., experts, hidden]`` outputs when needed (``metal_runtime.py:145-191``).
    Works on torch tensors (on their device) and numpy arrays.
    """
    output_shape = _shape(expert_outputs)
    route_shape = _shape(routes)
    score_shape = _shape(scores)
    if len(output_shape) < 2 or len(route_shape) == 0:
        raise ValueError("expert_outputs and routes need at least one dimension")
    if score_shape != route_shape:
        raise ValueError("routes and scores must have identical shapes")
    slots = route_shape[-1]
    if output_shape[:-1] == route_shape:
        selected = expert_outputs
    elif len(output_shape) == len(route_shape) + 1 and output_shape[-2] >= slots:
        if isinstance(routes, torch.Tensor):
            if routes.numel() and (int(routes.min()) < 0 or int(routes.max()) >= output_shape[-2]):
                raise ValueError("routes contain an expert outside expert_outputs")
            selected = torch.take_along_dim(expert_outputs, routes.long().unsqueeze(-1), dim=-2)
        else:
            r = np.asarray(routes)
            if r.size and (r.min() < 0 or r.max() >= output_shape[-2]):
                raise ValueError("routes contain an expert outside expert_outputs")
            selected = np.take_along_axis(np.asarray(expert_outputs), np.expand_dims(r, -1), axis=-2)
    else:
        raise ValueError(f"expert_outputs shape {output_shape} does not match routes {route_shape}")
    if _shape(selected)[:-1] != route_shape:
        raise ValueError("selected expert outputs do not match route slots")
    if isinstance(selected, torch.Tensor):
        return (selected * scores[..., None]).sum(dim=-2)
    return (selected * np.asarray(scores)[..., None]).sum(axis=-2)


def _projection_struct(proj: Q4G32Projection | None, pool=None, stream_pack=None,
                       layout=None, name: str = "") -> _lib.MqProjection:
    p = _lib.MqProjection()
    if proj is not None:
        p.weight = ptr(words32(proj.weight, f"{name}.weight"))
        p.scales = ptr(half16(proj.scales, f"{name}.scales"))
        p.biases = ptr(half16(proj.biases, f"{name}.biases"))
    if pool is not None or stream_pack is not None:
        p.pool = ptr(pool) if pool is not None else None
        p.stream_pack = ptr(stream_pack) if stream_pack is not None else None
        p.pool_header = HEADER_SIZE
        p.pool_stride = layout.record_stride
        if pool is not None:
            p.pool_slots = max(0, (pool.numel() * pool.element_size() - HEADER_SIZE) // layout.record_stride)
        if stream_pack is not None:
            p.stream_records = (stream_pack.numel() * stream_pack.element_size()) // layout.record_stride
        p.off_weight = layout.offset(name, "weight")
        p.off_scales = layout.offset(name, "scales")
        p.off_biases = layout.offset(name, "biases")
    return p


class HipMoEExecutor:
    """Bounded three-projection executor on gfx950 (no host fallback)."""

    def __init__(self, expert_count: int, hidden_size: int, top_k: int, backend: Any = None, *,
                 max_tokens: int = MAX_TOKENS, max_width: int = MAX_WIDTH,
                 profile_boundaries: bool | None = None, profile_boundary: str | None = None,
                 fused_up_swiglu: bool | None = None, group_size: int = GROUP_SIZE,
                 header_size: int = HEADER_SIZE) -> None:
        if not 1 <= expert_count <= MAX_EXPERTS:
            raise ValueError(f"expert_count must be in 1..{MAX_EXPERTS}")
        if hidden_size <= 0:
            raise ValueError("hidden_size must be positive")
        if not 1 <= top_k <= MAX_TOP_K:
            raise ValueError(f"top_k must be in 1..{MAX_TOP_K}")
        if top_k > expert_count:
            raise ValueError("top_k cannot exceed expert_count")
        if not 1 <= max_tokens <= MAX_TOKENS:
            raise ValueError(f"max_tokens must be in 1..{MAX_TOKENS}")
        if not 1 <= max_width <= MAX_WIDTH:
            raise ValueError(f"max_width must be in 1..{MAX_WIDTH}")
        if group_size not in SUPPORTED_GROUP_SIZES:
            raise ValueError(f"group_size must be one of {SUPPORTED_GROUP_SIZES}")
        if header_size != HEADER_SIZE:
            raise ValueError(f"header_size must be {HEADER_SIZE}")
        self.expert_count = int(expert_count)
        self.hidden_size = int(hidden_size)
        self.top_k = int(top_k)
        self.max_tokens = int(max_tokens)
        self.max_width = int(max_width)
        self.group_size = int(group_size)
        self.header_size = int(header_size)
        self.backend = backend
        self.capabilities = probe_capabilities(backend)
        self.last_path = "unavailable" if not self.capabilities.available else "custom-hip"
        self.fallback_reason = self.capabilities["reason"]
        self._boundary_profiler = BoundaryProfiler(profile_boundaries, boundary=profile_boundary)
        if fused_up_swiglu is None:
            fused_up_swiglu = os.environ.get("FLASHNEXT_FUSED_UP_SWIGLU") == "1"
        self.fused_up_swiglu = bool(fused_up_swiglu)

    @property
    def available(self) -> bool:
        return bool(self.capabilities["available"])

    @property
    def boundary_profile(self) -> dict[str, Any]:
        return self._boundary_profiler.snapshot()

    def reset_boundary_profile(self) -> None:
        self._boundary_profiler.reset()

    def _require_custom(self) -> None:
        if not self.capabilities.supports_custom_moe or not self.available:
            raise RuntimeError(f"custom MoE is unavailable on this backend: {self.capabilities.reason}")

    def execute(self, x: Any, routes: Any, projections: Any = None, *, return_all: bool = False,
                scores: Any = None, slab_pack: Any = None, stream_pack: Any = None,
                shared_y: Any = None, shared: Any = None, shared_gate: Any = None,
                shared_expert: Any = None) -> Any:
        """Run gate, up, activation and down for bounded flattened inputs.

        ``x``: ``(tokens, hidden_size)``; ``routes``: ``(tokens, top_k)`` route
        words (bit 31 selects a ``slab_pack`` slot).  Returns ``T[tokens,
        hidden]`` when ``scores`` is given, ``T[tokens, top_k, hidden]``
        otherwise, or ``(gate, up, down)`` with ``return_all``.
        ``shared_expert`` (an extension) is a ``{gate_proj, up_proj, down_proj}``
        mapping of one expert combined with ``shared_gate`` in-kernel.
        """
        # Combine-only probes (metal_runtime.py:781-797).
        if projections is not None and not isinstance(projections, (Mapping, list, tuple)):
            if not self.capabilities.supports_custom_moe:
                raise RuntimeError("custom MoE is unavailable on this backend")
            self.last_path, self.fallback_reason = "custom-hip", None
            return weighted_combine(x, routes, projections)
        if projections is None and scores is not None:
            if not self.capabilities.supports_custom_moe:
                raise RuntimeError("custom MoE is unavailable on this backend")
            self.last_path, self.fallback_reason = "custom-hip", None
            return weighted_combine(x, routes, scores)
        if projections is None:
            raise TypeError("packed execution needs gate, up, and down projections")

        x_shape, route_shape = _shape(x), _shape(routes)
        if len(x_shape) != 2 or x_shape[1] != self.hidden_size:
            raise ValueError("x must have shape (tokens, hidden_size)")
        if len(route_shape) != 2 or route_shape[1] != self.top_k:
            raise ValueError("routes must have shape (tokens, top_k)")
        if scores is not None and _shape(scores) != route_shape:
            raise ValueError("scores must have the same shape as routes")
        if (shared is None) != (shared_gate is None) and shared_expert is None:
            raise ValueError("shared and shared_gate must be provided together")
        if shared_expert is not None and shared_gate is None:
            raise ValueError("shared_expert needs shared_gate")
        if sum(v is not None for v in (shared_y, shared, shared_expert)) > 1:
            raise ValueError("provide shared_y or shared parts, not both")
        if stream_pack is not None and slab_pack is None:
            raise ValueError("stream pack requires a resident slab pack")
        tokens = x_shape[0]
        if route_shape[0] != tokens:
            raise ValueError("x and routes must have the same token count")
        if not 1 <= tokens <= self.max_tokens:
            raise ValueError(f"tokens must be in 1..{self.max_tokens}")
        if isinstance(routes, np.ndarray) and np.any(routes < 0):
            raise ValueError("routes contain an expert outside the configured bank")
        if isinstance(projections, Mapping):
            gate = _as_projection(projections["gate_proj"])
            up = _as_projection(projections["up_proj"])
            down = _as_projection(projections["down_proj"])
        else:
            if len(projections) != 3:
                raise ValueError("projections must contain gate, up, and down")
            gate, up, down = (_as_projection(item) for item in projections)

        gate_width, inter_width = _shape(gate.weight)[1], _shape(up.weight)[1]
        if gate_width != inter_width or gate_width > self.max_width:
            raise ValueError("gate and up projection widths must match the bound")
        _validate_projection(gate, None, self.hidden_size, gate_width, self.group_size)
        _validate_projection(up, None, self.hidden_size, inter_width, self.group_size)
        if self.hidden_size % self.group_size or inter_width % self.group_size:
            raise ValueError(f"Q4/G{self.group_size} projection inputs must be group aligned")
        _validate_projection(down, None, inter_width, self.hidden_size, self.group_size)

        self._require_custom()
        return self._run(x, routes, gate, up, down, inter_width, return_all=return_all,
                         scores=scores, slab_pack=slab_pack, stream_pack=stream_pack,
                         shared_y=shared_y, shared=shared, shared_gate=shared_gate,
                         shared_expert=shared_expert)

    # ------------------------------------------------------------------ device path
    def _run(self, x, routes, gate, up, down, inter, *, return_all, scores, slab_pack, stream_pack,
             shared_y, shared, shared_gate, shared_expert):
        x = require_cuda(x, "x")
        dt = act_dtype(x)
        dev = x.device
        tokens, slots, hidden = x.shape[0], self.top_k, self.hidden_size
        route_words = words32(routes.to(dev) if isinstance(routes, torch.Tensor) else
                              torch.as_tensor(np.asarray(routes, dtype=np.int64), device=dev), "routes")
        layout = None
        if slab_pack is not None:
            layout = make_layout(hidden, inter, self.group_size)
            slab_pack = require_cuda(slab_pack, "slab_pack")
            stream_pack = require_cuda(stream_pack, "stream_pack") if stream_pack is not None else None
        args = _lib.MqMoeArgs()
        args.x, args.x_dtype = ptr(x), dt
        args.gate = _projection_struct(gate, slab_pack, stream_pack, layout, "gate_proj")
        args.up = _projection_struct(up, slab_pack, stream_pack, layout, "up_proj")
        args.down = _projection_struct(down, slab_pack, stream_pack, layout, "down_proj")
        args.routes = ptr(route_words)
        args.tokens, args.slots, args.hidden, args.inter = tokens, slots, hidden, inter
        # Dense route words are bounded by the bank the arrays actually hold.
        args.expert_count = min(int(_shape(w.weight)[0]) for w in (gate, up, down))
        args.group_size = self.group_size
        keep_alive = [route_words]

        # Group 64 with bf16 activations and float32 scores combines in float32
        # (the reference's weighted_combine promotes to the score dtype,
        # metal_runtime.py:908-929) and returns float32: per-slot outputs from
        # the kernels, the combine here.  Every other scored call combines in
        # the down kernel, which follows the group-64 order itself.
        g64_f32 = (scores is not None and not return_all and self.group_size == 64 and x.dtype == torch.bfloat16
                   and getattr(scores, "dtype", None) not in (torch.bfloat16,))
        if g64_f32 and shared_expert is not None:
            raise ValueError("shared_expert with group 64, bf16 x and float32 scores is not supported: "
                             "pass shared_y or shared and shared_gate")
        if return_all or scores is None or g64_f32:
            gate_out = torch.empty((tokens, slots, inter), dtype=x.dtype, device=dev)
            up_out = torch.empty_like(gate_out)
            act = torch.empty_like(gate_out)
            down_out = torch.empty((tokens, slots, hidden), dtype=x.dtype, device=dev)
            args.gate_out, args.up_out, args.act_out, args.down_out = (
                ptr(gate_out), ptr(up_out), ptr(act), ptr(down_out))
            args.flags = _lib.MQ_DECODE_RETURN_ALL
            self._launch(args, "down_qmv")
            self.last_path, self.fallback_reason = "custom-hip", None
            if return_all:
                return gate_out, up_out, down_out
            if scores is None:
                return down_out
            out = weighted_combine(down_out, route_words, scores.to(dev).float())
            if shared_y is not None:
                out = out + shared_y.to(dev).reshape(out.shape)
            elif shared is not None:
                out = out + shared_gate.to(dev).reshape(tokens, 1) * shared.to(dev).reshape(out.shape)
            return out

        scores = require_cuda(scores.to(dev), "scores")
        if scores.dtype not in (torch.float32, torch.bfloat16):
            scores = scores.float()
        args.scores = ptr(scores)
        args.score_dtype = _lib.MQ_BF16 if scores.dtype == torch.bfloat16 else _lib.MQ_F32
        keep_alive.append(scores)
        if shared_y is not None:
            sy = require_cuda(shared_y.to(dev).reshape(tokens, hidden).to(x.dtype), "shared_y")
            args.shared_y = ptr(sy)
            keep_alive.append(sy)
        elif shared is not None or shared_expert is not None:
            sg = require_cuda(shared_gate.to(dev).reshape(tokens).to(torch.bfloat16), "shared_gate")
            args.shared_gate = ptr(sg)
            keep_alive.append(sg)
            if shared is not None:
                sh = require_cuda(shared.to(dev).reshape(tokens, hidden).to(x.dtype), "shared")
                args.shared = ptr(sh)
                keep_alive.append(sh)
            else:
                projs = (_lib.MqProjection * 3)()
                for i, name in enumerate(("gate_proj", "up_proj", "down_proj")):
                    projs[i] = _projection_struct(_as_projection(shared_expert[name]), name=name)
                args.shared_expert = ctypes_addr(projs)
                keep_alive.append(projs)
        out = torch.empty((tokens, hidden), dtype=x.dtype, device=dev)
        args.out = ptr(out)
        if not self.fused_up_swiglu:
            # The unfused order (separate up QMV, then SwiGLU) is bit-identical.
            gate_tmp = torch.empty((tokens, slots, inter), dtype=x.dtype, device=dev)
            up_tmp = torch.empty_like(gate_tmp)
            args.gate_out, args.up_out = ptr(gate_tmp), ptr(up_tmp)
            args.flags = _lib.MQ_DECODE_UNFUSED_UP
            keep_alive += [gate_tmp, up_tmp]
        n_act = tokens * slots + (tokens if shared_expert is not None else 0)
        act = torch.empty((n_act, inter), dtype=x.dtype, device=dev)
        args.act_out = ptr(act)
        keep_alive.append(act)
        self._launch(args, "fused_down")
        self.last_path, self.fallback_reason = "custom-hip", None
        return out

    def _launch(self, args, label):
        lib = _lib.load()
        stream = stream_handle()
        profiler = self._boundary_profiler
        if profiler.enabled and profiler.selected_for(label):
            profiler.measure(label, lambda: _lib.check(lib.mq_moe_decode(args, stream), lib))
        else:
            _lib.check(lib.mq_moe_decode(args, stream), lib)


def ctypes_addr(obj) -> int:
    import ctypes

    return ctypes.addressof(obj)


# The reference's executor name, for callers that look it up by attribute.
MetalMoEExecutor = HipMoEExecutor

__all__ = [
    "BITS", "GROUP_SIZE", "MAX_EXPERTS", "MAX_TOKENS", "MAX_TOP_K", "MAX_WIDTH",
    "BoundaryProfiler", "HipCapabilities", "HipMoEExecutor", "MetalMoEExecutor",
    "Q4G32Projection", "SUPPORTED_GROUP_SIZES", "probe_capabilities", "weighted_combine",
]
