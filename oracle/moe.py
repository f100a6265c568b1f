"""MoE expert compute: SwiGLU contract, fused combine, decode layer, prefill layer.

Restates (test infrastructure):

* SwiGLU epilogue of the fused Up kernel, the MLX bf16 sigmoid sequence
  ``m=|g|; e=exp(m); d=1+e; s=1/d; sig = g<0 ? s : 1-s; act = (g*sig)*u``
  with every step rounded to the activation type T
  (``models/flashnext/metal_runtime.py:267-285``), which the reference's
  contract harness proves equal to ``bf16(silu_bf16(g)*u)``
  (``models/flashnext/tests/bench/swiglu_contract.py:133-171, 210-219``).
  Each bf16 step is a float32 operation rounded to nearest-even, as bfloat
  arithmetic is; ``exp`` is the correctly rounded float32 exponential.
* ``weighted_combine`` (``metal_runtime.py:145-191``).
* fused down + score combine + shared epilogue: float32 ``acc += float(T(d)) *
  float(score)`` per slot with no contraction, then ``T(acc)`` and the shared
  add (``metal_runtime.py:291-336``).
* the generic combine used for more than eight tokens:
  ``(y * scores[..., None]).sum(-2) + shared_gate * shared`` in bf16
  (``models/flashnext/adaptive_topk.py:274-277``).
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16, f64_to_bf16
from .q4 import ExpertBank


# ---------------------------------------------------------------------------
# dtype plumbing: T is "bf16" (uint16 bits) or "f32" (float32 values)

def to_f32(values, dtype: str) -> np.ndarray:
    return bf16_to_f32(values) if dtype == "bf16" else np.asarray(values, dtype=np.float32)


def round_t(values_f32, dtype: str):
    """Round float32 values to T; returns T storage (bf16 bits or float32)."""
    v = np.asarray(values_f32, dtype=np.float32)
    return f32_to_bf16(v) if dtype == "bf16" else v


def round_t_f64(values_f64, dtype: str):
    v = np.asarray(values_f64, dtype=np.float64)
    return f64_to_bf16(v) if dtype == "bf16" else v.astype(np.float32)


def _t(values_f32, dtype: str) -> np.ndarray:
    """Round to T and widen back to float32 (one T-typed operation result)."""
    return to_f32(round_t(values_f32, dtype), dtype)


# ---------------------------------------------------------------------------
# SwiGLU / sigmoid

def exp_f32_correct(values_f32) -> np.ndarray:
    """float32 exponential, correctly rounded (via float64)."""
    with np.errstate(over="ignore"):
        return np.exp(np.asarray(values_f32, dtype=np.float64)).astype(np.float32)


def sigmoid_t(g_f32, dtype: str) -> np.ndarray:
    """MLX sigmoid sequence with every step rounded to T; returns float32 of T values."""
    g = np.asarray(g_f32, dtype=np.float32)
    m = np.abs(g)
    e = _t(exp_f32_correct(m), dtype)
    with np.errstate(over="ignore"):
        d = _t(np.float32(1.0) + e, dtype)
    with np.errstate(divide="ignore"):
        s = _t(np.float32(1.0) / d, dtype)
    one_minus = _t(np.float32(1.0) - s, dtype)
    return np.where(g < 0, s, one_minus).astype(np.float32)


def swiglu(gate, up, dtype: str = "bf16"):
    """``act = T(T(g * sigmoid_T(g)) * u)`` -> T storage."""
    g = to_f32(gate, dtype)
    u = to_f32(up, dtype)
    sig = sigmoid_t(g, dtype)
    silu = _t(g * sig, dtype)
    return round_t(silu * u, dtype)


def swiglu_fp32(gate_bits, up_bits):
    """The float32-epilogue candidate the reference rejects
    (``swiglu_contract.py:155-158``): ``bf16(u * (g / (1 + exp(-g))))``."""
    g = bf16_to_f32(gate_bits).astype(np.float64)
    u = bf16_to_f32(up_bits).astype(np.float64)
    g32 = g.astype(np.float32)
    with np.errstate(over="ignore"):
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g).astype(np.float32))).astype(np.float32)
    silu = (g32 * sig).astype(np.float32)
    return f32_to_bf16((silu * u.astype(np.float32)).astype(np.float32))


# ---------------------------------------------------------------------------
# combines

def weighted_combine(expert_outputs, routes, scores):
    """``(selected * scores[..., None]).sum(-2)`` with the reference's routing rule.

    Restates ``weighted_combine`` (``metal_runtime.py:145-191``) for numpy input.
    """
    out = np.asarray(expert_outputs)
    routes = np.asarray(routes)
    scores = np.asarray(scores)
    if out.ndim < 2 or routes.ndim == 0:
        raise ValueError("expert_outputs and routes need at least one dimension")
    if scores.shape != routes.shape:
        raise ValueError("routes and scores must have identical shapes")
    slots = routes.shape[-1]
    if out.shape[:-1] == routes.shape:
        selected = out
    elif out.ndim == routes.ndim + 1 and out.shape[-2] >= slots:
        if routes.size and (routes.min() < 0 or routes.max() >= out.shape[-2]):
            raise ValueError("routes contain an expert outside expert_outputs")
        selected = np.take_along_axis(out, np.expand_dims(routes, -1), axis=-2)
    else:
        raise ValueError(f"expert_outputs shape {out.shape} does not match routes {routes.shape}")
    return (selected * scores[..., None]).sum(axis=-2)


def down_combine(down_t, scores, dtype: str = "bf16", *, score_dtype: str = "f32",
                 shared_y=None, shared=None, shared_gate=None, keeps=None):
    """Fused down epilogue: per token ``acc += float(d_s) * float(score_s)``.

    ``down_t``: T storage ``[T, K, H]`` (already rounded per slot);
    ``scores``: ``[T, K]`` in ``score_dtype``.  ``keeps`` (optional) skips
    padded slots, whose score is zero.  Returns T storage ``[T, H]``.
    """
    d = to_f32(down_t, dtype)
    s = to_f32(scores, score_dtype)
    tokens, slots, hidden = d.shape
    acc = np.zeros((tokens, hidden), dtype=np.float32)
    for j in range(slots):
        active = np.ones(tokens, dtype=bool) if keeps is None else (np.asarray(keeps) > j)
        prod = (d[:, j, :] * s[:, j][:, None]).astype(np.float32)
        acc = np.where(active[:, None], (acc + prod).astype(np.float32), acc)
    routed = _t(acc, dtype)
    if shared_y is not None:
        return round_t(routed + to_f32(shared_y, dtype), dtype)
    if shared is not None:
        comp = _t(to_f32(shared, dtype) * to_f32(shared_gate, dtype).reshape(tokens, 1), dtype)
        return round_t(routed + comp, dtype)
    return round_t(routed, dtype)


def generic_decode_combine(down_bits, scores_bits, *, shared_y=None, keeps=None):
    """Group-64 decode combine: the reference keeps ``weighted_combine`` in the
    score dtype and adds ``shared_y`` afterwards (``metal_runtime.py:908-929``).
    With bf16 scores every product is rounded to bf16, the kept slots are summed
    in float32 in slot order and rounded once, then ``shared_y`` is added in
    bf16.  Padded slots (score 0) add nothing and are skipped.
    """
    d = bf16_to_f32(down_bits)
    s = bf16_to_f32(scores_bits)
    tokens, slots, _hidden = d.shape
    acc = np.zeros((tokens, d.shape[2]), dtype=np.float32)
    for j in range(slots):
        active = np.ones(tokens, dtype=bool) if keeps is None else (np.asarray(keeps) > j)
        prod = bf16_to_f32(f32_to_bf16((d[:, j, :] * s[:, j][:, None]).astype(np.float32)))
        acc = np.where(active[:, None], (acc + prod).astype(np.float32), acc)
    total = bf16_to_f32(f32_to_bf16(acc))
    if shared_y is None:
        return f32_to_bf16(total)
    return f32_to_bf16((total + bf16_to_f32(shared_y)).astype(np.float32))


def generic_combine(y_bits, scores_bits, shared_gate_bits=None, shared_bits=None):
    """bf16 ``(y * scores[..., None]).sum(-2) + shared_gate * shared``.

    Products are bf16-rounded, the slot sum accumulates in float32 in slot
    order and rounds once, the shared product and the final add are bf16.
    """
    y = bf16_to_f32(y_bits)
    s = bf16_to_f32(scores_bits)
    prod = bf16_to_f32(f32_to_bf16((y * s[..., None]).astype(np.float32)))
    acc = np.zeros(prod.shape[:-2] + prod.shape[-1:], dtype=np.float32)
    for j in range(prod.shape[-2]):
        acc = (acc + prod[..., j, :]).astype(np.float32)
    total = bf16_to_f32(f32_to_bf16(acc))
    if shared_bits is None:
        return f32_to_bf16(total)
    comp = bf16_to_f32(f32_to_bf16(
        (bf16_to_f32(shared_gate_bits).reshape(total.shape[:-1] + (1,)) * bf16_to_f32(shared_bits)).astype(np.float32)))
    return f32_to_bf16((total + comp).astype(np.float32))


# ---------------------------------------------------------------------------
# full layers

class ExpertRecordSet:
    """gate/up/down banks for the routed experts plus optional shared expert."""

    def __init__(self, gate: ExpertBank, up: ExpertBank, down: ExpertBank,
                 shared=None):
        self.gate, self.up, self.down = gate, up, down
        self.shared = shared  # (gate_bank, up_bank, down_bank) with one expert, or None


def expert_mlp(x_f32, banks, expert: int, dtype: str = "bf16", weights: str = "exact"):
    """One expert: T(gate), T(up), swiglu, T(down) for rows ``x_f32`` ``[n, H]``.

    ``weights``: "exact" dequantized weights, or "bf16" tiles (see
    ``ExpertBank.project``).  Returns (gate, up, act, down) in T storage.
    """
    gate_bank, up_bank, down_bank = banks
    g = round_t_f64(gate_bank.project(x_f32, expert, weights), dtype)
    u = round_t_f64(up_bank.project(x_f32, expert, weights), dtype)
    a = swiglu(g, u, dtype)
    d = round_t_f64(down_bank.project(to_f32(a, dtype), expert, weights), dtype)
    return g, u, a, d


def shared_gate_value(x_bits, w_sg_bits):
    """``sigmoid(x @ w_sg.T)`` in bf16 (``adaptive_topk.py:264``) -> bf16 [T]."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    w = bf16_to_f32(w_sg_bits).astype(np.float64).reshape(-1)
    logit = bf16_to_f32(f64_to_bf16(x @ w))
    return f32_to_bf16(sigmoid_t(logit, "bf16"))


def decode_layer(x, routes_experts, scores, records: ExpertRecordSet, *,
                 dtype: str = "bf16", score_dtype: str = "f32", keeps=None,
                 shared_y=None, shared=None, shared_gate=None,
                 shared_gate_weight=None, return_all: bool = False, combine: str = "fused"):
    """Fused-executor decode semantics (``MetalMoEExecutor.execute`` with scores).

    ``combine="generic"`` is the group-64 order (:func:`generic_decode_combine`,
    bf16 scores and activations only).

    ``routes_experts``: expert ids ``[T, K]`` (slot indirection already
    resolved).  When ``records.shared`` and ``shared_gate_weight`` are given the
    shared expert is computed here and combined as
    ``shared_y = bf16(sigmoid(x w_sg) * shared)``.
    """
    xf = to_f32(x, dtype)
    tokens, _hidden = xf.shape
    routes_experts = np.asarray(routes_experts)
    slots = routes_experts.shape[1]
    gate_o, up_o, act_o, down_o = [], [], [], []
    for t in range(tokens):
        row = []
        for j in range(slots):
            g, u, a, d = expert_mlp(xf[t:t + 1], (records.gate, records.up, records.down),
                                    int(routes_experts[t, j]), dtype)
            gate_o.append(g[0]); up_o.append(u[0]); act_o.append(a[0]); row.append(d[0])
        down_o.append(np.stack(row))
    down_t = np.stack(down_o)
    shape3 = (tokens, slots, -1)
    if return_all:
        return (np.stack(gate_o).reshape(shape3), np.stack(up_o).reshape(shape3),
                np.stack(act_o).reshape(shape3), down_t)
    if records.shared is not None and shared_gate_weight is not None:
        _g, _u, _a, sd = expert_mlp(xf, records.shared, 0, dtype)
        sg = shared_gate_value(x if dtype == "bf16" else f32_to_bf16(xf), shared_gate_weight)
        shared_y = f32_to_bf16(bf16_to_f32(sg)[:, None] * to_f32(sd, dtype)) if dtype == "bf16" else \
            (bf16_to_f32(sg)[:, None] * to_f32(sd, dtype)).astype(np.float32)
    if combine == "generic":
        if dtype != "bf16" or score_dtype != "bf16":
            raise ValueError("the generic decode combine is defined here for bf16 activations and scores")
        if shared is not None:
            shared_y = f32_to_bf16(to_f32(shared, dtype) * to_f32(shared_gate, dtype).reshape(tokens, 1))
        return generic_decode_combine(down_t, scores, shared_y=shared_y, keeps=keeps)
    return down_combine(down_t, scores, dtype, score_dtype=score_dtype, shared_y=shared_y,
                        shared=shared, shared_gate=shared_gate, keeps=keeps)


def prefill_layer(x_bits, inds, scores_bits, records: ExpertRecordSet, *,
                  shared_gate_weight=None, weights: str = "exact"):
    """Grouped (gather_qmm) path: per (token, slot) row the expert MLP in bf16,
    then the generic bf16 combine (``expert_cache.py:1790-1810``,
    ``adaptive_topk.py:274-277``).  Returns bf16 ``[T, H]`` and the per-slot
    outputs ``[T, K, H]``.
    """
    xf = bf16_to_f32(x_bits)
    tokens = xf.shape[0]
    inds = np.asarray(inds)
    slots = inds.shape[1]
    hidden = records.down.out_width
    y = np.zeros((tokens, slots, hidden), dtype=np.uint16)
    flat = inds.reshape(-1)
    for e in np.unique(flat):
        rows = np.nonzero(flat == e)[0]
        t_idx, s_idx = rows // slots, rows % slots
        _g, _u, _a, d = expert_mlp(xf[t_idx], (records.gate, records.up, records.down), int(e), "bf16", weights)
        y[t_idx, s_idx] = d
    if records.shared is not None and shared_gate_weight is not None:
        _g, _u, _a, sd = expert_mlp(xf, records.shared, 0, "bf16", weights)
        sg = shared_gate_value(x_bits, shared_gate_weight)
        return generic_combine(y, scores_bits, sg, sd), y
    return generic_combine(y, scores_bits), y
