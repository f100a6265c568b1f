"""Router chain: gate GEMV, softmax(precise), top-k, renorm, adaptive keep, slot words.

Restates (test infrastructure):

* ``_router_plain`` -- ``softmax(logits, precise=True)``, ``argpartition``
  top-k, ``take_along_axis``, ``topk_mass = sum(scores)``
  (``models/flashnext/compiled.py:61-65``; same chain inline at
  ``models/flashnext/adaptive_topk.py:57-64``).
* ``_renorm_plain`` -- ``scores / (topk_mass + blend*(selected_mass - topk_mass))``
  (``compiled.py:68-71``; ``adaptive_topk.py:256-261``), evaluated in bf16
  arithmetic: every binary op is a float32 op rounded to bf16.
* ``_keep_for_mass`` and the keep/pad rule (``adaptive_topk.py:43-50,
  75-114, 205-227``).
* route words ``0x80000000 | slot`` (``models/flashnext/expert_cache.py:1723-1725``,
  ``models/flashnext/expert_pool.py:34``).

The top-k order the reference leaves to ``argpartition`` is fixed here as
"score descending, expert index ascending on ties"; parity compares index
sets and reports bf16 ties at the k-th place separately.
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16, f64_to_bf16

SLOT_BIT = 0x80000000


def router_logits(x_bits, wg_bits) -> np.ndarray:
    """bf16 ``x @ Wg.T`` (``nn.Linear`` without bias), float64 accumulation."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    w = bf16_to_f32(wg_bits).astype(np.float64)
    return f64_to_bf16(x @ w.T)


def softmax_precise(logits_bits) -> np.ndarray:
    """``mx.softmax(logits, axis=-1, precise=True)`` -> bf16 bits.

    Computed in float64 (max-subtracted exp, sum, divide), rounded once.
    """
    l = bf16_to_f32(logits_bits).astype(np.float64)
    m = l.max(axis=-1, keepdims=True)
    e = np.exp(l - m)
    return f64_to_bf16(e / e.sum(axis=-1, keepdims=True))


def topk(gates_bits, k: int):
    """Top-k of bf16 gates: (inds uint32 [T,k], scores bf16 [T,k]).

    Order: gate value descending, expert index ascending on equal values.
    """
    g = np.asarray(gates_bits, dtype=np.uint16)
    t, e = g.shape
    # bf16 softmax outputs are non-negative, so their bit patterns order like
    # their values.  Sort by (-bits, index).
    order = np.lexsort((np.broadcast_to(np.arange(e), g.shape), -g.astype(np.int64)), axis=-1)
    inds = order[:, :k].astype(np.uint32)
    scores = np.take_along_axis(g, inds.astype(np.int64), axis=-1)
    return inds, scores


def kth_tie(gates_bits, k: int) -> np.ndarray:
    """Per row: True when the k-th and (k+1)-th largest gates are equal in bf16."""
    g = np.sort(np.asarray(gates_bits, dtype=np.uint16), axis=-1)[:, ::-1]
    if g.shape[1] <= k:
        return np.zeros(g.shape[0], dtype=bool)
    return g[:, k - 1] == g[:, k]


def bf16_sum(bits, axis=-1) -> np.ndarray:
    """bf16 reduction: float32 accumulation in index order, one final rounding."""
    v = bf16_to_f32(bits)
    acc = np.zeros(np.delete(v.shape, axis if axis >= 0 else v.ndim + axis), dtype=np.float32)
    for j in range(v.shape[axis]):
        acc = (acc + np.take(v, j, axis=axis)).astype(np.float32)
    return f32_to_bf16(acc)


def _bop(a_bits, b_bits, op) -> np.ndarray:
    a = bf16_to_f32(a_bits)
    b = bf16_to_f32(b_bits)
    with np.errstate(divide="ignore", invalid="ignore"):
        return f32_to_bf16(op(a, b).astype(np.float32))


def renorm(scores_bits, topk_mass_bits, blend: float = 1.0):
    """``_renorm_plain`` in bf16 arithmetic -> (scores bf16, normalizer bf16)."""
    selected = bf16_sum(scores_bits)[..., None]
    mass = np.asarray(topk_mass_bits, dtype=np.uint16).reshape(selected.shape)
    blend_bits = np.full(selected.shape, f32_to_bf16(np.float32(blend)), dtype=np.uint16)
    diff = _bop(selected, mass, np.subtract)
    prod = _bop(blend_bits, diff, np.multiply)
    norm = _bop(mass, prod, np.add)
    return _bop(scores_bits, np.broadcast_to(norm, np.shape(scores_bits)), np.divide), norm


def keep_for_mass(weights, threshold: float) -> int:
    """Shortest prefix whose normalised mass reaches ``threshold``.

    Restates ``_keep_for_mass`` (``adaptive_topk.py:43-50``) with Python floats.
    """
    total = sum(weights)
    accumulated = 0.0
    for position, weight in enumerate(weights):
        accumulated += weight / total
        if accumulated >= threshold:
            return position + 1
    return len(weights)


def adaptive_keep(scores_bits, threshold: float, min_keep: int = 1):
    """Keeps per row for sorted-descending scores (``adaptive_topk.py:104-114``)."""
    s = np.asarray(scores_bits, dtype=np.uint16)
    k = s.shape[-1]
    minimum = max(1, min(k, int(min_keep)))
    rows = bf16_to_f32(s).astype(np.float64).reshape(-1, k).tolist()
    return np.array([max(minimum, keep_for_mass(r, threshold)) for r in rows], dtype=np.int32)


def pad_dropped(inds, scores_bits, keeps):
    """Dropped slots repeat the row's first expert with score 0 (``adaptive_topk.py:213-227``).

    Returns full-width arrays plus ``width = max(keeps)``.
    """
    inds = np.array(inds, copy=True)
    scores = np.array(scores_bits, dtype=np.uint16, copy=True)
    pos = np.arange(inds.shape[-1])[None, :]
    dropped = pos >= np.asarray(keeps)[:, None]
    inds = np.where(dropped, inds[:, :1], inds)
    scores = np.where(dropped, np.uint16(0), scores)
    return inds.astype(np.uint32), scores.astype(np.uint16), int(np.max(keeps))


def slot_words(inds, slot_table=None) -> np.ndarray:
    """Route words: ``0x80000000 | slot[e]`` with a slot table, else the expert id."""
    inds = np.asarray(inds, dtype=np.uint32)
    if slot_table is None:
        return inds.copy()
    table = np.asarray(slot_table, dtype=np.uint32)
    return (np.uint32(SLOT_BIT) | table[inds.astype(np.int64)]).astype(np.uint32)


def route(x_bits, wg_bits, k: int, *, threshold: float = 1.0, min_keep: int = 1,
          blend: float = 1.0, slot_table=None, logits_bits=None):
    """Full router for a batch of tokens; mirrors ``_moe_call`` up to the renorm.

    Returns a dict with ``logits, gates, inds, scores_raw, topk_mass, keeps,
    width, scores, routes`` (routes already slot-encoded when a table is given).
    """
    logits = router_logits(x_bits, wg_bits) if logits_bits is None else np.asarray(logits_bits, np.uint16)
    gates = softmax_precise(logits)
    inds, raw = topk(gates, k)
    mass = bf16_sum(raw)
    keeps = np.full(inds.shape[0], k, dtype=np.int32)
    width = k
    padded_inds, padded_scores = inds, raw
    if threshold < 1.0:
        keeps = adaptive_keep(raw, threshold, min_keep)
        padded_inds, padded_scores, width = pad_dropped(inds, raw, keeps)
    scores, _norm = renorm(padded_scores, mass, blend)
    return {
        "logits": logits, "gates": gates, "inds": padded_inds,
        "scores_raw": raw, "topk_mass": mass, "keeps": keeps, "width": width,
        "scores": scores, "routes": slot_words(padded_inds, slot_table),
    }
