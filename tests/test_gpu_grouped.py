"""GPU parity of the prefill / verify grouped path against the CPU oracle.

The grouped GEMMs run on bf16 MFMA tiles, so the weights enter as
bf16(fma(q, s, b)).  Per-slot outputs y and the combined output are compared
with ``oracle.moe.prefill_layer(weights="bf16")`` (the same tiles, float64
accumulation, bf16 rounding of every projection, bf16 SwiGLU and combine)
elementwise within rtol 1e-2 / atol 3e-3, and with the exact-weight oracle
within the layer tolerance (max rel 1e-2 of the largest magnitude, cosine
>= 0.9999).  Execution variants (dense ids vs pool slot words, repeated
calls) must be bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, moe

from ._helpers import (MAX_REL, MIN_COSINE, assert_close, bf16_normal, from_dev_bf16, make_records,
                       pool_from_banks, say, to_dev_bank, to_dev_bf16, value_report)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


def _zipf_routes(tokens, slots, experts, seed, skew=1.1):
    """Distinct experts per token drawn with Zipf weights (heavy head, empty tail)."""
    rng = np.random.default_rng(seed)
    p = np.arange(1, experts + 1, dtype=np.float64) ** -skew
    p /= p.sum()
    inds = np.stack([rng.choice(experts, size=slots, replace=False, p=p) for _ in range(tokens)]).astype(np.int64)
    raw = rng.random((tokens, slots)).astype(np.float32) + 0.05
    scores = bf16.f32_to_bf16((raw / raw.sum(axis=1, keepdims=True)).astype(np.float32))
    return inds, scores


def _banks(records, torch):
    return tuple(to_dev_bank(b) for b in (records.gate, records.up, records.down))


def _check(got_bits, want_tiles_bits, want_exact_bits, msg):
    got = bf16.bf16_to_f32(got_bits)
    assert_close(got, bf16.bf16_to_f32(want_tiles_bits), msg + " (bf16 tiles)")
    rep = value_report(got, bf16.bf16_to_f32(want_exact_bits))
    assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, (msg + " (exact weights)", rep)


@pytest.mark.parametrize("tokens,experts,hidden,inter,group", [(256, 24, 2048, 512, 32), (96, 16, 2560, 640, 32),
                                                               (64, 8, 1024, 256, 64)])
def test_grouped_matches_oracle(torch_mod, tokens, experts, hidden, inter, group):
    torch = torch_mod
    say(f"case: grouped tokens={tokens} E={experts} H={hidden} I={inter} g={group}")
    from flashnext_hip.grouped import GroupedMoE

    slots = 8
    records = make_records(experts, hidden, inter, seed=300 + hidden, group=group)
    shared = make_records(1, hidden, inter, seed=301 + hidden, group=group)
    x = bf16_normal((tokens, hidden), seed=302)
    wsg = bf16_normal((1, hidden), seed=303, std=0.02)
    inds, scores = _zipf_routes(tokens, slots, experts, seed=304)
    records.shared = (shared.gate, shared.up, shared.down)
    want_out, want_y = moe.prefill_layer(x, inds, scores, records, shared_gate_weight=wsg, weights="bf16")
    exact_out, exact_y = moe.prefill_layer(x, inds, scores, records, shared_gate_weight=wsg)
    sg = moe.shared_gate_value(x, wsg)

    sh = tuple(tuple(t[:1] for t in to_dev_bank(b)) for b in (shared.gate, shared.up, shared.down))
    g = GroupedMoE(*_banks(records, torch), hidden=hidden, inter=inter, group_size=group, shared_expert=sh)
    out, y = g(to_dev_bf16(x), torch.from_numpy(inds.astype(np.int32)).cuda(), to_dev_bf16(scores),
               shared_gate=to_dev_bf16(sg))
    torch.cuda.synchronize()
    _check(from_dev_bf16(y), want_y, exact_y, "grouped per-slot y")
    _check(from_dev_bf16(out), want_out, exact_out, "grouped combined out")
    # a second call reuses the workspace and must reproduce the same bits
    out2, y2 = g(to_dev_bf16(x), torch.from_numpy(inds.astype(np.int32)).cuda(), to_dev_bf16(scores),
                 shared_gate=to_dev_bf16(sg))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


def test_grouped_heavy_expert_many_tiles_and_pool_words(torch_mod):
    """One expert gets > 3 tiles of rows; pool slot words give the same bits as dense ids."""
    torch = torch_mod
    say("case: grouped heavy expert + pool words")
    from flashnext_hip import _lib
    from flashnext_hip.grouped import GroupedMoE
    from flashnext_hip.layout import make_layout
    from flashnext_hip.moe_block import pool_projection

    tokens, slots, experts, hidden, inter = 600, 4, 12, 2048, 512
    records = make_records(experts, hidden, inter, seed=320)
    x = bf16_normal((tokens, hidden), seed=321)
    rng = np.random.default_rng(322)
    inds = np.stack([np.concatenate([[0], rng.choice(np.arange(1, experts), size=slots - 1, replace=False)])
                     for _ in range(tokens)]).astype(np.int64)  # expert 0 in every token: 600 rows
    scores = bf16.f32_to_bf16(np.full((tokens, slots), 0.25, np.float32))
    want_out, want_y = moe.prefill_layer(x, inds, scores, records, weights="bf16")
    exact_out, exact_y = moe.prefill_layer(x, inds, scores, records)
    dense = GroupedMoE(*_banks(records, torch), hidden=hidden, inter=inter)
    out_d, y_d = dense(to_dev_bf16(x), torch.from_numpy(inds.astype(np.int32)).cuda(), to_dev_bf16(scores))
    torch.cuda.synchronize()
    _check(from_dev_bf16(y_d), want_y, exact_y, "heavy y")
    _check(from_dev_bf16(out_d), want_out, exact_out, "heavy out")

    pool_slots = 20
    perm = rng.permutation(pool_slots)[:experts]
    img, _ = pool_from_banks(records, perm, pool_slots, hidden, inter)
    pool_t = torch.from_numpy(img).cuda()
    lay = make_layout(hidden, inter)
    projs = [pool_projection(pool_t, lay, n) for n in ("gate_proj", "up_proj", "down_proj")]
    pooled = GroupedMoE(*projs, hidden=hidden, inter=inter)
    words = (np.uint64(_lib.MQ_SLOT_BIT) | perm[inds].astype(np.uint64)).astype(np.uint32).view(np.int32)
    out_p, y_p = pooled(to_dev_bf16(x), torch.from_numpy(words).cuda(), to_dev_bf16(scores))
    torch.cuda.synchronize()
    assert torch.equal(y_d.view(torch.int16), y_p.view(torch.int16))
    assert torch.equal(out_d.view(torch.int16), out_p.view(torch.int16))


@pytest.mark.parametrize("pool_slots", [13000, 16400])
def test_grouped_large_pool_key_space_matches_dense(torch_mod, pool_slots):
    """Pools past the single-block sort's 12,288 keys: 13,000 slots sort with
    multi-block LDS histograms, 16,400 (past 16,384 keys) with wave-aggregated
    global atomics.  The bits must equal the dense call, which sorts in one
    block."""
    torch = torch_mod
    say(f"case: grouped large pool key space ({pool_slots} slots)")
    from flashnext_hip import _lib
    from flashnext_hip.grouped import GroupedMoE
    from flashnext_hip.layout import make_layout
    from flashnext_hip.moe_block import pool_projection

    tokens, slots, experts, hidden, inter = 300, 6, 10, 128, 128
    records = make_records(experts, hidden, inter, seed=340)
    x = bf16_normal((tokens, hidden), seed=341)
    inds, scores = _zipf_routes(tokens, slots, experts, seed=342)
    dense = GroupedMoE(*_banks(records, torch), hidden=hidden, inter=inter)
    out_d, y_d = dense(to_dev_bf16(x), torch.from_numpy(inds.astype(np.int32)).cuda(), to_dev_bf16(scores))
    torch.cuda.synchronize()
    want_out, want_y = moe.prefill_layer(x, inds, scores, records, weights="bf16")
    exact_out, exact_y = moe.prefill_layer(x, inds, scores, records)
    _check(from_dev_bf16(y_d), want_y, exact_y, "small-shape y")
    _check(from_dev_bf16(out_d), want_out, exact_out, "small-shape out")

    rng = np.random.default_rng(343)
    perm = np.concatenate([[pool_slots - 1, 12300], rng.choice(np.arange(12290), size=experts - 2, replace=False)])
    img, _ = pool_from_banks(records, perm, pool_slots, hidden, inter)
    pool_t = torch.from_numpy(img).cuda()
    del img
    lay = make_layout(hidden, inter)
    projs = [pool_projection(pool_t, lay, n) for n in ("gate_proj", "up_proj", "down_proj")]
    pooled = GroupedMoE(*projs, hidden=hidden, inter=inter)
    words = (np.uint64(_lib.MQ_SLOT_BIT) | perm[inds].astype(np.uint64)).astype(np.uint32).view(np.int32)
    out_p, y_p = pooled(to_dev_bf16(x), torch.from_numpy(words).cuda(), to_dev_bf16(scores))
    torch.cuda.synchronize()
    assert torch.equal(y_d.view(torch.int16), y_p.view(torch.int16))
    assert torch.equal(out_d.view(torch.int16), out_p.view(torch.int16))


def test_grouped_many_rows_multi_block_sort(torch_mod):
    """42,000 (token, slot) rows: past the single-block sort's 16,384, so the
    rows are counted and scattered by multi-block LDS histograms."""
    torch = torch_mod
    say("case: grouped 4200 tokens x 10 slots (multi-block sort)")
    from flashnext_hip.grouped import GroupedMoE

    tokens, slots, experts, hidden, inter = 4200, 10, 24, 128, 128
    records = make_records(experts, hidden, inter, seed=350)
    x = bf16_normal((tokens, hidden), seed=351)
    inds, scores = _zipf_routes(tokens, slots, experts, seed=352)
    want_out, want_y = moe.prefill_layer(x, inds, scores, records, weights="bf16")
    exact_out, exact_y = moe.prefill_layer(x, inds, scores, records)
    g = GroupedMoE(*_banks(records, torch), hidden=hidden, inter=inter)
    out, y = g(to_dev_bf16(x), torch.from_numpy(inds.astype(np.int32)).cuda(), to_dev_bf16(scores))
    torch.cuda.synchronize()
    _check(from_dev_bf16(y), want_y, exact_y, "many-row y")
    _check(from_dev_bf16(out), want_out, exact_out, "many-row out")


def test_grouped_invalid_route_word_flags_and_zeroes(torch_mod):
    torch = torch_mod
    say("case: grouped invalid route word")
    from flashnext_hip import _lib
    from flashnext_hip.grouped import GroupedMoE

    tokens, slots, experts, hidden, inter = 32, 2, 4, 1024, 256
    records = make_records(experts, hidden, inter, seed=330)
    x = bf16_normal((tokens, hidden), seed=331)
    inds = np.tile(np.array([[1, 2]], np.int64), (tokens, 1))
    scores = bf16.f32_to_bf16(np.full((tokens, slots), 0.5, np.float32))
    routes = inds.astype(np.int32).copy()
    routes[5, 1] = experts + 7  # out of range
    g = GroupedMoE(*_banks(records, torch), hidden=hidden, inter=inter)
    try:
        _lib.check_device_errors(None)  # clear flags left by earlier cases
    except ValueError:
        pass
    out, y = g(to_dev_bf16(x), torch.from_numpy(routes).cuda(), to_dev_bf16(scores))
    with pytest.raises(ValueError):
        _lib.check_device_errors(None)
    assert not torch.any(y[5, 1].view(torch.int16) != 0)
    _want_out, want_y = moe.prefill_layer(x, inds, scores, records, weights="bf16")
    mask = np.ones((tokens, slots), bool)
    mask[5, 1] = False
    assert_close(bf16.bf16_to_f32(from_dev_bf16(y))[mask], bf16.bf16_to_f32(want_y)[mask], "valid rows")
