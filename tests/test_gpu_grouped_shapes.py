"""Grouped path across the shapes its launch variants and partial tiles cover.

The grouped GEMMs pick their pipeline by the stage count K / 128 (weight ring
and group-window depth: 1, 2, 3 or 4 stages per window), cut the output into
128-feature (gate/up) and 256-feature (down) blocks, and round rows to 32-row
slabs inside 128-row tiles.  These cases put every stage-count class on both
GEMMs, output widths that leave a partial feature block, one to ten slots,
token counts that leave partial slabs and tiles, group 32 and 64, and runs with
and without the shared expert; each is compared with
``oracle.moe.prefill_layer`` as in ``test_gpu_grouped.py``: elementwise
against the bf16-tile oracle (rtol 1e-2 / atol 3e-3) and by cosine / max rel
against the exact-weight oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, moe

from ._helpers import (MAX_REL, MIN_COSINE, assert_close, bf16_normal, from_dev_bf16, make_records, say,
                       to_dev_bank, to_dev_bf16, value_report)

pytestmark = pytest.mark.gpu

# (tokens, experts, slots, hidden, inter, group, shared)
CASES = [
    (1, 1, 1, 128, 128, 32, True),        # gate/up 1 stage, down 1 stage, one row
    (37, 5, 3, 256, 384, 64, False),      # 2 / 3 stages, 3 gate/up feature blocks, partial slab
    (160, 24, 10, 384, 640, 32, True),    # 3 / 5 stages, down N = 384 (partial 256-feature block)
    (90, 12, 4, 640, 256, 32, False),     # 5 / 2 stages, down N = 640 (partial block)
    (33, 9, 9, 1024, 896, 64, True),      # 8 / 7 stages, inter 896 (7 gate/up blocks)
    (129, 3, 2, 1152, 128, 32, True),     # 9 / 1 stages, a 129-row expert (two tiles, one row in the second)
    (64, 40, 8, 512, 512, 32, False),     # 4 / 4 stages, many one-slab tiles
    (200, 2, 2, 768, 384, 32, True),      # 6 / 3 stages, two heavy experts (two full tiles each)
]


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


def _routes(tokens, slots, experts, seed):
    rng = np.random.default_rng(seed)
    p = np.arange(1, experts + 1, dtype=np.float64) ** -1.1
    p /= p.sum()
    inds = np.stack([rng.choice(experts, size=slots, replace=False, p=p) for _ in range(tokens)]).astype(np.int64)
    raw = rng.random((tokens, slots)).astype(np.float32) + 0.05
    return inds, bf16.f32_to_bf16((raw / raw.sum(axis=1, keepdims=True)).astype(np.float32))


def _check(got_bits, want_tiles_bits, want_exact_bits, msg):
    got = bf16.bf16_to_f32(got_bits)
    assert_close(got, bf16.bf16_to_f32(want_tiles_bits), msg + " (bf16 tiles)")
    rep = value_report(got, bf16.bf16_to_f32(want_exact_bits))
    assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, (msg + " (exact weights)", rep)


@pytest.mark.parametrize("tokens,experts,slots,hidden,inter,group,shared", CASES,
                         ids=[f"T{c[0]}-E{c[1]}-K{c[2]}-H{c[3]}-I{c[4]}-g{c[5]}{'-shared' if c[6] else ''}"
                              for c in CASES])
def test_grouped_shapes_match_oracle(torch_mod, tokens, experts, slots, hidden, inter, group, shared):
    torch = torch_mod
    say(f"case: grouped shapes T={tokens} E={experts} K={slots} H={hidden} I={inter} g={group} shared={shared}")
    from flashnext_hip.grouped import GroupedMoE

    seed = 7000 + tokens + hidden + inter
    records = make_records(experts, hidden, inter, seed=seed, group=group)
    x = bf16_normal((tokens, hidden), seed=seed + 10)
    inds, scores = _routes(tokens, slots, experts, seed + 11)
    kwargs, call_kwargs, wsg = {}, {}, None
    if shared:
        sh_rec = make_records(1, hidden, inter, seed=seed + 12, group=group)
        records.shared = (sh_rec.gate, sh_rec.up, sh_rec.down)
        wsg = bf16_normal((1, hidden), seed=seed + 13, std=0.02)
        kwargs["shared_expert"] = tuple(tuple(t[:1] for t in to_dev_bank(b))
                                        for b in (sh_rec.gate, sh_rec.up, sh_rec.down))
        call_kwargs["shared_gate"] = to_dev_bf16(moe.shared_gate_value(x, wsg))
    want_out, want_y = moe.prefill_layer(x, inds, scores, records, shared_gate_weight=wsg, weights="bf16")
    exact_out, exact_y = moe.prefill_layer(x, inds, scores, records, shared_gate_weight=wsg)

    banks = tuple(to_dev_bank(b) for b in (records.gate, records.up, records.down))
    g = GroupedMoE(*banks, hidden=hidden, inter=inter, group_size=group, **kwargs)
    out, y = g(to_dev_bf16(x), torch.from_numpy(inds.astype(np.int32)).cuda(), to_dev_bf16(scores), **call_kwargs)
    torch.cuda.synchronize()
    _check(from_dev_bf16(y), want_y, exact_y, "per-slot y")
    _check(from_dev_bf16(out), want_out, exact_out, "combined out")
