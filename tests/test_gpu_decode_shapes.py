"""Decode executor across the input-width classes of its kernels.

The decode kernels pick a lane layout by the input width of each projection
(64-lane slices for 2048 and 4096 inputs, 16-lane slices with one to eight
32-input chunks per lane otherwise) and tile the output rows by waves.  These
cases give the gate/up projections (input = hidden) and the down projection
(input = inter) each class, with one to ten slots and one to eight tokens (the executor's bound),
at group 32 (float32 scores, the fused combine, the in-kernel shared expert)
and group 64 (bf16 scores, the generic combine order), and compare the layer
with ``oracle.moe.decode_layer``: max rel 1e-2 of the largest magnitude and
cosine >= 0.9999 (the layer bar), and elementwise within rtol 1e-2 and an
absolute 2^-8, one bf16 step of the unit-sized terms the combine adds: at 4096
inputs a float32 dot product now and then rounds to the other bf16 neighbour
than the float64 oracle does, and where the terms cancel that step is the
whole difference (2 of 32,768 outputs at 4096 x 1024, 8 tokens).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, moe

from ._helpers import assert_close, bf16_normal, from_dev_bf16, make_records, say, to_dev_bank, to_dev_bf16

pytestmark = pytest.mark.gpu

# (tokens, experts, k, hidden, inter, group)
CASES = [
    (1, 4, 1, 256, 128, 32),      # gate/up 16-lane x1, down 16-lane x1
    (2, 12, 10, 640, 384, 32),    # 16-lane x2 (partly idle lanes), down x1 (12 of 16 chunks)
    (5, 16, 8, 1536, 640, 32),    # 16-lane x3, down x2 (20 chunks)
    (8, 9, 3, 4096, 1024, 32),    # 64-lane x2, down x2, the executor's 8 tokens
    (3, 20, 10, 2560, 768, 32),   # 16-lane x5 (the checkpoint width), down x2
    (4, 10, 4, 1024, 512, 64),    # 16-lane x2, down x1, group 64
    (1, 8, 8, 2048, 1024, 64),    # 64-lane x1, down x2, group 64
]


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


@pytest.mark.parametrize("tokens,experts,k,hidden,inter,group", CASES,
                         ids=[f"T{c[0]}-E{c[1]}-K{c[2]}-H{c[3]}-I{c[4]}-g{c[5]}" for c in CASES])
def test_decode_shapes_match_oracle(torch_mod, tokens, experts, k, hidden, inter, group):
    torch = torch_mod
    say(f"case: decode shapes T={tokens} E={experts} K={k} H={hidden} I={inter} g={group}")
    from flashnext_hip.hip_runtime import HipMoEExecutor

    seed = 9000 + hidden + inter + tokens
    records = make_records(experts, hidden, inter, seed=seed, group=group)
    x = bf16_normal((tokens, hidden), seed=seed + 1)
    rng = np.random.default_rng(seed + 2)
    inds = np.stack([rng.permutation(experts)[:k] for _ in range(tokens)]).astype(np.int64)
    raw = rng.uniform(0.1, 1.0, (tokens, k)).astype(np.float32)
    scores = (raw / raw.sum(axis=1, keepdims=True)).astype(np.float32)
    dev = {name: to_dev_bank(bank) for name, bank in
           (("gate_proj", records.gate), ("up_proj", records.up), ("down_proj", records.down))}
    ex = HipMoEExecutor(experts, hidden, k, group_size=group)
    if group == 32:
        shared = make_records(1, hidden, inter, seed=seed + 3, group=group)
        wsg = bf16_normal((1, hidden), seed=seed + 4, std=0.02)
        sg = to_dev_bf16(moe.shared_gate_value(x, wsg))
        sh = {n: tuple(t[:1] for t in to_dev_bank(b)) for n, b in
              (("gate_proj", shared.gate), ("up_proj", shared.up), ("down_proj", shared.down))}
        out = ex.execute(to_dev_bf16(x), torch.from_numpy(inds).cuda(), dev,
                         scores=torch.from_numpy(scores).cuda(), shared_gate=sg, shared_expert=sh)
        recs = moe.ExpertRecordSet(records.gate, records.up, records.down,
                                   shared=(shared.gate, shared.up, shared.down))
        want = moe.decode_layer(x, inds, scores, recs, shared_gate_weight=wsg)
    else:
        sb = bf16.f32_to_bf16(scores)
        out = ex.execute(to_dev_bf16(x), torch.from_numpy(inds).cuda(), dev, scores=to_dev_bf16(sb))
        want = moe.decode_layer(x, inds, sb, records, score_dtype="bf16", combine="generic")
    torch.cuda.synchronize()
    assert ex.last_path == "custom-hip"
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out)), bf16.bf16_to_f32(want),
                 f"decode T={tokens} K={k} H={hidden} I={inter} g={group}", atol=2.0 ** -8)
