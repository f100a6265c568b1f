"""GPU parity of the ``_moe_call`` composition at every token count, and the
segmented-equals-single premise of the sorted prefill path.

``MoEBlock`` runs up to 8 tokens through the routed decode layer (ordered
float32 combine, ``adaptive_topk.py:266-292``) and more through the router +
grouped path with the bf16 generic combine (``adaptive_topk.py:274-277``).
Routes are compared bit for bit with ``oracle.router.route``; outputs with
``oracle.moe.decode_layer`` or ``oracle.moe.prefill_layer`` at the layer
tolerance (rtol 1e-2, atol 3e-3, max rel 1e-2, cosine 0.9999).

The segmented test restates ``models/flashnext/tests/unit/test_prefill_pipeline_math.py:21-54``:
the (token, slot) rows sorted by expert and computed in contiguous expert
chunks must give the bits of one call over all rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, moe, router as orouter

from ._helpers import (MAX_REL, MIN_COSINE, assert_close, bf16_normal, from_dev_bf16, make_records,
                       pool_from_banks, say, to_dev_bank, to_dev_bf16, value_report)

pytestmark = pytest.mark.gpu

H, I, E, K = 2048, 512, 16, 10


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


@pytest.fixture(scope="module")
def layer(torch_mod):
    torch = torch_mod
    from flashnext_hip.layout import make_layout
    from flashnext_hip.moe_block import LayerWeights

    records = make_records(E, H, I, seed=500)
    shared = make_records(1, H, I, seed=501)
    slots = 24
    perm = np.random.default_rng(502).permutation(slots)[:E].astype(np.int32)
    img, _ = pool_from_banks(records, perm, slots, H, I)
    wg = bf16_normal((E, H), seed=503, std=0.02)
    wsg = bf16_normal((1, H), seed=504, std=0.02)
    sh = tuple(tuple(t[:1] for t in to_dev_bank(b)) for b in (shared.gate, shared.up, shared.down))
    weights = LayerWeights(make_layout(H, I), torch.from_numpy(img).cuda(), torch.from_numpy(perm).cuda(),
                           to_dev_bf16(wg), to_dev_bf16(wsg).reshape(-1), sh)
    recs = moe.ExpertRecordSet(records.gate, records.up, records.down, shared=(shared.gate, shared.up, shared.down))
    return weights, recs, perm, wg, wsg


@pytest.mark.parametrize("tokens,threshold,routed_max", [
    (1, 1.0, 64), (3, 0.85, 64), (4, 1.0, 64), (5, 0.85, 64), (8, 1.0, 64), (9, 1.0, 64), (40, 0.85, 64),
    (64, 1.0, 64), (9, 1.0, 0), (40, 0.85, 0), (130, 1.0, 64)])
def test_moe_block_matches_oracle_on_every_path(torch_mod, layer, tokens, threshold, routed_max):
    torch = torch_mod
    say(f"case: moe block tokens={tokens} threshold={threshold} routed_max={routed_max}")
    from flashnext_hip import _lib
    from flashnext_hip.moe_block import MoEBlock

    weights, recs, perm, wg, wsg = layer
    block = MoEBlock(weights, K, threshold=threshold, min_keep=2, routed_max_tokens=routed_max)
    x = bf16_normal((tokens, H), seed=510 + tokens)
    out = block(to_dev_bf16(x))
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0
    path = "fused" if tokens <= 8 else "routed" if tokens <= routed_max else "grouped"
    assert block.last_path == path
    ref = orouter.route(x, wg, K, threshold=threshold, min_keep=2, slot_table=perm.astype(np.uint32))
    r = block.last_route
    assert np.array_equal(r.routes.cpu().numpy().view(np.uint32), ref["routes"])
    assert np.array_equal(from_dev_bf16(r.scores), ref["scores"])
    got = bf16.bf16_to_f32(from_dev_bf16(out))
    keeps = ref["keeps"] if threshold < 1 else None
    if path == "fused":
        want = moe.decode_layer(x, ref["inds"], ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg,
                                keeps=keeps)
        assert_close(got, bf16.bf16_to_f32(want), f"fused block T={tokens}")
        return
    if path == "routed":  # the grouped path's semantics (generic bf16 combine) through the decode kernels
        want = moe.decode_layer(x, ref["inds"], ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg,
                                keeps=keeps, combine="generic")
        assert_close(got, bf16.bf16_to_f32(want), f"routed block T={tokens}")
        width = ref["width"]
        exact, _ = moe.prefill_layer(x, ref["inds"][:, :width], ref["scores"][:, :width], recs,
                                     shared_gate_weight=wsg)
        rep = value_report(got, bf16.bf16_to_f32(exact))
        assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, rep
        return
    width = ref["width"]
    tiles, _ = moe.prefill_layer(x, ref["inds"][:, :width], ref["scores"][:, :width], recs,
                                 shared_gate_weight=wsg, weights="bf16")
    exact, _ = moe.prefill_layer(x, ref["inds"][:, :width], ref["scores"][:, :width], recs,
                                 shared_gate_weight=wsg)
    assert_close(got, bf16.bf16_to_f32(tiles), f"grouped block T={tokens} (bf16 tiles)")
    rep = value_report(got, bf16.bf16_to_f32(exact))
    assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, rep
    # a second call at the same size reuses the grouped workspace and gives the same bits
    again = block(to_dev_bf16(x))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))


def test_routed_layer_sixteen_tokens_matches_separate_calls(torch_mod, layer):
    torch = torch_mod
    say("case: routed layer entry point at 16 tokens")
    from flashnext_hip.moe_block import DecodeLayer

    weights, recs, perm, wg, wsg = layer
    dl = DecodeLayer(weights, 16, K)
    x = bf16_normal((16, H), seed=520)
    dl.x.copy_(to_dev_bf16(x))
    dl.launch(None)
    torch.cuda.synchronize()
    out, routes = dl.out.clone(), dl.routes.clone()
    dl.launch_unfused(None)
    torch.cuda.synchronize()
    assert torch.equal(routes, dl.routes)
    assert torch.equal(out.view(torch.int16), dl.out.view(torch.int16))
    ref = orouter.route(x, wg, K, slot_table=perm.astype(np.uint32))
    want = moe.decode_layer(x, ref["inds"], ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg)
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out)), bf16.bf16_to_f32(want), "routed layer T=16")


def test_segmented_sorted_rows_equal_one_call(torch_mod):
    torch = torch_mod
    say("case: segmented grouped rows T=96 K=8 E=40 H=2560 I=640")
    from flashnext_hip.grouped import GroupedMoE

    tokens, slots, hidden, inter, experts, chunk = 96, 8, 2560, 640, 40, 11
    records = make_records(experts, hidden, inter, seed=530)
    x = bf16.f32_to_bf16((np.random.default_rng(531).normal(0, 0.5, (tokens, hidden))).astype(np.float32))
    inds = np.random.default_rng(532).integers(0, experts, (tokens, slots))
    banks = tuple(to_dev_bank(b) for b in (records.gate, records.up, records.down))
    xd = to_dev_bf16(x)
    _, y_all = GroupedMoE(*banks, hidden=hidden, inter=inter)(xd, torch.from_numpy(inds.astype(np.int32)).cuda(),
                                                              combine=False)
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")  # the sorted (token, slot) rows
    y_seg = torch.zeros_like(y_all)
    done = 0
    for start in range(0, experts, chunk):
        end = min(experts, start + chunk)
        rows = order[(flat[order] >= start) & (flat[order] < end)]
        if rows.size == 0:
            continue
        seg_banks = tuple(tuple(t[start:end] for t in bank) for bank in banks)
        g = GroupedMoE(*seg_banks, hidden=hidden, inter=inter)
        local = torch.from_numpy((flat[rows] - start).astype(np.int32).reshape(-1, 1)).cuda()
        t_idx = torch.from_numpy(rows // slots).cuda()
        s_idx = torch.from_numpy(rows % slots).cuda()
        _, y_c = g(xd[t_idx].contiguous(), local, combine=False)
        y_seg[t_idx, s_idx] = y_c[:, 0]
        done += rows.size
    torch.cuda.synchronize()
    assert done == tokens * slots
    assert torch.equal(y_all.view(torch.int16), y_seg.view(torch.int16))


@pytest.mark.parametrize("tokens", [3, 16])
def test_many_token_layer_rows_equal_single_token_layers(torch_mod, layer, tokens):
    """Tokens are independent: a many-token routed layer (16 tokens: one
    selection pass, the expert kernels taking several row groups per wave, the
    router's token groups; 3 tokens: the selection folded into gate/up, one
    token per wave) gives each token the bits of a 1-token layer (selection
    folded into gate/up, one row group per wave)."""
    torch = torch_mod
    say(f"case: {tokens}-token layer rows vs 1-token layers")
    from flashnext_hip.moe_block import DecodeLayer

    weights = layer[0]
    for threshold in (1.0, 0.85):
        many = DecodeLayer(weights, tokens, K, threshold=threshold, min_keep=2)
        one = DecodeLayer(weights, 1, K, threshold=threshold, min_keep=2)
        x = to_dev_bf16(bf16_normal((tokens, H), seed=540))
        many.x.copy_(x)
        many.launch(None)
        torch.cuda.synchronize()
        for t in range(tokens):
            one.x.copy_(x[t:t + 1])
            one.launch(None)
            torch.cuda.synchronize()
            for name in ("routes", "inds", "keeps", "logits"):
                assert torch.equal(getattr(many, name)[t:t + 1].view(-1), getattr(one, name).view(-1)), (name, t)
            for name in ("scores", "shared_gate", "out"):
                a, b = getattr(many, name)[t:t + 1], getattr(one, name)
                assert torch.equal(a.reshape(-1).view(torch.int16), b.reshape(-1).view(torch.int16)), (name, t)


def test_many_token_shared_epilogues_equal_single_token_calls(torch_mod):
    """shared_y and shared/shared_gate epilogues at 8 tokens (several row
    groups per down wave) against the same tokens one call at a time."""
    torch = torch_mod
    say("case: 8-token executor epilogues vs 1-token calls")
    from flashnext_hip.hip_runtime import HipMoEExecutor

    experts, tokens = 16, 8
    records = make_records(experts, H, I, seed=550)
    dev = {n: to_dev_bank(b) for n, b in (("gate_proj", records.gate), ("up_proj", records.up),
                                           ("down_proj", records.down))}
    rng = np.random.default_rng(551)
    inds = np.stack([rng.choice(experts, K, replace=False) for _ in range(tokens)]).astype(np.int64)
    raw = rng.random((tokens, K)).astype(np.float32) + 0.05
    sc = torch.from_numpy((raw / raw.sum(1, keepdims=True)).astype(np.float32)).cuda()
    x = to_dev_bf16(bf16_normal((tokens, H), seed=552))
    r = torch.from_numpy(inds).cuda()
    shared_y = to_dev_bf16(bf16_normal((tokens, H), seed=553, std=0.25))
    shared = to_dev_bf16(bf16_normal((tokens, H), seed=554, std=0.25))
    gate = to_dev_bf16(bf16.f32_to_bf16(rng.random((tokens, 1)).astype(np.float32)))
    ex = HipMoEExecutor(experts, H, K, max_tokens=tokens)
    for kw in ({}, {"shared_y": shared_y}, {"shared": shared, "shared_gate": gate}):
        full = ex.execute(x, r, dev, scores=sc, **kw)
        torch.cuda.synchronize()
        for t in range(tokens):
            kw1 = {k: v[t:t + 1] for k, v in kw.items()}
            one = ex.execute(x[t:t + 1], r[t:t + 1], dev, scores=sc[t:t + 1], **kw1)
            torch.cuda.synchronize()
            assert torch.equal(full[t:t + 1].view(torch.int16), one.view(torch.int16)), (sorted(kw), t)


def _build_layer(torch, hidden, inter, group, seed):
    from flashnext_hip.layout import make_layout
    from flashnext_hip.moe_block import LayerWeights

    records = make_records(E, hidden, inter, seed=seed, group=group)
    shared = make_records(1, hidden, inter, seed=seed + 1, group=group)
    slots = 24
    perm = np.random.default_rng(seed + 2).permutation(slots)[:E].astype(np.int32)
    img, _ = pool_from_banks(records, perm, slots, hidden, inter, group)
    wg = bf16_normal((E, hidden), seed=seed + 3, std=0.02)
    wsg = bf16_normal((1, hidden), seed=seed + 4, std=0.02)
    sh = tuple(tuple(t[:1] for t in to_dev_bank(b)) for b in (shared.gate, shared.up, shared.down))
    weights = LayerWeights(make_layout(hidden, inter, group), torch.from_numpy(img).cuda(),
                           torch.from_numpy(perm).cuda(), to_dev_bf16(wg), to_dev_bf16(wsg).reshape(-1), sh)
    recs = moe.ExpertRecordSet(records.gate, records.up, records.down, shared=(shared.gate, shared.up, shared.down))
    return weights, recs, perm, wg, wsg


@pytest.fixture(scope="module")
def checkpoint_shape_layers(torch_mod):
    say("building 2560/640 layers at group 32 and group 64")
    return {group: _build_layer(torch_mod, 2560, 640, group, seed=560 + group) for group in (32, 64)}


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("tokens", [3, 8, 9, 40])
def test_moe_block_checkpoint_shape_adaptive_keep(torch_mod, checkpoint_shape_layers, group, tokens):
    """``_moe_call`` at the checkpoint shape (hidden 2560, inter 640: the
    non-fast 640-wide down path) with the chat default keep threshold 0.85
    (``adaptive_topk.py:75-232``) on every path: the fused routed layer up to
    8 tokens (fused float32 combine at group 32, the generic bf16 order at group
    64, ``metal_runtime.py:908-929``), beyond it the routed layer with the
    generic bf16 combine and, with that path off, the grouped path."""
    torch = torch_mod
    say(f"case: moe block 2560/640 g{group} tokens={tokens} threshold=0.85")
    from flashnext_hip import _lib
    from flashnext_hip.moe_block import MoEBlock

    hidden = 2560
    weights, recs, perm, wg, wsg = checkpoint_shape_layers[group]
    block = MoEBlock(weights, K, threshold=0.85, min_keep=2)
    x = bf16_normal((tokens, hidden), seed=570 + tokens + group)
    out = block(to_dev_bf16(x))
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0
    ref = orouter.route(x, wg, K, threshold=0.85, min_keep=2, slot_table=perm.astype(np.uint32))
    r = block.last_route
    assert np.array_equal(r.routes.cpu().numpy().view(np.uint32), ref["routes"])
    assert np.array_equal(from_dev_bf16(r.scores), ref["scores"])
    assert np.array_equal(r.keeps.cpu().numpy(), ref["keeps"])
    assert (ref["keeps"] < K).any(), "the threshold should drop slots for some token"
    got = bf16.bf16_to_f32(from_dev_bf16(out))
    if tokens <= 8:
        assert block.last_path == "fused"
        want = moe.decode_layer(x, ref["inds"], ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg,
                                keeps=ref["keeps"], combine="generic" if group == 64 else "fused")
        assert_close(got, bf16.bf16_to_f32(want), f"fused block g{group} T={tokens}")
        return
    assert block.last_path == "routed"
    want = moe.decode_layer(x, ref["inds"], ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg,
                            keeps=ref["keeps"], combine="generic")
    assert_close(got, bf16.bf16_to_f32(want), f"routed block g{group} T={tokens}")
    # the grouped path at the same size (routed path off)
    grouped = MoEBlock(weights, K, threshold=0.85, min_keep=2, routed_max_tokens=0)
    got_g = bf16.bf16_to_f32(from_dev_bf16(grouped(to_dev_bf16(x))))
    torch.cuda.synchronize()
    assert grouped.last_path == "grouped"
    width = ref["width"]
    tiles, _ = moe.prefill_layer(x, ref["inds"][:, :width], ref["scores"][:, :width], recs,
                                 shared_gate_weight=wsg, weights="bf16")
    assert_close(got_g, bf16.bf16_to_f32(tiles), f"grouped block g{group} T={tokens} (bf16 tiles)")


def test_group64_executor_shared_expert_generic_order(torch_mod, checkpoint_shape_layers):
    """The group-64 executor with an in-kernel shared expert: the routed slots
    combine in the generic bf16 order and the shared expert is added (it is
    not dropped), against the oracle."""
    torch = torch_mod
    say("case: group-64 executor with shared expert")
    from flashnext_hip.hip_runtime import HipMoEExecutor
    from flashnext_hip import router

    hidden, inter, tokens = 2560, 640, 3
    weights, recs, perm, wg, wsg = checkpoint_shape_layers[64]
    banks = {n: to_dev_bank(b) for n, b in (("gate_proj", recs.gate), ("up_proj", recs.up),
                                             ("down_proj", recs.down))}
    sh = {n: tuple(t[:1] for t in to_dev_bank(b)) for n, b in zip(("gate_proj", "up_proj", "down_proj"), recs.shared)}
    x = bf16_normal((tokens, hidden), seed=580)
    ref = orouter.route(x, wg, K)
    sg = router.route(to_dev_bf16(x), to_dev_bf16(wg), K, shared_gate_w=to_dev_bf16(wsg)).shared_gate
    ex = HipMoEExecutor(E, hidden, K, group_size=64)
    out = ex.execute(to_dev_bf16(x), torch.from_numpy(ref["inds"].astype(np.int64)).cuda(), banks,
                     scores=to_dev_bf16(ref["scores"]), shared_gate=sg, shared_expert=sh)
    torch.cuda.synchronize()
    want = moe.decode_layer(x, ref["inds"], ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg,
                            combine="generic")
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out)), bf16.bf16_to_f32(want), "g64 executor + shared expert")
    no_shared = ex.execute(to_dev_bf16(x), torch.from_numpy(ref["inds"].astype(np.int64)).cuda(), banks,
                           scores=to_dev_bf16(ref["scores"]))
    assert not torch.equal(out.view(torch.int16), no_shared.view(torch.int16))
