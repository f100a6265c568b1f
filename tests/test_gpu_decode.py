"""GPU parity of the decode path against the CPU oracle.

Bit-exact: unpack, dequant, router (logits, gates, top-k indices, scores,
route words, keeps, shared gate).  Within tolerance (rtol 1e-2, atol 3e-3,
max rel 1e-2, cosine 0.9999): QMV and layer outputs.  Bit-identical between
execution variants: fused/unfused up, dense/pool/stream addressing, fused
shared epilogues vs the separate add.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, moe, q4, router as orouter

from ._helpers import (assert_close, bf16_normal, from_dev_bf16, make_bank, make_records,
                       pool_from_banks, say, to_dev_bank, to_dev_bf16)

pytestmark = pytest.mark.gpu

H, I, E = 2048, 512, 16


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


@pytest.fixture(scope="module")
def records():
    say("building seeded banks E=16 H=2048 I=512")
    return make_records(E, H, I, seed=100)


@pytest.fixture(scope="module")
def shared_records():
    return make_records(1, H, I, seed=200)


@pytest.fixture(scope="module")
def dev_records(torch_mod, records):
    return {name: to_dev_bank(bank) for name, bank in
            (("gate_proj", records.gate), ("up_proj", records.up), ("down_proj", records.down))}


# ---------------------------------------------------------------- Q4 primitives
def test_unpack_bit_exact(torch_mod):
    torch = torch_mod
    say("case: unpack 1M words")
    rng = np.random.default_rng(7)
    words = rng.integers(0, 2 ** 32, (1024, 1024), dtype=np.uint64).astype(np.uint32)
    from flashnext_hip import ops

    got = ops.unpack(torch.from_numpy(words.view(np.int32)).cuda()).cpu().numpy()
    assert np.array_equal(got, q4.unpack_q4(words))


def test_dequant_bit_exact(torch_mod, records):
    say("case: dequant bank expert 0..3 gate")
    from flashnext_hip import ops

    w, s, b = to_dev_bank(records.gate)
    got = from_dev_bf16(ops.dequantize(w[:4], s[:4], b[:4]))
    want = q4.dequantize_bf16(records.gate.packed[:4], records.gate.scales[:4], records.gate.biases[:4])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,out_w,in_w,group", [(1, 5120, 2048, 32), (3, 640, 2560, 32),
                                                   (2, 2048, 640, 32), (1, 1024, 2048, 64)])
def test_quantized_matmul_bf16(torch_mod, rows, out_w, in_w, group):
    say(f"case: quantized_matmul rows={rows} out={out_w} in={in_w} g={group}")
    from flashnext_hip import ops

    bank = make_bank(1, out_w, in_w, seed=11 + out_w, group=group)
    x = bf16_normal((rows, in_w), seed=12)
    w, s, b = to_dev_bank(bank)
    y = ops.quantized_matmul(to_dev_bf16(x), w[0], s[0], b[0], group_size=group)
    got = bf16.bf16_to_f32(from_dev_bf16(y))
    want_f64 = q4.qmv_f64(bf16.bf16_to_f32(x), bank.packed[0], bank.scales[0], bank.biases[0], group)
    want = bf16.bf16_to_f32(bf16.f64_to_bf16(want_f64))
    rep = assert_close(got, want, "quantized_matmul")
    # every output within one bf16 rounding of the exact value
    ulp = np.abs(bf16.bf16_to_f32(bf16.f64_to_bf16(want_f64)).astype(np.float64)) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want_f64) <= ulp), rep


def test_quantized_matmul_f32_activations(torch_mod):
    torch = torch_mod
    say("case: quantized_matmul f32 x")
    from flashnext_hip import ops

    bank = make_bank(1, 512, 2048, seed=21)
    rng = np.random.default_rng(22)
    x = (rng.normal(0, 1, (2, 2048)) / 64).astype(np.float32)
    w, s, b = to_dev_bank(bank)
    y = ops.quantized_matmul(torch.from_numpy(x).cuda(), w[0], s[0], b[0]).cpu().numpy()
    want = q4.qmv_f64(x.astype(np.float64), bank.packed[0], bank.scales[0], bank.biases[0])
    assert_close(y, want, "f32 quantized_matmul", rtol=1e-3, atol=1e-4)


def test_gather_qmm_decode_shape(torch_mod, records, dev_records):
    torch = torch_mod
    say("case: gather_qmm x[...,1,1,H] indices[...,K]")
    from flashnext_hip import ops

    x = bf16_normal((2, H), seed=31)
    idx = np.array([[3, 0, 7], [15, 3, 1]], dtype=np.int64)
    xd = to_dev_bf16(x).reshape(2, 1, 1, H)
    out = ops.gather_qmm(xd, *dev_records["gate_proj"], rhs_indices=torch.from_numpy(idx).cuda())
    assert tuple(out.shape) == (2, 3, 1, I)
    got = bf16.bf16_to_f32(from_dev_bf16(out)).reshape(2, 3, I)
    xr = np.repeat(x, 3, axis=0)
    want = bf16.bf16_to_f32(q4.gather_qmm(xr, records.gate, idx.reshape(-1))).reshape(2, 3, I)
    assert_close(got, want, "gather_qmm")


# ---------------------------------------------------------------- router
@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_router_bit_exact(torch_mod, tokens):
    torch = torch_mod
    say(f"case: router tokens={tokens}")
    from flashnext_hip import router

    x = bf16_normal((tokens, H), seed=40 + tokens)
    wg = bf16_normal((512, H), seed=41, std=0.02)
    wsg = bf16_normal((1, H), seed=42, std=0.02)
    perm = np.random.default_rng(43).permutation(512).astype(np.uint32)
    res = router.route(to_dev_bf16(x), to_dev_bf16(wg), 10, slot_table=torch.from_numpy(perm.view(np.int32)).cuda(),
                       shared_gate_w=to_dev_bf16(wsg))
    torch.cuda.synchronize()
    ref = orouter.route(x, wg, 10, slot_table=perm)
    assert np.array_equal(from_dev_bf16(res.logits), ref["logits"])
    assert np.array_equal(res.inds.cpu().numpy().astype(np.uint32), ref["inds"])
    assert np.array_equal(from_dev_bf16(res.scores_raw), ref["scores_raw"])
    assert np.array_equal(from_dev_bf16(res.scores), ref["scores"])
    assert np.array_equal(res.routes.cpu().numpy().view(np.uint32), ref["routes"])
    assert res.keeps.cpu().numpy().tolist() == [10] * tokens
    sg = moe.shared_gate_value(x, wsg)
    assert np.array_equal(from_dev_bf16(res.shared_gate), sg)


@pytest.mark.parametrize("scale", [0.3, 1.5, 6.0, "coarse"])
def test_router_bit_exact_many_tokens(torch_mod, scale):
    """8192 tokens per logit scale: the float32 softmax with its midpoint guard
    must give the float64-exact bf16 gates, selection and scores every time
    (coarse logits produce many exactly tied gates)."""
    torch = torch_mod
    say(f"case: router 8192 tokens scale={scale}")
    from flashnext_hip import router

    tokens = 8192
    rng = np.random.default_rng({0.3: 60, 1.5: 61, 6.0: 62, "coarse": 63}[scale])
    if scale == "coarse":
        raw = np.round(rng.normal(0, 1.0, (tokens, 512)) * 4.0) / 4.0
    else:
        raw = rng.normal(0, scale, (tokens, 512))
    logits = bf16.f32_to_bf16(raw.astype(np.float32))
    perm = rng.permutation(512).astype(np.uint32)
    res = router.route(None, None, 10, logits=to_dev_bf16(logits),
                       slot_table=torch.from_numpy(perm.view(np.int32)).cuda())
    torch.cuda.synchronize()
    ref = orouter.route(None, None, 10, logits_bits=logits, slot_table=perm)
    assert np.array_equal(res.inds.cpu().numpy().astype(np.uint32), ref["inds"])
    assert np.array_equal(from_dev_bf16(res.scores_raw), ref["scores_raw"])
    assert np.array_equal(from_dev_bf16(res.scores), ref["scores"])
    assert np.array_equal(res.routes.cpu().numpy().view(np.uint32), ref["routes"])


def test_router_adaptive_keep_and_logits_input(torch_mod):
    torch = torch_mod
    say("case: router threshold=0.85 min_keep=2 from logits")
    from flashnext_hip import router

    tokens = 32
    rng = np.random.default_rng(50)
    logits = bf16.f32_to_bf16((rng.normal(0, 1.5, (tokens, 512))).astype(np.float32))
    res = router.route(None, None, 10, threshold=0.85, min_keep=2, logits=to_dev_bf16(logits),
                       score_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = orouter.route(None, None, 10, threshold=0.85, min_keep=2, logits_bits=logits)
    assert res.keeps.cpu().numpy().tolist() == ref["keeps"].tolist()
    assert np.array_equal(res.inds.cpu().numpy().astype(np.uint32), ref["inds"])
    assert np.array_equal(res.scores.cpu().numpy(), bf16.bf16_to_f32(ref["scores"]))
    assert res.width() == ref["width"]


def test_router_ties_pick_lowest_index(torch_mod):
    torch = torch_mod
    say("case: router all-equal logits")
    from flashnext_hip import router

    logits = np.zeros((2, 512), dtype=np.uint16)
    res = router.route(None, None, 10, logits=to_dev_bf16(logits))
    torch.cuda.synchronize()
    assert res.inds.cpu().numpy().tolist() == [list(range(10))] * 2
    assert np.all(from_dev_bf16(res.scores) == bf16.f32_to_bf16(np.float32(0.1)))


# ---------------------------------------------------------------- executor
def _executor(top_k, **kw):
    from flashnext_hip.hip_runtime import HipMoEExecutor

    return HipMoEExecutor(E, H, top_k, **kw)


def _routes_scores(tokens, k, seed):
    rng = np.random.default_rng(seed)
    inds = np.stack([rng.permutation(E)[:k] for _ in range(tokens)]).astype(np.int64)
    raw = rng.uniform(0.1, 1.0, (tokens, k)).astype(np.float32)
    scores = (raw / raw.sum(axis=1, keepdims=True)).astype(np.float32)
    return inds, scores


@pytest.mark.parametrize("tokens,k", [(1, 10), (4, 10), (8, 4), (2, 1)])
def test_decode_layer_matches_oracle(torch_mod, records, dev_records, tokens, k):
    torch = torch_mod
    say(f"case: decode layer tokens={tokens} k={k}")
    x = bf16_normal((tokens, H), seed=60 + tokens)
    inds, scores = _routes_scores(tokens, k, 61 + k)
    ex = _executor(k, fused_up_swiglu=True)
    out = ex.execute(to_dev_bf16(x), torch.from_numpy(inds).cuda(), dev_records,
                     scores=torch.from_numpy(scores).cuda())
    assert ex.last_path == "custom-hip"
    got = bf16.bf16_to_f32(from_dev_bf16(out))
    want = bf16.bf16_to_f32(moe.decode_layer(x, inds, scores, records))
    assert_close(got, want, f"decode T={tokens} K={k}")


def test_decode_return_all_matches_oracle(torch_mod, records, dev_records):
    torch = torch_mod
    say("case: decode return_all")
    x = bf16_normal((2, H), seed=70)
    inds, _ = _routes_scores(2, 10, 71)
    ex = _executor(10)
    g, u, d = ex.execute(to_dev_bf16(x), torch.from_numpy(inds).cuda(), dev_records, return_all=True)
    og, ou, _oa, od = moe.decode_layer(x, inds, None, records, return_all=True)
    for name, a, b in (("gate", g, og), ("up", u, ou), ("down", d, od)):
        assert_close(bf16.bf16_to_f32(from_dev_bf16(a)), bf16.bf16_to_f32(b), f"return_all {name}")


def test_fused_and_unfused_up_are_bit_identical(torch_mod, dev_records):
    torch = torch_mod
    say("case: fused vs unfused up")
    x = to_dev_bf16(bf16_normal((4, H), seed=80))
    inds, scores = _routes_scores(4, 10, 81)
    r, s = torch.from_numpy(inds).cuda(), torch.from_numpy(scores).cuda()
    a = _executor(10, fused_up_swiglu=True).execute(x, r, dev_records, scores=s)
    b = _executor(10, fused_up_swiglu=False).execute(x, r, dev_records, scores=s)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_shared_epilogues_bit_identical_to_separate_add(torch_mod, dev_records):
    torch = torch_mod
    say("case: shared_y / shared parts epilogues")
    x = to_dev_bf16(bf16_normal((2, H), seed=90))
    inds, scores = _routes_scores(2, 10, 91)
    r, s = torch.from_numpy(inds).cuda(), torch.from_numpy(scores).cuda()
    ex = _executor(10)
    base = ex.execute(x, r, dev_records, scores=s)
    shared_y = to_dev_bf16(bf16_normal((2, H), seed=92, std=0.25))
    fused = ex.execute(x, r, dev_records, scores=s, shared_y=shared_y)
    assert torch.equal(fused.view(torch.int16), (base.float() + shared_y.float()).bfloat16().view(torch.int16))
    shared = to_dev_bf16(bf16_normal((2, H), seed=93, std=0.25))
    gate = torch.tensor([[0.333984375], [0.75]], dtype=torch.bfloat16, device="cuda")
    fused = ex.execute(x, r, dev_records, scores=s, shared=shared, shared_gate=gate)
    comp = (gate.float() * shared.float()).bfloat16()
    assert torch.equal(fused.view(torch.int16), (base.float() + comp.float()).bfloat16().view(torch.int16))


def test_shared_expert_in_kernel_matches_oracle(torch_mod, records, dev_records, shared_records):
    torch = torch_mod
    say("case: in-kernel shared expert + sigmoid gate")
    tokens = 3
    x = bf16_normal((tokens, H), seed=100)
    wsg = bf16_normal((1, H), seed=101, std=0.02)
    inds, scores = _routes_scores(tokens, 10, 102)
    from flashnext_hip import router

    sg = router.route(to_dev_bf16(x), to_dev_bf16(bf16_normal((E, H), seed=103, std=0.02)), 10,
                      shared_gate_w=to_dev_bf16(wsg)).shared_gate
    sh = {n: tuple(t[:1] for t in to_dev_bank(b)) for n, b in
          (("gate_proj", shared_records.gate), ("up_proj", shared_records.up), ("down_proj", shared_records.down))}
    out = _executor(10).execute(to_dev_bf16(x), torch.from_numpy(inds).cuda(), dev_records,
                                scores=torch.from_numpy(scores).cuda(), shared_gate=sg, shared_expert=sh)
    recs = moe.ExpertRecordSet(records.gate, records.up, records.down,
                               shared=(shared_records.gate, shared_records.up, shared_records.down))
    want = moe.decode_layer(x, inds, scores, recs, shared_gate_weight=wsg)
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out)), bf16.bf16_to_f32(want), "shared expert layer")


def test_pool_and_stream_pack_addressing_bit_identical(torch_mod, records, dev_records):
    torch = torch_mod
    say("case: pool slot words and stream pack")
    tokens, k = 2, 10
    x = to_dev_bf16(bf16_normal((tokens, H), seed=110))
    inds, scores = _routes_scores(tokens, k, 111)
    s = torch.from_numpy(scores).cuda()
    ex = _executor(k)
    dense = ex.execute(x, torch.from_numpy(inds).cuda(), dev_records, scores=s)
    slots = 24
    perm = np.random.default_rng(112).permutation(slots)[:E]
    img, stride = pool_from_banks(records, perm, slots, H, I)
    pool_t = torch.from_numpy(img).cuda()
    words = (np.uint64(0x80000000) | perm[inds].astype(np.uint64)).astype(np.int64)
    pooled = ex.execute(x, torch.from_numpy(words).cuda(), dev_records, scores=s, slab_pack=pool_t)
    assert torch.equal(dense.view(torch.int16), pooled.view(torch.int16))
    # streamed experts: expert-major records without header, plain expert ids
    stream_img = img[4096:].copy()
    stream_t = torch.from_numpy(stream_img).cuda()
    inv = np.empty(slots, dtype=np.int64)
    inv[perm] = np.arange(E)
    mixed = perm[inds].astype(np.int64)  # stream record index = slot position
    streamed = ex.execute(x, torch.from_numpy(mixed).cuda(), dev_records, scores=s, slab_pack=pool_t,
                          stream_pack=stream_t)
    assert torch.equal(dense.view(torch.int16), streamed.view(torch.int16))


@pytest.mark.parametrize("tokens,threshold", [(1, 1.0), (4, 1.0), (8, 0.85)])
def test_fused_routed_layer_matches_unfused_and_oracle(torch_mod, records, shared_records, tokens, threshold):
    torch = torch_mod
    say(f"case: fused routed layer tokens={tokens} threshold={threshold}")
    from flashnext_hip.layout import make_layout
    from flashnext_hip.moe_block import DecodeLayer, LayerWeights

    slots = 24
    perm = np.random.default_rng(160).permutation(slots)[:E].astype(np.int32)
    img, _ = pool_from_banks(records, perm, slots, H, I)
    wg = bf16_normal((E, H), seed=161, std=0.02)
    wsg = bf16_normal((1, H), seed=162, std=0.02)
    sh = tuple(tuple(t[:1] for t in to_dev_bank(b)) for b in (shared_records.gate, shared_records.up,
                                                               shared_records.down))
    weights = LayerWeights(make_layout(H, I), torch.from_numpy(img).cuda(), torch.from_numpy(perm).cuda(),
                           to_dev_bf16(wg), to_dev_bf16(wsg).reshape(-1), sh)
    layer = DecodeLayer(weights, tokens, 10, threshold=threshold, min_keep=2)
    x = bf16_normal((tokens, H), seed=163)
    layer.x.copy_(to_dev_bf16(x))
    layer.launch(None)
    torch.cuda.synchronize()
    fused = layer.out.clone()
    published = [t.clone() for t in (layer.routes, layer.inds, layer.scores, layer.shared_gate)]
    if threshold < 1:
        published.append(layer.keeps.clone())
    layer.launch_unfused(None)
    torch.cuda.synchronize()
    again = [layer.routes, layer.inds, layer.scores, layer.shared_gate] + ([layer.keeps] if threshold < 1 else [])
    for a, b in zip(published, again):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)
    assert torch.equal(fused.view(torch.int16), layer.out.view(torch.int16))
    from flashnext_hip import _lib

    assert _lib.check_device_errors() == 0
    ref = orouter.route(x, wg, 10, threshold=threshold, min_keep=2, slot_table=perm.astype(np.uint32))
    assert np.array_equal(layer.inds.cpu().numpy().astype(np.uint32), ref["inds"])
    assert np.array_equal(layer.routes.cpu().numpy().view(np.uint32), ref["routes"])
    recs = moe.ExpertRecordSet(records.gate, records.up, records.down,
                               shared=(shared_records.gate, shared_records.up, shared_records.down))
    want = moe.decode_layer(x, ref["inds"], ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg,
                            keeps=ref["keeps"] if threshold < 1 else None)
    assert_close(bf16.bf16_to_f32(from_dev_bf16(fused)), bf16.bf16_to_f32(want), "fused routed layer")


def _routed_layer(torch, records, shared_records, tokens, top_k, threshold, seed):
    from flashnext_hip.layout import make_layout
    from flashnext_hip.moe_block import DecodeLayer, LayerWeights

    slots = 24
    perm = np.random.default_rng(seed).permutation(slots)[:E].astype(np.int32)
    img, _ = pool_from_banks(records, perm, slots, H, I)
    sh = tuple(tuple(t[:1] for t in to_dev_bank(b)) for b in (shared_records.gate, shared_records.up,
                                                               shared_records.down))
    weights = LayerWeights(make_layout(H, I), torch.from_numpy(img).cuda(), torch.from_numpy(perm).cuda(),
                           to_dev_bf16(bf16_normal((E, H), seed=seed + 1, std=0.02)),
                           to_dev_bf16(bf16_normal((1, H), seed=seed + 2, std=0.02)).reshape(-1), sh)
    return DecodeLayer(weights, tokens, top_k, threshold=threshold, min_keep=2)


def test_routed_layer_repeated_launches_graph_replays_and_mixed_shapes(torch_mod, records, shared_records):
    """The routed layer entry point (router + selection folded into gate/up +
    down) must match the separate router and expert calls bit for bit across
    back-to-back eager launches, graph replays with fresh tokens between
    replays, and layers of different slot counts and keep thresholds run in
    turn, with no device error flag raised."""
    torch = torch_mod
    from flashnext_hip import _lib

    layers = [_routed_layer(torch, records, shared_records, 1, 10, 1.0, 170),
              _routed_layer(torch, records, shared_records, 1, 8, 1.0, 180),
              _routed_layer(torch, records, shared_records, 1, 10, 0.85, 190)]
    rng = np.random.default_rng(175)

    def check(layer, tag):
        fused = layer.out.clone()
        routes = layer.routes.clone()
        layer.launch_unfused(None)
        torch.cuda.synchronize()
        assert torch.equal(routes, layer.routes), tag
        assert torch.equal(fused.view(torch.int16), layer.out.view(torch.int16)), tag

    for it in range(4):
        for n, layer in enumerate(layers):
            say(f"case: eager fused launch iteration {it} layer {n}")
            layer.x.copy_(to_dev_bf16(bf16.f32_to_bf16(rng.normal(0, 1, (1, H)).astype(np.float32))))
            layer.launch(None)
            torch.cuda.synchronize()
            check(layer, f"eager it={it} layer={n}")
    assert _lib.check_device_errors() == 0
    stream = torch.cuda.Stream()
    handle = stream.cuda_stream
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        for layer in layers:
            layer.launch(handle)
    for rep in range(4):
        say(f"case: graph replay {rep} of three fused layers")
        xs = [to_dev_bf16(bf16.f32_to_bf16(rng.normal(0, 1, (1, H)).astype(np.float32))) for _ in layers]
        for layer, xv in zip(layers, xs):
            layer.x.copy_(xv)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        outs = [layer.out.clone() for layer in layers]
        for n, (layer, o) in enumerate(zip(layers, outs)):
            layer.launch_unfused(None)
            torch.cuda.synchronize()
            assert torch.equal(o.view(torch.int16), layer.out.view(torch.int16)), f"replay {rep} layer {n}"
    assert _lib.check_device_errors() == 0


def test_out_of_range_route_word_is_skipped_and_flagged(torch_mod, records, dev_records):
    torch = torch_mod
    say("case: slot word beyond the pool is bound-checked in-kernel")
    from flashnext_hip import _lib

    _lib.check_device_errors()  # start clean
    x = to_dev_bf16(bf16_normal((1, H), seed=115))
    slots = 4
    img, _stride = pool_from_banks(records, np.arange(slots), slots, H, I)
    pool_t = torch.from_numpy(img).cuda()
    scores = torch.tensor([[0.5, 0.5]], dtype=torch.float32, device="cuda")
    good = np.array([[0x80000000 | 1, 0x80000000 | 2]], dtype=np.int64)
    bad = np.array([[0x80000000 | 1, 0x80000000 | 1000]], dtype=np.int64)
    ex = _executor(2)
    ex.execute(x, torch.from_numpy(good).cuda(), dev_records, scores=scores, slab_pack=pool_t)
    assert _lib.check_device_errors() == 0
    half = ex.execute(x, torch.from_numpy(bad).cuda(), dev_records, scores=scores, slab_pack=pool_t)
    with pytest.raises(ValueError, match="route word"):
        _lib.check_device_errors()
    # the bad slot contributed nothing: equal to a single-slot route scaled by 0.5
    one = ex.execute(x, torch.from_numpy(good[:, :1].repeat(2, axis=1)).cuda(), dev_records,
                     scores=torch.tensor([[0.5, 0.0]], device="cuda"), slab_pack=pool_t)
    assert torch.equal(half.view(torch.int16), one.view(torch.int16))
    assert _lib.check_device_errors() == 0


def test_f32_activations_decode(torch_mod, records, dev_records):
    torch = torch_mod
    say("case: decode f32 activations")
    x = (np.random.default_rng(120).normal(0, 1, (1, H)) / 16).astype(np.float32)
    inds, scores = _routes_scores(1, 3, 121)
    out = _executor(3).execute(torch.from_numpy(x).cuda(), torch.from_numpy(inds).cuda(), dev_records,
                               scores=torch.from_numpy(scores).cuda())
    want = moe.decode_layer(x, inds, scores, records, dtype="f32")
    assert_close(out.cpu().numpy(), want, "f32 decode", rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("width", list(range(1, 11)))
def test_adaptive_widths(torch_mod, records, dev_records, width):
    torch = torch_mod
    say(f"case: width {width}")
    x = bf16_normal((1, H), seed=130)
    inds = np.arange(width, dtype=np.int64).reshape(1, width)
    sc = np.arange(1, width + 1, dtype=np.float32).reshape(1, width)
    sc = sc / sc.sum(axis=-1, keepdims=True)
    out = _executor(width).execute(to_dev_bf16(x), torch.from_numpy(inds).cuda(), dev_records,
                                   scores=torch.from_numpy(sc).cuda())
    want = moe.decode_layer(x, inds, sc, records)
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out)), bf16.bf16_to_f32(want), f"width {width}")


def test_checkpoint_shape_seven_slots(torch_mod):
    torch = torch_mod
    say("case: checkpoint shape 2560/640, 7 slots")
    from flashnext_hip.hip_runtime import HipMoEExecutor

    recs = make_records(8, 2560, 640, seed=140)
    dev = {n: to_dev_bank(b) for n, b in (("gate_proj", recs.gate), ("up_proj", recs.up), ("down_proj", recs.down))}
    x = bf16_normal((1, 2560), seed=141)
    inds = np.arange(7, dtype=np.int64).reshape(1, 7)
    sc = np.arange(1, 8, dtype=np.float32).reshape(1, 7)
    sc = sc / sc.sum()
    out = HipMoEExecutor(8, 2560, 7).execute(to_dev_bf16(x), torch.from_numpy(inds).cuda(), dev,
                                               scores=torch.from_numpy(sc).cuda())
    want = moe.decode_layer(x, inds, sc, recs)
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out)), bf16.bf16_to_f32(want), "checkpoint shape")


def test_keeps_skip_padded_slots(torch_mod, records, dev_records):
    torch = torch_mod
    say("case: keeps from adaptive router skip padded slots")
    from flashnext_hip import _lib
    from flashnext_hip._tensors import ptr, stream_handle

    x = bf16_normal((2, H), seed=150)
    inds, scores = _routes_scores(2, 10, 151)
    keeps = np.array([3, 10], dtype=np.int32)
    pad_inds = np.where(np.arange(10)[None] >= keeps[:, None], inds[:, :1], inds)
    pad_scores = np.where(np.arange(10)[None] >= keeps[:, None], 0.0, scores).astype(np.float32)
    want = moe.decode_layer(x, pad_inds, pad_scores, records)
    ex = _executor(10)
    full = ex.execute(to_dev_bf16(x), torch.from_numpy(pad_inds).cuda(), dev_records,
                      scores=torch.from_numpy(pad_scores).cuda())
    assert_close(bf16.bf16_to_f32(from_dev_bf16(full)), bf16.bf16_to_f32(want), "padded slots")
    # same call through the C ABI with keeps: padded slots are skipped, result identical
    xd = to_dev_bf16(x)
    routes = torch.from_numpy(pad_inds.astype(np.int32)).cuda()
    sd = torch.from_numpy(pad_scores).cuda()
    kd = torch.from_numpy(keeps).cuda()
    out = torch.empty((2, H), dtype=torch.bfloat16, device="cuda")
    act = torch.empty((20, I), dtype=torch.bfloat16, device="cuda")
    a = _lib.MqMoeArgs()
    a.x, a.x_dtype = ptr(xd), _lib.MQ_BF16
    from flashnext_hip.ops import dense_projection

    a.gate = dense_projection(*dev_records["gate_proj"])
    a.up = dense_projection(*dev_records["up_proj"])
    a.down = dense_projection(*dev_records["down_proj"])
    a.routes, a.scores, a.score_dtype, a.keeps = ptr(routes), ptr(sd), _lib.MQ_F32, ptr(kd)
    a.out, a.act_out = ptr(out), ptr(act)
    a.tokens, a.slots, a.hidden, a.inter, a.expert_count, a.group_size = 2, 10, H, I, E, 32
    lib = _lib.load()
    _lib.check(lib.mq_moe_decode(a, stream_handle()), lib)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))
