"""GPU parity at the full benchmark shapes (hidden 2048, 512 experts top-10 +
shared, inter 512, affine Q4 g32).

* Decode layer, 1 token, with the top-10 selection folded into the gate/up
  kernel, and the 4- and 16-token verify batches; routes into a random
  permutation of 512 pool slots.  Indices, scores and route words bit-exact
  against ``oracle.router.route``; outputs against ``oracle.moe.decode_layer``
  at the layer tolerance (rtol 1e-2, atol 3e-3, max rel 1e-2, cosine 0.9999).
* The 4096-token prefill chunk with Zipf(1.1) expert counts over 512 experts
  through the grouped path: every row of the 8 heaviest and 8 lightest
  experts and the combined rows of 256 random tokens against
  ``oracle.moe`` (bf16 tiles elementwise at the reference's rtol 2e-2 / atol
  3e-3 over 7.5 million values; exact weights by max rel / cosine),
  and the segmented-equals-single property of the sorted prefill
  (``models/flashnext/tests/unit/test_prefill_pipeline_math.py:21-54``) at
  full size: four 1024-token calls give the bits of the one 4096-token call.
* The 48-block stack decoded through a 6 GB LRU hot pool (and a 64-slot pool
  that evicts within every step) with pinned-host refills: every layer's
  output bit-identical to the same layer run with all 512 experts resident
  (``models/flashnext/expert_pool.py:88-145``, ``expert_cache.py:1694-1741``).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, moe, q4, router as orouter

from ._helpers import (MAX_REL, MIN_COSINE, REF_RTOL, assert_close, bf16_normal, from_dev_bf16, say, to_dev_bf16,
                       value_report)

pytestmark = pytest.mark.gpu

H, I, E, K, G = 2048, 512, 512, 10, 32


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


def _host_bank(torch, dense_bank, experts):
    sel = torch.tensor(list(experts), device=dense_bank.weight.device, dtype=torch.long)
    return q4.ExpertBank(dense_bank.weight[sel].cpu().numpy().view(np.uint32),
                         dense_bank.scales[sel].view(torch.int16).cpu().numpy().view(np.uint16),
                         dense_bank.biases[sel].view(torch.int16).cpu().numpy().view(np.uint16), G)


def _records_for(torch, dense, experts, shared=None):
    """ExpertRecordSet of the listed experts (local ids 0..n-1) and the remap."""
    experts = sorted(set(int(e) for e in experts))
    recs = moe.ExpertRecordSet(*(_host_bank(torch, b, experts) for b in dense),
                               shared=None if shared is None else tuple(_host_bank(torch, b, [0]) for b in shared))
    return recs, {e: i for i, e in enumerate(experts)}


@pytest.fixture(scope="module")
def decode_layer_512(torch_mod):
    from flashnext_hip.moe_block import LayerWeights
    from flashnext_hip.synthetic import make_layer

    say("building a 512-expert layer (slot permutation, dense copy kept)")
    lay = make_layer(H, I, E, seed=7100, keep_dense=True)
    w = LayerWeights(lay.layout, lay.pool, lay.slot_table, lay.router_w, lay.shared_gate_w,
                     tuple(b.as_tuple() for b in lay.shared))
    return lay, w


@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 16])  # up to 4: selection folded into gate/up, one token per wave
def test_decode_layer_512_experts_matches_oracle(torch_mod, decode_layer_512, tokens):
    torch = torch_mod
    say(f"case: 512-expert routed decode layer tokens={tokens}")
    from flashnext_hip import _lib
    from flashnext_hip.moe_block import DecodeLayer

    lay, w = decode_layer_512
    dl = DecodeLayer(w, tokens, K)
    x = bf16_normal((tokens, H), seed=7200 + tokens)
    dl.x.copy_(to_dev_bf16(x))
    dl.launch(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0
    wg = from_dev_bf16(lay.router_w)
    wsg = from_dev_bf16(lay.shared_gate_w).reshape(1, -1)
    table = lay.slot_table.cpu().numpy().astype(np.uint32)
    ref = orouter.route(x, wg, K, slot_table=table)
    assert np.array_equal(dl.inds.cpu().numpy().astype(np.uint32), ref["inds"])
    assert np.array_equal(from_dev_bf16(dl.scores), ref["scores"])
    assert np.array_equal(dl.routes.cpu().numpy().view(np.uint32), ref["routes"])
    recs, remap = _records_for(torch, lay.dense, ref["inds"].reshape(-1), shared=lay.shared)
    local = np.vectorize(remap.get)(ref["inds"])
    want = moe.decode_layer(x, local, ref["scores"], recs, score_dtype="bf16", shared_gate_weight=wsg)
    assert_close(bf16.bf16_to_f32(from_dev_bf16(dl.out)), bf16.bf16_to_f32(want), f"decode T={tokens}")


def _zipf_routes(tokens, experts, k, seed, skew=1.1):
    """Per-token top-k distinct experts with Zipf(skew) weights (Gumbel top-k)."""
    rng = np.random.default_rng(seed)
    logp = -skew * np.log(np.arange(1, experts + 1, dtype=np.float64))
    keys = logp[None, :] + rng.gumbel(size=(tokens, experts))
    inds = np.argsort(-keys, axis=1)[:, :k].astype(np.int32)
    raw = rng.random((tokens, k)).astype(np.float32) + 0.05
    scores = bf16.f32_to_bf16((raw / raw.sum(axis=1, keepdims=True)).astype(np.float32))
    return inds, scores


def test_prefill_4096_zipf_512_experts_matches_oracle(torch_mod):
    torch = torch_mod
    say("case: 4096-token Zipf(1.1) prefill over 512 experts")
    from flashnext_hip import _lib
    from flashnext_hip.grouped import GroupedMoE
    from flashnext_hip.synthetic import make_bank

    T = 4096
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7300)
    dense = tuple(make_bank(E, o, i, gen, "cuda", group=G) for (o, i) in ((I, H), (I, H), (H, I)))
    inds, scores = _zipf_routes(T, E, K, seed=7301)
    counts = np.bincount(inds.reshape(-1), minlength=E)
    assert counts.max() > 2000 and counts.min() < 40  # a real Zipf skew: multi-tile heads, one-slab tails
    x = bf16_normal((T, H), seed=7302)
    g = GroupedMoE(*(b.as_tuple() for b in dense), hidden=H, inter=I, group_size=G)
    xd, rd, sd = to_dev_bf16(x), torch.from_numpy(inds).cuda(), to_dev_bf16(scores)
    out, y = g(xd, rd, sd)
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0
    y_bits, out_bits = from_dev_bf16(y), from_dev_bf16(out)

    # segmented == single: four chunks of 1024 tokens, bit for bit
    for c in range(4):
        sl = slice(1024 * c, 1024 * (c + 1))
        oc, yc = g(xd[sl].contiguous(), rd[sl].contiguous(), sd[sl].contiguous())
        assert np.array_equal(from_dev_bf16(yc), y_bits[sl]), f"chunk {c}: per-slot outputs differ"
        assert np.array_equal(from_dev_bf16(oc), out_bits[sl]), f"chunk {c}: combined outputs differ"

    order = np.argsort(counts, kind="stable")
    heavy, light = order[-8:][::-1], order[:8]
    rng = np.random.default_rng(7303)
    sample_tokens = np.sort(rng.choice(T, 256, replace=False))
    experts = set(int(e) for e in heavy) | set(int(e) for e in light) | set(inds[sample_tokens].reshape(-1).tolist())
    recs, remap = _records_for(torch, dense, experts)
    banks = (recs.gate, recs.up, recs.down)
    xf = bf16.bf16_to_f32(x)
    flat = inds.reshape(-1)

    def rows_of(e, rows):
        want = {}
        for mode in ("bf16", "exact"):
            want[mode] = moe.expert_mlp(xf[rows // K], banks, remap[e], "bf16", mode)[3]
        return want

    for e in list(heavy) + list(light):
        rows = np.nonzero(flat == e)[0]
        want = rows_of(int(e), rows)
        got = y_bits.reshape(T * K, H)[rows]
        assert_close(bf16.bf16_to_f32(got), bf16.bf16_to_f32(want["bf16"]), f"expert {e} ({rows.size} rows, tiles)",
                     rtol=REF_RTOL)
        rep = value_report(bf16.bf16_to_f32(got), bf16.bf16_to_f32(want["exact"]))
        assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, (f"expert {e} exact", rep)

    # combined rows of the sampled tokens: every slot's row from the oracle, then the bf16 combine
    y_want = {m: np.zeros((sample_tokens.size, K, H), dtype=np.uint16) for m in ("bf16", "exact")}
    sub = inds[sample_tokens]
    for e in np.unique(sub):
        ti, si = np.nonzero(sub == e)
        rows = sample_tokens[ti] * K + si
        want = rows_of(int(e), rows)
        for m in ("bf16", "exact"):
            y_want[m][ti, si] = want[m]
    for m in ("bf16", "exact"):
        want_out = moe.generic_combine(y_want[m], scores[sample_tokens])
        got_out = bf16.bf16_to_f32(out_bits[sample_tokens])
        if m == "bf16":
            assert_close(got_out, bf16.bf16_to_f32(want_out), "combined rows (tiles)", rtol=REF_RTOL)
        else:
            rep = value_report(got_out, bf16.bf16_to_f32(want_out))
            assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, ("combined rows exact", rep)


@pytest.fixture(scope="module")
def stack48(torch_mod):
    torch = torch_mod
    from flashnext_hip.moe_block import DecodeLayer, LayerWeights
    from flashnext_hip.synthetic import make_layer

    say("building the 48-block stack (512 experts per block, HBM slot pools)")
    layers, resident = [], []
    for l in range(48):
        lay = make_layer(H, I, E, seed=7400 + l, keep_dense=(l == 0))
        w = LayerWeights(lay.layout, lay.pool, lay.slot_table, lay.router_w, lay.shared_gate_w,
                         tuple(b.as_tuple() for b in lay.shared))
        layers.append(lay)
        resident.append(DecodeLayer(w, 1, K))
    torch.cuda.synchronize()
    return layers, resident


def _hot_pool_run(torch, layers, resident, pool_bytes, steps, seed, method="gather"):
    """Decode `steps` tokens through all layers twice: resident, and through an
    LRU hot pool refilled from pinned host records (`method`: the gather kernel
    or one hipMemcpyAsync per record).  Returns the pool and the list of
    (step, layer, resident bits, hot bits)."""
    from flashnext_hip import _lib
    from flashnext_hip.layout import HEADER_SIZE
    from flashnext_hip.moe_block import DecodeLayer, LayerWeights
    from flashnext_hip.pool import HipExpertPool, HostRecordStore

    pool = HipExpertPool(pool_bytes, H, I, G, device="cuda")
    stride = pool.stride
    store = HostRecordStore(pool.layout)
    tables = [lay.slot_table.cpu().tolist() for lay in layers]

    def record(l, e):  # pinned host image of (layer, expert), copied once from its resident pool
        key = (l, e)
        if key not in store._records:
            base = HEADER_SIZE + int(tables[l][e]) * stride
            img = torch.empty(stride, dtype=torch.uint8, pin_memory=True)
            img.copy_(layers[l].pool[base:base + stride])
            store._records[key] = img
        return store._records[key]

    table = torch.zeros(E, dtype=torch.int32, device="cuda")
    hot = []
    for r in resident:
        w = LayerWeights(r.w.layout, pool.buffer, table, r.w.router_w, r.w.shared_gate_w, r.w.shared)
        hot.append(DecodeLayer(w, 1, K))
    stream = torch.cuda.current_stream()
    handle = stream.cuda_stream
    copy_streams = [torch.cuda.Stream() for _ in range(2)]
    rng = np.random.default_rng(seed)
    results = []
    for s in range(steps):
        for l in range(len(layers)):
            x = to_dev_bf16(bf16_normal((1, H), seed=int(rng.integers(1 << 30))))
            resident[l].x.copy_(x)
            resident[l].launch(handle)
            res_bits = from_dev_bf16(resident[l].out)
            dl = hot[l]
            dl.x.copy_(x)
            dl.launch_router(handle)
            inds = dl.inds.cpu()
            experts = sorted(set(inds.reshape(-1).tolist()))
            for e in experts:
                record(l, e)
            slots, misses = pool.assign(l, experts)
            pool.fill(l, misses, store, compute_stream=stream, copy_stream=copy_streams, method=method)
            dl.routes.copy_(HipExpertPool.route_words(slots, inds).to("cuda"))
            dl.launch_experts(handle)
            torch.cuda.synchronize()
            assert np.array_equal(inds.numpy(), resident[l].inds.cpu().numpy()), f"step {s} layer {l}: routes differ"
            results.append((s, l, res_bits, from_dev_bf16(dl.out)))
    assert _lib.check_device_errors(handle) == 0
    return pool, results


def test_stack48_hot_pool_bit_identical_to_resident(torch_mod, stack48):
    torch = torch_mod
    say("case: 48-block stack through a 6 GB hot pool, 2 steps")
    layers, resident = stack48
    pool, results = _hot_pool_run(torch, layers, resident, int(6e9), steps=2, seed=7500)
    assert pool.slots == 3051
    assert 0 < pool.misses <= pool.hits + pool.misses <= 2 * 48 * K
    for s, l, a, b in results:
        assert np.array_equal(a, b), f"step {s} layer {l}: hot-pool output differs from resident"

    # layer 0 of the first step against the oracle
    lay = layers[0]
    x = from_dev_bf16(resident[0].x)  # the last token of layer 0; recompute it through the oracle
    wg = from_dev_bf16(lay.router_w)
    wsg = from_dev_bf16(lay.shared_gate_w).reshape(1, -1)
    ref = orouter.route(x, wg, K)
    recs, remap = _records_for(torch, lay.dense, ref["inds"].reshape(-1), shared=lay.shared)
    want = moe.decode_layer(x, np.vectorize(remap.get)(ref["inds"]), ref["scores"], recs, score_dtype="bf16",
                            shared_gate_weight=wsg)
    assert_close(bf16.bf16_to_f32(from_dev_bf16(resident[0].out)), bf16.bf16_to_f32(want), "stack layer 0")


def test_stack48_small_pool_evictions_bit_identical(torch_mod, stack48):
    torch = torch_mod
    say("case: 48-block stack through a 64-slot pool (evictions every step), one hipMemcpyAsync per record")
    from flashnext_hip.layout import make_layout

    layers, resident = stack48
    stride = make_layout(H, I, G).record_stride
    pool, results = _hot_pool_run(torch, layers, resident, 4096 + 64 * stride, steps=1, seed=7600, method="memcpy")
    assert pool.slots == 64
    assert pool.misses > 64  # the pool wrapped: later layers evicted earlier ones
    for s, l, a, b in results:
        assert np.array_equal(a, b), f"layer {l}: output through the evicting pool differs from resident"
