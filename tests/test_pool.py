"""Expert slot pool: LRU assignment against the reference KAT and the oracle
(CPU), and byte-exact pinned-host refills addressed by the decode kernels
(GPU)."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import pool as opool

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _pool_cpu(slots, hidden=2048, inter=512):
    from flashnext_hip.pool import HEADER_SIZE, HipExpertPool, make_layout

    stride = make_layout(hidden, inter).record_stride
    return HipExpertPool(HEADER_SIZE + slots * stride, hidden, inter, device="cpu")


def test_pool_assign_reference_kat():
    """models/flashnext/tests/unit/test_expert_pool.py:32-49."""
    pool = _pool_cpu(16)
    slots, misses = pool.assign(1, list(range(10)))
    assert len(misses) == 10 and len(set(slots.values())) == 10
    slots2, misses2 = pool.assign(1, [3, 4, 20])
    assert slots2[3] == slots[3] and [e for e, _ in misses2] == [20]
    pool.assign(2, list(range(5)))
    slots3, misses3 = pool.assign(1, [3, 4, 30, 31])
    assert slots3[3] == slots[3] and slots3[4] == slots[4]
    assert {slot for _, slot in misses3} == {slots[0], slots[1]}
    assert pool.hits == 4 and pool.misses == 10 + 1 + 5 + 2


def test_pool_too_small_is_refused():
    with pytest.raises(ValueError):
        _pool_cpu(4)


def test_pool_assign_matches_oracle_on_random_traffic():
    rng = np.random.default_rng(11)
    pool, lru = _pool_cpu(40), opool.LruSlots(40)
    for step in range(300):
        layer = int(rng.integers(0, 6))
        experts = [int(e) for e in rng.choice(64, size=int(rng.integers(1, 12)), replace=False)]
        assert pool.assign(layer, experts) == lru.assign(layer, experts), step
    assert (pool.hits, pool.misses) == (lru.hits, lru.misses)


def test_pool_assign_golden_calls():
    kat = KATS["lru_assign"]
    pool = _pool_cpu(kat["slots"])
    lru = opool.LruSlots(kat["slots"])
    for layer, experts in kat["calls"]:
        assert pool.assign(layer, experts) == lru.assign(layer, experts)


@pytest.mark.gpu
def test_pool_refill_bytes_and_decode_through_slots():
    import torch

    from flashnext_hip import _lib
    from flashnext_hip.hip_runtime import HipMoEExecutor
    from flashnext_hip.pool import HEADER_SIZE, HipExpertPool, HostRecordStore

    from ._helpers import bf16_normal, make_records, say, to_dev_bank, to_dev_bf16

    assert torch.cuda.is_available()
    say("case: pool refill + decode via slot words")
    H, I, E = 1024, 256, 12
    rec = make_records(E, H, I, seed=400)
    banks = {n: to_dev_bank(b) for n, b in (("gate_proj", rec.gate), ("up_proj", rec.up), ("down_proj", rec.down))}
    pool = HipExpertPool(HEADER_SIZE + 16 * _lib.record_layout(H, I)[1], H, I)
    store = HostRecordStore(pool.layout)
    store.add_banks(3, banks)
    copy = torch.cuda.Stream()
    experts = [7, 2, 9, 0, 11]
    slots, misses = pool.assign(3, experts)
    pool.fill(3, misses, store, copy_stream=copy)
    torch.cuda.synchronize()
    for e, slot in misses:
        assert torch.equal(pool.record_bytes(slot).cpu(), store.record(3, e)), (e, slot)
    # decode two tokens through slot words == through dense expert ids
    tokens, k = 2, 4
    x = to_dev_bf16(bf16_normal((tokens, H), seed=401))
    inds = torch.tensor([[7, 2, 9, 0], [11, 9, 7, 2]], dtype=torch.int64)
    scores = torch.full((tokens, k), 0.25, device="cuda")
    ex = HipMoEExecutor(E, H, k, max_tokens=8)
    dense = ex.execute(x, inds.cuda(), banks, scores=scores)
    words = HipExpertPool.route_words(slots, inds).cuda()
    pooled = ex.execute(x, words, banks, scores=scores, slab_pack=pool.buffer)
    assert torch.equal(dense.view(torch.int16), pooled.view(torch.int16))
    # evict and refill: 16 slots, 5 used; 14 new experts of another layer evict the oldest
    store.add_banks(4, banks)
    slots4, misses4 = pool.assign(4, list(range(11)) + [0, 1, 2])
    pool.fill(4, misses4, store, copy_stream=copy)
    torch.cuda.synchronize()
    for e, slot in misses4:
        assert torch.equal(pool.record_bytes(slot).cpu(), store.record(4, e))
    # one hipMemcpyAsync per record, split over two copy streams: the same bytes in the same places
    store.add_banks(5, banks)
    slots5, misses5 = pool.assign(5, [3, 8, 1, 10, 6])
    events = pool.fill(5, misses5, store, copy_stream=[copy, torch.cuda.Stream()], method="memcpy")
    assert isinstance(events, list) and len(events) == 2
    torch.cuda.synchronize()
    for e, slot in misses5:
        assert torch.equal(pool.record_bytes(slot).cpu(), store.record(5, e))
    # the gather kernel (the default): one launch per fill on the first copy stream
    store.add_banks(6, banks)
    slots6, misses6 = pool.assign(6, list(range(12)))
    events = pool.fill(6, misses6, store, copy_stream=[copy, torch.cuda.Stream()])
    assert isinstance(events, list) and len(events) == 1
    torch.cuda.synchronize()
    for e, slot in misses6:
        assert torch.equal(pool.record_bytes(slot).cpu(), store.record(6, e)), (e, slot)
    # 17 records in one call: two launches (16 records per launch), slot 0 written by both, in stream order
    lib = _lib.load()
    import ctypes

    recs = [store.record(6, e % 12) for e in range(17)]
    slots17 = list(range(16)) + [0]
    pool.buffer[HEADER_SIZE:HEADER_SIZE + 16 * pool.stride].zero_()
    n = len(recs)
    _lib.check(lib.mq_pool_refill_gather_async(
        ctypes.c_void_p(pool.buffer.data_ptr()), HEADER_SIZE, pool.stride, pool.slots,
        (ctypes.c_uint32 * n)(*slots17), (ctypes.c_void_p * n)(*[r.data_ptr() for r in recs]), n, pool.stride,
        ctypes.c_void_p(copy.cuda_stream), None), lib)
    torch.cuda.synchronize()
    for i in range(1, 16):
        assert torch.equal(pool.record_bytes(slots17[i]).cpu(), recs[i]), i
    assert torch.equal(pool.record_bytes(0).cpu(), recs[16])
    with pytest.raises(ValueError):  # pageable memory is refused before any launch
        pageable = torch.zeros(pool.stride, dtype=torch.uint8)
        _lib.check(lib.mq_pool_refill_gather_async(
            ctypes.c_void_p(pool.buffer.data_ptr()), HEADER_SIZE, pool.stride, pool.slots,
            (ctypes.c_uint32 * 1)(1), (ctypes.c_void_p * 1)(pageable.data_ptr()), 1, pool.stride,
            ctypes.c_void_p(copy.cuda_stream), None), lib)
    with pytest.raises(ValueError):  # a slot outside the pool is rejected before any copy
        lib = _lib.load()
        import ctypes

        bad = (ctypes.c_uint32 * 1)(pool.slots)
        ptrs = (ctypes.c_void_p * 1)(store.record(4, 0).data_ptr())
        _lib.check(lib.mq_pool_refill_async(ctypes.c_void_p(pool.buffer.data_ptr()), HEADER_SIZE, pool.stride,
                                            pool.slots, bad, ptrs, 1, pool.stride, None, None), lib)
