"""C-ABI surface checks that need no GPU: load, exports, layout, error paths."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from flashnext_hip import _lib, layout
from oracle import pool

HEADER = Path(__file__).resolve().parent.parent / "include" / "mqmoe.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|uint64_t)\s+(mq_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert names, "header parse found no declarations"
    for name in names:
        assert hasattr(lib, name), f"{name} missing from libmqmoe.so"
    assert set(names) == set(_lib.EXPORTS)


def test_version_and_last_error_round_trip():
    lib = _lib.load()
    assert lib.mq_version() >= 100
    # Invalid arguments are rejected before any device call.
    assert lib.mq_route_topk(None, None) == _lib.MQ_ERR_INVALID
    assert "NULL" in _lib.last_error(lib)
    assert lib.mq_moe_decode(None, None) == _lib.MQ_ERR_INVALID
    buf = ctypes.create_string_buffer(4)
    assert lib.mq_last_error(buf, 4) == 0 and len(buf.value) <= 3


@pytest.mark.parametrize("hidden,inter,group", [(2560, 640, 32), (2560, 640, 64), (2048, 512, 32),
                                                (1024, 256, 64), (4096, 1536, 32)])
def test_record_layout_c_python_oracle_agree(hidden, inter, group):
    offs_c, stride_c = _lib.record_layout(hidden, inter, group)
    lay = layout.make_layout(hidden, inter, group)
    offs_o, stride_o, _ = pool.record_layout(hidden, inter, group)
    keys = [f"{p}.{q}" for p, q in layout.PART_KEYS]
    assert stride_c == lay.record_stride == stride_o
    assert offs_c == [lay.offset(*k) for k in layout.PART_KEYS] == [offs_o[k] for k in keys]


def test_record_layout_rejects_bad_shapes():
    with pytest.raises(ValueError):
        _lib.record_layout(2048, 500, 32)
    with pytest.raises(ValueError):
        _lib.record_layout(2048, 512, 16)


def test_validation_errors_without_device():
    lib = _lib.load()
    args = _lib.MqRouteArgs()
    args.tokens, args.experts, args.top_k = 1, 512, 11
    assert lib.mq_route_topk(args, None) == _lib.MQ_ERR_INVALID  # no outputs
    args.experts, args.top_k = 600, 10
    assert lib.mq_route_topk(args, None) == _lib.MQ_ERR_INVALID
    assert "experts" in _lib.last_error(lib)
    assert lib.mq_q4_dequant(None, None, None, None, 1, 32, 32, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_q4_unpack(None, None, 0, None) == _lib.MQ_OK  # empty is a no-op
    # mq_swiglu checks pointers and flags before any launch (the pointers are never read here).
    dummy = ctypes.c_void_p(16)
    both = _lib.MQ_SWIGLU_SCALAR | _lib.MQ_SWIGLU_TABLE
    assert lib.mq_swiglu(dummy, dummy, dummy, 4, _lib.MQ_BF16, both, None) == _lib.MQ_ERR_INVALID
    assert "exclude" in _lib.last_error(lib)
    assert lib.mq_swiglu(dummy, dummy, dummy, 4, _lib.MQ_BF16, 4, None) == _lib.MQ_ERR_INVALID
    assert "flags" in _lib.last_error(lib)
    # the gather refill checks its arguments before any HIP call
    slots = (ctypes.c_uint32 * 1)(0)
    recs = (ctypes.c_void_p * 1)(16)
    assert lib.mq_pool_refill_gather_async(None, 4096, 1 << 20, 4, slots, recs, 1, 1 << 20, None, None) \
        == _lib.MQ_ERR_INVALID
    assert lib.mq_pool_refill_gather_async(dummy, 4096, 1 << 20, 4, slots, recs, 1, 1000, None, None) \
        == _lib.MQ_ERR_INVALID
    assert "16-byte" in _lib.last_error(lib)
    recs[0] = 24  # unaligned record
    assert lib.mq_pool_refill_gather_async(dummy, 4096, 1 << 20, 4, slots, recs, 1, 1 << 20, None, None) \
        == _lib.MQ_ERR_INVALID
    assert "aligned" in _lib.last_error(lib)
    recs[0] = 32
    slots[0] = 4  # outside the pool
    assert lib.mq_pool_refill_gather_async(dummy, 4096, 1 << 20, 4, slots, recs, 1, 1 << 20, None, None) \
        == _lib.MQ_ERR_INVALID
    assert "outside" in _lib.last_error(lib)
    # the latency probes check their arguments before any launch
    assert lib.mq_stream_probe(None, 11, 1 << 20, 704, dummy, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_stream_probe(dummy, 11, 1000, 704, dummy, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_stream_probe(dummy, 11, 1 << 20, 700, dummy, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_hop_probe(dummy, 0, dummy, 0, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_hop_probe(dummy, 9, dummy, 0, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_hop_probe(None, 4, dummy, 0, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_hop_probe(dummy, 4, dummy, 64, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_mfma_probe(100, 256, None, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_mfma_probe(0, 256, dummy, None) == _lib.MQ_ERR_INVALID
    assert lib.mq_mfma_probe(100, 0, dummy, None) == _lib.MQ_ERR_INVALID


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.NativeUnavailable):
        _lib.load(tmp_path / "missing.so")
