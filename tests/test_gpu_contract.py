"""GPU bit contract of the bf16 SwiGLU, sigmoid and rounding sequences.

The reference requires the SwiGLU epilogue to equal the bf16 sequence for
every one of the 65,536 bf16 gates at up = 0x3F9E and 0x3F80, and on its
representative bits (``models/flashnext/tests/unit/test_swiglu_contract.py:21-31, 37-83``).
Here the device sequences the kernels run -- per element (decode epilogue),
four at a time, four at a time with the sigmoid from the per-block table
(grouped gate/up epilogue), and the sigmoid alone (shared-expert gate) -- are
compared bit for bit with ``oracle.moe.swiglu`` / ``sigmoid_t`` over
every gate pattern at those ups and a few more.  NaN outputs must be NaN (the
sign and payload of a NaN are not fixed by IEEE arithmetic and are not
compared).  The one-instruction bf16 rounding is checked against integer
round-to-nearest-even over all 2^32 float32 patterns.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import bf16, moe

from ._helpers import bf16_normal, from_dev_bf16, say, to_dev_bf16

pytestmark = pytest.mark.gpu

ALL_GATES = np.arange(65536, dtype=np.uint32).astype(np.uint16)
UPS = (0x3F9E, 0x3F80, 0x3FA0, 0x3F00, 0x4020, 0xC000, 0x0000, 0x7F80)


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


def _assert_bits(got, want, what):
    got = np.asarray(got, dtype=np.uint16)
    want = np.asarray(want, dtype=np.uint16)
    nan_want = np.isnan(bf16.bf16_to_f32(want))
    nan_got = np.isnan(bf16.bf16_to_f32(got))
    assert np.array_equal(nan_got, nan_want), f"{what}: NaN positions differ"
    bad = np.flatnonzero((got != want) & ~nan_want)
    assert bad.size == 0, (f"{what}: {bad.size} mismatches, first gates "
                           f"{[hex(int(ALL_GATES[i % 65536])) for i in bad[:6]]} "
                           f"got {[hex(int(got[i])) for i in bad[:6]]} want {[hex(int(want[i])) for i in bad[:6]]}")


@pytest.mark.parametrize("seq", ["runs", "scalar", "table"], ids=["four-at-a-time", "per-element", "table"])
def test_swiglu_all_gates_bit_exact(torch_mod, seq):
    say(f"case: swiglu all 65536 gates x {len(UPS)} ups sequence={seq}")
    from flashnext_hip import ops

    gates = np.tile(ALL_GATES, len(UPS))
    ups = np.repeat(np.array(UPS, dtype=np.uint16), 65536)
    got = from_dev_bf16(ops.swiglu(to_dev_bf16(gates), to_dev_bf16(ups), scalar=seq == "scalar",
                                   table=seq == "table"))
    _assert_bits(got, moe.swiglu(gates, ups), f"swiglu sequence={seq}")


def test_swiglu_reference_representative_bits(torch_mod):
    say("case: swiglu representative bits")
    from flashnext_hip import ops

    g = np.array([0x0000, 0x3F80, 0xBF80, 0x4120, 0xC120], dtype=np.uint16)
    u = np.array([0x3F80, 0x3FA0, 0x3F00, 0x4020, 0xC000], dtype=np.uint16)
    for scalar, table in ((False, False), (True, False), (False, True)):
        # a 5-element call covers one run of four plus a one-element tail
        got = from_dev_bf16(ops.swiglu(to_dev_bf16(g), to_dev_bf16(u), scalar=scalar, table=table))
        assert got.tolist() == moe.swiglu(g, u).tolist()


def test_sigmoid_all_patterns_bit_exact(torch_mod):
    say("case: sigmoid all 65536 patterns")
    from flashnext_hip import ops

    got = from_dev_bf16(ops.sigmoid(to_dev_bf16(ALL_GATES)))
    want = bf16.f32_to_bf16(moe.sigmoid_t(bf16.bf16_to_f32(ALL_GATES), "bf16"))
    _assert_bits(got, want, "sigmoid")


def test_swiglu_float32_sequence(torch_mod):
    torch = torch_mod
    say("case: swiglu float32")
    from flashnext_hip import ops

    rng = np.random.default_rng(3)
    g = (rng.normal(0, 4, 4096)).astype(np.float32)
    u = (rng.normal(0, 1, 4096)).astype(np.float32)
    got = ops.swiglu(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), moe.swiglu(g, u, "f32").view(np.uint32))


def test_bf16_rounding_all_float32_patterns(torch_mod):
    torch = torch_mod
    say("case: bf16 rounding over all 2^32 float32 patterns")
    from flashnext_hip import _lib

    lib = _lib.load()
    counts = torch.zeros(2, dtype=torch.int64, device="cuda")
    step = 1 << 30
    for first in range(0, 1 << 32, step):
        _lib.check(lib.mq_bf16_round_check(first, step, ctypes.c_void_p(counts.data_ptr()), None), lib)
    torch.cuda.synchronize()
    assert counts.cpu().tolist() == [0, 0]


def test_decode_return_all_act_bits_equal_swiglu_of_outputs(torch_mod):
    torch = torch_mod
    say("case: return_all act == swiglu(gate_out, up_out)")
    from flashnext_hip import _lib
    from flashnext_hip.ops import dense_projection

    from ._helpers import make_records, to_dev_bank

    H, I, E, T, K = 2048, 512, 8, 3, 6
    recs = make_records(E, H, I, seed=900)
    banks = [to_dev_bank(b) for b in (recs.gate, recs.up, recs.down)]
    x = to_dev_bf16(bf16_normal((T, H), seed=901))
    routes = torch.from_numpy(np.random.default_rng(902).integers(0, E, (T, K)).astype(np.int32)).cuda()
    g = torch.empty((T, K, I), dtype=torch.bfloat16, device="cuda")
    u, act = torch.empty_like(g), torch.empty_like(g)
    d = torch.empty((T, K, H), dtype=torch.bfloat16, device="cuda")
    a = _lib.MqMoeArgs()
    a.x, a.x_dtype = x.data_ptr(), _lib.MQ_BF16
    a.gate, a.up, a.down = (dense_projection(*b) for b in banks)
    a.routes = routes.data_ptr()
    a.gate_out, a.up_out, a.act_out, a.down_out = g.data_ptr(), u.data_ptr(), act.data_ptr(), d.data_ptr()
    a.tokens, a.slots, a.hidden, a.inter, a.expert_count, a.group_size = T, K, H, I, E, 32
    a.flags = _lib.MQ_DECODE_RETURN_ALL
    lib = _lib.load()
    _lib.check(lib.mq_moe_decode(ctypes.byref(a), None), lib)
    torch.cuda.synchronize()
    _assert_bits(from_dev_bf16(act).reshape(-1), moe.swiglu(from_dev_bf16(g).reshape(-1), from_dev_bf16(u).reshape(-1)),
                 "fused act vs swiglu(gate_out, up_out)")
