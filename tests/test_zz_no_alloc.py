"""The allocation-free grouped entry point against the workspace one.

``mq_moe_grouped_static`` runs the grouped path in the library's static
per-device scratch.  Through the C-ABI, two calls in a row (the second with
fewer tokens, so stale scratch contents from the first call must not leak
into it) must give the bits of ``mq_moe_grouped`` with a caller workspace,
for the per-slot outputs and the combined output, with a shared expert run as
an extra group.  A call that needs more than the static maximum is rejected
before anything runs.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from ._helpers import bf16_normal, make_records, say, to_dev_bank, to_dev_bf16

pytestmark = pytest.mark.gpu

H, I, E, K = 2048, 512, 24, 10


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


def _args(torch, banks, shared_projs, x, routes, scores, shared_gate, y, out):
    from flashnext_hip import _lib
    from flashnext_hip.ops import dense_projection

    a = _lib.MqGroupedArgs()
    a.x = x.data_ptr()
    a.gate, a.up, a.down = (dense_projection(*b) for b in banks)
    a.routes, a.scores = routes.data_ptr(), scores.data_ptr()
    a.shared_expert = ctypes.addressof(shared_projs)
    a.shared_gate = shared_gate.data_ptr()
    a.out, a.y = out.data_ptr(), y.data_ptr()
    a.tokens, a.slots, a.hidden, a.inter = x.shape[0], routes.shape[1], H, I
    a.expert_count, a.group_size = E, 32
    return a


def test_static_scratch_matches_workspace_call_twice(torch_mod):
    torch = torch_mod
    from flashnext_hip import _lib
    from flashnext_hip.ops import dense_projection

    lib = _lib.load()
    recs = make_records(E, H, I, seed=8100)
    shared = make_records(1, H, I, seed=8101)
    banks = [to_dev_bank(b) for b in (recs.gate, recs.up, recs.down)]
    sh_banks = [to_dev_bank(b) for b in (shared.gate, shared.up, shared.down)]
    shared_projs = (_lib.MqProjection * 3)(*[dense_projection(*b) for b in sh_banks])
    rng = np.random.default_rng(8102)
    for tokens in (300, 70):  # the second call is smaller: nothing may leak from the first
        say(f"case: static-scratch grouped call tokens={tokens}")
        x = to_dev_bf16(bf16_normal((tokens, H), seed=8103 + tokens))
        inds = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)]).astype(np.int32)
        routes = torch.from_numpy(inds).cuda()
        raw = rng.random((tokens, K)).astype(np.float32) + 0.05
        scores = torch.from_numpy(raw / raw.sum(1, keepdims=True)).cuda().to(torch.bfloat16)
        shared_gate = torch.from_numpy(rng.random(tokens).astype(np.float32)).cuda().to(torch.bfloat16)
        results = []
        for static in (False, True):
            y = torch.full((tokens, K, H), float("nan"), dtype=torch.bfloat16, device="cuda")
            out = torch.full((tokens, H), float("nan"), dtype=torch.bfloat16, device="cuda")
            a = _args(torch, banks, shared_projs, x, routes, scores, shared_gate, y, out)
            if static:
                rc = lib.mq_moe_grouped_static(ctypes.byref(a), None)
            else:
                need = lib.mq_grouped_workspace_size(tokens, K, H, I, E, 1)
                ws = torch.empty(int(need), dtype=torch.uint8, device="cuda")
                a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
                rc = lib.mq_moe_grouped(ctypes.byref(a), None)
            _lib.check(rc, lib)
            torch.cuda.synchronize()
            assert _lib.check_device_errors() == 0
            results.append((y.clone(), out.clone()))
        (y0, o0), (y1, o1) = results
        assert not torch.isnan(o0.float()).any()
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), f"tokens={tokens}: per-slot outputs differ"
        assert torch.equal(o0.view(torch.int16), o1.view(torch.int16)), f"tokens={tokens}: combined outputs differ"


def test_static_scratch_rejects_oversized_call(torch_mod):
    torch = torch_mod
    say("case: static-scratch grouped call above the maximum is rejected")
    from flashnext_hip import _lib
    from flashnext_hip.ops import dense_projection

    lib = _lib.load()
    tokens = 8192  # 81,920 rows: about 84 MB of activations, above the 64 MiB scratch
    need = lib.mq_grouped_workspace_size(tokens, K, H, I, E, 0)
    assert need > (64 << 20)
    recs = make_records(2, H, I, seed=8104)
    banks = [to_dev_bank(b) for b in (recs.gate, recs.up, recs.down)]
    x = torch.zeros((tokens, H), dtype=torch.bfloat16, device="cuda")
    routes = torch.zeros((tokens, K), dtype=torch.int32, device="cuda")
    y = torch.empty((1,), dtype=torch.bfloat16, device="cuda")  # never written: the call fails first
    a = _lib.MqGroupedArgs()
    a.x, a.routes, a.y = x.data_ptr(), routes.data_ptr(), y.data_ptr()
    a.gate, a.up, a.down = (dense_projection(*b) for b in banks)
    a.tokens, a.slots, a.hidden, a.inter, a.expert_count, a.group_size = tokens, K, H, I, E, 32
    rc = lib.mq_moe_grouped_static(ctypes.byref(a), None)
    assert rc == _lib.MQ_ERR_INVALID
    assert "static maximum" in _lib.last_error(lib)
