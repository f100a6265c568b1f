"""GPU parity of ``ops.gather_qmm`` (``mx.gather_qmm``) at the reference's
prefill / verify call shapes.

The reference's prefill pass sorts the flattened (token, slot) rows by expert
and calls ``mx.gather_qmm(x[T*k, 1, H], w, s, b, rhs_indices, transpose=True,
sorted_indices=True)`` once per projection
(``models/flashnext/expert_cache.py:787-810``, ``_issue`` at ``:1790-1806``);
verify batches call it unsorted on ``x[T, 1, 1, H]`` against indices
``[T, k]``.  Here:

* 4096 x 10 = 40,960 sorted rows over 512 experts with Zipf(1.1) counts, at
  the gate shape (2048 -> 512) and the down shape (512 -> 2048): every row of
  the 8 heaviest and 8 lightest experts and 256 random rows against
  ``oracle.q4.gather_qmm`` -- bf16 weight tiles elementwise at the reference's
  rtol 2e-2 / atol 3e-3, exact weights by max rel 1e-2 / cosine 0.9999;
* at the same size, size-independent properties: the unsorted call gives
  each row the bits of the sorted call, and two calls over the halves give
  the bits of one call (``test_prefill_pipeline_math.py:21-54``);
* the verify shape and explicit ``lhs_indices`` (rows read through a row
  map), the per-row GEMV path below 64 rows and for float32 x;
* an expert index outside the bank raises the device flag, its row reads
  zero weights and the other rows are unchanged; a row map entry past the
  end of x (C-ABI) raises MQ_DEVFLAG_BAD_ROW and reads zero inputs.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import bf16, q4

from ._helpers import (MAX_REL, MIN_COSINE, REF_RTOL, assert_close, bf16_normal, from_dev_bf16, make_bank, say,
                       to_dev_bank, to_dev_bf16, value_report)

pytestmark = pytest.mark.gpu

H, I, E, K, G, T = 2048, 512, 512, 10, 32, 4096


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


def _zipf_rows(tokens, experts, k, seed, skew=1.1):
    """Top-k distinct experts per token with Zipf(skew) weights (Gumbel top-k)."""
    rng = np.random.default_rng(seed)
    logp = -skew * np.log(np.arange(1, experts + 1, dtype=np.float64))
    keys = logp[None, :] + rng.gumbel(size=(tokens, experts))
    return np.argsort(-keys, axis=1)[:, :k].astype(np.int64)


def _host_bank(torch, dense, experts):
    sel = torch.tensor(sorted(experts), device=dense.weight.device, dtype=torch.long)
    return q4.ExpertBank(dense.weight[sel].cpu().numpy().view(np.uint32),
                         dense.scales[sel].view(torch.int16).cpu().numpy().view(np.uint16),
                         dense.biases[sel].view(torch.int16).cpu().numpy().view(np.uint16), G)


def _check_rows(torch, dense, x_bits, idx, got_bits, rows, what):
    """Rows `rows` of a gather output against the oracle, one expert at a time
    (each expert's weights are copied to the host only while it is checked)."""
    for e in np.unique(idx[rows]):
        r = rows[idx[rows] == e]
        bank = _host_bank(torch, dense, [int(e)])
        local = np.zeros(r.size, dtype=np.int64)
        want_t = q4.gather_qmm(x_bits[r], bank, local, "bf16")
        want_x = q4.gather_qmm(x_bits[r], bank, local, "exact")
        got = bf16.bf16_to_f32(got_bits[r])
        assert_close(got, bf16.bf16_to_f32(want_t), f"{what}: expert {e} ({r.size} rows, tiles)", rtol=REF_RTOL)
        rep = value_report(got, bf16.bf16_to_f32(want_x))
        assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, (f"{what}: expert {e} exact", rep)


@pytest.fixture(scope="module")
def prefill_case(torch_mod):
    torch = torch_mod
    from flashnext_hip.synthetic import make_bank as dev_bank

    say("building 512-expert gate (2048->512) and down (512->2048) banks")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(8100)
    gate = dev_bank(E, I, H, gen, "cuda", group=G)
    down = dev_bank(E, H, I, gen, "cuda", group=G)
    inds = _zipf_rows(T, E, K, seed=8101)
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")  # mlx-vlm _gather_sort: rows sorted by expert
    counts = np.bincount(flat, minlength=E)
    assert counts.max() > 2000 and counts.min() < 40
    return gate, down, flat, order, counts


@pytest.mark.parametrize("shape", ["gate", "down"])
def test_gather_qmm_sorted_prefill_rows_match_oracle(torch_mod, prefill_case, shape):
    torch = torch_mod
    say(f"case: gather_qmm sorted prefill rows 40960, {shape} shape")
    from flashnext_hip import _lib, ops

    gate, down, flat, order, counts = prefill_case
    dense, k_in, n_out = (gate, H, I) if shape == "gate" else (down, I, H)
    x_tok = bf16_normal((T, k_in), seed=8102)
    xs = x_tok[order // K]                 # x[T*k, 1, K] after the sort
    idx = flat[order]
    xd = to_dev_bf16(xs).reshape(T * K, 1, k_in)
    out = ops.gather_qmm(xd, dense.weight, dense.scales, dense.biases, rhs_indices=torch.from_numpy(idx).cuda(),
                         sorted_indices=True)
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0
    assert tuple(out.shape) == (T * K, 1, n_out)
    got = from_dev_bf16(out).reshape(T * K, n_out)
    by_count = np.argsort(counts, kind="stable")
    heavy, light = by_count[-8:], by_count[:8]
    rows = np.nonzero(np.isin(idx, np.concatenate([heavy, light])))[0]
    rng = np.random.default_rng(8103)
    rows = np.union1d(rows, rng.choice(T * K, 256, replace=False))
    _check_rows(torch, dense, xs, idx, got, rows, f"{shape} sorted prefill")


def test_gather_qmm_row_order_and_segments_bit_identical(torch_mod, prefill_case):
    torch = torch_mod
    say("case: gather_qmm unsorted == sorted, halves == one call (40960 rows)")
    from flashnext_hip import ops

    gate, _, flat, order, _ = prefill_case
    x_tok = bf16_normal((T, H), seed=8104)
    xs = to_dev_bf16(x_tok[order // K]).reshape(T * K, 1, H)
    idx = torch.from_numpy(flat[order]).cuda()
    args = (gate.weight, gate.scales, gate.biases)
    one = from_dev_bf16(ops.gather_qmm(xs, *args, rhs_indices=idx, sorted_indices=True))
    perm = torch.from_numpy(np.random.default_rng(8105).permutation(T * K)).cuda()
    shuffled = from_dev_bf16(ops.gather_qmm(xs[perm].contiguous(), *args, rhs_indices=idx[perm].contiguous()))
    inv = np.argsort(perm.cpu().numpy())
    assert np.array_equal(shuffled[inv], one), "row order changed a row's bits"
    half = T * K // 2
    a = from_dev_bf16(ops.gather_qmm(xs[:half].contiguous(), *args, rhs_indices=idx[:half].contiguous()))
    b = from_dev_bf16(ops.gather_qmm(xs[half:].contiguous(), *args, rhs_indices=idx[half:].contiguous()))
    assert np.array_equal(np.concatenate([a, b]), one), "segmented calls differ from one call"


def test_gather_qmm_verify_shape_and_lhs_indices(torch_mod):
    torch = torch_mod
    say("case: gather_qmm verify x[16,1,1,H] x indices[16,10]; explicit lhs_indices")
    from flashnext_hip import _lib, ops

    bank = make_bank(24, 256, 512, seed=8200)
    dev = to_dev_bank(bank)
    # verify: 160 rows through the grouped GEMM, x rows read through the row map
    x = bf16_normal((16, 512), seed=8201)
    idx = np.random.default_rng(8202).integers(0, 24, (16, 10))
    out = ops.gather_qmm(to_dev_bf16(x).reshape(16, 1, 1, 512), *dev, rhs_indices=torch.from_numpy(idx).cuda())
    assert tuple(out.shape) == (16, 10, 1, 256)
    got = from_dev_bf16(out).reshape(160, 256)
    xr = np.repeat(x, 10, axis=0)
    assert_close(bf16.bf16_to_f32(got), bf16.bf16_to_f32(q4.gather_qmm(xr, bank, idx.reshape(-1), "bf16")),
                 "verify shape (tiles)")
    # lhs_indices: x [4, 8, K] batches picked per output batch, 12 x 8 = 96 rows
    xb = bf16_normal((4, 8, 512), seed=8203)
    lhs = np.random.default_rng(8204).integers(0, 4, 12)
    rhs = np.random.default_rng(8205).integers(0, 24, 12)
    out = ops.gather_qmm(to_dev_bf16(xb), *dev, lhs_indices=torch.from_numpy(lhs).cuda(),
                         rhs_indices=torch.from_numpy(rhs).cuda())
    assert tuple(out.shape) == (12, 8, 256)
    want = q4.gather_qmm(xb[lhs].reshape(96, 512), bank, np.repeat(rhs, 8), "bf16")
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out).reshape(96, 256)), bf16.bf16_to_f32(want), "lhs_indices")
    # default indices: x [24, 3, K] against every expert
    xe = bf16_normal((24, 3, 512), seed=8206)
    out = ops.gather_qmm(to_dev_bf16(xe), *dev)
    want = q4.gather_qmm(xe.reshape(72, 512), bank, np.repeat(np.arange(24), 3), "bf16")
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out).reshape(72, 256)), bf16.bf16_to_f32(want), "default indices")
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0


def test_gather_qmm_gemv_rows_and_float32(torch_mod):
    torch = torch_mod
    say("case: gather_qmm GEMV path: 40 bf16 rows with a row map, 128 float32 rows")
    from flashnext_hip import _lib, ops

    bank = make_bank(8, 128, 256, seed=8300)
    dev = to_dev_bank(bank)
    xb = bf16_normal((5, 8, 256), seed=8301)
    lhs = np.array([4, 0, 2, 2, 1])
    rhs = np.array([7, 3, 3, 0, 5])
    out = ops.gather_qmm(to_dev_bf16(xb), *dev, lhs_indices=torch.from_numpy(lhs).cuda(),
                         rhs_indices=torch.from_numpy(rhs).cuda())
    want = q4.gather_qmm(xb[lhs].reshape(40, 256), bank, np.repeat(rhs, 8))
    assert_close(bf16.bf16_to_f32(from_dev_bf16(out).reshape(40, 128)), bf16.bf16_to_f32(want), "bf16 GEMV rows")
    rng = np.random.default_rng(8302)
    xf = (rng.normal(0, 1, (128, 256)) / 16).astype(np.float32)
    idx = rng.integers(0, 8, 128)
    out = ops.gather_qmm(torch.from_numpy(xf).cuda().reshape(128, 1, 256), *dev, rhs_indices=torch.from_numpy(idx).cuda())
    want = np.stack([q4.qmv_f64(xf[r:r + 1].astype(np.float64), bank.packed[idx[r]], bank.scales[idx[r]],
                                bank.biases[idx[r]])[0] for r in range(128)])
    assert_close(out.reshape(128, 128).cpu().numpy(), want, "float32 rows", rtol=1e-3, atol=1e-4)
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0


@pytest.mark.parametrize("rows", [96, 16], ids=["grouped", "gemv"])
def test_gather_qmm_bad_expert_raises_flag(torch_mod, rows):
    torch = torch_mod
    say(f"case: gather_qmm expert index outside the bank, {rows} rows")
    from flashnext_hip import _lib, ops

    bank = make_bank(6, 128, 256, seed=8400)
    dev = to_dev_bank(bank)
    x = bf16_normal((rows, 256), seed=8401)
    idx = np.random.default_rng(8402).integers(0, 6, rows)
    idx[5] = 6  # one past the bank
    out = ops.gather_qmm(to_dev_bf16(x).reshape(rows, 1, 256), *dev, rhs_indices=torch.from_numpy(idx).cuda())
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="route word"):
        _lib.check_device_errors()
    assert _lib.check_device_errors() == 0  # reading the flags cleared them
    got = from_dev_bf16(out).reshape(rows, 128)
    assert np.all(bf16.bf16_to_f32(got[5]) == 0.0)
    ok = np.arange(rows) != 5
    want = q4.gather_qmm(x[ok], bank, idx[ok], "bf16" if rows >= 64 else "exact")
    assert_close(bf16.bf16_to_f32(got[ok]), bf16.bf16_to_f32(want), "rows beside the bad one")


def test_gather_qmm_c_abi_row_map_bounds(torch_mod):
    torch = torch_mod
    say("case: mq_gather_qmm row map entry past x raises MQ_DEVFLAG_BAD_ROW")
    from flashnext_hip import _lib
    from flashnext_hip.ops import dense_projection

    lib = _lib.load()
    bank = make_bank(4, 128, 256, seed=8500)
    w, s, b = to_dev_bank(bank)
    x = bf16_normal((10, 256), seed=8501)
    xd = to_dev_bf16(x)
    rows = 80
    xr = np.random.default_rng(8502).integers(0, 10, rows).astype(np.int32)
    xr[7] = 10  # one past x
    routes = np.random.default_rng(8503).integers(0, 4, rows).astype(np.int32)
    xr_d, routes_d = torch.from_numpy(xr).cuda(), torch.from_numpy(routes).cuda()
    out = torch.full((rows, 128), 1.0, dtype=torch.bfloat16, device="cuda")
    a = _lib.MqGatherArgs()
    a.x, a.x_rows, a.routes, a.out = xd.data_ptr(), xr_d.data_ptr(), routes_d.data_ptr(), out.data_ptr()
    a.w = dense_projection(w, s, b)
    a.x_count, a.rows, a.in_width, a.out_width, a.expert_count, a.group_size = 10, rows, 256, 128, 4, 32
    ws_bytes = int(lib.mq_gather_qmm_workspace_size(rows, 4))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes - 1
    assert lib.mq_gather_qmm(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID  # workspace one byte short
    a.workspace_bytes = ws_bytes
    _lib.check(lib.mq_gather_qmm(ctypes.byref(a), None), lib)
    flags = ctypes.c_uint32(0)
    assert lib.mq_check_device_errors(None, ctypes.byref(flags)) == _lib.MQ_ERR_INVALID
    assert flags.value == _lib.MQ_DEVFLAG_BAD_ROW
    got = from_dev_bf16(out)
    assert np.all(bf16.bf16_to_f32(got[7]) == 0.0)
    ok = np.arange(rows) != 7
    want = q4.gather_qmm(x[xr[ok]], bank, routes[ok], "bf16")
    assert_close(bf16.bf16_to_f32(got[ok]), bf16.bf16_to_f32(want), "rows beside the bad one")
