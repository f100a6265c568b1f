"""Pin the CPU oracle: reference known-answer tests, closed forms, brute force.

Every oracle function used as a parity checker is exercised here against
values fixed independently of its own formula (see ``oracle.PINNING``).
"""
from __future__ import annotations

import json
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import bf16, moe, pool, q4, router

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


# ---------------------------------------------------------------- bf16
def test_f32_to_bf16_rounding_cases():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -0.0, np.inf, -np.inf, 3.4e38,
                     1.0 + 2 ** -8 + 2 ** -20], dtype=np.float32)
    expected = [0x3F80, 0x3F80, 0x3F82, 0x8000, 0x7F80, 0xFF80, 0x7F80, 0x3F81]
    assert bf16.f32_to_bf16(vals).tolist() == expected
    assert int(bf16.f32_to_bf16(np.float32(np.nan))) == 0x7FC0


def _exact_bf16(value: float) -> int:
    """Brute force: nearest-even bf16 of an exact rational (finite, normal range)."""
    f = Fraction(value)
    if f == 0:
        return 0x8000 if np.signbit(value) else 0
    sign = 0x8000 if f < 0 else 0
    f = abs(f)
    best = None
    # candidate bf16 values around the float32 neighbourhood
    approx = np.float32(float(f))
    base = int(bf16.f32_to_bf16(approx)) & 0x7FFF
    cands = [c for c in range(max(0, base - 2), min(0x7F7F, base + 2) + 1)]
    for c in cands:
        v = Fraction(float(bf16.bf16_to_f32(np.uint16(c))))
        d = abs(v - f)
        if best is None or d < best[0] or (d == best[0] and (c & 1) == 0):
            best = (d, c)
    return sign | best[1]


def test_f64_to_bf16_matches_exact_rational_rounding():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.normal(0, 1, 2000) * 10.0 ** rng.integers(-20, 20, 2000),
        # exact bf16 midpoints nudged by one float64 ulp either way (double-rounding traps)
        np.array([1.0 + 2 ** -8 + 2 ** -40, 1.0 + 2 ** -8 - 2 ** -40, 1.0 + 3 * 2 ** -8 - 2 ** -45]),
    ])
    got = bf16.f64_to_bf16(vals)
    want = np.array([_exact_bf16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)
    # single rounding: f32-then-bf16 would get the first trap wrong
    assert int(bf16.f64_to_bf16(np.float64(1.0 + 2 ** -8 + 2 ** -40))) == 0x3F81


# ---------------------------------------------------------------- q4
def test_pack_order_matches_reference_packer():
    q = np.arange(8, dtype=np.uint8)[None, :]
    assert q4.pack_q4(q).tolist() == [[0x76543210]]
    rng = np.random.default_rng(0)
    vals = rng.integers(0, 16, (3, 5, 64), dtype=np.uint8)
    # reference loop: packed[..., k // 8] |= (v & 15) << ((k & 7) * 4)
    ref = np.zeros((3, 5, 8), dtype=np.uint32)
    for k in range(64):
        ref[:, :, k // 8] |= (vals[:, :, k].astype(np.uint32) & 15) << ((k & 7) * 4)
    assert np.array_equal(q4.pack_q4(vals), ref)
    assert np.array_equal(q4.unpack_q4(ref), vals)


def test_qmv_integer_closed_form():
    rng = np.random.default_rng(3)
    k, n = 256, 7
    q = rng.integers(0, 16, (n, k), dtype=np.uint8)
    packed = q4.pack_q4(q)
    ones = np.full((n, k // 32), 0x3F80, dtype=np.uint16)
    zeros = np.zeros((n, k // 32), dtype=np.uint16)
    x = rng.integers(-8, 8, (2, k)).astype(np.float64)
    got = q4.qmv_f64(x, packed, ones, zeros)
    assert np.array_equal(got, x @ q.T.astype(np.float64))


def test_gather_qmm_integer_closed_form_and_row_order():
    """gather_qmm row r = bf16(x_r . W_{e_r}) with each row's own expert: with
    scales 1 and biases 0 the products are integer dots, exact in bf16 when
    small; every expert's rows differ (distinct weights), so a row sent to
    the wrong expert or a transposed operand fails; permuting the rows
    permutes the outputs; both weight modes agree on bf16-exact weights."""
    rng = np.random.default_rng(6)
    experts, n, k = 5, 6, 64
    q = rng.integers(0, 16, (experts, n, k), dtype=np.uint8)
    packed = q4.pack_q4(q)
    ones = np.full((experts, n, k // 32), 0x3F80, dtype=np.uint16)
    zeros = np.zeros((experts, n, k // 32), dtype=np.uint16)
    bank = q4.ExpertBank(packed, ones, zeros, 32)
    # x in [-2, 2] on the first 8 inputs, 0 elsewhere: |dot| <= 2*15*8 = 240 < 256,
    # so every integer result is exact in bf16's 8-bit significand
    x = np.zeros((23, k), dtype=np.float32)
    x[:, :8] = rng.integers(-2, 3, (23, 8))
    idx = rng.integers(0, experts, 23)
    got = bf16.bf16_to_f32(q4.gather_qmm(bf16.f32_to_bf16(x), bank, idx)).astype(np.float64)
    want = np.stack([x[r].astype(np.float64) @ q[idx[r]].T.astype(np.float64) for r in range(23)])
    assert np.array_equal(got, want)
    perm = rng.permutation(23)
    got_p = q4.gather_qmm(bf16.f32_to_bf16(x[perm]), bank, idx[perm])
    assert np.array_equal(got_p, q4.gather_qmm(bf16.f32_to_bf16(x), bank, idx)[perm])
    assert np.array_equal(q4.gather_qmm(bf16.f32_to_bf16(x), bank, idx, "bf16"),
                          q4.gather_qmm(bf16.f32_to_bf16(x), bank, idx))


def test_qmv_affine_linearity_and_group64():
    rng = np.random.default_rng(4)
    k, n = 128, 5
    q = rng.integers(0, 16, (n, k), dtype=np.uint8)
    packed = q4.pack_q4(q)
    for group in (32, 64):
        s = bf16.f32_to_bf16(rng.uniform(0.01, 0.1, (n, k // group)).astype(np.float32))
        b = bf16.f32_to_bf16(rng.uniform(-0.1, 0.1, (n, k // group)).astype(np.float32))
        x = rng.normal(0, 1, (3, k))
        got = q4.qmv_f64(x, packed, s, b, group)
        sf = bf16.bf16_to_f32(s).astype(np.float64)
        bfv = bf16.bf16_to_f32(b).astype(np.float64)
        want = np.zeros((3, n))
        for g in range(k // group):
            sl = slice(g * group, (g + 1) * group)
            want += sf[:, g] * (x[:, sl] @ q[:, sl].T) + bfv[:, g] * x[:, sl].sum(axis=1, keepdims=True)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_dequant_bf16_single_rounding():
    packed = q4.pack_q4(np.array([[15, 0, 1, 2, 3, 4, 5, 6] * 4], dtype=np.uint8))
    s = np.array([[0x3F80]], dtype=np.uint16)  # 1.0
    b = np.array([[0x3F00]], dtype=np.uint16)  # 0.5
    out = bf16.bf16_to_f32(q4.dequantize_bf16(packed, s, b))
    assert out[0, :8].tolist() == [15.5, 0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5]


# ---------------------------------------------------------------- router
def test_softmax_uniform_and_topk_ties():
    logits = np.zeros((2, 512), dtype=np.uint16)  # all 0.0
    gates = router.softmax_precise(logits)
    assert np.all(gates == 0x3B00)  # 1/512 = 2^-9
    inds, scores = router.topk(gates, 10)
    assert inds.tolist() == [list(range(10))] * 2  # ties -> lowest indices first
    assert router.kth_tie(gates, 10).all()


def test_topk_matches_brute_force_sort():
    rng = np.random.default_rng(5)
    gates = bf16.f32_to_bf16(rng.uniform(0, 1, (50, 64)).astype(np.float32) ** 4)
    inds, scores = router.topk(gates, 6)
    for r in range(50):
        order = sorted(range(64), key=lambda e: (-int(gates[r, e]), e))[:6]
        assert inds[r].tolist() == order
        assert scores[r].tolist() == [int(gates[r, e]) for e in order]


def test_softmax_closed_form_two_values():
    # logits (0, ln 3) -> gates (1/4, 3/4); ln 3 is not bf16-exact, so use its bf16 value
    l1 = float(bf16.bf16_to_f32(bf16.f32_to_bf16(np.float32(np.log(3.0)))))
    logits = bf16.f32_to_bf16(np.array([[0.0, l1]], dtype=np.float32))
    e1 = np.exp(l1)
    want = bf16.f64_to_bf16(np.array([1 / (1 + e1), e1 / (1 + e1)]))
    assert np.array_equal(router.softmax_precise(logits)[0], want)


def test_renorm_bf16_arithmetic():
    s = bf16.f32_to_bf16(np.array([[0.25, 0.25]], dtype=np.float32))
    mass = router.bf16_sum(s)
    out, norm = router.renorm(s, mass)
    assert bf16.bf16_to_f32(out).tolist() == [[0.5, 0.5]]
    # three thirds: 1/3 in bf16 is 0.333984375; mass = bf16(1.001953125) = 1.0
    third = bf16.f32_to_bf16(np.full((1, 3), 1 / 3, dtype=np.float32))
    assert bf16.bf16_to_f32(third)[0, 0] == 0.333984375
    out, norm = router.renorm(third, router.bf16_sum(third))
    assert bf16.bf16_to_f32(norm).tolist() == [[1.0]]
    assert bf16.bf16_to_f32(out).tolist() == [[0.333984375] * 3]


def test_keep_for_mass_and_padding():
    assert router.keep_for_mass([0.5, 0.3, 0.2], 0.85) == 3
    assert router.keep_for_mass([0.5, 0.3, 0.2], 0.75) == 2
    assert router.keep_for_mass([0.9, 0.05, 0.05], 0.85) == 1
    inds = np.array([[7, 3, 9]], dtype=np.uint32)
    scores = bf16.f32_to_bf16(np.array([[0.5, 0.3, 0.2]], dtype=np.float32))
    keeps = router.adaptive_keep(scores, 0.75, min_keep=1)
    assert keeps.tolist() == [2]
    p_inds, p_scores, width = router.pad_dropped(inds, scores, keeps)
    assert p_inds.tolist() == [[7, 3, 7]] and p_scores[0, 2] == 0 and width == 2
    assert router.adaptive_keep(scores, 0.3, min_keep=2).tolist() == [2]


def test_slot_word_encoding_kat():
    kat = KATS["route_encoding"]
    table = np.arange(16, dtype=np.uint32)
    word = router.slot_words(np.array([[kat["slot"]]]), table)[0, 0]
    assert int(word) == kat["word"]
    assert int(word) & 0x80000000 and (int(word) & 0x7FFFFFFF) == kat["slot"]
    assert int(router.slot_words(np.array([[kat["streamed"]]]))[0, 0]) == kat["streamed"]


# ---------------------------------------------------------------- SwiGLU / combine
def test_swiglu_representative_bits_hand_computed():
    kat = KATS["swiglu_representative"]
    g = np.array(kat["gate_bits"], dtype=np.uint16)
    u = np.array(kat["up_bits"], dtype=np.uint16)
    assert moe.swiglu(g, u).tolist() == kat["expected_bits"]


def test_swiglu_fp32_candidate_differs_on_exhaustive_scan():
    # reference contract: the float32 epilogue is NOT the bf16 sequence
    # (tests/unit/test_swiglu_contract.py:33-45).
    gates = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(bf16.bf16_to_f32(gates))
    gates = gates[finite]
    for up_bits in (0x3F9E, 0x3F80):
        up = np.full(gates.shape, up_bits, dtype=np.uint16)
        a = moe.swiglu(gates, up)
        b = moe.swiglu_fp32(gates, up)
        assert np.count_nonzero(a != b) > 0


def test_swiglu_limits():
    big = bf16.f32_to_bf16(np.array([100.0, -100.0, 1e-30], dtype=np.float32))
    one = np.full(3, 0x3F80, dtype=np.uint16)
    out = bf16.bf16_to_f32(moe.swiglu(big, one))
    assert out[0] == 100.0            # sigmoid saturates to 1
    assert out[1] == 0.0              # and to 0 for large negative gates
    assert out[2] == bf16.bf16_to_f32(bf16.f32_to_bf16(np.float32(0.5e-30)))


def test_weighted_combine_reference_kat():
    kat = KATS["weighted_combine"]
    out = moe.weighted_combine(np.array(kat["expert_outputs"], dtype=np.float32),
                               np.array(kat["routes"]), np.array(kat["scores"], dtype=np.float32))
    assert out.tolist() == kat["expected"]
    with pytest.raises(ValueError):
        moe.weighted_combine(np.zeros((2, 3, 2)), np.array([[0, 3]]), np.ones((1, 2)))


def test_down_combine_closed_form_and_shared_epilogues():
    d = bf16.f32_to_bf16(np.array([[[1.0, -2.0], [4.0, 8.0]]], dtype=np.float32))  # [T=1,K=2,H=2]
    scores = np.array([[0.25, 0.5]], dtype=np.float32)
    out = bf16.bf16_to_f32(moe.down_combine(d, scores))
    assert out.tolist() == [[2.25, 3.5]]
    sy = bf16.f32_to_bf16(np.array([[0.75, -0.5]], dtype=np.float32))
    assert bf16.bf16_to_f32(moe.down_combine(d, scores, shared_y=sy)).tolist() == [[3.0, 3.0]]
    sh = bf16.f32_to_bf16(np.array([[3.0, 3.0]], dtype=np.float32))
    gate = bf16.f32_to_bf16(np.array([KATS["shared_gate_value"]], dtype=np.float32))
    got = bf16.bf16_to_f32(moe.down_combine(d, scores, shared=sh, shared_gate=gate))
    comp = float(bf16.bf16_to_f32(bf16.f32_to_bf16(np.float32(3.0 * 0.333984375))))
    want = [float(bf16.bf16_to_f32(bf16.f32_to_bf16(np.float32(2.25 + comp)))),
            float(bf16.bf16_to_f32(bf16.f32_to_bf16(np.float32(3.5 + comp))))]
    assert got.tolist() == [want]
    # keeps: a padded slot is skipped (equal to a zero score)
    assert bf16.bf16_to_f32(moe.down_combine(d, scores, keeps=[1])).tolist() == [[0.25, -0.5]]


def test_generic_combine_bf16_order():
    y = bf16.f32_to_bf16(np.array([[[1.0, 2.0], [3.0, 4.0]]], dtype=np.float32))
    s = bf16.f32_to_bf16(np.array([[0.5, 0.25]], dtype=np.float32))
    assert bf16.bf16_to_f32(moe.generic_combine(y, s)).tolist() == [[1.25, 2.0]]


def test_generic_decode_combine_rounds_each_product():
    # Group 64 keeps weighted_combine in the score dtype (metal_runtime.py:908-929):
    # 1.5078125 * 1.5078125 = 2.27349853515625 rounds up to 2.28125 in bf16, so
    # three such products sum to 6.84375 (0x40DB); the fused float32 order sums
    # the unrounded products to 6.82049560546875, which rounds to 6.8125 (0x40DA).
    d = np.full((1, 3, 1), 0x3FC1, dtype=np.uint16)
    s = np.full((1, 3), 0x3FC1, dtype=np.uint16)
    assert moe.generic_decode_combine(d, s).tolist() == [[0x40DB]]
    assert moe.down_combine(d, s, score_dtype="bf16").tolist() == [[0x40DA]]
    one = np.array([[0x3F80]], dtype=np.uint16)
    assert moe.generic_decode_combine(d, s, shared_y=one).tolist() == [[0x40FB]]  # 7.84375
    assert moe.generic_decode_combine(d, s, keeps=[1]).tolist() == [[0x4012]]     # 2.28125


def _bf16_exact(value):
    """Nearest-even bf16 of a rational (8 significant bits, denormals below 2^-126)."""
    from fractions import Fraction

    v = Fraction(value)
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    quantum = Fraction(2) ** (max(e, -126) - 7)
    q, r = divmod(a, quantum)
    if r * 2 > quantum or (r * 2 == quantum and q % 2 == 1):
        q += 1
    return sign * q * quantum


def _f32_exact(value):
    """Nearest-even float32 of a rational (24 significant bits, denormals below 2^-126)."""
    from fractions import Fraction

    v = Fraction(value)
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    quantum = Fraction(2) ** (max(e, -126) - 23)
    q, r = divmod(a, quantum)
    if r * 2 > quantum or (r * 2 == quantum and q % 2 == 1):
        q += 1
    return sign * q * quantum


def test_swiglu_denormal_tail_matches_exact_rationals():
    # For gates near -88 the sigmoid 1/(1+e^88) lies below 2^-126: the bf16
    # sequence keeps it as a denormal (a flushing reciprocal would give -0).
    # Every step is recomputed here with exact rationals and float64 exp.
    import math
    from fractions import Fraction

    gates = np.arange(0xC2A0, 0xC2B2, dtype=np.uint16)  # -80.0 .. -89.0
    up = np.full(gates.shape, 0x3F80, dtype=np.uint16)
    got = moe.swiglu(gates, up)
    for g_bits, out_bits in zip(gates.tolist(), got.tolist()):
        g = Fraction(float(bf16.bf16_to_f32(np.uint16(g_bits))))
        m = -g
        e = _bf16_exact(_f32_exact(Fraction(math.exp(float(m)))))
        d = _bf16_exact(1 + e)
        sig = _bf16_exact(_f32_exact(1 / d))
        act = _bf16_exact(_f32_exact(_bf16_exact(_f32_exact(g * sig)) * 1))
        want = float(act)
        assert float(bf16.bf16_to_f32(np.uint16(out_bits))) == want, (hex(g_bits), hex(out_bits), want)
    tail = dict(zip(gates.tolist(), got.tolist()))
    assert (tail[0xC2AF], tail[0xC2B0], tail[0xC2B1]) == (0x8395, 0x8336, 0x82DD)  # -87.5, -88.0, -88.5


# ---------------------------------------------------------------- pool / layout
def test_layout_reference_constants():
    kat = KATS["layout_checkpoint_g32"]
    offs, stride, sizes = pool.record_layout(kat["hidden"], kat["inter"], kat["group"])
    assert stride == kat["stride"] and stride % 4096 == 0
    assert offs == kat["offsets"]
    assert sizes["gate_proj.weight"] == kat["part_bytes"]["weight"]
    assert offs["down_proj.biases"] + sizes["down_proj.biases"] == stride
    _, stride64, sizes64 = pool.record_layout(2560, 640, 64)
    assert sizes64["gate_proj.scales"] == 51200 and stride64 == 2764800
    _, stride_b, _ = pool.record_layout(2048, 512, 32)
    assert stride_b == 1966080


def test_lru_assign_reference_kat():
    kat = KATS["lru_assign"]
    lru = pool.LruSlots(kat["slots"])
    results = [lru.assign(layer, experts) for layer, experts in kat["calls"]]
    slots1, misses1 = results[0]
    assert len(misses1) == 10 and len(set(slots1.values())) == 10
    slots2, misses2 = results[1]
    assert slots2[3] == slots1[3] and [e for e, _ in misses2] == [20]
    slots4, misses4 = results[3]
    assert slots4[3] == slots1[3] and slots4[4] == slots1[4]
    assert {s for _, s in misses4} == {slots1[e] for e in kat["evicted_from_first_call"]}
    assert lru.hits == kat["expected_hits"] and lru.misses == kat["expected_misses"]
    with pytest.raises(ValueError):
        pool.LruSlots(kat["too_small_slots"])


def test_bf16_tile_weights_are_rounded_exact_weights():
    """The bf16-tile weight mode equals bf16(float32(exact dequant)): q*s + b is
    exact in float64, so one float32 rounding is the fused multiply-add."""
    from oracle import q4
    from oracle.bf16 import bf16_to_f32, f32_to_bf16

    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, (2, 64, 128)).astype(np.float32)
    packed, scales, biases = q4.quantize_affine(w, 32)
    bank = q4.ExpertBank(packed, scales, biases, 32)
    for e in range(2):
        exact = bank.dense(e)
        tiles = bank.dense_bf16(e)
        assert np.array_equal(tiles, bf16_to_f32(f32_to_bf16(exact.astype(np.float32))).astype(np.float64))
        # a bf16 tile differs from the exact weight by at most half a bf16 ulp
        assert np.all(np.abs(tiles - exact) <= np.abs(exact) * 2.0 ** -8 + 1e-30)


def test_router_logits_exact_rounding():
    """x @ Wg.T accumulated exactly and rounded once: with small integer-valued
    bf16 inputs the dot products are exact integers, so the bf16 logits must be
    the bf16 rounding of the integer dot product (odd sums exercise ties)."""
    rng = np.random.default_rng(12)
    x = rng.integers(-8, 9, (3, 64)).astype(np.float32)
    w = rng.integers(-8, 9, (5, 64)).astype(np.float32)
    got = router.router_logits(bf16.f32_to_bf16(x), bf16.f32_to_bf16(w))
    want = bf16.f32_to_bf16((x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32))
    assert np.array_equal(got, want)
    big = np.full((1, 64), 3.0, np.float32)  # 64 * 3 * 3 = 576 -> bf16 576 exactly; 577 -> tie case below
    assert bf16.bf16_to_f32(router.router_logits(bf16.f32_to_bf16(big), bf16.f32_to_bf16(big)))[0, 0] == 576.0
