"""The C restatement of the oracle agrees with the numpy restatement."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, cbase, moe, q4, router

from ._helpers import bf16_normal, make_records


@pytest.fixture(scope="module")
def small():
    hidden, inter, experts = 256, 64, 12
    recs = make_records(experts, hidden, inter, seed=7)
    shared = make_records(1, hidden, inter, seed=8)
    wg = bf16_normal((experts, hidden), seed=9, std=0.05)
    wsg = bf16_normal((1, hidden), seed=10, std=0.05)
    return recs, shared, wg, wsg


def test_c_qmv_matches_numpy(small):
    recs = small[0]
    x = bf16_normal((2, 256), seed=11)
    y = cbase.qmv(x, recs.gate.packed[3], recs.gate.scales[3], recs.gate.biases[3])
    want = q4.qmv_f64(bf16.bf16_to_f32(x), recs.gate.packed[3], recs.gate.scales[3], recs.gate.biases[3])
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)


def test_c_decode_layer_matches_numpy_oracle(small):
    recs, shared, wg, wsg = small
    x = bf16_normal((3, 256), seed=12)
    out, inds = cbase.decode_layer(x, wg, recs, 4, shared=(shared.gate, shared.up, shared.down),
                                   shared_gate_w=wsg)
    ref = router.route(x, wg, 4)
    assert np.array_equal(inds, ref["inds"])
    full = moe.ExpertRecordSet(recs.gate, recs.up, recs.down, shared=(shared.gate, shared.up, shared.down))
    want = moe.decode_layer(x, ref["inds"], ref["scores"], full, score_dtype="bf16", shared_gate_weight=wsg)
    a, b = bf16.bf16_to_f32(out), bf16.bf16_to_f32(want)
    np.testing.assert_allclose(a, b, rtol=1e-2, atol=3e-3)
    assert float(np.dot(a.ravel(), b.ravel()) / (np.linalg.norm(a) * np.linalg.norm(b))) >= 0.9999
