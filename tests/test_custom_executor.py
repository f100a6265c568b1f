"""The layer-benchmark plug-in (``flashnext_hip.custom_executor``).

CPU: the module exposes what ``bench_runtime_layer.py`` looks for
(``:85-101``), its builder and runner take only names the benchmark's context
provides (``:383-408``), and unsupported formats are refused before any device
work.  GPU: the runner's output matches the oracle's grouped path (unsorted
gather_qmm chain + bf16 combine) within the layer tolerance, with and without
scores, for a leading batch dimension as the benchmark passes it.
"""
from __future__ import annotations

import inspect

import numpy as np
import pytest

from oracle import bf16, moe

from ._helpers import MAX_REL, MIN_COSINE, assert_close, bf16_normal, make_records, say, value_report

CONTEXT_KEYS = {"x", "inputs", "hidden_states", "packs", "weights", "expert_weights", "projections", "gate", "up",
                "down", "gate_proj", "up_proj", "down_proj", "indices", "rhs_indices", "expert_indices", "route",
                "expert_ids", "miss_fraction", "miss", "scores", "gating_scores", "routes", "route_indices",
                "expert_outputs", "expert_values", "group_size", "bits", "mode", "activation", "expert_count",
                "hidden_size", "top_k"}


def test_plugin_entry_points_take_benchmark_context_names():
    from flashnext_hip import custom_executor as ce

    assert callable(getattr(ce, "build_executor"))
    for fn in (ce.build_executor, ce.LayerRunner.execute, ce.LayerRunner.run):
        params = [p for p in inspect.signature(fn).parameters.values() if p.name != "self"]
        required = {p.name for p in params if p.default is inspect.Parameter.empty}
        assert required <= CONTEXT_KEYS, (fn, required - CONTEXT_KEYS)
        assert all(p.kind != inspect.Parameter.POSITIONAL_ONLY for p in params)


class SwiGLU:  # stands in for the benchmark's nn.SwiGLU instance
    pass


class GELU:
    pass


@pytest.mark.parametrize("kw", [{"bits": 8}, {"mode": "mxfp4"}, {"group_size": 128}, {"activation": GELU()},
                                {"activation": "gelu"}])
def test_builder_refuses_other_formats_before_device_work(kw):
    from flashnext_hip.custom_executor import build_executor

    args = {"packs": {}, "group_size": 32, "bits": 4, "mode": "affine", "activation": SwiGLU()}
    args.update(kw)
    with pytest.raises(ValueError):
        build_executor(**args)


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [3, 20])
def test_plugin_runner_matches_oracle(tokens):
    import torch

    from flashnext_hip.custom_executor import build_executor

    say(f"case: layer-benchmark plug-in tokens={tokens}")
    experts, hidden, inter, k = 12, 2048, 512, 8
    recs = make_records(experts, hidden, inter, seed=600)
    packs = {name: (bank.packed.view(np.uint32), bank.scales, bank.biases)
             for name, bank in (("gate_proj", recs.gate), ("up_proj", recs.up), ("down_proj", recs.down))}
    runner = build_executor(packs=packs, group_size=32, bits=4, mode="affine", activation=SwiGLU())
    rng = np.random.default_rng(601)
    inds = np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)]).astype(np.int64)
    raw = rng.random((tokens, k)).astype(np.float32) + 0.05
    scores = (raw / raw.sum(1, keepdims=True)).astype(np.float32)
    x = bf16_normal((tokens, hidden), seed=602)
    xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).cuda().reshape(1, tokens, hidden)
    out = runner.execute(x=xd, indices=inds[None], scores=scores[None])
    y = runner.run(x=xd, indices=inds[None])
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, tokens, hidden) and tuple(y.shape) == (1, tokens, k, hidden)
    sb = bf16.f32_to_bf16(scores)
    want_out, want_y = moe.prefill_layer(x, inds, sb, recs, weights="bf16")
    exact_out, _ = moe.prefill_layer(x, inds, sb, recs)
    got = lambda t: bf16.bf16_to_f32(t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
    assert_close(got(out)[0], bf16.bf16_to_f32(want_out), "plug-in combined")
    assert_close(got(y)[0], bf16.bf16_to_f32(want_y), "plug-in per-slot")
    rep = value_report(got(out)[0], bf16.bf16_to_f32(exact_out))
    assert rep["cosine"] >= MIN_COSINE and rep["max_rel"] <= MAX_REL, rep
