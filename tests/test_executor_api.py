"""Executor argument handling and capability seam, mirroring the reference's
checkpoint-free tests (models/flashnext/tests/unit/test_metal_runtime.py:19-263).
No kernel runs here."""
from __future__ import annotations

import json
import os
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest

from flashnext_hip.hip_runtime import (HipMoEExecutor, MetalMoEExecutor, probe_capabilities,
                                       weighted_combine)

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


@pytest.mark.parametrize("kwargs", [
    {"expert_count": 0, "hidden_size": 2, "top_k": 1},
    {"expert_count": 2, "hidden_size": 0, "top_k": 1},
    {"expert_count": 2, "hidden_size": 2, "top_k": 0},
    {"expert_count": 2, "hidden_size": 2, "top_k": 3},
    {"expert_count": 513, "hidden_size": 2, "top_k": 1},
    {"expert_count": 2, "hidden_size": 2, "top_k": 1, "group_size": 16},
    {"expert_count": 2, "hidden_size": 2, "top_k": 1, "max_tokens": 9},
])
def test_constructor_rejects_bad_arguments(kwargs):
    with pytest.raises(ValueError):
        HipMoEExecutor(**kwargs)


def test_reference_name_alias():
    assert MetalMoEExecutor is HipMoEExecutor


def test_combine_rejects_incompatible_shapes_and_out_of_range_routes():
    with pytest.raises(ValueError):
        weighted_combine(np.zeros((2, 3, 2)), np.zeros((2, 2), dtype=np.int32), np.ones((2, 1)))
    with pytest.raises(ValueError):
        weighted_combine(np.zeros((2, 3, 2)), np.array([[0, 3]]), np.ones((1, 2)))


def test_execute_rejects_malformed_q4_pack():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    bad = (np.zeros((2, 4, 3), dtype=np.uint32), np.zeros((2, 4, 1), np.float32), np.zeros((2, 4, 1), np.float32))
    good = (np.zeros((2, 4, 4), dtype=np.uint32), np.zeros((2, 4, 1), np.float32), np.zeros((2, 4, 1), np.float32))
    down = (np.zeros((2, 32, 4), dtype=np.uint32), np.zeros((2, 32, 1), np.float32), np.zeros((2, 32, 1), np.float32))
    with pytest.raises(ValueError, match="weight shape"):
        executor.execute(np.zeros((1, 32), np.float32), np.zeros((1, 1), np.int32),
                         {"gate_proj": bad, "up_proj": good, "down_proj": down})


def test_execute_rejects_route_token_mismatch():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    with pytest.raises(ValueError, match="same token count"):
        executor.execute(np.zeros((2, 32), np.float32), np.zeros((1, 1), np.int32), {})


def test_execute_without_device_raises_instead_of_falling_back():
    executor = HipMoEExecutor(expert_count=2, hidden_size=32, top_k=1, backend="reference")
    proj = (np.zeros((2, 32, 4), dtype=np.uint32), np.zeros((2, 32, 1), np.float32), np.zeros((2, 32, 1), np.float32))
    down = (np.zeros((2, 32, 4), dtype=np.uint32), np.zeros((2, 32, 1), np.float32), np.zeros((2, 32, 1), np.float32))
    with pytest.raises(RuntimeError, match="unavailable"):
        executor.execute(np.zeros((1, 32), np.float32), np.zeros((1, 1), np.int32),
                         {"gate_proj": proj, "up_proj": proj, "down_proj": down})
    assert executor.last_path == "unavailable"


def test_fused_up_swiglu_flag_default_constructor_and_env(monkeypatch):
    monkeypatch.delenv("FLASHNEXT_FUSED_UP_SWIGLU", raising=False)
    assert not HipMoEExecutor(2, 32, 1).fused_up_swiglu
    assert HipMoEExecutor(2, 32, 1, fused_up_swiglu=True).fused_up_swiglu
    monkeypatch.setenv("FLASHNEXT_FUSED_UP_SWIGLU", "1")
    assert HipMoEExecutor(2, 32, 1).fused_up_swiglu


def test_capabilities_of_injected_backends():
    caps = probe_capabilities(SimpleNamespace(available=False, supports_custom_moe=False))
    assert not caps.available and not caps.supports_custom_moe
    caps = probe_capabilities(SimpleNamespace(available=True, supports_custom_moe=True))
    assert caps.available and caps["supports_custom_moe"]
    assert not probe_capabilities("reference").available
    assert not probe_capabilities("metal").available


def test_unsupported_backend_fails_before_execution():
    executor = HipMoEExecutor(2, 2, 1, backend=SimpleNamespace(available=True, supports_custom_moe=False))
    with pytest.raises(RuntimeError, match="custom MoE"):
        executor.execute(np.zeros((1, 2), np.float32), np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32))


def test_combine_probe_uses_reference_route_math():
    kat = KATS["weighted_combine"]
    executor = HipMoEExecutor(3, 2, 2, backend=SimpleNamespace(available=True, supports_custom_moe=True))
    out = executor.execute(np.array(kat["expert_outputs"], np.float32), np.array(kat["routes"]),
                           np.array(kat["scores"], np.float32))
    assert out.tolist() == kat["expected"]
    assert executor.last_path == "custom-hip"
