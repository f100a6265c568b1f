"""bench.py's committed inputs: the roofline traffic figure it reads from the
expert-stage rocprofv3 --pmc summary must parse as a byte count close to the
algorithmic expert bytes of one decode layer (11 records of 1,966,080 B)."""
from __future__ import annotations

import importlib.util
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_module", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_expert_stage_traffic_parses():
    traffic = _bench().load_traffic("decode_expert_stage")
    assert isinstance(traffic, int)
    algorithmic = 11 * 1_966_080
    assert algorithmic <= traffic <= 1.1 * algorithmic, traffic


def test_missing_profile_gives_none():
    assert _bench().load_traffic("no_such_kernel") is None
