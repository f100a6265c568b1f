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


def test_more_than_one_gpu_is_refused_before_any_device_work():
    import subprocess
    import sys

    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no benchmark line


def test_zipf_routes_are_distinct_seeded_and_skewed():
    import numpy as np

    b = _bench()
    inds = b.zipf_routes(512, 64, 10, seed=3)
    assert inds.shape == (512, 10) and inds.dtype == np.int32
    assert all(len(set(row)) == 10 for row in inds.tolist())  # top-k without replacement
    assert np.array_equal(inds, b.zipf_routes(512, 64, 10, seed=3))
    counts = np.bincount(inds.reshape(-1), minlength=64)
    assert counts.max() <= 512 and counts[0] > counts[-1]  # the head expert is the hottest


def test_per_kernel_rooflines_parse_from_the_kernel_trace():
    r = _bench().kernel_rooflines(11 * 1_966_080, 512 * 2048 * 2)
    assert r is not None
    names = [k["kernel"] for k in r["kernels"]]
    assert "down_combine_kernel" in names and "gateup_kernel, routes given" in names
    for k in r["kernels"]:
        assert k["profiled_us"] > 0 and 0 < k["frac"] < 1
