"""Write tests/golden/reference_kats.json: the known-answer vectors that the
reference's own unit tests hold for the expert path, transcribed as data.

Sources (paths relative to the reference checkout):
* weighted_combine: models/flashnext/tests/unit/test_metal_runtime.py:222-263
* LRU assign:       models/flashnext/tests/unit/test_expert_pool.py:32-49
* record layout:    models/flashnext/tests/unit/test_slab_pack.py:50-63
* route encoding:   models/flashnext/tests/unit/test_metal_slab.py:17-25
* SwiGLU bits:      models/flashnext/tests/unit/test_swiglu_contract.py:21-31
  (the reference checks these against live MLX; the expected outputs here are
  computed by hand from the bf16 sigmoid sequence, see tests/test_oracle_kats.py)
* shared gate:      models/flashnext/tests/unit/test_metal_runtime.py:703 (0.333984375)
Run: python tests/golden/make_golden.py
"""
import json
from pathlib import Path

KATS = {
    "weighted_combine": {
        "expert_outputs": [[[1.0, 2.0], [10.0, 20.0], [100.0, 200.0]],
                           [[3.0, 4.0], [30.0, 40.0], [300.0, 400.0]]],
        "routes": [[2, 0], [1, 2]],
        "scores": [[0.25, 0.75], [0.4, 0.6]],
        "expected": [[25.75, 51.5], [192.0, 256.0]],
    },
    "lru_assign": {
        "slots": 16,
        "calls": [[1, list(range(10))], [1, [3, 4, 20]], [2, list(range(5))], [1, [3, 4, 30, 31]]],
        "expected_hits": 4,
        "expected_misses": 18,
        "evicted_from_first_call": [0, 1],
        "too_small_slots": 4,
    },
    "layout_checkpoint_g32": {
        "hidden": 2560, "inter": 640, "group": 32, "header": 4096, "stride": 3072000,
        "offsets": {"gate_proj.weight": 0, "gate_proj.scales": 819200, "gate_proj.biases": 921600,
                    "up_proj.weight": 1024000, "up_proj.scales": 1843200, "up_proj.biases": 1945600,
                    "down_proj.weight": 2048000, "down_proj.scales": 2867200,
                    "down_proj.biases": 2969600},
        "part_bytes": {"weight": 819200, "scales": 102400, "biases": 102400},
    },
    "route_encoding": {"slot": 5, "word": 0x80000005, "streamed": 3},
    "swiglu_representative": {
        "gate_bits": [0x0000, 0x3F80, 0xBF80, 0x4120, 0xC120],
        "up_bits": [0x3F80, 0x3FA0, 0x3F00, 0x4020, 0xC000],
        "expected_bits": [0x0000, 0x3F6A, 0xBE0A, 0x41C8, 0x3A6F],
    },
    "shared_gate_value": 0.333984375,
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_kats.json")
    out.write_text(json.dumps(KATS, indent=1, sort_keys=True) + "\n")
    print(f"wrote {out}")
