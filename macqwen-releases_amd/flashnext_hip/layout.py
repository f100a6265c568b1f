"""Expert record layout: the reference's slab/pool record generalised to any shape.

A record holds one expert's nine parts in the order gate/up/down x
weight/scales/biases, back to back, and the record stride is rounded up to a
whole 4096-byte page (``models/flashnext/slab_pack.py:77-149``).  The pool
puts a 4096-byte header before slot 0 (``models/flashnext/expert_pool.py:36``).
At the checkpoint shape (hidden 2560, intermediate 640, group 32) this gives
the reference's constants: stride 3,072,000 and offsets 0, 819,200, ...,
2,969,600.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

HEADER_SIZE = 4096
PAGE_SIZE = 4096
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
PARTS = ("weight", "scales", "biases")
PART_KEYS = tuple((proj, part) for proj in PROJECTIONS for part in PARTS)


@dataclass(frozen=True)
class SlabLayout:
    """Immutable record layout for one (hidden, intermediate, group) shape."""

    hidden: int
    inter: int
    group_size: int
    record_stride: int
    record_bytes: int
    shapes: Tuple[Tuple[str, Tuple[int, int]], ...]
    offsets: Tuple[Tuple[str, int], ...]

    @property
    def name(self) -> str:
        return f"q4-g{self.group_size}-h{self.hidden}-i{self.inter}"

    def shape(self, projection: str, part: str) -> Tuple[int, int]:
        return dict(self.shapes)[f"{projection}.{part}"]

    def offset(self, projection: str, part: str) -> int:
        return dict(self.offsets)[f"{projection}.{part}"]

    def part_bytes(self, projection: str, part: str) -> int:
        rows, cols = self.shape(projection, part)
        return rows * cols * (4 if part == "weight" else 2)


def make_layout(hidden: int, inter: int, group_size: int = 32) -> SlabLayout:
    if group_size not in (32, 64):
        raise ValueError(f"Unsupported quantization group size: {group_size}")
    if hidden <= 0 or inter <= 0 or hidden % group_size or inter % group_size:
        raise ValueError("hidden and intermediate must be positive multiples of the group size")
    dims = {"gate_proj": (inter, hidden), "up_proj": (inter, hidden), "down_proj": (hidden, inter)}
    shapes, offsets, cursor = [], [], 0
    for proj in PROJECTIONS:
        rows, cols = dims[proj]
        for part in PARTS:
            shape = (rows, cols // 8) if part == "weight" else (rows, cols // group_size)
            shapes.append((f"{proj}.{part}", shape))
            offsets.append((f"{proj}.{part}", cursor))
            cursor += shape[0] * shape[1] * (4 if part == "weight" else 2)
    stride = -(-cursor // PAGE_SIZE) * PAGE_SIZE
    return SlabLayout(hidden, inter, group_size, stride, cursor, tuple(shapes), tuple(offsets))


CHECKPOINT_G32 = make_layout(2560, 640, 32)
CHECKPOINT_G64 = make_layout(2560, 640, 64)
H2048_I512_G32 = make_layout(2048, 512, 32)
