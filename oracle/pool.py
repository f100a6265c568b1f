"""Expert record layout and LRU slot assignment (test infrastructure).

* Record layout: parts in the order gate/up/down x weight/scales/biases, each
  part packed back to back, a 4096-byte header before slot 0, and a record
  stride rounded up to whole 4096-byte pages
  (``models/flashnext/slab_pack.py:96-149``, generalised from the fixed
  2560/640 checkpoint shape to any hidden/intermediate/group).
* Address of a part: ``base + header + slot * stride + offset(part)``
  (``models/flashnext/metal_runtime.py:194-228``, 64-bit).
* ``LruSlots.assign`` restates ``ExpertPool.assign``
  (``models/flashnext/expert_pool.py:88-110``): hits move to the MRU end
  first; then each miss takes a free slot (free list popped from the end of
  a descending list, i.e. ascending slots) or evicts the LRU key.
"""
from __future__ import annotations

from collections import OrderedDict

HEADER = 4096
PAGE = 4096
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
PARTS = ("weight", "scales", "biases")


def record_layout(hidden: int, inter: int, group_size: int = 32, page: int = PAGE):
    """Return (offsets dict ``"proj.part" -> bytes``, stride, part sizes dict)."""
    sizes = {}
    for proj, rows, cols in (("gate_proj", inter, hidden), ("up_proj", inter, hidden),
                             ("down_proj", hidden, inter)):
        sizes[f"{proj}.weight"] = rows * cols // 2          # uint32, 8 nibbles/word
        sizes[f"{proj}.scales"] = rows * (cols // group_size) * 2   # bf16
        sizes[f"{proj}.biases"] = rows * (cols // group_size) * 2
    offsets, cursor = {}, 0
    for proj in PROJECTIONS:
        for part in PARTS:
            key = f"{proj}.{part}"
            offsets[key] = cursor
            cursor += sizes[key]
    stride = -(-cursor // page) * page
    return offsets, stride, sizes


def part_address(base: int, slot: int, offset: int, stride: int, header: int = HEADER) -> int:
    return base + header + slot * stride + offset


class LruSlots:
    """Slot bookkeeping of the expert pool (no storage)."""

    def __init__(self, slots: int, min_slots: int = 16):
        if slots < min_slots:
            raise ValueError("expert pool is too small for one decode layer")
        self.slots = int(slots)
        self._slot_of: "OrderedDict[tuple, int]" = OrderedDict()
        self._free = list(range(self.slots - 1, -1, -1))
        self.hits = 0
        self.misses = 0

    def assign(self, layer: int, experts):
        slot_of = self._slot_of
        slots, misses = {}, []
        for expert in experts:
            key = (layer, expert)
            slot = slot_of.get(key)
            if slot is not None:
                slot_of.move_to_end(key)
                slots[expert] = slot
        self.hits += len(slots)
        for expert in experts:
            if expert in slots:
                continue
            if self._free:
                slot = self._free.pop()
            else:
                _old, slot = slot_of.popitem(last=False)
            slot_of[(layer, expert)] = slot
            slots[expert] = slot
            misses.append((expert, slot))
        self.misses += len(misses)
        return slots, misses
