"""HBM expert slot pool with LRU assignment and pinned-host refill.

Mirrors ``models/flashnext/expert_pool.py`` (``ExpertPool``): one region
laid out like the slab pack (a 4 KiB header, then fixed-stride records with
the nine parts at the layout offsets), an LRU over ``(layer, expert)`` keys
(:meth:`HipExpertPool.assign` restates ``assign`` ``:88-110``: hits move to
the most recent end first, then every miss takes a free slot, ascending from
slot 0, or evicts the least recently used key), and a fill of the missed
records (``fill`` ``:133-145``).

The region is HBM (a device tensor), the decode and grouped kernels address
its records in place through slot words (``0x80000000 | slot``), and a miss
is one pinned host-to-device copy of the whole record image on a side stream
instead of nine file reads: by default one gather kernel per fill that reads
the pinned records over PCIe (``mq_pool_refill_gather_async``), or one
``hipMemcpyAsync`` per record (``mq_pool_refill_async``).  Ordering follows the
reference's rule that a slot is only overwritten after its last reader
finished: the copy stream first waits for everything already queued on the
compute stream, and the compute stream then waits for the copies.
"""
from __future__ import annotations

import ctypes
from collections import OrderedDict

import torch

from . import _lib
from .layout import HEADER_SIZE, PART_KEYS, SlabLayout, make_layout

SLOT_BIT = _lib.MQ_SLOT_BIT
MIN_SLOTS = 16  # one decode layer (expert_pool.py:64-65)


class HostRecordStore:
    """Record images of experts in pinned host memory, keyed by (layer, expert).

    Each image is ``record_stride`` bytes with the nine parts at their layout
    offsets, so one contiguous copy places a whole record in a pool slot.
    """

    def __init__(self, layout: SlabLayout):
        self.layout = layout
        self._records: dict[tuple[int, int], torch.Tensor] = {}

    def add(self, layer: int, expert: int, parts: dict) -> None:
        """``parts``: ``"gate_proj.weight" -> tensor`` (any dtype, host or device)."""
        img = torch.zeros(self.layout.record_stride, dtype=torch.uint8, pin_memory=True)
        for proj, part in PART_KEYS:
            data = parts[f"{proj}.{part}"].detach().contiguous().view(torch.uint8).reshape(-1).cpu()
            off = self.layout.offset(proj, part)
            img[off:off + data.numel()].copy_(data)
        self._records[(int(layer), int(expert))] = img

    def add_banks(self, layer: int, banks: dict) -> None:
        """``banks``: ``"gate_proj" -> (weight [E,...], scales, biases)``; adds every expert."""
        experts = banks["gate_proj"][0].shape[0]
        for e in range(experts):
            parts = {}
            for proj in ("gate_proj", "up_proj", "down_proj"):
                w, s, b = banks[proj]
                parts[f"{proj}.weight"], parts[f"{proj}.scales"], parts[f"{proj}.biases"] = w[e], s[e], b[e]
            self.add(layer, e, parts)

    def record(self, layer: int, expert: int) -> torch.Tensor:
        try:
            return self._records[(int(layer), int(expert))]
        except KeyError:
            raise KeyError(f"no host record for layer {layer} expert {expert}") from None


class HipExpertPool:
    """LRU pool of expert records resident in HBM."""

    def __init__(self, size_bytes: int, hidden: int, inter: int, group_size: int = 32, *, device="cuda"):
        self.layout = make_layout(hidden, inter, group_size)
        self.stride = self.layout.record_stride
        self.slots = (int(size_bytes) - HEADER_SIZE) // self.stride
        if self.slots < MIN_SLOTS:
            raise ValueError("expert pool is too small for one decode layer")
        self.buffer = torch.zeros(HEADER_SIZE + self.slots * self.stride, dtype=torch.uint8, device=device)
        # (layer, expert) -> slot, least recently used first.
        self._lru: "OrderedDict[tuple, int]" = OrderedDict()
        self._unused = 0  # slots [_unused, slots) have never held a record
        self.hits = 0
        self.misses = 0
        self._lib = _lib.load()
        # Events of the fills, created once per stream: `ready` marks the
        # compute stream's position for the copy streams, `done` each copy
        # stream's completion.  The first record of a torch event creates the
        # HIP event (about 12 us on the host), so new events per fill cost more
        # host time than the refill launch itself.
        self._events: dict = {}

    def _claim_slot(self) -> int:
        """A never-used slot (lowest first) while any is left, else the slot of
        the least recently used key, which is dropped."""
        if self._unused < self.slots:
            self._unused += 1
            return self._unused - 1
        _key, slot = self._lru.popitem(last=False)
        return slot

    # ------------------------------------------------------------ LRU (expert_pool.py:88-110)
    def assign(self, layer: int, experts):
        """Slots for one layer's experts: ``({expert: slot}, [(expert, slot), ...])``.

        The order rules are the reference pool's, which its tests fix: every
        requested expert already resident is refreshed first, in request order,
        so none of them can be evicted by this call's misses while older keys
        remain; the misses then claim slots in request order (untouched slots
        from slot 0 upwards, then the least recently used keys).  The second
        list names the slots whose records must be filled.
        """
        requested = list(experts)
        placed: dict = {}
        for expert in requested:
            key = (layer, expert)
            slot = self._lru.pop(key, None)
            if slot is not None:
                self._lru[key] = slot  # re-inserted at the most recent end
                placed[expert] = slot
        self.hits += len(placed)
        to_fill = []
        for expert in requested:
            if expert not in placed:
                slot = self._claim_slot()
                self._lru[(layer, expert)] = slot
                placed[expert] = slot
                to_fill.append((expert, slot))
        self.misses += len(to_fill)
        return placed, to_fill

    # ------------------------------------------------------------ refill (expert_pool.py:112-145)
    def fill(self, layer: int, misses, store: HostRecordStore, *, compute_stream=None, copy_stream=None,
             method: str = "gather"):
        """Copy the missed records from pinned host memory into their slots.

        The copies run on ``copy_stream`` after everything already queued on
        ``compute_stream`` (earlier readers of the victim slots); the compute
        stream then waits for them.  ``method="gather"`` moves all misses with
        one kernel that reads the pinned records over PCIe
        (``mq_pool_refill_gather_async``) on the first copy stream;
        ``method="memcpy"`` issues one ``hipMemcpyAsync`` per record
        (``mq_pool_refill_async``), and then ``copy_stream`` may be a sequence
        of streams: the misses are split into contiguous shares, one per
        stream, so that several DMA engines move them at once.  Returns the
        completion events (one per copy stream used) as a list when
        ``copy_stream`` is a sequence, else the single event.  The events
        belong to the pool and are recorded again by its next fill on the same
        copy stream.  With no copy stream (or the compute stream itself) the
        copies are simply queued on the compute stream.
        """
        if method not in ("gather", "memcpy"):
            raise ValueError(f"method must be 'gather' or 'memcpy', got {method!r}")
        compute = compute_stream if compute_stream is not None else torch.cuda.current_stream(self.buffer.device)
        copies = list(copy_stream) if isinstance(copy_stream, (list, tuple)) else \
            [copy_stream if copy_stream is not None else compute]
        if method == "gather":
            copies = copies[:1]
        refill = self._lib.mq_pool_refill_gather_async if method == "gather" else self._lib.mq_pool_refill_async
        misses = list(misses)
        recs = [store.record(layer, e) for e, _slot in misses]  # owned by the store: outlive the copies
        share = -(-len(misses) // len(copies)) if misses else 0
        ready = None
        events = []
        for i, copy in enumerate(copies):
            part = misses[i * share:(i + 1) * share]
            part_recs = recs[i * share:(i + 1) * share]
            side = copy.cuda_stream != compute.cuda_stream
            if side:  # the copies start after everything queued on the compute stream
                if ready is None:
                    ready = self._event(("ready", compute.cuda_stream))
                    ready.record(compute)
                copy.wait_event(ready)
            done = self._event(("done", copy.cuda_stream))
            n = len(part)
            slots = (ctypes.c_uint32 * max(n, 1))(*[int(slot) for _e, slot in part])
            ptrs = (ctypes.c_void_p * max(n, 1))(*[r.data_ptr() for r in part_recs])
            rc = refill(ctypes.c_void_p(self.buffer.data_ptr()), HEADER_SIZE, self.stride, self.slots, slots, ptrs, n,
                        self.stride, ctypes.c_void_p(copy.cuda_stream), None)
            _lib.check(rc, self._lib)
            done.record(copy)
            events.append(done)
            if side:
                compute.wait_event(done)
        return events if isinstance(copy_stream, (list, tuple)) else events[0]

    def _event(self, key) -> torch.cuda.Event:
        ev = self._events.get(key)
        if ev is None:
            ev = self._events[key] = torch.cuda.Event()
        return ev

    # ------------------------------------------------------------ addressing
    def projection(self, name: str) -> _lib.MqProjection:
        p = _lib.MqProjection()
        p.pool = self.buffer.data_ptr()
        p.pool_header = HEADER_SIZE
        p.pool_stride = self.stride
        p.pool_slots = self.slots
        p.off_weight = self.layout.offset(name, "weight")
        p.off_scales = self.layout.offset(name, "scales")
        p.off_biases = self.layout.offset(name, "biases")
        return p

    @staticmethod
    def route_words(slots: dict, inds) -> torch.Tensor:
        """Slot words ``0x80000000 | slot`` (as int32 bits) for an expert-id tensor."""
        import numpy as np

        flat = np.array([SLOT_BIT | slots[int(e)] for e in inds.reshape(-1).tolist()], dtype=np.uint32)
        return torch.from_numpy(flat.view(np.int32).reshape(tuple(inds.shape)))

    def record_bytes(self, slot: int) -> torch.Tensor:
        """Device view of one slot's record (for checks)."""
        base = HEADER_SIZE + int(slot) * self.stride
        return self.buffer[base:base + self.stride]
