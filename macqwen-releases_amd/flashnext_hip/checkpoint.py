"""Checkpoint reader: safetensors shards to HBM slot-pool records.

Restates the reference's random-access reader (``models/flashnext/store.py``:
``SafeTensorStore.__init__`` / ``add_shard`` ``:174-205`` parse the shard
index and every shard header once; ``TensorRef`` ``:100-109`` keeps a
tensor's dtype, shape and data start; the first dimension of an expert tensor
is the expert, so one expert is one row) without MLX: tensors are numpy
memory maps and rows are gathered with fancy indexing.

The MoE block's tensors follow the model's module paths
(``models/flashnext/loader.py:344``)::

    language_model.model.layers.{L}.mlp.gate.weight                  bf16 [E, H]   router
    language_model.model.layers.{L}.mlp.switch_mlp.{p}.weight         u32  [E, O, I*bits/32]
    language_model.model.layers.{L}.mlp.switch_mlp.{p}.scales|biases  bf16 [E, O, I/g]
    language_model.model.layers.{L}.mlp.shared_expert.{p}.weight|scales|biases   (one expert)
    language_model.model.layers.{L}.mlp.shared_expert_gate.weight     bf16 [1, H]

for ``p`` in gate_proj / up_proj / down_proj.  The group size and bit width of
a layer are inferred from its tensor shapes exactly as
``infer_switch_quantization`` (``models/flashnext/loader.py:360-382``) does.

Records are laid out by :mod:`.layout` (the nine parts back to back at the
reference's record offsets, page-rounded stride, 4 KiB pool header), so a
loaded pool is addressed by the decode and grouped kernels through slot words
like any other pool.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, Iterable, Optional, Sequence, Tuple

import numpy as np

from .layout import HEADER_SIZE, PART_KEYS, PROJECTIONS, SlabLayout, make_layout

# safetensors dtype -> numpy storage dtype (bf16 travels as uint16 bits)
_DTYPES: Dict[str, np.dtype] = {
    "F32": np.dtype("<f4"), "F16": np.dtype("<f2"), "BF16": np.dtype("<u2"), "U32": np.dtype("<u4"),
    "I32": np.dtype("<i4"), "I64": np.dtype("<i8"), "U64": np.dtype("<u8"), "F64": np.dtype("<f8"),
    "BOOL": np.dtype("?"), "U16": np.dtype("<u2"), "U8": np.dtype("u1"), "I8": np.dtype("i1"),
}

LAYER_PREFIX = "language_model.model.layers.{layer}.mlp"


@dataclass(frozen=True)
class TensorRef:
    shard: str
    dtype: str
    shape: Tuple[int, ...]
    start: int  # byte offset of the tensor data in its shard


class SafeTensorIndex:
    """Every tensor of a sharded safetensors checkpoint, memory-mapped on demand.

    ``model_dir`` holds ``model.safetensors.index.json`` (a ``weight_map`` of
    tensor name to shard file) and the shards; a directory with a single
    ``model.safetensors`` and no index is accepted too.
    """

    def __init__(self, model_dir: str):
        self.dir = os.path.expanduser(model_dir)
        self.refs: Dict[str, TensorRef] = {}
        self._views: Dict[str, np.ndarray] = {}
        index_path = os.path.join(self.dir, "model.safetensors.index.json")
        if os.path.exists(index_path):
            with open(index_path) as handle:
                shards = sorted(set(json.load(handle)["weight_map"].values()))
        elif os.path.exists(os.path.join(self.dir, "model.safetensors")):
            shards = ["model.safetensors"]
        else:
            raise FileNotFoundError(f"no safetensors checkpoint in {self.dir}")
        for shard in shards:
            self.add_shard(shard)

    def add_shard(self, shard: str) -> None:
        path = os.path.join(self.dir, shard)
        with open(path, "rb") as handle:
            header_len = struct.unpack("<Q", handle.read(8))[0]
            header = json.loads(handle.read(header_len))
        data_start = 8 + header_len
        for name, meta in header.items():
            if name == "__metadata__":
                continue
            if meta["dtype"] not in _DTYPES:
                raise ValueError(f"{name}: unsupported safetensors dtype {meta['dtype']}")
            begin, end = meta["data_offsets"]
            shape = tuple(int(d) for d in meta["shape"])
            if end - begin != int(np.prod(shape, dtype=np.int64)) * _DTYPES[meta["dtype"]].itemsize:
                raise ValueError(f"{name}: data size does not match its shape")
            self.refs[name] = TensorRef(shard, meta["dtype"], shape, data_start + begin)

    def __contains__(self, name: str) -> bool:
        return name in self.refs

    def shape(self, name: str) -> Tuple[int, ...]:
        return self.refs[name].shape

    def dtype(self, name: str) -> str:
        return self.refs[name].dtype

    def array(self, name: str) -> np.ndarray:
        """Read-only memory map of the whole tensor (bf16 as uint16 bits)."""
        view = self._views.get(name)
        if view is None:
            ref = self.refs[name]
            view = np.memmap(os.path.join(self.dir, ref.shard), dtype=_DTYPES[ref.dtype], mode="r",
                             offset=ref.start, shape=ref.shape)
            self._views[name] = view
        return view

    def rows(self, name: str, indices: Sequence[int]) -> np.ndarray:
        """Rows (first-dimension slices, e.g. experts) gathered into memory."""
        return np.ascontiguousarray(self.array(name)[list(indices)])


def infer_switch_quantization(index: SafeTensorIndex, prefix: str) -> Tuple[int, int]:
    """(group_size, bits) of an expert block from its tensor shapes.

    ``down_proj.weight`` is ``[E, hidden, packed_inter]``, so its second
    dimension is the input width of gate/up; the bit width follows from the
    packed gate width and the group size from the gate scale count
    (``models/flashnext/loader.py:360-382``).
    """
    packed = int(index.shape(f"{prefix}.gate_proj.weight")[-1])
    groups = int(index.shape(f"{prefix}.gate_proj.scales")[-1])
    hidden = int(index.shape(f"{prefix}.down_proj.weight")[1])
    if packed <= 0 or groups <= 0 or hidden <= 0:
        raise ValueError(f"invalid switch quantization shapes at {prefix}")
    packed_bits = packed * 32
    if packed_bits % hidden or hidden % groups:
        raise ValueError(f"incompatible switch quantization shapes at {prefix}")
    return hidden // groups, packed_bits // hidden


@dataclass
class CheckpointLayer:
    """One MoE layer's tensors (memory maps) and its record layout."""

    layer: int
    layout: SlabLayout
    experts: int
    parts: Dict[str, np.ndarray]        # "gate_proj.weight" -> [E, ...] memory map
    router_w: Optional[np.ndarray]      # bf16 bits [E, H]
    shared: Optional[Dict[str, np.ndarray]]  # "gate_proj.weight" -> [O, ...] (one expert)
    shared_gate_w: Optional[np.ndarray]  # bf16 bits [H]


def read_layer(index: SafeTensorIndex, layer: int) -> CheckpointLayer:
    """The tensors of MoE layer ``layer``; raises for shapes the kernels do not take.

    The expert tensors must be 4-bit with group 32 or 64 (the record layouts
    of ``models/flashnext/slab_pack.py:96-104``) and agree with one another.
    """
    base = LAYER_PREFIX.format(layer=layer)
    prefix = f"{base}.switch_mlp"
    if f"{prefix}.gate_proj.weight" not in index:
        raise KeyError(f"layer {layer} has no switch_mlp expert tensors")
    group, bits = infer_switch_quantization(index, prefix)
    if bits != 4:
        raise ValueError(f"layer {layer}: {bits}-bit experts are not supported (4-bit only)")
    experts, inter, _ = index.shape(f"{prefix}.gate_proj.weight")
    hidden = int(index.shape(f"{prefix}.down_proj.weight")[1])
    layout = make_layout(hidden, inter, group)
    parts = {}
    for proj, part in PART_KEYS:
        name = f"{prefix}.{proj}.{part}"
        want = (experts,) + layout.shape(proj, part)
        got = index.shape(name)
        if got != want:
            raise ValueError(f"{name}: shape {got}, expected {want}")
        if index.dtype(name) != ("U32" if part == "weight" else "BF16"):
            raise ValueError(f"{name}: dtype {index.dtype(name)}")
        parts[f"{proj}.{part}"] = index.array(name)
    router = f"{base}.gate.weight"
    router_w = index.array(router) if router in index else None
    if router_w is not None and (router_w.shape != (experts, hidden) or index.dtype(router) != "BF16"):
        raise ValueError(f"{router}: expected bf16 [{experts}, {hidden}]")
    shared = None
    if f"{base}.shared_expert.gate_proj.weight" in index:
        shared = {}
        for proj, part in PART_KEYS:
            name = f"{base}.shared_expert.{proj}.{part}"
            want = layout.shape(proj, part)
            if index.shape(name) != want:
                raise ValueError(f"{name}: shape {index.shape(name)}, expected {want}")
            shared[f"{proj}.{part}"] = index.array(name)
    sg = f"{base}.shared_expert_gate.weight"
    shared_gate_w = index.array(sg).reshape(-1) if sg in index else None
    return CheckpointLayer(layer, layout, experts, parts, router_w, shared, shared_gate_w)


def record_images(ckpt: CheckpointLayer, experts: Sequence[int]) -> np.ndarray:
    """uint8 ``[len(experts), record_stride]``: each row one expert's record
    (the nine parts at their layout offsets, zero padding to the stride)."""
    lay = ckpt.layout
    out = np.zeros((len(experts), lay.record_stride), dtype=np.uint8)
    sel = list(experts)
    for proj, part in PART_KEYS:
        data = np.ascontiguousarray(ckpt.parts[f"{proj}.{part}"][sel]).view(np.uint8).reshape(len(sel), -1)
        off = lay.offset(proj, part)
        out[:, off:off + data.shape[1]] = data
    return out


def load_pool(ckpt: CheckpointLayer, device="cuda", *, slots: Optional[int] = None,
              slot_of_expert: Optional[Sequence[int]] = None, chunk: int = 64):
    """A device slot pool holding every expert of the layer.

    Returns ``(pool, slot_table)``: pool is uint8 ``[HEADER + slots * stride]``
    and ``slot_table[e]`` (int32) the slot of expert ``e`` (identity unless
    ``slot_of_expert`` is given).  Records are staged ``chunk`` experts at a
    time, so host memory stays bounded by ``chunk`` records.
    """
    import torch

    lay = ckpt.layout
    slots = ckpt.experts if slots is None else int(slots)
    table = np.arange(ckpt.experts, dtype=np.int32) if slot_of_expert is None else \
        np.asarray(slot_of_expert, dtype=np.int32)
    if table.shape != (ckpt.experts,) or table.min() < 0 or table.max() >= slots or \
            len(np.unique(table)) != ckpt.experts:
        raise ValueError("slot_of_expert must map the experts to distinct slots below `slots`")
    pool = torch.zeros(HEADER_SIZE + slots * lay.record_stride, dtype=torch.uint8, device=device)
    records = pool[HEADER_SIZE:].view(slots, lay.record_stride)
    for start in range(0, ckpt.experts, chunk):
        sel = list(range(start, min(start + chunk, ckpt.experts)))
        imgs = torch.from_numpy(record_images(ckpt, sel))
        records[torch.from_numpy(table[sel]).long().to(records.device)] = imgs.to(records.device)
    return pool, torch.from_numpy(table).to(device)


def layer_weights(ckpt: CheckpointLayer, device="cuda", *, slots: Optional[int] = None,
                  slot_of_expert: Optional[Sequence[int]] = None):
    """:class:`~.moe_block.LayerWeights` for a :class:`~.moe_block.DecodeLayer`:
    the experts in a device slot pool, the router, the shared expert and its gate."""
    import torch

    from .moe_block import LayerWeights

    if ckpt.router_w is None:
        raise ValueError(f"layer {ckpt.layer} has no router weight (mlp.gate.weight)")
    pool, table = load_pool(ckpt, device, slots=slots, slot_of_expert=slot_of_expert)

    def bf16(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(torch.bfloat16)

    shared = None
    if ckpt.shared is not None:
        shared = tuple(
            (torch.from_numpy(np.ascontiguousarray(ckpt.shared[f"{p}.weight"]).view(np.int32)[None]).to(device),
             bf16(ckpt.shared[f"{p}.scales"][None]), bf16(ckpt.shared[f"{p}.biases"][None]))
            for p in PROJECTIONS)
    sg = bf16(ckpt.shared_gate_w) if ckpt.shared_gate_w is not None and shared is not None else None
    return LayerWeights(ckpt.layout, pool, table, bf16(ckpt.router_w), sg, shared)


def fill_record_store(ckpt: CheckpointLayer, store, experts: Optional[Iterable[int]] = None) -> None:
    """Adds the layer's records to a :class:`~.pool.HostRecordStore` (pinned
    host images for the LRU hot pool's refills)."""
    import torch

    if store.layout != ckpt.layout:
        raise ValueError("record store layout differs from the checkpoint layer's")
    sel = list(range(ckpt.experts)) if experts is None else [int(e) for e in experts]
    for e in sel:
        parts = {f"{proj}.{part}": torch.from_numpy(np.ascontiguousarray(ckpt.parts[f"{proj}.{part}"][e]).view(np.uint8))
                 for proj, part in PART_KEYS}
        store.add(ckpt.layer, e, parts)
