"""Seeded synthetic MoE layers built on the GPU, in the pool record layout.

Used by the benchmark to build the Flash-Next-shaped decode workload without
checkpoints: weights ~N(0, std) are quantised on the device to affine Q4
(group ``g``: ``bias = min``, ``scale = (max - min) / 15``, bf16 metadata,
``q = round((w - bias) / scale)``) and packed eight nibbles per uint32, LSB
first -- the format of the reference's expert rows.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .layout import HEADER_SIZE, PART_KEYS, SlabLayout, make_layout


def quantize_q4(w: torch.Tensor, group: int = 32):
    """Quantise float weights ``[..., out, in]`` -> (packed int32, bf16 scales, bf16 biases)."""
    shape = w.shape
    g = w.float().reshape(*shape[:-1], shape[-1] // group, group)
    lo = g.amin(dim=-1)
    hi = g.amax(dim=-1)
    scale = ((hi - lo) / 15.0).clamp_min(1e-8).to(torch.bfloat16)
    bias = lo.to(torch.bfloat16)
    q = torch.round((g - bias.float()[..., None]) / scale.float()[..., None]).clamp_(0, 15).to(torch.int64)
    q = q.reshape(*shape[:-1], shape[-1] // 8, 8)
    shifts = (4 * torch.arange(8, device=w.device, dtype=torch.int64))
    words = (q << shifts).sum(dim=-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    return words, scale, bias


@dataclass
class DenseBank:
    weight: torch.Tensor  # int32 [E, out, in/8]
    scales: torch.Tensor  # bf16 [E, out, in/g]
    biases: torch.Tensor

    def as_tuple(self):
        return self.weight, self.scales, self.biases


def make_bank(experts: int, out_w: int, in_w: int, generator: torch.Generator, device, group=32,
              std: float = 0.02, chunk: int = 64) -> DenseBank:
    ws, ss, bs = [], [], []
    for start in range(0, experts, chunk):
        n = min(chunk, experts - start)
        w = torch.randn((n, out_w, in_w), generator=generator, device=device, dtype=torch.float32) * std
        p, s, b = quantize_q4(w, group)
        ws.append(p)
        ss.append(s)
        bs.append(b)
        del w
    return DenseBank(torch.cat(ws), torch.cat(ss), torch.cat(bs))


@dataclass
class SyntheticLayer:
    layout: SlabLayout
    pool: torch.Tensor            # uint8 [HEADER + slots * stride]
    slot_table: torch.Tensor      # int32 [experts] -> slot
    router_w: torch.Tensor        # bf16 [experts, hidden]
    shared_gate_w: torch.Tensor   # bf16 [hidden]
    shared: tuple                 # 3 DenseBank with one expert
    dense: tuple | None           # (gate, up, down) DenseBank, kept when requested


def write_records(pool: torch.Tensor, layout: SlabLayout, banks, slot_of_expert: torch.Tensor,
                  slots: int) -> None:
    """Scatter dense banks into the pool's fixed-stride records at their slots."""
    records = pool[HEADER_SIZE:HEADER_SIZE + slots * layout.record_stride].view(slots, layout.record_stride)
    by_name = dict(zip(("gate_proj", "up_proj", "down_proj"), banks))
    order = slot_of_expert.long()
    for proj, part in PART_KEYS:
        src = getattr(by_name[proj], {"weight": "weight", "scales": "scales", "biases": "biases"}[part])
        flat = src.reshape(src.shape[0], -1)
        nbytes = flat.shape[1] * flat.element_size()
        off = layout.offset(proj, part)
        dst = records[:, off:off + nbytes].view(torch.int32 if part == "weight" else torch.int16)
        dst[order] = flat.view(dst.dtype)


def make_layer(hidden: int, inter: int, experts: int, seed: int, device="cuda", group: int = 32,
               slots: int | None = None, keep_dense: bool = False, permute: bool = True) -> SyntheticLayer:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    layout = make_layout(hidden, inter, group)
    slots = experts if slots is None else slots
    pool = torch.zeros(HEADER_SIZE + slots * layout.record_stride, dtype=torch.uint8, device=device)
    if permute:
        slot_table = torch.randperm(slots, generator=gen, device=device)[:experts].to(torch.int32)
    else:
        slot_table = torch.arange(experts, device=device, dtype=torch.int32)
    gate = make_bank(experts, inter, hidden, gen, device, group)
    up = make_bank(experts, inter, hidden, gen, device, group)
    down = make_bank(experts, hidden, inter, gen, device, group)
    write_records(pool, layout, (gate, up, down), slot_table, slots)
    router_w = (torch.randn((experts, hidden), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    shared_gate_w = (torch.randn((hidden,), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    shared = (make_bank(1, inter, hidden, gen, device, group), make_bank(1, inter, hidden, gen, device, group),
              make_bank(1, hidden, inter, gen, device, group))
    dense = (gate, up, down) if keep_dense else None
    if not keep_dense:
        del gate, up, down
    return SyntheticLayer(layout, pool, slot_table, router_w, shared_gate_w, shared, dense)
