"""Checkpoint reader: safetensors parsing, quantisation inference and pool
records (CPU).

The record bytes are checked against the oracle's record layout
(``oracle.pool.record_layout``, which restates slab_pack.py:96-149) and the
quantisation inference against the closed form of
``models/flashnext/loader.py:360-382`` on g32, g64 and inconsistent shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import pool as opool

from ._helpers import write_moe_checkpoint, write_safetensors

E, H, I = 6, 256, 128


@pytest.fixture(scope="module")
def ckpt_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    written = write_moe_checkpoint(str(d), 2, experts=E, hidden=H, inter=I, groups=(32, 64), seed=300)
    return str(d), written


def test_index_reads_shapes_dtypes_and_data(ckpt_dir):
    from flashnext_hip.checkpoint import SafeTensorIndex

    d, written = ckpt_dir
    idx = SafeTensorIndex(d)
    for layer in (0, 1):
        for name, (dtype, arr) in written[layer]["tensors"].items():
            assert idx.shape(name) == arr.shape
            assert idx.dtype(name) == dtype
            assert np.array_equal(np.asarray(idx.array(name)).view(arr.dtype), arr)
    name = "language_model.model.layers.0.mlp.switch_mlp.up_proj.scales"
    assert np.array_equal(idx.rows(name, [4, 1]), written[0]["tensors"][name][1][[4, 1]])


def test_infer_switch_quantization(ckpt_dir, tmp_path):
    from flashnext_hip.checkpoint import SafeTensorIndex, infer_switch_quantization

    d, _ = ckpt_dir
    idx = SafeTensorIndex(d)
    assert infer_switch_quantization(idx, "language_model.model.layers.0.mlp.switch_mlp") == (32, 4)
    assert infer_switch_quantization(idx, "language_model.model.layers.1.mlp.switch_mlp") == (64, 4)
    # 8-bit packing of the same widths: 64 words per 256 inputs
    p = "language_model.model.layers.0.mlp.switch_mlp"
    tensors = {
        f"{p}.gate_proj.weight": ("U32", np.zeros((2, 8, 64), np.uint32)),
        f"{p}.gate_proj.scales": ("BF16", np.zeros((2, 8, 8), np.uint16)),
        f"{p}.down_proj.weight": ("U32", np.zeros((2, 256, 2), np.uint32)),
    }
    write_safetensors(str(tmp_path / "model.safetensors"), tensors)
    assert infer_switch_quantization(SafeTensorIndex(str(tmp_path)), p) == (32, 8)
    # packed bits that do not divide the input width
    bad = dict(tensors)
    bad[f"{p}.gate_proj.weight"] = ("U32", np.zeros((2, 8, 63), np.uint32))
    write_safetensors(str(tmp_path / "model.safetensors"), bad)
    with pytest.raises(ValueError, match="incompatible"):
        infer_switch_quantization(SafeTensorIndex(str(tmp_path)), p)


def test_record_images_match_the_record_layout(ckpt_dir):
    from flashnext_hip.checkpoint import SafeTensorIndex, read_layer, record_images

    d, written = ckpt_dir
    idx = SafeTensorIndex(d)
    for layer, group in ((0, 32), (1, 64)):
        ck = read_layer(idx, layer)
        offsets, stride, sizes = opool.record_layout(H, I, group)
        assert ck.layout.record_stride == stride and ck.experts == E
        imgs = record_images(ck, [3, 0, 5])
        assert imgs.shape == (3, stride)
        recs = written[layer]["records"]
        for row, e in enumerate((3, 0, 5)):
            for proj, bank in (("gate_proj", recs.gate), ("up_proj", recs.up), ("down_proj", recs.down)):
                for part, arr in (("weight", bank.packed), ("scales", bank.scales), ("biases", bank.biases)):
                    key = f"{proj}.{part}"
                    got = imgs[row, offsets[key]:offsets[key] + sizes[key]]
                    assert np.array_equal(got, np.ascontiguousarray(arr[e]).view(np.uint8).reshape(-1)), (layer, e, key)
            end = max(offsets[k] + sizes[k] for k in offsets)
            assert not imgs[row, end:].any()


def test_load_pool_places_records_at_their_slots(ckpt_dir):
    from flashnext_hip.checkpoint import SafeTensorIndex, load_pool, read_layer, record_images
    from flashnext_hip.layout import HEADER_SIZE

    d, _ = ckpt_dir
    ck = read_layer(SafeTensorIndex(d), 0)
    perm = [7, 2, 0, 5, 1, 6]
    pool, table = load_pool(ck, "cpu", slots=8, slot_of_expert=perm, chunk=4)
    stride = ck.layout.record_stride
    assert pool.numel() == HEADER_SIZE + 8 * stride
    imgs = record_images(ck, range(E))
    host = pool.numpy()
    assert not host[:HEADER_SIZE].any()
    for e, slot in enumerate(perm):
        assert np.array_equal(host[HEADER_SIZE + slot * stride:HEADER_SIZE + (slot + 1) * stride], imgs[e])
    for slot in set(range(8)) - set(perm):
        assert not host[HEADER_SIZE + slot * stride:HEADER_SIZE + (slot + 1) * stride].any()
    assert table.tolist() == perm
    with pytest.raises(ValueError):
        load_pool(ck, "cpu", slots=4, slot_of_expert=perm)


def test_read_layer_rejects_other_bit_widths(tmp_path):
    from flashnext_hip.checkpoint import SafeTensorIndex, read_layer

    p = "language_model.model.layers.0.mlp.switch_mlp"
    tensors = {}
    for proj, (o, i) in (("gate_proj", (8, 256)), ("up_proj", (8, 256)), ("down_proj", (256, 8))):
        tensors[f"{p}.{proj}.weight"] = ("U32", np.zeros((2, o, i // 4), np.uint32))  # 8-bit
        tensors[f"{p}.{proj}.scales"] = ("BF16", np.zeros((2, o, max(i // 32, 1)), np.uint16))
        tensors[f"{p}.{proj}.biases"] = ("BF16", np.zeros((2, o, max(i // 32, 1)), np.uint16))
    write_safetensors(str(tmp_path / "model.safetensors"), tensors)
    with pytest.raises(ValueError, match="4-bit"):
        read_layer(SafeTensorIndex(str(tmp_path)), 0)

