"""A decode layer built from a safetensors checkpoint matches the oracle.

The checkpoint is written with the model's tensor names (two layers, g32 at
hidden 2048 / inter 512 and g64 at the 2560 / 640 shape), read back by
``flashnext_hip.checkpoint`` into a permuted HBM slot pool, and run through
the routed layer; routes are bit-exact against ``oracle.router.route`` and the
output within the bf16 tolerance of ``oracle.moe.decode_layer``.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, moe, router as orouter

from ._helpers import assert_close, from_dev_bf16, say, to_dev_bf16, write_moe_checkpoint, bf16_normal

pytestmark = pytest.mark.gpu

E = 16


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch


@pytest.mark.parametrize("hidden,inter,group", [(2048, 512, 32), (2560, 640, 64)])
def test_decode_layer_from_checkpoint_matches_oracle(torch_mod, tmp_path, hidden, inter, group):
    torch = torch_mod
    say(f"case: checkpoint layer hidden={hidden} inter={inter} group={group}")
    from flashnext_hip import _lib
    from flashnext_hip.checkpoint import SafeTensorIndex, layer_weights, read_layer
    from flashnext_hip.moe_block import DecodeLayer

    written = write_moe_checkpoint(str(tmp_path), 1, experts=E, hidden=hidden, inter=inter, groups=(group,),
                                   seed=400 + group)
    ck = read_layer(SafeTensorIndex(str(tmp_path)), 0)
    assert ck.layout.group_size == group
    perm = np.random.default_rng(401).permutation(24)[:E].astype(np.int32)
    weights = layer_weights(ck, "cuda", slots=24, slot_of_expert=perm)
    tokens, top_k = 2, 10
    layer = DecodeLayer(weights, tokens, top_k)
    x = bf16_normal((tokens, hidden), seed=402)
    layer.x.copy_(to_dev_bf16(x))
    layer.launch(None)
    torch.cuda.synchronize()
    assert _lib.check_device_errors() == 0
    t = written[0]["tensors"]
    wg = t["language_model.model.layers.0.mlp.gate.weight"][1]
    wsg = t["language_model.model.layers.0.mlp.shared_expert_gate.weight"][1]
    ref = orouter.route(x, wg, top_k, slot_table=perm.astype(np.uint32))
    assert np.array_equal(layer.inds.cpu().numpy().astype(np.uint32), ref["inds"])
    assert np.array_equal(layer.routes.cpu().numpy().view(np.uint32), ref["routes"])
    recs, sh = written[0]["records"], written[0]["shared"]
    rs = moe.ExpertRecordSet(recs.gate, recs.up, recs.down, shared=(sh.gate, sh.up, sh.down))
    # Group 64 combines in the reference's generic order (bf16 products, metal_runtime.py:908-929).
    want = moe.decode_layer(x, ref["inds"], ref["scores"], rs, score_dtype="bf16", shared_gate_weight=wsg,
                            combine="generic" if group == 64 else "fused")
    assert_close(bf16.bf16_to_f32(from_dev_bf16(layer.out)), bf16.bf16_to_f32(want), f"checkpoint g{group}")


def test_record_store_images_equal_checkpoint_records(torch_mod, tmp_path):
    say("case: host record store filled from a checkpoint")
    from flashnext_hip.checkpoint import SafeTensorIndex, fill_record_store, read_layer, record_images
    from flashnext_hip.pool import HostRecordStore

    write_moe_checkpoint(str(tmp_path), 1, experts=4, hidden=512, inter=256, groups=(32,), seed=410)
    ck = read_layer(SafeTensorIndex(str(tmp_path)), 0)
    store = HostRecordStore(ck.layout)
    fill_record_store(ck, store, experts=[2, 0])
    imgs = record_images(ck, [2, 0])
    assert np.array_equal(store.record(0, 2).numpy(), imgs[0])
    assert np.array_equal(store.record(0, 0).numpy(), imgs[1])
