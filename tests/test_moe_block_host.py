"""Host-side argument checks of ``MoEBlock`` (``_moe_call`` composition); no device work."""
from __future__ import annotations

import pytest


def test_moe_block_validates_arguments_before_device_work():
    import torch

    from flashnext_hip.layout import make_layout
    from flashnext_hip.moe_block import LayerWeights, MoEBlock

    lay = make_layout(256, 128)
    pool = torch.zeros(4096 + 4 * lay.record_stride, dtype=torch.uint8)
    w = LayerWeights(lay, pool, torch.arange(4, dtype=torch.int32), torch.zeros((4, 256), dtype=torch.bfloat16),
                     None, None)
    with pytest.raises(ValueError):
        MoEBlock(w, 2, fused_max_tokens=9)
    with pytest.raises(ValueError):
        MoEBlock(w, 2, routed_max_tokens=65)
    with pytest.raises(ValueError):
        MoEBlock(w, 2, fused_max_tokens=8, routed_max_tokens=5)
    assert MoEBlock(w, 2, routed_max_tokens=0).routed_max_tokens == 0
    block = MoEBlock(w, 2)
    with pytest.raises(ValueError):
        block(torch.zeros((3, 128), dtype=torch.bfloat16))   # wrong width
    with pytest.raises(ValueError):
        block(torch.zeros((3, 256), dtype=torch.float32))    # wrong dtype
    with pytest.raises(ValueError):
        block(torch.zeros((0, 256), dtype=torch.bfloat16))   # no tokens
