"""GPU checks of the measurement entry points (`mq_stream_probe`, `mq_hop_probe`,
`mq_mfma_probe`): each runs on the device, reads only what it is given, and
returns what its header comment promises, so the floors and ceilings that
bench.py reports come from kernels that did the stated work."""
from __future__ import annotations

import numpy as np
import pytest

from ._helpers import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    from flashnext_hip import _lib

    lib = _lib.load()
    assert lib.mq_available() == 1, _lib.last_error(lib)
    return torch, _lib, lib


def test_stream_probe_reads_segments_and_keeps_the_sink(env):
    torch, _lib, lib = env
    say("case: stream probe, 11 zero segments of 64 KiB, 44 blocks, and the empty launch")
    n, each = 11, 64 << 10
    buf = torch.zeros(n * each, dtype=torch.uint8, device="cuda")
    segs = torch.tensor([buf.data_ptr() + i * each for i in range(n)], dtype=torch.int64, device="cuda")
    sink = torch.full((1,), 0x1234567, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.mq_stream_probe(segs.data_ptr(), n, each, 4 * n, sink.data_ptr(), stream), lib)
    _lib.check(lib.mq_stream_probe(None, 0, 0, 0, sink.data_ptr(), stream), lib)  # the empty kernel
    torch.cuda.synchronize()
    # zero segments fold to checksum 0, which never equals the probe's sentinel
    assert int(sink.item()) == 0x1234567


@pytest.mark.parametrize("block,hops", [(0, 1), (1, 4), (5, 8)])
def test_hop_probe_follows_the_chain(env, block, hops):
    torch, _lib, lib = env
    say(f"case: hop probe block={block} hops={hops}")
    stride = 4096 // 8  # links 4 KiB apart
    links = torch.zeros(9 * stride, dtype=torch.int64, device="cuda")
    base = links.data_ptr()
    addrs = [base + i * stride * 8 for i in range(9)]
    host = np.zeros(9 * stride, dtype=np.int64)
    for i in range(8):
        host[i * stride] = addrs[i + 1]
    links.copy_(torch.from_numpy(host))
    stamps = torch.zeros(10, dtype=torch.int64, device="cuda")
    _lib.check(lib.mq_hop_probe(addrs[0], hops, stamps.data_ptr(), block,
                                torch.cuda.current_stream().cuda_stream), lib)
    torch.cuda.synchronize()
    st = stamps.cpu().numpy().astype(np.uint64)
    assert int(st[9]) == addrs[hops], "the probe must end on the link after `hops` dereferences"
    clock = st[:9]
    assert np.all(np.diff(clock.astype(np.int64)) >= 0), clock
    assert np.all(clock[hops + 1:] == clock[hops]), "unused stamps repeat the last one"


def test_mfma_probe_accumulates_linearly(env):
    torch, _lib, lib = env
    say("case: mfma probe, 8 blocks, 1/2/4 rounds")
    blocks = 8
    stream = torch.cuda.current_stream().cuda_stream
    sums = {}
    for iters in (1, 2, 4):
        sink = torch.zeros(blocks * 512, dtype=torch.float32, device="cuda")
        _lib.check(lib.mq_mfma_probe(iters, blocks, sink.data_ptr(), stream), lib)
        torch.cuda.synchronize()
        sums[iters] = sink.cpu().numpy().astype(np.float64)
    s1 = sums[1]
    assert np.all(np.isfinite(s1)) and np.count_nonzero(s1) > 0.9 * s1.size
    # every round adds the same products, so the sums grow linearly with the rounds
    np.testing.assert_allclose(sums[2], 2 * s1, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(sums[4], 4 * s1, rtol=1e-5, atol=1e-6)
    # every block computes the same values
    per_block = s1.reshape(blocks, 512)
    assert np.array_equal(per_block, np.broadcast_to(per_block[0], per_block.shape))
