#!/usr/bin/env python3
"""Benchmark of the gfx950 Flash-Next MoE decode layer.

Workload (one "step"): one MoE decode layer for one token -- hidden 2048,
512 routed experts (top-10) plus one shared expert, intermediate 512, affine
Q4 with group 32 and bf16 metadata -- i.e. router GEMV + softmax/top-10/
renorm + slot lookup, then gate/up -> SwiGLU -> down for the 10 routed
experts and the shared expert, combined with the router scores.  To keep the
expert bytes coming from HBM rather than the 256 MB last-level cache, the
benchmark holds 48 distinct layers (~48 GB of expert records in the HBM slot
pool) and steps through them in turn, each with its own fresh N(0,1) token.

Prints one JSON line.  ``value`` is microseconds per token-layer (lower is
better); ``hbm_gbps`` is the algorithmic expert bytes (11 x 1,966,080) per
layer divided by the step time.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "macqwen-releases_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
HIDDEN, INTER, EXPERTS, TOP_K, GROUP = 2048, 512, 512, 10, 32


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes_per_record(hidden=HIDDEN, inter=INTER, group=GROUP) -> int:
    # packed q + bf16 scales + bf16 biases for gate, up (inter x hidden) and down (hidden x inter)
    per_proj = inter * hidden // 2 + 2 * 2 * inter * hidden // group
    return 3 * per_proj


def build_layers(n_layers: int, device, seed: int = 1234):
    from flashnext_hip.moe_block import DecodeLayer, LayerWeights
    from flashnext_hip.synthetic import make_layer

    runners, layers = [], []
    for l in range(n_layers):
        lay = make_layer(HIDDEN, INTER, EXPERTS, seed + l, device=device, group=GROUP, keep_dense=(l == 0))
        w = LayerWeights(lay.layout, lay.pool, lay.slot_table, lay.router_w, lay.shared_gate_w,
                         tuple(b.as_tuple() for b in lay.shared))
        runners.append(DecodeLayer(w, 1, TOP_K, device=device))
        layers.append(lay)
        if (l + 1) % 8 == 0:
            log(f"built {l + 1}/{n_layers} layers")
    return layers, runners


def time_graph(torch, graph, replays: int, stream) -> float:
    """Milliseconds for `replays` launches of `graph` on `stream` (events on the same stream)."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):  # CUDAGraph.replay() launches on the current stream
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def capture(torch, fn, stream):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def check_layer0(torch, layer, runner) -> dict:
    """Compare the GPU output of layer 0 for its current token with the oracle."""
    import numpy as np

    from oracle import bf16, moe, q4, router as orouter

    x = runner.x.view(torch.int16).cpu().numpy().view(np.uint16)
    wg = layer.router_w.view(torch.int16).cpu().numpy().view(np.uint16)
    wsg = layer.shared_gate_w.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = orouter.route(x, wg, TOP_K)
    inds_gpu = runner.inds.cpu().numpy().astype(np.uint32)
    experts = sorted(set(ref["inds"].reshape(-1).tolist()))

    def host_bank(dense_bank, sel):
        w = dense_bank.weight[sel].cpu().numpy().view(np.uint32)
        s = dense_bank.scales[sel].view(torch.int16).cpu().numpy().view(np.uint16)
        b = dense_bank.biases[sel].view(torch.int16).cpu().numpy().view(np.uint16)
        return q4.ExpertBank(w, s, b, GROUP)

    sel = torch.tensor(experts, device=layer.dense[0].weight.device)
    remap = {e: i for i, e in enumerate(experts)}
    recs = moe.ExpertRecordSet(*(host_bank(b, sel) for b in layer.dense),
                               shared=tuple(host_bank(b, torch.tensor([0], device=sel.device)) for b in layer.shared))
    local = np.vectorize(remap.get)(ref["inds"])
    want = bf16.bf16_to_f32(moe.decode_layer(x, local, ref["scores"], recs, score_dtype="bf16",
                                             shared_gate_weight=wsg))
    got = bf16.bf16_to_f32(runner.out.view(torch.int16).cpu().numpy().view(np.uint16))
    diff = np.abs(got.astype(np.float64) - want)
    return {"inds_exact": bool(np.array_equal(inds_gpu, ref["inds"])),
            "max_rel": float(diff.max() / np.abs(want).max()),
            "cosine": float(np.dot(got.ravel(), want.ravel()) / (np.linalg.norm(got) * np.linalg.norm(want)))}


def cpu_baseline(torch, layer, seconds: float) -> dict:
    """Time the oracle's C restatement (OpenMP) of the same decode layer on host cores."""
    import numpy as np

    from oracle import cbase, moe, q4

    threads = min(16, len(os.sched_getaffinity(0)))

    def host_bank(b):
        return q4.ExpertBank(b.weight.cpu().numpy().view(np.uint32), b.scales.view(torch.int16).cpu().numpy().view(np.uint16),
                             b.biases.view(torch.int16).cpu().numpy().view(np.uint16), GROUP)

    recs = moe.ExpertRecordSet(*(host_bank(b) for b in layer.dense))
    shared = tuple(host_bank(b) for b in layer.shared)
    wg = layer.router_w.view(torch.int16).cpu().numpy().view(np.uint16)
    wsg = layer.shared_gate_w.view(torch.int16).cpu().numpy().view(np.uint16)
    rng = np.random.default_rng(7)
    from oracle import bf16

    xs = bf16.f32_to_bf16(rng.normal(0, 1, (256, 1, HIDDEN)).astype(np.float32))
    cbase.decode_layer(xs[0], wg, recs, TOP_K, shared=shared, shared_gate_w=wsg, threads=threads)  # warm
    n, t0 = 0, time.perf_counter()
    while n < xs.shape[0]:
        cbase.decode_layer(xs[n], wg, recs, TOP_K, shared=shared, shared_gate_w=wsg, threads=threads)
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    elapsed = time.perf_counter() - t0
    return {"value": round(elapsed / n * 1e6, 1), "unit": "us/token", "cores": threads, "kind": "port",
            "sample": f"{n} decode tokens of one layer (router + 10 routed + shared experts), "
                      f"C restatement with OpenMP; MLX CPU unavailable on this host"}


def zipf_routes(tokens: int, experts: int, k: int, seed: int, skew: float = 1.1):
    """Per-token top-k distinct experts drawn without replacement with Zipf(skew)
    weights (Gumbel top-k): expert row counts follow the Zipf profile, capped
    by one row per token per expert."""
    import numpy as np

    rng = np.random.default_rng(seed)
    logp = -skew * np.log(np.arange(1, experts + 1, dtype=np.float64))
    keys = logp[None, :] + rng.gumbel(size=(tokens, experts))
    return np.argsort(-keys, axis=1)[:, :k].astype(np.int32)


def prefill_bench(torch, dev, reps: int = 24, warm: int = 48, layers: int = 4) -> dict:
    """4096-token prefill chunk through the grouped path (sort + grouped
    gate/up/SwiGLU/down MFMA GEMMs + combine), routed experts only.

    The chunk runs through `layers` distinct expert banks in turn (about
    1 GB of Q4 weights each, so no call finds the weights of its layer in
    the 256 MB last-level cache from the call before), as the layers of a
    long prompt's chunks do.  `warm` untimed calls (about 30 ms of back-to-
    back chunks) precede the `reps` timed ones: after two calls alone the
    same chunk measures about 15% slower while the clocks ramp up."""
    from flashnext_hip.grouped import GroupedMoE
    from flashnext_hip.synthetic import make_bank

    T = 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(4096)
    stacks = [[make_bank(EXPERTS, o, i, gen, dev, group=GROUP) for (o, i) in ((INTER, HIDDEN), (INTER, HIDDEN),
                                                                               (HIDDEN, INTER))]
              for _ in range(layers)]
    inds = zipf_routes(T, EXPERTS, TOP_K, seed=11)
    x = torch.randn((T, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    scores = torch.full((T, TOP_K), 1.0 / TOP_K, device=dev, dtype=torch.bfloat16)
    routes = torch.from_numpy(inds).to(dev)
    gs = [GroupedMoE(*[b.as_tuple() for b in banks], hidden=HIDDEN, inter=INTER, group_size=GROUP)
          for banks in stacks]
    for i in range(warm):
        gs[i % layers](x, routes, scores)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(reps):
        gs[i % layers](x, routes, scores)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    flops = 2.0 * T * TOP_K * 3 * HIDDEN * INTER
    tflops = flops / (ms * 1e-3) / 1e12
    import numpy as np

    counts = np.bincount(inds.reshape(-1), minlength=EXPERTS)
    out, y = gs[0](x, routes, scores)
    check = prefill_check(torch, stacks[0], x, inds, scores, out, y, counts)
    chain = gather_chain_bench(torch, dev, stacks, x, inds, reps=reps // 2, warm=warm // 2)
    del stacks, gs
    return {"workload": f"{T} tokens x top-{TOP_K}, {EXPERTS} experts, Zipf(1.1) rows "
                        f"(max {int(counts.max())}, median {int(np.median(counts))}, min {int(counts.min())}), "
                        f"{layers} layers' expert banks in turn",
            "us": round(ms * 1000, 1), "gflop": round(flops / 1e9, 1), "tflops": round(tflops, 1),
            "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            "note": (f"sort + grouped MFMA GEMMs + bf16 combine timed together over {reps} calls after {warm} "
                     "untimed ones (sustained chunk rate); routed experts only"),
            "check": check, "gather_qmm_chain": chain}


def gather_chain_bench(torch, dev, stacks, x, inds, reps: int, warm: int) -> dict:
    """The reference's per-projection prefill chain on the same chunk, through
    the drop-in op: rows sorted by expert (x[T*k, 1, H]), then gather_qmm for
    gate and up, swiglu, gather_qmm for down (models/flashnext/expert_cache.py:
    1790-1806), each layer's banks in turn.  The sort and row gather happen
    before the timed region, as in the reference's _gather_sort."""
    import numpy as np

    from flashnext_hip import ops

    T = x.shape[0]
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")
    xs = x.index_select(0, torch.from_numpy(order // TOP_K).to(dev)).reshape(T * TOP_K, 1, HIDDEN)
    rhs = torch.from_numpy(flat[order].astype(np.int64)).to(dev)

    def chain(banks):
        gate, up, down = banks
        g = ops.gather_qmm(xs, gate.weight, gate.scales, gate.biases, rhs_indices=rhs, sorted_indices=True)
        u = ops.gather_qmm(xs, up.weight, up.scales, up.biases, rhs_indices=rhs, sorted_indices=True)
        return ops.gather_qmm(ops.swiglu(g, u), down.weight, down.scales, down.biases, rhs_indices=rhs,
                              sorted_indices=True)

    for i in range(warm):
        chain(stacks[i % len(stacks)])
    torch.cuda.synchronize()
    times = []
    for _ in range(3):  # median of three timed blocks
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(reps):
            chain(stacks[i % len(stacks)])
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / reps)
    ms = sorted(times)[1]
    flops = 2.0 * T * TOP_K * 3 * HIDDEN * INTER
    return {"ops": f"3 x ops.gather_qmm (mq_gather_qmm) + ops.swiglu over {T * TOP_K} sorted rows",
            "us": round(ms * 1000, 1), "us_blocks": [round(t * 1000, 1) for t in times],
            "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}


def prefill_check(torch, banks, x, inds, scores, out, y, counts) -> dict:
    """Oracle check of the prefill chunk after timing: every row of the two
    heaviest and two lightest experts, and the combined rows of 16 random
    tokens (bf16-tile weights, the MFMA operands; float64 accumulation)."""
    import numpy as np

    from oracle import bf16, moe, q4

    T = x.shape[0]
    order = np.argsort(counts, kind="stable")
    rng = np.random.default_rng(17)
    tokens = np.sort(rng.choice(T, 16, replace=False))
    inds_np = inds.reshape(T, TOP_K)
    experts = sorted(set(order[-2:].tolist()) | set(order[:2].tolist()) | set(inds_np[tokens].reshape(-1).tolist()))
    sel = torch.tensor(experts, device=x.device)
    host = [q4.ExpertBank(b.weight[sel].cpu().numpy().view(np.uint32),
                          b.scales[sel].view(torch.int16).cpu().numpy().view(np.uint16),
                          b.biases[sel].view(torch.int16).cpu().numpy().view(np.uint16), GROUP) for b in banks]
    remap = {e: i for i, e in enumerate(experts)}
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    xf = bf16.bf16_to_f32(xb)
    yb = y.view(torch.int16).cpu().numpy().view(np.uint16).reshape(T * TOP_K, HIDDEN)
    flat = inds_np.reshape(-1)
    got_rows, want_rows = [], []
    for e in list(order[-2:]) + list(order[:2]):
        rows = np.nonzero(flat == e)[0]
        want_rows.append(moe.expert_mlp(xf[rows // TOP_K], host, remap[int(e)], "bf16", "bf16")[3])
        got_rows.append(yb[rows])
    sub = inds_np[tokens]
    y_want = np.zeros((tokens.size, TOP_K, HIDDEN), dtype=np.uint16)
    for e in np.unique(sub):
        ti, si = np.nonzero(sub == e)
        y_want[ti, si] = moe.expert_mlp(xf[tokens[ti]], host, remap[int(e)], "bf16", "bf16")[3]
    sc = scores.view(torch.int16).cpu().numpy().view(np.uint16)[tokens]
    want_out = bf16.bf16_to_f32(moe.generic_combine(y_want, sc))
    got_out = bf16.bf16_to_f32(out.view(torch.int16).cpu().numpy().view(np.uint16)[tokens])
    got = np.concatenate([bf16.bf16_to_f32(r).ravel() for r in got_rows] + [got_out.ravel()]).astype(np.float64)
    want = np.concatenate([bf16.bf16_to_f32(r).ravel() for r in want_rows] + [want_out.ravel()]).astype(np.float64)
    return {"rows_checked": int(sum(r.shape[0] for r in got_rows)), "tokens_checked": int(tokens.size),
            "max_rel": float(np.abs(got - want).max() / np.abs(want).max()),
            "cosine": float(np.dot(got, want) / (np.linalg.norm(got) * np.linalg.norm(want)))}


def qmv_bench(torch, dev, lib, stream, copies: int = 64, reps: int = 50) -> dict:
    """Single Q4/g32 QMV, x bf16 [1,2048] times W [5120,2048]^T, through
    ``mq_q4_qmv``; ``copies`` distinct weight matrices (about 420 MB) are
    stepped through in a graph so the bytes come from HBM."""
    from flashnext_hip import _lib
    from flashnext_hip.synthetic import make_bank

    out_w, in_w = 5120, HIDDEN
    gen = torch.Generator(device=dev)
    gen.manual_seed(5120)
    bank = make_bank(copies, out_w, in_w, gen, dev, group=GROUP, chunk=8)
    x = torch.randn((1, in_w), generator=gen, device=dev).to(torch.bfloat16)
    y = torch.empty((copies, out_w), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    handle = stream.cuda_stream

    def run():
        for c in range(copies):
            rc = lib.mq_q4_qmv(x.data_ptr(), _lib.MQ_BF16, bank.weight[c].data_ptr(), bank.scales[c].data_ptr(),
                               bank.biases[c].data_ptr(), y[c].data_ptr(), 1, out_w, in_w, GROUP, handle)
            if rc:
                _lib.check(rc, lib)

    with torch.cuda.stream(stream):
        run()
    torch.cuda.synchronize()
    g = capture(torch, run, stream)
    time_graph(torch, g, 3, stream)
    ms = time_graph(torch, g, reps, stream) / (reps * copies)
    nbytes = out_w * in_w // 2 + 2 * 2 * out_w * in_w // GROUP + 2 * in_w + 2 * out_w
    # check one product against a float64 dequantised matmul (bf16 output rounding)
    wq = bank.weight[0].view(torch.int32)
    shifts = 4 * torch.arange(8, device=dev, dtype=torch.int32)
    q = ((wq[..., None] >> shifts) & 15).reshape(out_w, in_w).double()
    s = bank.scales[0].double().repeat_interleave(GROUP, dim=1)
    b = bank.biases[0].double().repeat_interleave(GROUP, dim=1)
    want = ((s * q + b) @ x[0].double())
    got = y[0].double()
    del bank, g
    return {"workload": f"Q4 g{GROUP} QMV [1,{in_w}] x [{out_w},{in_w}]^T, {copies} distinct weight copies in a graph",
            "us": round(ms * 1000, 3), "bytes": nbytes, "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "max_rel": float((got - want).abs().max() / want.abs().max())}


def verify_bench(torch, dev, runners, stream, tokens: int, reps: int = 10) -> dict:
    """Small-batch decode / speculative verify: ``tokens`` independent rows per
    layer over the same rotating layers; bytes are the exact unique routed
    experts of each layer's seeded routes plus the shared expert."""
    from flashnext_hip import _lib
    from flashnext_hip.moe_block import DecodeLayer

    handle = stream.cuda_stream
    gen = torch.Generator(device=dev)
    gen.manual_seed(1000 + tokens)
    rs = []
    for r in runners:
        v = DecodeLayer(r.w, tokens, TOP_K, device=dev)
        v.x.copy_(torch.randn(v.x.shape, generator=gen, device=dev).to(torch.bfloat16))
        rs.append(v)
    def run():
        for v in rs:
            v.launch(handle)

    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        run()
    _lib.check_device_errors(handle)
    unique = [len(set(v.inds.cpu().reshape(-1).tolist())) for v in rs]
    g = capture(torch, run, stream)
    time_graph(torch, g, 2, stream)
    ms = time_graph(torch, g, reps, stream) / (reps * len(rs))
    nbytes = (sum(unique) / len(unique) + 1) * expert_bytes_per_record()
    # Check (untimed): every token row of layer 0, as the graph left it, is
    # bit-identical to the same token through a one-token layer.
    one = DecodeLayer(runners[0].w, 1, TOP_K, device=dev)
    same = 0
    with torch.cuda.stream(stream):
        for t in range(tokens):
            one.x.copy_(rs[0].x[t:t + 1])
            one.launch(handle)
            torch.cuda.synchronize()
            same += int(torch.equal(one.out.view(torch.int16), rs[0].out[t:t + 1].view(torch.int16)))
    del g, rs, one
    return {"tokens": tokens, "path": "mq_moe_layer",
            "us_per_layer": round(ms * 1000, 3), "us_per_token": round(ms * 1000 / tokens, 3),
            "unique_experts_mean": round(sum(unique) / len(unique), 2), "expert_bytes_per_layer": int(nbytes),
            "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "check": {"rows_bit_identical_to_one_token_layers": same, "rows": tokens}}


def stack_bench(torch, dev, runners, stream, steps: int = 128) -> dict:
    """48 stacked MoE blocks, ``steps`` decode steps, each with a fresh N(0,1)
    hidden state per layer written into the layers' inputs before the step."""
    from flashnext_hip import _lib
    from flashnext_hip.moe_block import DecodeLayer

    handle = stream.cuda_stream
    L = len(runners)
    gen = torch.Generator(device=dev)
    gen.manual_seed(128)
    xbuf = torch.zeros((L, 1, HIDDEN), dtype=torch.bfloat16, device=dev)
    xs = torch.randn((steps, L, 1, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    rs = [DecodeLayer(r.w, 1, TOP_K, device=dev, x=xbuf[l]) for l, r in enumerate(runners)]
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for v in rs:
            v.launch(handle)
    _lib.check_device_errors(handle)
    g = capture(torch, lambda: [v.launch(handle) for v in rs], stream)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        xbuf.copy_(xs[0])
        g.replay()  # warm
        start.record(stream)
        for s in range(steps):
            xbuf.copy_(xs[s])
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    nbytes = L * (TOP_K + 1) * expert_bytes_per_record()
    # Check (untimed): the last step's outputs from the graph equal an eager
    # run of the same step, layer by layer, bit for bit.
    graph_out = [v.out.clone() for v in rs]
    with torch.cuda.stream(stream):
        for v in rs:
            v.launch(handle)
    torch.cuda.synchronize()
    same = sum(int(torch.equal(a.view(torch.int16), v.out.view(torch.int16))) for a, v in zip(graph_out, rs))
    del g, rs, graph_out
    return {"workload": f"{L} stacked MoE blocks, {steps} decode steps, fresh N(0,1) hidden per step and layer, "
                        f"{L * EXPERTS} expert records in the HBM pool",
            "us_per_token": round(ms * 1000, 2), "expert_bytes_per_token": nbytes,
            "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "router_bytes_per_token": L * EXPERTS * HIDDEN * 2,
            "check": {"layers_bit_identical_to_eager": same, "layers": L}}


def hotpool_bench(torch, dev, layers, runners, stream, steps: int = 16, warm_steps: int = 2,
                  pool_gb: float = 6.0, copy_engines: int = 4, method: str = "gather") -> dict:
    """The 48-block stack decoded through a 6 GB LRU hot pool: per layer the
    router runs, its experts are assigned slots on the host (hits move to the
    LRU tail, misses evict the head), missed records are copied from pinned
    host memory (`method`: one gather kernel per layer on the compute stream,
    or one hipMemcpyAsync per record over `copy_engines` copy streams), and
    the expert kernels read the pool through slot words.  One host synchronisation per layer (the route hand-off), as in
    the reference's pool pass.  Host images are the 512 records of layer 0,
    shared by every layer (same bytes per copy as distinct images)."""
    import numpy as np

    from flashnext_hip.layout import HEADER_SIZE
    from flashnext_hip.moe_block import DecodeLayer, LayerWeights
    from flashnext_hip.pool import HipExpertPool, HostRecordStore

    handle = stream.cuda_stream
    L = len(runners)
    pool = HipExpertPool(int(pool_gb * 1e9), HIDDEN, INTER, GROUP, device=dev)
    stride = pool.stride
    store = HostRecordStore(pool.layout)
    src = layers[0].pool
    table0 = layers[0].slot_table.cpu().tolist()
    images = []
    for e in range(EXPERTS):
        base = HEADER_SIZE + int(table0[e]) * stride
        img = torch.empty(stride, dtype=torch.uint8, pin_memory=True)
        img.copy_(src[base:base + stride])
        images.append(img)
    for l in range(L):
        for e in range(EXPERTS):
            store._records[(l, e)] = images[e]
    table = torch.zeros(EXPERTS, dtype=torch.int32, device=dev)  # words are rewritten on the host per layer
    dls = []
    for r in runners:
        w = LayerWeights(r.w.layout, pool.buffer, table, r.w.router_w, r.w.shared_gate_w, r.w.shared)
        dls.append(DecodeLayer(w, 1, TOP_K, device=dev))
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    xs = torch.randn((warm_steps + steps, L, 1, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    # The gather kernel runs on the compute stream: the layer's experts wait
    # for it either way, and a side stream would add two cross-stream event
    # waits per layer (11-16 us of host time each, measured) while the GPU
    # idles.  One hipMemcpyAsync per record spreads over the copy engines.
    copies = [torch.cuda.Stream() for _ in range(copy_engines)] if method == "memcpy" else None
    # Pinned staging for the route words, so that their upload queues behind
    # the refill on the compute stream instead of waiting for it on the host.
    routes_host = [torch.empty(dl.routes.shape, dtype=dl.routes.dtype, pin_memory=True) for dl in dls]
    torch.cuda.synchronize()

    def step(s):
        for l, dl in enumerate(dls):
            dl.x.copy_(xs[s, l])
            dl.launch_router(handle)
            inds = dl.inds.cpu()  # the route hand-off (synchronises the stream)
            slots, misses = pool.assign(l, sorted(set(inds.reshape(-1).tolist())))
            pool.fill(l, misses, store, compute_stream=stream, copy_stream=copies, method=method)
            routes_host[l].copy_(HipExpertPool.route_words(slots, inds).view(dl.routes.shape))
            dl.routes.copy_(routes_host[l], non_blocking=True)
            dl.launch_experts(handle)

    with torch.cuda.stream(stream):
        for s in range(warm_steps):
            step(s)
        torch.cuda.synchronize()
        pool.hits = pool.misses = 0
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        wall0 = time.perf_counter()
        start.record(stream)
        for s in range(warm_steps, warm_steps + steps):
            step(s)
        end.record(stream)
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - wall0) * 1e3
    from flashnext_hip import _lib

    _lib.check_device_errors(handle)
    hits_timed, misses_timed = pool.hits, pool.misses
    # Untimed check: one more step in which every layer also runs fully
    # resident on the same token; the hot-pool output must be bit-identical.
    # The resident twin of layer l has layer l's router and shared expert and
    # layer 0's routed experts, like the host images above.
    twins = [DecodeLayer(LayerWeights(r.w.layout, layers[0].pool, layers[0].slot_table, r.w.router_w,
                                      r.w.shared_gate_w, r.w.shared), 1, TOP_K, device=dev) for r in runners]
    identical = 0
    with torch.cuda.stream(stream):
        for l, dl in enumerate(dls):
            twins[l].x.copy_(xs[0, l])
            twins[l].launch(handle)
            dl.x.copy_(xs[0, l])
            dl.launch_router(handle)
            inds = dl.inds.cpu()
            slots, misses = pool.assign(l, sorted(set(inds.reshape(-1).tolist())))
            pool.fill(l, misses, store, compute_stream=stream, copy_stream=copies, method=method)
            dl.routes.copy_(HipExpertPool.route_words(slots, inds).to(dev, non_blocking=False))
            dl.launch_experts(handle)
            torch.cuda.synchronize()
            identical += int(torch.equal(twins[l].out.view(torch.int16), dl.out.view(torch.int16)))
    _lib.check_device_errors(handle)
    ms = start.elapsed_time(end) / steps
    misses = misses_timed / steps
    lookups = (hits_timed + misses_timed) / steps
    miss_bytes = misses * stride
    out = {"workload": f"{L} stacked MoE blocks through a {pool_gb:g} GB LRU hot pool ({pool.slots} slots), "
                       f"{steps} decode steps, fresh N(0,1) hidden per step and layer, misses copied from pinned "
                       + ("host memory by one gather kernel per layer on the compute stream (PCIe reads of the "
                          "mapped records)"
                          if method == "gather" else
                          f"host memory by one hipMemcpyAsync per record on {copy_engines} copy streams"),
           "refill": method,
           "us_per_token": round(ms * 1000, 1), "wall_us_per_token": round(wall_ms * 1000 / steps, 1),
           "slots": pool.slots, "expert_lookups_per_token": round(lookups, 1),
           "misses_per_token": round(misses, 1), "hit_rate": round(1 - misses / lookups, 4),
           "miss_bytes_per_token": int(miss_bytes),
           "h2d_gbps": round(miss_bytes / (ms * 1e-3) / 1e9, 1),
           "check": {"layers_bit_identical_to_resident": identical, "layers": L}}
    del dls, pool, store, images, twins
    return out


def floors_bench(torch, dev, layers, stream, graph_launches: int = 48, replays: int = 20) -> dict:
    """Latency floors of the decode layer on this GPU, each as microseconds per
    launch over HIP graphs of `graph_launches` launches: an empty kernel; 704
    blocks of 256 threads that read next to nothing (the expert kernels' grid); one
    kernel streaming a layer's expert bytes (11 records of 1,966,080 B, no
    compute) from random slots of the 48 layers' pools (a new set per launch,
    so from HBM), from one contiguous region, and from the same 11 records
    every launch (resident in the last-level cache); the gate/up share then
    the down share of the 11 records as two kernels; and a pointer chase of
    eight links 2 MB apart, each chain written by the kernel before it, whose
    first link is the first dependent load after a kernel boundary."""
    import numpy as np

    from flashnext_hip import _lib
    from flashnext_hip.layout import HEADER_SIZE

    lib = _lib.load()
    handle = stream.cuda_stream
    lay0 = layers[0].layout
    stride = lay0.record_stride
    down_off = lay0.offset("down_proj", "weight")
    G, N = graph_launches, TOP_K + 1
    rng = np.random.default_rng(5)
    L = len(layers)
    assert all(lay.pool.numel() >= HEADER_SIZE + EXPERTS * stride for lay in layers)
    bases = [lay.pool.data_ptr() + HEADER_SIZE for lay in layers]
    rec = np.array([[bases[int(l)] + int(s) * stride for l, s in zip(rng.integers(0, L, N), rng.integers(0, EXPERTS, N))]
                    for _ in range(G)], dtype=np.uint64)
    contig = np.array([[bases[k % L] + (k // L) * N * stride] for k in range(G)], dtype=np.uint64)
    assert all((k // L + 1) * N <= EXPERTS for k in range(G))  # the contiguous runs stay inside one pool
    segs = torch.from_numpy(rec.view(np.int64)).to(dev)
    segs_down = torch.from_numpy((rec + np.uint64(down_off)).view(np.int64)).to(dev)
    segs_contig = torch.from_numpy(contig.view(np.int64)).to(dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    blocks = N * 64

    def probe(seg_tensor, k, n, nbytes):
        ptr = ctypes.c_void_p(seg_tensor.data_ptr() + 8 * n * k) if n else None
        _lib.check(lib.mq_stream_probe(ptr, n, nbytes, blocks if n else 1, ctypes.c_void_p(sink.data_ptr()), handle), lib)

    cases = {
        "empty_kernel": lambda: [probe(segs, k, 0, 0) for k in range(G)],
        "dispatch_704_blocks": lambda: [probe(segs, k, N, 16) for k in range(G)],
        "layer_bytes_random_records": lambda: [probe(segs, k, N, stride) for k in range(G)],
        "layer_bytes_contiguous": lambda: [_lib.check(lib.mq_stream_probe(
            ctypes.c_void_p(segs_contig.data_ptr() + 8 * k), 1, N * stride, blocks, ctypes.c_void_p(sink.data_ptr()),
            handle), lib) for k in range(G)],
        "layer_bytes_cache_resident": lambda: [probe(segs, 0, N, stride) for _ in range(G)],
        "gateup_then_down_two_kernels": lambda: [(probe(segs, k, N, down_off), probe(segs_down, k, N, stride - down_off))
                                                 for k in range(G)],
    }
    out = {"workload": f"HIP graphs of {G} launches; 11 records = {N * stride} B per launch",
           "record_bytes": stride}
    with torch.cuda.stream(stream):
        for name, fn in cases.items():
            fn()  # eager run (also checks the arguments)
            torch.cuda.synchronize()
            g = capture(torch, fn, stream)
            time_graph(torch, g, 2, stream)
            us = time_graph(torch, g, replays, stream) * 1000 / (replays * G)
            row = {"us_per_launch": round(us, 3)}
            if name.startswith("layer_bytes"):
                row["tbps"] = round(N * stride / (us * 1e-6) / 1e12, 2)
            out[name] = row
            del g
        # Pointer chase: chain k has 8 links 2 MB apart in its own 16 MB region.
        hops, span = 8, 2 << 20
        buf = torch.zeros(G * hops * span // 8, dtype=torch.int64, device=dev)
        base = buf.data_ptr()
        here = np.arange(G * hops, dtype=np.int64) * span
        last = (np.arange(G * hops) % hops) == hops - 1
        nxt = np.where(last, here, here + span)  # the last value is read, never followed
        assert int(nxt.max()) + 8 <= buf.numel() * 8
        idx = torch.from_numpy(here // 8).to(dev).view(G, hops)
        vals = torch.from_numpy(base + nxt).to(dev).view(G, hops)
        stamps = torch.zeros((G, 10), dtype=torch.int64, device=dev)
        torch.cuda.synchronize()
        chains = {}
        for reader in (0, 1, 5):  # the block of the reading thread: XCD 0 (the writer's, one block), 1, 5

            def chase():  # each chain is written by one kernel and followed by the next, as route words are
                for k in range(G):
                    buf.index_put_((idx[k],), vals[k])
                    _lib.check(lib.mq_hop_probe(ctypes.c_void_p(base + k * hops * span), hops,
                                                ctypes.c_void_p(stamps[k].data_ptr()), reader, handle), lib)
            chase()
            torch.cuda.synchronize()
            g = capture(torch, chase, stream)
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            st = stamps.cpu().numpy()
            d = np.diff(st[:, :hops + 1], axis=1) * 0.01  # 100 MHz ticks -> us
            chains[f"reader_block_{reader}"] = {"first_link_us_median": round(float(np.median(d[:, 0])), 3),
                                                "later_links_us_median": round(float(np.median(d[:, 1:])), 3)}
            del g
        chains["note"] = ("one thread, links 2 MB apart in device memory, each chain written by a one-block "
                          "index_put_ kernel just before and followed right after the kernel boundary by a thread "
                          "of the given block (blocks go to XCDs round-robin); 100 MHz real-time clock")
        out["dependent_load_chain"] = chains
        del buf
    return out


def peaks_bench(torch, dev) -> dict:
    """Measured ceilings on this GPU: a 1 GiB device copy and a bf16 GEMM."""
    a = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(10):
        b.copy_(a)
    end.record()
    torch.cuda.synchronize()
    copy_gbps = 2 * a.numel() * 10 / (start.elapsed_time(end) * 1e-3) / 1e9
    del b
    h = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    d = a[:h.numel()]
    for _ in range(2):
        d.copy_(h, non_blocking=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(10):
        d.copy_(h, non_blocking=True)
    end.record()
    torch.cuda.synchronize()
    h2d_gbps = h.numel() * 10 / (start.elapsed_time(end) * 1e-3) / 1e9
    del a, d, h
    n = 8192
    m1 = torch.randn((n, n), device=dev).to(torch.bfloat16)
    m2 = torch.randn((n, n), device=dev).to(torch.bfloat16)
    for _ in range(3):
        torch.matmul(m1, m2)
    torch.cuda.synchronize()
    start.record()
    for _ in range(20):
        torch.matmul(m1, m2)
    end.record()
    torch.cuda.synchronize()
    tflops = 2 * n ** 3 * 20 / (start.elapsed_time(end) * 1e-3) / 1e12
    del m1, m2
    # Sustained issue rate of the grouped GEMMs' MFMA (v_mfma_f32_32x32x16_bf16,
    # two waves per SIMD, register operands): the practical matrix ceiling.
    from flashnext_hip import _lib
    lib = _lib.load()
    blocks, iters = 256, 20000
    sink = torch.empty(blocks * 512, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.mq_mfma_probe(200, blocks, sink.data_ptr(), stream), lib)
    torch.cuda.synchronize()
    start.record()
    _lib.check(lib.mq_mfma_probe(iters, blocks, sink.data_ptr(), stream), lib)
    end.record()
    torch.cuda.synchronize()
    mfma_tflops = 2.0 * 32 * 32 * 16 * 4 * iters * 8 * blocks / (start.elapsed_time(end) * 1e-3) / 1e12
    del sink
    # Sustained HBM read rate: mq_stream_probe over 2 GiB in 64 segments with
    # 32 blocks of 256 threads each (about eight blocks per CU), and with one
    # block per CU, the grouped GEMMs' occupancy.
    total, n_seg = 2 << 30, 64
    each = total // n_seg
    src = torch.ones(total, dtype=torch.uint8, device=dev)
    segs = torch.tensor([src.data_ptr() + i * each for i in range(n_seg)], dtype=torch.int64, device=dev)
    word = torch.zeros(1, dtype=torch.int32, device=dev)
    read_tbps = {}
    for grid in (2048, 256):
        for _ in range(2):
            _lib.check(lib.mq_stream_probe(segs.data_ptr(), n_seg, each, grid, word.data_ptr(), stream), lib)
        torch.cuda.synchronize()
        start.record()
        for _ in range(5):
            _lib.check(lib.mq_stream_probe(segs.data_ptr(), n_seg, each, grid, word.data_ptr(), stream), lib)
        end.record()
        torch.cuda.synchronize()
        read_tbps[grid] = total * 5 / (start.elapsed_time(end) * 1e-3) / 1e12
    del src, segs
    return {"copy_gbps": round(copy_gbps, 1), "h2d_pinned_gbps": round(h2d_gbps, 1),
            "bf16_gemm_tflops_8192": round(tflops, 1), "bf16_mfma_issue_tflops": round(mfma_tflops, 1),
            "hbm_read_tbps": round(read_tbps[2048], 2), "hbm_read_tbps_one_block_per_cu": round(read_tbps[256], 2),
            "note": "device-to-device copy counts read + write bytes; host-to-device from 256 MiB of pinned "
                    "memory; GEMM through torch.matmul (hipBLASLt); MFMA issue rate from mq_mfma_probe "
                    "(256 blocks x 8 waves x 80,000 independent v_mfma_f32_32x32x16_bf16 each); HBM read rate "
                    "from mq_stream_probe over 2 GiB (2048 blocks of 256 threads, then 256)"}


def load_traffic(kernel_tag: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    path = ROOT / "profiles" / f"{kernel_tag}_pmc.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            fields = line.split(":", 1)[1].split()
            try:
                return int(float(fields[0]))
            except (IndexError, ValueError):
                return None
    return None


def kernel_rooflines(expert_bytes: int, router_bytes: int):
    """Per-kernel rooflines of the decode layer from the committed rocprofv3
    kernel trace (average duration per launch inside 48-layer graph replays,
    which includes the dispatch gap to the previous kernel): each kernel's
    algorithmic bytes over its duration, against the 8 TB/s peak."""
    path = ROOT / "profiles" / "decode_layer_kernel_stats.md"
    if not path.exists():
        return None
    avg = {}
    for line in path.read_text().splitlines():
        cells = [c.strip().strip("`") for c in line.split("|")[1:-1]]
        if len(cells) == 5 and cells[0].endswith((">", "_kernel")):
            try:
                avg[cells[0]] = float(cells[2])
            except ValueError:
                pass
    gateup_bytes = expert_bytes * 2 // 3  # gate + up parts of each record (two of its three projections)
    rows = [("gateup_kernel, routes given", "gateup_kernel<mq::BF16T, 64, 1, 2, false>", gateup_bytes),
            ("gateup_kernel, selection folded in", "gateup_kernel<mq::BF16T, 64, 1, 2, true>", gateup_bytes),
            ("down_combine_kernel", "down_combine_kernel<mq::BF16T, 16, 1, 3, 2>", expert_bytes - gateup_bytes),
            ("router_logits_kernel", "router_logits_kernel", router_bytes)]
    out = []
    for label, name, nbytes in rows:
        us = avg.get(name)
        if us:
            gbps = nbytes / (us * 1e-6) / 1e9
            out.append({"kernel": label, "bytes": nbytes, "profiled_us": us, "achieved": round(gbps, 1),
                        "frac": round(gbps / HBM_PEAK_GBPS, 4)})
    return {"source": "profiles/decode_layer_kernel_stats.md", "unit": "GB/s", "peak": HBM_PEAK_GBPS,
            "kernels": out} if out else None


def pmc_pass(torch, runners, stream, handle, copy_mb: int = 256) -> None:
    """Eager launches for `rocprofv3 --pmc`: a plain device copy of known size
    (the counter calibration) and the expert stage of every layer."""
    a = torch.empty(copy_mb << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for r in runners:
            r.launch_experts(handle)
    torch.cuda.synchronize()
    log(f"pmc pass: {copy_mb} MiB copy x3 and {len(runners)} expert-stage launches")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4800)
    ap.add_argument("--warmup", type=int, default=480)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the QMV / verify / stack / peak rows")
    ap.add_argument("--pmc-pass", action="store_true", help="eager launches for rocprofv3 --pmc, no timing")
    ap.add_argument("--prefill-only", action="store_true", help="time only the 4096-token prefill grouped path")
    ap.add_argument("--verify-only", action="store_true", help="time only the 4- and 16-token verify layers")
    ap.add_argument("--hotpool-only", action="store_true", help="time only the 6 GB hot-pool stack")
    ap.add_argument("--floors-only", action="store_true", help="time only the decode latency floors")
    ap.add_argument("--peaks-only", action="store_true", help="time only the measured ceilings")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the expert-parallel "
              "sharding across GPUs is a design note, not part of this build", file=sys.stderr)
        return 2

    import torch

    from flashnext_hip import _lib

    lib = _lib.load()
    if not torch.cuda.is_available() or lib.mq_available() != 1:
        print(f"no usable gfx950 device: {_lib.last_error(lib)}", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_bench(torch, dev)}), flush=True)
        return 0
    if args.peaks_only:
        print(json.dumps({"peaks_measured": peaks_bench(torch, dev)}), flush=True)
        return 0
    L = args.layers
    log(f"building {L} layers of {EXPERTS} experts (~{L * EXPERTS * expert_bytes_per_record() / 1e9:.1f} GB pool)")
    layers, runners = build_layers(L, dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    for r in runners:
        r.x.copy_(torch.randn(r.x.shape, generator=gen, device=dev).to(torch.bfloat16))
    # The weights, slot tables and tokens were written on the default stream;
    # the side stream below must not start before they are complete.
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    handle = stream.cuda_stream
    with torch.cuda.stream(stream):
        for r in runners:  # eager pass allocates library scratch before capture
            r.launch(handle)
    _lib.check_device_errors(handle)  # raises if any route word was out of range
    torch.cuda.synchronize()
    if args.pmc_pass:
        pmc_pass(torch, runners, stream, handle)
        return 0
    if args.verify_only:
        print(json.dumps({"verify": [verify_bench(torch, dev, runners, stream, t) for t in (4, 16)]}), flush=True)
        return 0
    if args.floors_only:
        print(json.dumps({"floors": floors_bench(torch, dev, layers, stream)}), flush=True)
        return 0
    if args.hotpool_only:
        runs = [hotpool_bench(torch, dev, layers, runners, stream, method="gather")]
        runs += [hotpool_bench(torch, dev, layers, runners, stream, copy_engines=n, method="memcpy") for n in (1, 4)]
        print(json.dumps({"stack_hot_pool": runs}), flush=True)
        return 0
    log("capturing graphs")
    # Step i decodes one token through layer i mod L.  The timed K steps (and
    # the W warmup steps) are whole graph replays: K // L replays of the
    # L-step graph, then one graph of the first K mod L layer steps.
    g_all = capture(torch, lambda: [r.launch(handle) for r in runners], stream)
    g_exp = capture(torch, lambda: [r.launch_experts(handle) for r in runners], stream)
    g_unf = capture(torch, lambda: [r.launch_unfused(handle) for r in runners], stream)
    tails = {}

    def replay_steps(n):
        full, rem = divmod(n, L)
        for _ in range(full):
            g_all.replay()
        if rem:
            if rem not in tails:
                raise RuntimeError("tail graph not captured")
            tails[rem].replay()

    for n in (args.steps, args.warmup):
        if n % L and n % L not in tails:
            tails[n % L] = capture(torch, lambda m=n % L: [r.launch(handle) for r in runners[:m]], stream)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        replay_steps(args.warmup)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    with torch.cuda.stream(stream):  # replays and events on the same stream
        start.record(stream)
        replay_steps(args.steps)
        end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - wall0) * 1e3
    total_ms = start.elapsed_time(end)
    log(f"timed {args.steps} steps ({args.steps // L} replays of a {L}-step graph + a {args.steps % L}-step graph): "
        f"events {total_ms:.3f} ms, wall {wall_ms:.3f} ms")
    ms_per_step = total_ms / args.steps
    us_per_token = ms_per_step * 1000.0

    reps = max(4, args.steps // L)
    exp_ms = time_graph(torch, g_exp, reps, stream) / (reps * L)
    unf_ms = time_graph(torch, g_unf, reps, stream) / (reps * L)
    expert_bytes = (TOP_K + 1) * expert_bytes_per_record()
    router_bytes = EXPERTS * HIDDEN * 2
    layer_gbps = expert_bytes / (ms_per_step * 1e-3) / 1e9
    exp_gbps = expert_bytes / (exp_ms * 1e-3) / 1e9

    check = check_layer0(torch, layers[0], runners[0])
    log(f"check layer0: {check}")
    extras = {}
    if not args.no_extras:
        log("timing the QMV, small-batch verify and 48-block stack workloads")
        extras["qmv"] = qmv_bench(torch, dev, lib, stream)
        log(f"qmv: {extras['qmv']}")
        extras["verify"] = [verify_bench(torch, dev, runners, stream, t) for t in (4, 16)]
        log(f"verify: {extras['verify']}")
        extras["stack"] = stack_bench(torch, dev, runners, stream)
        log(f"stack: {extras['stack']}")
        extras["stack_hot_pool"] = hotpool_bench(torch, dev, layers, runners, stream, method="gather")
        memcpy = hotpool_bench(torch, dev, layers, runners, stream, method="memcpy")
        extras["stack_hot_pool"]["memcpy_refill"] = {k: memcpy[k] for k in ("workload", "us_per_token", "h2d_gbps",
                                                                            "check")}
        log(f"stack hot pool: {extras['stack_hot_pool']}")
        extras["floors"] = floors_bench(torch, dev, layers, stream)
        log(f"floors: {extras['floors']}")
        extras["peaks_measured"] = peaks_bench(torch, dev)
        log(f"peaks: {extras['peaks_measured']}")
    prefill = None
    if not args.no_prefill:
        log("timing the 4096-token prefill grouped path")
        prefill = prefill_bench(torch, dev)
        peaks = extras.get("peaks_measured")
        if peaks:  # the same rate against what the matrix cores sustain on this box
            prefill["mfma_frac_of_issue_rate"] = round(prefill["tflops"] / peaks["bf16_mfma_issue_tflops"], 4)
        log(f"prefill: {prefill}")
    cpu = None
    if not args.no_cpu:
        log("timing CPU baseline")
        cpu = cpu_baseline(torch, layers[0], args.cpu_seconds)

    line = {
        "metric": "MoE-layer decode us/token (hidden 2048, 512 experts top-10 + shared, Q4 g32)",
        "value": round(us_per_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"decode MoE layer, 1 token, hidden 2048, 512 routed experts top-10 + 1 shared, "
                               f"inter 512, affine Q4 g32 bf16 metadata, {L} distinct layers in an HBM slot pool "
                               f"(random slot permutation); step i runs layer i mod {L}; the {args.steps} timed steps "
                               f"are {args.steps // L} replays of a {L}-step HIP graph plus one {args.steps % L}-step "
                               f"graph",
                   "tokens": 1, "layers_rotated": L, "expert_bytes_per_token": expert_bytes,
                   "router_bytes_per_token": router_bytes},
        "hbm_gbps": round(layer_gbps, 1),
        "hbm_frac": round(layer_gbps / HBM_PEAK_GBPS, 4),
        "breakdown_us": {"layer_fused": round(us_per_token, 3), "layer_unfused": round(unf_ms * 1000, 3),
                         "experts_only": round(exp_ms * 1000, 3)},
        "roofline": {"bound": "hbm",
                     "kernel": "expert stage of the layer (gateup_kernel + down_combine_kernel, 11 experts)",
                     "achieved": round(exp_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(exp_gbps / HBM_PEAK_GBPS, 4), "traffic": load_traffic("decode_expert_stage"),
                     "algorithmic_bytes_per_launch": expert_bytes, "us_per_launch": round(exp_ms * 1000, 3),
                     "per_kernel": kernel_rooflines(expert_bytes, router_bytes)},
        "prefill": prefill,
        **extras,
        "cpu_baseline": cpu,
        "check": check,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
