"""CPU oracle for the Flash-Next quantized MoE expert path (test infrastructure).

This package restates, on the CPU, the semantics of the reference's Q4/g32
MoE expert path so the HIP kernels can be checked against it.  It is NOT part
of the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the timed CPU baseline.  The product path never calls into it.

Modules (each function cites the reference file:line it restates):

* ``bf16``    bfloat16 bit helpers (round-to-nearest-even, exact f64 rounding)
* ``q4``      uint32 nibble packing/unpacking, affine dequant, QMV, gather_qmm
* ``router``  softmax(precise) / top-k / renorm / adaptive keep / slot words
* ``moe``     SwiGLU bf16 sequence, fused down+combine rounding, decode layer,
              generic (prefill) combine
* ``pool``    record layout (generalised to any hidden/intermediate/group) and
              the LRU slot assignment of the expert pool
* ``c/``      a C restatement of the QMV and decode layer, used as the timed
              CPU baseline and cross-checked against the numpy restatement

Pinning status of every function is listed in ``PINNING`` below and in the
project's design notes; each is checked by tests under ``tests/`` against the
reference's own known-answer tests, closed forms or brute force.
"""

PINNING = {
    "bf16.f32_to_bf16": "closed form: RNE on hand-picked bit patterns incl. ties and NaN",
    "bf16.f64_to_bf16": "brute force vs exact rational rounding (fractions) on random + tie inputs",
    "q4.pack_q4/unpack_q4": "reference packing loop test_metal_runtime_g64.py:16-26; round trip; hand KAT",
    "q4.qmv": "closed form (scales=1,biases=0 integer dot; affine linearity) + brute force vs fractions",
    "q4.gather_qmm": "closed form (scales=1, biases=0 integer dots per row's own expert) + row-permutation "
                     "equivariance; rows are q4.ExpertBank.project, whose weights are pinned below",
    "router.softmax_topk": "brute force sort on tiny inputs; tie order; closed-form softmax values",
    "router.renorm": "closed form bf16 arithmetic on hand-computed cases",
    "router.keep_for_mass": "hand KAT of adaptive_topk.py:43-50 semantics",
    "router.slot_words": "reference KAT test_metal_slab.py:17-25 (0x80000000|5)",
    "moe.swiglu_bf16": "hand-computed closed-form KATs on the reference's representative bits "
                       "(test_swiglu_contract.py:21-31) + fp32 variant differs (test_swiglu_contract.py:33-45)",
    "moe.weighted_combine": "reference KAT test_metal_runtime.py:222-263 ([[25.75,51.5],[192,256]])",
    "moe.down_combine": "closed form on exactly representable values; slot-order invariance on exact sums",
    "pool.record_layout": "reference constants test_slab_pack.py:50-63 (3,072,000 stride and offsets)",
    "pool.LruSlots": "reference KAT test_expert_pool.py:32-49 (hits 4, misses 18, evicted slot0/slot1)",
    "router.router_logits": "closed form: integer-valued bf16 inputs give exact dot products, rounded once",
    "router.adaptive_keep/pad_dropped": "hand KAT of adaptive_topk.py:43-50, 213-227 (keep, padding, width)",
    "moe.generic_combine": "closed form on exactly representable values (bf16 products, slot-order f32 sum)",
    "q4.ExpertBank.dense_bf16": "closed form: equals bf16(float32(exact dequant)); within half a bf16 ulp",
    "moe.decode_layer / moe.prefill_layer": "compositions of the pinned parts above; decode_layer "
                                            "cross-checked against the independent C restatement",
    "c.mqo_decode_layer / c.mqo_qmv": "cross-checked against the numpy restatement (tests/test_oracle_c.py)",
}
# Functions whose values only MLX itself could fix (parity unpinned at the MLX
# boundary): MLX's own qmv/gather_qmm fp32 reduction order and bf16 output
# bits, argpartition tie order, softmax(precise=True) last-ulp behaviour and
# the bf16 rounding inside mx.exp.  The oracle fixes these as exact rounding
# (float64 accumulation rounded once; correctly rounded exp; ties to the lower
# expert index).
