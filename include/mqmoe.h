/*
 * mqmoe.h -- C ABI of the MI355X (gfx950) Flash-Next quantized MoE expert path.
 *
 * Every pointer argument is a caller-owned device pointer unless stated
 * otherwise; every size is in elements unless it says bytes.  Streams and
 * events are passed as opaque pointers (hipStream_t / hipEvent_t; NULL is the
 * default stream).  Functions return 0 on success and a negative MQ_ERR_*
 * code on failure; the message of the last failure on the calling thread is
 * available from mq_last_error().  No function throws across the ABI.
 *
 * Weights use the reference's affine Q4 format: uint32 words holding eight
 * 4-bit values LSB first (value k of a row in word k>>3, bits 4*(k&7)), with
 * bf16 scales and biases per group of `group_size` inputs, w = s*q + b.
 * Activations ("T") are bf16 (MQ_BF16) or float32 (MQ_F32).
 */
#ifndef MQMOE_H
#define MQMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_OK 0
#define MQ_ERR_INVALID (-1)     /* bad argument, shape or bound */
#define MQ_ERR_DEVICE (-2)      /* no usable gfx950 device */
#define MQ_ERR_LAUNCH (-3)      /* a HIP call or kernel launch failed */
#define MQ_ERR_UNSUPPORTED (-4) /* valid request this build does not implement */

#define MQ_F32 0
#define MQ_BF16 1

#define MQ_SLOT_BIT 0x80000000u /* route word: bit 31 set = pool slot */

/* Bounds of the decode entry points.  The reference executor takes at most 8
 * tokens (models/flashnext/metal_runtime.py:26-31); mq_moe_decode and
 * mq_moe_layer accept up to 64 (speculative-verify batches). */
#define MQ_MAX_TOKENS 64
#define MQ_MAX_EXPERTS 512
#define MQ_MAX_TOP_K 10
#define MQ_MAX_WIDTH 16384

/*
 * One projection (gate, up or down) of an expert bank.  A route word with
 * MQ_SLOT_BIT set addresses a record in `pool`:
 *   base = pool + pool_header + (uint64)(word & 0x7FFFFFFF) * pool_stride
 *   weight = base + off_weight, scales = base + off_scales, biases = base + off_biases
 * (models/flashnext/metal_runtime.py:194-228).  Any other word indexes the
 * expert-major record pack `stream_pack` when it is set (same record layout,
 * no header: base = stream_pack + word * pool_stride), else the dense arrays
 * weight [E, out, in/8], scales/biases [E, out, in/group].
 *
 * Route words are produced on the device, so kernels bound-check them: a slot
 * must be < pool_slots, a stream index < stream_records, a dense expert <
 * the call's expert count.  An out-of-range word is never dereferenced; its
 * contribution is skipped and a device error flag is raised, reported by
 * mq_check_device_errors().
 */
typedef struct MqProjection {
  const uint32_t *weight;
  const uint16_t *scales;
  const uint16_t *biases;
  const uint8_t *pool;
  uint64_t pool_header;
  uint64_t pool_stride;
  uint64_t off_weight;
  uint64_t off_scales;
  uint64_t off_biases;
  const uint8_t *stream_pack;
  uint32_t pool_slots;      /* records in `pool` */
  uint32_t stream_records;  /* records in `stream_pack` */
} MqProjection;

/* Arguments of mq_moe_decode: the fields of the reference's native bridge
 * struct FlashNextMoEArgs (tests/bench/metal_runtime_native.mm:175-194) plus
 * the pool, score combine and shared-expert epilogues of
 * MetalMoEExecutor.execute (models/flashnext/metal_runtime.py:764-932). */
typedef struct MqMoeArgs {
  const void *x;          /* [tokens, hidden] T */
  int x_dtype;            /* MQ_BF16 or MQ_F32; outputs use the same T */
  MqProjection gate;      /* [E, inter, hidden/8] */
  MqProjection up;        /* [E, inter, hidden/8] */
  MqProjection down;      /* [E, hidden, inter/8] */
  const uint32_t *routes; /* [tokens, slots] route words */
  const void *scores;     /* [tokens, slots] or NULL (then return_all must be 1) */
  int score_dtype;        /* MQ_F32 or MQ_BF16 */
  const int32_t *keeps;   /* [tokens] active slot prefix per token, or NULL (= slots) */
  /* shared epilogue: at most one of shared_y / (shared, shared_gate) / shared expert */
  const void *shared_y;      /* [tokens, hidden] T: out = T(T(acc) + shared_y) */
  const void *shared;        /* [tokens, hidden] T: out = T(T(acc) + T(shared*gate)) */
  const uint16_t *shared_gate; /* [tokens] bf16 sigmoid gate (with `shared` or shared expert) */
  const MqProjection *shared_expert; /* NULL or a HOST array of 3 projections {gate, up, down}
                                        of one expert (route word 0), read during the call;
                                        computed in-kernel and combined like `shared` with
                                        `shared_gate` */
  void *out;              /* [tokens, hidden] T (combined) */
  void *gate_out;         /* optional [tokens, slots, inter] T (return_all diagnostics) */
  void *up_out;           /* optional [tokens, slots, inter] T */
  void *act_out;          /* REQUIRED [tokens, slots(+1 with shared expert), inter] T: the
                             SwiGLU activations (the library allocates nothing) */
  void *down_out;         /* optional [tokens, slots, hidden] T, per-slot down (return_all) */
  uint32_t tokens;
  uint32_t slots;
  uint32_t hidden;
  uint32_t inter;
  uint32_t expert_count;
  uint32_t group_size;    /* 32 or 64 */
  uint32_t flags;         /* MQ_DECODE_* */
} MqMoeArgs;

#define MQ_DECODE_RETURN_ALL 1u    /* write gate_out/up_out/act_out/down_out, skip combine */
#define MQ_DECODE_UNFUSED_UP 2u    /* separate up projection + SwiGLU pass (bit-identical) */
/* Combine in the reference's generic order at any group size: every score
 * product rounded to T, the kept slots summed in float32 in slot order and
 * rounded once, then the shared term (weighted_combine, metal_runtime.py:908-929;
 * the order of _moe_call's gather_qmm path beyond the fused executor's token
 * bound, adaptive_topk.py:274-277).  Group 64 always combines this way. */
#define MQ_DECODE_GENERIC_COMBINE 4u

/* Arguments of mq_route_topk: the router chain of _moe_call
 * (models/flashnext/adaptive_topk.py:53-64, 75-261; compiled.py:61-71) and
 * the slot lookup of StreamingSwitchGLU._pool_pass
 * (models/flashnext/expert_cache.py:1694-1725). */
typedef struct MqRouteArgs {
  const uint16_t *x;        /* [tokens, hidden] bf16 */
  const uint16_t *gate_w;   /* [experts, hidden] bf16 router gate, or NULL when logits_in */
  const uint16_t *logits_in;/* [tokens, experts] bf16 precomputed logits, or NULL */
  const uint16_t *shared_gate_w; /* [hidden] bf16 shared-expert gate row, or NULL */
  const uint32_t *slot_table;    /* [experts] pool slot per expert, or NULL (routes = expert ids) */
  uint16_t *logits_out;     /* [tokens, experts] bf16, required unless logits_in is given */
  uint32_t *inds;           /* [tokens, top_k] expert ids, score-descending, ties by index */
  void *scores;             /* [tokens, top_k] renormalised scores */
  int score_dtype;          /* MQ_BF16 (bf16 arithmetic result) or MQ_F32 (widened) */
  uint16_t *scores_raw;     /* optional [tokens, top_k] bf16 softmax gates before renorm */
  uint32_t *routes;         /* optional [tokens, top_k] route words */
  int32_t *keeps;           /* optional [tokens] adaptive keep count */
  uint16_t *shared_gate;    /* optional [tokens] bf16 sigmoid(x . shared_gate_w) */
  uint32_t tokens;
  uint32_t hidden;
  uint32_t experts;
  uint32_t top_k;
  float threshold;          /* >= 1: keep all top_k; < 1: adaptive keep + pad */
  uint32_t min_keep;
  float blend;              /* renorm blend (1 = divide by selected mass) */
} MqRouteArgs;

/* Arguments of mq_moe_grouped: the >8-token (prefill / verify) path of
 * StreamingSwitchGLU._one_pass/_issue (models/flashnext/expert_cache.py:1743-1810):
 * the (token, slot) rows are sorted by expert (build_plan, :750-760, and
 * mlx-vlm _gather_sort), gather_qmm gate/up -> SwiGLU -> gather_qmm down run
 * as grouped bf16 MFMA GEMMs over the sorted rows, the per-slot outputs are
 * unsorted into y, and the bf16 generic combine
 * (models/flashnext/adaptive_topk.py:274-277) produces out. */
typedef struct MqGroupedArgs {
  const uint16_t *x;        /* [tokens, hidden] bf16 */
  MqProjection gate, up, down;
  const uint32_t *routes;   /* [tokens, slots] route words */
  const uint16_t *scores;   /* [tokens, slots] bf16; required when out is set */
  const uint16_t *shared;   /* optional precomputed shared expert output [tokens, hidden] bf16 */
  const MqProjection *shared_expert; /* optional HOST array of 3 (gate, up, down) dense
                                        single-expert projections, run as one more group */
  const uint16_t *shared_gate; /* [tokens] bf16, required with shared or shared_expert */
  uint16_t *out;            /* [tokens, hidden] bf16 combined, or NULL */
  uint16_t *y;              /* [tokens, slots, hidden] bf16 per-slot outputs (required) */
  void *workspace;          /* device scratch of mq_grouped_workspace_size() bytes */
  uint64_t workspace_bytes;
  uint32_t tokens, slots, hidden, inter;
  uint32_t expert_count;    /* dense experts addressed by plain route ids (0 with a pool) */
  uint32_t group_size;
} MqGroupedArgs;

/* ---- capability and errors (tests/bench/metal_runtime_native.mm:196-205) ---- */

/* 1 when a gfx950 device is usable from this process, else 0. */
int mq_available(void);

/* Resolve the library's per-device state (the device error flags, a static
 * __device__ array; nothing is allocated) on the current device.  Entry
 * points do this lazily; calling it first is optional.  Idempotent. */
int mq_init(void);

/* Copy the calling thread's last error message into buf (NUL-terminated). */
int mq_last_error(char *buf, uint32_t max_len);

/* Synchronise `stream`, then read and clear the current device's error flags
 * raised by kernels (MQ_DEVFLAG_*).  Returns MQ_OK when none were raised,
 * else MQ_ERR_INVALID with the flags described by mq_last_error(). */
int mq_check_device_errors(void *stream, uint32_t *flags_out);
#define MQ_DEVFLAG_BAD_ROUTE 1u /* a route word addressed no valid record/expert */
#define MQ_DEVFLAG_BAD_ROW 2u   /* an x row index (MqGatherArgs.x_rows) was >= x_count */

/* Library version as major*10000 + minor*100 + patch. */
int mq_version(void);

/* sizeof() of the ABI structs as compiled into the library, so bindings can
 * verify their layout: which = 0 MqProjection, 1 MqMoeArgs, 2 MqRouteArgs,
 * 3 MqGroupedArgs, 4 MqGatherArgs; 0 for an unknown id. */
uint64_t mq_abi_struct_size(int which);

/* ---- record layout (models/flashnext/slab_pack.py:96-149) ---- */

/* Byte offsets of the nine parts (gate/up/down x weight/scales/biases) and the
 * page-aligned record stride for a (hidden, inter, group) expert. */
int mq_record_layout(uint32_t hidden, uint32_t inter, uint32_t group_size,
                     uint64_t offsets[9], uint64_t *stride);

/* ---- Q4 primitives ---- */

/* Unpack n_words packed words into 8*n_words uint8 values (metal_runtime.py:980). */
int mq_q4_unpack(const uint32_t *words, uint8_t *values, uint64_t n_words, void *stream);

/* bf16(s*q + b) for a [rows, cols] Q4 matrix (mx.dequantize semantics). */
int mq_q4_dequant(const uint32_t *weight, const uint16_t *scales, const uint16_t *biases,
                  uint16_t *out, uint32_t rows, uint32_t cols, uint32_t group_size,
                  void *stream);

/* y[m, n] = T(sum_k x[m, k] * (s*q + b)[n, k]) for m < rows_x:
 * mx.quantized_matmul(x, w, s, b, transpose=True, group_size, bits=4) as
 * reached through nn.QuantizedLinear (models/flashnext/loader.py:190-217).
 * x and y share dtype x_dtype. */
int mq_q4_qmv(const void *x, int x_dtype, const uint32_t *weight, const uint16_t *scales,
              const uint16_t *biases, void *y, uint32_t rows_x, uint32_t out_features,
              uint32_t in_features, uint32_t group_size, void *stream);

/* out[t, s, :] = T(W_{route[t,s]} . x[t or (t,s)]): the per-projection QMV of
 * MetalMoEExecutor._metal_projection (models/flashnext/metal_runtime.py:640-667)
 * and mx.gather_qmm for decode shapes (models/flashnext/expert_cache.py:799-810).
 * slot_input != 0 reads x as [tokens, slots, in]. */
int mq_gather_qmv(const void *x, int x_dtype, int slot_input, const MqProjection *proj,
                  const uint32_t *routes, void *out, uint32_t tokens, uint32_t slots,
                  uint32_t in_features, uint32_t out_features, uint32_t expert_count,
                  uint32_t group_size, void *stream);

/* ---- elementwise activations ---- */

/* out = swiglu(gate, up) over n T values: MLX's swiglu as the reference's
 * unfused up path calls it (models/flashnext/metal_runtime.py:895-907), with
 * the fused Up epilogue's rounding points (:278-287): m = |g|, e = T(exp(m)),
 * d = T(1 + e), s = T(1 / d), sig = g < 0 ? s : T(1 - s), out = T(T(g * sig) * u),
 * exp correctly rounded to float32.  bf16 runs take the four-at-a-time
 * sequence, with MQ_SWIGLU_SCALAR the decode kernels'
 * per-element sequence, or with MQ_SWIGLU_TABLE the grouped gate/up
 * epilogue's sequence with the sigmoid looked up in a per-block table
 * (bit-identical by construction; all are exported so each can be checked on
 * its own).  The two flags exclude each other.  n < 2^31. */
#define MQ_SWIGLU_SCALAR 1u
#define MQ_SWIGLU_TABLE 2u
int mq_swiglu(const void *gate, const void *up, void *out, uint64_t n, int dtype, uint32_t flags,
              void *stream);

/* out = sigmoid(x) over n T values with the same T-rounded sequence
 * (mx.sigmoid of the shared-expert gate, models/flashnext/adaptive_topk.py:264). */
int mq_sigmoid(const void *x, void *out, uint64_t n, int dtype, void *stream);

/* Device check of the bf16 rounding the kernels use, over the float32 bit
 * patterns [first, first + count) within [0, 2^32): adds to counts[0] the
 * patterns where the kernels' round-to-bf16 differs from integer
 * round-to-nearest-even with a canonical quiet NaN, and to counts[1] the
 * non-NaN patterns where the one-instruction conversion differs from it.
 * `counts` is a device array of two uint64 the caller zeroes.  No reference
 * counterpart: it exists so the exactness claim is tested on each device. */
int mq_bf16_round_check(uint64_t first, uint64_t count, unsigned long long *counts, void *stream);

/* ---- latency floors of the decode path (measurement only) ----
 * No reference counterpart: they measure, on the device at hand, what a
 * kernel boundary, a stream of expert bytes with no compute, and a dependent
 * load cost, which bound the decode layer from below (bench.py --floors).
 *
 * mq_stream_probe: one kernel reading n segments of bytes_each bytes (a
 * multiple of 16) at the device addresses segments[0..n) (a DEVICE array)
 * with non-temporal 16-byte loads, `blocks` blocks (a multiple of n) of 256
 * threads splitting them; `sink` is a device word written only on a
 * checksum match.  n = 0 launches an empty kernel.
 * mq_hop_probe: thread 0 of block `block` (0..63; blocks are dealt to the
 * XCDs round-robin, so the block picks the XCD) follows `hops` (1..8) links of
 * a pointer chain in device memory starting at `chain` (each link holds the
 * device address of the next; the caller makes every dereferenced link
 * valid) and writes 10 words to `stamps`: the 100 MHz real-time clock at the
 * start and after each link (unused entries repeat the last), then the final
 * value read. */
int mq_stream_probe(const uint64_t *segments, uint32_t n, uint64_t bytes_each, uint32_t blocks, uint32_t *sink,
                    void *stream);
int mq_hop_probe(const uint64_t *chain, uint32_t hops, uint64_t *stamps, uint32_t block, void *stream);
/* mq_mfma_probe: `blocks` blocks of 512 threads (two waves per SIMD at one
 * block per CU), each wave issuing `iters` (1..2^24) rounds of four
 * independent v_mfma_f32_32x32x16_bf16 (32,768 FLOP each) on register
 * operands; `sink` is a device array of blocks * 512 floats.  Timing the
 * launch gives the sustained bf16 MFMA rate at the clock the matrix cores
 * hold under load, the practical ceiling of the grouped GEMMs.  No reference
 * counterpart. */
int mq_mfma_probe(uint32_t iters, uint32_t blocks, float *sink, void *stream);

/* ---- router ---- */
int mq_route_topk(const MqRouteArgs *args, void *stream);

/* ---- decode executor (MetalMoEExecutor.execute, metal_runtime.py:764-932) ---- */
int mq_moe_decode(const MqMoeArgs *args, void *stream);

/* One routed decode layer, _moe_call with the fused executor
 * (models/flashnext/adaptive_topk.py:53-292).  Up to 4 tokens: router
 * logits, then a gate/up kernel that performs the top-k selection itself (one
 * token per wave of each block; writing route->inds, scores (bf16), routes,
 * keeps, shared_gate) and runs gate/up/SwiGLU, then down + combine.
 * 5..64 tokens: mq_route_topk, then the expert kernels with the routes given
 * (same outputs).  route->x must equal moe->x (bf16); route->logits_out and
 * route->routes are required; moe->routes/scores/keeps/shared_gate are taken
 * from the route outputs.  moe->flags: 0 or MQ_DECODE_GENERIC_COMBINE. */
int mq_moe_layer(const MqRouteArgs *route, const MqMoeArgs *moe, void *stream);

/* ---- prefill / verify grouped path ---- */
/* Workspace bytes for mq_moe_grouped: `route_keys` is the number of distinct
 * route targets (pool slots + plain expert ids addressable by the routes),
 * `shared` is 1 when a shared expert runs as an extra group. */
uint64_t mq_grouped_workspace_size(uint32_t tokens, uint32_t slots, uint32_t hidden,
                                   uint32_t inter, uint32_t route_keys, int shared);
int mq_moe_grouped(const MqGroupedArgs *args, void *stream);

/* One grouped projection: out[r, :] = bf16(W_{route[r]} . x[x_rows[r]]) for
 * r < rows, fp32 accumulate over bf16(s*q + b) weights.  This is
 * mx.gather_qmm(x, w, scales, biases, rhs_indices, transpose=True,
 * group_size, bits=4, sorted_indices) at the prefill / verify call shape
 * (models/flashnext/expert_cache.py:799-810, called three times per pass from
 * _issue at :1790-1806 on rows sorted by expert): the rows are counting-sorted
 * by route key on the device and run through the same MFMA GEMM as
 * mq_moe_grouped's down projection, with no combine.  Row order in `routes`
 * does not change any value (sorted_indices is only a hint there too).
 * Route words as in MqMoeArgs (plain ids < expert_count, or MQ_SLOT_BIT|slot
 * with a pool projection); a word that addresses nothing raises
 * MQ_DEVFLAG_BAD_ROUTE and its row reads zero weights; an x_rows entry
 * >= x_count raises MQ_DEVFLAG_BAD_ROW and its row reads zero inputs. */
typedef struct MqGatherArgs {
  const uint16_t *x;        /* [x_count, in_width] bf16 */
  const uint32_t *x_rows;   /* [rows] x row of each output row, or NULL: row r reads x row r
                               (then x_count >= rows) */
  const uint32_t *routes;   /* [rows] route words */
  uint16_t *out;            /* [rows, out_width] bf16 */
  MqProjection w;
  void *workspace;          /* device scratch of mq_gather_qmm_workspace_size() bytes */
  uint64_t workspace_bytes;
  uint32_t x_count, rows, in_width, out_width;
  uint32_t expert_count;    /* dense experts addressed by plain route ids (0 with a pool) */
  uint32_t group_size;
} MqGatherArgs;

/* Workspace bytes for mq_gather_qmm; `route_keys` as for mq_grouped_workspace_size. */
uint64_t mq_gather_qmm_workspace_size(uint32_t rows, uint32_t route_keys);
int mq_gather_qmm(const MqGatherArgs *args, void *stream);

/* mq_moe_grouped with the library's own static scratch instead of a
 * workspace: it calls no allocator (no hipMalloc, hipFree or allocating
 * runtime routine), for callers that cannot allocate -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation.  No
 * counterpart in the reference.  args->workspace and workspace_bytes are
 * ignored.  The scratch is a file-scope __device__ array of
 * MQ_GROUPED_STATIC_SCRATCH_BYTES per device (held until the process ends);
 * a call whose mq_grouped_workspace_size() exceeds it fails with
 * MQ_ERR_INVALID before anything is launched.  Every call on one device shares
 * that device's scratch: calls that overlap on one device (different streams
 * or threads without ordering) race.  64 MiB covers the 4096-token prefill
 * chunk at hidden 2048 / inter 512 over 512 experts with a shared expert. */
#define MQ_GROUPED_STATIC_SCRATCH_BYTES (64ull << 20)
int mq_moe_grouped_static(const MqGroupedArgs *args, void *stream);

/* ---- expert slot pool refill (models/flashnext/expert_pool.py:112-145) ----
 * Copy n records of record_bytes each from pinned host memory to pool slots
 * (slot i lands at pool + pool_header + slots[i] * pool_stride) on
 * copy_stream, then record done_event (if not NULL) on that stream.  The
 * reference reads the nine rows of each missed expert into its slot; here a
 * host record already holds the nine parts at their layout offsets.
 * `slots` and `host_records` are HOST arrays of n entries; each
 * host_records[i] must be host-pinned memory (hipHostMalloc).  Slots at or
 * beyond pool_slots are rejected.  The caller orders the copies after the
 * last kernel that reads a refilled slot (an event wait on copy_stream) and
 * makes consumers wait on done_event. */
int mq_pool_refill_async(uint8_t *pool, uint64_t pool_header, uint64_t pool_stride, uint32_t pool_slots,
                         const uint32_t *slots, const void *const *host_records,
                         uint32_t n, uint64_t record_bytes, void *copy_stream,
                         void *done_event);

/* The same refill (same arguments, ordering and slot checks) as one gather
 * kernel on copy_stream that reads the records through their device mapping
 * (PCIe reads of pinned host memory) instead of one hipMemcpyAsync per
 * record; up to 16 records per launch.  Each host_records[i] must be pinned
 * and device-mapped (hipHostMalloc; checked with hipHostGetDevicePointer
 * before any launch) and 16-byte aligned, and record_bytes, pool_header and
 * pool_stride multiples of 16.  The records must stay allocated until
 * done_event (or the stream) completes.  Replaces the same fill
 * (models/flashnext/expert_pool.py:133-145) as mq_pool_refill_async. */
int mq_pool_refill_gather_async(uint8_t *pool, uint64_t pool_header, uint64_t pool_stride, uint32_t pool_slots,
                                const uint32_t *slots, const void *const *host_records,
                                uint32_t n, uint64_t record_bytes, void *copy_stream,
                                void *done_event);

#ifdef __cplusplus
}
#endif

#endif /* MQMOE_H */
