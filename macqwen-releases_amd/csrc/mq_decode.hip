// Decode-path kernels for gfx950: Q4 QMV, fused gate/up + SwiGLU (with the
// router selection folded in), and down + score combine + shared epilogue.
//
// Row engine.  A row of a Q4 matrix is cut into 32-input chunks (one chunk =
// 4 uint32 = 32 nibbles = one 128-bit load).  A "slice" of SW lanes (SW = 64
// or 16) owns one output row per step: lane li loads chunks {li, li+SW, ...}
// (CPL chunks), so each load instruction of a slice reads SW*16 contiguous
// bytes.  Weights are streamed with non-temporal loads.  Nibble pairs are
// turned into bf16 pairs (128+q) with one v_bfi_b32 each and multiplied with
// the activation chunk (kept in registers as matching bf16 pairs) by
// v_dot2_f32_bf16; the 128 offset is removed with the chunk sum, and the group
// scale/bias are applied in float32.  A slice reduces its row with DPP
// (16 lanes) or DPP + readlane (64 lanes).  Every wave issues all of its loads
// before its first dependent instruction.
//
// Rounding points follow the reference executor
// (models/flashnext/metal_runtime.py:231-336): every projection output is
// rounded to the activation type T, the SwiGLU epilogue rounds each step to
// T, and the score combine accumulates float(T(d)) * float(score) in float32
// with no contraction before the final T rounding and shared add.
#include <math.h>

#include "mq_internal.h"
#include "mq_select.h"

namespace mq {

int launch_router_logits(const uint16_t *x, const uint16_t *gate_w, const uint16_t *shared_gate_w,
                         uint16_t *logits, uint16_t *shared_logit, uint32_t tokens, uint32_t hidden,
                         uint32_t routed_rows, hipStream_t stream);
int validate_route_args(const MqRouteArgs &a);
SelectParams select_params(const MqRouteArgs &a, const uint16_t *logits);

namespace {

constexpr int kWaves = 4;  // waves per block
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kMaxSlots = 16;      // routed slots per token in the fused kernels
constexpr uint32_t kMaxLayerTokens = 8;  // tokens of the fused routed layer

// ------------------------------------------------------------------ slices
template <int SW>
struct Slice {
  static_assert(SW == 16 || SW == 64, "slice width must be 16 or 64 lanes");
  static constexpr int kRows = 64 / SW;  // rows per wave step
  __device__ static __forceinline__ int sub(int lane) { return lane / SW; }
  __device__ static __forceinline__ int li(int lane) { return lane % SW; }
  // Row sum; valid in lane 0 of the slice (all lanes for SW = 64).
  __device__ static __forceinline__ float reduce(float v) {
    if constexpr (SW == 16) return row16_sum(v);
    else return wave_sum(v);
  }
};

// (128+q_k, 128+q_{k+4}) bf16 pair from nibbles k and k+4 of w (one v_bfi_b32).
__device__ __forceinline__ uint32_t nib_pair_bfi(uint32_t w, int k) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(0x000f000fu), "v"(w >> (4 * k)), "v"(0x43004300u));
  return r;
}

// Four independent accumulation chains (one per packed word) for ILP.
__device__ __forceinline__ float q4_dot(const uint4 &w, const XChunk &x) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float d[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    d[j] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) d[j] = dot2_bf16(x.p[4 * j + k], nib_pair_bfi(ws[j], k), d[j]);
  }
  return ((d[0] + d[1]) + (d[2] + d[3])) - 128.0f * x.osum;
}

// Sum of the 32 bf16 values of a chunk (four independent chains).
__device__ __forceinline__ float pair_sum4(const XChunk &x) {
  float s[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s[j] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) s[j] = dot2_bf16(x.p[4 * j + k], 0x3f803f80u, s[j]);
  }
  return (s[0] + s[1]) + (s[2] + s[3]);
}

// ------------------------------------------------------------------ activations
// Activation chunk(s) of one lane: bf16 inputs need one pair chunk, float32
// inputs are split into bf16 hi + lo chunks (x = hi + lo to 16 bits).  The
// loads are issued by issue() and consumed by finish(), so a kernel can put
// the (cache-resident) activation loads ahead of its weight stream and convert
// them while the weights are still in flight.
template <class TT>
struct XLane;

template <>
struct XLane<BF16T> {
  static constexpr int kParts = 1;
  XChunk part[1];
  float bias_sum;  // sum of the inputs, multiplies the group bias
  uint4 raw[4];
  // Loads the 64-byte chunk at byte offset `off` of the row (zeros when out of range).
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t row, uint32_t off) {
#pragma unroll
    for (int j = 0; j < 4; ++j) raw[j] = buf_load16(row, off + 16u * j);
  }
  __device__ __forceinline__ void finish() {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
      pairs_from_words(u, &part[0].p[4 * j]);
    }
    part[0].osum = pair_sum4(part[0]);
    bias_sum = part[0].osum;
  }
};

template <>
struct XLane<F32T> {
  static constexpr int kParts = 2;
  XChunk part[2];
  float bias_sum;
  uint4 raw[8];
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t row, uint32_t off) {
#pragma unroll
    for (int j = 0; j < 8; ++j) raw[j] = buf_load16(row, off + 16u * j);
  }
  __device__ __forceinline__ void finish() {
    uint32_t hi[16], lo[16];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f[4] = {__uint_as_float(raw[j].x), __uint_as_float(raw[j].y), __uint_as_float(raw[j].z),
                          __uint_as_float(raw[j].w)};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int idx = 4 * j + k;
        const uint16_t h = f32_to_bf16(f[k]);
        const uint16_t l = f32_to_bf16(f[k] - bf16_to_f32(h));
        s += f[k];
        if (idx & 1) {
          hi[idx >> 1] |= static_cast<uint32_t>(h) << 16;
          lo[idx >> 1] |= static_cast<uint32_t>(l) << 16;
        } else {
          hi[idx >> 1] = h;
          lo[idx >> 1] = l;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pairs_from_words(&hi[4 * j], &part[0].p[4 * j]);
      pairs_from_words(&lo[4 * j], &part[1].p[4 * j]);
    }
    part[0].osum = pair_sum4(part[0]);
    part[1].osum = pair_sum4(part[1]);
    bias_sum = s;
  }
};

// Row descriptor of an activation row of `in_w` values.
template <class TT>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_rsrc(const typename TT::storage *row, uint32_t in_w) {
  return make_rsrc(row, in_w * static_cast<uint32_t>(sizeof(typename TT::storage)));
}

template <class TT, int SW, int CPL>
__device__ __forceinline__ void issue_x(XLane<TT> *x, __amdgpu_buffer_rsrc_t row, uint32_t in_w, int li,
                                        bool valid = true) {
  const uint32_t chunks = in_w >> 5;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t c = static_cast<uint32_t>(j * SW + li);
    const uint32_t off = valid && c < chunks ? c * 32u * static_cast<uint32_t>(sizeof(typename TT::storage)) : kOutOfRange;
    x[j].issue(row, off);
  }
}

template <class TT, int CPL>
__device__ __forceinline__ void finish_x(XLane<TT> *x) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) x[j].finish();
}

// ------------------------------------------------------------------ weight rows
template <int CPL>
struct RowLoad {
  uint4 w[CPL];
  uint16_t s[CPL];
  uint16_t b[CPL];
};

// Issue the loads of one lane's chunks of row `row`.  Masked chunks (row out
// of range, tail chunk, invalid record) use an out-of-range offset and read as
// zero, so the loads are issued back to back with no branches.
template <int SW, int CPL>
__device__ __forceinline__ void load_row(RowLoad<CPL> &r, const ExpertRsrc &e, uint32_t row, uint32_t in_w,
                                         uint32_t group, int li, bool row_ok) {
  const uint32_t chunks = in_w >> 5;
  const uint32_t words = in_w >> 3;
  const uint32_t groups = in_w / group;
  const uint32_t shift = group == 64 ? 1 : 0;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t c = static_cast<uint32_t>(j * SW + li);
    const bool ok = row_ok && c < chunks;
    const uint32_t off_w = ok ? (row * words + c * 4u) * 4u : kOutOfRange;
    const uint32_t off_g = ok ? (row * groups + (c >> shift)) * 2u : kOutOfRange;
    r.w[j] = buf_load16<kNonTemporal>(e.w, off_w);
    r.s[j] = buf_load2(e.s, off_g);
    r.b[j] = buf_load2(e.b, off_g);
  }
}

// Lane partial of sum_g s_g * sum(x q) + b_g * sum(x) over the lane's chunks.
template <class TT, int CPL>
__device__ __forceinline__ float row_partial(const RowLoad<CPL> &r, const XLane<TT> *x) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float dq = 0.0f;
#pragma unroll
    for (int p = 0; p < XLane<TT>::kParts; ++p) dq += q4_dot(r.w[j], x[j].part[p]);
    acc = fmaf(bf16_to_f32(r.s[j]), dq, acc);
    acc = fmaf(bf16_to_f32(r.b[j]), x[j].bias_sum, acc);
  }
  return acc;
}

// ------------------------------------------------------------------ kernels

// The shared expert's three projections, passed by value as a kernel argument.
struct SharedExpert {
  MqProjection p[3];  // gate, up, down; addressed with route word 0
};

// Projection QMV: out[pair, row] = T(W_route(pair) . x(pair)).  A wave handles
// R steps of Slice<SW>::kRows rows of one pair.
template <class TT, int SW, int CPL, int R>
__global__ __launch_bounds__(kThreads) void gather_qmv_kernel(
    const typename TT::storage *__restrict__ x, int slot_input, MqProjection proj,
    const uint32_t *__restrict__ routes, typename TT::storage *__restrict__ out, uint32_t pairs, uint32_t slots,
    uint32_t in_w, uint32_t out_w, uint32_t group, uint32_t dense_count, unsigned int *__restrict__ err) {
  using Sl = Slice<SW>;
  constexpr int kTileRows = R * Sl::kRows;
  const int lane = threadIdx.x & 63;
  const int li = Sl::li(lane);
  const int sub = Sl::sub(lane);
  const uint32_t tiles_per_pair = (out_w + kTileRows - 1) / kTileRows;
  const uint32_t tile = blockIdx.x * kWaves + wave_id();
  if (tile >= pairs * tiles_per_pair) return;  // wave-uniform
  const uint32_t pair = tile / tiles_per_pair;
  const uint32_t row0 = (tile % tiles_per_pair) * kTileRows;
  const uint32_t token = pair / slots;
  XLane<TT> xl[CPL];
  issue_x<TT, SW, CPL>(xl, x_rsrc<TT>(x + static_cast<uint64_t>(slot_input ? pair : token) * in_w, in_w), in_w, li);
  const uint32_t word = routes ? routes[pair] : 0u;
  const ExpertPtrs e = expert_ptrs(proj, word, out_w, in_w, group, dense_count);
  if (!e.ok && lane == 0) raise_flag(err, MQ_DEVFLAG_BAD_ROUTE);  // its rows read as zero
  const ExpertRsrc er = expert_rsrc(e, out_w, in_w, group);
  RowLoad<CPL> r[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t row = row0 + i * Sl::kRows + sub;
    load_row<SW, CPL>(r[i], er, row, in_w, group, li, row < out_w);
  }
  finish_x<TT, CPL>(xl);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t row = row0 + i * Sl::kRows + sub;
    const float v = Sl::reduce(row_partial<TT, CPL>(r[i], xl));
    if (li == 0 && row < out_w) out[static_cast<uint64_t>(pair) * out_w + row] = TT::store(v);
  }
}

// Router selection staged in LDS for the fused layer kernel.
struct RouteLds {
  uint32_t word[kMaxLayerTokens * kMaxSlots];
  int32_t keep[kMaxLayerTokens];
};

struct SelectOutputs {  // global outputs of the selection (written by block 0)
  uint32_t *inds;
  uint16_t *scores;     // bf16
  uint16_t *scores_raw;
  uint32_t *routes;
  int32_t *keeps;
  uint16_t *shared_gate;
  const uint16_t *shared_logit;
};

// Fused gate + up + SwiGLU: act[pair, row] = swiglu(T(gate), T(up)).
// Pairs [0, tokens*slots) are routed, pairs [tokens*slots, +tokens) are the
// shared expert of each token.  Tiles run the shared pairs first (they do not
// depend on routing).  With SELECT, every block that has routed tiles runs
// the router selection itself (one wave per token, from the logits) and keeps
// the route words in LDS; block 0 also publishes the selection.
template <class TT, int SW, int CPL, int R, bool SELECT>
// The arguments are ordered for the kernel-argument preload (14 dwords): first
// what the selection and the activation loads need at the start, then the rest.
__global__ __launch_bounds__(kThreads) void gateup_kernel(
    const uint16_t *__restrict__ sel_logits, const uint32_t *__restrict__ sel_slot_table,
    const typename TT::storage *__restrict__ x, uint32_t sel_experts, uint32_t sel_top_k, uint32_t tokens,
    uint32_t slots, uint32_t tile_limit, uint32_t has_shared_u, uint32_t hidden, uint32_t inter,
    uint32_t sel_min_keep, float sel_threshold, float sel_blend, MqProjection gate, MqProjection up,
    SharedExpert shared, const uint32_t *__restrict__ routes, const int32_t *__restrict__ keeps,
    SelectOutputs sel_out, typename TT::storage *__restrict__ act, typename TT::storage *__restrict__ gate_out,
    typename TT::storage *__restrict__ up_out, uint32_t group, uint32_t dense_count, unsigned int *__restrict__ err) {
  const SelectParams sel{sel_logits, sel_slot_table, sel_experts, sel_top_k, sel_min_keep, sel_threshold, sel_blend};
  const bool has_shared = has_shared_u != 0u;
  using Sl = Slice<SW>;
  constexpr int kTileRows = R * Sl::kRows;
  __shared__ RouteLds lds;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = wave_id();
  const int li = Sl::li(lane);
  const int sub = Sl::sub(lane);
  const uint32_t tiles_per_pair = (inter + kTileRows - 1) / kTileRows;
  const uint32_t routed_pairs = tokens * slots;
  const uint32_t shared_pairs = has_shared ? tokens : 0u;
  const uint32_t total_tiles = min((routed_pairs + shared_pairs) * tiles_per_pair, tile_limit);
  const uint32_t shared_tiles = shared_pairs * tiles_per_pair;
  const uint32_t block_first = blockIdx.x * kWaves;

  // The wave's tile: shared tiles first, then routed tiles.  The token (and
  // so the activation row) is known before routing, so its loads go first.
  const uint32_t tile = block_first + wave;
  const bool tile_ok = tile < total_tiles;
  const bool is_shared = tile < shared_tiles;
  const uint32_t local = is_shared ? tile : tile - shared_tiles;
  const uint32_t pair = is_shared ? routed_pairs + local / tiles_per_pair : local / tiles_per_pair;
  const uint32_t row0 = (local % tiles_per_pair) * kTileRows;
  const uint32_t token = min(is_shared ? pair - routed_pairs : pair / slots, tokens - 1u);
  XLane<TT> xl[CPL];
  issue_x<TT, SW, CPL>(xl, x_rsrc<TT>(x + static_cast<uint64_t>(token) * hidden, hidden), hidden, li, tile_ok);

  if constexpr (SELECT) {
    // Does this block own any routed tile?  (uniform per block)
    const uint32_t block_last = min(block_first + kWaves, total_tiles);
    if (block_last > shared_tiles || blockIdx.x == 0) {
      for (uint32_t t = wave; t < tokens; t += kWaves) {
        const SelectLane s = select_token(sel, t, lane);
        if (static_cast<uint32_t>(lane) < slots) lds.word[t * slots + lane] = s.word;
        if (lane == 0) lds.keep[t] = static_cast<int32_t>(s.keep);
        if (blockIdx.x == 0) {
          const uint64_t base = static_cast<uint64_t>(t) * slots;
          if (static_cast<uint32_t>(lane) < slots) {
            sel_out.inds[base + lane] = s.ind;
            sel_out.scores[base + lane] = f32_to_bf16(s.score);
            if (sel_out.scores_raw) sel_out.scores_raw[base + lane] = f32_to_bf16(s.raw);
            sel_out.routes[base + lane] = s.word;
          } else if (lane == 63) {
            if (sel_out.keeps) sel_out.keeps[t] = static_cast<int32_t>(s.keep);
            if (sel_out.shared_gate)
              sel_out.shared_gate[t] = f32_to_bf16(sigmoid_bf16(bf16_to_f32(sel_out.shared_logit[t])));
          }
        }
      }
      __syncthreads();
    }
  }

  if (!tile_ok) return;
  uint32_t word = 0u;
  if (!is_shared) {
    int32_t keep_t;
    if constexpr (SELECT) {
      word = uniform(lds.word[pair]);
      keep_t = static_cast<int32_t>(uniform(static_cast<uint32_t>(lds.keep[token])));
    } else {
      word = routes[pair];
      keep_t = keeps != nullptr ? keeps[token] : static_cast<int32_t>(slots);
    }
    if ((pair % slots) >= static_cast<uint32_t>(keep_t)) return;  // padded slot
  }
  // Wave-uniform branch (choosing a projection by reference would copy the
  // kernel-argument structs to private memory).
  ExpertPtrs eg, eu;
  if (is_shared) {
    eg = expert_ptrs(shared.p[0], 0u, inter, hidden, group, 1u);
    eu = expert_ptrs(shared.p[1], 0u, inter, hidden, group, 1u);
  } else {
    eg = expert_ptrs(gate, word, inter, hidden, group, dense_count);
    eu = expert_ptrs(up, word, inter, hidden, group, dense_count);
  }
  if ((!eg.ok || !eu.ok) && lane == 0) raise_flag(err, MQ_DEVFLAG_BAD_ROUTE);  // rows read as zero
  const ExpertRsrc rgs = expert_rsrc(eg, inter, hidden, group);
  const ExpertRsrc rus = expert_rsrc(eu, inter, hidden, group);
  RowLoad<CPL> rg[R], ru[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t row = row0 + i * Sl::kRows + sub;
    load_row<SW, CPL>(rg[i], rgs, row, hidden, group, li, row < inter);
    load_row<SW, CPL>(ru[i], rus, row, hidden, group, li, row < inter);
  }
  finish_x<TT, CPL>(xl);
  float gv[R], uv[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    gv[i] = Sl::reduce(row_partial<TT, CPL>(rg[i], xl));
    uv[i] = Sl::reduce(row_partial<TT, CPL>(ru[i], xl));
  }
  // Epilogue in one pass: lane i takes row i of the wave (SW = 64; the row
  // sums are wave-uniform) or lane 0 of each slice its slice's row (SW = 16),
  // so the SwiGLU sequence runs once for all of the wave's rows.
  float gsel = gv[0], usel = uv[0];
  uint32_t rsel = row0 + sub;
  bool mine = li == 0;
  if constexpr (SW == 64) {
#pragma unroll
    for (int i = 1; i < R; ++i) {
      gsel = lane == i ? gv[i] : gsel;
      usel = lane == i ? uv[i] : usel;
    }
    rsel = row0 + static_cast<uint32_t>(lane) * Sl::kRows;
    mine = lane < R;
  }
  if (mine && rsel < inter) {
    const float gt = TT::round(gsel);
    const float ut = TT::round(usel);
    const uint64_t idx = static_cast<uint64_t>(pair) * inter + rsel;
    act[idx] = TT::store(swiglu_t<TT>(gt, ut));
    if (gate_out != nullptr && !is_shared) gate_out[idx] = TT::store(gt);
    if (up_out != nullptr && !is_shared) up_out[idx] = TT::store(ut);
  }
}

// SwiGLU over precomputed T gate/up projections (unfused path).
template <class TT>
__global__ void swiglu_kernel(const typename TT::storage *__restrict__ g, const typename TT::storage *__restrict__ u,
                              typename TT::storage *__restrict__ out, uint64_t n) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = TT::store(swiglu_t<TT>(TT::load(g[i]), TT::load(u[i])));
}

enum SharedMode : int { kSharedNone = 0, kSharedY = 1, kSharedParts = 2, kSharedExpert = 3 };

// Down + score combine + shared epilogue.  A block owns Slice<SW>::kRows
// output rows of one token; its four waves split the token's sources
// round-robin, so every wave streams only its sources' weight rows and
// activation chunks, and the grid has (hidden / kRows) * tokens blocks to
// spread the weight stream over the whole chip.  Source 0 is the in-kernel
// shared expert (when present), then routed slots 0, 1, ...: a source's
// activation row does not depend on the keep count, so the activation loads
// are issued before anything has arrived.  The token's route words, scores
// and keep count come in one round of loads (lane s holds slot s).  Each wave
// handles its sources in batches of SPW: activations first, then the weight
// rows once the route words are in, then the row dots (independent chains).
// The T-rounded projections d go to LDS and wave 0 combines them in slot
// order: acc += float(d) * float(score[t,s]) in float32 with no contraction
// (models/flashnext/metal_runtime.py:291-336), then T(acc) and the shared
// epilogue.  With `generic` (group 64) every product is rounded to T first,
// the order of the reference's weighted_combine in the score dtype
// (metal_runtime.py:908-929).  Padded slots (s >= keep) carry score 0 and are
// skipped.
template <class TT, int SW, int CPL, int SPW, int R>
// The arguments are ordered for the kernel-argument preload: first the inputs
// of the first round of loads (route words, scores, keep count, activations).
__global__ __launch_bounds__(kThreads) void down_combine_kernel(
    const uint32_t *__restrict__ routes, const void *__restrict__ scores, const int32_t *__restrict__ keeps,
    const typename TT::storage *__restrict__ act, const uint16_t *__restrict__ shared_gate, int score_dtype,
    int shared_mode, uint32_t tokens, uint32_t slots, uint32_t inter, MqProjection down, SharedExpert shared,
    const typename TT::storage *__restrict__ shared_vec, typename TT::storage *__restrict__ out, uint32_t hidden,
    uint32_t group, uint32_t dense_count, uint32_t generic_u, unsigned int *__restrict__ err) {
  const bool generic = generic_u != 0u;
  using Sl = Slice<SW>;
  constexpr uint32_t kMaxSources = kMaxSlots + 1;
  constexpr uint32_t kBlockRows = Sl::kRows * R;  // R row groups of kRows rows
  static_assert(kBlockRows <= 64, "the combine takes one lane per block row");
  __shared__ float dsum[kMaxSources][kBlockRows];

  const int lane = threadIdx.x & 63;
  const uint32_t wave = wave_id();
  const int li = Sl::li(lane);
  const int sub = Sl::sub(lane);
  const uint32_t token = blockIdx.y;
  const uint32_t row0 = blockIdx.x * kBlockRows;  // rows row0 + r * kRows + sub, r < R
  const uint32_t ulane0 = static_cast<uint32_t>(lane);
  const uint32_t fin_row = row0 + ulane0;  // the row this lane combines (lanes < kBlockRows)
  const bool fin_ok = ulane0 < kBlockRows && fin_row < hidden;
  const bool with_shared_expert = shared_mode == kSharedExpert;
  const uint32_t first_routed = with_shared_expert ? 1u : 0u;  // source index of routed slot 0
  const uint32_t n_src = slots + first_routed;                // sources before the keep count is known
  const uint32_t routed_pairs = tokens * slots;
  const uint64_t pair0 = static_cast<uint64_t>(token) * slots;
  const uint32_t ulane = static_cast<uint32_t>(lane);

  // One round of small loads: route word and score of slot `lane`, the keep
  // count, the shared inputs.  Buffer loads with out-of-range offsets for the
  // unused lanes, so nothing waits on anything else.
  const uint32_t lane_word =
      buf_load4(make_rsrc(routes + pair0, slots * 4u), ulane < slots ? ulane * 4u : kOutOfRange);
  const bool bf16_scores = score_dtype == MQ_BF16;
  const uint32_t score_bytes = bf16_scores ? 2u : 4u;
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(static_cast<const uint8_t *>(scores) + pair0 * score_bytes, slots * score_bytes);
  const uint16_t score16 = buf_load2(sr, bf16_scores && ulane < slots ? ulane * 2u : kOutOfRange);
  const uint32_t score32 = buf_load4(sr, !bf16_scores && ulane < slots ? ulane * 4u : kOutOfRange);
  const uint32_t keep_raw =
      keeps != nullptr ? buf_load4(make_rsrc(keeps + token, 4u), 0u) : static_cast<uint32_t>(slots);
  float shared_in = 0.0f, gate_in = 0.0f;
  if (shared_mode == kSharedY || shared_mode == kSharedParts)
    shared_in = TT::load(shared_vec[static_cast<uint64_t>(token) * hidden + min(fin_row, hidden - 1u)]);
  if (shared_mode == kSharedParts || with_shared_expert) gate_in = bf16_to_f32(shared_gate[token]);

  uint32_t keep = slots, n_act = n_src;
  for (uint32_t base = wave; base < n_src; base += kWaves * SPW) {
    XLane<TT> xl[SPW][CPL];
    RowLoad<CPL> rw[SPW][R];
#pragma unroll
    for (int i = 0; i < SPW; ++i) {  // activations first (independent of the route words)
      const uint32_t a = base + kWaves * i;
      const uint64_t pair = a < first_routed ? static_cast<uint64_t>(routed_pairs) + token : pair0 + (a - first_routed);
      issue_x<TT, SW, CPL>(xl[i], x_rsrc<TT>(act + pair * inter, inter), inter, li, a < n_src);
    }
    keep = min(uniform(keep_raw), slots);
    n_act = keep + first_routed;
#pragma unroll
    for (int i = 0; i < SPW; ++i) {  // then the weight rows
      const uint32_t a = base + kWaves * i;
      ExpertPtrs e{nullptr, nullptr, nullptr, false};
      if (a < first_routed) {
        e = expert_ptrs(shared.p[2], 0u, hidden, inter, group, 1u);
      } else if (a < n_act) {
        const uint32_t word = readlane_u(lane_word, static_cast<int>(a - first_routed));
        e = expert_ptrs(down, word, hidden, inter, group, dense_count);
      }
      if (a < n_act && !e.ok && lane == 0) raise_flag(err, MQ_DEVFLAG_BAD_ROUTE);
      const ExpertRsrc er = expert_rsrc(e, hidden, inter, group);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t row = row0 + static_cast<uint32_t>(r) * Sl::kRows + static_cast<uint32_t>(sub);
        load_row<SW, CPL>(rw[i][r], er, row, inter, group, li, row < hidden);
      }
    }
    float v[SPW][R];
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      finish_x<TT, CPL>(xl[i]);
#pragma unroll
      for (int r = 0; r < R; ++r) v[i][r] = Sl::reduce(row_partial<TT, CPL>(rw[i][r], xl[i]));
    }
    if (li == 0) {
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        const uint32_t a = base + kWaves * i;
#pragma unroll
        for (int r = 0; r < R; ++r)  // a bad route reads as zero weights: d = 0
          if (a < n_act) dsum[a][static_cast<uint32_t>(r) * Sl::kRows + static_cast<uint32_t>(sub)] = TT::round(v[i][r]);
      }
    }
  }
  __syncthreads();
  if (wave != 0) return;
  // Scores as wave-uniform values (slot s from lane s), read before the lane mask.
  const float score_lane = bf16_scores ? bf16_to_f32(score16) : __uint_as_float(score32);
  float score[kMaxSlots];
#pragma unroll
  for (uint32_t s = 0; s < kMaxSlots; ++s) score[s] = readlane_f(score_lane, min(s, kMaxSlots - 1u));
  if (!fin_ok) return;

  // Fused order: float32 products summed unrounded.  Generic order (group
  // 64): every product rounded to T before the float32 slot-order sum.
  float acc = 0.0f;
#pragma unroll
  for (uint32_t s = 0; s < kMaxSlots; ++s) {
    if (s < keep) {
      const float prod = __fmul_rn(dsum[s + first_routed][ulane0], score[s]);
      acc = __fadd_rn(acc, generic ? TT::round(prod) : prod);
    }
  }
  const float routed = TT::round(acc);
  float final_value = routed;
  if (shared_mode == kSharedY) {
    final_value = __fadd_rn(routed, shared_in);
  } else if (shared_mode == kSharedParts) {
    final_value = __fadd_rn(routed, TT::round(__fmul_rn(shared_in, gate_in)));
  } else if (with_shared_expert) {
    final_value = __fadd_rn(routed, TT::round(__fmul_rn(dsum[0][ulane0], gate_in)));
  }
  out[static_cast<uint64_t>(token) * hidden + fin_row] = TT::store(final_value);
}

// ------------------------------------------------------------------ dispatch
// Slice width and chunks per lane for an input width: 64-lane slices when the
// 32-input chunks fill the wave, otherwise 16-lane slices (tail chunks masked).
struct Geometry {
  int sw;
  int cpl;
};

inline Geometry geometry(uint32_t in_w) {
  const uint32_t chunks = in_w / 32;
  if (chunks % 64 == 0 && chunks / 64 <= 2) return {64, static_cast<int>(chunks / 64)};
  return {16, static_cast<int>((chunks + 15) / 16)};
}

#define MQ_GEOM_SWITCH(g, ...)                                                               \
  do {                                                                                       \
    if ((g).sw == 64 && (g).cpl == 1) { constexpr int SW = 64, CPL = 1; __VA_ARGS__; }              \
    else if ((g).sw == 64 && (g).cpl == 2) { constexpr int SW = 64, CPL = 2; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 1) { constexpr int SW = 16, CPL = 1; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 2) { constexpr int SW = 16, CPL = 2; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 3) { constexpr int SW = 16, CPL = 3; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 4) { constexpr int SW = 16, CPL = 4; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 5) { constexpr int SW = 16, CPL = 5; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 6) { constexpr int SW = 16, CPL = 6; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 7) { constexpr int SW = 16, CPL = 7; __VA_ARGS__; }         \
    else if ((g).sw == 16 && (g).cpl == 8) { constexpr int SW = 16, CPL = 8; __VA_ARGS__; }         \
    else return fail(MQ_ERR_UNSUPPORTED, "input width needs %d chunks per lane", (g).cpl);   \
  } while (0)

// Rows per wave step count: 2 steps for 64-lane slices, 1 for 16-lane slices.
template <int SW>
constexpr int steps_for() {
  return SW == 64 ? 2 : 1;
}

int validate_proj(const MqProjection *p, const char *name) {
  if (p == nullptr) return fail(MQ_ERR_INVALID, "%s projection is NULL", name);
  if (p->pool == nullptr && p->stream_pack == nullptr &&
      (p->weight == nullptr || p->scales == nullptr || p->biases == nullptr))
    return fail(MQ_ERR_INVALID, "%s projection needs dense arrays, a pool or a stream pack", name);
  if ((p->pool != nullptr || p->stream_pack != nullptr) && p->pool_stride == 0)
    return fail(MQ_ERR_INVALID, "%s projection record stride is zero", name);
  return MQ_OK;
}

int validate_shape(uint32_t in_w, uint32_t out_w, uint32_t group) {
  if (group != 32 && group != 64) return fail(MQ_ERR_INVALID, "group_size must be 32 or 64 (got %u)", group);
  if (in_w == 0 || out_w == 0) return fail(MQ_ERR_INVALID, "projection widths must be positive");
  if (in_w % group) return fail(MQ_ERR_INVALID, "input width %u is not a multiple of group %u", in_w, group);
  if (in_w % 32) return fail(MQ_ERR_INVALID, "input width %u is not a multiple of 32", in_w);
  if (in_w > MQ_MAX_WIDTH || out_w > MQ_MAX_WIDTH * 4)
    return fail(MQ_ERR_INVALID, "projection width out of bounds (%u x %u)", out_w, in_w);
  if (in_w / 32 > 128) return fail(MQ_ERR_UNSUPPORTED, "input width %u exceeds 4096", in_w);
  return MQ_OK;
}

// Device error flags of the current device (allocated on first use).
int device_flags(unsigned int **flags, hipStream_t stream) {
  DeviceWorkspace *ws = nullptr;
  const int rc = workspace(&ws, stream);
  if (rc) return rc;
  *flags = ws->flags;
  return MQ_OK;
}

template <class TT>
int launch_gather_qmv(const void *x, int slot_input, const MqProjection &proj, const uint32_t *routes, void *out,
                      uint32_t pairs, uint32_t slots, uint32_t in_w, uint32_t out_w, uint32_t group,
                      uint32_t dense_count, hipStream_t stream) {
  using S = typename TT::storage;
  unsigned int *err = nullptr;
  int rc = device_flags(&err, stream);
  if (rc) return rc;
  const Geometry g = geometry(in_w);
  MQ_GEOM_SWITCH(g, {
    constexpr int R = steps_for<SW>();
    constexpr int kTileRows = R * Slice<SW>::kRows;
    const uint32_t tiles = pairs * ceil_div(out_w, kTileRows);
    hipLaunchKernelGGL((gather_qmv_kernel<TT, SW, CPL, R>), dim3(ceil_div(tiles, kWaves)), dim3(kThreads), 0,
                       stream, static_cast<const S *>(x), slot_input, proj, routes, static_cast<S *>(out), pairs,
                       slots, in_w, out_w, group, dense_count, err);
  });
  return check_launch("gather_qmv_kernel");
}

// Blocks of `kernel` that can be resident at once on the current device
// (cached per kernel and device).
template <const void *(*KERNEL)()>
int64_t resident_blocks() {
  static int64_t cached[64];
  static bool known[64];
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 0;
  if (!known[device]) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, KERNEL(), kThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return 0;
    cached[device] = static_cast<int64_t>(per_cu) * cus;
    known[device] = true;
  }
  return cached[device];
}

template <class TT, int SW, int CPL, int R, bool SELECT>
const void *gateup_ptr() {
  return reinterpret_cast<const void *>(gateup_kernel<TT, SW, CPL, R, SELECT>);
}

template <class TT, int SW, int CPL, int R, bool SELECT>
void launch_gateup_r(const MqMoeArgs &a, const SharedExpert &shared, bool has_shared, const int32_t *keeps,
                     const SelectParams &sel, const SelectOutputs &sel_out, typename TT::storage *act,
                     unsigned int *err, uint32_t pairs, hipStream_t stream) {
  using S = typename TT::storage;
  constexpr int kTileRows = R * Slice<SW>::kRows;
  const uint32_t tiles = pairs * ceil_div(a.inter, kTileRows);
  hipLaunchKernelGGL((gateup_kernel<TT, SW, CPL, R, SELECT>), dim3(ceil_div(tiles, kWaves)), dim3(kThreads), 0,
                     stream, sel.logits, sel.slot_table, static_cast<const S *>(a.x), sel.experts, sel.top_k,
                     a.tokens, a.slots, tiles, has_shared ? 1u : 0u, a.hidden, a.inter, sel.min_keep, sel.threshold,
                     sel.blend, a.gate, a.up, shared, a.routes, keeps, sel_out, act, static_cast<S *>(a.gate_out),
                     static_cast<S *>(a.up_out), a.group_size, a.expert_count, err);
}

// Gate/up launch.  With 64-lane slices a wave takes 2, 4 or 8 rows per tile:
// the smallest count whose grid is resident at once, so that many-token calls
// (speculative verify) stream in one round of blocks rather than in
// successive rounds that each pay the full memory latency (and, with the
// selection folded in, the selection's latency).
template <class TT, bool SELECT>
int launch_gateup(const MqMoeArgs &a, const SharedExpert &shared, bool has_shared, const int32_t *keeps,
                  const SelectParams &sel, const SelectOutputs &sel_out, typename TT::storage *act,
                  unsigned int *err, hipStream_t stream) {
  const Geometry g = geometry(a.hidden);
  const uint32_t pairs = a.tokens * a.slots + (has_shared ? a.tokens : 0u);
  MQ_GEOM_SWITCH(g, {
    if constexpr (SW == 64) {
      const auto blocks = [&](uint32_t r) { return static_cast<int64_t>(ceil_div(pairs * ceil_div(a.inter, r), kWaves)); };
      if (blocks(2) <= resident_blocks<gateup_ptr<TT, SW, CPL, 2, SELECT>>()) {
        launch_gateup_r<TT, SW, CPL, 2, SELECT>(a, shared, has_shared, keeps, sel, sel_out, act, err, pairs, stream);
      } else if (blocks(4) <= resident_blocks<gateup_ptr<TT, SW, CPL, 4, SELECT>>()) {
        launch_gateup_r<TT, SW, CPL, 4, SELECT>(a, shared, has_shared, keeps, sel, sel_out, act, err, pairs, stream);
      } else {
        launch_gateup_r<TT, SW, CPL, 8, SELECT>(a, shared, has_shared, keeps, sel, sel_out, act, err, pairs, stream);
      }
    } else {
      constexpr int R = steps_for<SW>();
      launch_gateup_r<TT, SW, CPL, R, SELECT>(a, shared, has_shared, keeps, sel, sel_out, act, err, pairs, stream);
    }
  });
  return check_launch("gateup_kernel");
}

template <class TT, int SW, int CPL, int SPW, int R>
void launch_down_r(const MqMoeArgs &a, const SharedExpert &shared, int shared_mode,
                   const typename TT::storage *shared_vec, const int32_t *keeps, const typename TT::storage *act,
                   unsigned int *err, hipStream_t stream) {
  using S = typename TT::storage;
  const dim3 grid(ceil_div(a.hidden, Slice<SW>::kRows * R), a.tokens);
  hipLaunchKernelGGL((down_combine_kernel<TT, SW, CPL, SPW, R>), grid, dim3(kThreads), 0, stream, a.routes, a.scores,
                     keeps, act, a.shared_gate, a.score_dtype, shared_mode, a.tokens, a.slots, a.inter, a.down, shared,
                     shared_vec, static_cast<S *>(a.out), a.hidden, a.group_size, a.expert_count,
                     (a.group_size == 64 || (a.flags & MQ_DECODE_GENERIC_COMBINE) != 0) ? 1u : 0u, err);
}

template <class TT, int SW, int CPL, int SPW, int R>
const void *down_ptr() {
  return reinterpret_cast<const void *>(down_combine_kernel<TT, SW, CPL, SPW, R>);
}

// Down launch for SPW sources per wave.  With 16-lane slices (bf16, at most
// two chunks per lane, at most three sources per wave) a wave takes 2, 4 or
// 8 row groups: the smallest count of at least two whose grid is resident at
// once, so that a verify batch streams in one round of blocks instead of
// rounds that each pay the route-word and weight latencies (one token: two
// row groups, measured faster than one).
template <class TT, int SW, int CPL, int SPW>
void launch_down_spw(const MqMoeArgs &a, const SharedExpert &shared, int shared_mode,
                     const typename TT::storage *shared_vec, const int32_t *keeps, const typename TT::storage *act,
                     unsigned int *err, hipStream_t stream) {
  if constexpr (TT::dtype == MQ_BF16 && SW == 16 && CPL <= 2 && SPW <= 3) {
    const auto blocks = [&](uint32_t r) {
      return static_cast<int64_t>(ceil_div(a.hidden, Slice<SW>::kRows * r)) * a.tokens;
    };
    if (blocks(2) <= resident_blocks<down_ptr<TT, SW, CPL, SPW, 2>>())
      launch_down_r<TT, SW, CPL, SPW, 2>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
    else if (blocks(4) <= resident_blocks<down_ptr<TT, SW, CPL, SPW, 4>>() || SPW == 3)
      launch_down_r<TT, SW, CPL, SPW, 4>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
    else
      launch_down_r<TT, SW, CPL, SPW, (SPW <= 2 ? 8 : 4)>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
    return;
  }
  launch_down_r<TT, SW, CPL, SPW, 1>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
}

template <class TT>
int launch_down(const MqMoeArgs &a, const SharedExpert &shared, int shared_mode, const typename TT::storage *shared_vec,
                const int32_t *keeps, const typename TT::storage *act, unsigned int *err, hipStream_t stream) {
  const Geometry g = geometry(a.inter);
  const uint32_t n_src = a.slots + (shared_mode == kSharedExpert ? 1u : 0u);
  const uint32_t per_wave = ceil_div(n_src, kWaves);
  MQ_GEOM_SWITCH(g, {
    // Sources per batch: all of a wave's sources when their registers fit.
    if constexpr (CPL == 1) {
      if (per_wave <= 1) launch_down_spw<TT, SW, CPL, 1>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
      else if (per_wave <= 2) launch_down_spw<TT, SW, CPL, 2>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
      else if (per_wave <= 3) launch_down_spw<TT, SW, CPL, 3>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
      else launch_down_spw<TT, SW, CPL, 5>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
    } else if constexpr (CPL == 2) {
      if (per_wave <= 1) launch_down_spw<TT, SW, CPL, 1>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
      else launch_down_spw<TT, SW, CPL, 2>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
    } else {
      launch_down_spw<TT, SW, CPL, 1>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
    }
  });
  return check_launch("down_combine_kernel");
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" int mq_gather_qmv(const void *x, int x_dtype, int slot_input, const MqProjection *proj,
                             const uint32_t *routes, void *out, uint32_t tokens, uint32_t slots,
                             uint32_t in_features, uint32_t out_features, uint32_t expert_count,
                             uint32_t group_size, void *stream) {
  if (x == nullptr || out == nullptr || routes == nullptr)
    return fail(MQ_ERR_INVALID, "x, routes and out are required");
  int rc = validate_proj(proj, "gather");
  if (rc) return rc;
  if ((rc = validate_shape(in_features, out_features, group_size))) return rc;
  if (tokens == 0 || slots == 0) return fail(MQ_ERR_INVALID, "tokens and slots must be positive");
  const uint32_t pairs = tokens * slots;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == MQ_BF16)
    return launch_gather_qmv<BF16T>(x, slot_input, *proj, routes, out, pairs, slots, in_features, out_features,
                                    group_size, expert_count, s);
  if (x_dtype == MQ_F32)
    return launch_gather_qmv<F32T>(x, slot_input, *proj, routes, out, pairs, slots, in_features, out_features,
                                   group_size, expert_count, s);
  return fail(MQ_ERR_INVALID, "x_dtype must be MQ_BF16 or MQ_F32");
}

extern "C" int mq_q4_qmv(const void *x, int x_dtype, const uint32_t *weight, const uint16_t *scales,
                         const uint16_t *biases, void *y, uint32_t rows_x, uint32_t out_features,
                         uint32_t in_features, uint32_t group_size, void *stream) {
  if (x == nullptr || y == nullptr || weight == nullptr || scales == nullptr || biases == nullptr)
    return fail(MQ_ERR_INVALID, "x, weight, scales, biases and y are required");
  int rc = validate_shape(in_features, out_features, group_size);
  if (rc) return rc;
  if (rows_x == 0) return fail(MQ_ERR_INVALID, "rows_x must be positive");
  MqProjection p{};
  p.weight = weight;
  p.scales = scales;
  p.biases = biases;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // One "pair" per activation row, all addressing expert 0 (routes == NULL).
  if (x_dtype == MQ_BF16)
    return launch_gather_qmv<BF16T>(x, 0, p, nullptr, y, rows_x, 1, in_features, out_features, group_size, 1u, s);
  if (x_dtype == MQ_F32)
    return launch_gather_qmv<F32T>(x, 0, p, nullptr, y, rows_x, 1, in_features, out_features, group_size, 1u, s);
  return fail(MQ_ERR_INVALID, "x_dtype must be MQ_BF16 or MQ_F32");
}

namespace mq {
namespace {

template <class TT>
int moe_decode_t(const MqMoeArgs &a, hipStream_t stream, const MqRouteArgs *route, const uint16_t *logits) {
  using S = typename TT::storage;
  const uint32_t routed_pairs = a.tokens * a.slots;
  const bool return_all = (a.flags & MQ_DECODE_RETURN_ALL) != 0;
  const bool has_shared_expert = a.shared_expert != nullptr && !return_all;
  const uint32_t pairs = routed_pairs + (has_shared_expert ? a.tokens : 0u);

  unsigned int *err = nullptr;
  int rc = device_flags(&err, stream);
  if (rc) return rc;

  // Activations [pairs, inter] in the caller's act_out (checked by validate_moe_args).
  S *act = static_cast<S *>(a.act_out);
  (void)pairs;

  SharedExpert shared{};
  if (has_shared_expert)
    for (int i = 0; i < 3; ++i) shared.p[i] = a.shared_expert[i];
  const int32_t *keeps = return_all ? nullptr : a.keeps;
  const uint32_t ne = a.expert_count;

  if (route != nullptr) {
    // Fused routed layer: the gate/up kernel runs the selection itself.
    SelectOutputs so{};
    so.inds = route->inds;
    so.scores = static_cast<uint16_t *>(route->scores);
    so.scores_raw = route->scores_raw;
    so.routes = route->routes;
    so.keeps = route->keeps;
    so.shared_gate = route->shared_gate;
    so.shared_logit = route->shared_gate;
    const SelectParams sel = select_params(*route, logits);
    rc = launch_gateup<TT, true>(a, shared, has_shared_expert, nullptr, sel, so, act, err, stream);
    if (rc) return rc;
    keeps = route->threshold < 1.0f ? route->keeps : nullptr;
  } else if (a.flags & MQ_DECODE_UNFUSED_UP) {
    // Separate gate/up QMVs then SwiGLU: bit-identical to the fused kernel.
    S *g = static_cast<S *>(a.gate_out);
    S *u = static_cast<S *>(a.up_out);
    if (g == nullptr || u == nullptr) return fail(MQ_ERR_INVALID, "unfused up path needs gate_out and up_out buffers");
    rc = launch_gather_qmv<TT>(a.x, 0, a.gate, a.routes, g, routed_pairs, a.slots, a.hidden, a.inter, a.group_size,
                               ne, stream);
    if (rc) return rc;
    rc = launch_gather_qmv<TT>(a.x, 0, a.up, a.routes, u, routed_pairs, a.slots, a.hidden, a.inter, a.group_size,
                               ne, stream);
    if (rc) return rc;
    const uint64_t n = static_cast<uint64_t>(routed_pairs) * a.inter;
    hipLaunchKernelGGL(swiglu_kernel<TT>, dim3(ceil_div(n, 256)), dim3(256), 0, stream, g, u, act, n);
    if ((rc = check_launch("swiglu_kernel"))) return rc;
    if (has_shared_expert) {
      // Only the shared pairs (the routed pairs were computed above): the
      // shared tiles come first, so a tile limit of `shared tiles` covers them.
      const Geometry g2 = geometry(a.hidden);
      MQ_GEOM_SWITCH(g2, {
        constexpr int R = steps_for<SW>();
        constexpr int kTileRows = R * Slice<SW>::kRows;
        const uint32_t tiles = a.tokens * ceil_div(a.inter, kTileRows);
        hipLaunchKernelGGL((gateup_kernel<TT, SW, CPL, R, false>), dim3(ceil_div(tiles, kWaves)), dim3(kThreads), 0,
                           stream, static_cast<const uint16_t *>(nullptr), static_cast<const uint32_t *>(nullptr),
                           static_cast<const S *>(a.x), 0u, 0u, a.tokens, a.slots, tiles, 1u, a.hidden, a.inter, 0u,
                           0.0f, 0.0f, a.gate, a.up, shared, a.routes, keeps, SelectOutputs{}, act,
                           static_cast<S *>(nullptr), static_cast<S *>(nullptr), a.group_size, ne, err);
      });
      if ((rc = check_launch("gateup_kernel"))) return rc;
    }
  } else {
    rc = launch_gateup<TT, false>(a, shared, has_shared_expert, keeps, SelectParams{}, SelectOutputs{}, act, err,
                                  stream);
    if (rc) return rc;
  }

  if (return_all) {
    if (a.down_out == nullptr) return fail(MQ_ERR_INVALID, "return_all needs down_out");
    return launch_gather_qmv<TT>(act, 1, a.down, a.routes, a.down_out, routed_pairs, a.slots, a.inter, a.hidden,
                                 a.group_size, ne, stream);
  }

  int shared_mode = kSharedNone;
  const S *shared_vec = nullptr;
  if (a.shared_y != nullptr) {
    shared_mode = kSharedY;
    shared_vec = static_cast<const S *>(a.shared_y);
  } else if (a.shared != nullptr) {
    shared_mode = kSharedParts;
    shared_vec = static_cast<const S *>(a.shared);
  } else if (has_shared_expert) {
    shared_mode = kSharedExpert;
  }
  return launch_down<TT>(a, shared, shared_mode, shared_vec, keeps, act, err, stream);
}

int validate_moe_args(const MqMoeArgs &a, bool routed_layer) {
  if (a.x == nullptr) return fail(MQ_ERR_INVALID, "x is required");
  if (!routed_layer && a.routes == nullptr) return fail(MQ_ERR_INVALID, "x and routes are required");
  if (a.tokens == 0 || a.tokens > MQ_MAX_TOKENS)
    return fail(MQ_ERR_INVALID, "tokens must be in 1..%d (got %u)", MQ_MAX_TOKENS, a.tokens);
  if (a.slots == 0 || a.slots > kMaxSlots) return fail(MQ_ERR_INVALID, "slots must be in 1..16 (got %u)", a.slots);
  if (a.act_out == nullptr)
    return fail(MQ_ERR_INVALID, "act_out is required ([tokens, slots (+1 with a shared expert), inter] activations)");
  int rc;
  if ((rc = validate_proj(&a.gate, "gate")) || (rc = validate_proj(&a.up, "up")) || (rc = validate_proj(&a.down, "down")))
    return rc;
  if ((rc = validate_shape(a.hidden, a.inter, a.group_size)) || (rc = validate_shape(a.inter, a.hidden, a.group_size)))
    return rc;
  const bool return_all = (a.flags & MQ_DECODE_RETURN_ALL) != 0;
  if (!return_all) {
    if (!routed_layer && a.scores == nullptr) return fail(MQ_ERR_INVALID, "scores are required unless return_all is set");
    if (a.out == nullptr) return fail(MQ_ERR_INVALID, "out is required");
    if (a.score_dtype != MQ_F32 && a.score_dtype != MQ_BF16) return fail(MQ_ERR_INVALID, "bad score dtype");
    if ((a.group_size == 64 || (a.flags & MQ_DECODE_GENERIC_COMBINE)) && a.x_dtype == MQ_BF16 &&
        a.score_dtype == MQ_F32)
      return fail(MQ_ERR_UNSUPPORTED,
                  "the generic combine (group 64, or MQ_DECODE_GENERIC_COMBINE) is in the score dtype, so bf16 "
                  "activations with float32 scores give a float32 result: use MQ_DECODE_RETURN_ALL and combine on "
                  "the caller's side");
    const int modes = (a.shared_y != nullptr) + (a.shared != nullptr) + (a.shared_expert != nullptr);
    if (modes > 1) return fail(MQ_ERR_INVALID, "provide shared_y, shared parts or a shared expert, not several");
    if ((a.shared != nullptr || a.shared_expert != nullptr) && a.shared_gate == nullptr)
      return fail(MQ_ERR_INVALID, "shared and shared_gate must be provided together");
    if (a.shared_expert != nullptr)
      for (int i = 0; i < 3; ++i)
        if ((rc = validate_proj(&a.shared_expert[i], "shared"))) return rc;
  }
  return MQ_OK;
}

}  // namespace
}  // namespace mq

extern "C" int mq_moe_decode(const MqMoeArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  const MqMoeArgs &a = *args;
  int rc = validate_moe_args(a, false);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.x_dtype == MQ_BF16) return moe_decode_t<BF16T>(a, s, nullptr, nullptr);
  if (a.x_dtype == MQ_F32) return moe_decode_t<F32T>(a, s, nullptr, nullptr);
  return fail(MQ_ERR_INVALID, "x_dtype must be MQ_BF16 or MQ_F32");
}

extern "C" int mq_moe_layer(const MqRouteArgs *route, const MqMoeArgs *moe, void *stream) {
  if (route == nullptr || moe == nullptr) return fail(MQ_ERR_INVALID, "route and moe args are required");
  const MqRouteArgs &r = *route;
  MqMoeArgs a = *moe;
  int rc = validate_route_args(r);
  if (rc) return rc;
  if (r.logits_in != nullptr || r.logits_out == nullptr || r.routes == nullptr || r.x == nullptr)
    return fail(MQ_ERR_INVALID, "the routed layer needs x, gate_w, logits_out and routes (no logits_in)");
  if (r.score_dtype != MQ_BF16) return fail(MQ_ERR_INVALID, "the routed layer produces bf16 scores");
  if (moe->x_dtype != MQ_BF16 || moe->x != r.x) return fail(MQ_ERR_INVALID, "the routed layer needs the same bf16 x");
  if (r.tokens != moe->tokens || r.top_k != moe->slots || r.hidden != moe->hidden)
    return fail(MQ_ERR_INVALID, "route and moe shapes disagree");
  if (moe->flags & ~MQ_DECODE_GENERIC_COMBINE)
    return fail(MQ_ERR_INVALID, "the routed layer supports no MQ_DECODE flag but MQ_DECODE_GENERIC_COMBINE");
  if ((moe->shared_expert != nullptr) != (r.shared_gate != nullptr))
    return fail(MQ_ERR_INVALID, "a shared expert needs the router's shared_gate output and vice versa");
  a.routes = r.routes;
  a.scores = r.scores;
  a.score_dtype = MQ_BF16;
  a.shared_gate = r.shared_gate;
  a.keeps = r.keeps;
  if ((rc = validate_moe_args(a, true))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (r.tokens > static_cast<uint32_t>(kWaves)) {
    // More tokens than a block has waves: one selection pass, then the expert
    // kernels with routes given.  Folded into every gate/up block (as for up
    // to four tokens, one per wave, in parallel) the selection would take
    // several rounds per block, and the larger grid several rounds of blocks.
    if ((rc = mq_route_topk(&r, stream))) return rc;
    if (r.threshold >= 1.0f) a.keeps = nullptr;
    return moe_decode_t<BF16T>(a, s, nullptr, nullptr);
  }
  rc = launch_router_logits(r.x, r.gate_w, r.shared_gate != nullptr ? r.shared_gate_w : nullptr, r.logits_out,
                            r.shared_gate, r.tokens, r.hidden, r.experts, s);
  if (rc) return rc;
  return moe_decode_t<BF16T>(a, s, &r, r.logits_out);
}
