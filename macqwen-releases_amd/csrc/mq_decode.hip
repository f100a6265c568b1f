// Decode-path kernels for gfx950: Q4 QMV, fused gate/up + SwiGLU, and
// down + score combine + shared epilogue.
//
// Work mapping.  A wave64 is four 16-lane slices (one DPP row each).  A slice
// computes one output row: lane i of the slice owns the CPL consecutive
// 32-input chunks [i*CPL, (i+1)*CPL) of the row, loads them with 128-bit
// loads (one chunk = 4 uint32 = 32 nibbles), dequantises in registers into
// bf16 pairs (128+q) and accumulates with v_dot2_f32_bf16 against the
// activation chunk it keeps in registers.  The row sum is a 4-step DPP
// reduction inside the slice, so a wave retires four rows per step with no
// LDS traffic.  Input widths that are multiples of 512 (16 lanes x 32) use
// every lane; other multiples of 32 mask the tail chunks.
//
// Rounding points follow the reference executor
// (models/flashnext/metal_runtime.py:231-336): every projection output is
// rounded to the activation type T, the SwiGLU epilogue rounds each step to
// T, and the score combine accumulates float(T(d)) * float(score) in float32
// with no contraction before the final T rounding and shared add.
#include <math.h>

#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kWaves = 4;           // waves per block
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWave = 4;     // one row per 16-lane slice

// ------------------------------------------------------------------ activations

// Activation chunk(s) of one lane: bf16 inputs need one pair chunk, float32
// inputs are split into bf16 hi + lo chunks (x = hi + lo to 16 bits).
template <class TT>
struct XLane;

template <>
struct XLane<BF16T> {
  static constexpr int kParts = 1;
  XChunk part[1];
  float bias_sum;  // sum of the inputs, multiplies the group bias
  __device__ __forceinline__ void load(const uint16_t *src, bool valid) {
    if (valid) {
      const uint4 *v = reinterpret_cast<const uint4 *>(src);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 q = v[j];
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
        pairs_from_words(u, &part[0].p[4 * j]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) part[0].p[i] = 0u;
    }
    part[0].osum = chunk_pair_sum(part[0]);
    bias_sum = part[0].osum;
  }
  __device__ __forceinline__ void load_words(const uint32_t w[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) pairs_from_words(&w[4 * j], &part[0].p[4 * j]);
    part[0].osum = chunk_pair_sum(part[0]);
    bias_sum = part[0].osum;
  }
};

template <>
struct XLane<F32T> {
  static constexpr int kParts = 2;
  XChunk part[2];
  float bias_sum;
  __device__ __forceinline__ void load(const float *src, bool valid) {
    uint32_t hi[16], lo[16];
    float s = 0.0f;
    if (valid) {
      const float4 *v = reinterpret_cast<const float4 *>(src);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float4 q = v[j];
        const float f[4] = {q.x, q.y, q.z, q.w};
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
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) hi[i] = lo[i] = 0u;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pairs_from_words(&hi[4 * j], &part[0].p[4 * j]);
      pairs_from_words(&lo[4 * j], &part[1].p[4 * j]);
    }
    part[0].osum = chunk_pair_sum(part[0]);
    part[1].osum = chunk_pair_sum(part[1]);
    bias_sum = s;
  }
};

// ------------------------------------------------------------------ weight rows

template <int CPL>
struct RowLoad {
  uint4 w[CPL];
  uint16_t s[CPL];
  uint16_t b[CPL];
};

// Issue the loads of one lane's chunks of row `row` (masked chunks read as 0).
template <int CPL>
__device__ __forceinline__ void load_row(RowLoad<CPL> &r, const ExpertPtrs &e, uint32_t row,
                                         uint32_t in_w, uint32_t group, int li, bool row_ok) {
  const uint32_t chunks = in_w >> 5;
  const uint32_t words = in_w >> 3;
  const uint32_t groups = in_w / group;
  const uint32_t shift = group == 64 ? 1 : 0;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t c = static_cast<uint32_t>(li) * CPL + j;
    if (row_ok && c < chunks) {
      r.w[j] = *reinterpret_cast<const uint4 *>(e.w + static_cast<uint64_t>(row) * words + c * 4);
      const uint64_t gi = static_cast<uint64_t>(row) * groups + (c >> shift);
      r.s[j] = e.s[gi];
      r.b[j] = e.b[gi];
    } else {
      r.w[j] = make_uint4(0u, 0u, 0u, 0u);
      r.s[j] = 0;
      r.b[j] = 0;
    }
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
    for (int p = 0; p < XLane<TT>::kParts; ++p) dq += q4_chunk_dot(r.w[j], x[j].part[p]);
    acc = fmaf(bf16_to_f32(r.s[j]), dq, acc);
    acc = fmaf(bf16_to_f32(r.b[j]), x[j].bias_sum, acc);
  }
  return acc;
}

template <class TT, int CPL>
__device__ __forceinline__ void load_x(XLane<TT> *x, const typename TT::storage *src, uint32_t in_w,
                                       int li) {
  const uint32_t chunks = in_w >> 5;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t c = static_cast<uint32_t>(li) * CPL + j;
    x[j].load(src + c * 32, c < chunks);
  }
}

// ------------------------------------------------------------------ SwiGLU

// MLX's sigmoid sequence with each step rounded to T
// (models/flashnext/metal_runtime.py:278-284): m=|g|; e=T(exp(m));
// d=T(1+e); s=T(1/d); sig = g<0 ? s : T(1-s).  exp is the float32
// exponential correctly rounded (evaluated in double).
template <class TT>
__device__ __forceinline__ float sigmoid_t(float g) {
  const float m = fabsf(g);
  const float e = TT::round(static_cast<float>(exp(static_cast<double>(m))));
  const float d = TT::round(__fadd_rn(1.0f, e));
  const float s = TT::round(__fdiv_rn(1.0f, d));
  const float om = TT::round(__fsub_rn(1.0f, s));
  return g < 0.0f ? s : om;
}

// act = T(T(g * sigmoid_T(g)) * u) for T-valued g and u.
template <class TT>
__device__ __forceinline__ float swiglu_t(float g, float u) {
  const float sig = sigmoid_t<TT>(g);
  const float silu = TT::round(__fmul_rn(g, sig));
  return TT::round(__fmul_rn(silu, u));
}

// ------------------------------------------------------------------ kernels

// The shared expert's three projections, passed by value as a kernel argument.
struct SharedExpert {
  MqProjection p[3];  // gate, up, down; addressed with route word 0
};

// Projection QMV: out[pair, row] = T(W_route(pair) . x(pair)).
// Grid: one wave per 4-row tile; tiles enumerate (pair, row/4).
template <class TT, int CPL>
__global__ __launch_bounds__(kThreads) void gather_qmv_kernel(
    const typename TT::storage *__restrict__ x, int slot_input, MqProjection proj,
    const uint32_t *__restrict__ routes, typename TT::storage *__restrict__ out,
    uint32_t pairs, uint32_t slots, uint32_t in_w, uint32_t out_w, uint32_t group) {
  using S = typename TT::storage;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int slice = lane >> 4;
  const uint32_t tiles_per_pair = (out_w + kRowsPerWave - 1) / kRowsPerWave;
  const uint32_t tile = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (tile >= pairs * tiles_per_pair) return;  // wave-uniform
  const uint32_t pair = tile / tiles_per_pair;
  const uint32_t row = (tile % tiles_per_pair) * kRowsPerWave + slice;
  const bool row_ok = row < out_w;
  const uint32_t word = routes ? routes[pair] : 0u;
  const ExpertPtrs e = expert_ptrs(proj, word, out_w, in_w, group);

  RowLoad<CPL> r;
  load_row<CPL>(r, e, row, in_w, group, li, row_ok);
  const uint32_t token = pair / slots;
  const S *src = x + static_cast<uint64_t>(slot_input ? pair : token) * in_w;
  XLane<TT> xl[CPL];
  load_x<TT, CPL>(xl, src, in_w, li);
  const float v = row16_sum(row_partial<TT, CPL>(r, xl));
  if (li == 0 && row_ok) out[static_cast<uint64_t>(pair) * out_w + row] = TT::store(v);
}

// Fused gate + up + SwiGLU: act[pair, row] = swiglu(T(gate), T(up)).
// Pairs [0, tokens*slots) are routed; with a shared expert, pairs
// [tokens*slots, tokens*slots + tokens) are the shared expert of each token.
template <class TT, int CPL>
__global__ __launch_bounds__(kThreads) void gateup_swiglu_kernel(
    const typename TT::storage *__restrict__ x, MqProjection gate, MqProjection up,
    SharedExpert shared, const uint32_t *__restrict__ routes,
    const int32_t *__restrict__ keeps, typename TT::storage *__restrict__ act,
    typename TT::storage *__restrict__ gate_out, typename TT::storage *__restrict__ up_out,
    uint32_t tokens, uint32_t slots, uint32_t pair_base, uint32_t pairs, uint32_t hidden,
    uint32_t inter, uint32_t group) {
  using S = typename TT::storage;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int slice = lane >> 4;
  const uint32_t tiles_per_pair = (inter + kRowsPerWave - 1) / kRowsPerWave;
  const uint32_t tile = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (tile >= pairs * tiles_per_pair) return;
  const uint32_t pair = pair_base + tile / tiles_per_pair;
  const uint32_t row = (tile % tiles_per_pair) * kRowsPerWave + slice;
  const bool row_ok = row < inter;
  const uint32_t routed_pairs = tokens * slots;
  const bool is_shared = pair >= routed_pairs;
  const uint32_t token = is_shared ? pair - routed_pairs : pair / slots;
  if (!is_shared && keeps != nullptr && (pair % slots) >= static_cast<uint32_t>(keeps[token])) return;

  MqProjection gp, upp;
  uint32_t word;
  if (is_shared) {
    gp = shared.p[0];
    upp = shared.p[1];
    word = 0u;
  } else {
    gp = gate;
    upp = up;
    word = routes[pair];
  }
  const ExpertPtrs eg = expert_ptrs(gp, word, inter, hidden, group);
  const ExpertPtrs eu = expert_ptrs(upp, word, inter, hidden, group);
  RowLoad<CPL> rg, ru;
  load_row<CPL>(rg, eg, row, hidden, group, li, row_ok);
  load_row<CPL>(ru, eu, row, hidden, group, li, row_ok);
  XLane<TT> xl[CPL];
  load_x<TT, CPL>(xl, x + static_cast<uint64_t>(token) * hidden, hidden, li);
  const float g = row16_sum(row_partial<TT, CPL>(rg, xl));
  const float u = row16_sum(row_partial<TT, CPL>(ru, xl));
  if (li == 0 && row_ok) {
    const float gt = TT::round(g);
    const float ut = TT::round(u);
    const uint64_t idx = static_cast<uint64_t>(pair) * inter + row;
    act[idx] = TT::store(swiglu_t<TT>(gt, ut));
    if (gate_out != nullptr && !is_shared) gate_out[idx] = TT::store(gt);
    if (up_out != nullptr && !is_shared) up_out[idx] = TT::store(ut);
  }
}

// SwiGLU over precomputed T gate/up projections (unfused path).
template <class TT>
__global__ void swiglu_kernel(const typename TT::storage *__restrict__ g,
                              const typename TT::storage *__restrict__ u,
                              typename TT::storage *__restrict__ out, uint64_t n) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = TT::store(swiglu_t<TT>(TT::load(g[i]), TT::load(u[i])));
}

enum SharedMode : int { kSharedNone = 0, kSharedY = 1, kSharedParts = 2, kSharedExpert = 3 };

// Down + score combine + shared epilogue for one token and four output rows
// per wave.  For each routed slot s < keep: d = T(W_down . act[t,s]);
// acc += float(d) * float(score[t,s]) in float32 with no contraction
// (models/flashnext/metal_runtime.py:291-336).  The activations of the
// block's token are staged in LDS once per block.
template <class TT, int CPL>
__global__ __launch_bounds__(kThreads) void down_combine_kernel(
    const typename TT::storage *__restrict__ act, MqProjection down,
    SharedExpert shared, const uint32_t *__restrict__ routes,
    const void *__restrict__ scores, int score_dtype, const int32_t *__restrict__ keeps,
    int shared_mode, const typename TT::storage *__restrict__ shared_vec,
    const uint16_t *__restrict__ shared_gate, typename TT::storage *__restrict__ out,
    uint32_t tokens, uint32_t slots, uint32_t hidden, uint32_t inter, uint32_t group,
    uint32_t tiles_per_token) {
  using S = typename TT::storage;
  extern __shared__ __align__(16) unsigned char smem[];
  S *lds_act = reinterpret_cast<S *>(smem);

  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int slice = lane >> 4;
  const uint32_t token = blockIdx.y;
  const uint32_t tile = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const uint32_t row = tile * kRowsPerWave + slice;
  const bool row_ok = tile < tiles_per_token && row < hidden;
  const uint32_t keep = keeps ? static_cast<uint32_t>(keeps[token]) : slots;
  const bool with_shared_expert = shared_mode == kSharedExpert;
  const uint32_t n_src = slots + (with_shared_expert ? 1u : 0u);

  // Stage this token's activations: routed pairs, then the shared pair.
  const uint32_t routed_pairs = tokens * slots;
  const uint32_t elems = n_src * inter;
  const uint32_t vec = 16 / sizeof(S);
  for (uint32_t i = threadIdx.x * vec; i < elems; i += kThreads * vec) {
    const uint32_t src_pair_local = i / inter;
    const uint32_t col = i % inter;
    const uint64_t pair = src_pair_local < slots
                              ? static_cast<uint64_t>(token) * slots + src_pair_local
                              : static_cast<uint64_t>(routed_pairs) + token;
    if (src_pair_local < slots && src_pair_local >= keep) continue;
    *reinterpret_cast<uint4 *>(&lds_act[i]) =
        *reinterpret_cast<const uint4 *>(&act[pair * inter + col]);
  }
  __syncthreads();
  if (!(tile < tiles_per_token)) return;

  float acc = 0.0f;
  for (uint32_t s = 0; s < slots; ++s) {
    if (s >= keep) break;  // padded slots carry score 0 and add exact zeros
    const uint32_t pair = token * slots + s;
    const ExpertPtrs e = expert_ptrs(down, routes[pair], hidden, inter, group);
    RowLoad<CPL> r;
    load_row<CPL>(r, e, row, inter, group, li, row_ok);
    XLane<TT> xl[CPL];
    load_x<TT, CPL>(xl, lds_act + s * inter, inter, li);
    const float v = row16_sum(row_partial<TT, CPL>(r, xl));
    const float score = score_dtype == MQ_BF16
                            ? bf16_to_f32(static_cast<const uint16_t *>(scores)[pair])
                            : static_cast<const float *>(scores)[pair];
    acc = __fadd_rn(acc, __fmul_rn(TT::round(v), score));
  }
  float shared_term = 0.0f;
  bool has_shared = false;
  if (with_shared_expert) {
    const ExpertPtrs e = expert_ptrs(shared.p[2], 0u, hidden, inter, group);
    RowLoad<CPL> r;
    load_row<CPL>(r, e, row, inter, group, li, row_ok);
    XLane<TT> xl[CPL];
    load_x<TT, CPL>(xl, lds_act + slots * inter, inter, li);
    const float v = row16_sum(row_partial<TT, CPL>(r, xl));
    shared_term = TT::round(__fmul_rn(TT::round(v), bf16_to_f32(shared_gate[token])));
    has_shared = true;
  }
  if (li == 0 && row_ok) {
    const uint64_t idx = static_cast<uint64_t>(token) * hidden + row;
    const float routed = TT::round(acc);
    float final_value = routed;
    if (shared_mode == kSharedY) {
      final_value = __fadd_rn(routed, TT::load(shared_vec[idx]));
    } else if (shared_mode == kSharedParts) {
      const float comp = TT::round(__fmul_rn(TT::load(shared_vec[idx]), bf16_to_f32(shared_gate[token])));
      final_value = __fadd_rn(routed, comp);
    } else if (has_shared) {
      final_value = __fadd_rn(routed, shared_term);
    }
    out[idx] = TT::store(final_value);
  }
}

// ------------------------------------------------------------------ dispatch helpers

inline int cpl_for(uint32_t in_w) {
  const uint32_t chunks = in_w / 32;
  return static_cast<int>((chunks + 15) / 16);
}

#define MQ_CPL_SWITCH(cpl, BODY)                  \
  switch (cpl) {                                  \
    case 1: { constexpr int CPL = 1; BODY; } break; \
    case 2: { constexpr int CPL = 2; BODY; } break; \
    case 3: { constexpr int CPL = 3; BODY; } break; \
    case 4: { constexpr int CPL = 4; BODY; } break; \
    case 5: { constexpr int CPL = 5; BODY; } break; \
    case 6: { constexpr int CPL = 6; BODY; } break; \
    case 7: { constexpr int CPL = 7; BODY; } break; \
    case 8: { constexpr int CPL = 8; BODY; } break; \
    default: return fail(MQ_ERR_UNSUPPORTED, "input width needs %d chunks per lane (max 8)", cpl); \
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
  return MQ_OK;
}

template <class TT>
int launch_gather_qmv(const void *x, int slot_input, const MqProjection &proj, const uint32_t *routes,
                      void *out, uint32_t pairs, uint32_t slots, uint32_t in_w, uint32_t out_w,
                      uint32_t group, hipStream_t stream) {
  using S = typename TT::storage;
  const uint32_t tiles = pairs * ceil_div(out_w, kRowsPerWave);
  const dim3 grid(ceil_div(tiles, kWaves));
  MQ_CPL_SWITCH(cpl_for(in_w), {
    hipLaunchKernelGGL((gather_qmv_kernel<TT, CPL>), grid, dim3(kThreads), 0, stream,
                       static_cast<const S *>(x), slot_input, proj, routes, static_cast<S *>(out),
                       pairs, slots, in_w, out_w, group);
  });
  return check_launch("gather_qmv_kernel");
}

}  // namespace

}  // namespace mq

using namespace mq;

extern "C" int mq_gather_qmv(const void *x, int x_dtype, int slot_input, const MqProjection *proj,
                             const uint32_t *routes, void *out, uint32_t tokens, uint32_t slots,
                             uint32_t in_features, uint32_t out_features, uint32_t expert_count,
                             uint32_t group_size, void *stream) {
  if (x == nullptr || out == nullptr || routes == nullptr) return fail(MQ_ERR_INVALID, "x, routes and out are required");
  int rc = validate_proj(proj, "gather");
  if (rc) return rc;
  if ((rc = validate_shape(in_features, out_features, group_size))) return rc;
  if (tokens == 0 || slots == 0) return fail(MQ_ERR_INVALID, "tokens and slots must be positive");
  (void)expert_count;
  const uint32_t pairs = tokens * slots;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == MQ_BF16)
    return launch_gather_qmv<BF16T>(x, slot_input, *proj, routes, out, pairs, slots, in_features,
                                    out_features, group_size, s);
  if (x_dtype == MQ_F32)
    return launch_gather_qmv<F32T>(x, slot_input, *proj, routes, out, pairs, slots, in_features,
                                   out_features, group_size, s);
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
    return launch_gather_qmv<BF16T>(x, 0, p, nullptr, y, rows_x, 1, in_features, out_features,
                                    group_size, s);
  if (x_dtype == MQ_F32)
    return launch_gather_qmv<F32T>(x, 0, p, nullptr, y, rows_x, 1, in_features, out_features,
                                   group_size, s);
  return fail(MQ_ERR_INVALID, "x_dtype must be MQ_BF16 or MQ_F32");
}

namespace mq {
namespace {

template <class TT>
int moe_decode_t(const MqMoeArgs &a, hipStream_t stream) {
  using S = typename TT::storage;
  const uint32_t routed_pairs = a.tokens * a.slots;
  const bool return_all = (a.flags & MQ_DECODE_RETURN_ALL) != 0;
  const bool has_shared_expert = a.shared_expert != nullptr && !return_all;
  const uint32_t pairs = routed_pairs + (has_shared_expert ? a.tokens : 0u);

  // Activations: caller buffer or a library scratch buffer.
  S *act = static_cast<S *>(a.act_out);
  static thread_local void *scratch = nullptr;
  static thread_local size_t scratch_bytes = 0;
  static thread_local int scratch_dev = -1;
  int device = 0;
  MQ_TRY_HIP(hipGetDevice(&device));
  const size_t need = static_cast<size_t>(pairs) * a.inter * sizeof(S);
  if (act == nullptr) {
    if (scratch == nullptr || scratch_bytes < need || scratch_dev != device) {
      if (scratch != nullptr && scratch_dev == device) {
        MQ_TRY_HIP(hipDeviceSynchronize());
        (void)hipFree(scratch);
      }
      scratch = nullptr;
      MQ_TRY_HIP(hipMalloc(&scratch, need));
      scratch_bytes = need;
      scratch_dev = device;
    }
    act = static_cast<S *>(scratch);
  }

  SharedExpert shared_dev{};
  if (has_shared_expert) {
    for (int i = 0; i < 3; ++i) shared_dev.p[i] = a.shared_expert[i];
  }
  const int32_t *keeps = return_all ? nullptr : a.keeps;

  if (a.flags & MQ_DECODE_UNFUSED_UP) {
    // Separate gate/up QMVs then SwiGLU: bit-identical to the fused kernel.
    S *g = static_cast<S *>(a.gate_out);
    S *u = static_cast<S *>(a.up_out);
    if (g == nullptr || u == nullptr)
      return fail(MQ_ERR_INVALID, "unfused up path needs gate_out and up_out buffers");
    int rc = launch_gather_qmv<TT>(a.x, 0, a.gate, a.routes, g, routed_pairs, a.slots, a.hidden,
                                   a.inter, a.group_size, stream);
    if (rc) return rc;
    rc = launch_gather_qmv<TT>(a.x, 0, a.up, a.routes, u, routed_pairs, a.slots, a.hidden, a.inter,
                               a.group_size, stream);
    if (rc) return rc;
    const uint64_t n = static_cast<uint64_t>(routed_pairs) * a.inter;
    hipLaunchKernelGGL(swiglu_kernel<TT>, dim3(ceil_div(n, 256)), dim3(256), 0, stream, g, u, act, n);
    if ((rc = check_launch("swiglu_kernel"))) return rc;
    if (has_shared_expert) {
      // Shared pairs follow the routed pairs: pair_base = tokens * slots.
      const uint32_t tiles = a.tokens * ceil_div(a.inter, kRowsPerWave);
      MQ_CPL_SWITCH(cpl_for(a.hidden), {
        hipLaunchKernelGGL((gateup_swiglu_kernel<TT, CPL>), dim3(ceil_div(tiles, kWaves)), dim3(kThreads), 0,
                           stream, static_cast<const S *>(a.x), a.gate, a.up, shared_dev, a.routes,
                           keeps, act, nullptr, nullptr, a.tokens, a.slots, routed_pairs, a.tokens,
                           a.hidden, a.inter, a.group_size);
      });
      if ((rc = check_launch("gateup_swiglu_kernel"))) return rc;
    }
  } else {
    const uint32_t tiles = pairs * ceil_div(a.inter, kRowsPerWave);
    MQ_CPL_SWITCH(cpl_for(a.hidden), {
      hipLaunchKernelGGL((gateup_swiglu_kernel<TT, CPL>), dim3(ceil_div(tiles, kWaves)), dim3(kThreads), 0,
                         stream, static_cast<const S *>(a.x), a.gate, a.up, shared_dev, a.routes, keeps,
                         act, static_cast<S *>(a.gate_out), static_cast<S *>(a.up_out), a.tokens, a.slots,
                         0u, pairs, a.hidden, a.inter, a.group_size);
    });
    int rc = check_launch("gateup_swiglu_kernel");
    if (rc) return rc;
  }

  if (return_all) {
    if (a.down_out == nullptr) return fail(MQ_ERR_INVALID, "return_all needs down_out");
    return launch_gather_qmv<TT>(act, 1, a.down, a.routes, a.down_out, routed_pairs, a.slots, a.inter,
                                 a.hidden, a.group_size, stream);
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
  const uint32_t tiles_per_token = ceil_div(a.hidden, kRowsPerWave);
  const dim3 grid(ceil_div(tiles_per_token, kWaves), a.tokens);
  const size_t lds = static_cast<size_t>(a.slots + 1) * a.inter * sizeof(S);
  if (lds > 160 * 1024) return fail(MQ_ERR_UNSUPPORTED, "activation staging needs %zu bytes of LDS", lds);
  MQ_CPL_SWITCH(cpl_for(a.inter), {
    hipLaunchKernelGGL((down_combine_kernel<TT, CPL>), grid, dim3(kThreads), lds, stream, act, a.down,
                       shared_dev, a.routes, a.scores, a.score_dtype, keeps, shared_mode, shared_vec,
                       a.shared_gate, static_cast<S *>(a.out), a.tokens, a.slots, a.hidden, a.inter,
                       a.group_size, tiles_per_token);
  });
  return check_launch("down_combine_kernel");
}

}  // namespace
}  // namespace mq

extern "C" int mq_moe_decode(const MqMoeArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  const MqMoeArgs &a = *args;
  if (a.x == nullptr || a.routes == nullptr) return fail(MQ_ERR_INVALID, "x and routes are required");
  if (a.tokens == 0 || a.tokens > 64) return fail(MQ_ERR_INVALID, "tokens must be in 1..64 (got %u)", a.tokens);
  if (a.slots == 0 || a.slots > 16) return fail(MQ_ERR_INVALID, "slots must be in 1..16 (got %u)", a.slots);
  int rc;
  if ((rc = validate_proj(&a.gate, "gate")) || (rc = validate_proj(&a.up, "up")) ||
      (rc = validate_proj(&a.down, "down")))
    return rc;
  if ((rc = validate_shape(a.hidden, a.inter, a.group_size)) ||
      (rc = validate_shape(a.inter, a.hidden, a.group_size)))
    return rc;
  const bool return_all = (a.flags & MQ_DECODE_RETURN_ALL) != 0;
  if (!return_all) {
    if (a.scores == nullptr) return fail(MQ_ERR_INVALID, "scores are required unless return_all is set");
    if (a.out == nullptr) return fail(MQ_ERR_INVALID, "out is required");
    if (a.score_dtype != MQ_F32 && a.score_dtype != MQ_BF16) return fail(MQ_ERR_INVALID, "bad score dtype");
    const int modes = (a.shared_y != nullptr) + (a.shared != nullptr) + (a.shared_expert != nullptr);
    if (modes > 1) return fail(MQ_ERR_INVALID, "provide shared_y, shared parts or a shared expert, not several");
    if ((a.shared != nullptr || a.shared_expert != nullptr) && a.shared_gate == nullptr)
      return fail(MQ_ERR_INVALID, "shared and shared_gate must be provided together");
    if (a.shared_expert != nullptr) {
      for (int i = 0; i < 3; ++i)
        if ((rc = validate_proj(&a.shared_expert[i], "shared"))) return rc;
    }
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.x_dtype == MQ_BF16) return moe_decode_t<BF16T>(a, s);
  if (a.x_dtype == MQ_F32) return moe_decode_t<F32T>(a, s);
  return fail(MQ_ERR_INVALID, "x_dtype must be MQ_BF16 or MQ_F32");
}
