// Router chain for gfx950: gate GEMV, softmax, top-k, renorm, adaptive keep,
// slot lookup and the shared-expert sigmoid gate.
//
// The reference chain is softmax(precise) -> argpartition top-k ->
// take_along_axis -> renorm (models/flashnext/compiled.py:61-71,
// models/flashnext/adaptive_topk.py:53-64, 256-261).  Logits and softmax are
// evaluated in float64 and rounded once to bf16, so the bf16 gates are the
// correctly rounded values; top-k then selects on those bits with the order
// "gate descending, expert ascending", making indices, scores and route words
// reproducible bit for bit (mq_select.h).
#include <math.h>

#include "mq_internal.h"
#include "mq_select.h"

namespace mq {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_nt(const uint16_t *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// bf16 dot of one 32-value chunk: products are exact in float32 (bf16 x bf16),
// accumulated in float64 in two independent chains (even and odd inputs).
__device__ __forceinline__ double chunk_dot_f64(const uint4 *a, const uint4 *b) {
  double acc0 = 0.0, acc1 = 0.0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t ua[4] = {a[j].x, a[j].y, a[j].z, a[j].w};
    const uint32_t ub[4] = {b[j].x, b[j].y, b[j].z, b[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a0 = __uint_as_float(ua[k] << 16), a1 = __uint_as_float(ua[k] & 0xffff0000u);
      const float b0 = __uint_as_float(ub[k] << 16), b1 = __uint_as_float(ub[k] & 0xffff0000u);
      acc0 += static_cast<double>(a0 * b0);
      acc1 += static_cast<double>(a1 * b1);
    }
  }
  return acc0 + acc1;
}

// logits[t, e] = bf16(sum_k x[t,k] * W[e,k]) for e < routed_rows; the extra
// row (when shared_gate_w is set) is the shared-expert gate, written to
// shared_logit[t].  One wave per weight row (lane = 32-input chunk); the
// tokens go in groups of kTokenGroup, spread over gridDim.y blocks per row
// (group blockIdx.y, then every gridDim.y-th).  The weight row is loaded once
// per block (non-temporal), and a group's activation loads, dot chains and
// wave sums are independent of one another.
constexpr uint32_t kTokenGroup = 4;      // tokens per group
constexpr uint32_t kMaxGroupBlocks = 64;  // blocks per weight row

// Logits of tokens t0 .. t0 + G - 1 (all below `tokens`) for the wave's row.
template <uint32_t G>
__device__ __forceinline__ void row_logits(const uint4 (&wv)[4][4], const uint16_t *__restrict__ x, uint32_t t0,
                                           uint32_t hidden, uint32_t chunks, int lane, uint32_t row,
                                           uint32_t routed_rows, uint16_t *__restrict__ logits,
                                           uint16_t *__restrict__ shared_logit) {
  double acc[G];
#pragma unroll
  for (uint32_t g = 0; g < G; ++g) acc[g] = 0.0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t c = lane + 64 * j;
    if (c < chunks) {
      uint4 xv[G][4];
#pragma unroll
      for (uint32_t g = 0; g < G; ++g) {
        const uint4 *xr = reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(t0 + g) * hidden + c * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) xv[g][q] = xr[q];
      }
#pragma unroll
      for (uint32_t g = 0; g < G; ++g) acc[g] += chunk_dot_f64(wv[j], xv[g]);
    }
  }
#pragma unroll
  for (uint32_t g = 0; g < G; ++g) acc[g] = wave_sum_f64_uniform(acc[g]);
  if (lane == 0) {
#pragma unroll
    for (uint32_t g = 0; g < G; ++g) {
      const uint16_t v = f64_to_bf16(acc[g]);
      if (row < routed_rows)
        logits[static_cast<uint64_t>(t0 + g) * routed_rows + row] = v;
      else
        shared_logit[t0 + g] = v;
    }
  }
}

constexpr uint32_t kLogitsWaves = 1;  // one weight row per block: the rows spread over every CU

__global__ __launch_bounds__(64 * kLogitsWaves) void router_logits_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate_w,
    const uint16_t *__restrict__ shared_gate_w, uint16_t *__restrict__ logits,
    uint16_t *__restrict__ shared_logit, uint32_t tokens, uint32_t hidden, uint32_t routed_rows) {
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * kLogitsWaves + (threadIdx.x >> 6);
  const uint32_t rows = routed_rows + (shared_gate_w ? 1u : 0u);
  if (row >= rows) return;
  const uint16_t *w = row < routed_rows ? gate_w + static_cast<uint64_t>(row) * hidden : shared_gate_w;
  const uint32_t chunks = hidden >> 5;
  uint4 wv[4][4];  // hidden <= 8192: at most four 32-input chunks per lane
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t c = lane + 64 * j;
#pragma unroll
    for (int q = 0; q < 4; ++q) wv[j][q] = c < chunks ? ld_nt(w + c * 32 + q * 8) : make_uint4(0, 0, 0, 0);
  }
  const uint32_t groups = (tokens + kTokenGroup - 1u) / kTokenGroup;
  for (uint32_t grp = blockIdx.y; grp < groups; grp += gridDim.y) {
    const uint32_t t0 = grp * kTokenGroup;
    if (tokens - t0 >= kTokenGroup) {
      row_logits<kTokenGroup>(wv, x, t0, hidden, chunks, lane, row, routed_rows, logits, shared_logit);
    } else {  // the last 1..3 tokens one at a time (a single token pays for no idle chains)
      for (uint32_t t = t0; t < tokens; ++t)
        row_logits<1>(wv, x, t, hidden, chunks, lane, row, routed_rows, logits, shared_logit);
    }
  }
}

struct SelectArgs {
  SelectParams p;
  const uint16_t *shared_logit;
  uint32_t *inds;
  void *scores;
  int score_dtype;
  uint16_t *scores_raw;
  uint32_t *routes;
  int32_t *keeps;
  uint16_t *shared_gate;
  uint32_t tokens;
};

// One wave per token.
__global__ __launch_bounds__(kThreads) void router_select_kernel(SelectArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (t >= a.tokens) return;
  const SelectLane s = select_token(a.p, t, lane);
  const uint32_t k = a.p.top_k;
  const uint64_t base = static_cast<uint64_t>(t) * k;
  if (static_cast<uint32_t>(lane) < k) {
    a.inds[base + lane] = s.ind;
    if (a.score_dtype == MQ_BF16)
      static_cast<uint16_t *>(a.scores)[base + lane] = f32_to_bf16(s.score);
    else
      static_cast<float *>(a.scores)[base + lane] = s.score;
    if (a.scores_raw) a.scores_raw[base + lane] = f32_to_bf16(s.raw);
    if (a.routes) a.routes[base + lane] = s.word;
  } else if (lane == 63) {
    if (a.keeps) a.keeps[t] = static_cast<int32_t>(s.keep);
    if (a.shared_gate) a.shared_gate[t] = f32_to_bf16(sigmoid_bf16(bf16_to_f32(a.shared_logit[t])));
  }
}

}  // namespace

int launch_router_logits(const uint16_t *x, const uint16_t *gate_w, const uint16_t *shared_gate_w,
                         uint16_t *logits, uint16_t *shared_logit, uint32_t tokens, uint32_t hidden,
                         uint32_t routed_rows, hipStream_t stream) {
  if (hidden > 8192) return fail(MQ_ERR_UNSUPPORTED, "router hidden size %u exceeds 8192", hidden);
  const uint32_t rows = routed_rows + (shared_gate_w ? 1u : 0u);
  if (rows == 0) return MQ_OK;
  const uint32_t group_blocks = std::min(ceil_div(tokens, kTokenGroup), kMaxGroupBlocks);
  hipLaunchKernelGGL(router_logits_kernel, dim3(ceil_div(rows, kLogitsWaves), group_blocks), dim3(64 * kLogitsWaves), 0,
                     stream, x, gate_w, shared_gate_w, logits, shared_logit, tokens, hidden, routed_rows);
  return check_launch("router_logits_kernel");
}

int validate_route_args(const MqRouteArgs &a) {
  if (a.tokens == 0) return fail(MQ_ERR_INVALID, "tokens must be positive");
  if (a.experts == 0 || a.experts > MQ_MAX_EXPERTS)
    return fail(MQ_ERR_INVALID, "experts must be in 1..%d (got %u)", MQ_MAX_EXPERTS, a.experts);
  if (a.top_k == 0 || a.top_k > static_cast<uint32_t>(kSelMaxTopK) || a.top_k > a.experts)
    return fail(MQ_ERR_INVALID, "top_k must be in 1..min(16, experts) (got %u)", a.top_k);
  if (a.inds == nullptr || a.scores == nullptr) return fail(MQ_ERR_INVALID, "inds and scores are required");
  if (a.score_dtype != MQ_F32 && a.score_dtype != MQ_BF16) return fail(MQ_ERR_INVALID, "bad score dtype");
  if (a.logits_in == nullptr && (a.x == nullptr || a.gate_w == nullptr))
    return fail(MQ_ERR_INVALID, "x and gate_w are required without logits_in");
  if (a.shared_gate != nullptr && (a.shared_gate_w == nullptr || a.x == nullptr))
    return fail(MQ_ERR_INVALID, "shared_gate output needs x and shared_gate_w");
  if (a.x != nullptr && (a.hidden == 0 || a.hidden % 32))
    return fail(MQ_ERR_INVALID, "hidden must be a positive multiple of 32 (got %u)", a.hidden);
  if (!(a.threshold == a.threshold)) return fail(MQ_ERR_INVALID, "threshold is NaN");
  return MQ_OK;
}

SelectParams select_params(const MqRouteArgs &a, const uint16_t *logits) {
  SelectParams p{};
  p.logits = logits;
  p.slot_table = a.slot_table;
  p.experts = a.experts;
  p.top_k = a.top_k;
  p.min_keep = a.min_keep;
  p.threshold = a.threshold;
  p.blend = a.blend;
  return p;
}

}  // namespace mq

using namespace mq;

extern "C" int mq_route_topk(const MqRouteArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  const MqRouteArgs &a = *args;
  int rc = validate_route_args(a);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);

  // Logits go to the caller's buffer (the library allocates nothing).
  uint16_t *logits = a.logits_out;
  const bool need_logits = a.logits_in == nullptr;
  const bool need_shared = a.shared_gate != nullptr;
  if (need_logits && logits == nullptr)
    return fail(MQ_ERR_INVALID, "logits_out is required when the logits are computed (logits_in is NULL)");
  // The shared-gate logit is parked in the shared_gate output, which the
  // select kernel then overwrites with its sigmoid.
  uint16_t *shared_logit = need_shared ? a.shared_gate : nullptr;
  if (need_logits || need_shared) {
    rc = launch_router_logits(a.x, a.gate_w, need_shared ? a.shared_gate_w : nullptr, logits, shared_logit,
                              a.tokens, a.hidden, need_logits ? a.experts : 0u, s);
    if (rc) return rc;
  }
  SelectArgs sa{};
  sa.p = select_params(a, need_logits ? logits : a.logits_in);
  sa.shared_logit = shared_logit;
  sa.inds = a.inds;
  sa.scores = a.scores;
  sa.score_dtype = a.score_dtype;
  sa.scores_raw = a.scores_raw;
  sa.routes = a.routes;
  sa.keeps = a.keeps;
  sa.shared_gate = a.shared_gate;
  sa.tokens = a.tokens;
  hipLaunchKernelGGL(router_select_kernel, dim3(ceil_div(a.tokens, kWaves)), dim3(kThreads), 0, s, sa);
  return check_launch("router_select_kernel");
}
