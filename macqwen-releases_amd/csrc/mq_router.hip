// Router chain for gfx950: gate GEMV, softmax, top-k, renorm, adaptive keep,
// slot lookup and the shared-expert sigmoid gate.
//
// The reference chain is softmax(precise) -> argpartition top-k ->
// take_along_axis -> renorm (models/flashnext/compiled.py:61-71,
// models/flashnext/adaptive_topk.py:53-64, 256-261).  Logits and softmax are
// evaluated in float64 and rounded once to bf16, so the bf16 gates are the
// correctly rounded values; top-k then selects on those bits with the order
// "gate descending, expert ascending", making indices, scores and route words
// reproducible bit for bit.  The renorm is bf16 arithmetic (float32 op, then
// round to nearest even), as MLX evaluates it.
#include <math.h>

#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

// float64 -> bf16 with a single round-to-nearest-even: round to float32 with
// round-to-odd (truncate, then set the sticky bit when inexact), then RNE.
__device__ __forceinline__ uint16_t f64_to_bf16(double d) {
  float t = static_cast<float>(d);
  uint32_t bits = __float_as_uint(t);
  if (isfinite(d)) {
    if (fabs(static_cast<double>(t)) > fabs(d)) bits -= 1u;  // toward zero
    if (static_cast<double>(__uint_as_float(bits)) != d) bits |= 1u;
  }
  return f32_to_bf16(__uint_as_float(bits));
}

__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// bf16 dot of one 32-value chunk, exact products accumulated in float64.
__device__ __forceinline__ double chunk_dot_f64(const uint4 *a, const uint4 *b) {
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 qa = a[j];
    const uint4 qb = b[j];
    const uint32_t ua[4] = {qa.x, qa.y, qa.z, qa.w};
    const uint32_t ub[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a0 = __uint_as_float(ua[k] << 16), a1 = __uint_as_float(ua[k] & 0xffff0000u);
      const float b0 = __uint_as_float(ub[k] << 16), b1 = __uint_as_float(ub[k] & 0xffff0000u);
      acc += static_cast<double>(a0 * b0);  // bf16 x bf16 is exact in float32
      acc += static_cast<double>(a1 * b1);
    }
  }
  return acc;
}

// logits[t, e] = bf16(sum_k x[t,k] * W[e,k]); row `experts` (when present) is
// the shared-expert gate row, written to shared_logit[t].
// One wave per weight row, looping over tokens; x is read through L2.
__global__ __launch_bounds__(kThreads) void router_logits_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate_w,
    const uint16_t *__restrict__ shared_gate_w, uint16_t *__restrict__ logits,
    uint16_t *__restrict__ shared_logit, uint32_t tokens, uint32_t hidden, uint32_t experts) {
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const uint32_t rows = experts + (shared_gate_w ? 1u : 0u);
  if (row >= rows) return;
  const uint16_t *w = row < experts ? gate_w + static_cast<uint64_t>(row) * hidden : shared_gate_w;
  const uint32_t chunks = hidden >> 5;
  const uint32_t cpl = (chunks + 63) / 64;
  for (uint32_t t = 0; t < tokens; ++t) {
    double acc = 0.0;
    for (uint32_t j = 0; j < cpl; ++j) {
      const uint32_t c = lane + 64 * j;
      if (c < chunks) {
        acc += chunk_dot_f64(reinterpret_cast<const uint4 *>(w + c * 32),
                             reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(t) * hidden + c * 32));
      }
    }
    acc = wave_sum_f64(acc);
    if (lane == 0) {
      const uint16_t v = f64_to_bf16(acc);
      if (row < experts)
        logits[static_cast<uint64_t>(t) * experts + row] = v;
      else
        shared_logit[t] = v;
    }
  }
}

// bf16 binary op as MLX evaluates it: float32 op, round to nearest even.
__device__ __forceinline__ float bsub(float a, float b) { return round_bf16(__fsub_rn(a, b)); }
__device__ __forceinline__ float badd(float a, float b) { return round_bf16(__fadd_rn(a, b)); }
__device__ __forceinline__ float bmul(float a, float b) { return round_bf16(__fmul_rn(a, b)); }
__device__ __forceinline__ float bdiv(float a, float b) { return round_bf16(__fdiv_rn(a, b)); }

// MLX bf16 sigmoid sequence (each step rounded to bf16, float32 exp correctly rounded).
__device__ __forceinline__ float sigmoid_bf16(float g) {
  const float m = fabsf(g);
  const float e = round_bf16(static_cast<float>(exp(static_cast<double>(m))));
  const float d = round_bf16(__fadd_rn(1.0f, e));
  const float s = round_bf16(__fdiv_rn(1.0f, d));
  const float om = round_bf16(__fsub_rn(1.0f, s));
  return g < 0.0f ? s : om;
}

struct SelectArgs {
  const uint16_t *logits;      // [tokens, experts]
  const uint16_t *shared_logit;
  const uint32_t *slot_table;
  uint32_t *inds;
  void *scores;
  int score_dtype;
  uint16_t *scores_raw;
  uint32_t *routes;
  int32_t *keeps;
  uint16_t *shared_gate;
  uint32_t tokens, experts, top_k, min_keep;
  float threshold, blend;
};

constexpr int kMaxPerLane = 8;  // experts <= 512
constexpr int kMaxTopK = 16;

// One wave per token: softmax (float64), top-k on bf16 gate bits, renorm,
// adaptive keep and padding, slot words, shared gate.
__global__ __launch_bounds__(kThreads) void router_select_kernel(SelectArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (t >= a.tokens) return;
  const uint16_t *lrow = a.logits + static_cast<uint64_t>(t) * a.experts;

  double lv[kMaxPerLane];
  double m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const uint32_t e = lane + 64 * i;
    lv[i] = e < a.experts ? static_cast<double>(bf16_to_f32(lrow[e])) : -INFINITY;
    m = fmax(m, lv[i]);
  }
  for (int off = 32; off > 0; off >>= 1) m = fmax(m, __shfl_xor(m, off, 64));
  double ev[kMaxPerLane];
  double sum = 0.0;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const uint32_t e = lane + 64 * i;
    ev[i] = e < a.experts ? exp(lv[i] - m) : 0.0;
    sum += ev[i];
  }
  sum = wave_sum_f64(sum);
  // Sort key: bf16 gate bits (non-negative, so they order like values) in the
  // high half, inverted expert index in the low half (ties -> lower index).
  uint32_t key[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const uint32_t e = lane + 64 * i;
    key[i] = e < a.experts ? (static_cast<uint32_t>(f64_to_bf16(ev[i] / sum)) << 16) | (0xffffu - e) : 0u;
  }
  uint32_t sel[kMaxTopK];
  for (uint32_t j = 0; j < a.top_k; ++j) {
    uint32_t best = 0u;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) best = key[i] > best ? key[i] : best;
    best = wave_max_u32(best);
    sel[j] = best;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i)
      if (key[i] == best) key[i] = 0u;
  }
  if (lane != 0) return;

  const uint32_t k = a.top_k;
  uint32_t ind[kMaxTopK];
  float raw[kMaxTopK];
  float mass32 = 0.0f;
  for (uint32_t j = 0; j < k; ++j) {
    ind[j] = 0xffffu - (sel[j] & 0xffffu);
    raw[j] = bf16_to_f32(static_cast<uint16_t>(sel[j] >> 16));
    mass32 = __fadd_rn(mass32, raw[j]);
  }
  const float mass = round_bf16(mass32);

  // Adaptive keep (models/flashnext/adaptive_topk.py:43-50, 104-114): float64
  // prefix sums in slot order, exactly as the Python loop evaluates them.
  uint32_t keep = k;
  if (a.threshold < 1.0f) {
    double total = 0.0;
    for (uint32_t j = 0; j < k; ++j) total += static_cast<double>(raw[j]);
    double accumulated = 0.0;
    uint32_t found = k;
    for (uint32_t j = 0; j < k; ++j) {
      accumulated += static_cast<double>(raw[j]) / total;
      if (accumulated >= static_cast<double>(a.threshold)) {
        found = j + 1;
        break;
      }
    }
    const uint32_t minimum = a.min_keep < 1u ? 1u : (a.min_keep > k ? k : a.min_keep);
    keep = found > minimum ? found : minimum;
  }
  // Padding: dropped slots repeat slot 0's expert with score 0
  // (models/flashnext/adaptive_topk.py:213-227).
  float padded[kMaxTopK];
  float sel32 = 0.0f;
  for (uint32_t j = 0; j < k; ++j) {
    if (j >= keep) ind[j] = ind[0];
    padded[j] = j < keep ? raw[j] : 0.0f;
    sel32 = __fadd_rn(sel32, padded[j]);
  }
  // Renorm in bf16 arithmetic (compiled.py:68-71).
  const float selected = round_bf16(sel32);
  const float blend = round_bf16(a.blend);
  const float norm = badd(mass, bmul(blend, bsub(selected, mass)));
  const uint64_t base = static_cast<uint64_t>(t) * k;
  for (uint32_t j = 0; j < k; ++j) {
    const float sc = bdiv(padded[j], norm);
    a.inds[base + j] = ind[j];
    if (a.score_dtype == MQ_BF16)
      static_cast<uint16_t *>(a.scores)[base + j] = f32_to_bf16(sc);
    else
      static_cast<float *>(a.scores)[base + j] = sc;
    if (a.scores_raw) a.scores_raw[base + j] = f32_to_bf16(raw[j]);
    if (a.routes) a.routes[base + j] = a.slot_table ? (MQ_SLOT_BIT | a.slot_table[ind[j]]) : ind[j];
  }
  if (a.keeps) a.keeps[t] = static_cast<int32_t>(keep);
  if (a.shared_gate) a.shared_gate[t] = f32_to_bf16(sigmoid_bf16(bf16_to_f32(a.shared_logit[t])));
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" int mq_route_topk(const MqRouteArgs *args, void *stream) {
  if (args == nullptr) return fail(MQ_ERR_INVALID, "args is NULL");
  const MqRouteArgs &a = *args;
  if (a.tokens == 0) return fail(MQ_ERR_INVALID, "tokens must be positive");
  if (a.experts == 0 || a.experts > MQ_MAX_EXPERTS)
    return fail(MQ_ERR_INVALID, "experts must be in 1..%d (got %u)", MQ_MAX_EXPERTS, a.experts);
  if (a.top_k == 0 || a.top_k > 16 || a.top_k > a.experts)
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
  hipStream_t s = static_cast<hipStream_t>(stream);

  // Logits go to the caller's buffer or a grow-only library scratch buffer.
  uint16_t *logits = a.logits_out;
  static thread_local uint16_t *scratch = nullptr;
  static thread_local size_t scratch_elems = 0;
  static thread_local int scratch_dev = -1;
  int device = 0;
  MQ_TRY_HIP(hipGetDevice(&device));
  const bool need_logits = a.logits_in == nullptr;
  const bool need_shared = a.shared_gate != nullptr;
  const size_t elems = static_cast<size_t>(a.tokens) * a.experts + a.tokens;
  if ((need_logits && logits == nullptr) || need_shared) {
    if (scratch == nullptr || scratch_elems < elems || scratch_dev != device) {
      if (scratch != nullptr && scratch_dev == device) {
        MQ_TRY_HIP(hipDeviceSynchronize());
        (void)hipFree(scratch);
      }
      scratch = nullptr;
      MQ_TRY_HIP(hipMalloc(&scratch, elems * sizeof(uint16_t)));
      scratch_elems = elems;
      scratch_dev = device;
    }
  }
  if (need_logits && logits == nullptr) logits = scratch;
  uint16_t *shared_logit = need_shared ? scratch + static_cast<size_t>(a.tokens) * a.experts : nullptr;

  if (need_logits || need_shared) {
    // Rows [0, routed_rows) are router rows; one more row is the shared gate.
    const uint32_t routed_rows = need_logits ? a.experts : 0u;
    const uint32_t total_rows = routed_rows + (need_shared ? 1u : 0u);
    hipLaunchKernelGGL(router_logits_kernel, dim3(ceil_div(total_rows, kWaves)), dim3(kThreads), 0, s,
                       a.x, a.gate_w, need_shared ? a.shared_gate_w : nullptr, logits, shared_logit,
                       a.tokens, a.hidden, routed_rows);
    int rc = check_launch("router_logits_kernel");
    if (rc) return rc;
  }
  SelectArgs sa{};
  sa.logits = need_logits ? logits : a.logits_in;
  sa.shared_logit = shared_logit;
  sa.slot_table = a.slot_table;
  sa.inds = a.inds;
  sa.scores = a.scores;
  sa.score_dtype = a.score_dtype;
  sa.scores_raw = a.scores_raw;
  sa.routes = a.routes;
  sa.keeps = a.keeps;
  sa.shared_gate = a.shared_gate;
  sa.tokens = a.tokens;
  sa.experts = a.experts;
  sa.top_k = a.top_k;
  sa.min_keep = a.min_keep;
  sa.threshold = a.threshold;
  sa.blend = a.blend;
  hipLaunchKernelGGL(router_select_kernel, dim3(ceil_div(a.tokens, kWaves)), dim3(kThreads), 0, s, sa);
  return check_launch("router_select_kernel");
}
