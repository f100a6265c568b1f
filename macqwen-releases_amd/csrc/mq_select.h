// Router selection for one token by one wave: softmax (float64) over bf16
// logits, top-k on the bf16 gate bits (gate descending, expert ascending),
// adaptive keep and padding, bf16 renorm and slot words.
//
// Restates the chain of models/flashnext/compiled.py:61-71 and
// models/flashnext/adaptive_topk.py:43-64, 75-261: softmax(precise=True),
// argpartition top-k, take_along_axis, topk_mass, _keep_for_mass, padding of
// dropped slots with slot 0's expert and score 0, and
// scores / (mass + blend * (selected - mass)) in bf16 arithmetic.  Logits are
// exact-rounded bf16 and the softmax is evaluated in float64, so the bf16
// gates (and everything after) are reproducible bit for bit.
#pragma once

#include <math.h>

#include "mq_internal.h"

namespace mq {

constexpr int kSelMaxPerLane = 8;  // experts <= 512
constexpr int kSelMaxTopK = 16;

// float64 -> bf16 with one round-to-nearest-even (round-to-odd to float32 first).
__device__ __forceinline__ uint16_t f64_to_bf16(double d) {
  float t = static_cast<float>(d);
  uint32_t bits = __float_as_uint(t);
  if (isfinite(d)) {
    if (fabs(static_cast<double>(t)) > fabs(d)) bits -= 1u;
    if (static_cast<double>(__uint_as_float(bits)) != d) bits |= 1u;
  }
  return f32_to_bf16(__uint_as_float(bits));
}

// bf16 binary ops as MLX evaluates them: float32 op, round to nearest even.
__device__ __forceinline__ float bsub(float a, float b) { return round_bf16(__fsub_rn(a, b)); }
__device__ __forceinline__ float badd(float a, float b) { return round_bf16(__fadd_rn(a, b)); }
__device__ __forceinline__ float bmul(float a, float b) { return round_bf16(__fmul_rn(a, b)); }
__device__ __forceinline__ float bdiv(float a, float b) { return round_bf16(__fdiv_rn(a, b)); }

// bf16(exp(m)) where exp is the correctly rounded float32 exponential.
// expf is within 2 float32 ulps of exp(m); its bf16 rounding can only differ
// from that of the correctly rounded value when the float32 result lies
// within those ulps of a bf16 rounding midpoint (low 16 bits near 0x8000), and
// only then is the exponential re-evaluated in float64.
__device__ __forceinline__ float exp_bf16(float m) {
  const float e = expf(m);
  const int low = static_cast<int>(__float_as_uint(e) & 0xffffu);
  if (abs(low - 0x8000) <= 4 || !isfinite(e)) return round_bf16(static_cast<float>(exp(static_cast<double>(m))));
  return round_bf16(e);
}

// MLX bf16 sigmoid sequence (each step rounded to bf16, float32 exp correctly rounded).
__device__ __forceinline__ float sigmoid_bf16(float g) {
  const float m = fabsf(g);
  const float e = exp_bf16(m);
  const float d = round_bf16(__fadd_rn(1.0f, e));
  const float s = round_bf16(__fdiv_rn(1.0f, d));
  const float om = round_bf16(__fsub_rn(1.0f, s));
  return g < 0.0f ? s : om;
}

struct SelectParams {
  const uint16_t *logits;      // [tokens, experts] bf16
  const uint32_t *slot_table;  // [experts] or nullptr
  uint32_t experts, top_k, min_keep;
  float threshold, blend;
};

// Per-lane result: lane j < top_k holds slot j; `keep` is wave-uniform.
struct SelectLane {
  uint32_t ind;    // expert id (padded slots repeat slot 0's expert)
  uint32_t word;   // route word
  float raw;       // bf16 softmax gate before renorm (as float)
  float score;     // bf16 renormalised score (as float)
  uint32_t keep;
};

// Top-k over unique keys: k rounds of "wave max of the lanes' best key".
__device__ __forceinline__ void select_keys(uint32_t *key, uint32_t k, uint32_t *sel) {
#pragma unroll
  for (uint32_t j = 0; j < kSelMaxTopK; ++j) {
    sel[j] = 0u;
    if (j < k) {
      uint32_t best = 0u;
#pragma unroll
      for (int i = 0; i < kSelMaxPerLane; ++i) best = key[i] > best ? key[i] : best;
      best = wave_max_u32_uniform(best);
      sel[j] = best;
#pragma unroll
      for (int i = 0; i < kSelMaxPerLane; ++i)
        if (key[i] == best) key[i] = 0u;
    }
  }
}

__device__ __forceinline__ float wave_max_f32_uniform(float v) {
  v = fmaxf(v, dpp_f<0xb1>(v));
  v = fmaxf(v, dpp_f<0x4e>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  v = fmaxf(v, dpp_f<0x128>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// All 64 lanes of the wave must call this together.
//
// The gates are first evaluated in float32: exp(l - m) by expf (<= 2 ulp;
// l - m is exact), a fixed-order sum and a correctly rounded division, which
// bounds each gate's relative error by about 16 float32 ulps.  A gate's bf16
// bits are then exact unless its float32 value lies within that bound of a
// bf16 rounding midpoint.  Only gates within one bf16 step of the k-th gate
// can change the selection or the scores; if any of them is that close to a
// midpoint the token is re-evaluated in float64 (exp, sum and division),
// which is exact for all practical inputs.
__device__ __forceinline__ SelectLane select_token(const SelectParams &a, uint32_t t, int lane) {
  const uint16_t *lrow = a.logits + static_cast<uint64_t>(t) * a.experts;
  float lv[kSelMaxPerLane];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    const uint32_t e = lane + 64 * i;
    lv[i] = e < a.experts ? bf16_to_f32(lrow[e]) : -INFINITY;
    m = fmaxf(m, lv[i]);
  }
  m = wave_max_f32_uniform(m);
  float ev[kSelMaxPerLane];
  bool wide[kSelMaxPerLane];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    const uint32_t e = lane + 64 * i;
    const float d = lv[i] - m;  // exact while |d| <= 32 for bf16 inputs of this range
    wide[i] = !(d >= -32.0f);
    ev[i] = e < a.experts ? expf(d) : 0.0f;
    sum += ev[i];
  }
  sum = wave_sum(sum);
  // Key: bf16 gate bits (non-negative, so they order like values) high,
  // inverted expert index low (ties -> lower index).  Keys are unique.
  uint32_t key[kSelMaxPerLane], gbits[kSelMaxPerLane];
  bool near[kSelMaxPerLane];
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    const uint32_t e = lane + 64 * i;
    const float g = __fdiv_rn(ev[i], sum);
    const int low = static_cast<int>(__float_as_uint(g) & 0xffffu);
    gbits[i] = e < a.experts ? f32_to_bf16(g) : 0u;
    near[i] = e < a.experts && (abs(low - 0x8000) <= 48 || wide[i]);
    key[i] = e < a.experts ? (gbits[i] << 16) | (0xffffu - e) : 0u;
  }
  const uint32_t k = a.top_k;
  uint32_t sel[kSelMaxTopK];
  select_keys(key, k, sel);
  uint32_t kth = 0u;
#pragma unroll
  for (uint32_t j = 0; j < kSelMaxTopK; ++j)
    if (j + 1 == k) kth = sel[j] >> 16;
  bool risky = false;
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) risky |= near[i] && gbits[i] + 1u >= kth;
  if (__ballot(risky) != 0ull) {  // wave-uniform: redo this token in float64
    double dm = static_cast<double>(m), dsum = 0.0;
    double dv[kSelMaxPerLane];
#pragma unroll
    for (int i = 0; i < kSelMaxPerLane; ++i) {
      const uint32_t e = lane + 64 * i;
      dv[i] = e < a.experts ? exp(static_cast<double>(lv[i]) - dm) : 0.0;
      dsum += dv[i];
    }
    dsum = wave_sum_f64_uniform(dsum);
#pragma unroll
    for (int i = 0; i < kSelMaxPerLane; ++i) {
      const uint32_t e = lane + 64 * i;
      key[i] = e < a.experts ? (static_cast<uint32_t>(f64_to_bf16(dv[i] / dsum)) << 16) | (0xffffu - e) : 0u;
    }
    select_keys(key, k, sel);
  }
  uint32_t ind[kSelMaxTopK];
  float raw[kSelMaxTopK];
  float mass32 = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < kSelMaxTopK; ++j) {
    ind[j] = 0xffffu - (sel[j] & 0xffffu);
    raw[j] = bf16_to_f32(static_cast<uint16_t>(sel[j] >> 16));
    if (j < k) mass32 = __fadd_rn(mass32, raw[j]);
  }
  const float mass = round_bf16(mass32);
  uint32_t keep = k;
  if (a.threshold < 1.0f) {
    double total = 0.0;
#pragma unroll
    for (uint32_t j = 0; j < kSelMaxTopK; ++j)
      if (j < k) total += static_cast<double>(raw[j]);
    double accumulated = 0.0;
    uint32_t found = k;
#pragma unroll
    for (uint32_t j = 0; j < kSelMaxTopK; ++j) {
      if (j < k && found == k) {
        accumulated += static_cast<double>(raw[j]) / total;
        if (accumulated >= static_cast<double>(a.threshold)) found = j + 1;
      }
    }
    const uint32_t minimum = a.min_keep < 1u ? 1u : (a.min_keep > k ? k : a.min_keep);
    keep = found > minimum ? found : minimum;
  }
  float padded[kSelMaxTopK];
  float sel32 = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < kSelMaxTopK; ++j) {
    if (j >= keep) ind[j] = ind[0];
    padded[j] = j < keep ? raw[j] : 0.0f;
    if (j < k) sel32 = __fadd_rn(sel32, padded[j]);
  }
  const float selected = round_bf16(sel32);
  const float blend = round_bf16(a.blend);
  const float norm = badd(mass, bmul(blend, bsub(selected, mass)));
  SelectLane out{0u, 0u, 0.0f, 0.0f, keep};
#pragma unroll
  for (uint32_t j = 0; j < kSelMaxTopK; ++j) {
    if (static_cast<uint32_t>(lane) == j) {
      out.ind = ind[j];
      out.raw = raw[j];
      out.score = padded[j];
    }
  }
  if (static_cast<uint32_t>(lane) < k) {
    out.score = bdiv(out.score, norm);
    out.word = a.slot_table ? (MQ_SLOT_BIT | a.slot_table[out.ind]) : out.ind;
  }
  return out;
}

}  // namespace mq
