// Router selection for one token by one wave: softmax over bf16 logits
// (float32 with an exactness guard, float64 fallback), top-k on the bf16 gate
// bits (gate descending, expert ascending),
// adaptive keep and padding, bf16 renorm and slot words.
//
// Restates the chain of models/flashnext/compiled.py:61-71 and
// models/flashnext/adaptive_topk.py:43-64, 75-261: softmax(precise=True),
// argpartition top-k, take_along_axis, topk_mass, _keep_for_mass, padding of
// dropped slots with slot 0's expert and score 0, and
// scores / (mass + blend * (selected - mass)) in bf16 arithmetic.  Logits are
// exact-rounded bf16 and every bf16 gate equals the correctly rounded softmax
// value, so the gates (and everything after) are reproducible bit for bit.
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

// bf16 round-to-nearest-even in one v_cvt_pk_bf16_f32.  Equal to round_bf16
// for every non-NaN float32, denormals and infinities included (checked over
// all 2^32 bit patterns on gfx950); only NaN payloads may differ, so it is used
// inside the sequences below, whose stored results are rounded again.
__device__ __forceinline__ float round_bf16_hw(float f) {
  return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f))) << 16);
}

// bf16(exp(m)) where exp is the correctly rounded float32 exponential.
// expf is within 2 float32 ulps of exp(m); its bf16 rounding can only differ
// from that of the correctly rounded value when the float32 result lies
// within those ulps of a bf16 rounding midpoint (low 16 bits near 0x8000), and
// only then is the exponential re-evaluated in float64.
__device__ __forceinline__ float exp_bf16(float m) {
  const float e = expf(m);
  const int low = static_cast<int>(__float_as_uint(e) & 0xffffu);
  if (abs(low - 0x8000) <= 4 || !isfinite(e)) return round_bf16(static_cast<float>(exp(static_cast<double>(m))));
  return round_bf16_hw(e);
}

// bf16(1 / d) for a bf16 value d >= 2 (or inf), equal to the bf16 rounding of
// the correctly rounded float32 quotient.  It takes the hardware reciprocal
// (within 1 float32 ulp) instead of a division.  Normal results (d <= 2^126):
// d = D * 2^k with D < 256; unless D is a power of two (then 1/d is exact
// either way), the odd part D' >= 3 of D puts 1/d at a relative distance
// >= 2^-8 / D' > 2^-16 from every bf16 rounding midpoint (an odd multiple of
// 2^-9 times a power of two), far beyond the reciprocal's 2^-23, so both
// round to the same bf16.  Denormal results (d > 2^126): v_rcp_f32 flushes
// them to zero, so the reciprocal of d/4 (normal, exact scaling) is taken and
// multiplied by 1/4, which rounds once onto the float32 denormal grid
// (spacing 2^-149).  The bf16 denormal midpoints are odd multiples of 2^-134,
// and 1/d = 2^-k / D' (D' odd >= 3) lies at least 2^-134 / 255 > 2^-142 from
// each of them, while the two roundings move it by at most 2^-150 + 2^-150;
// the correctly rounded float32 quotient is within 2^-150 as well, so both
// give the same bf16.  d = inf gives 0 either way.
__device__ __forceinline__ float recip_bf16(float d) {
  const bool tiny = d > 0x1p126f;
  const float r = __builtin_amdgcn_rcpf(tiny ? __fmul_rn(d, 0.25f) : d);
  return round_bf16_hw(tiny ? __fmul_rn(r, 0.25f) : r);
}

// MLX bf16 sigmoid sequence (each step rounded to bf16, float32 exp correctly rounded).
__device__ __forceinline__ float sigmoid_bf16(float g) {
  const float m = fabsf(g);
  const float e = exp_bf16(m);
  const float d = round_bf16_hw(__fadd_rn(1.0f, e));
  const float s = recip_bf16(d);
  const float om = round_bf16_hw(__fsub_rn(1.0f, s));
  return g < 0.0f ? s : om;
}

// bf16 SwiGLU of bf16-valued g and u: bf16(bf16(g * sigmoid_bf16(g)) * u)
// (models/flashnext/metal_runtime.py:278-287).
__device__ __forceinline__ float swiglu_bf16(float g, float u) {
  const float silu = round_bf16_hw(__fmul_rn(g, sigmoid_bf16(g)));
  return round_bf16(__fmul_rn(silu, u));
}

// swiglu_bf16 of N values at once, bit for bit: the float32 exponentials are
// taken together and the rare float64 re-evaluation runs behind one
// wave-uniform branch, so the N sequences stay free of divergent control flow
// and interleave.
//
// The sigmoid depends on the gate only through m = |g| (s = bf16(1 / d) and
// om = bf16(1 - s) with d = bf16(1 + bf16(exp(m)))) and the sign, which picks
// s (g < 0) or om; sigmoid_parts_n is that |g|-only part.
template <int N>
__device__ __forceinline__ void sigmoid_parts_n(const float (&m)[N], float (&s)[N], float (&om)[N]) {
  float e[N];
  uint32_t redo = 0u;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float ef = expf(m[i]);
    const int low = static_cast<int>(__float_as_uint(ef) & 0xffffu);
    if (abs(low - 0x8000) <= 4 || !isfinite(ef)) redo |= 1u << i;
    e[i] = round_bf16_hw(ef);
  }
  if (__ballot(redo != 0u) != 0ull) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((redo >> i) & 1u) e[i] = round_bf16(static_cast<float>(exp(static_cast<double>(m[i]))));
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float d = round_bf16_hw(__fadd_rn(1.0f, e[i]));
    s[i] = recip_bf16(d);
    om[i] = round_bf16_hw(__fsub_rn(1.0f, s[i]));
  }
}

template <int N>
__device__ __forceinline__ void swiglu_bf16_n(const float (&g)[N], const float (&u)[N], float (&out)[N]) {
  float m[N], s[N], om[N];
#pragma unroll
  for (int i = 0; i < N; ++i) m[i] = fabsf(g[i]);
  sigmoid_parts_n<N>(m, s, om);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float silu = round_bf16_hw(__fmul_rn(g[i], g[i] < 0.0f ? s[i] : om[i]));
    out[i] = round_bf16(__fmul_rn(silu, u[i]));
  }
}

// Sigmoid table for bf16 gates: one word per |g| (bf16 bits of s in the low
// half, of om in the high half), made by sigmoid_parts_n itself, so a lookup
// equals the sequence bit for bit.  Entry 0 serves every |g| below 2^-8
// (there exp(|g|) < 1 + 2^-8 - 2^-17 rounds to e = 1, the same as at 0);
// entries 1.. hold the bf16 values 2^-8 <= |g| < 2^7, one per value (15
// binades of 128).  |g| >= 2^7 (the float32 exponential overflows from about
// 88.7), infinities and NaN take the full sequence.  7.7 KB, for LDS.
constexpr uint32_t kSigTabFirst = 0x3b80u;  // bf16 bits of 2^-8
constexpr uint32_t kSigTabEnd = 0x4300u;    // bf16 bits of 2^7
constexpr uint32_t kSigTabEntries = kSigTabEnd - kSigTabFirst + 1u;

__device__ __forceinline__ float sig_tab_gate(uint32_t i) {
  return i == 0u ? 0.0f : __uint_as_float((kSigTabFirst + i - 1u) << 16);
}

// Fills tab[0 .. kSigTabEntries) with `threads` threads (this one `t`), four
// entries per thread and round.  The caller synchronizes before any lookup.
__device__ __forceinline__ void fill_sig_tab(uint32_t *tab, uint32_t t, uint32_t threads) {
  for (uint32_t i0 = 4u * t; i0 < kSigTabEntries; i0 += 4u * threads) {
    float m[4], s[4], om[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) m[k] = sig_tab_gate(min(i0 + k, kSigTabEntries - 1u));
    sigmoid_parts_n<4>(m, s, om);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (i0 + k < kSigTabEntries) tab[i0 + k] = (__float_as_uint(s[k]) >> 16) | (__float_as_uint(om[k]) & 0xffff0000u);
  }
}

// swiglu_bf16_n for bf16-valued gates with the sigmoid looked up in `tab`
// (filled by fill_sig_tab); gates outside the table take swiglu_bf16_n behind
// one wave-uniform branch.  Bit-identical to swiglu_bf16_n.
template <int N>
__device__ __forceinline__ void swiglu_bf16_tab_n(const float (&g)[N], const float (&u)[N], float (&out)[N],
                                                  const uint32_t *tab) {
  uint32_t slow = 0u;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t b = (__float_as_uint(g[i]) >> 16) & 0x7fffu;  // |g| as bf16 bits
    if (b >= kSigTabEnd) slow |= 1u << i;
    const uint32_t c = b < kSigTabEnd ? b : kSigTabEnd - 1u;  // keeps the read in the table
    const uint32_t w = tab[c >= kSigTabFirst ? c - kSigTabFirst + 1u : 0u];
    const float sel = __uint_as_float(g[i] < 0.0f ? w << 16 : w & 0xffff0000u);
    const float silu = round_bf16_hw(__fmul_rn(g[i], sel));
    out[i] = round_bf16(__fmul_rn(silu, u[i]));
  }
  if (__ballot(slow != 0u) != 0ull) {
    float full[N];
    swiglu_bf16_n<N>(g, u, full);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((slow >> i) & 1u) out[i] = full[i];
  }
}

// MLX's sigmoid sequence with each step rounded to T
// (models/flashnext/metal_runtime.py:278-284): m=|g|; e=T(exp(m));
// d=T(1+e); s=T(1/d); sig = g<0 ? s : T(1-s).  exp is the float32
// exponential correctly rounded.
template <class TT>
__device__ __forceinline__ float sigmoid_t(float g) {
  if constexpr (TT::dtype == MQ_BF16) {
    return sigmoid_bf16(g);
  } else {
    const float e = static_cast<float>(exp(static_cast<double>(fabsf(g))));
    const float d = TT::round(__fadd_rn(1.0f, e));
    const float s = TT::round(__fdiv_rn(1.0f, d));
    const float om = TT::round(__fsub_rn(1.0f, s));
    return g < 0.0f ? s : om;
  }
}

// act = T(T(g * sigmoid_T(g)) * u) for T-valued g and u.
template <class TT>
__device__ __forceinline__ float swiglu_t(float g, float u) {
  if constexpr (TT::dtype == MQ_BF16) {
    return swiglu_bf16(g, u);
  } else {
    const float silu = TT::round(__fmul_rn(g, sigmoid_t<TT>(g)));
    return TT::round(__fmul_rn(silu, u));
  }
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

// Sorts a lane's eight keys in descending order (19 compare-exchanges,
// depth 6).
__device__ __forceinline__ void sort8_desc(uint32_t (&key)[kSelMaxPerLane]) {
  constexpr int kNet[19][2] = {{0, 2}, {1, 3}, {4, 6}, {5, 7}, {0, 4}, {1, 5}, {2, 6}, {3, 7}, {0, 1}, {2, 3},
                               {4, 5}, {6, 7}, {2, 4}, {3, 5}, {1, 4}, {3, 6}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
  for (int c = 0; c < 19; ++c) {
    const uint32_t a = key[kNet[c][0]], b = key[kNet[c][1]];
    key[kNet[c][0]] = max(a, b);
    key[kNet[c][1]] = min(a, b);
  }
}

// Top-k over unique keys.  Each lane sorts its keys; round j takes the wave
// max of the lanes' heads and the winning lane pops its head.  Lane j keeps
// the j-th selected key (descending); other lanes get 0.  `key` is consumed.
__device__ __forceinline__ uint32_t select_keys(uint32_t (&key)[kSelMaxPerLane], uint32_t k, int lane) {
  sort8_desc(key);
  uint32_t mine = 0u;
#pragma unroll
  for (uint32_t j = 0; j < static_cast<uint32_t>(kSelMaxTopK); ++j) {
    if (j < k) {  // wave-uniform
      const uint32_t best = wave_max_u32_uniform(key[0]);
      mine = static_cast<uint32_t>(lane) == j ? best : mine;
      const bool win = key[0] == best;
#pragma unroll
      for (int i = 0; i < kSelMaxPerLane - 1; ++i) key[i] = win ? key[i + 1] : key[i];
      key[kSelMaxPerLane - 1] = win ? 0u : key[kSelMaxPerLane - 1];
    }
  }
  return mine;
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

__device__ __forceinline__ float readlane_f(float v, uint32_t lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), static_cast<int>(lane)));
}

// Selection window: float32 gates whose low 16 bits lie within this many
// float32 ulps of the bf16 rounding midpoint (0x8000) may round differently
// from the exact gate (see select_token).
constexpr int kMidpointWindow = 64;
// log2(e) split into float32 head and tail: d * log2(e) = fma(d, hi, d * lo)
// carries one rounding (|error| <= 2^-19 for |d| <= 32).
constexpr float kLog2eHi = 1.44269502162933349609375f;
constexpr float kLog2eLo = 1.925963033500011e-08f;

// All 64 lanes of the wave must call this together.
//
// The gates are first evaluated in float32: e = exp2((l - m) * log2(e)) with
// the hardware exp2 (l - m is exact for bf16 logits within 32 of the max; the
// argument carries one rounding, <= 2^-19, i.e. <= 22 ulps of the result,
// and exp2 itself about 1 ulp), a fixed-order tree sum of depth <= 14
// (<= 14 ulps) and one correctly rounded reciprocal and product (1 ulp): each
// gate is within ~40 float32 ulps of the exact value, inside kMidpointWindow.  A gate's bf16 bits are then exact unless its
// float32 value lies within the window of a bf16 rounding midpoint (or its
// logit is more than 32 below the max).  Only gates within one bf16 step of
// the k-th gate can change the selection or the scores; if any of them is that
// close to a midpoint the token is re-evaluated in float64 (exp, sum and
// division), which is exact for all practical inputs.
__device__ __forceinline__ SelectLane select_token(const SelectParams &a, uint32_t t, int lane) {
  const uint16_t *lrow = a.logits + static_cast<uint64_t>(t) * a.experts;
  // All loads are unconditional (clamped indices, results masked afterwards)
  // so they are issued back to back; the slot table is fetched alongside the
  // logits and indexed later through a lane permute.
  float lv[kSelMaxPerLane];
  uint32_t slot_of[kSelMaxPerLane];
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    const uint32_t e = min(static_cast<uint32_t>(lane + 64 * i), a.experts - 1u);
    lv[i] = bf16_to_f32(lrow[e]);
    slot_of[i] = a.slot_table ? a.slot_table[e] : 0u;
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    if (static_cast<uint32_t>(lane + 64 * i) >= a.experts) lv[i] = -INFINITY;
    m = fmaxf(m, lv[i]);
  }
  m = wave_max_f32_uniform(m);
  float ev[kSelMaxPerLane];
  bool wide[kSelMaxPerLane];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    const float d = lv[i] - m;
    wide[i] = !(d >= -32.0f);
    ev[i] = static_cast<uint32_t>(lane + 64 * i) < a.experts
                ? __builtin_amdgcn_exp2f(__fmaf_rn(d, kLog2eHi, __fmul_rn(d, kLog2eLo)))
                : 0.0f;
    sum += ev[i];
  }
  sum = wave_sum(sum);
  const float rsum = __fdiv_rn(1.0f, sum);
  // Key: bf16 gate bits (non-negative, so they order like values) high,
  // inverted expert index low (ties -> lower index).  Keys are unique.
  uint32_t key[kSelMaxPerLane], gbits[kSelMaxPerLane];
  bool near[kSelMaxPerLane];
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    const uint32_t e = lane + 64 * i;
    const float g = __fmul_rn(ev[i], rsum);
    const int low = static_cast<int>(__float_as_uint(g) & 0xffffu);
    gbits[i] = e < a.experts ? f32_to_bf16(g) : 0u;
    near[i] = e < a.experts && (abs(low - 0x8000) <= kMidpointWindow || wide[i]);
    key[i] = e < a.experts ? (gbits[i] << 16) | (0xffffu - e) : 0u;
  }
  const uint32_t k = a.top_k;
  uint32_t mine = select_keys(key, k, lane);
  const uint32_t kth = readlane_u(mine, static_cast<int>(k - 1u)) >> 16;
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
    mine = select_keys(key, k, lane);
  }
  // Lane j < k: slot j.  Reductions over slots run in slot order (the
  // readlanes are unrolled and independent; only the adds chain).
  const bool slot_lane = static_cast<uint32_t>(lane) < k;
  uint32_t ind = 0xffffu - (mine & 0xffffu);
  const float raw = slot_lane ? bf16_to_f32(static_cast<uint16_t>(mine >> 16)) : 0.0f;
  float raws[kSelMaxTopK];
#pragma unroll
  for (int j = 0; j < kSelMaxTopK; ++j) raws[j] = readlane_f(raw, static_cast<uint32_t>(j));
  float mass32 = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < static_cast<uint32_t>(kSelMaxTopK); ++j)
    if (j < k) mass32 = __fadd_rn(mass32, raws[j]);
  const float mass = round_bf16(mass32);
  uint32_t keep = k;
  if (a.threshold < 1.0f) {
    double total = 0.0;
#pragma unroll
    for (uint32_t j = 0; j < static_cast<uint32_t>(kSelMaxTopK); ++j)
      if (j < k) total += static_cast<double>(raws[j]);
    double accumulated = 0.0;
    uint32_t found = k;
#pragma unroll
    for (uint32_t j = 0; j < static_cast<uint32_t>(kSelMaxTopK); ++j) {
      if (j < k && found == k) {
        accumulated += static_cast<double>(raws[j]) / total;
        if (accumulated >= static_cast<double>(a.threshold)) found = j + 1;
      }
    }
    const uint32_t minimum = a.min_keep < 1u ? 1u : (a.min_keep > k ? k : a.min_keep);
    keep = found > minimum ? found : minimum;
  }
  // Dropped slots repeat slot 0's expert with score 0.
  const uint32_t ind0 = readlane_u(ind, 0);
  const bool kept = static_cast<uint32_t>(lane) < keep;
  ind = kept ? ind : ind0;
  const float padded = kept ? raw : 0.0f;
  float sel32 = mass32;  // every slot kept: the same sum in the same order
  if (keep < k) {
    sel32 = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < static_cast<uint32_t>(kSelMaxTopK); ++j)
      if (j < k) sel32 = __fadd_rn(sel32, j < keep ? raws[j] : 0.0f);
  }
  const float selected = round_bf16(sel32);
  const float blend = round_bf16(a.blend);
  const float norm = badd(mass, bmul(blend, bsub(selected, mass)));
  // slot_table[ind]: entry ind sits in register ind / 64 of lane ind % 64.
  uint32_t slot = 0u;
#pragma unroll
  for (int i = 0; i < kSelMaxPerLane; ++i) {
    const uint32_t v = static_cast<uint32_t>(
        __builtin_amdgcn_ds_bpermute(static_cast<int>((ind & 63u) << 2), static_cast<int>(slot_of[i])));
    slot = (ind >> 6) == static_cast<uint32_t>(i) ? v : slot;
  }
  SelectLane out{ind, 0u, raw, 0.0f, keep};
  if (slot_lane) {
    out.score = bdiv(padded, norm);
    out.word = a.slot_table ? (MQ_SLOT_BIT | slot) : ind;
  }
  return out;
}

}  // namespace mq
