// Internal helpers shared by the gfx950 kernels of the quantized MoE path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mqmoe.h"

namespace mq {

// ---------------------------------------------------------------- errors
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t err, const char *what);
int check_launch(const char *what);
#define MQ_TRY_HIP(expr)                                  \
  do {                                                    \
    hipError_t _e = (expr);                               \
    if (_e != hipSuccess) return ::mq::hip_fail(_e, #expr); \
  } while (0)

// Per-device library state: the device error flags raised by kernels.  The
// flags live in a file-scope __device__ array (one copy per device, loaded
// with the code object), so the library never allocates device memory; the
// per-device address is resolved once with hipGetSymbolAddress.
struct DeviceWorkspace {
  unsigned int *flags;  // kFlagWords words; word 0 holds the MQ_DEVFLAG_* bits
};
constexpr int kFlagWords = 64;
// The current device's workspace (resolved on first use; no allocation, so
// it is also safe inside graph capture).
int workspace(DeviceWorkspace **out, hipStream_t stream);

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16; NaN -> quiet NaN with the sign kept.
// Branch-free: both results are formed and one is selected.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet_nan = ((u >> 16) & 0x8000u) | 0x7fc0u;
  return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? quiet_nan : rounded);
}

// round_bf16(f) = bf16_to_f32(f32_to_bf16(f)).  v_cvt_pk_bf16_f32 rounds to
// nearest even exactly like f32_to_bf16 for every non-NaN float32 (denormals
// and infinities included; checked over all 2^32 bit patterns on gfx950), so
// the conversion is one instruction, with f32_to_bf16's canonical quiet NaN
// selected for NaN inputs.
__device__ __forceinline__ float round_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t hw = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f))) << 16;
  const uint32_t quiet_nan = (u & 0x80000000u) | 0x7fc00000u;
  return __uint_as_float((u & 0x7fffffffu) > 0x7f800000u ? quiet_nan : hw);
}

// Activation type traits: T storage and "one T-typed operation" rounding.
struct BF16T {
  using storage = uint16_t;
  static constexpr int dtype = MQ_BF16;
  __device__ static __forceinline__ float load(storage v) { return bf16_to_f32(v); }
  __device__ static __forceinline__ storage store(float f) { return f32_to_bf16(f); }
  __device__ static __forceinline__ float round(float f) { return round_bf16(f); }
};
struct F32T {
  using storage = float;
  static constexpr int dtype = MQ_F32;
  __device__ static __forceinline__ float load(storage v) { return v; }
  __device__ static __forceinline__ storage store(float f) { return f; }
  __device__ static __forceinline__ float round(float f) { return f; }
};

// ---------------------------------------------------------------- packed bf16 math
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// acc + a.lo*b.lo + a.hi*b.hi with bf16 pairs packed in 32-bit words.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// Activation chunk of 32 inputs held as 16 bf16 pairs in the order of the
// weights' nibble pairs (nibbles k and k+4 of a packed word, as the bf16 pair
// (128+q_k, 128+q_{k+4}); 0x4300 is bf16 128.0, whose 7 mantissa bits count
// in units of 1): for word j (inputs 8j..8j+7), p[4j+k] = (x[8j+k], x[8j+k+4]).
struct XChunk {
  uint32_t p[16];
  float osum;  // sum of the 32 bf16 values held in p (removes the 128 offset)
};

// Build the pair layout from 4 consecutive uint32 (8 bf16 values).
__device__ __forceinline__ void pairs_from_words(const uint32_t u[4], uint32_t *p) {
  // u0 = (x0,x1) u1 = (x2,x3) u2 = (x4,x5) u3 = (x6,x7), low half first.
  p[0] = __builtin_amdgcn_perm(u[2], u[0], 0x05040100u);  // (x0, x4)
  p[1] = __builtin_amdgcn_perm(u[2], u[0], 0x07060302u);  // (x1, x5)
  p[2] = __builtin_amdgcn_perm(u[3], u[1], 0x05040100u);  // (x2, x6)
  p[3] = __builtin_amdgcn_perm(u[3], u[1], 0x07060302u);  // (x3, x7)
}

// ---------------------------------------------------------------- DPP reductions
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over each 16-lane DPP row; every lane of the row receives a row sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x124>(v);  // row_ror:4
  v += dpp_f<0x128>(v);  // row_ror:8
  return v;
}

// Full 64-lane sum, uniform result (read through lane 0 of each DPP row).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, false));
}

template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = dpp_u<CTRL>(static_cast<uint32_t>(u));
  const uint32_t hi = dpp_u<CTRL>(static_cast<uint32_t>(u >> 32));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = readlane_u(static_cast<uint32_t>(u), lane);
  const uint64_t hi = readlane_u(static_cast<uint32_t>(u >> 32), lane);
  return __builtin_bit_cast(double, (hi << 32) | lo);
}

// Wave-uniform max of unsigned keys (all 64 lanes active).
__device__ __forceinline__ uint32_t wave_max_u32_uniform(uint32_t v) {
  v = max(v, dpp_u<0xb1>(v));
  v = max(v, dpp_u<0x4e>(v));
  v = max(v, dpp_u<0x124>(v));
  v = max(v, dpp_u<0x128>(v));
  return max(max(readlane_u(v, 0), readlane_u(v, 16)), max(readlane_u(v, 32), readlane_u(v, 48)));
}

// Wave-uniform float64 sum (all 64 lanes active).  The order is fixed:
// quads, then rows of 16, then the four rows.
__device__ __forceinline__ double wave_sum_f64_uniform(double v) {
  v += dpp_d<0xb1>(v);
  v += dpp_d<0x4e>(v);
  v += dpp_d<0x124>(v);
  v += dpp_d<0x128>(v);
  return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

// ---------------------------------------------------------------- expert addressing
struct ExpertPtrs {
  const uint32_t *w;
  const uint16_t *s;
  const uint16_t *b;
  bool ok;  // false: the word addresses no valid record; nothing may be read
};

// Resolve a route word to the rows of one projection
// (models/flashnext/metal_runtime.py:194-228; 64-bit pool offsets).  Words
// are bound-checked against the record or expert counts.
__device__ __forceinline__ ExpertPtrs expert_ptrs(const MqProjection &p, uint32_t word,
                                                  uint32_t out_w, uint32_t in_w,
                                                  uint32_t group, uint32_t dense_count) {
  ExpertPtrs r{nullptr, nullptr, nullptr, false};
  const uint8_t *rec = nullptr;
  if (word & MQ_SLOT_BIT) {
    const uint32_t slot = word & 0x7fffffffu;
    if (p.pool != nullptr && slot < p.pool_slots)
      rec = p.pool + p.pool_header + static_cast<uint64_t>(slot) * p.pool_stride;
  } else if (p.stream_pack != nullptr) {
    if (word < p.stream_records) rec = p.stream_pack + static_cast<uint64_t>(word) * p.pool_stride;
  } else if (p.weight != nullptr && word < dense_count) {
    const uint64_t e = word;
    r.w = p.weight + e * out_w * (in_w / 8);
    r.s = p.scales + e * out_w * (in_w / group);
    r.b = p.biases + e * out_w * (in_w / group);
    r.ok = true;
    return r;
  }
  if (rec != nullptr) {
    r.w = reinterpret_cast<const uint32_t *>(rec + p.off_weight);
    r.s = reinterpret_cast<const uint16_t *>(rec + p.off_scales);
    r.b = reinterpret_cast<const uint16_t *>(rec + p.off_biases);
    r.ok = true;
  }
  return r;
}

// ---------------------------------------------------------------- buffer resources
// Raw buffer descriptors (gfx9 descriptor word 3).  A buffer load whose byte
// offset lies beyond the descriptor's size returns zero without touching
// memory, so tails, masked rows and invalid records are handled without any
// branch around a load (a branch would make the compiler wait for each load
// before the next is issued).
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kOutOfRange = 0x80000000u;  // byte offset beyond every descriptor used here
constexpr int kNonTemporal = 2;                // buffer-load cache policy: non-temporal (streamed once)

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           kBufferWord3);
}

template <int AUX = 0>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, AUX);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint16_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, 0);
}

__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0));
}

// Descriptors of one projection of one expert (size 0 when the word is invalid).
struct ExpertRsrc {
  __amdgpu_buffer_rsrc_t w, s, b;
};

__device__ __forceinline__ ExpertRsrc expert_rsrc(const ExpertPtrs &e, uint32_t out_w, uint32_t in_w,
                                                  uint32_t group) {
  const uint32_t wbytes = e.ok ? out_w * (in_w / 8u) * 4u : 0u;
  const uint32_t gbytes = e.ok ? out_w * (in_w / group) * 2u : 0u;
  return {make_rsrc(e.w, wbytes), make_rsrc(e.s, gbytes), make_rsrc(e.b, gbytes)};
}

// Wave index as a scalar (uniform) value, so that everything derived from it
// (tiles, pairs, route words, record addresses) stays in scalar registers.
__device__ __forceinline__ uint32_t wave_id() {
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)));
}

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// Raise a device error flag (vector atomic from one lane).
__device__ __forceinline__ void raise_flag(unsigned int *flags, unsigned int bit) {
  if (flags != nullptr)
    __hip_atomic_fetch_or(flags, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- host helpers
inline uint32_t ceil_div(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

}  // namespace mq
