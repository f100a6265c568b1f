// Q4 primitives: nibble unpack and affine dequantisation to bf16.
//
// Unpack order is the reference's: value k of a row is nibble (k & 7) of
// word k >> 3, LSB first (models/flashnext/metal_runtime.py:980).  Dequant
// is bf16(s*q + b) with the product exact in float32 and one float32
// rounding for the add (mx.dequantize's arithmetic in float).
#include "mq_internal.h"

namespace mq {
namespace {

__global__ void unpack_kernel(const uint32_t *__restrict__ words, uint2 *__restrict__ out, uint64_t n) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t w = words[i];
  // Spread 8 nibbles into 8 bytes: byte k = nibble k.
  uint32_t lo = (w & 0xfu) | ((w & 0xf0u) << 4) | ((w & 0xf00u) << 8) | ((w & 0xf000u) << 12);
  const uint32_t h = w >> 16;
  uint32_t hi = (h & 0xfu) | ((h & 0xf0u) << 4) | ((h & 0xf00u) << 8) | ((h & 0xf000u) << 12);
  out[i] = make_uint2(lo, hi);
}

// One thread per packed word: 8 outputs written as one 16-byte store.
__global__ void dequant_kernel(const uint32_t *__restrict__ w, const uint16_t *__restrict__ s,
                               const uint16_t *__restrict__ b, uint4 *__restrict__ out, uint32_t rows,
                               uint32_t cols, uint32_t group) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint32_t words_per_row = cols / 8;
  if (i >= static_cast<uint64_t>(rows) * words_per_row) return;
  const uint64_t row = i / words_per_row;
  const uint32_t word = static_cast<uint32_t>(i % words_per_row);
  const uint32_t g = word * 8 / group;
  const uint64_t gi = row * (cols / group) + g;
  const float sc = bf16_to_f32(s[gi]);
  const float bi = bf16_to_f32(b[gi]);
  const uint32_t v = w[i];
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float q0 = static_cast<float>((v >> (8 * k)) & 15u);
    const float q1 = static_cast<float>((v >> (8 * k + 4)) & 15u);
    const uint16_t d0 = f32_to_bf16(__fadd_rn(__fmul_rn(sc, q0), bi));
    const uint16_t d1 = f32_to_bf16(__fadd_rn(__fmul_rn(sc, q1), bi));
    o[k] = static_cast<uint32_t>(d0) | (static_cast<uint32_t>(d1) << 16);
  }
  out[i] = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" int mq_q4_unpack(const uint32_t *words, uint8_t *values, uint64_t n_words, void *stream) {
  if (n_words == 0) return MQ_OK;
  if (words == nullptr || values == nullptr) return fail(MQ_ERR_INVALID, "words and values are required");
  hipLaunchKernelGGL(unpack_kernel, dim3(ceil_div(n_words, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     words, reinterpret_cast<uint2 *>(values), n_words);
  return check_launch("unpack_kernel");
}

extern "C" int mq_q4_dequant(const uint32_t *weight, const uint16_t *scales, const uint16_t *biases,
                             uint16_t *out, uint32_t rows, uint32_t cols, uint32_t group_size,
                             void *stream) {
  if (weight == nullptr || scales == nullptr || biases == nullptr || out == nullptr)
    return fail(MQ_ERR_INVALID, "weight, scales, biases and out are required");
  if (group_size != 32 && group_size != 64) return fail(MQ_ERR_INVALID, "group_size must be 32 or 64");
  if (cols == 0 || cols % group_size) return fail(MQ_ERR_INVALID, "cols must be a positive multiple of group_size");
  if (rows == 0) return MQ_OK;
  const uint64_t n = static_cast<uint64_t>(rows) * (cols / 8);
  hipLaunchKernelGGL(dequant_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     weight, scales, biases, reinterpret_cast<uint4 *>(out), rows, cols, group_size);
  return check_launch("dequant_kernel");
}
