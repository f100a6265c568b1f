// Floors measured on the device the library runs on: the cost of a kernel
// boundary, of streaming a layer's expert bytes with no compute, and of a
// dependent load right after a kernel starts (the decode layer is a chain of
// such boundaries and hops, so these bound it from below), and the sustained
// issue rate of the bf16 MFMA the grouped GEMMs use.  No reference
// counterpart.
#include <hip/hip_runtime.h>

#include "mq_internal.h"

namespace mq {
namespace {

constexpr uint32_t kProbeThreads = 256;
constexpr uint32_t kProbeUnroll = 4;  // 16-byte loads in flight per thread
constexpr uint32_t kProbeHops = 8;

typedef unsigned int u32x4p_t __attribute__((ext_vector_type(4)));

// Block b streams share b / n of segment b % n (non-temporal 16-byte loads,
// as the expert kernels read weights) and folds the words into a checksum
// that is stored only if it matches `never`, so the loads are kept.
__global__ __launch_bounds__(kProbeThreads) void stream_probe_kernel(const uint64_t *__restrict__ segs, uint32_t n,
                                                                     uint64_t chunks, uint32_t never,
                                                                     uint32_t *__restrict__ sink) {
  if (n == 0) return;
  const uint32_t seg = blockIdx.x % n, part = blockIdx.x / n, parts = gridDim.x / n;
  const u32x4p_t *src = reinterpret_cast<const u32x4p_t *>(segs[seg]);
  const uint64_t begin = chunks * part / parts, end = chunks * (part + 1) / parts;
  uint32_t acc = 0u;
  for (uint64_t i = begin + threadIdx.x; i < end; i += kProbeThreads * kProbeUnroll) {
    u32x4p_t v[kProbeUnroll];
#pragma unroll
    for (uint32_t k = 0; k < kProbeUnroll; ++k) {
      const uint64_t c = i + k * kProbeThreads;
      v[k] = c < end ? __builtin_nontemporal_load(src + c) : u32x4p_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (uint32_t k = 0; k < kProbeUnroll; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  if (acc == never) sink[0] = acc;
}

// Thread 0 of the last block (block b runs on XCD b mod 8) follows a pointer
// chain of `hops` links from `chain` and records the real-time clock
// (100 MHz) at the start and after each arrival.
__global__ void hop_probe_kernel(const uint64_t *chain, uint32_t hops, uint64_t *__restrict__ stamps) {
  if (blockIdx.x + 1 != gridDim.x || threadIdx.x != 0) return;
  uint64_t t[kProbeHops + 1];
  t[0] = __builtin_amdgcn_s_memrealtime();
  uint64_t p = reinterpret_cast<uint64_t>(chain);
#pragma unroll
  for (uint32_t h = 0; h < kProbeHops; ++h) {
    if (h < hops) {
      p = *reinterpret_cast<const uint64_t *>(p);  // an ordinary cached load, as the kernels' loads are
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clock read waits for the link to arrive
      t[h + 1] = __builtin_amdgcn_s_memrealtime();
    } else {
      t[h + 1] = t[h];
    }
  }
#pragma unroll
  for (uint32_t h = 0; h <= kProbeHops; ++h) stamps[h] = t[h];
  stamps[kProbeHops + 1] = p;  // the chain's end, so the loads are kept
}

// Each wave issues `iters` rounds of four independent bf16 MFMAs
// (v_mfma_f32_32x32x16_bf16) on register operands, two waves per SIMD as the
// grouped GEMM runs; the sums go to `sink` so the MFMAs are kept.
typedef __bf16 bf16x8p_t __attribute__((ext_vector_type(8)));
typedef float f32x16p_t __attribute__((ext_vector_type(16)));
constexpr uint32_t kMfmaProbeThreads = 512;

__global__ __launch_bounds__(kMfmaProbeThreads, 1) void mfma_probe_kernel(uint32_t iters, float *__restrict__ sink) {
  bf16x8p_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(0.001f * static_cast<float>(threadIdx.x + i));
    b[i] = static_cast<__bf16>(0.002f * static_cast<float>(i));
  }
  f32x16p_t acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
  for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[t], 0, 0, 0);
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[t][r];
  sink[static_cast<uint64_t>(blockIdx.x) * kMfmaProbeThreads + threadIdx.x] = s;
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" int mq_mfma_probe(uint32_t iters, uint32_t blocks, float *sink, void *stream) {
  if (sink == nullptr) return fail(MQ_ERR_INVALID, "sink is required");
  if (iters == 0 || iters > (1u << 24)) return fail(MQ_ERR_INVALID, "iters must be in 1..2^24");
  if (blocks == 0 || blocks > 65535u) return fail(MQ_ERR_INVALID, "blocks must be in 1..65535");
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(kMfmaProbeThreads), 0, static_cast<hipStream_t>(stream),
                     iters, sink);
  return check_launch("mfma_probe_kernel");
}

extern "C" int mq_stream_probe(const uint64_t *segments, uint32_t n, uint64_t bytes_each, uint32_t blocks,
                               uint32_t *sink, void *stream) {
  if (n > 0 && (segments == nullptr || sink == nullptr)) return fail(MQ_ERR_INVALID, "segments and sink are required");
  if (bytes_each % 16u) return fail(MQ_ERR_INVALID, "bytes_each must be a multiple of 16");
  if (n > 0 && (blocks < n || blocks % n)) return fail(MQ_ERR_INVALID, "blocks must be a positive multiple of n");
  hipLaunchKernelGGL(stream_probe_kernel, dim3(n > 0 ? blocks : 1u), dim3(kProbeThreads), 0,
                     static_cast<hipStream_t>(stream), segments, n, bytes_each / 16u, 0x9e3779b9u, sink);
  return check_launch("stream_probe_kernel");
}

extern "C" int mq_hop_probe(const uint64_t *chain, uint32_t hops, uint64_t *stamps, uint32_t block, void *stream) {
  if (chain == nullptr || stamps == nullptr) return fail(MQ_ERR_INVALID, "chain and stamps are required");
  if (hops == 0 || hops > kProbeHops) return fail(MQ_ERR_INVALID, "hops must be in 1..%u", kProbeHops);
  if (block > 63) return fail(MQ_ERR_INVALID, "block must be in 0..63");
  hipLaunchKernelGGL(hop_probe_kernel, dim3(block + 1), dim3(64), 0, static_cast<hipStream_t>(stream), chain, hops,
                     stamps);
  return check_launch("hop_probe_kernel");
}
