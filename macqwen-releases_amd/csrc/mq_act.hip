// Elementwise activations of the expert path and a device check of the bf16
// rounding the kernels use.
//
// mq_swiglu is MLX's swiglu(gate, up) as the reference executor calls it on
// its unfused up path (models/flashnext/metal_runtime.py:895-907), with the
// rounding points of the fused Up kernel's epilogue (:278-287): every step of
// the sigmoid sequence and both products rounded to T.  mq_sigmoid is the
// same sigmoid sequence alone (the shared-expert gate, mx.sigmoid in
// models/flashnext/adaptive_topk.py:264).  Both run the exact device
// sequences the decode and grouped kernels run (swiglu_bf16 per element,
// swiglu_bf16_n<4> in runs of four, with MQ_SWIGLU_TABLE the grouped gate/up
// epilogue's table-driven swiglu_bf16_tab_n<4>, sigmoid_bf16), so their
// outputs pin those sequences bit for bit.
#include <algorithm>

#include "mq_internal.h"
#include "mq_select.h"

namespace mq {
namespace {

constexpr int kActThreads = 256;

// Four elements per thread.  Runs of four use swiglu_bf16_n<4> unless `seq`
// selects the per-element sequence (the decode gate/up epilogue and the
// unfused decode pass) or the table-driven one of the grouped gate/up
// epilogue (the block fills its LDS table as the grouped kernel does); a
// tail of fewer than four elements always goes one at a time.
enum SwigluSeq : int { kSeqRuns = 0, kSeqScalar = 1, kSeqTable = 2 };

__global__ __launch_bounds__(kActThreads) void swiglu_bf16_kernel(const uint16_t *__restrict__ g,
                                                                   const uint16_t *__restrict__ u,
                                                                   uint16_t *__restrict__ out, uint64_t n, int seq) {
  __shared__ uint32_t sig_tab[kSigTabEntries];
  if (seq == kSeqTable) {  // uniform
    fill_sig_tab(sig_tab, threadIdx.x, kActThreads);
    __syncthreads();
  }
  const uint64_t i0 = (static_cast<uint64_t>(blockIdx.x) * kActThreads + threadIdx.x) * 4u;
  if (i0 >= n) return;
  if (i0 + 4u <= n && seq != kSeqScalar) {
    float gv[4], uv[4], v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gv[e] = bf16_to_f32(g[i0 + e]);
      uv[e] = bf16_to_f32(u[i0 + e]);
    }
    if (seq == kSeqTable) swiglu_bf16_tab_n<4>(gv, uv, v, sig_tab);
    else swiglu_bf16_n<4>(gv, uv, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) out[i0 + e] = f32_to_bf16(v[e]);
    return;
  }
  const uint64_t end = i0 + 4u < n ? i0 + 4u : n;
  for (uint64_t i = i0; i < end; ++i) out[i] = f32_to_bf16(swiglu_bf16(bf16_to_f32(g[i]), bf16_to_f32(u[i])));
}

__global__ __launch_bounds__(kActThreads) void swiglu_f32_kernel(const float *__restrict__ g,
                                                                  const float *__restrict__ u,
                                                                  float *__restrict__ out, uint64_t n) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kActThreads + threadIdx.x;
  if (i < n) out[i] = swiglu_t<F32T>(g[i], u[i]);
}

template <class TT>
__global__ __launch_bounds__(kActThreads) void sigmoid_kernel(const typename TT::storage *__restrict__ x,
                                                               typename TT::storage *__restrict__ out, uint64_t n) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kActThreads + threadIdx.x;
  if (i < n) out[i] = TT::store(sigmoid_t<TT>(TT::load(x[i])));
}

// For float32 bit patterns [first, first + count): counts[0] += patterns where
// round_bf16 differs from the integer round-to-nearest-even with canonical
// quiet NaN (f32_to_bf16), counts[1] += non-NaN patterns where the
// one-instruction conversion round_bf16_hw differs from it.  Grid-stride;
// one 64-bit atomic per thread that saw a mismatch.
__global__ __launch_bounds__(kActThreads) void bf16_round_check_kernel(uint64_t first, uint64_t count,
                                                                        unsigned long long *__restrict__ counts) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kActThreads;
  unsigned long long bad_round = 0, bad_hw = 0;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kActThreads + threadIdx.x; i < count; i += stride) {
    const uint32_t bits = static_cast<uint32_t>(first + i);
    const float f = __uint_as_float(bits);
    const uint32_t want = static_cast<uint32_t>(f32_to_bf16(f)) << 16;
    bad_round += __float_as_uint(round_bf16(f)) != want;
    const bool nan = (bits & 0x7fffffffu) > 0x7f800000u;
    bad_hw += !nan && __float_as_uint(round_bf16_hw(f)) != want;
  }
  if (bad_round) atomicAdd(&counts[0], bad_round);
  if (bad_hw) atomicAdd(&counts[1], bad_hw);
}

int check_elementwise(const void *a, const void *b, const void *out, uint64_t n, int dtype) {
  if (a == nullptr || b == nullptr || out == nullptr) return fail(MQ_ERR_INVALID, "inputs and out are required");
  if (dtype != MQ_BF16 && dtype != MQ_F32) return fail(MQ_ERR_INVALID, "dtype must be MQ_BF16 or MQ_F32");
  if (n >= (1ull << 31)) return fail(MQ_ERR_INVALID, "n must be below 2^31 (got %llu)", static_cast<unsigned long long>(n));
  return MQ_OK;
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" int mq_swiglu(const void *gate, const void *up, void *out, uint64_t n, int dtype, uint32_t flags,
                         void *stream) {
  int rc = check_elementwise(gate, up, out, n, dtype);
  if (rc) return rc;
  if (flags & ~(MQ_SWIGLU_SCALAR | MQ_SWIGLU_TABLE)) return fail(MQ_ERR_INVALID, "unknown flags 0x%x", flags);
  if ((flags & MQ_SWIGLU_SCALAR) && (flags & MQ_SWIGLU_TABLE))
    return fail(MQ_ERR_INVALID, "MQ_SWIGLU_SCALAR and MQ_SWIGLU_TABLE exclude each other");
  if (n == 0) return MQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MQ_BF16) {
    const uint64_t threads = (n + 3u) / 4u;
    hipLaunchKernelGGL(swiglu_bf16_kernel, dim3(ceil_div(threads, kActThreads)), dim3(kActThreads), 0, s,
                       static_cast<const uint16_t *>(gate), static_cast<const uint16_t *>(up),
                       static_cast<uint16_t *>(out), n,
                       (flags & MQ_SWIGLU_SCALAR) ? kSeqScalar : (flags & MQ_SWIGLU_TABLE) ? kSeqTable : kSeqRuns);
  } else {
    hipLaunchKernelGGL(swiglu_f32_kernel, dim3(ceil_div(n, kActThreads)), dim3(kActThreads), 0, s,
                       static_cast<const float *>(gate), static_cast<const float *>(up), static_cast<float *>(out),
                       n);
  }
  return check_launch("swiglu kernel");
}

extern "C" int mq_sigmoid(const void *x, void *out, uint64_t n, int dtype, void *stream) {
  int rc = check_elementwise(x, x, out, n, dtype);
  if (rc) return rc;
  if (n == 0) return MQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MQ_BF16)
    hipLaunchKernelGGL(sigmoid_kernel<BF16T>, dim3(ceil_div(n, kActThreads)), dim3(kActThreads), 0, s,
                       static_cast<const uint16_t *>(x), static_cast<uint16_t *>(out), n);
  else
    hipLaunchKernelGGL(sigmoid_kernel<F32T>, dim3(ceil_div(n, kActThreads)), dim3(kActThreads), 0, s,
                       static_cast<const float *>(x), static_cast<float *>(out), n);
  return check_launch("sigmoid kernel");
}

extern "C" int mq_bf16_round_check(uint64_t first, uint64_t count, unsigned long long *counts, void *stream) {
  if (counts == nullptr) return fail(MQ_ERR_INVALID, "counts is required");
  if (first > (1ull << 32) || count > (1ull << 32) - first)
    return fail(MQ_ERR_INVALID, "patterns [first, first + count) must lie in [0, 2^32)");
  if (count == 0) return MQ_OK;
  const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>(ceil_div(count, kActThreads), 8192u));
  hipLaunchKernelGGL(bf16_round_check_kernel, dim3(blocks), dim3(kActThreads), 0, static_cast<hipStream_t>(stream),
                     first, count, counts);
  return check_launch("bf16_round_check_kernel");
}
