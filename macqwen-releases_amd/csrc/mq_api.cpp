// Host-side ABI plumbing: error reporting, capability probe, record layout,
// per-device workspace and the expert-pool refill.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "mq_internal.h"

namespace mq {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t err, const char *what) {
  return fail(MQ_ERR_LAUNCH, "%s failed: %s", what, hipGetErrorString(err));
}

int check_launch(const char *what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(MQ_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(err));
  return MQ_OK;
}

namespace {
// Device error flags: one copy per device, zero-initialised when the code
// object is loaded.  Host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device.
__device__ __align__(256) unsigned int g_device_flags[kFlagWords];
}  // namespace

int workspace(DeviceWorkspace **out, hipStream_t stream) {
  (void)stream;
  static std::mutex mu;
  static DeviceWorkspace per_device[64];
  static bool ready[64] = {};
  int device = 0;
  MQ_TRY_HIP(hipGetDevice(&device));
  if (device < 0 || device >= 64) return fail(MQ_ERR_DEVICE, "device ordinal %d out of range", device);
  std::lock_guard<std::mutex> lock(mu);
  if (!ready[device]) {
    void *flags = nullptr;
    MQ_TRY_HIP(hipGetSymbolAddress(&flags, HIP_SYMBOL(g_device_flags)));
    per_device[device].flags = static_cast<unsigned int *>(flags);
    ready[device] = true;
  }
  *out = &per_device[device];
  return MQ_OK;
}

}  // namespace mq

using namespace mq;

extern "C" int mq_last_error(char *buf, uint32_t max_len) {
  if (buf == nullptr || max_len == 0) return MQ_ERR_INVALID;
  std::strncpy(buf, g_last_error.c_str(), max_len - 1);
  buf[max_len - 1] = '\0';
  return MQ_OK;
}

extern "C" int mq_version(void) { return 100; }

extern "C" int mq_init(void) {
  DeviceWorkspace *ws = nullptr;
  return workspace(&ws, nullptr);
}

extern "C" int mq_check_device_errors(void *stream, uint32_t *flags_out) {
  DeviceWorkspace *ws = nullptr;
  int rc = workspace(&ws, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  MQ_TRY_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  unsigned int flags = 0;
  MQ_TRY_HIP(hipMemcpy(&flags, ws->flags, sizeof(flags), hipMemcpyDeviceToHost));
  if (flags) {
    const unsigned int zero = 0u;
    MQ_TRY_HIP(hipMemcpy(ws->flags, &zero, sizeof(zero), hipMemcpyHostToDevice));
  }
  if (flags_out) *flags_out = flags;
  if (flags & MQ_DEVFLAG_BAD_ROUTE)
    return fail(MQ_ERR_INVALID, "a kernel skipped a route word that addressed no valid record or expert");
  if (flags & MQ_DEVFLAG_BAD_ROW)
    return fail(MQ_ERR_INVALID, "a gather row index was at or past the end of x");
  if (flags) return fail(MQ_ERR_INVALID, "device error flags 0x%x", flags);
  return MQ_OK;
}

extern "C" uint64_t mq_abi_struct_size(int which) {
  switch (which) {
    case 0: return sizeof(MqProjection);
    case 1: return sizeof(MqMoeArgs);
    case 2: return sizeof(MqRouteArgs);
    case 3: return sizeof(MqGroupedArgs);
    case 4: return sizeof(MqGatherArgs);
    default: return 0;
  }
}

extern "C" int mq_available(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    fail(MQ_ERR_DEVICE, "no HIP device visible");
    return 0;
  }
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    fail(MQ_ERR_DEVICE, "device %d is %s, this library is built for gfx950", device, prop.gcnArchName);
    return 0;
  }
  return 1;
}

// Part sizes in the reference's order gate/up/down x weight/scales/biases,
// packed back to back and rounded to a whole 4096-byte page
// (models/flashnext/slab_pack.py:96-149, generalised from 2560/640).
extern "C" int mq_record_layout(uint32_t hidden, uint32_t inter, uint32_t group_size, uint64_t offsets[9],
                                uint64_t *stride) {
  if (offsets == nullptr || stride == nullptr) return fail(MQ_ERR_INVALID, "offsets and stride are required");
  if (group_size != 32 && group_size != 64) return fail(MQ_ERR_INVALID, "group_size must be 32 or 64");
  if (hidden == 0 || inter == 0 || hidden % group_size || inter % group_size)
    return fail(MQ_ERR_INVALID, "hidden and inter must be positive multiples of group_size");
  const uint64_t shapes[3][2] = {{inter, hidden}, {inter, hidden}, {hidden, inter}};
  uint64_t cursor = 0;
  for (int p = 0; p < 3; ++p) {
    const uint64_t rows = shapes[p][0], cols = shapes[p][1];
    offsets[3 * p + 0] = cursor;
    cursor += rows * cols / 2;
    offsets[3 * p + 1] = cursor;
    cursor += rows * (cols / group_size) * 2;
    offsets[3 * p + 2] = cursor;
    cursor += rows * (cols / group_size) * 2;
  }
  *stride = (cursor + 4095) / 4096 * 4096;
  return MQ_OK;
}

extern "C" int mq_pool_refill_async(uint8_t *pool, uint64_t pool_header, uint64_t pool_stride, uint32_t pool_slots,
                                    const uint32_t *slots, const void *const *host_records, uint32_t n,
                                    uint64_t record_bytes, void *copy_stream, void *done_event) {
  if (n == 0) {
    if (done_event) MQ_TRY_HIP(hipEventRecord(static_cast<hipEvent_t>(done_event), static_cast<hipStream_t>(copy_stream)));
    return MQ_OK;
  }
  if (pool == nullptr || slots == nullptr || host_records == nullptr)
    return fail(MQ_ERR_INVALID, "pool, slots and host_records are required");
  if (record_bytes == 0 || record_bytes > pool_stride)
    return fail(MQ_ERR_INVALID, "record_bytes must be in 1..pool_stride");
  hipStream_t s = static_cast<hipStream_t>(copy_stream);
  for (uint32_t i = 0; i < n; ++i) {  // validate everything before the first copy
    if (host_records[i] == nullptr) return fail(MQ_ERR_INVALID, "host record %u is NULL", i);
    if ((slots[i] & 0x7fffffffu) >= pool_slots)
      return fail(MQ_ERR_INVALID, "slot %u is outside the pool (%u slots)", slots[i] & 0x7fffffffu, pool_slots);
  }
  for (uint32_t i = 0; i < n; ++i) {
    uint8_t *dst = pool + pool_header + static_cast<uint64_t>(slots[i] & 0x7fffffffu) * pool_stride;
    MQ_TRY_HIP(hipMemcpyAsync(dst, host_records[i], record_bytes, hipMemcpyHostToDevice, s));
  }
  if (done_event) MQ_TRY_HIP(hipEventRecord(static_cast<hipEvent_t>(done_event), s));
  return MQ_OK;
}
