// Runtime services of the C ABI: errors, devices, memory, streams, events.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace cnhip {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int ws_alloc(void** ptr, size_t bytes, hipStream_t stream, const char* where) {
  static std::atomic<uint64_t> configured{0};  // one bit per device (< 64)
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), where));
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && !(configured.load(std::memory_order_acquire) & bit)) {
    hipMemPool_t pool;
    CNHIP_TRY(check_hip(hipDeviceGetDefaultMemPool(&pool, dev), where));
    uint64_t keep = UINT64_MAX;
    CNHIP_TRY(check_hip(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep), where));
    configured.fetch_or(bit, std::memory_order_acq_rel);
  }
  return check_hip(hipMallocAsync(ptr, bytes, stream), where);
}

namespace {
struct ScratchEntry {
  int dev;
  hipStream_t stream;
  int slot;
  void* p;
  size_t cap;
};
std::mutex g_scratch_mu;
std::vector<ScratchEntry> g_scratch;
}  // namespace

int scratch(hipStream_t stream, int slot, size_t bytes, void** ptr, const char* where) {
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), where));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchEntry* e = nullptr;
  for (auto& x : g_scratch)
    if (x.dev == dev && x.stream == stream && x.slot == slot) e = &x;
  if (!e) {
    g_scratch.push_back(ScratchEntry{dev, stream, slot, nullptr, 0});
    e = &g_scratch.back();
  }
  if (e->cap < bytes) {
    if (e->p) {
      void* old = e->p;
      e->p = nullptr;
      e->cap = 0;
      CNHIP_TRY(check_hip(hipFreeAsync(old, stream), where));
    }
    // grow with headroom, in 2 MiB steps, so slowly rising sizes settle
    size_t cap = bytes + bytes / 4;
    cap = (cap + ((size_t)2 << 20) - 1) & ~(((size_t)2 << 20) - 1);
    CNHIP_TRY(ws_alloc(&e->p, cap, stream, where));
    e->cap = cap;
  }
  *ptr = e->p;
  return CNHIP_OK;
}

}  // namespace cnhip

using cnhip::as_stream;
using cnhip::check_hip;

extern "C" {

const char* cnhip_last_error(void) { return cnhip::g_last_error; }

const char* cnhip_version(void) { return "cnhip 0.1 gfx950"; }

int cnhip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

int cnhip_set_device(int device) { return check_hip(hipSetDevice(device), "cnhip_set_device"); }

int cnhip_malloc(void** ptr, size_t bytes) {
  CNHIP_REQUIRE(ptr != nullptr, "cnhip_malloc: ptr is NULL");
  *ptr = nullptr;
  if (bytes == 0) return CNHIP_OK;
  return check_hip(hipMalloc(ptr, bytes), "cnhip_malloc");
}

int cnhip_free(void* ptr) {
  if (ptr == nullptr) return CNHIP_OK;
  return check_hip(hipFree(ptr), "cnhip_free");
}

int cnhip_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                       cnhip_stream_t stream) {
  if (bytes == 0) return CNHIP_OK;
  CNHIP_REQUIRE(dst && src, "cnhip_memcpy_async: NULL pointer");
  hipMemcpyKind k;
  switch (kind) {
    case 0: k = hipMemcpyHostToDevice; break;
    case 1: k = hipMemcpyDeviceToHost; break;
    case 2: k = hipMemcpyDeviceToDevice; break;
    default: cnhip::set_error("cnhip_memcpy_async: bad kind %d", kind); return CNHIP_EINVAL;
  }
  return check_hip(hipMemcpyAsync(dst, src, bytes, k, as_stream(stream)), "cnhip_memcpy_async");
}

int cnhip_memset_async(void* dst, int value, size_t bytes, cnhip_stream_t stream) {
  if (bytes == 0) return CNHIP_OK;
  CNHIP_REQUIRE(dst, "cnhip_memset_async: NULL pointer");
  return check_hip(hipMemsetAsync(dst, value, bytes, as_stream(stream)), "cnhip_memset_async");
}

int cnhip_stream_create(cnhip_stream_t* stream) {
  CNHIP_REQUIRE(stream, "cnhip_stream_create: NULL out pointer");
  hipStream_t s = nullptr;
  // Default priority only: streams of mixed priorities are not used here.
  int st = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "cnhip_stream_create");
  *stream = reinterpret_cast<cnhip_stream_t>(s);
  return st;
}

int cnhip_stream_destroy(cnhip_stream_t stream) {
  if (!stream) return CNHIP_OK;
  return check_hip(hipStreamDestroy(as_stream(stream)), "cnhip_stream_destroy");
}

int cnhip_stream_synchronize(cnhip_stream_t stream) {
  return check_hip(hipStreamSynchronize(as_stream(stream)), "cnhip_stream_synchronize");
}

int cnhip_device_synchronize(void) {
  return check_hip(hipDeviceSynchronize(), "cnhip_device_synchronize");
}

int cnhip_is_device_pointer(const void* ptr) {
  if (!ptr) return 0;
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged) ? 1 : 0;
}

int cnhip_event_create(void** event) {
  CNHIP_REQUIRE(event, "cnhip_event_create: NULL out pointer");
  hipEvent_t e = nullptr;
  int st = check_hip(hipEventCreate(&e), "cnhip_event_create");
  *event = reinterpret_cast<void*>(e);
  return st;
}

int cnhip_event_destroy(void* event) {
  if (!event) return CNHIP_OK;
  return check_hip(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "cnhip_event_destroy");
}

int cnhip_event_record(void* event, cnhip_stream_t stream) {
  CNHIP_REQUIRE(event, "cnhip_event_record: NULL event");
  return check_hip(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)),
                   "cnhip_event_record");
}

int cnhip_event_elapsed_ms(float* ms, void* start, void* stop) {
  CNHIP_REQUIRE(ms && start && stop, "cnhip_event_elapsed_ms: NULL argument");
  CNHIP_TRY(check_hip(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)),
                      "cnhip_event_elapsed_ms"));
  return check_hip(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                       reinterpret_cast<hipEvent_t>(stop)),
                   "cnhip_event_elapsed_ms");
}

}  // extern "C"
