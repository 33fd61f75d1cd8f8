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
  uint64_t gen;  // which allocation p is (unique over the process)
};
uint64_t g_scratch_gens = 0;
std::mutex g_scratch_mu;
std::vector<ScratchEntry> g_scratch;
// Streams whose scratch slots a captured graph refers to: their buffers
// must keep their addresses, so a request that would grow one fails.
std::vector<std::pair<int, hipStream_t>> g_frozen;

bool frozen(int dev, hipStream_t stream) {
  for (auto& f : g_frozen)
    if (f.first == dev && f.second == stream) return true;
  return false;
}

__global__ void fill_bytes_kernel(unsigned char* __restrict__ dst, uint32_t word, size_t n16,
                                  size_t tail) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint4* d4 = reinterpret_cast<uint4*>(dst);
  const uint4 v = make_uint4(word, word, word, word);
  for (size_t i = t0; i < n16; i += stride) d4[i] = v;
  if (t0 < tail) dst[n16 * 16 + t0] = (unsigned char)(word & 0xffu);
}

__global__ void fill_bytes_unaligned_kernel(unsigned char* __restrict__ dst, unsigned char v,
                                            size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = v;
}
}  // namespace

int fill_bytes(void* dst, int value, size_t bytes, hipStream_t stream, const char* where) {
  if (bytes == 0) return CNHIP_OK;
  const uint32_t b = (uint32_t)value & 0xffu;
  unsigned char* d = static_cast<unsigned char*>(dst);
  HbmTimer timer("fill_bytes_kernel", (double)bytes, stream);
  if (aligned16(dst)) {
    const size_t n16 = bytes / 16, tail = bytes % 16;
    const unsigned grid = elementwise_grid((int64_t)(n16 > tail ? n16 : tail), 256);
    hipLaunchKernelGGL(fill_bytes_kernel, dim3(grid), dim3(256), 0, stream, d,
                       b * 0x01010101u, n16, tail);
  } else {
    hipLaunchKernelGGL(fill_bytes_unaligned_kernel, dim3(elementwise_grid((int64_t)bytes, 256)),
                       dim3(256), 0, stream, d, (unsigned char)b, bytes);
  }
  return check_launch(where);
}

namespace {
struct FixedWs {
  void* p = nullptr;
  size_t cap = 0;
};
thread_local FixedWs t_fixed;
}  // namespace

FixedScratch::FixedScratch(void* p, size_t cap) { t_fixed = FixedWs{p, cap}; }
FixedScratch::~FixedScratch() { t_fixed = FixedWs{}; }
bool fixed_scratch_active() { return t_fixed.p != nullptr; }

namespace {
std::mutex g_persist_mu;
struct PersistOrder {
  hipEvent_t ev = nullptr;
  bool recorded = false;
};
PersistOrder g_persist_order[64];  // per device
}  // namespace

void persist_order_lock() { g_persist_mu.lock(); }
void persist_order_unlock() { g_persist_mu.unlock(); }

int persist_order_enter(hipStream_t stream, const char* who, int* dev) {
  CNHIP_TRY(check_hip(hipGetDevice(dev), who));
  CNHIP_REQUIRE(*dev >= 0 && *dev < 64, "%s: device %d is beyond the 64 supported", who, *dev);
  PersistOrder& o = g_persist_order[*dev];
  if (o.recorded) CNHIP_TRY(check_hip(hipStreamWaitEvent(stream, o.ev, 0), who));
  return CNHIP_OK;
}

int persist_order_leave(hipStream_t stream, int dev, const char* who) {
  PersistOrder& o = g_persist_order[dev];
  if (!o.ev) CNHIP_TRY(check_hip(hipEventCreateWithFlags(&o.ev, hipEventDisableTiming), who));
  CNHIP_TRY(check_hip(hipEventRecord(o.ev, stream), who));
  o.recorded = true;
  return CNHIP_OK;
}

int scratch(hipStream_t stream, int slot, size_t bytes, void** ptr, const char* where) {
  return scratch(stream, slot, bytes, ptr, nullptr, where);
}

int scratch(hipStream_t stream, int slot, size_t bytes, void** ptr, uint64_t* gen, const char* where) {
  if (t_fixed.p) {
    if (slot != kScratchGemm) {
      set_error("%s: scratch slot %d requested inside a no-allocation call", where, slot);
      return CNHIP_EUNSUPPORTED;
    }
    if (bytes > t_fixed.cap) {
      set_error("%s: needs %zu bytes of workspace; the fixed device workspace holds %zu", where, bytes,
                t_fixed.cap);
      return CNHIP_EINVAL;
    }
    *ptr = t_fixed.p;
    if (gen) *gen = 0;
    return CNHIP_OK;
  }
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), where));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchEntry* e = nullptr;
  for (auto& x : g_scratch)
    if (x.dev == dev && x.stream == stream && x.slot == slot) e = &x;
  if (!e) {
    g_scratch.push_back(ScratchEntry{dev, stream, slot, nullptr, 0, 0});
    e = &g_scratch.back();
  }
  if (e->cap < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    CNHIP_TRY(check_hip(hipStreamIsCapturing(stream, &cs), where));
    if (cs != hipStreamCaptureStatusNone || frozen(dev, stream)) {
      set_error("%s: scratch slot %d of this stream must grow to %zu bytes (has %zu) while a "
                "captured graph uses it; run the work once uncaptured before capturing it",
                where, slot, bytes, e->cap);
      return CNHIP_EUNSUPPORTED;
    }
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
    e->gen = ++g_scratch_gens;
  }
  *ptr = e->p;
  if (gen) *gen = e->gen;
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

int cnhip_get_device(int* device) {
  CNHIP_REQUIRE(device, "cnhip_get_device: NULL out pointer");
  return check_hip(hipGetDevice(device), "cnhip_get_device");
}

int cnhip_host_alloc(void** ptr, size_t bytes) {
  CNHIP_REQUIRE(ptr != nullptr, "cnhip_host_alloc: ptr is NULL");
  *ptr = nullptr;
  if (bytes == 0) return CNHIP_OK;
  return check_hip(hipHostMalloc(ptr, bytes, hipHostMallocDefault), "cnhip_host_alloc");
}

int cnhip_host_free(void* ptr) {
  if (!ptr) return CNHIP_OK;
  return check_hip(hipHostFree(ptr), "cnhip_host_free");
}

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
  return cnhip::fill_bytes(dst, value, bytes, as_stream(stream), "cnhip_memset_async");
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

int cnhip_event_synchronize(void* event) {
  CNHIP_REQUIRE(event, "cnhip_event_synchronize: NULL event");
  return check_hip(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)), "cnhip_event_synchronize");
}

int cnhip_stream_wait_event(cnhip_stream_t stream, void* event) {
  CNHIP_REQUIRE(event, "cnhip_stream_wait_event: NULL event");
  return check_hip(hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0),
                   "cnhip_stream_wait_event");
}

int cnhip_event_elapsed_ms(float* ms, void* start, void* stop) {
  CNHIP_REQUIRE(ms && start && stop, "cnhip_event_elapsed_ms: NULL argument");
  CNHIP_TRY(check_hip(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)),
                      "cnhip_event_elapsed_ms"));
  return check_hip(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                       reinterpret_cast<hipEvent_t>(stop)),
                   "cnhip_event_elapsed_ms");
}

// ---- graphs: capture of a stream's work, replay -------------------------
namespace {
struct Graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int dev = 0;
  hipStream_t stream = nullptr;  // whose scratch slots the graph uses
};
}  // namespace

int cnhip_graph_begin_capture(cnhip_stream_t stream) {
  const char* who = "cnhip_graph_begin_capture";
  CNHIP_REQUIRE(stream != nullptr, "%s: capture needs a created stream, not the default stream", who);
  CNHIP_REQUIRE(!cnhip::timing_on(), "%s: per-launch kernel timing is enabled; disable it first", who);
  // Relaxed: allocations of not-yet-cached buffers by the host layer may
  // call hipMalloc while the capture is open (that is not stream work).
  return check_hip(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeRelaxed), who);
}

int cnhip_graph_end_capture(cnhip_stream_t stream, int ok, cnhip_graph_t* graph) {
  const char* who = "cnhip_graph_end_capture";
  CNHIP_REQUIRE(stream != nullptr, "%s: NULL stream", who);
  if (graph) *graph = nullptr;
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(as_stream(stream), &g);
  if (e != hipSuccess || !ok || !graph) {
    if (g) (void)hipGraphDestroy(g);
    if (e != hipSuccess) return check_hip(e, who);
    CNHIP_REQUIRE(graph, "%s: NULL out pointer", who);
    return CNHIP_OK;  // capture abandoned by the caller
  }
  auto* G = new Graph;
  G->graph = g;
  G->stream = as_stream(stream);
  int st = check_hip(hipGetDevice(&G->dev), who);
  if (st == CNHIP_OK) st = check_hip(hipGraphInstantiate(&G->exec, g, nullptr, nullptr, 0), who);
  if (st != CNHIP_OK) {
    (void)hipGraphDestroy(g);
    delete G;
    return st;
  }
  {
    std::lock_guard<std::mutex> lock(cnhip::g_scratch_mu);
    cnhip::g_frozen.emplace_back(G->dev, G->stream);
  }
  *graph = G;
  return CNHIP_OK;
}

int cnhip_graph_launch(cnhip_graph_t graph, cnhip_stream_t stream) {
  CNHIP_REQUIRE(graph, "cnhip_graph_launch: NULL graph");
  // a persistent recurrence launch of an earlier replay that gave up is
  // reported here, before anything is replayed on top of its outputs
  CNHIP_TRY(cnhip::recurrence_fault_check(as_stream(stream), "cnhip_graph_launch"));
  auto* G = static_cast<Graph*>(graph);
  CNHIP_REQUIRE(as_stream(stream) == G->stream,
                "cnhip_graph_launch: a graph replays on the stream it was captured on (its scratch "
                "slots are that stream's)");
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  CNHIP_TRY(check_hip(hipStreamIsCapturing(as_stream(stream), &cs), "cnhip_graph_launch"));
  return cnhip::persist_ordered(as_stream(stream), cs != hipStreamCaptureStatusNone, "cnhip_graph_launch", [&] {
    return check_hip(hipGraphLaunch(G->exec, as_stream(stream)), "cnhip_graph_launch");
  });
}

int cnhip_graph_destroy(cnhip_graph_t graph) {
  if (!graph) return CNHIP_OK;
  auto* G = static_cast<Graph*>(graph);
  int st = check_hip(hipStreamSynchronize(G->stream), "cnhip_graph_destroy");
  if (G->exec) (void)hipGraphExecDestroy(G->exec);
  if (G->graph) (void)hipGraphDestroy(G->graph);
  {
    std::lock_guard<std::mutex> lock(cnhip::g_scratch_mu);
    auto& fz = cnhip::g_frozen;
    for (size_t i = 0; i < fz.size(); ++i)
      if (fz[i].first == G->dev && fz[i].second == G->stream) {
        fz.erase(fz.begin() + (long)i);  // one entry per live graph
        break;
      }
  }
  delete G;
  return st;
}

}  // extern "C"
