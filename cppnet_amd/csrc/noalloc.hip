// The Linear backward for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  It runs the kernels of cnhip_linear_backward_act; their
// workspace -- the split-K partials of the dW / dX GEMMs and the row-chunk
// partials of the one-pass head backward -- comes from the fixed device
// array `scratch` below instead of the stream's growable scratch slot, and
// shapes whose workspace would not fit are refused before anything runs.
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.hpp"

// 32 MiB per device.  Each GPU the library runs on holds its own copy from
// the code object's load on that device until the process ends.  In host
// code `scratch` only names the symbol; its device address is looked up per
// device with hipGetSymbolAddress (scratch_address) and only that address
// is handed to kernels.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace cnhip {
size_t linear_backward_act_scratch_bytes(const float* X, const float* W, const float* dY,
                                         const float* grad_W, const float* dX, const float* act_aux, int64_t B,
                                         int64_t I, int64_t O, int trainable, int act);
}  // namespace cnhip

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// The current device's address of `scratch`, looked up on its first use on
// that device (with that device current) and kept.
int scratch_address(void** out, const char* who) {
  int dev = 0;
  CNHIP_TRY(cnhip::check_hip(hipGetDevice(&dev), who));
  CNHIP_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d is beyond the %d supported", who, dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    CNHIP_TRY(cnhip::check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), who));
    CNHIP_REQUIRE(p != nullptr, "%s: no device address for the workspace on device %d", who, dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CNHIP_OK;
}

}  // namespace

extern "C" int cnhip_linear_backward_act_noalloc(const float* X, const float* W, const float* dY, float* grad_W,
                                                 float* grad_b, float* dX, const float* act_aux, int64_t batch,
                                                 int64_t in_features, int64_t out_features, int trainable,
                                                 int accumulate, int act, cnhip_stream_t stream) {
  const char* who = "cnhip_linear_backward_act_noalloc";
  CNHIP_REQUIRE(batch >= 0 && in_features > 0 && out_features > 0, "%s: bad shape batch=%lld in=%lld out=%lld",
                who, (long long)batch, (long long)in_features, (long long)out_features);
  CNHIP_REQUIRE(act >= CNHIP_ACT_NONE && act <= CNHIP_ACT_RESIDUAL, "%s: bad activation %d", who, act);
  const size_t need = cnhip::linear_backward_act_scratch_bytes(X, W, dY, grad_W, dX, act_aux, batch, in_features,
                                                               out_features, trainable, act);
  CNHIP_REQUIRE(need <= kNoAllocScratchBytes,
                "%s: batch=%lld in=%lld out=%lld needs %zu bytes of workspace; the fixed device workspace "
                "holds %zu (cnhip_linear_backward_act has no such limit)",
                who, (long long)batch, (long long)in_features, (long long)out_features, need,
                kNoAllocScratchBytes);
  void* ptr = nullptr;
  CNHIP_TRY(scratch_address(&ptr, who));
  cnhip::FixedScratch fixed(ptr, kNoAllocScratchBytes);
  return cnhip_linear_backward_act(X, W, dY, grad_W, grad_b, dX, act_aux, batch, in_features, out_features,
                                   trainable, accumulate, act, stream);
}
