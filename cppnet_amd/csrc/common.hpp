// Shared helpers of the HIP library: status/error plumbing and launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "cnhip.h"

namespace cnhip {

// Records the message returned by cnhip_last_error() for this host thread.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline hipStream_t as_stream(cnhip_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that was just enqueued.
inline int check_launch(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", where, hipGetErrorString(e));
    return CNHIP_EHIP;
  }
  return CNHIP_OK;
}

// Stream-ordered workspace allocation (split-K partials, scratch).  The
// first call on a device raises the release threshold of its default memory
// pool to the maximum, so freed workspaces stay pooled across
// synchronizations (a training step re-allocates the same sizes every step;
// with the default threshold of 0 the pool hands memory back at each sync and
// the next step pays for real allocations).
int ws_alloc(void** ptr, size_t bytes, hipStream_t stream, const char* where);

// Reusable workspace for work queued on `stream`: a buffer of >= bytes held
// per (device, stream, slot) and handed out again on later calls, so a
// training step allocates nothing once sizes have been seen (stream-ordered
// allocate/free cost ~50-120 us of host time per call on this runtime, more
// than the kernels they serve).  Every user of a slot runs its kernels on
// that stream, which orders the reuse; growth releases the old buffer in
// stream order too.  Slot 0 is the GEMM's split-K partials, slot 1 the
// layer-level workspaces (which may call the GEMM while holding theirs).
// Calls on one stream from several host threads at once are not supported.
constexpr int kScratchGemm = 0, kScratchLayer = 1;
int scratch(hipStream_t stream, int slot, size_t bytes, void** ptr, const char* where);
// The same, also returning in *gen which allocation the buffer is: a number
// unique over the process, new whenever the slot's buffer is (re)allocated
// (its contents are then undefined).  Not for the no-allocation calls.
int scratch(hipStream_t stream, int slot, size_t bytes, void** ptr, uint64_t* gen, const char* where);

// While one is in scope on this host thread, a caller-provided device
// buffer of `cap` bytes stands in for the GEMM scratch slot of every stream
// (the no-allocation entry points): scratch() hands out `p` for slot
// kScratchGemm when the request fits, fails with CNHIP_EINVAL when it does
// not, and refuses the other slots; the per-launch timing records are
// switched off, since they create events on first use.  Nothing is
// allocated while it is active.  Not nestable.
struct FixedScratch {
  FixedScratch(void* p, size_t cap);
  ~FixedScratch();
  FixedScratch(const FixedScratch&) = delete;
  FixedScratch& operator=(const FixedScratch&) = delete;
};
bool fixed_scratch_active();

// Runs launch(), which enqueues device work on `stream` that must not run
// at the same time as other such work of this process on the device: the
// persistent recurrence kernels (a grid that spins until all of its blocks
// have run a step; two such grids dispatched at once could each be left
// partly resident) and the replay of a graph that may contain one.  The
// stream first waits for the device's previous such launch (an event), and
// an event recorded after launch() marks this one.  Under stream capture
// nothing is waited for or recorded (graph replays are ordered by
// cnhip_graph_launch itself).
int persist_order_enter(hipStream_t stream, const char* who, int* dev);
int persist_order_leave(hipStream_t stream, int dev, const char* who);
void persist_order_lock();
void persist_order_unlock();
template <class F>
int persist_ordered(hipStream_t stream, bool capturing, const char* who, F&& launch) {
  if (capturing) return launch();
  persist_order_lock();
  int dev = 0;
  int st = persist_order_enter(stream, who, &dev);
  if (st == CNHIP_OK) st = launch();
  if (st == CNHIP_OK) st = persist_order_leave(stream, dev, who);
  persist_order_unlock();
  return st;
}

// Optimizer guard.  A persistent recurrence launch that gives up waiting
// sets the current device's guard word; while it is set, every optimizer
// kernel leaves its tensors unchanged and lowers *first_withheld to its
// launch's sequence number, so invalid recurrent outputs never reach the
// parameters.  update_guard fills the current device's words and the next
// sequence number (update_seq_last() returns it to the caller's thread).
// recurrence_fault_check reports a pending fault (CNHIP_EHIP) and takes it:
// it synchronizes the device, clears the guard and records the range of
// sequence numbers withheld (update_withheld(seq): 1 for a launch in one;
// update_faults_taken() counts the faults taken); without a pending fault it
// costs one read of a host word.
struct UpdateGuard {
  const unsigned* withhold;
  unsigned long long* first_withheld;
  unsigned long long seq;
};
int update_guard(UpdateGuard* out, const char* who);
int recurrence_fault_check(hipStream_t st, const char* who);
int update_withheld(int64_t seq);
int64_t update_faults_taken();
int64_t update_seq_last();

// In an optimizer kernel: whether this launch is withheld (the block's first
// thread then records it).
__device__ __forceinline__ bool update_withheld(const UpdateGuard& g) {
  if (__builtin_expect(*g.withhold == 0u, 1)) return false;
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_fetch_min(g.first_withheld, g.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// The arguments of one GEMM (the parameters of gemm_f32_core in
// gemm_f32.hip: op(A) is M x K, op(B) K x N, C M x N, all column-major,
// strides between batch entries).
struct GemmSpec {
  int trans_a, trans_b;
  int64_t M, N, K;
  float alpha;
  const float* A;
  int64_t lda, stride_a;
  const float* B;
  int64_t ldb, stride_b;
  float beta;
  float* C;
  int64_t ldc, stride_c, batches;
  const float* bias;
  int epilogue;
  const float* aux_in;
  float* aux_out;
  int64_t ld_aux;
};

// x then y, in one launch where both GEMMs are of a shape that leaves half
// of the chip's block slots empty (gemm_f32.hip); otherwise one after the
// other.  The two must be independent: neither reads what the other writes.
// With cs_out set, also cs_out[c] (+)= the sum of column c of the
// column-major [cs_rows, cs_cols] cs_in (a bias gradient), in the launch of
// y's split-K reduce when there is one (the same bits as column_sum).
int gemm_f32_pair(const GemmSpec& x, const GemmSpec& y, hipStream_t st, const char* who,
                  const float* cs_in = nullptr, float* cs_out = nullptr, int64_t cs_rows = 0, int64_t cs_cols = 0,
                  int cs_accumulate = 0);

// Bytes of GEMM scratch (split-K partials) that gemm_f32_core requests for
// this shape: 0 when it runs without a split.
size_t gemm_scratch_bytes(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, int64_t batches);

inline int check_hip(hipError_t e, const char* where) {
  if (e != hipSuccess) {
    set_error("%s: %s", where, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? CNHIP_ENOMEM : CNHIP_EHIP;
  }
  return CNHIP_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Grid size for a grid-stride elementwise kernel: enough waves to fill the
// 256 CUs (8 XCDs x 32) several times over without launching one block per
// element for very large n.
inline unsigned elementwise_grid(int64_t work_items, int block) {
  int64_t blocks = (work_items + block - 1) / block;
  const int64_t cap = 256 * 32;  // 32 blocks per CU
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return static_cast<unsigned>(blocks);
}

// Per-launch timing of the MFMA GEMM-shaped kernels (cnhip_gemm_timing_*):
// while enabled, a launch site brackets its kernel with rec->start/stop on
// the launch stream.  timing_slot returns nullptr when timing is off.
struct TimingRec {
  hipEvent_t start, stop;
  double flops;         // MFMA records: algorithmic flops of the launch
  const char* kernel;   // HBM records: kernel name (static string), else nullptr
  double bytes;         // HBM records: algorithmic bytes of the launch
};
TimingRec* timing_slot(double flops);
// Per-launch timing of the bandwidth-bound kernels (cnhip_hbm_timing_*),
// credited with the launch's algorithmic HBM bytes; nullptr when off.
TimingRec* hbm_timing_slot(const char* kernel, double bytes);
bool timing_on();  // either kind of per-launch timing is enabled

// Brackets the launches of its scope with an HBM timing record.
struct HbmTimer {
  TimingRec* rec;
  hipStream_t st;
  HbmTimer(const char* kernel, double bytes, hipStream_t s) : rec(hbm_timing_slot(kernel, bytes)), st(s) {
    if (rec) (void)hipEventRecord(rec->start, st);
  }
  ~HbmTimer() {
    if (rec) (void)hipEventRecord(rec->stop, st);
  }
  HbmTimer(const HbmTimer&) = delete;
  HbmTimer& operator=(const HbmTimer&) = delete;
};

// Fills `bytes` bytes at dst with the byte `value` by a kernel on `stream`
// (not hipMemsetAsync: a memset node recorded into a captured graph has
// given wrong results on replays after the first on this platform).
int fill_bytes(void* dst, int value, size_t bytes, hipStream_t stream, const char* where);

}  // namespace cnhip

#define CNHIP_REQUIRE(cond, ...)           \
  do {                                     \
    if (!(cond)) {                         \
      ::cnhip::set_error(__VA_ARGS__);     \
      return CNHIP_EINVAL;                 \
    }                                      \
  } while (0)

#define CNHIP_TRY(expr)               \
  do {                                \
    int _st = (expr);                 \
    if (_st != CNHIP_OK) return _st;  \
  } while (0)
