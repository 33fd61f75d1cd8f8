// LSTM and GRU forward / backward-through-time on MI355X.
//
// ref: LSTM::forward/backward src/CppNet/layers/lstm.cpp:63-253,
//      GRU::forward/backward  src/CppNet/layers/gru.cpp:56-297,
//      lstm_cell.cu:21-114, gru_cell.cu:20-140 (reference gpu gate kernels,
//      driven with per-timestep host round trips of every cache).
//
// Layout: X [B,S,I], Y [B,S,H] ColMajor, i.e. [B*S, I] / [B*S, H] matrices
// whose row index is n + B*t, so timestep t is the row block [B*t, B*t+B).
// The reference computes x_t W_ih and every weight gradient inside its time
// loop.  Here the parts that do not depend on the recurrence run once over
// all B*S rows as large MFMA GEMMs:
//   forward : G = X W_ih (all steps), then the recurrence h_{t-1} W_hh with
//             the LSTM cell fused, all timesteps in one persistent launch
//             (lstm_fwd_persist_kernel) where the shape suits it, else one
//             launch per step (lstm_step_fwd_kernel)
//   backward: dh_t = dY_t + dG_{t+1} W_hh^T with the cell backward fused, in
//             one persistent launch (lstm_bwd_persist_kernel) or one launch
//             per step (lstm_step_bwd_kernel); afterwards dW_ih = X^T dG,
//             dW_hh = Y_{t-1}^T dG, db = colsum dG, dX = dG W_ih^T, each a
//             single GEMM over all B*S rows.
// The cell kernels fuse every elementwise gate computation of a step into one
// pass (one thread per (n, d); n fastest for coalescing) and evaluate the
// reference expressions in the reference's operation order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "mfma_kpack.hpp"

namespace cnhip {

int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who);
int column_sum(const float* in, float* out, int64_t rows, int64_t cols, int accumulate,
               hipStream_t st, const char* who);
int gemm_f32_core(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                  const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                  int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c,
                  int64_t batches, const float* bias, int epilogue, const float* aux_in,
                  float* aux_out, int64_t ld_aux, hipStream_t st, const char* who);
int fill_bytes(void* dst, int value, size_t bytes, hipStream_t stream, const char* where);
constexpr int EPI_TANH = 6;  // GEMM epilogue C = tanh(v) (gemm_f32.hip)

namespace {

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// Tile index of this block, XCD-aware: blocks are dealt to the 8 XCDs round
// robin (block b runs on XCD b % 8), so when the grid divides evenly, XCD x
// is given the contiguous tile range [x * n/8, (x+1) * n/8).  With tiles
// numbered sample-tile fastest, the blocks that share a unit tile's W_hh
// slice then sit on one XCD and read it through one L2, instead of each
// fetching it into a different XCD's L2.
__device__ __forceinline__ int64_t xcd_tile() {
  const int64_t n = gridDim.x, b = blockIdx.x;
  return n % 8 == 0 ? (b % 8) * (n / 8) + b / 8 : b;
}

// The LSTM cell arithmetic, evaluated as written with no fused multiply-adds
// (as the reference's Eigen expressions are on the CPU): every kernel that
// runs it -- first and last steps, the per-step launches and the persistent
// recurrence -- then produces the same bits, whatever contraction the
// compiler would have chosen in each context.
// c_t = f * c_{t-1} + i * g   (lstm.cpp:128-129)
__device__ __forceinline__ float lstm_cell_c(float fg, float cprev, float ig, float gg) {
#pragma clang fp contract(off)
  return fg * cprev + ig * gg;
}
// lstm.cpp:196-219: dc = dh o (1 - tanh(c)^2) + dc_{t+1} f_{t+1} (dc_in), the
// four gate-gradients, and dc * f handed to step t-1
__device__ __forceinline__ void lstm_cell_bwd(float ig, float fg, float gg, float og, float tc, float dh,
                                              float dc_in, float cprev, float& di, float& df, float& dgg,
                                              float& dout, float& dc_next) {
#pragma clang fp contract(off)
  const float dc = dh * og * (1.0f - tc * tc) + dc_in;
  di = dc * gg * ig * (1.0f - ig);
  df = dc * cprev * fg * (1.0f - fg);
  dgg = dc * ig * (1.0f - gg * gg);
  dout = dh * tc * og * (1.0f - og);
  dc_next = dc * fg;
}

// ---------------------------------------------------------------- LSTM cell
// Step t = 0 (h_0 = c_0 = 0, so no recurrent term): the rows of step 0 of
// gates hold x W_ih and are overwritten with the activations i, f, g, o
// (lstm.cpp:115-134); later steps run lstm_step_fwd_kernel.
__global__ void __launch_bounds__(256) lstm_cell_fwd0_kernel(float* __restrict__ gates,
                                                             const float* __restrict__ bias,
                                                             float* __restrict__ c,
                                                             float* __restrict__ tanh_c,
                                                             float* __restrict__ Y, int64_t B,
                                                             int64_t S, int64_t H) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n;
  float* g = gates + row;
  const float ig = sigm(g[BS * d] + bias[d]);
  const float fg = sigm(g[BS * (d + H)] + bias[d + H]);
  const float gg = tanhf(g[BS * (d + 2 * H)] + bias[d + 2 * H]);
  const float og = sigm(g[BS * (d + 3 * H)] + bias[d + 3 * H]);
  const float ct = lstm_cell_c(fg, 0.0f, ig, gg);
  const float tc = tanhf(ct);
  g[BS * d] = ig;
  g[BS * (d + H)] = fg;
  g[BS * (d + 2 * H)] = gg;
  g[BS * (d + 3 * H)] = og;
  c[row + BS * d] = ct;
  tanh_c[row + BS * d] = tc;
  Y[row + BS * d] = og * tc;
}

// One forward timestep t >= 1 in one launch: the recurrent GEMM
// h_{t-1} W_hh for a tile of 32 samples x (8 hidden units x 4 gates) and
// the cell update of those 256 (sample, unit) pairs in its epilogue.  The 4
// gate columns of a unit sit in one tile, so no other block's result is
// needed; the k-tile (64) is split over 4 wave groups whose partial sums are
// added in a fixed order.  256 blocks cover B = 128, H = 512.
using kp::f32x4;
using LstmFwdCfg = kp::Cfg<1, 1, 1, 1, 16, 4>;
constexpr int kLstmUnits = 8;  // hidden units per tile

template <class LstmCfg, bool FAST>
struct LstmFwdStage {
  using OA = kp::Operand<false, 32, LstmCfg::NT, LstmCfg::KT>;  // h(b, k) = Y[b + B(t-1) + BS k]
  using OB = kp::Operand<true, 32, LstmCfg::NT, LstmCfg::KT>;   // W_hh(k, col(n)), k-contiguous
  const float* A;  // Y + B*(t-1)
  const float* W;
  int64_t BS, B, H, b0, j0;
  f32x4 ra[2][OA::REGS], rb[2][OB::REGS];

  __device__ LstmFwdStage(const float* A_, const float* W_, int64_t BS_, int64_t B_, int64_t H_,
                          int64_t b0_, int64_t j0_)
      : A(A_), W(W_), BS(BS_), B(B_), H(H_), b0(b0_), j0(j0_) {}

  template <int S>
  __device__ __forceinline__ void load(int t) {
    const int64_t k0 = (int64_t)t * LstmCfg::KT;
    OA::template load<FAST>(A, BS, b0, k0, B, H, ra[S]);
#pragma unroll
    for (int p = 0; p < OB::PER; ++p) {
      int r, k;
      if (!OB::origin(p, r, k)) break;
      // tile column r = gate * 8 + unit: W_hh column gate*H + j0 + unit
      const int64_t j = j0 + r % kLstmUnits, gk = k0 + k;
      const float* col = W + H * ((r / kLstmUnits) * H + j);
      if (FAST) {
        rb[S][p] = *reinterpret_cast<const f32x4*>(col + gk);
      } else {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (j < H && gk + e < H) ? col[gk + e] : 0.f;
        rb[S][p] = v;
      }
    }
  }
  template <int S>
  __device__ __forceinline__ void store(float* buf) {
    OA::store(buf, ra[S]);
    OB::store(buf + OA::FLOATS, rb[S]);
  }
};

template <class LstmCfg, bool FAST>
__global__ void __launch_bounds__(LstmCfg::NT) lstm_step_fwd_kernel(
    float* __restrict__ gates, const float* __restrict__ bias, float* __restrict__ c,
    float* __restrict__ tanh_c, float* __restrict__ Y, const float* __restrict__ W_hh, int64_t B,
    int64_t S, int64_t H, int64_t t) {
  constexpr int FLOATS = 2 * kp::stage_floats<LstmFwdStage<LstmCfg, FAST>>();
  static_assert((LstmCfg::WGK - 1) * 1024 <= FLOATS, "reduce_wgk needs more LDS");
  __shared__ __align__(16) float lds[FLOATS];
  __shared__ float tile[32 * 33];  // [col][row], padded
  const int64_t BS = B * S;
  const int nbt = (int)((B + 31) / 32);
  const int64_t ti = xcd_tile();
  const int64_t b0 = (ti % nbt) * 32;
  const int64_t j0 = (ti / nbt) * kLstmUnits;
  kp::f32x16 acc[1][1];
  kp::zero_acc<LstmCfg>(acc);
  LstmFwdStage<LstmCfg, FAST> s(Y + B * (t - 1), W_hh, BS, B, H, b0, j0);
  kp::pipeline<LstmCfg>((int)((H + LstmCfg::KT - 1) / LstmCfg::KT), lds, s, acc);
  kp::reduce_wgk<LstmCfg>(lds, acc);
  kp::for_each_acc_run<LstmCfg>(acc, [&](int ml, int nl, const kp::f32x4& v) {
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[(ml + e) + 33 * nl] = v[e];
  });
  __syncthreads();
  // thread -> (sample, unit): the cell of lstm_cell_fwd0_kernel with the
  // recurrent term h W_hh taken from the tile
  static_assert(LstmCfg::NT >= 32 * kLstmUnits, "one thread per (sample, unit)");
  const int bl = threadIdx.x % 32, u = threadIdx.x / 32;
  if (u >= kLstmUnits) return;
  const int64_t n = b0 + bl, d = j0 + u;
  if (n >= B || d >= H) return;
  const int64_t row = n + B * t;
  float* g = gates + row;
  auto pre = [&](int gate, int64_t j) { return tile[bl + 33 * (gate * kLstmUnits + u)] + g[BS * j]; };
  const float ig = sigm(pre(0, d) + bias[d]);
  const float fg = sigm(pre(1, d + H) + bias[d + H]);
  const float gg = tanhf(pre(2, d + 2 * H) + bias[d + 2 * H]);
  const float og = sigm(pre(3, d + 3 * H) + bias[d + 3 * H]);
  const float cprev = c[row - B + BS * d];
  const float ct = lstm_cell_c(fg, cprev, ig, gg);
  const float tc = tanhf(ct);
  g[BS * d] = ig;
  g[BS * (d + H)] = fg;
  g[BS * (d + 2 * H)] = gg;
  g[BS * (d + 3 * H)] = og;
  c[row + BS * d] = ct;
  tanh_c[row + BS * d] = tc;
  Y[row + BS * d] = og * tc;
}

// ---------------------------------------------------------------- persistent recurrence
// All timesteps of the LSTM forward, or of its backward through time, in ONE
// launch.  A per-timestep launch (lstm_step_fwd/bwd_kernel) costs 8-9 us at
// B 128, H 512: launch ramp, reloading its W_hh slice and h_{t-1} through L2,
// then ~2 us of MFMA.  Here every block keeps its W_hh slice in registers for
// the whole sequence and the blocks hand each other the recurrent values
// directly, which measured ~3 us per step for the hand-over on MI355X.
//
// Tiling.  A tile is 16 samples x 16 hidden units, i.e. those units' 4 gate
// columns (64 columns of W_hh), computed by one block of 4 waves.  The blocks
// of one sample tile exchange values every step, so all of them run on ONE
// XCD and exchange through its L2.  The hardware deals a grid's blocks to
// the 8 XCDs round robin, but from a starting XCD that depends on earlier
// dispatches, so a block does not take its tile from blockIdx: it reads the
// XCD it runs on (XCC_ID) and takes the next slot i of that XCD's counter;
// XCD x then serves the sample tiles x, x + 8, x + 16, ... with H/16 blocks
// each (tile x + 8 (i / (H/16)), units 16 (i % (H/16))).  grid = 8 (H/16)
// ceil(nst/8) for nst = B/16 sample tiles gives every XCD as many blocks as
// it has slots; blocks with a slot past the last sample tile exit.
//
// Exchange.  A value handed to another block travels as one 64-bit word
// (float bits, stamp) in a double-buffered exchange area.  The stamp is the
// launch's epoch (16 bits, from a per-device counter) times 65536 plus the
// step, so words left by earlier launches never match: the area is zeroed
// only when its buffer is new, when the counter wraps, and before every
// launch recorded into a graph (whose replays all reuse epoch 0; a zeroed
// word carries stamp 0, which no step uses).  The fault word is tagged with
// the epoch the same way.  The XCD slot counters come in three sets: the
// launches of one buffer alternate between sets 0 and 1, and the first block
// placed on an XCD zeroes that XCD's counter of the other set for the next
// launch (the previous launch, which used it, has finished: persistent
// launches are ordered); a launch recorded into a graph uses set 2, zeroed
// with the rest of the area before each replay.  A block whose slot is
// beyond gridDim.x / 8 (an XCD dealt more blocks than that) raises the
// fault instead of taking a tile.  The
// writer stores the word; the reader invalidates its CU's L1 (buffer_inv
// sc0) and loads the words (nontemporal) until each carries the stamp it
// waits for.  A word is stored and loaded whole, so a value is never taken
// without its own stamp: a read that comes too early only waits longer.
// Slot t & 1 is rewritten at step t + 2 only after the writer has read every
// block's words of step t + 1, which each block wrote after its reads of
// step t were complete, so no word is overwritten while it may still be read.
//
// Every wait is bounded: after spin_limit polls a thread gives up and sets
// the launch's fault word (which every waiting thread checks while it polls,
// then exits), the device's optimizer guard (while it is set, every
// optimizer launch on the device leaves its tensors as they are, so the
// invalid outputs never reach the parameters) and the host-visible word,
// which the next recurrent call, graph replay or training-session sync point
// reports (cnhip_recurrence_fault_check).  A negative spin limit gives up at
// once (the tests of the fault path).
constexpr int kPt = 16;            // samples and hidden units per tile
constexpr int kPersistMaxH = 512;  // W_hh slice of H x 64 floats: H/4 registers per lane
typedef unsigned long long u64;

struct PersistSync {
  unsigned* fault;       // device word: fault_mark(epoch) once this launch faulted
  unsigned* slots;       // [8] this launch's per-XCD block counters (0 at its start)
  unsigned* slots_next;  // [8] the next launch's counters, zeroed here; null under capture
  unsigned* guard;       // the device's optimizer guard (set with the fault)
  unsigned* fault_host;  // pinned host word, or null
  long long spin_limit;
  unsigned epoch;        // 0 .. 65535; stamps are epoch << 16 | step
};

__device__ __forceinline__ unsigned fault_mark(unsigned epoch) { return 0x80000000u | epoch; }
__device__ __forceinline__ unsigned ex_stamp(const PersistSync& ps, int step) { return (ps.epoch << 16) | (unsigned)step; }

__device__ __forceinline__ void persist_fail(const PersistSync& ps) {
  __hip_atomic_store(ps.fault, fault_mark(ps.epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(ps.guard, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (ps.fault_host) __hip_atomic_store(ps.fault_host, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ bool persist_faulted(const PersistSync& ps) {
  return __hip_atomic_load(ps.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == fault_mark(ps.epoch);
}

__device__ __forceinline__ unsigned xcc_id() {
  return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 0xfu;  // hwreg(HW_REG_XCC_ID, 0, 4)
}

// The block's sample tile (>= nst when it has none) and unit tile, from the
// XCD it runs on; false (after raising the fault) when XCC_ID is not 0..7 or
// the XCD was dealt more than gridDim.x / 8 blocks.
__device__ __forceinline__ bool persist_place(const PersistSync& ps, int nut, int& st, int& ut, int* place) {
  if (threadIdx.x == 0) {
    const unsigned x = xcc_id();
    const unsigned i = x < 8u ? __hip_atomic_fetch_add(ps.slots + x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : ~0u;
    if (i == 0u && ps.slots_next)
      __hip_atomic_store(ps.slots_next + x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (i < gridDim.x / 8u) {
      place[0] = (int)x + 8 * ((int)i / nut);
      place[1] = (int)i % nut;
    } else {
      place[0] = -1;
      persist_fail(ps);
    }
  }
  __syncthreads();
  st = place[0];
  ut = place[1];
  return st >= 0;
}

__device__ __forceinline__ u64 ex_word(float v, unsigned stamp) {
  return ((u64)stamp << 32) | (u64)__float_as_uint(v);
}
__device__ __forceinline__ void ex_store(u64* p, u64 w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));  // two (value bits, stamp) words

// Two adjacent words (a, stamp), (b, stamp) at byte offset voff + soff of a
// buffer resource, in one 16-byte store (cache policy sc0, as ex_store).
// Each 8-byte word lies inside the one store, so a reader never sees a value
// without its stamp; the store covers half as many cache-line pieces per
// instruction as two 8-byte stores.
__device__ __forceinline__ void ex_store_pair(__amdgpu_buffer_rsrc_t rs, unsigned voff, unsigned soff, float a,
                                              float b, unsigned stamp) {
  const u32x4 v = {__float_as_uint(a), stamp, __float_as_uint(b), stamp};
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, voff, soff, 1);
}

// Raw buffer resource over the exchange area (32-bit byte offsets).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ex_rsrc(const u64* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<u64*>(base), 0, 0x7fffffff, 0x00020000);
}

// One thread: w[k] = the two adjacent words at byte offset voff + soff +
// k * STRIDE of the exchange area (k < N, one 16-byte load each), once every
// one of them carries `stamp`.  The k-dependent part of the offset is
// uniform, so it travels in the load's scalar offset.  ex_issue sends the
// first round of loads (after `sleep` s_sleep units: the words a thread
// has just written itself take about that long to reach the others); other
// work may run before ex_finish, which waits for them, checks the stamps and
// polls again for the words not yet written.  false: the launch faulted or
// this wait gave up.
template <int N, int STRIDE, int SLEEP = 0>
__device__ __forceinline__ void ex_issue(__amdgpu_buffer_rsrc_t rs, unsigned voff, unsigned soff, u32x4 (&w)[N]) {
  if constexpr (SLEEP > 0) __builtin_amdgcn_s_sleep(SLEEP);
  asm volatile("buffer_inv sc0" ::: "memory");
#pragma unroll
  for (int k = 0; k < N; ++k) w[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff + k * STRIDE, 2);
}

template <int N, int STRIDE>
__device__ __forceinline__ bool ex_finish(const PersistSync& ps, __amdgpu_buffer_rsrc_t rs, unsigned voff,
                                          unsigned soff, unsigned stamp, u32x4 (&w)[N]) {
  if (ps.spin_limit < 0) {
    persist_fail(ps);
    return false;
  }
  for (long long spins = 0;; ++spins) {
    bool all = true;
#pragma unroll
    for (int k = 0; k < N; ++k) all = all && w[k].y == stamp && w[k].w == stamp;
    if (all) return true;
    if ((spins & 63) == 63 && persist_faulted(ps)) return false;
    if (spins >= ps.spin_limit) {
      persist_fail(ps);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
    asm volatile("buffer_inv sc0" ::: "memory");
#pragma unroll
    for (int k = 0; k < N; ++k)
      if (w[k].y != stamp || w[k].w != stamp)
        w[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff + k * STRIDE, 2);
  }
}

struct LstmFwdPersistArgs {
  float* gates;
  const float* bias;
  float* c;
  float* tanh_c;
  float* Y;
  const float* W_hh;
  u64* ex;  // [2 slots][nst][H][16]: h_t of (unit, sample), stamp of step t + 1
  int B, S, nst;
  PersistSync sync;
  // input projection computed in the kernel (IT > 0): X [B*S, I], W_ih [I, 4H]
  const float* X;
  const float* W_ih;
  u64* stamps;  // measurement aid (null: off), see phase_stamp
};

// Measurement aid: thread 0 of each block records the constant-rate
// realtime counter (100 MHz) at the phase boundaries of every timestep, at
// stamps[((block) S + t) 8 + phase], block = sample tile * (H / 16) + unit
// tile, when the host has set a buffer (cnhip_lstm_phase_stamps).
__device__ __forceinline__ void phase_stamp(u64* stamps, int block, int S, int t, int phase) {
  if (stamps && threadIdx.x == 0) stamps[((int64_t)block * S + t) * 8 + phase] = __builtin_amdgcn_s_memrealtime();
}

// Forward, t = 0 .. S-1.  Per step t >= 1 a block waits for h_{t-1} of its
// 16 samples (all H units, from the H/16 blocks of its sample tile) and
// stages it in LDS; wave w computes the 16 x 16 recurrent pre-activations of
// its 4 units j0 + 4 w .. j0 + 4 w + 3 for all 4 gates (column c = gate 4 +
// unit; v_mfma_f32_16x16x4f32 over k ascending in blocks of 16: lane (q, r)
// supplies k = 16 kb + 4 q + e to MFMA (kb, e)).  A 4 x 4 transpose between
// lanes and accumulator registers then hands each lane the 4 gates of one
// cell (sample 4 q + r / 4, unit 4 w + r % 4), which it runs exactly as
// lstm_cell_fwd0_kernel / lstm_step_fwd_kernel do: it writes the caches and
// Y, and hands h_t on.  One barrier per step (the wait's vote, which also
// publishes the staged h_{t-1}): a wave rewrites the staging area only after
// it has seen every wave's h_t, which each wave stores after its last read
// of the area.
// s_sleep units before the forward's first poll of a step (~64 clocks each):
// sooner than that the other blocks' h_t cannot have arrived, and a poll of
// 64 KB per block that returns stale words only delays the next one.
constexpr int kFirstPollSleep = 12;

// The transpose of a 4 x 4 block between lane bits 2..3 and the register
// index: afterwards lane (g, j) (g = lane bits 2..3, j = bits 0..1) holds in
// register i what lane (i, j) held in register g.  Lanes 16 apart are
// independent.
__device__ __forceinline__ f32x4 xpose_lanes4(f32x4 v, int lane) {
  {  // lane bit 2 <-> register bit 0
    const bool l = (lane >> 2) & 1;
    const float ra = __shfl_xor(l ? v[0] : v[1], 4, 64), rb = __shfl_xor(l ? v[2] : v[3], 4, 64);
    if (l) {
      v[0] = ra;
      v[2] = rb;
    } else {
      v[1] = ra;
      v[3] = rb;
    }
  }
  {  // lane bit 3 <-> register bit 1
    const bool l = (lane >> 3) & 1;
    const float ra = __shfl_xor(l ? v[0] : v[2], 8, 64), rb = __shfl_xor(l ? v[1] : v[3], 8, 64);
    if (l) {
      v[0] = ra;
      v[1] = rb;
    } else {
      v[2] = ra;
      v[3] = rb;
    }
  }
  return v;
}

// IT > 0 (I = 64 IT inputs): the kernel also computes the input projection
// x_t W_ih of its 16 samples and 64 columns (the GEMM it replaces wrote all
// B S x 4H pre-activations only for this kernel to read them back).  Each
// block holds its W_ih slice in registers like the W_hh slice; x_t is staged
// in LDS (double-buffered, two 16-byte loads per thread) one step ahead and
// published by the step's vote; its 4 I/16 MFMAs per wave run while the
// block waits for h_{t-1}.  The x term has its own accumulator, so the gate
// is still (recurrent + x W_ih) + bias.
template <int H, int IT>
__global__ void __launch_bounds__(256) lstm_fwd_persist_kernel(LstmFwdPersistArgs a) {
  constexpr int NKB = H / 16;  // k-blocks; also the words per thread of h_{t-1}
  constexpr int NUT = H / kPt;
  constexpr bool FUSE = IT > 0;
  constexpr int I = 64 * IT, NKX = I / 16;  // inputs; their k-blocks
  __shared__ __align__(16) f32x4 hs[H / 4 * kPt];  // h_{t-1}: [k/4][sample], k..k+3
  __shared__ __align__(16) f32x4 xs[FUSE ? 2 * I / 4 * kPt : 1];  // x_t, [t & 1][i/4][sample]
  __shared__ int place[2];
  int st, ut;
  if (!persist_place(a.sync, NUT, st, ut, place)) return;
  if (st >= a.nst) return;
  const int B = a.B;
  const int64_t BS = (int64_t)B * a.S;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int b0 = st * kPt, j0 = ut * kPt;
  // W_hh(k, column (r / 4) H + j0 + 4 wave + r % 4) for k = 16 kb + 4 q + e
  f32x4 wv[NKB];
  {
    const float* wc = a.W_hh + (int64_t)H * ((int64_t)(r >> 2) * H + j0 + 4 * wave + (r & 3)) + 4 * q;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) wv[kb] = *reinterpret_cast<const f32x4*>(wc + 16 * kb);
  }
  // cell thread: sample m, unit u
  const int m = 4 * q + (r >> 2), u = 4 * wave + (r & 3);
  const int64_t n = b0 + m, d = j0 + u;
  const float bi = a.bias[d], bf = a.bias[d + H], bg = a.bias[d + 2 * H], bo = a.bias[d + 3 * H];
  u64* const ex = a.ex + (int64_t)st * H * kPt;
  const __amdgpu_buffer_rsrc_t rs = ex_rsrc(ex);
  const unsigned slot_bytes = (unsigned)a.nst * H * kPt * 8u;
  float xi = 0.f, xf = 0.f, xg = 0.f, xo = 0.f;  // this step's x W_ih terms
  if constexpr (!FUSE) {
    const float* g = a.gates + n;
    xi = g[BS * d];
    xf = g[BS * (d + H)];
    xg = g[BS * (d + 2 * H)];
    xo = g[BS * (d + 3 * H)];
  }
  // W_ih(i, column (r / 4) H + j0 + 4 wave + r % 4) for i = 16 kb + 4 q + e
  f32x4 wi[FUSE ? NKX : 1];
  // staging of x_t: thread tid loads samples b0 + 4 g .. + 3 of input i,
  // (i, g) = ((tid + 256 j) / 4, (tid + 256 j) % 4), j < IT
  f32x4 xr[FUSE ? IT : 1];
  float* xsf = reinterpret_cast<float*>(xs);
  auto x_issue = [&](int t) {
    if constexpr (FUSE) {
#pragma unroll
      for (int j = 0; j < IT; ++j) {
        const int e = tid + 256 * j, i = e >> 2, g = e & 3;
        xr[j] = *reinterpret_cast<const f32x4*>(a.X + b0 + 4 * g + (int64_t)B * t + BS * i);
      }
    }
  };
  auto x_write = [&](int buf) {
    if constexpr (FUSE) {
#pragma unroll
      for (int j = 0; j < IT; ++j) {
        const int e = tid + 256 * j, i = e >> 2, g = e & 3;
#pragma unroll
        for (int v = 0; v < 4; ++v) xsf[((buf * (I / 4) + (i >> 2)) * kPt + 4 * g + v) * 4 + (i & 3)] = xr[j][v];
      }
    }
  };
  // acc[i]: x_t W_ih of sample 4 q + i, this wave's column r
  auto x_mfma = [&](int buf) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (FUSE) {
#pragma unroll
      for (int kb = 0; kb < NKX; ++kb) {
        const f32x4 x4 = xs[(buf * (I / 4) + 4 * kb + q) * kPt + r];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x4[e], wi[kb][e], acc, 0, 0, 0);
      }
    }
    return acc;
  };
  if constexpr (FUSE) {
    const float* wc = a.W_ih + (int64_t)I * ((int64_t)(r >> 2) * H + j0 + 4 * wave + (r & 3)) + 4 * q;
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) wi[kb] = *reinterpret_cast<const f32x4*>(wc + 16 * kb);
    x_issue(0);
    x_write(0);
    if (a.S > 1) {
      x_issue(1);
      x_write(1);
    }
    __syncthreads();
  }
  float c_prev = 0.0f;
  float* hsf = reinterpret_cast<float*>(hs);
  const int sblk = st * NUT + ut;
  for (int t = 0; t < a.S; ++t) {
    const int64_t row = n + (int64_t)B * t;
    float ig, fg, gg, og;
    phase_stamp(a.stamps, sblk, a.S, t, 0);  // step start
    if (t == 0) {  // h_0 = c_0 = 0 (lstm_cell_fwd0_kernel's arithmetic)
      if constexpr (FUSE) {
        const f32x4 ax = xpose_lanes4(x_mfma(0), lane);
        xi = ax[0];
        xf = ax[1];
        xg = ax[2];
        xo = ax[3];
      }
      ig = sigm(xi + bi);
      fg = sigm(xf + bf);
      gg = tanhf(xg + bg);
      og = sigm(xo + bo);
    } else {
      // h_{t-1}: word (k, s) at [slot (t-1) & 1][k][s]; this thread takes
      // s = 2 (tid % 8) and the next, k = tid / 8 + 32 j (byte offset tid 16
      // + j 4096)
      u32x4 w[NKB / 2];
      const unsigned voff = (unsigned)tid * 16u, soff = ((t - 1) & 1) * slot_bytes;
      // x_{t+1} staged while waiting: its loads go first, written to the
      // other buffer (last read at step t - 1, before that step's vote)
      if (t + 1 < a.S) x_issue(t + 1);
      ex_issue<NKB / 2, 256 * 16, kFirstPollSleep>(rs, voff, soff, w);
      const f32x4 axr = x_mfma(t & 1);
      const bool ok = ex_finish<NKB / 2, 256 * 16>(a.sync, rs, voff, soff, ex_stamp(a.sync, t), w);
      phase_stamp(a.stamps, sblk, a.S, t, 1);  // h_{t-1} arrived
#pragma unroll
      for (int j = 0; j < NKB / 2; ++j) {
        const int k = (tid >> 3) + 32 * j, s2 = 2 * (tid & 7);
        hsf[((k >> 2) * kPt + s2) * 4 + (k & 3)] = __uint_as_float(w[j].x);
        hsf[((k >> 2) * kPt + s2 + 1) * 4 + (k & 3)] = __uint_as_float(w[j].z);
      }
      if (t + 1 < a.S) x_write((t + 1) & 1);
      if (__syncthreads_or(!ok)) return;
      phase_stamp(a.stamps, sblk, a.S, t, 2);  // the block's vote
      if constexpr (FUSE) {
        const f32x4 ax = xpose_lanes4(axr, lane);
        xi = ax[0];
        xf = ax[1];
        xg = ax[2];
        xo = ax[3];
      }
      // two accumulation chains (even and odd k-blocks), added at the end:
      // one chain of 4 NKB dependent MFMAs leaves the single wave of each
      // SIMD waiting on each result
      f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < NKB; kb += 2) {
        const f32x4 h4 = hs[(4 * kb + q) * kPt + r];
        const f32x4 h5 = hs[(4 * (kb + 1) + q) * kPt + r];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(h4[e], wv[kb][e], acc, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(h5[e], wv[kb + 1][e], acc1, 0, 0, 0);
        }
      }
      acc += acc1;
      // acc[i]: sample 4 q + i, gate r / 4, unit 4 wave + r % 4; after the
      // transpose acc[g]: gate g of this lane's cell
      acc = xpose_lanes4(acc, lane);
      // as lstm_step_fwd_kernel: (recurrent + x W_ih) + bias
      ig = sigm((acc[0] + xi) + bi);
      fg = sigm((acc[1] + xf) + bf);
      gg = tanhf((acc[2] + xg) + bg);
      og = sigm((acc[3] + xo) + bo);
    }
    phase_stamp(a.stamps, sblk, a.S, t, 3);  // recurrent product and gates
    const float ct = lstm_cell_c(fg, c_prev, ig, gg);
    const float tc = tanhf(ct);
    const float h = og * tc;
    if (t + 1 < a.S)
      ex_store(ex + (int64_t)(t & 1) * (slot_bytes / 8) + (int64_t)d * kPt + m, ex_word(h, ex_stamp(a.sync, t + 1)));
    float* g = a.gates + row;
    g[BS * d] = ig;
    g[BS * (d + H)] = fg;
    g[BS * (d + 2 * H)] = gg;
    g[BS * (d + 3 * H)] = og;
    a.c[row + BS * d] = ct;
    a.tanh_c[row + BS * d] = tc;
    a.Y[row + BS * d] = h;
    c_prev = ct;
    phase_stamp(a.stamps, sblk, a.S, t, 4);  // cell update, h_t handed on, caches written
    if (!FUSE && t + 1 < a.S) {
      const float* gn = g + B;
      xi = gn[BS * d];
      xf = gn[BS * (d + H)];
      xg = gn[BS * (d + 2 * H)];
      xo = gn[BS * (d + 3 * H)];
    }
  }
}

struct LstmBwdPersistArgs {
  const float* gates;
  const float* c;
  const float* tanh_c;
  const float* dY;
  const float* W_hh;
  float* dG;
  u64* ex;  // [2 slots][nst][H/16 writers][H][16]: partial dG_t W_hh^T, stamp of step t + 1
  int B, S, nst;
  PersistSync sync;
  // fused weight gradients (IT > 0): X [B*S, I], Y [B*S, H] and the
  // per-sample-tile partials [nst][H*4H | I*4H | 4H] (dW_hh, dW_ih, db)
  const float* X;
  const float* Y;
  float* part;
  int I;
  int dy_last;  // dY is [B, H], the gradient of the last step only (0 at the others)
  u64* stamps;  // measurement aid (null: off), see phase_stamp
};

// Backward through time, t = S-1 .. 0.  The recurrent term dG_{t+1} W_hh^T
// is split by columns of W_hh: the block that computed dG_t for its 16
// units (64 columns) multiplies it by its W_hh columns for ALL H units
// (16 x H partial products, K = 64: wave w takes H/64 output tiles, MFMA
// (kb, e) over local column 16 kb + 4 q + e, i.e. gate kb), and hands them
// on; at step t-1 each block adds, for its units, the H/16 partials of its
// sample tile in block order.  Each block only multiplies its own dG, and
// exchanges 16 x 16 words per partner per step.  The cell backward is
// lstm_cell_bwd_last_kernel's at t = S-1 and lstm_step_bwd_kernel's after.
//
// IT > 0 (I = 64 IT inputs) also accumulates the block's share of the weight
// gradients while it waits for the next step's partials: dW_hh += h_{t-1}^T
// dG_t (t >= 1) and dW_ih += x_t^T dG_t over its 16 samples and its 64
// columns (MFMA tiles of 16 k x 16 columns over the 16 samples; wave w takes
// the k-tiles w H/64 .. and w IT ..), and db += dG_t per cell thread.  The
// first poll's loads of step t's wait are sent before step t+1's
// accumulation, so their latency and the MFMAs overlap.  The sums run over
// t descending, then over the block's samples; at the end the block writes
// its partials, which lstm_dw_reduce_kernel adds over the sample tiles in
// order.  (The separate GEMMs these replace sum over all B S rows instead.)
template <int H, int IT>
__global__ void __launch_bounds__(256) lstm_bwd_persist_kernel(LstmBwdPersistArgs a) {
  constexpr int NUT = H / kPt;  // blocks (writers) per sample tile
  constexpr int TPW = H / 64;   // output tiles of 16 units per wave; dW_hh k-tiles per wave
  constexpr bool FUSE = IT > 0;
  // the W_hh slice (H 64 floats) moves to LDS when the weight-gradient
  // accumulators would not fit beside it in registers
  constexpr bool WLDS = FUSE && H > 256;
  __shared__ __align__(16) f32x4 dgs[64 / 4 * kPt];  // dG_t of the 64 columns: [c/4][sample]
  __shared__ __align__(16) f32x4 wl[WLDS ? H * 64 / 4 : 1];
  __shared__ float dbr[FUSE ? 64 * kPt : 1];  // db reduction: [column][sample]
  __shared__ float red[2][kPt][kPt];          // half sums of the partials: [half][unit][sample]
  __shared__ int place[2];
  int st, ut;
  if (!persist_place(a.sync, NUT, st, ut, place)) return;
  if (st >= a.nst) return;
  const int B = a.B, S = a.S;
  const int64_t BS = (int64_t)B * S;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int b0 = st * kPt, j0 = ut * kPt;
  // W_hh(unit 16 (wave TPW + tt) + r, column kb H + j0 + 4 q + e), in
  // registers, or (WLDS) in LDS at wl[((wave TPW + tt) 4 + kb) 64 + lane],
  // read back by the lane that wrote it
  f32x4 wv[WLDS ? 1 : TPW][4];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 w4;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w4[e] = a.W_hh[(16 * (wave * TPW + tt) + r) + (int64_t)H * ((int64_t)kb * H + j0 + 4 * q + e)];
      if constexpr (WLDS)
        wl[((wave * TPW + tt) * 4 + kb) * 64 + lane] = w4;
      else
        wv[tt][kb] = w4;
    }
  // cell thread: sample m, unit u
  const int m = tid & 15, u = tid >> 4;
  const int64_t n = b0 + m, d = j0 + u;
  u64* const ex = a.ex + (int64_t)st * NUT * H * kPt;  // + writer * H * 16
  const __amdgpu_buffer_rsrc_t rs = ex_rsrc(ex);
  const unsigned slot_bytes = (unsigned)a.nst * NUT * H * kPt * 8u;
  float* dgsf = reinterpret_cast<float*>(dgs);
  // weight-gradient accumulators: [k-tile][column tile = gate]
  f32x4 ahh[FUSE ? TPW : 1][4], aih[FUSE ? IT : 1][4];
  float dbs[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (FUSE) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
      for (int kt = 0; kt < TPW; ++kt) ahh[kt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int it = 0; it < IT; ++it) aih[it][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // Step p's accumulation, dgs holding dG_p.  MFMA (ks) of tile (kt, ct)
  // sums over the samples 4 q + ks of lane group q (any order of the 16
  // samples gives the same sum up to rounding): row operands h_{p-1}(sample,
  // k) in hA and x_p(sample, i) in xA with k, i = 16 (tile) + r, one 16-byte
  // load of 4 samples each; column operand dG_p(sample, column 16 ct + r)
  // from dgs.  Tile by tile, each row operand is reloaded with step p-1's
  // rows right after its last MFMA: the loads issue while the MFMAs run (16
  // rows apart each, they are slow to issue) and have a whole step to land.
  f32x4 hA[FUSE ? TPW : 1], xA[FUSE ? IT : 1];
  const int64_t smp = b0 + 4 * q;
  auto load_h = [&](int kt, int p) {  // h_{p-1}, zero for p = 0
    hA[kt] = p > 0 ? *reinterpret_cast<const f32x4*>(a.Y + smp + (int64_t)B * (p - 1) +
                                                      BS * (16 * (wave * TPW + kt) + r))
                   : f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto load_x = [&](int it, int p) {  // x_p
    xA[it] = *reinterpret_cast<const f32x4*>(a.X + smp + (int64_t)B * p + BS * (16 * (wave * IT + it) + r));
  };
  auto dw_step = [&](int p) {
    if constexpr (FUSE) {
      float bv[4][4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int col = 16 * ct + r;
        const f32x4* gp = reinterpret_cast<const f32x4*>(dgsf + ((col >> 2) * kPt + 4 * q) * 4);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) bv[ct][ks] = reinterpret_cast<const float*>(gp + ks)[col & 3];
      }
#pragma unroll
      for (int it = 0; it < IT; ++it) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            aih[it][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(xA[it][ks], bv[ct][ks], aih[it][ct], 0, 0, 0);
        if (p > 0) load_x(it, p - 1);
      }
#pragma unroll
      for (int kt = 0; kt < TPW; ++kt) {
        if (p > 0) {
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
              ahh[kt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(hA[kt][ks], bv[ct][ks], ahh[kt][ct], 0, 0, 0);
          load_h(kt, p - 1);
        }
      }
    }
  };
  // operands of step t (no dependence on the recurrence), loaded a step ahead
  float ig, fg, gg, og, tc, cprev, dy;
  auto load_step = [&](int t) {
    const int64_t row = n + (int64_t)B * t;
    ig = a.gates[row + BS * d];
    fg = a.gates[row + BS * (d + H)];
    gg = a.gates[row + BS * (d + 2 * H)];
    og = a.gates[row + BS * (d + 3 * H)];
    tc = a.tanh_c[row + BS * d];
    cprev = t > 0 ? a.c[row - B + BS * d] : 0.0f;
    dy = !a.dy_last ? a.dY[row + BS * d] : t == S - 1 ? a.dY[n + (int64_t)B * d] : 0.0f;
  };
  load_step(S - 1);
  if constexpr (FUSE) {
#pragma unroll
    for (int kt = 0; kt < TPW; ++kt) load_h(kt, S - 1);
#pragma unroll
    for (int it = 0; it < IT; ++it) load_x(it, S - 1);
  }
  float dc_next = 0.0f;
  const int sblk = st * NUT + ut;
  for (int t = S - 1; t >= 0; --t) {
    const int64_t row = n + (int64_t)B * t;
    float dh = dy;
    phase_stamp(a.stamps, sblk, S, t, 0);  // step start
    if (t < S - 1) {
      // partials of step t+1: writer w's word (unit, sample) at [slot (t+1)
      // & 1][w][unit][sample], stamp of step t + 2.  Thread (half, u2, p2) loads the
      // words (j0 + u2, 2 p2) and (j0 + u2, 2 p2 + 1) of writers half NUT/2
      // .. half NUT/2 + NUT/2 - 1 and sums them in writer order; the cell
      // thread adds its two half sums.
      const int half = tid >> 7, u2 = (tid >> 3) & 15, p2 = tid & 7;
      u32x4 w[NUT / 2];
      const unsigned voff = (unsigned)((j0 + u2) * kPt + 2 * p2) * 8u;
      const unsigned soff = ((t + 1) & 1) * slot_bytes + (unsigned)half * (NUT / 2) * H * kPt * 8u;
      ex_issue<NUT / 2, H * kPt * 8>(rs, voff, soff, w);
      dw_step(t + 1);  // dgs still holds dG_{t+1}
      phase_stamp(a.stamps, sblk, S, t, 1);  // weight-gradient MFMAs of step t + 1
      const bool ok = ex_finish<NUT / 2, H * kPt * 8>(a.sync, rs, voff, soff, ex_stamp(a.sync, t + 2), w);
      phase_stamp(a.stamps, sblk, S, t, 2);  // partials of step t + 1 arrived
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int k = 0; k < NUT / 2; ++k) {
        s0 += __uint_as_float(w[k].x);
        s1 += __uint_as_float(w[k].z);
      }
      red[half][u2][2 * p2] = s0;
      red[half][u2][2 * p2 + 1] = s1;
      if (__syncthreads_or(!ok)) return;
      phase_stamp(a.stamps, sblk, S, t, 3);  // the block's vote
      dh = dy + (red[0][u][m] + red[1][u][m]);
    }
    float di, df, dgg, dout;
    lstm_cell_bwd(ig, fg, gg, og, tc, dh, t == S - 1 ? 0.0f : dc_next, cprev, di, df, dgg, dout, dc_next);
    a.dG[row + BS * d] = di;
    a.dG[row + BS * (d + H)] = df;
    a.dG[row + BS * (d + 2 * H)] = dgg;
    a.dG[row + BS * (d + 3 * H)] = dout;
    if constexpr (FUSE) {
      dbs[0] += di;
      dbs[1] += df;
      dbs[2] += dgg;
      dbs[3] += dout;
    }
    if (t == 0 && !FUSE) break;
    // local column gate * 16 + u at dgs[(col / 4) * 16 + m][col % 4]
    dgsf[(((0 * 16 + u) >> 2) * kPt + m) * 4 + (u & 3)] = di;
    dgsf[(((1 * 16 + u) >> 2) * kPt + m) * 4 + (u & 3)] = df;
    dgsf[(((2 * 16 + u) >> 2) * kPt + m) * 4 + (u & 3)] = dgg;
    dgsf[(((3 * 16 + u) >> 2) * kPt + m) * 4 + (u & 3)] = dout;
    if (t > 0) load_step(t - 1);
    __syncthreads();
    phase_stamp(a.stamps, sblk, S, t, 4);  // cell backward, dG_t staged
    if (t == 0) break;
    const unsigned so = (unsigned)(t & 1) * slot_bytes + (unsigned)ut * H * kPt * 8u;
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const f32x4 g4 = dgs[(4 * kb + q) * kPt + r];
        f32x4 w4;
        if constexpr (WLDS)
          w4 = wl[((wave * TPW + tt) * 4 + kb) * 64 + lane];
        else
          w4 = wv[tt][kb];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(g4[e], w4[e], acc, 0, 0, 0);
      }
      // acc[i]: sample 4 q + i, unit 16 (wave TPW + tt) + r, words
      // [slot t & 1][writer ut][unit][sample], the lane's four adjacent
      const unsigned vo = (unsigned)((16 * (wave * TPW + tt) + r) * kPt + 4 * q) * 8u;
      ex_store_pair(rs, vo, so, acc[0], acc[1], ex_stamp(a.sync, t + 1));
      ex_store_pair(rs, vo + 16, so, acc[2], acc[3], ex_stamp(a.sync, t + 1));
    }
    phase_stamp(a.stamps, sblk, S, t, 5);  // recurrent partials handed on
    // dgs is rewritten at the next step only after the wait's block-wide vote
  }
  if constexpr (FUSE) {
    // step 0's accumulation (dgs holds dG_0, made visible by the barrier above)
    dw_step(0);
    // the block's partials: acc[i] of tile (kt, ct) is row 16 kt' + 4 q + i,
    // column ct H + j0 + r of dW (kt' = the wave's k-tile)
    const int64_t G = 4 * (int64_t)H, I = a.I;
    float* phh = a.part + (int64_t)st * (H * G + I * G + G);
    float* pih = phh + H * G;
    float* pb = pih + I * G;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int64_t col = (int64_t)ct * H + j0 + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int kt = 0; kt < TPW; ++kt) phh[(16 * (wave * TPW + kt) + 4 * q + i) + H * col] = ahh[kt][ct][i];
#pragma unroll
        for (int it = 0; it < IT; ++it) pih[(16 * (wave * IT + it) + 4 * q + i) + I * col] = aih[it][ct][i];
      }
    }
    // db: the 16 samples' running sums of each column added in sample order
#pragma unroll
    for (int g = 0; g < 4; ++g) dbr[(16 * g + u) * kPt + m] = dbs[g];
    __syncthreads();
    if (tid < 64) {
      float v = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < kPt; ++s2) v += dbr[tid * kPt + s2];
      pb[(int64_t)(tid >> 4) * H + j0 + (tid & 15)] = v;
    }
  }
}

// out_k[e] = sum over the sample tiles s = 0 .. nst-1, in order, of
// part[s][e] (the persistent backward's weight-gradient partials), for the
// concatenation e of dW_hh | dW_ih | db into their three buffers.
__global__ void __launch_bounds__(256) lstm_dw_reduce_kernel(const float* __restrict__ part, int nst, int64_t n_hh,
                                                             int64_t n_ih, int64_t n_b, float* __restrict__ gW_hh,
                                                             float* __restrict__ gW_ih, float* __restrict__ gb) {
  const int64_t total = n_hh + n_ih + n_b;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    float v = 0.f;
    for (int s2 = 0; s2 < nst; ++s2) v += part[(int64_t)s2 * total + e];
    if (e < n_hh) gW_hh[e] = v;
    else if (e < n_hh + n_ih) gW_ih[e - n_hh] = v;
    else gb[e - n_hh - n_ih] = v;
  }
}

// lstm.cpp:184-219, 247-249, the last step t = S-1: dh = dY (no later step)
// and dc starts from 0; dc_buf [B, H] (ld B) receives dc * f for step t-1.
// Earlier steps run lstm_step_bwd_kernel.
__global__ void __launch_bounds__(256) lstm_cell_bwd_last_kernel(
    const float* __restrict__ gates, const float* __restrict__ c, const float* __restrict__ tanh_c,
    const float* __restrict__ dY, float* __restrict__ dc_buf, float* __restrict__ dG, int64_t B,
    int64_t S, int64_t H) {
  const int64_t BS = B * S, t = S - 1;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float ig = gates[row + BS * d], fg = gates[row + BS * (d + H)];
  const float gg = gates[row + BS * (d + 2 * H)], og = gates[row + BS * (d + 3 * H)];
  const float tc = tanh_c[row + BS * d];
  const float dh = dY[row + BS * d];
  const float cprev = t > 0 ? c[row - B + BS * d] : 0.0f;
  float di, df, dgg, dout, dcn;
  lstm_cell_bwd(ig, fg, gg, og, tc, dh, 0.0f, cprev, di, df, dgg, dout, dcn);
  dG[row + BS * d] = di;
  dG[row + BS * (d + H)] = df;
  dG[row + BS * (d + 2 * H)] = dgg;
  dG[row + BS * (d + 3 * H)] = dout;
  dc_buf[e] = dcn;
}

// One backward timestep t <= S-2 in one launch: dh_t = dY_t + dG_{t+1} W_hh^T
// for a tile of 16 samples x 16 hidden units (K = 4H split over the wave
// groups of the block, added in a fixed order), then lstm_cell_bwd_last_kernel's
// arithmetic for those 256 (sample, unit) pairs in the epilogue.  16 x 16
// tiles give 256 blocks at B = 128, H = 512.
using LstmBwdCfgDefault = kp::Cfg16<1, 1, 1, 1, 32, 8>;  // fastest of a measured sweep

template <class LstmBwdCfg, bool FAST>
struct LstmBwdStage {
  using OA = kp::Operand<false, 16, LstmBwdCfg::NT, LstmBwdCfg::KT>;  // dG(b, k) = dG[b + BS k]
  using OB = kp::Operand<false, 16, LstmBwdCfg::NT, LstmBwdCfg::KT>;  // W_hh^T(j, k) = W_hh[j + H k]
  const float* A;  // dG + B*(t+1)
  const float* W;
  int64_t BS, B, H, b0, j0;
  f32x4 ra[2][OA::REGS], rb[2][OB::REGS];

  __device__ LstmBwdStage(const float* A_, const float* W_, int64_t BS_, int64_t B_, int64_t H_,
                          int64_t b0_, int64_t j0_)
      : A(A_), W(W_), BS(BS_), B(B_), H(H_), b0(b0_), j0(j0_) {}

  template <int S>
  __device__ __forceinline__ void load(int t) {
    const int64_t k0 = (int64_t)t * LstmBwdCfg::KT;
    OA::template load<FAST>(A, BS, b0, k0, B, 4 * H, ra[S]);
    OB::template load<FAST>(W, H, j0, k0, H, 4 * H, rb[S]);
  }
  template <int S>
  __device__ __forceinline__ void store(float* buf) {
    OA::store(buf, ra[S]);
    OB::store(buf + OA::FLOATS, rb[S]);
  }
};

template <class LstmBwdCfg, bool FAST>
__global__ void __launch_bounds__(LstmBwdCfg::NT) lstm_step_bwd_kernel(
    const float* __restrict__ gates, const float* __restrict__ c, const float* __restrict__ tanh_c,
    const float* __restrict__ dY, const float* __restrict__ W_hh, float* __restrict__ dc_buf,
    float* __restrict__ dG, int64_t B, int64_t S, int64_t H, int64_t t) {
  constexpr int FLOATS = 2 * kp::stage_floats<LstmBwdStage<LstmBwdCfg, FAST>>();
  static_assert((LstmBwdCfg::WGK - 1) * 4 * 64 <= FLOATS, "reduce_wgk16 needs more LDS");
  __shared__ __align__(16) float lds[FLOATS];
  __shared__ float tile[16 * 17];  // [unit][sample], padded
  const int64_t BS = B * S;
  const int nbt = (int)((B + 15) / 16);
  const int64_t ti = xcd_tile();
  const int64_t b0 = (ti % nbt) * 16;
  const int64_t j0 = (ti / nbt) * 16;
  f32x4 acc[1][1];
  kp::zero_acc16<LstmBwdCfg>(acc);
  LstmBwdStage<LstmBwdCfg, FAST> s(dG + B * (t + 1), W_hh, BS, B, H, b0, j0);
  kp::pipeline<LstmBwdCfg>((int)((4 * H + LstmBwdCfg::KT - 1) / LstmBwdCfg::KT), lds, s, acc);
  kp::reduce_wgk16<LstmBwdCfg>(lds, acc);
  kp::for_each_acc_run16<LstmBwdCfg>(acc, [&](int ml, int nl, const f32x4& v) {
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[(ml + e) + 17 * nl] = v[e];
  });
  __syncthreads();
  static_assert(LstmBwdCfg::NT >= 256, "one thread per (sample, unit)");
  const int bl = threadIdx.x % 16, jl = threadIdx.x / 16;
  if (jl >= 16) return;
  const int64_t n = b0 + bl, d = j0 + jl;
  if (n >= B || d >= H) return;
  const int64_t e = n + B * d, row = n + B * t;
  const float ig = gates[row + BS * d], fg = gates[row + BS * (d + H)];
  const float gg = gates[row + BS * (d + 2 * H)], og = gates[row + BS * (d + 3 * H)];
  const float tc = tanh_c[row + BS * d];
  const float dh = dY[row + BS * d] + tile[bl + 17 * jl];
  const float cprev = t > 0 ? c[row - B + BS * d] : 0.0f;
  float di, df, dgg, dout, dcn;
  lstm_cell_bwd(ig, fg, gg, og, tc, dh, dc_buf[e], cprev, di, df, dgg, dout, dcn);
  dG[row + BS * d] = di;
  dG[row + BS * (d + H)] = df;
  dG[row + BS * (d + 2 * H)] = dgg;
  dG[row + BS * (d + 3 * H)] = dout;
  dc_buf[e] = dcn;
}

// ---------------------------------------------------------------- GRU cells
// gru.cpp:102-109: z, r from x W_ih + h W_hh (+ b); rh = r * h_prev.
// hz: [B, 2H] dense = h_{t-1} W_hh[:, 0:2H] (ignored at t = 0, where h = 0).
__global__ void __launch_bounds__(256) gru_zr_kernel(float* __restrict__ gates,
                                                     const float* __restrict__ hz,
                                                     const float* __restrict__ bias,
                                                     const float* __restrict__ Y,
                                                     float* __restrict__ rh, int64_t B, int64_t S,
                                                     int64_t H, int64_t t) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float hzz = t > 0 ? hz[n + B * d] : 0.0f;
  const float hzr = t > 0 ? hz[n + B * (d + H)] : 0.0f;
  const float zg = sigm((gates[row + BS * d] + hzz) + bias[d]);
  const float rg = sigm((gates[row + BS * (d + H)] + hzr) + bias[d + H]);
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  gates[row + BS * d] = zg;
  gates[row + BS * (d + H)] = rg;
  rh[row + BS * d] = rg * hp;
}

// gru.cpp:120-133: n = tanh(x W_in + rh W_hn + b_n), h = (1-z) n + z h_prev.
__global__ void __launch_bounds__(256) gru_n_kernel(float* __restrict__ gates,
                                                    const float* __restrict__ proj,
                                                    const float* __restrict__ bias,
                                                    float* __restrict__ Y, int64_t B, int64_t S,
                                                    int64_t H, int64_t t) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float zg = gates[row + BS * d];
  const float nc = tanhf((gates[row + BS * (d + 2 * H)] + proj[n + B * d]) + bias[d + 2 * H]);
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  gates[row + BS * (d + 2 * H)] = nc;
  Y[row + BS * d] = (1.0f - zg) * nc + zg * hp;
}

// gru.cpp:188-209.  dh: [B,H] dense, holds dh_next on entry (ignored when
// first) and dh_prev's direct part (dh * z) on exit.
__global__ void __launch_bounds__(256) gru_bwd_a_kernel(const float* __restrict__ gates,
                                                        const float* __restrict__ Y,
                                                        const float* __restrict__ dY,
                                                        float* __restrict__ dh,
                                                        float* __restrict__ dG, int64_t B,
                                                        int64_t S, int64_t H, int64_t t,
                                                        int first) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float zg = gates[row + BS * d], nc = gates[row + BS * (d + 2 * H)];
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  const float dhv = dY[row + BS * d] + (first ? 0.0f : dh[e]);
  const float dn = dhv * (1.0f - zg);
  const float dz = dhv * (hp - nc);
  dG[row + BS * d] = dz * zg * (1.0f - zg);
  dG[row + BS * (d + 2 * H)] = dn * (1.0f - nc * nc);
  dh[e] = dhv * zg;
}

// gru.cpp:214-225: with d_rh = dn_raw W_hn^T, dr_raw and dh_prev += d_rh * r.
__global__ void __launch_bounds__(256) gru_bwd_b_kernel(const float* __restrict__ gates,
                                                        const float* __restrict__ Y,
                                                        const float* __restrict__ d_rh,
                                                        float* __restrict__ dh,
                                                        float* __restrict__ dG, int64_t B,
                                                        int64_t S, int64_t H, int64_t t) {
  const int64_t BS = B * S;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, row = n + B * t;
  const float rg = gates[row + BS * (d + H)];
  const float hp = t > 0 ? Y[row - B + BS * d] : 0.0f;
  const float dr = d_rh[e] * hp;
  dG[row + BS * (d + H)] = dr * rg * (1.0f - rg);
  dh[e] += d_rh[e] * rg;
}

// out[B, D] = Y[:, t, :]  /  Y = 0 except Y[:, t, :] = in
__global__ void __launch_bounds__(256) seq_select_kernel(const float* __restrict__ Y,
                                                         float* __restrict__ out, int64_t B,
                                                         int64_t S, int64_t D, int64_t t) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * D) return;
  const int64_t n = e % B, d = e / B;
  out[e] = Y[n + B * t + B * S * d];
}

__global__ void __launch_bounds__(256) seq_scatter_kernel(const float* __restrict__ in,
                                                          float* __restrict__ Y, int64_t B,
                                                          int64_t S, int64_t D, int64_t t) {
  const int64_t total = B * S * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i % B, s = (i / B) % S, d = i / (B * S);
    Y[i] = s == t ? in[n + B * d] : 0.0f;
  }
}

unsigned cell_grid(int64_t B, int64_t H) { return (unsigned)((B * H + 255) / 256); }

// ---------------------------------------------------------------- Elman RNN
// rnn.cpp:48-100: step 0 has no recurrent term (h_0 = 0): its rows of Y hold
// x_0 W_ih and become tanh(x_0 W_ih + b).
__global__ void __launch_bounds__(256) rnn_step0_kernel(float* __restrict__ Y, const float* __restrict__ b,
                                                        int64_t B, int64_t BS, int64_t H) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B;
  float* y = Y + n + BS * d;
  *y = tanhf(*y + b[d]);
}
// rnn.cpp:118-131: dtanh_t = (dY_t + dh_next) * (1 - h_t^2) into dT's rows of
// step t (dh_next == nullptr at the last step: dh_next is zero there).
__global__ void __launch_bounds__(256) rnn_bwd_cell_kernel(const float* __restrict__ dY,
                                                           const float* __restrict__ Y,
                                                           const float* __restrict__ dh_next,
                                                           float* __restrict__ dT, int64_t B, int64_t BS,
                                                           int64_t H, int64_t t) {
#pragma clang fp contract(off)
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= B * H) return;
  const int64_t n = e % B, d = e / B, i = n + B * t + BS * d;
  const float dh = dh_next ? dY[i] + dh_next[n + B * d] : dY[i];
  const float h = Y[i];
  dT[i] = dh * (1.0f - h * h);
}

// Per-step launches of the fused LSTM kernels for steps t = 1 .. S-1
// (forward) and t = S-2 .. 0 (backward), each timed like a GEMM (2*B*4H*H
// flops) for the per-launch roofline.
template <class Cfg>
int lstm_fwd_steps(float* gates, const float* b, float* c, float* tanh_c, float* Y,
                   const float* W_hh, int64_t B, int64_t S, int64_t H, hipStream_t st,
                   const char* who) {
  const int64_t nbt = (B + 31) / 32, nbu = (H + kLstmUnits - 1) / kLstmUnits;
  CNHIP_REQUIRE(nbt * nbu < ((int64_t)1 << 31), "%s: too many tiles", who);
  // FAST: full tiles, whole k-tiles, 16-byte aligned rows of Y and W_hh
  const bool fast = B % 32 == 0 && H % Cfg::KT == 0 && H % kLstmUnits == 0 && (B * S) % 4 == 0 &&
                    aligned16(Y) && aligned16(W_hh);
  const auto kern = fast ? &lstm_step_fwd_kernel<Cfg, true> : &lstm_step_fwd_kernel<Cfg, false>;
  for (int64_t t = 1; t < S; ++t) {
    TimingRec* rec = timing_slot(2.0 * B * 4 * H * H);
    if (rec) (void)hipEventRecord(rec->start, st);
    hipLaunchKernelGGL(kern, dim3((unsigned)(nbt * nbu)), dim3(Cfg::NT), 0, st, gates, b, c, tanh_c,
                       Y, W_hh, B, S, H, t);
    CNHIP_TRY(check_launch(who));
    if (rec) (void)hipEventRecord(rec->stop, st);
  }
  return CNHIP_OK;
}

template <class Cfg>
int lstm_bwd_steps(const float* gates, const float* c, const float* tanh_c, const float* dY,
                   const float* W_hh, float* dc, float* dG, int64_t B, int64_t S, int64_t H,
                   hipStream_t st, const char* who) {
  const int64_t nbt = (B + 15) / 16, nbu = (H + 15) / 16;
  CNHIP_REQUIRE(nbt * nbu < ((int64_t)1 << 31), "%s: too many tiles", who);
  // FAST: full tiles, whole k-tiles, 16-byte aligned rows (dG is a scratch buffer)
  const bool fast = B % 16 == 0 && H % 16 == 0 && (4 * H) % Cfg::KT == 0 && (B * S) % 4 == 0 &&
                    aligned16(W_hh);
  const auto kern = fast ? &lstm_step_bwd_kernel<Cfg, true> : &lstm_step_bwd_kernel<Cfg, false>;
  for (int64_t t = S - 2; t >= 0; --t) {
    TimingRec* rec = timing_slot(2.0 * B * 4 * H * H);
    if (rec) (void)hipEventRecord(rec->start, st);
    hipLaunchKernelGGL(kern, dim3((unsigned)(nbt * nbu)), dim3(Cfg::NT), 0, st, gates, c, tanh_c, dY,
                       W_hh, dc, dG, B, S, H, t);
    CNHIP_TRY(check_launch(who));
    if (rec) (void)hipEventRecord(rec->stop, st);
  }
  return CNHIP_OK;
}

// ---- persistent-launch plumbing
constexpr int kScratchRecur = 2;  // scratch slot of the fault word and the exchange area
constexpr int kScratchSeq = 3;    // scratch slot of a last-step gradient spread over all steps

// Per device: the epoch of the next launch, and the exchange buffers
// (scratch allocations, by generation) zeroed or run in since the counter
// last started over, each with the number of launches run in it since it
// was zeroed (whose parity picks the launch's XCD counter set).
struct PersistEpochs {
  unsigned next = 1;
  std::vector<std::pair<uint64_t, unsigned>> clean;
};
std::mutex g_epoch_mu;
PersistEpochs g_epochs[64];

void persist_forget_clean(int dev) {
  if (dev < 0 || dev >= 64) return;
  std::lock_guard<std::mutex> lock(g_epoch_mu);
  g_epochs[dev].clean.clear();
}

// Pinned host fault word per device (the kernels set it when a wait gives up).
unsigned* fault_host_word(int dev) {
  static std::mutex mu;
  static unsigned* words[64] = {};
  if (dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!words[dev]) {
    void* p = nullptr;
    if (hipHostMalloc(&p, 64, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    *static_cast<unsigned*>(p) = 0u;
    words[dev] = static_cast<unsigned*>(p);
  }
  return words[dev];
}

}  // namespace

// ---- optimizer guard
// Per GPU (each device holds its own copy of these words): g_update_guard is
// set by a persistent launch that gave up waiting; while it is set, every
// optimizer launch on the device leaves its tensors unchanged and lowers
// g_first_withheld to its sequence number.  Both are reset when the host
// takes the fault (recurrence_fault_check).
__device__ unsigned g_update_guard = 0u;
__device__ unsigned long long g_first_withheld = ~0ull;

namespace {
struct GuardWords {
  unsigned* guard = nullptr;
  unsigned long long* first = nullptr;
};
std::mutex g_guard_mu;
GuardWords g_guard_words[64];
// per device: the sequence numbers [first, last] of the optimizer launches
// withheld by each fault taken
std::vector<std::pair<unsigned long long, unsigned long long>> g_withheld[64];
std::atomic<unsigned long long> g_update_seq{0};
std::atomic<long long> g_faults_taken{0};
thread_local long long t_last_update_seq = -1;

// The device addresses of the current device's guard words, looked up once
// per device with that device current.
int guard_words(GuardWords* out, int* dev_out, const char* who) {
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), who));
  CNHIP_REQUIRE(dev >= 0 && dev < 64, "%s: device %d out of range", who, dev);
  std::lock_guard<std::mutex> lock(g_guard_mu);
  GuardWords& g = g_guard_words[dev];
  if (!g.guard) {
    void* a = nullptr;
    void* b = nullptr;
    CNHIP_TRY(check_hip(hipGetSymbolAddress(&a, HIP_SYMBOL(g_update_guard)), who));
    CNHIP_TRY(check_hip(hipGetSymbolAddress(&b, HIP_SYMBOL(g_first_withheld)), who));
    g.guard = static_cast<unsigned*>(a);
    g.first = static_cast<unsigned long long*>(b);
  }
  *out = g;
  if (dev_out) *dev_out = dev;
  return CNHIP_OK;
}
}  // namespace

int update_guard(UpdateGuard* out, const char* who) {
  GuardWords g;
  CNHIP_TRY(guard_words(&g, nullptr, who));
  out->withhold = g.guard;
  out->first_withheld = g.first;
  out->seq = ++g_update_seq;
  t_last_update_seq = (long long)out->seq;
  return CNHIP_OK;
}

int recurrence_fault_check(hipStream_t st, const char* who) {
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), who));
  unsigned* w = dev >= 0 && dev < 64 ? fault_host_word(dev) : nullptr;
  if (!w || __atomic_load_n(w, __ATOMIC_ACQUIRE) == 0u) return CNHIP_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  CNHIP_TRY(check_hip(hipStreamIsCapturing(st, &cs), who));
  if (cs != hipStreamCaptureStatusNone) {
    set_error("%s: a persistent recurrence launch on this device gave up waiting for its other blocks; "
              "the fault is taken outside graph capture", who);
    return CNHIP_EHIP;
  }
  // every launch queued so far has run: the faulted one and the optimizer
  // launches it withheld
  CNHIP_TRY(check_hip(hipDeviceSynchronize(), who));
  GuardWords g;
  CNHIP_TRY(guard_words(&g, nullptr, who));
  unsigned long long first = ~0ull;
  const unsigned zero = 0u;
  const unsigned long long none = ~0ull;
  CNHIP_TRY(check_hip(hipMemcpy(&first, g.first, sizeof(first), hipMemcpyDeviceToHost), who));
  CNHIP_TRY(check_hip(hipMemcpy(g.first, &none, sizeof(none), hipMemcpyHostToDevice), who));
  CNHIP_TRY(check_hip(hipMemcpy(g.guard, &zero, sizeof(zero), hipMemcpyHostToDevice), who));
  __atomic_store_n(w, 0u, __ATOMIC_RELEASE);
  persist_forget_clean(dev);  // the faulted launch may have left its counters and words anywhere
  if (first != ~0ull) {
    // every optimizer launch from the first withheld one to the last one
    // made so far has run (the device is synchronized) with the guard set
    std::lock_guard<std::mutex> lock(g_guard_mu);
    g_withheld[dev].emplace_back(first, g_update_seq.load());
  }
  ++g_faults_taken;
  set_error("%s: a persistent recurrence launch on this device gave up waiting for its other blocks; its "
            "outputs are invalid, and the optimizer updates queued after it were withheld (%s)",
            who, first != ~0ull ? "parameters and optimizer state are as before them" : "none was queued");
  return CNHIP_EHIP;
}

int update_withheld(int64_t seq) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lock(g_guard_mu);
  for (const auto& r : g_withheld[dev])
    if (seq >= 0 && (unsigned long long)seq >= r.first && (unsigned long long)seq <= r.second) return 1;
  return 0;
}

int64_t update_faults_taken() { return g_faults_taken.load(); }

int64_t update_seq_last() { return t_last_update_seq; }

namespace {

long long persist_spin_limit() {
  const char* e = std::getenv("CNHIP_RECURRENCE_SPIN_LIMIT");
  return e ? std::atoll(e) : (1LL << 20);
}

// The persistent recurrence is the default wherever the shape suits it;
// CNHIP_RECURRENCE_PERSISTENT=0 keeps the per-step launches (which compute
// the recurrent products in another summation order, so the two paths agree
// to rounding, not bit for bit).
bool persist_enabled() {
  const char* e = std::getenv("CNHIP_RECURRENCE_PERSISTENT");
  return !(e && e[0] == '0');
}

// Whether `grid` blocks of `kernel` (`threads` threads) can all be resident.
// The device attributes and the kernel's occupancy are queried once per
// (device, kernel) and cached: the occupancy query costs milliseconds of host
// time, far more than the launch it guards.
bool persist_fits(const void* kernel, int64_t grid, int threads, const char* who) {
  struct Fit {
    int dev;
    const void* kernel;
    int threads;
    int64_t capacity;  // resident blocks, 0 when a cooperative launch is impossible or XCDs != 8
  };
  static std::mutex mu;
  static std::vector<Fit> cache;
  (void)who;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  std::lock_guard<std::mutex> lock(mu);
  for (const Fit& f : cache)
    if (f.dev == dev && f.kernel == kernel && f.threads == threads) return f.capacity > 0 && grid <= f.capacity;
  // The tile placement takes XCC_ID 0..7 and gridDim.x / 8 blocks per XCD
  // (the hardware's round-robin deal of a grid over the 8 XCDs of a device
  // in SPX mode): a device partitioned into fewer XCDs runs the per-step
  // launches instead.
  int cus = 0, coop = 0, per_cu = 0, xccs = 0;
  int64_t capacity = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) == hipSuccess &&
      hipDeviceGetAttribute(&xccs, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) == hipSuccess) {
    if (coop != 0 && per_cu > 0 && xccs == 8 && cus % 8 == 0) capacity = (int64_t)cus * per_cu;
  } else {
    (void)hipGetLastError();
  }
  cache.push_back({dev, kernel, threads, capacity});
  return capacity > 0 && grid <= capacity;
}

// Whether the persistent kernels are launched cooperatively
// (CNHIP_RECURRENCE_COOPERATIVE=1: the runtime then guarantees every block
// resident, or refuses the launch).  By default they are launched plainly,
// as under graph capture: on this ROCm a cooperative launch costs ~23 us
// more per launch (C4: 1.226 vs 1.180 ms per step) and rocprofv3 cannot
// trace it (it crashes at exit without writing its results).  The grid is
// within the device's resident capacity (persist_fits), and this process's
// persistent launches (and graph replays) are ordered one after another
// (persist_ordered), so no two such grids share the device; other work
// holding CUs drains by itself while the blocks already running wait
// (bounded), and a wait that gives up is reported as an error, never a hang.
bool persist_cooperative() {
  const char* e = std::getenv("CNHIP_RECURRENCE_COOPERATIVE");
  return e && e[0] == '1';
}

// The epoch of the next launch on `dev`, and whether its buffer (allocation
// `gen`) must be zeroed first: when no launch has run in it since the epoch
// counter last started over at 1 (a new buffer holds arbitrary words; after
// the wrap, words of earlier launches may carry the epochs to come), or
// since a fault was reported.  A launch recorded into a graph takes epoch 0
// and is always preceded by the zeroing (every replay reuses its stamps).
unsigned persist_epoch(int dev, uint64_t gen, bool capturing, bool* zero, int* set) {
  if (capturing || dev < 0 || dev >= 64) {
    *zero = true;
    *set = 2;
    return 0;
  }
  std::lock_guard<std::mutex> lock(g_epoch_mu);
  PersistEpochs& e = g_epochs[dev];
  if (e.next > 0xffffu) {
    e.next = 1;
    e.clean.clear();
  }
  auto it = std::find_if(e.clean.begin(), e.clean.end(), [gen](const auto& c) { return c.first == gen; });
  *zero = it == e.clean.end();
  if (*zero) it = e.clean.insert(e.clean.end(), {gen, 0u});
  *set = (int)(it->second++ & 1u);
  return e.next++;
}

// Zeroes the fault word, the XCD slot counters and the exchange area
// (ex_bytes, after a 256-byte header) where persist_epoch asks for it, then
// launches `kernel` with one argument (cooperatively only when asked to
// above, and never while the stream is being captured into a graph).
// Header words: 0 the fault word, 16 + 8 k the counter set k (k = 0, 1, 2).
template <class Args>
int persist_launch(const void* kernel, int64_t grid, int threads, Args& args, size_t ex_bytes, hipStream_t st,
                   const char* who) {
  void* ws = nullptr;
  uint64_t gen = 0;
  const size_t bytes = 256 + ex_bytes;
  CNHIP_TRY(scratch(st, kScratchRecur, bytes, &ws, &gen, who));
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), who));
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  CNHIP_TRY(check_hip(hipStreamIsCapturing(st, &cs), who));
  const bool capturing = cs != hipStreamCaptureStatusNone;
  GuardWords g;
  CNHIP_TRY(guard_words(&g, nullptr, who));
  unsigned* head = static_cast<unsigned*>(ws);
  args.sync.fault = head;
  args.sync.guard = g.guard;
  args.sync.fault_host = fault_host_word(dev);
  args.sync.spin_limit = persist_spin_limit();
  args.ex = reinterpret_cast<u64*>(static_cast<char*>(ws) + 256);
  void* params[] = {&args};
  return persist_ordered(st, capturing, who, [&] {
    bool zero = true;
    int set = 2;
    args.sync.epoch = persist_epoch(dev, gen, capturing, &zero, &set);
    args.sync.slots = head + 16 + 8 * set;
    args.sync.slots_next = set == 2 ? nullptr : head + 16 + 8 * (1 - set);
    if (zero) CNHIP_TRY(fill_bytes(ws, 0, bytes, st, who));
    if (!capturing && persist_cooperative())
      CNHIP_TRY(check_hip(hipLaunchCooperativeKernel(kernel, dim3((unsigned)grid), dim3(threads), params, 0, st), who));
    else
      CNHIP_TRY(check_hip(hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(threads), params, 0, st), who));
    return check_launch(who);
  });
}

// Shapes the persistent kernels take: 16-sample tiles, H a multiple of 64
// up to kPersistMaxH, steps below 65535 (the step part of a stamp), 32-bit
// row indices.  grid = 8 (H/16) ceil(nst/8).
bool persist_shape(int64_t B, int64_t S, int64_t H, int64_t& nst, int64_t& nut, int64_t& grid) {
  if (B % kPt != 0 || H % 64 != 0 || H > kPersistMaxH || S < 2 || S > 65000 || B * S * 4 * H > INT32_MAX)
    return false;
  nst = B / kPt;
  nut = H / kPt;
  grid = 8 * nut * ((nst + 7) / 8);
  return true;
}

template <int H>
const void* fwd_persist_kernel(int it) {
  switch (it) {
    case 0: return reinterpret_cast<const void*>(&lstm_fwd_persist_kernel<H, 0>);
    case 1: return reinterpret_cast<const void*>(&lstm_fwd_persist_kernel<H, 1>);
    case 2: return reinterpret_cast<const void*>(&lstm_fwd_persist_kernel<H, 2>);
    default: return nullptr;
  }
}
template <int H>
const void* bwd_persist_kernel(int it) {
  switch (it) {
    case 0: return reinterpret_cast<const void*>(&lstm_bwd_persist_kernel<H, 0>);
    case 1: return reinterpret_cast<const void*>(&lstm_bwd_persist_kernel<H, 1>);
    case 2: return reinterpret_cast<const void*>(&lstm_bwd_persist_kernel<H, 2>);
    default: return nullptr;
  }
}

// The instantiated hidden sizes (W_hh slice of H/4 registers per lane) and
// input widths I = 64 it whose input projection (forward) or weight
// gradients (backward) the kernel computes itself (it = 0: not fused).
const void* persist_kernel(bool fwd, int64_t H, int it = 0) {
  switch (H) {
    case 64: return fwd ? fwd_persist_kernel<64>(it) : bwd_persist_kernel<64>(it);
    case 128: return fwd ? fwd_persist_kernel<128>(it) : bwd_persist_kernel<128>(it);
    case 256: return fwd ? fwd_persist_kernel<256>(it) : bwd_persist_kernel<256>(it);
    case 512: return fwd ? fwd_persist_kernel<512>(it) : bwd_persist_kernel<512>(it);
    default: return nullptr;
  }
}

// Whether the persistent forward can compute the input projection itself
// (CNHIP_RECURRENCE_FUSED_X=0 turns it off): I a multiple of 64 up to 128,
// X and W_ih 16-byte aligned.  Returns I / 64, or 0.
int fwd_fused_inputs(const float* X, const float* W_ih, int64_t I) {
  const char* e = std::getenv("CNHIP_RECURRENCE_FUSED_X");
  if (e && e[0] == '0') return 0;
  if (I % 64 != 0 || I / 64 > 2 || !aligned16(X) || !aligned16(W_ih)) return 0;
  return (int)(I / 64);
}

// Whether the persistent backward can also accumulate the weight gradients
// (CNHIP_RECURRENCE_FUSED_DW=0 turns it off): I a multiple of 64 up to 128
// and 16-byte aligned X and Y (the kernel reads 4 samples per load).
// Returns I / 64, or 0.
int bwd_fused_inputs(const float* X, const float* Y, int64_t I) {
  const char* e = std::getenv("CNHIP_RECURRENCE_FUSED_DW");
  if (e && e[0] == '0') return 0;
  if (I % 64 != 0 || I / 64 > 2 || !aligned16(X) || !aligned16(Y)) return 0;
  return (int)(I / 64);
}

// Phase-stamp buffers of the persistent launches (cnhip_lstm_phase_stamps):
// forward, backward, and their capacity in 64-bit entries.
u64* g_stamps[2] = {nullptr, nullptr};
int64_t g_stamps_cap = 0;
u64* stamps_for(bool fwd, int64_t blocks, int64_t S) {
  return g_stamps[fwd ? 0 : 1] && blocks * S * 8 <= g_stamps_cap ? g_stamps[fwd ? 0 : 1] : nullptr;
}

// The whole BPTT recurrence in one persistent launch when the shape suits
// it (dG: [B*S, 4H], fully written); false in *done to fall back.  With
// `part` (nst (4H^2 + 4HI + 4H) floats) the launch also accumulates the
// weight gradients and a reduction writes gW_hh, gW_ih and gb (*fused).
int lstm_bwd_persistent(const float* gates, const float* c, const float* tanh_c, const float* dY, bool dy_last,
                        const float* W_hh, float* dG, const float* X, const float* Y, float* part, int64_t I,
                        float* gW_hh, float* gW_ih, float* gb, int64_t B, int64_t S, int64_t H, hipStream_t st,
                        const char* who, bool* done, bool* fused) {
  *done = false;
  *fused = false;
  int64_t nst, nut, grid;
  int it = part ? bwd_fused_inputs(X, Y, I) : 0;
  const void* kern = persist_kernel(false, H, it);
  if (!persist_enabled() || !kern || !persist_shape(B, S, H, nst, nut, grid)) return CNHIP_OK;
  const size_t ex_bytes = (size_t)2 * nst * nut * H * kPt * sizeof(u64);
  if (ex_bytes > 0x7fffffffu) return CNHIP_OK;
  if (it && !persist_fits(kern, grid, 256, who)) {
    // the fused kernel holds fewer blocks per CU: the unfused one may fit
    it = 0;
    kern = persist_kernel(false, H, 0);
  }
  if (!persist_fits(kern, grid, 256, who)) return CNHIP_OK;
  LstmBwdPersistArgs args{gates, c, tanh_c, dY, W_hh, dG, nullptr, (int)B, (int)S, (int)nst, {},
                          X, Y, it ? part : nullptr, (int)I, dy_last ? 1 : 0, stamps_for(false, nst * nut, S)};
  const double G = 4.0 * H;
  double flops = 2.0 * B * G * H * (double)(S - 1);
  if (it) flops += 2.0 * H * G * B * (double)(S - 1) + 2.0 * I * G * B * (double)S;
  TimingRec* rec = timing_slot(flops);
  if (rec) (void)hipEventRecord(rec->start, st);
  CNHIP_TRY(persist_launch(kern, grid, 256, args, ex_bytes, st, who));
  if (rec) (void)hipEventRecord(rec->stop, st);
  *done = true;
  if (!it) return CNHIP_OK;
  const int64_t n_hh = H * 4 * H, n_ih = I * 4 * H, n_b = 4 * H;
  {
    HbmTimer timer("lstm_dw_reduce_kernel", 4.0 * (double)(n_hh + n_ih + n_b) * (nst + 1), st);
    hipLaunchKernelGGL(lstm_dw_reduce_kernel, dim3(elementwise_grid(n_hh + n_ih + n_b, 256)), dim3(256), 0, st, part,
                       (int)nst, n_hh, n_ih, n_b, gW_hh, gW_ih, gb);
    CNHIP_TRY(check_launch(who));
  }
  *fused = true;
  return CNHIP_OK;
}

// The whole forward recurrence (t = 0 .. S-1) in one persistent launch, when
// the shape suits it; false in *done to fall back to the per-step launches.
// fused: the launch that also computes the input projection (the caller has
// not run the GEMM), tried only where fwd_fused_inputs allows it; otherwise
// the launch that reads the projection from gates.
int lstm_fwd_persistent(float* gates, const float* b, float* c, float* tanh_c, float* Y, const float* W_hh,
                        const float* X, const float* W_ih, int64_t I, bool fused, int64_t B, int64_t S, int64_t H,
                        hipStream_t st, const char* who, bool* done) {
  *done = false;
  int64_t nst, nut, grid;
  const int it = fused ? fwd_fused_inputs(X, W_ih, I) : 0;
  if (fused && !it) return CNHIP_OK;
  const void* kern = persist_kernel(true, H, it);
  if (!persist_enabled() || !kern || !persist_shape(B, S, H, nst, nut, grid) || !aligned16(W_hh)) return CNHIP_OK;
  const size_t ex_bytes = (size_t)2 * nst * H * kPt * sizeof(u64);
  if (ex_bytes > 0x7fffffffu || !persist_fits(kern, grid, 256, who)) return CNHIP_OK;
  LstmFwdPersistArgs args{gates, b, c, tanh_c, Y, W_hh, nullptr, (int)B, (int)S, (int)nst, {}, X, W_ih,
                          stamps_for(true, nst * nut, S)};
  double flops = 2.0 * B * 4 * H * H * (double)(S - 1);
  if (it) flops += 2.0 * B * 4 * H * I * (double)S;
  TimingRec* rec = timing_slot(flops);
  if (rec) (void)hipEventRecord(rec->start, st);
  CNHIP_TRY(persist_launch(kern, grid, 256, args, ex_bytes, st, who));
  if (rec) (void)hipEventRecord(rec->stop, st);
  *done = true;
  return CNHIP_OK;
}

int check_rnn(int64_t B, int64_t S, int64_t I, int64_t H, const char* who) {
  CNHIP_REQUIRE(B > 0 && S > 0 && I > 0 && H > 0, "%s: bad shape B=%lld S=%lld I=%lld H=%lld", who,
                (long long)B, (long long)S, (long long)I, (long long)H);
  CNHIP_REQUIRE(B * H < ((int64_t)1 << 31), "%s: B*H too large", who);
  return CNHIP_OK;
}

struct Workspace {
  void* p = nullptr;
  hipStream_t st;
  explicit Workspace(hipStream_t s) : st(s) {}
  int alloc(size_t bytes, const char* who) { return scratch(st, kScratchLayer, bytes, &p, who); }
  ~Workspace() {
    // nothing to free: the stream's scratch slot is reused by later calls
  }
};

// BPTT of the LSTM (lstm.cpp:184-253).  dy_last: dY is [B, H], the
// gradient of the last step's output only (a SequenceLast after the layer);
// the persistent kernel reads it as such, the per-step path from a [B, S, H]
// copy with zeros elsewhere.
int lstm_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y, const float* gates,
                  const float* c, const float* tanh_c, const float* dY, bool dy_last, float* gW_ih, float* gW_hh,
                  float* gb, float* dX, int64_t B, int64_t S, int64_t I, int64_t H, hipStream_t st,
                  const char* who) {
  CNHIP_TRY(check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && Y && gates && c && tanh_c && dY && gW_ih && gW_hh && gb,
                "%s: NULL pointer", who);
  CNHIP_TRY(recurrence_fault_check(st, who));
  const int64_t G = 4 * H, BS = B * S;
  Workspace ws(st);
  // dG, dc and, for the fused weight gradients, one partial per 16-sample tile
  const int64_t n_part = bwd_fused_inputs(X, Y, I) ? (B / 16) * (G * H + G * I + G) : 0;
  CNHIP_TRY(ws.alloc((size_t)(BS * G + B * H + n_part) * sizeof(float), who));
  float* dG = static_cast<float*>(ws.p);
  float* dc = dG + BS * G;
  float* part = n_part ? dc + B * H : nullptr;
  bool done = false, fused = false;
  CNHIP_TRY(lstm_bwd_persistent(gates, c, tanh_c, dY, dy_last, W_hh, dG, X, Y, part, I, gW_hh, gW_ih, gb, B, S, H,
                                st, who, &done, &fused));
  if (!done) {
    const float* dYs = dY;
    if (dy_last) {
      void* p = nullptr;
      CNHIP_TRY(scratch(st, kScratchSeq, (size_t)BS * H * sizeof(float), &p, who));
      float* full = static_cast<float*>(p);
      hipLaunchKernelGGL(seq_scatter_kernel, dim3(elementwise_grid(BS * H, 256)), dim3(256), 0, st, dY, full, B,
                         S, H, S - 1);
      CNHIP_TRY(check_launch(who));
      dYs = full;
    }
    // t = S-1: dh = dY only; then per step one fused launch of
    // dh_t = dY_t + dG_{t+1} W_hh^T (lstm.cpp:244) and the cell backward
    hipLaunchKernelGGL(lstm_cell_bwd_last_kernel, dim3(cell_grid(B, H)), dim3(256), 0, st, gates, c, tanh_c, dYs,
                       dc, dG, B, S, H);
    CNHIP_TRY(check_launch(who));
    CNHIP_TRY(lstm_bwd_steps<LstmBwdCfgDefault>(gates, c, tanh_c, dYs, W_hh, dc, dG, B, S, H, st, who));
  }
  if (!fused) {
    CNHIP_TRY(gemm_f32(1, 0, I, G, BS, 1.f, X, BS, dG, BS, 0.f, gW_ih, I, nullptr, 0, st, who));
    CNHIP_TRY(gemm_f32(1, 0, H, G, B * (S - 1), 1.f, Y, BS, dG + B, BS, 0.f, gW_hh, H, nullptr, 0, st, who));
    CNHIP_TRY(column_sum(dG, gb, BS, G, 0, st, who));
  }
  if (dX) CNHIP_TRY(gemm_f32(0, 1, BS, I, G, 1.f, dG, BS, W_ih, I, 0.f, dX, BS, nullptr, 0, st, who));
  return CNHIP_OK;
}

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

extern "C" {

int cnhip_lstm_phase_stamps(uint64_t* fwd, uint64_t* bwd, int64_t capacity) {
  CNHIP_REQUIRE(capacity >= 0, "cnhip_lstm_phase_stamps: negative capacity");
  cnhip::g_stamps[0] = reinterpret_cast<cnhip::u64*>(fwd);
  cnhip::g_stamps[1] = reinterpret_cast<cnhip::u64*>(bwd);
  cnhip::g_stamps_cap = capacity;
  return CNHIP_OK;
}

int cnhip_recurrence_fault_check(cnhip_stream_t stream) {
  return cnhip::recurrence_fault_check(as_stream(stream), "cnhip_recurrence_fault_check");
}

int64_t cnhip_update_faults_taken(void) { return cnhip::update_faults_taken(); }

int cnhip_update_withheld(int64_t seq) { return cnhip::update_withheld(seq); }

int64_t cnhip_update_seq_last(void) { return cnhip::update_seq_last(); }

int cnhip_lstm_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                       float* Y, float* gates, float* c, float* tanh_c, int64_t B, int64_t S,
                       int64_t I, int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_lstm_forward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && b && Y && gates && c && tanh_c, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  CNHIP_TRY(cnhip::recurrence_fault_check(st, who));
  const int64_t G = 4 * H, BS = B * S;
  bool done = false;
  CNHIP_TRY(cnhip::lstm_fwd_persistent(gates, b, c, tanh_c, Y, W_hh, X, W_ih, I, true, B, S, H, st, who, &done));
  if (done) return CNHIP_OK;
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, G, I, 1.f, X, BS, W_ih, I, 0.f, gates, BS, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::lstm_fwd_persistent(gates, b, c, tanh_c, Y, W_hh, X, W_ih, I, false, B, S, H, st, who, &done));
  if (done) return CNHIP_OK;
  // t = 0: h_0 = 0, no recurrent term; then one fused GEMM + cell launch per step
  hipLaunchKernelGGL(cnhip::lstm_cell_fwd0_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                     gates, b, c, tanh_c, Y, B, S, H);
  CNHIP_TRY(cnhip::check_launch(who));
  return cnhip::lstm_fwd_steps<cnhip::LstmFwdCfg>(gates, b, c, tanh_c, Y, W_hh, B, S, H, st, who);
}

int cnhip_lstm_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                        const float* gates, const float* c, const float* tanh_c, const float* dY,
                        float* gW_ih, float* gW_hh, float* gb, float* dX, int64_t B, int64_t S,
                        int64_t I, int64_t H, cnhip_stream_t stream) {
  return cnhip::lstm_backward(X, W_ih, W_hh, Y, gates, c, tanh_c, dY, false, gW_ih, gW_hh, gb, dX, B, S, I, H,
                              as_stream(stream), "cnhip_lstm_backward");
}

int cnhip_lstm_backward_last(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                             const float* gates, const float* c, const float* tanh_c, const float* dY_last,
                             float* gW_ih, float* gW_hh, float* gb, float* dX, int64_t B, int64_t S,
                             int64_t I, int64_t H, cnhip_stream_t stream) {
  return cnhip::lstm_backward(X, W_ih, W_hh, Y, gates, c, tanh_c, dY_last, true, gW_ih, gW_hh, gb, dX, B, S, I,
                              H, as_stream(stream), "cnhip_lstm_backward_last");
}

int cnhip_gru_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                      float* Y, float* gates, float* rh, int64_t B, int64_t S, int64_t I,
                      int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_gru_forward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && b && Y && gates && rh, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t G = 3 * H, BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(3 * B * H) * sizeof(float), who));
  float* hz = static_cast<float*>(ws.p);  // [B, 2H]
  float* proj = hz + 2 * B * H;           // [B, H]
  const float* W_hn = W_hh + H * 2 * H;
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, G, I, 1.f, X, BS, W_ih, I, 0.f, gates, BS, nullptr, 0, st, who));
  for (int64_t t = 0; t < S; ++t) {
    if (t > 0)
      CNHIP_TRY(cnhip::gemm_f32(0, 0, B, 2 * H, H, 1.f, Y + B * (t - 1), BS, W_hh, H, 0.f, hz, B,
                                nullptr, 0, st, who));
    hipLaunchKernelGGL(cnhip::gru_zr_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, gates,
                       hz, b, Y, rh, B, S, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
    CNHIP_TRY(cnhip::gemm_f32(0, 0, B, H, H, 1.f, rh + B * t, BS, W_hn, H, 0.f, proj, B, nullptr, 0,
                              st, who));
    hipLaunchKernelGGL(cnhip::gru_n_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, gates,
                       proj, b, Y, B, S, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
  }
  return CNHIP_OK;
}

int cnhip_gru_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y,
                       const float* gates, const float* rh, const float* dY, float* gW_ih,
                       float* gW_hh, float* gb, float* dX, int64_t B, int64_t S, int64_t I,
                       int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_gru_backward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && Y && gates && rh && dY && gW_ih && gW_hh && gb,
                "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t G = 3 * H, BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(BS * G + 2 * B * H) * sizeof(float), who));
  float* dG = static_cast<float*>(ws.p);
  float* dh = dG + BS * G;
  float* drh = dh + B * H;
  const float* W_hn = W_hh + H * 2 * H;
  for (int64_t t = S - 1; t >= 0; --t) {
    hipLaunchKernelGGL(cnhip::gru_bwd_a_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                       gates, Y, dY, dh, dG, B, S, H, t, t == S - 1 ? 1 : 0);
    CNHIP_TRY(cnhip::check_launch(who));
    // d_rh = dn_raw W_hn^T
    CNHIP_TRY(cnhip::gemm_f32(0, 1, B, H, H, 1.f, dG + B * t + BS * 2 * H, BS, W_hn, H, 0.f, drh, B,
                              nullptr, 0, st, who));
    hipLaunchKernelGGL(cnhip::gru_bwd_b_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st,
                       gates, Y, drh, dh, dG, B, S, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
    // dh_next = dh_prev + dG_t[z,r] W_hh[:, 0:2H]^T
    if (t > 0)
      CNHIP_TRY(cnhip::gemm_f32(0, 1, B, H, 2 * H, 1.f, dG + B * t, BS, W_hh, H, 1.f, dh, B, nullptr,
                                0, st, who));
  }
  CNHIP_TRY(cnhip::gemm_f32(1, 0, I, G, BS, 1.f, X, BS, dG, BS, 0.f, gW_ih, I, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, H, 2 * H, B * (S - 1), 1.f, Y, BS, dG + B, BS, 0.f, gW_hh, H,
                            nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, H, H, BS, 1.f, rh, BS, dG + BS * 2 * H, BS, 0.f, gW_hh + H * 2 * H,
                            H, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::column_sum(dG, gb, BS, G, 0, st, who));
  if (dX)
    CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, I, G, 1.f, dG, BS, W_ih, I, 0.f, dX, BS, nullptr, 0, st, who));
  return CNHIP_OK;
}

int cnhip_seq_select(const float* Y, float* out, int64_t B, int64_t S, int64_t D, int64_t t,
                     cnhip_stream_t stream) {
  const char* who = "cnhip_seq_select";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0 && t >= 0 && t < S, "%s: bad shape or step", who);
  CNHIP_REQUIRE(Y && out, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("seq_select_kernel", 8.0 * (double)B * (double)D, as_stream(stream));
  hipLaunchKernelGGL(cnhip::seq_select_kernel, dim3((unsigned)((B * D + 255) / 256)), dim3(256), 0,
                     as_stream(stream), Y, out, B, S, D, t);
  return cnhip::check_launch(who);
}

int cnhip_seq_scatter(const float* in, float* Y, int64_t B, int64_t S, int64_t D, int64_t t,
                      cnhip_stream_t stream) {
  const char* who = "cnhip_seq_scatter";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0 && t >= 0 && t < S, "%s: bad shape or step", who);
  CNHIP_REQUIRE(Y && in, "%s: NULL pointer", who);
  // the step's rows read; the whole sequence gradient written (zeros elsewhere)
  cnhip::HbmTimer timer("seq_scatter_kernel", 4.0 * (double)B * (double)D * (double)(S + 1),
                        as_stream(stream));
  hipLaunchKernelGGL(cnhip::seq_scatter_kernel, dim3(cnhip::elementwise_grid(B * S * D, 256)),
                     dim3(256), 0, as_stream(stream), in, Y, B, S, D, t);
  return cnhip::check_launch(who);
}

int cnhip_rnn_forward(const float* X, const float* W_ih, const float* W_hh, const float* b, float* Y,
                      int64_t B, int64_t S, int64_t I, int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_rnn_forward";
  CNHIP_REQUIRE(B > 0 && S > 0 && I > 0 && H > 0, "%s: bad shape B=%lld S=%lld I=%lld H=%lld", who,
                (long long)B, (long long)S, (long long)I, (long long)H);
  CNHIP_REQUIRE(X && W_ih && W_hh && b && Y, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t BS = B * S;
  // x_t W_ih for every step at once (rnn.cpp:73-74), then the recurrence:
  // step t's rows of Y = tanh(h_{t-1} W_hh + Y_t + b), the GEMM adding the
  // x-projection (beta = 1) and the bias and applying tanh in its epilogue
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, H, I, 1.f, X, BS, W_ih, I, 0.f, Y, BS, nullptr, 0, st, who));
  hipLaunchKernelGGL(cnhip::rnn_step0_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, Y, b, B, BS, H);
  CNHIP_TRY(cnhip::check_launch(who));
  for (int64_t t = 1; t < S; ++t)
    CNHIP_TRY(cnhip::gemm_f32_core(0, 0, B, H, H, 1.f, Y + B * (t - 1), BS, 0, W_hh, H, 0, 1.f, Y + B * t, BS,
                                   0, 1, b, cnhip::EPI_TANH, nullptr, nullptr, 0, st, who));
  return CNHIP_OK;
}

int cnhip_rnn_backward(const float* X, const float* W_ih, const float* W_hh, const float* Y, const float* dY,
                       float* gW_ih, float* gW_hh, float* gb, float* dX, int64_t B, int64_t S, int64_t I,
                       int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_rnn_backward";
  CNHIP_REQUIRE(B > 0 && S > 0 && I > 0 && H > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(X && W_ih && W_hh && Y && dY && gW_ih && gW_hh && gb, "%s: NULL pointer", who);
  hipStream_t st = as_stream(stream);
  const int64_t BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(BS * H + B * H) * sizeof(float), who));
  float* dT = static_cast<float*>(ws.p);  // dtanh of every step, [B*S, H]
  float* dh = dT + BS * H;                // dh_next = dtanh_{t+1} W_hh^T, [B, H]
  for (int64_t t = S - 1; t >= 0; --t) {
    hipLaunchKernelGGL(cnhip::rnn_bwd_cell_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0, st, dY, Y,
                       t == S - 1 ? nullptr : dh, dT, B, BS, H, t);
    CNHIP_TRY(cnhip::check_launch(who));
    if (t > 0)
      CNHIP_TRY(cnhip::gemm_f32(0, 1, B, H, H, 1.f, dT + B * t, BS, W_hh, H, 0.f, dh, B, nullptr, 0, st, who));
  }
  // weight grads over all B*S rows (rnn.cpp:136-142): gW_ih = X^T dT,
  // gW_hh = [h_0 .. h_{S-2}]^T dT[steps 1..S-1] (h_{-1} = 0 adds nothing),
  // gb = colsum dT; dX = dT W_ih^T (rnn.cpp:145-149)
  CNHIP_TRY(cnhip::gemm_f32(1, 0, I, H, BS, 1.f, X, BS, dT, BS, 0.f, gW_ih, I, nullptr, 0, st, who));
  if (S > 1)
    CNHIP_TRY(cnhip::gemm_f32(1, 0, H, H, B * (S - 1), 1.f, Y, BS, dT + B, BS, 0.f, gW_hh, H, nullptr, 0, st,
                              who));
  else
    CNHIP_TRY(cnhip::fill_bytes(gW_hh, 0, (size_t)(H * H) * sizeof(float), st, who));
  CNHIP_TRY(cnhip::column_sum(dT, gb, BS, H, 0, st, who));
  if (dX) CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, I, H, 1.f, dT, BS, W_ih, I, 0.f, dX, BS, nullptr, 0, st, who));
  return CNHIP_OK;
}

}  // extern "C"
