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
//   forward : G = X W_ih (all steps), then per step one launch of
//             h_{t-1} W_hh with the LSTM cell in its epilogue
//   backward: per step one launch of dh_t = dY_t + dG_{t+1} W_hh^T with the
//             cell backward in its epilogue; afterwards dW_ih = X^T dG,
//             dW_hh = Y_{t-1}^T dG, db = colsum dG, dX = dG W_ih^T, each a
//             single GEMM over all B*S rows.
// The cell kernels fuse every elementwise gate computation of a step into one
// pass (one thread per (n, d); n fastest for coalescing) and evaluate the
// reference expressions in the reference's operation order.
#include <hip/hip_runtime.h>

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
// All timesteps of the LSTM forward in ONE launch.  The grid is the same
// 32-sample x 8-unit tiling as lstm_step_fwd_kernel (256 blocks at B = 128,
// H = 512), one block per CU, every block resident for the whole sequence:
// a block keeps its W_hh slice (H x 32, 64 KB at H = 512) in LDS for all S
// steps and its units' cell state c in registers, so per step it reads only
// h_{t-1} of its 32 samples and the step's x W_ih terms.  Between steps the
// blocks of one sample tile synchronise through a counter: after writing its
// part of h_t (agent-coherent stores, below) a block adds 1; before step t a
// block waits until its tile's counter reaches units_tiles * t and then
// reads h_{t-1} with agent-coherent loads.  Each wave runs exactly the MFMA sequence of the per-step
// kernel (same k per lane per step, same order) and the four waves' partial
// tiles are added in the same order, so both paths give identical bits.
//
// Every wait is bounded: after spin_limit polls a block gives up, sets the
// launch's fault word (device memory; every waiting block sees it at its
// next poll and exits) and the host-visible fault word, and returns -- so the
// grid always drains, even if the blocks were not all resident.  The host
// reports a set fault word as an error at the next recurrent launch.
constexpr int kPersistMaxH = 512;  // LDS: W slice + h tile of H x 32 floats each

struct PersistSync {
  unsigned* counters;  // [sample tiles], zeroed before the launch
  unsigned* fault;     // device word, zeroed before the launch
  unsigned* fault_host;  // pinned host word, or null
  long long spin_limit;
};

__device__ __forceinline__ void persist_fail(const PersistSync& ps) {
  __hip_atomic_store(ps.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (ps.fault_host) __hip_atomic_store(ps.fault_host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Thread 0 of a block: wait until *ctr >= target.  false: gave up (fault).
__device__ __forceinline__ bool persist_wait(const PersistSync& ps, unsigned* ctr, unsigned target) {
  if (ps.spin_limit < 0) {  // a negative limit gives up at once (tests of the fault path)
    persist_fail(ps);
    return false;
  }
  // relaxed polls of the agent-coherent counter
  for (long long spins = 0;; ++spins) {
    if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) return true;
    if (__hip_atomic_load(ps.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return false;
    if (spins >= ps.spin_limit) {
      persist_fail(ps);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Values one block hands to the others between steps (h_t forward, dG_t
// backward) are written and read with agent-coherent accesses: relaxed
// agent-scope atomic stores write through to the memory level all XCDs
// share, and relaxed agent-scope atomic loads read from it, so a stale line
// in an XCD's L2 is never read.  The step counter then needs no fence: a
// wave's stores have completed (s_waitcnt) before the barrier, and thread 0
// increments the counter after it; a reader polls the counter, passes the
// barrier, then loads.  (An agent-scope release/acquire pair would instead
// write back and invalidate the XCD's whole L2 for every block and step,
// which measured several times the per-step launches' cost.)
__device__ __forceinline__ void xstore(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 xload4(const float* p) {
  f32x4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = __hip_atomic_load(p + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return v;
}

// All threads: wait until the tile's counter reaches target (thread 0
// polls).  Returns false (uniformly) when the launch has faulted.
__device__ __forceinline__ bool persist_block_wait(const PersistSync& ps, unsigned* ctr, unsigned target,
                                                   int* flag) {
  if (threadIdx.x == 0) *flag = persist_wait(ps, ctr, target) ? 1 : 0;
  __syncthreads();
  return *flag != 0;
}

// All threads: each wave's exchanged stores complete, then thread 0 counts.
__device__ __forceinline__ void persist_block_signal(unsigned* ctr) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct LstmFwdPersistArgs {
  float* gates;
  const float* bias;
  float* c;
  float* tanh_c;
  float* Y;
  const float* W_hh;
  int B, S, H, nbt;
  PersistSync sync;
};

__global__ void __launch_bounds__(256) lstm_fwd_persist_kernel(LstmFwdPersistArgs a) {
  __shared__ __align__(16) float Ws[kPersistMaxH * 32];  // [k][col], col = gate * 8 + unit
  __shared__ __align__(16) float hs[kPersistMaxH * 32];  // [k][sample]
  __shared__ float red[4][32 * 33];                        // per-wave partial tiles, [col][sample]
  __shared__ int flag;
  const int H = a.H, B = a.B;
  const int64_t BS = (int64_t)B * a.S;
  const int bt = (int)(blockIdx.x % a.nbt), ut = (int)(blockIdx.x / a.nbt);
  const int b0 = bt * 32, j0 = ut * kLstmUnits;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  unsigned* ctr = a.sync.counters + bt;

  // the block's W_hh columns gate * H + j0 + unit, k-contiguous in memory
  for (int idx = tid; idx < H * 8; idx += 256) {  // 32 columns x H/4 float4s
    const int col = idx / (H / 4), k = (idx % (H / 4)) * 4;
    const float* src = a.W_hh + k + (int64_t)H * ((col / kLstmUnits) * H + j0 + col % kLstmUnits);
    const f32x4 v = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
    for (int e = 0; e < 4; ++e) Ws[(k + e) * 32 + col] = v[e];
  }
  // thread -> (sample bl, unit u) of the cell update, as lstm_step_fwd_kernel
  const int bl = tid % 32, u = tid / 32;
  const int64_t n = b0 + bl, d = j0 + u;
  float c_prev = 0.0f;
  __syncthreads();

  for (int t = 0; t < a.S; ++t) {
    const int64_t row = n + (int64_t)B * t;
    float* g = a.gates + row;
    // this step's x W_ih terms do not depend on the recurrence
    const float xi = g[BS * d], xf = g[BS * (d + H)], xg = g[BS * (d + 2 * H)], xo = g[BS * (d + 3 * H)];
    float ig, fg, gg, og;
    if (t == 0) {  // h_0 = c_0 = 0 (lstm_cell_fwd0_kernel's arithmetic)
      ig = sigm(xi + a.bias[d]);
      fg = sigm(xf + a.bias[d + H]);
      gg = tanhf(xg + a.bias[d + 2 * H]);
      og = sigm(xo + a.bias[d + 3 * H]);
    } else {
      if (!persist_block_wait(a.sync, ctr, (unsigned)(a.H / kLstmUnits) * (unsigned)t, &flag)) return;
      // h_{t-1} of the tile's 32 samples: hs[k][m] = Y[b0 + m + B (t-1) + BS k].
      // All of a thread's loads are issued before its LDS stores, so their
      // latencies overlap (a load-store loop waits for each load in turn).
      const float* Yp = a.Y + b0 + (int64_t)B * (t - 1);
      constexpr int kPer = kPersistMaxH * 8 / 256;
      f32x4 hv[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int idx = tid + 256 * j;
        if (idx < H * 8) hv[j] = xload4(Yp + (idx & 7) * 4 + BS * (idx >> 3));
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int idx = tid + 256 * j;
        if (idx < H * 8) *reinterpret_cast<f32x4*>(hs + (idx >> 3) * 32 + (idx & 7) * 4) = hv[j];
      }
      __syncthreads();
      // wave w: k = kt*64 + 16w + 8h + 4c + e, in lstm_step_fwd_kernel's order
      kp::f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
      const int r32 = lane & 31, hf = lane >> 5;
      for (int kt = 0; kt < H / 64; ++kt) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int k = kt * 64 + wave * 16 + 8 * hf + 4 * c + e;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(hs[k * 32 + r32], Ws[k * 32 + r32], acc, 0, 0, 0);
          }
      }
      // partial tile of this wave: lane holds column r32, rows 8(r/4) + 4hf + r%4
#pragma unroll
      for (int r = 0; r < 16; ++r) red[wave][r32 * 33 + 8 * (r / 4) + 4 * hf + (r % 4)] = acc[r];
      __syncthreads();
      // waves summed in order 0, 1, 2, 3 (reduce_wgk's order)
      float pre[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int at = (q * kLstmUnits + u) * 33 + bl;
        pre[q] = ((red[0][at] + red[1][at]) + red[2][at]) + red[3][at];
      }
      ig = sigm((pre[0] + xi) + a.bias[d]);
      fg = sigm((pre[1] + xf) + a.bias[d + H]);
      gg = tanhf((pre[2] + xg) + a.bias[d + 2 * H]);
      og = sigm((pre[3] + xo) + a.bias[d + 3 * H]);
    }
    const float ct = lstm_cell_c(fg, t == 0 ? 0.0f : c_prev, ig, gg);
    const float tc = tanhf(ct);
    g[BS * d] = ig;
    g[BS * (d + H)] = fg;
    g[BS * (d + 2 * H)] = gg;
    g[BS * (d + 3 * H)] = og;
    a.c[row + BS * d] = ct;
    a.tanh_c[row + BS * d] = tc;
    xstore(a.Y + row + BS * d, og * tc);
    c_prev = ct;
    if (t + 1 < a.S) persist_block_signal(ctr);
  }
}

// All backward timesteps (t = S-1 .. 0) in ONE launch, the tiling of
// lstm_step_bwd_kernel (16 samples x 16 units, 8 waves, 256 blocks at
// B = 128, H = 512).  A block keeps its slice of W_hh^T (16 units x 4H) in
// registers -- wave w only ever needs the k of its own slices, 64 values per
// lane -- and its units' dc in registers; per step it stages dG_{t+1} of its
// 16 samples (16 x 4H, [sample][k] in LDS) and runs the per-step kernel's
// MFMA sequence and 8-way reduction, then the cell backward.  Blocks of one
// sample tile synchronise as in lstm_fwd_persist_kernel.
constexpr int kPersistBwdMaxG = 2048;  // 4H <= 2048
constexpr int kPersistBwdLd = kPersistBwdMaxG + 4;

struct LstmBwdPersistArgs {
  const float* gates;
  const float* c;
  const float* tanh_c;
  const float* dY;
  const float* W_hh;
  float* dG;
  int B, S, H, nbt;
  PersistSync sync;
};

__global__ void __launch_bounds__(512) lstm_bwd_persist_kernel(LstmBwdPersistArgs a) {
  __shared__ __align__(16) float As[16 * kPersistBwdLd];  // dG_{t+1}: [sample][k]
  __shared__ float red[7][4 * 64];                         // partials of waves 1..7
  __shared__ float tile[16 * 17];                          // [unit][sample]
  __shared__ int flag;
  const int H = a.H, B = a.B, G = 4 * H;
  const int64_t BS = (int64_t)B * a.S;
  const int bt = (int)(blockIdx.x % a.nbt), ut = (int)(blockIdx.x / a.nbt);
  const int b0 = bt * 16, j0 = ut * 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  unsigned* ctr = a.sync.counters + bt;
  const int nkt = G / 256;  // k-tiles of 256 (G % 256 == 0)

  // W_hh^T(j, k) = W_hh[j + H k] for this lane's unit j0 + r16 and the k of
  // its MFMA steps: k = kt*256 + 32*wave + 16c + 4q + e
  constexpr int kMaxKt = kPersistBwdMaxG / 256;
  float wv[kMaxKt * 8];  // unrolled loops below: register-indexed only
#pragma unroll
  for (int kt = 0; kt < kMaxKt; ++kt)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = kt * 256 + 32 * wave + 16 * c + 4 * q + e;
        wv[(kt * 2 + c) * 4 + e] = kt < nkt ? a.W_hh[(j0 + r16) + (int64_t)H * k] : 0.0f;
      }
  // thread -> (sample bl, unit jl) of the cell backward (threads 0..255)
  const int bl = tid % 16, jl = tid / 16;
  const bool cell = tid < 256;
  const int64_t n = b0 + bl, d = j0 + jl;
  float dc_next = 0.0f;

  for (int t = a.S - 1; t >= 0; --t) {
    const int64_t row = n + (int64_t)B * t;
    float rec = 0.0f;  // dG_{t+1} W_hh^T for (n, d)
    if (t < a.S - 1) {
      if (!persist_block_wait(a.sync, ctr, (unsigned)(H / 16) * (unsigned)(a.S - 1 - t), &flag)) return;
      // As[m][k] = dG[b0 + m + B (t+1) + BS k]
      // (loads first, then the LDS stores, as in the forward kernel)
      const float* src = a.dG + b0 + (int64_t)B * (t + 1);
      constexpr int kPer = kPersistBwdMaxG * 4 / 512;
      f32x4 gv[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int idx = tid + 512 * j;
        if (idx < G * 4) gv[j] = xload4(src + (idx & 3) * 4 + BS * (idx >> 2));
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int idx = tid + 512 * j;
        if (idx < G * 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) As[((idx & 3) * 4 + e) * kPersistBwdLd + (idx >> 2)] = gv[j][e];
        }
      }
      __syncthreads();
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < kMaxKt; ++kt)
        if (kt < nkt)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int k = kt * 256 + 32 * wave + 16 * c + 4 * q;
          const f32x4 av = *reinterpret_cast<const f32x4*>(As + r16 * kPersistBwdLd + k);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], wv[(kt * 2 + c) * 4 + e], acc, 0, 0, 0);
        }
      // waves 1..7 hand their partials to wave 0, which adds them in order
      if (wave > 0) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) red[wave - 1][rr * 64 + lane] = acc[rr];
      }
      __syncthreads();
      if (wave == 0) {
        for (int g = 0; g < 7; ++g)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) acc[rr] += red[g][rr * 64 + lane];
        // lane holds unit column r16 and samples 4q + rr
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) tile[(4 * q + rr) + 17 * r16] = acc[rr];
      }
      __syncthreads();
      if (cell) rec = tile[bl + 17 * jl];
    }
    if (cell) {
      const float ig = a.gates[row + BS * d], fg = a.gates[row + BS * (d + H)];
      const float gg = a.gates[row + BS * (d + 2 * H)], og = a.gates[row + BS * (d + 3 * H)];
      const float tc = a.tanh_c[row + BS * d];
      // the last step (lstm_cell_bwd_last_kernel) has no later step: dh = dY, dc_in = 0
      const float dh = t == a.S - 1 ? a.dY[row + BS * d] : a.dY[row + BS * d] + rec;
      const float cprev = t > 0 ? a.c[row - B + BS * d] : 0.0f;
      float di, df, dgg, dout;
      lstm_cell_bwd(ig, fg, gg, og, tc, dh, t == a.S - 1 ? 0.0f : dc_next, cprev, di, df, dgg, dout, dc_next);
      xstore(a.dG + row + BS * d, di);
      xstore(a.dG + row + BS * (d + H), df);
      xstore(a.dG + row + BS * (d + 2 * H), dgg);
      xstore(a.dG + row + BS * (d + 3 * H), dout);
    }
    if (t > 0) persist_block_signal(ctr);
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
constexpr int kScratchRecur = 2;  // scratch slot of the counters and fault word

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

// A fault left by an earlier persistent launch on this device: reported
// (and cleared) at the next recurrent call.
int persist_take_fault(const char* who) {
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), who));
  unsigned* w = fault_host_word(dev);
  if (w && __atomic_exchange_n(w, 0u, __ATOMIC_ACQ_REL) != 0u) {
    set_error("%s: an earlier persistent recurrence launch on this device gave up waiting for its other "
              "blocks (not all co-resident?); its outputs are invalid", who);
    return CNHIP_EHIP;
  }
  return CNHIP_OK;
}

long long persist_spin_limit() {
  const char* e = std::getenv("CNHIP_RECURRENCE_SPIN_LIMIT");
  return e ? std::atoll(e) : (1LL << 20);
}

// The persistent kernels run only with CNHIP_RECURRENCE_PERSISTENT=1: on the
// MI355X they measure slower than the per-step launches (C4 shape: 0.85 ms
// forward and 1.6 ms backward against 0.55 and 0.89 ms), because every step
// re-reads each sample tile's h_{t-1} (or dG_{t+1}) from the memory level
// all XCDs share -- the per-XCD L2s are not coherent with each other within
// a launch -- where the per-step kernels read it through L2.  Both paths
// compute the same bits.
bool persist_enabled() {
  const char* e = std::getenv("CNHIP_RECURRENCE_PERSISTENT");
  return e && e[0] == '1';
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
    int64_t capacity;  // resident blocks, 0 when a cooperative launch is impossible
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
  int cus = 0, coop = 0, per_cu = 0;
  int64_t capacity = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) == hipSuccess) {
    if (coop != 0 && per_cu > 0) capacity = (int64_t)cus * per_cu;
  } else {
    (void)hipGetLastError();
  }
  cache.push_back({dev, kernel, threads, capacity});
  return capacity > 0 && grid <= capacity;
}

// Zeroes the counters and fault word, then launches `kernel` with one
// argument (cooperatively; a plain launch of the same kernel while the
// stream is being captured into a graph).
template <class Args>
int persist_launch(const void* kernel, int64_t grid, int threads, Args& args, int tiles, hipStream_t st,
                   const char* who) {
  void* ws = nullptr;
  const size_t bytes = (size_t)(tiles + 1) * sizeof(unsigned);
  CNHIP_TRY(scratch(st, kScratchRecur, bytes, &ws, who));
  CNHIP_TRY(fill_bytes(ws, 0, bytes, st, who));
  int dev = 0;
  CNHIP_TRY(check_hip(hipGetDevice(&dev), who));
  args.sync.counters = static_cast<unsigned*>(ws);
  args.sync.fault = static_cast<unsigned*>(ws) + tiles;
  args.sync.fault_host = fault_host_word(dev);
  args.sync.spin_limit = persist_spin_limit();
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  CNHIP_TRY(check_hip(hipStreamIsCapturing(st, &cs), who));
  void* params[] = {&args};
  if (cs == hipStreamCaptureStatusNone)
    CNHIP_TRY(check_hip(hipLaunchCooperativeKernel(kernel, dim3((unsigned)grid), dim3(threads), params, 0, st), who));
  else
    CNHIP_TRY(check_hip(hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(threads), params, 0, st), who));
  return check_launch(who);
}

// The whole BPTT recurrence in one persistent launch when the shape suits
// it (dG: [B*S, 4H], fully written); false in *done to fall back.
int lstm_bwd_persistent(const float* gates, const float* c, const float* tanh_c, const float* dY,
                        const float* W_hh, float* dG, int64_t B, int64_t S, int64_t H, hipStream_t st,
                        const char* who, bool* done) {
  *done = false;
  if (!persist_enabled() || B % 16 != 0 || H % 64 != 0 || 4 * H > kPersistBwdMaxG || (B * S) % 4 != 0 ||
      !aligned16(dG) || B * S > INT32_MAX)
    return CNHIP_OK;
  const int64_t nbt = B / 16, grid = nbt * (H / 16);
  const void* kern = reinterpret_cast<const void*>(&lstm_bwd_persist_kernel);
  if (!persist_fits(kern, grid, 512, who)) return CNHIP_OK;
  LstmBwdPersistArgs args{gates, c, tanh_c, dY, W_hh, dG, (int)B, (int)S, (int)H, (int)nbt, {}};
  TimingRec* rec = timing_slot(2.0 * B * 4 * H * H * (double)(S - 1));
  if (rec) (void)hipEventRecord(rec->start, st);
  CNHIP_TRY(persist_launch(kern, grid, 512, args, (int)nbt, st, who));
  if (rec) (void)hipEventRecord(rec->stop, st);
  *done = true;
  return CNHIP_OK;
}

// The whole forward recurrence (t = 0 .. S-1) in one persistent launch, when
// the shape suits it: returns false to fall back to the per-step launches.
int lstm_fwd_persistent(float* gates, const float* b, float* c, float* tanh_c, float* Y, const float* W_hh,
                        int64_t B, int64_t S, int64_t H, hipStream_t st, const char* who, bool* done) {
  *done = false;
  if (!persist_enabled() || B % 32 != 0 || H % 64 != 0 || H > kPersistMaxH || (B * S) % 4 != 0 ||
      !aligned16(Y) || !aligned16(W_hh) || B * S > INT32_MAX)
    return CNHIP_OK;
  const int64_t nbt = B / 32, grid = nbt * (H / kLstmUnits);
  const void* kern = reinterpret_cast<const void*>(&lstm_fwd_persist_kernel);
  if (!persist_fits(kern, grid, 256, who)) return CNHIP_OK;
  LstmFwdPersistArgs args{gates, b, c, tanh_c, Y, W_hh, (int)B, (int)S, (int)H, (int)nbt, {}};
  TimingRec* rec = timing_slot(2.0 * B * 4 * H * H * (double)(S - 1));
  if (rec) (void)hipEventRecord(rec->start, st);
  CNHIP_TRY(persist_launch(kern, grid, 256, args, (int)nbt, st, who));
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

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

extern "C" {

int cnhip_lstm_forward(const float* X, const float* W_ih, const float* W_hh, const float* b,
                       float* Y, float* gates, float* c, float* tanh_c, int64_t B, int64_t S,
                       int64_t I, int64_t H, cnhip_stream_t stream) {
  const char* who = "cnhip_lstm_forward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && b && Y && gates && c && tanh_c, "%s: NULL pointer", who);
  CNHIP_TRY(cnhip::persist_take_fault(who));
  hipStream_t st = as_stream(stream);
  const int64_t G = 4 * H, BS = B * S;
  CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, G, I, 1.f, X, BS, W_ih, I, 0.f, gates, BS, nullptr, 0, st, who));
  bool done = false;
  CNHIP_TRY(cnhip::lstm_fwd_persistent(gates, b, c, tanh_c, Y, W_hh, B, S, H, st, who, &done));
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
  const char* who = "cnhip_lstm_backward";
  CNHIP_TRY(cnhip::check_rnn(B, S, I, H, who));
  CNHIP_REQUIRE(X && W_ih && W_hh && Y && gates && c && tanh_c && dY && gW_ih && gW_hh && gb,
                "%s: NULL pointer", who);
  CNHIP_TRY(cnhip::persist_take_fault(who));
  hipStream_t st = as_stream(stream);
  const int64_t G = 4 * H, BS = B * S;
  cnhip::Workspace ws(st);
  CNHIP_TRY(ws.alloc((size_t)(BS * G + B * H) * sizeof(float), who));
  float* dG = static_cast<float*>(ws.p);
  float* dc = dG + BS * G;
  bool done = false;
  CNHIP_TRY(cnhip::lstm_bwd_persistent(gates, c, tanh_c, dY, W_hh, dG, B, S, H, st, who, &done));
  if (!done) {
    // t = S-1: dh = dY only; then per step one fused launch of
    // dh_t = dY_t + dG_{t+1} W_hh^T (lstm.cpp:244) and the cell backward
    hipLaunchKernelGGL(cnhip::lstm_cell_bwd_last_kernel, dim3(cnhip::cell_grid(B, H)), dim3(256), 0,
                       st, gates, c, tanh_c, dY, dc, dG, B, S, H);
    CNHIP_TRY(cnhip::check_launch(who));
    CNHIP_TRY(cnhip::lstm_bwd_steps<cnhip::LstmBwdCfgDefault>(gates, c, tanh_c, dY, W_hh, dc, dG, B, S,
                                                              H, st, who));
  }
  CNHIP_TRY(cnhip::gemm_f32(1, 0, I, G, BS, 1.f, X, BS, dG, BS, 0.f, gW_ih, I, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, H, G, B * (S - 1), 1.f, Y, BS, dG + B, BS, 0.f, gW_hh, H, nullptr,
                            0, st, who));
  CNHIP_TRY(cnhip::column_sum(dG, gb, BS, G, 0, st, who));
  if (dX)
    CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, I, G, 1.f, dG, BS, W_ih, I, 0.f, dX, BS, nullptr, 0, st, who));
  return CNHIP_OK;
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
