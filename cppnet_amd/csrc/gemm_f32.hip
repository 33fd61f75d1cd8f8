// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2f32), ColMajor operands.
//
//   C[M,N] = alpha * op(A)[M,K] * op(B)[K,N] + beta * C (+ bias[n]) (ReLU)
//
// One kernel template covers the three shapes a Linear layer needs
// (forward NN, weight-grad TN, input-grad NT; ref: matmul.cu:16-71,
// matmul_grad_weight.cu:14-69, matmul_grad_input.cu:14-68).  The reference
// computes one output per thread with atomicAdd accumulation; here a 256-
// thread block owns a 128x128 tile, each 64-wide wavefront a 64x64 sub-tile
// (2x2 MFMA 32x32 blocks, 64 accumulators per lane), K advances 16 at a time
// through double-buffered LDS, and no atomics are used: split-K partials go
// to a stream-ordered workspace and are summed by a second kernel in a fixed
// order, so results are deterministic.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "common.hpp"

namespace cnhip {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 16;
constexpr int NT = 256;          // threads per block (4 wavefronts)
constexpr int LDS_STRIDE = 132;  // floats per k-row of a staged tile (128 + 4 pad)
constexpr int TILE_FLOATS = BK * LDS_STRIDE;

struct GemmArgs {
  int64_t M, N, K;
  const float* A;
  int64_t lda;
  const float* B;
  int64_t ldb;
  float* C;
  int64_t ldc;
  float alpha, beta;
  const float* bias;
  int epilogue;
  int vec_ok;            // every ld % 4 == 0 and A, B 16-byte aligned
  int c_vec_ok;          // ldc % 4 == 0 and C 16-byte aligned
  int64_t k_per_split;   // multiple of BK
  float* partial;        // split-K workspace [splits][M*N], ColMajor ld=M; null = direct
};

// Staging of one operand tile (128 rows of the outer dim x 16 of K) into
// registers.  KCONTIG: X(r,k) = X[k + ld*r]  (else X[r + ld*k]).
// Each thread moves 2 float4 (512 float4 per tile).
template <bool KCONTIG>
__device__ __forceinline__ void load_tile(const float* __restrict__ X, int64_t ld, int64_t r0,
                                          int64_t k0, int64_t R, int64_t K, bool fast,
                                          f32x4 (&regs)[2]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int idx = tid + NT * p;
    int rr, kk;
    if (KCONTIG) {
      rr = idx >> 2;
      kk = (idx & 3) * 4;
    } else {
      kk = idx >> 5;
      rr = (idx & 31) * 4;
    }
    const int64_t r = r0 + rr, k = k0 + kk;
    if (fast) {
      const float* src = KCONTIG ? (X + k + ld * r) : (X + r + ld * k);
      regs[p] = *reinterpret_cast<const f32x4*>(src);
    } else {
      f32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t rj = KCONTIG ? r : r + j;
        const int64_t kj = KCONTIG ? k + j : k;
        float x = 0.f;
        if (rj < R && kj < K) x = KCONTIG ? X[kj + ld * rj] : X[rj + ld * kj];
        v[j] = x;
      }
      regs[p] = v;
    }
  }
}

// Writes a staged tile into LDS as [k][r] rows (r contiguous) so that an
// MFMA fragment read (lane -> r = lane%32, k = lane/32) is one conflict-free
// ds_read_b32.
template <bool KCONTIG>
__device__ __forceinline__ void store_tile(float* __restrict__ lds, const f32x4 (&regs)[2]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int idx = tid + NT * p;
    if (KCONTIG) {
      const int rr = idx >> 2, kk = (idx & 3) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) lds[(kk + j) * LDS_STRIDE + rr] = regs[p][j];
    } else {
      const int kk = idx >> 5, rr = (idx & 31) * 4;
      *reinterpret_cast<f32x4*>(lds + kk * LDS_STRIDE + rr) = regs[p];
    }
  }
}

__device__ __forceinline__ float epilogue_value(const GemmArgs& g, float acc, int64_t m, int64_t n) {
  float v = g.alpha * acc;
  if (g.beta != 0.f) v += g.beta * g.C[m + g.ldc * n];
  if (g.bias) v += g.bias[n];
  if (g.epilogue == CNHIP_EPI_RELU) v = fmaxf(v, 0.f);
  return v;
}

// Block -> output tile.  Hardware dispatch places consecutive block ids on
// consecutive XCDs (8 of them, each with its own L2); remap so that every XCD
// owns a contiguous range of tiles, then walk tiles in groups of 8 tile-rows
// so neighbouring blocks on one XCD share A rows and B columns in its L2.
__device__ __forceinline__ void tile_of_block(int nbm, int nbn, int& tm, int& tn) {
  const int total = nbm * nbn;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  const int base = total >> 3, rem = total & 7;
  const int tile = xcd * base + min(xcd, rem) + local;
  constexpr int GROUP = 8;
  const int per_group = GROUP * nbn;
  const int group = tile / per_group;
  const int first_m = group * GROUP;
  const int gsz = min(nbm - first_m, GROUP);
  const int in_group = tile - group * per_group;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

template <bool TA, bool TB>
__global__ void __launch_bounds__(NT, 2) gemm_f32_kernel(GemmArgs g) {
  __shared__ float lds_a[2][TILE_FLOATS];
  __shared__ float lds_b[2][TILE_FLOATS];

  const int nbm = (int)((g.M + BM - 1) / BM);
  const int nbn = (int)((g.N + BN - 1) / BN);
  int tm, tn;
  tile_of_block(nbm, nbn, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

  const int64_t k_begin = (int64_t)blockIdx.z * g.k_per_split;
  const int64_t k_end = min(g.K, k_begin + g.k_per_split);
  const int ntiles = (int)((k_end - k_begin + BK - 1) / BK);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, lhi = lane >> 5;

  const bool full_mn = (m0 + BM <= g.M) && (n0 + BN <= g.N);

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  f32x4 ra[2], rb[2];
  if (ntiles > 0) {
    const bool fast = g.vec_ok && full_mn && (k_begin + BK <= k_end);
    load_tile<TA>(g.A, g.lda, m0, k_begin, g.M, k_end, fast, ra);
    load_tile<!TB>(g.B, g.ldb, n0, k_begin, g.N, k_end, fast, rb);
    store_tile<TA>(lds_a[0], ra);
    store_tile<!TB>(lds_b[0], rb);
  }
  __syncthreads();

  for (int kt = 0; kt < ntiles; ++kt) {
    const int cur = kt & 1;
    const bool has_next = kt + 1 < ntiles;
    if (has_next) {
      const int64_t kn = k_begin + (int64_t)(kt + 1) * BK;
      const bool fast = g.vec_ok && full_mn && (kn + BK <= k_end);
      load_tile<TA>(g.A, g.lda, m0, kn, g.M, k_end, fast, ra);
      load_tile<!TB>(g.B, g.ldb, n0, kn, g.N, k_end, fast, rb);
    }
    const float* la = lds_a[cur] + wm * 64 + l32;
    const float* lb = lds_b[cur] + wn * 64 + l32;
#pragma unroll
    for (int s = 0; s < BK / 2; ++s) {
      const int k = 2 * s + lhi;
      const float a0 = la[k * LDS_STRIDE];
      const float a1 = la[k * LDS_STRIDE + 32];
      const float b0 = lb[k * LDS_STRIDE];
      const float b1 = lb[k * LDS_STRIDE + 32];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (has_next) {
      store_tile<TA>(lds_a[cur ^ 1], ra);
      store_tile<!TB>(lds_b[cur ^ 1], rb);
    }
    __syncthreads();
  }

  // Accumulator layout of v_mfma_f32_32x32x2f32: lane holds column
  // n = lane%32 and rows 8*(r/4) + 4*(lane/32) + r%4 for r = 0..15, i.e.
  // four runs of 4 consecutive rows -> one float4 each in ColMajor C.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 64 + j * 32 + l32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t m = m0 + wm * 64 + i * 32 + 8 * q + 4 * lhi;
        if (g.partial) {
          float* P = g.partial + (int64_t)blockIdx.z * g.M * g.N;
          if (n < g.N) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (m + e < g.M) P[(m + e) + g.M * n] = acc[i][j][4 * q + e];
          }
          continue;
        }
        if (n >= g.N) continue;
        if (g.c_vec_ok && m + 3 < g.M) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = epilogue_value(g, acc[i][j][4 * q + e], m + e, n);
          *reinterpret_cast<f32x4*>(g.C + m + g.ldc * n) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (m + e < g.M) g.C[(m + e) + g.ldc * n] = epilogue_value(g, acc[i][j][4 * q + e], m + e, n);
        }
      }
    }
  }
}

// Sums split-K partials in split order and applies the epilogue.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs g, int splits) {
  const int64_t total = g.M * g.N;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int z = 0; z < splits; ++z) s += g.partial[(int64_t)z * total + idx];
    const int64_t m = idx % g.M, n = idx / g.M;
    g.C[m + g.ldc * n] = epilogue_value(g, s, m, n);
  }
}

template <bool TA, bool TB>
void launch_gemm(const GemmArgs& g, int nblocks, int splits, hipStream_t st) {
  hipLaunchKernelGGL((gemm_f32_kernel<TA, TB>), dim3(nblocks, 1, splits), dim3(NT), 0, st, g);
}

// Per-launch event timing (cnhip_gemm_timing_*): a pool of event pairs
// reused across enable() calls.
struct TimingRec {
  hipEvent_t start, stop;
  double flops;
};
struct Timing {
  bool on = false;
  std::vector<TimingRec> pool;
  size_t used = 0;
};
thread_local Timing g_timing;

TimingRec* timing_slot(double flops) {
  Timing& t = g_timing;
  if (!t.on) return nullptr;
  if (t.used == t.pool.size()) {
    TimingRec r{};
    if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    t.pool.push_back(r);
  }
  TimingRec* r = &t.pool[t.used++];
  r->flops = flops;
  return r;
}

}  // namespace

int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who) {
  CNHIP_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative GEMM size (M=%lld N=%lld K=%lld)", who,
                (long long)M, (long long)N, (long long)K);
  CNHIP_REQUIRE(epilogue == CNHIP_EPI_NONE || epilogue == CNHIP_EPI_RELU, "%s: bad epilogue %d",
                who, epilogue);
  if (M == 0 || N == 0) return CNHIP_OK;
  CNHIP_REQUIRE(C != nullptr, "%s: C is NULL", who);
  CNHIP_REQUIRE(ldc >= M, "%s: ldc=%lld < M=%lld", who, (long long)ldc, (long long)M);
  if (K > 0) {
    CNHIP_REQUIRE(A && B, "%s: A or B is NULL", who);
    CNHIP_REQUIRE(lda >= (trans_a ? K : M), "%s: lda=%lld too small", who, (long long)lda);
    CNHIP_REQUIRE(ldb >= (trans_b ? N : K), "%s: ldb=%lld too small", who, (long long)ldb);
  }
  const int64_t nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
  CNHIP_REQUIRE(nbm * nbn < (int64_t)1 << 30, "%s: GEMM too large", who);

  GemmArgs g;
  g.M = M; g.N = N; g.K = K;
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc;
  g.alpha = alpha; g.beta = beta; g.bias = bias; g.epilogue = epilogue;
  g.vec_ok = (lda % 4 == 0) && (ldb % 4 == 0) && aligned16(A) && aligned16(B);
  g.c_vec_ok = (ldc % 4 == 0) && aligned16(C);
  g.partial = nullptr;

  // Split K when the output tiles alone cannot fill the 256 CUs.
  const int64_t tiles = nbm * nbn;
  int splits = 1;
  if (tiles < 256 && K >= 4 * BK) {
    int64_t want = (512 + tiles - 1) / tiles;
    int64_t max_by_k = K / (4 * BK);  // keep >= 4 K-tiles per split
    splits = (int)std::max<int64_t>(1, std::min<int64_t>({want, max_by_k, 64}));
  }
  int64_t kps = (K + splits - 1) / splits;
  kps = ((kps + BK - 1) / BK) * BK;
  if (kps == 0) kps = BK;
  splits = (int)((K + kps - 1) / kps);
  if (splits < 1) splits = 1;
  g.k_per_split = kps;

  if (splits > 1) {
    void* ws = nullptr;
    const size_t bytes = (size_t)splits * (size_t)M * (size_t)N * sizeof(float);
    CNHIP_TRY(check_hip(hipMallocAsync(&ws, bytes, st), who));
    g.partial = static_cast<float*>(ws);
  }

  const int nblocks = (int)tiles;
  TimingRec* rec = timing_slot(2.0 * (double)M * (double)N * (double)K);
  if (rec) (void)hipEventRecord(rec->start, st);
  if (!trans_a && !trans_b) launch_gemm<false, false>(g, nblocks, splits, st);
  else if (trans_a && !trans_b) launch_gemm<true, false>(g, nblocks, splits, st);
  else if (!trans_a && trans_b) launch_gemm<false, true>(g, nblocks, splits, st);
  else launch_gemm<true, true>(g, nblocks, splits, st);
  int status = check_launch(who);
  if (rec) (void)hipEventRecord(rec->stop, st);

  if (splits > 1) {
    if (status == CNHIP_OK) {
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3(elementwise_grid(M * N, 256)), dim3(256), 0, st,
                         g, splits);
      status = check_launch(who);
    }
    int st2 = check_hip(hipFreeAsync(g.partial, st), who);
    if (status == CNHIP_OK) status = st2;
  }
  return status;
}

}  // namespace cnhip

extern "C" int cnhip_gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                              float alpha, const float* A, int64_t lda, const float* B,
                              int64_t ldb, float beta, float* C, int64_t ldc, const float* bias,
                              int epilogue, cnhip_stream_t stream) {
  return cnhip::gemm_f32(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias,
                         epilogue, cnhip::as_stream(stream), "cnhip_gemm_f32");
}

extern "C" int cnhip_gemm_timing_enable(int on) {
  cnhip::g_timing.on = on != 0;
  cnhip::g_timing.used = 0;
  return CNHIP_OK;
}

extern "C" int cnhip_gemm_timing_read(int64_t* launches, double* total_ms, double* total_flops) {
  CNHIP_REQUIRE(launches && total_ms && total_flops, "cnhip_gemm_timing_read: NULL argument");
  cnhip::Timing& t = cnhip::g_timing;
  double ms = 0.0, fl = 0.0;
  for (size_t i = 0; i < t.used; ++i) {
    float e = 0.f;
    CNHIP_TRY(cnhip::check_hip(hipEventSynchronize(t.pool[i].stop), "cnhip_gemm_timing_read"));
    CNHIP_TRY(cnhip::check_hip(hipEventElapsedTime(&e, t.pool[i].start, t.pool[i].stop),
                               "cnhip_gemm_timing_read"));
    ms += e;
    fl += t.pool[i].flops;
  }
  *launches = (int64_t)t.used;
  *total_ms = ms;
  *total_flops = fl;
  return CNHIP_OK;
}
