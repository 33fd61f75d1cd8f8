// Kernels and entry points of the transformer rows: MultiHeadAttention,
// Embedding, BatchNorm, GELU, MeanPool1D and the residual add.
//
// ref: attention.cpp:60-587 (MHA cpu-eigen semantics), attention_scores.cu
// (reference softmax kernels, which index row-major into ColMajor data),
// embedding.cpp:33-185 / embedding_*.cu, batch_norm.cpp:204-401 /
// batch_norm_*.cu, mean_pool1d.cpp:24-150 / mean_pool1d.cu, residual.cpp /
// elementwise.cu (op 0 = add).  GELU has no reference implementation.
//
// Attention layout.  Activations are ColMajor [B, S, D], i.e. [B*S, D]
// matrices with row b + B*s: the projections and every weight gradient are
// single GEMMs over all B*S rows.  The per-sample products (scores, context
// and their gradients) need each sample's [S, D] block contiguous, so the
// projected Q, K, V are transposed once into a per-sample layout
// (s + S*d + S*D*b) by a tiled LDS transpose, and the batched MFMA GEMM runs
// over the B samples.  Attention weights are kept as A^T per sample (row i of
// A is contiguous), so the row softmax and its Jacobian are wave64 reductions
// over contiguous memory.
//
// Row order by sample.  The [B*S, D] activations may instead hold row
// s + S*b (CNHIP_ROWS_BY_SAMPLE): sample b's [S, D] block is then rows
// S*b .. S*b + S - 1 of the matrix, an ordinary strided operand (leading
// dimension B*S, batch stride S), and the attention products read and write
// it in place with no transposes.  Everything row-wise (projections, FFN,
// BatchNorm, GELU, adds) is indifferent to the row order; Embedding,
// MeanPool1D and attention take it as an argument.  A model that runs
// Embedding -> ... -> MeanPool1D uses it end to end: the order never shows
// outside.
#include <hip/hip_runtime.h>

#include <cmath>

#include "act_math.hpp"
#include "common.hpp"

namespace cnhip {

int gemm_f32(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
             int64_t ldc, const float* bias, int epilogue, hipStream_t st, const char* who);
int gemm_f32_batched(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                     const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                     int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c,
                     int64_t batches, const float* bias, int epilogue, hipStream_t st,
                     const char* who);
int gemm_f32_act(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const float* A,
                 int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc, const float* bias,
                 int epilogue, const float* aux_in, float* aux_out, int64_t ld_aux, hipStream_t st,
                 const char* who);
int gemm_f32_core(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                  const float* A, int64_t lda, int64_t stride_a, const float* B, int64_t ldb,
                  int64_t stride_b, float beta, float* C, int64_t ldc, int64_t stride_c,
                  int64_t batches, const float* bias, int epilogue, const float* aux_in,
                  float* aux_out, int64_t ld_aux, hipStream_t st, const char* who);
constexpr int EPI_ADD = 5;  // GEMM epilogue C = v + aux_in (gemm_f32.hip)

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- transpose
// ColMajor in [R, C] -> out [C, R]: out[c + C*r] = in[r + R*c], TR x TC tiles
// through LDS (a column of the tile padded to TR + 1 floats, so both the
// r-contiguous writes and the c-contiguous reads of LDS are conflict-free).
// VEC (R, C multiples of 4, 16-byte aligned pointers): global loads are
// float4s along r and stores float4s along c.  The tile is shaped to R: the
// per-sample relayouts of attention have R = batch (32), where a 64 x 64
// tile would leave half its rows empty.
constexpr int TT = 64;  // token tile of the embedding kernels

template <int TR, int TC, bool VEC>
__global__ void __launch_bounds__(256) transpose_kernel(const float* __restrict__ in,
                                                        float* __restrict__ out, int64_t R,
                                                        int64_t C) {
  __shared__ float tile[TC][TR + 1];
  const int64_t r0 = (int64_t)blockIdx.x * TR, c0 = (int64_t)blockIdx.y * TC;
  const int t = threadIdx.x;
  if (VEC) {
    constexpr int R4 = TR / 4, C4 = TC / 4;
    for (int i = t; i < R4 * TC; i += 256) {
      const int r = (i % R4) * 4, c = i / R4;
      if (r0 + r < R && c0 + c < C) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(in + (r0 + r) + R * (c0 + c));
#pragma unroll
        for (int k = 0; k < 4; ++k) tile[c][r + k] = v[k];
      }
    }
    __syncthreads();
    for (int i = t; i < C4 * TR; i += 256) {
      const int c = (i % C4) * 4, r = i / C4;
      if (r0 + r < R && c0 + c < C) {
        f32x4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = tile[c + k][r];
        *reinterpret_cast<f32x4*>(out + (c0 + c) + C * (r0 + r)) = v;
      }
    }
  } else {
    for (int i = t; i < TR * TC; i += 256) {
      const int r = i % TR, c = i / TR;
      if (r0 + r < R && c0 + c < C) tile[c][r] = in[(r0 + r) + R * (c0 + c)];
    }
    __syncthreads();
    for (int i = t; i < TC * TR; i += 256) {
      const int c = i % TC, r = i / TC;
      if (r0 + r < R && c0 + c < C) out[(c0 + c) + C * (r0 + r)] = tile[c][r];
    }
  }
}

template <int TR, int TC>
int transpose_t(const float* in, float* out, int64_t R, int64_t C, hipStream_t st, const char* who) {
  CNHIP_REQUIRE((R + TR - 1) / TR < (1ll << 31) && (C + TC - 1) / TC <= 65535,
                "%s: transpose %lld x %lld too large", who, (long long)R, (long long)C);
  const dim3 grid((unsigned)((R + TR - 1) / TR), (unsigned)((C + TC - 1) / TC));
  const bool vec = R % 4 == 0 && C % 4 == 0 && aligned16(in) && aligned16(out);
  if (vec)
    hipLaunchKernelGGL((transpose_kernel<TR, TC, true>), grid, dim3(256), 0, st, in, out, R, C);
  else
    hipLaunchKernelGGL((transpose_kernel<TR, TC, false>), grid, dim3(256), 0, st, in, out, R, C);
  return check_launch(who);
}

int transpose(const float* in, float* out, int64_t R, int64_t C, hipStream_t st, const char* who) {
  HbmTimer timer("transpose_kernel", 8.0 * (double)R * (double)C, st);
  if (R <= 16) return transpose_t<16, 256>(in, out, R, C, st, who);
  if (R <= 32) return transpose_t<32, 128>(in, out, R, C, st, who);
  if (C <= 32) return transpose_t<128, 32>(in, out, R, C, st, who);
  return transpose_t<64, 64>(in, out, R, C, st, who);
}

// ---------------------------------------------------------------- row softmax
// x / y: rows of length L contiguous (row r at r*L); one wave64 per row.
// attention.cpp:191-205: max, exp(x - max), sum, divide.
__global__ void __launch_bounds__(256) softmax_rows_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, int64_t rows,
                                                           int64_t L) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = x + r * L;
  float* yr = y + r * L;
  float mx = -INFINITY;
  for (int64_t j = lane; j < L; j += 64) mx = fmaxf(mx, xr[j]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = 0.f;
  for (int64_t j = lane; j < L; j += 64) {
    const float e = expf(xr[j] - mx);
    yr[j] = e;
    sum += e;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  for (int64_t j = lane; j < L; j += 64) yr[j] = yr[j] / sum;
}

// attention.cpp:541-551: g = (A * (dA - sum_j dA A)) * scale
__global__ void __launch_bounds__(256) softmax_rows_bwd_kernel(const float* __restrict__ A,
                                                               const float* __restrict__ dA,
                                                               float* __restrict__ g, int64_t rows,
                                                               int64_t L, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* ar = A + r * L;
  const float* dr = dA + r * L;
  float dot = 0.f;
  for (int64_t j = lane; j < L; j += 64) dot += dr[j] * ar[j];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
  for (int64_t j = lane; j < L; j += 64) g[r * L + j] = (ar[j] * (dr[j] - dot)) * scale;
}

// softmax_rows_kernel / softmax_rows_bwd_kernel for L <= 64 * PER: the row
// stays in registers (lane holds j = lane, lane + 64, ..), so x (A, dA) is
// read once and y (g) written once; the same operations in the same order,
// so the results are identical to the looping kernels.
template <int PER>
__global__ void __launch_bounds__(256) softmax_rows_reg_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y, int64_t rows,
                                                               int64_t L) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = x + r * L;
  float* yr = y + r * L;
  float v[PER];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t j = lane + 64 * i;
    v[i] = j < L ? xr[j] : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (lane + 64 * i < L) {
      v[i] = expf(v[i] - mx);
      sum += v[i];
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t j = lane + 64 * i;
    if (j < L) yr[j] = v[i] / sum;
  }
}

template <int PER>
__global__ void __launch_bounds__(256) softmax_rows_bwd_reg_kernel(const float* __restrict__ A,
                                                                   const float* __restrict__ dA,
                                                                   float* __restrict__ g, int64_t rows,
                                                                   int64_t L, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* ar = A + r * L;
  const float* dr = dA + r * L;
  float a[PER], d[PER];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t j = lane + 64 * i;
    a[i] = j < L ? ar[j] : 0.f;
    d[i] = j < L ? dr[j] : 0.f;
    if (j < L) dot += d[i] * a[i];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t j = lane + 64 * i;
    if (j < L) g[r * L + j] = (a[i] * (d[i] - dot)) * scale;
  }
}

int softmax_rows(const float* x, float* y, int64_t rows, int64_t L, hipStream_t st, const char* who) {
  HbmTimer timer("softmax_rows_kernel", 8.0 * (double)rows * (double)L, st);
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (L <= 256)
    hipLaunchKernelGGL(softmax_rows_reg_kernel<4>, grid, dim3(256), 0, st, x, y, rows, L);
  else if (L <= 1024)
    hipLaunchKernelGGL(softmax_rows_reg_kernel<16>, grid, dim3(256), 0, st, x, y, rows, L);
  else
    hipLaunchKernelGGL(softmax_rows_kernel, grid, dim3(256), 0, st, x, y, rows, L);
  return check_launch(who);
}

int softmax_rows_bwd(const float* A, const float* dA, float* g, int64_t rows, int64_t L, float scale,
                     hipStream_t st, const char* who) {
  HbmTimer timer("softmax_rows_bwd_kernel", 12.0 * (double)rows * (double)L, st);
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (L <= 256)
    hipLaunchKernelGGL(softmax_rows_bwd_reg_kernel<4>, grid, dim3(256), 0, st, A, dA, g, rows, L, scale);
  else if (L <= 1024)
    hipLaunchKernelGGL(softmax_rows_bwd_reg_kernel<16>, grid, dim3(256), 0, st, A, dA, g, rows, L, scale);
  else
    hipLaunchKernelGGL(softmax_rows_bwd_kernel, grid, dim3(256), 0, st, A, dA, g, rows, L, scale);
  return check_launch(who);
}

// ---------------------------------------------------------------- embedding
// Weights are kept token-major, Wt[d + D*v] (the reference's ColMajor [V, D]
// transposed), so one token's row is contiguous.  out[p + BS*d] with
// p = b + B*s (or s + S*b by sample): a 64-token x 64-feature tile is read
// along d and written along p through LDS.  Out-of-range ids produce zeros
// and are counted.
__global__ void __launch_bounds__(256) embedding_fwd_kernel(const int32_t* __restrict__ ids,
                                                            const float* __restrict__ Wt,
                                                            float* __restrict__ out, int64_t B,
                                                            int64_t S, int64_t V, int64_t D,
                                                            int by_sample,
                                                            int32_t* __restrict__ oob) {
  const int64_t BS = B * S;
  __shared__ float tile[TT][TT + 1];
  __shared__ int32_t tok[TT];
  const int64_t p0 = (int64_t)blockIdx.x * TT, d0 = (int64_t)blockIdx.y * TT;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  if (threadIdx.x < TT) {
    const int64_t p = p0 + threadIdx.x;
    // ids are ColMajor [B, S]: position (b, s) at b + B*s
    int32_t id = p < BS ? ids[by_sample ? (p % S) * B + p / S : p] : 0;
    if (p < BS && (id < 0 || id >= V)) {
      if (oob && blockIdx.y == 0) atomicAdd(oob, 1);
      id = -1;
    }
    tok[threadIdx.x] = id;
  }
  __syncthreads();
  {
    // token j = ty + 4 jj, feature tx: contiguous along d; all TT / 4 loads
    // of a thread in flight before its LDS stores
    float v[TT / 4];
    const int64_t d = d0 + tx;
#pragma unroll
    for (int jj = 0; jj < TT / 4; ++jj) {
      const int32_t id = tok[ty + 4 * jj];
      v[jj] = (d < D && id >= 0) ? Wt[d + D * (int64_t)id] : 0.f;
    }
#pragma unroll
    for (int jj = 0; jj < TT / 4; ++jj) tile[ty + 4 * jj][tx] = v[jj];
  }
  __syncthreads();
  for (int j = ty; j < TT; j += 4) {  // feature j, token tx: contiguous along p
    const int64_t p = p0 + tx, d = d0 + j;
    if (p < BS && d < D) out[p + BS * d] = tile[tx][j];
  }
}

// Deterministic scatter-add: bucket the positions by token id (counting sort,
// keys ascending inside a bucket), then every token row sums its bucket's
// gradient rows in key order.
__global__ void __launch_bounds__(256) emb_count_kernel(const int32_t* __restrict__ ids,
                                                        int32_t* __restrict__ counts, int64_t BS,
                                                        int64_t V) {
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < BS;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int32_t id = ids[p];
    if (id >= 0 && id < V) atomicAdd(&counts[id], 1);
  }
}

// exclusive scan of counts[V] into offsets[V+1] (one block, fixed order)
__global__ void __launch_bounds__(1024) emb_scan_kernel(const int32_t* __restrict__ counts,
                                                        int32_t* __restrict__ offsets, int64_t V) {
  __shared__ int32_t wave_total[16];
  const int64_t per = (V + 1023) / 1024;
  const int64_t lo = threadIdx.x * per, hi = min(V, lo + per);
  // up to 8 counts per thread (V <= 8192) are loaded together into
  // registers: a loop of dependent loads waited for each one in turn
  constexpr int R = 8;
  int32_t c[R];
  int32_t s = 0;
  if (per <= R) {
#pragma unroll
    for (int i = 0; i < R; ++i) c[i] = lo + i < hi ? counts[lo + i] : 0;
#pragma unroll
    for (int i = 0; i < R; ++i) s += c[i];
  } else {
    for (int64_t v = lo; v < hi; ++v) s += counts[v];
  }
  // exclusive scan of the 1024 per-thread counts: an inclusive shuffle scan
  // within each wave, then the 16 wave totals (integer sums: exact in any order)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int32_t x = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_total[wave] = x;
  __syncthreads();
  int32_t before = 0;
  for (int w = 0; w < wave; ++w) before += wave_total[w];
  int32_t run = before + x - s;
  if (threadIdx.x == 1023) offsets[V] = run + s;
  if (per <= R) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (lo + i < hi) offsets[lo + i] = run;
      run += c[i];
    }
  } else {
    for (int64_t v = lo; v < hi; ++v) {
      offsets[v] = run;
      run += counts[v];
    }
  }
}

// Bucket entries are keys b*S + s (sample-major), the order in which the
// reference's cpu-eigen loop (embedding.cpp:161-168: n outer, s inner) adds the
// gradient rows; position p = b + B*s of the ColMajor [B, S] ids.
__global__ void __launch_bounds__(256) emb_fill_kernel(const int32_t* __restrict__ ids,
                                                       const int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ cursor,
                                                       int32_t* __restrict__ keys, int64_t B,
                                                       int64_t S, int64_t V) {
  const int64_t BS = B * S;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < BS;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int32_t id = ids[p];
    if (id >= 0 && id < V)
      keys[offsets[id] + atomicAdd(&cursor[id], 1)] = (int32_t)((p % B) * S + p / B);
  }
}

// The whole bucketing above (count, scan, fill, per-bucket sort) in one
// block for up to 8192 tokens over up to 8192 ids, with the counters, the
// offsets and the keys in LDS: the four launches and the counters' clearing
// it replaces each cost a launch for a few microseconds of work.  Same
// counts, offsets and per-bucket key order, so the same outputs.
constexpr int kEmbSmall = 8192;

__global__ void __launch_bounds__(1024) emb_bucket_small_kernel(const int32_t* __restrict__ ids,
                                                                int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ pos, int B, int S, int V) {
  __shared__ int32_t cnt[kEmbSmall];  // counts, then the fill cursors
  __shared__ int32_t off[kEmbSmall + 1];
  __shared__ int32_t key[kEmbSmall];
  __shared__ int32_t wave_total[16];
  constexpr int R = kEmbSmall / 1024;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, BS = B * S;
  for (int v = tid; v < V; v += 1024) cnt[v] = 0;
  int32_t id[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int p = tid + 1024 * i;
    id[i] = p < BS ? ids[p] : -1;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (id[i] >= 0 && id[i] < V) atomicAdd(&cnt[id[i]], 1);
  __syncthreads();
  // exclusive scan: thread t owns ids 8 t .. 8 t + 7
  int32_t c[R];
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int v = R * tid + i;
    c[i] = v < V ? cnt[v] : 0;
    s += c[i];
  }
  int32_t x = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_total[wave] = x;
  __syncthreads();
  int32_t run = x - s;
  for (int w = 0; w < wave; ++w) run += wave_total[w];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int v = R * tid + i;
    if (v < V) off[v] = cnt[v] = run;
    run += c[i];
  }
  if (tid == 1023) off[V] = run;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (id[i] >= 0 && id[i] < V) {
      const int p = tid + 1024 * i;
      key[atomicAdd(&cnt[id[i]], 1)] = (p % B) * S + p / B;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int v = R * tid + i;
    if (v >= V) break;
    const int lo = off[v], hi = off[v + 1];
    for (int a = lo + 1; a < hi; ++a) {
      const int32_t k = key[a];
      int b = a - 1;
      while (b >= lo && key[b] > k) {
        key[b + 1] = key[b];
        --b;
      }
      key[b + 1] = k;
    }
  }
  __syncthreads();
  for (int v = tid; v <= V; v += 1024) offsets[v] = off[v];
  const int total = off[V];
  for (int j = tid; j < total; j += 1024) pos[j] = key[j];
}

// Sort each bucket ascending (buckets are tiny: BS/V entries on average).
__global__ void __launch_bounds__(256) emb_sort_kernel(const int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ pos, int64_t V) {
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < V;
       v += (int64_t)gridDim.x * blockDim.x) {
    const int32_t lo = offsets[v], hi = offsets[v + 1];
    for (int32_t i = lo + 1; i < hi; ++i) {
      const int32_t key = pos[i];
      int32_t j = i - 1;
      while (j >= lo && pos[j] > key) {
        pos[j + 1] = pos[j];
        --j;
      }
      pos[j + 1] = key;
    }
  }
}

// gWt[d + D*v] = sum over the bucket, in key order, of dYt[d + D*p]
// (dYt = dY transposed, one position's gradient row contiguous; key b*S + s
// is row p = b + B*s, or p = key by sample); empty buckets write zeros.
__global__ void __launch_bounds__(128) emb_sum_kernel(const int32_t* __restrict__ offsets,
                                                      const int32_t* __restrict__ keys,
                                                      const float* __restrict__ dYt,
                                                      float* __restrict__ gWt, int64_t B,
                                                      int64_t S, int64_t D, int by_sample) {
  const int64_t v = blockIdx.x;
  const int32_t lo = offsets[v], hi = offsets[v + 1];
  // four features per thread, so each bucket entry's key is read once and
  // four independent loads are in flight per entry
  constexpr int U = 4;
  for (int64_t d0 = threadIdx.x; d0 < D; d0 += U * blockDim.x) {
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) s[u] = 0.f;
    for (int32_t i = lo; i < hi; ++i) {
      const int64_t key = keys[i];
      const float* src = dYt + D * (by_sample ? key : key / S + B * (key % S));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t d = d0 + (int64_t)u * blockDim.x;
        if (d < D) s[u] += src[d];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t d = d0 + (int64_t)u * blockDim.x;
      if (d < D) gWt[d + D * v] = s[u];
    }
  }
}

// emb_sum_kernel when D % 4 == 0: a wave per token, lane l summing the
// float4 columns l, l + 64 (two in flight per bucket entry); each element's
// sum runs over the bucket in key order, as there
__global__ void __launch_bounds__(256) emb_sum_vec_kernel(const int32_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ keys,
                                                          const float* __restrict__ dYt,
                                                          float* __restrict__ gWt, int B, int S, int D,
                                                          int V, int by_sample) {
  const int lane = threadIdx.x & 63;
  const int v = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (v >= V) return;
  const int32_t lo = offsets[v], hi = offsets[v + 1];
  const int D4 = D / 4;
  f32x4* out = reinterpret_cast<f32x4*>(gWt + (int64_t)D * v);
  for (int c0 = lane; c0 < D4; c0 += 128) {
    const int c1 = c0 + 64;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
    for (int32_t i = lo; i < hi; ++i) {
      const int key = keys[i];
      const int64_t row = by_sample ? key : key / S + (int64_t)B * (key % S);
      const f32x4* src = reinterpret_cast<const f32x4*>(dYt + (int64_t)D * row);
      s0 += src[c0];
      if (c1 < D4) s1 += src[c1];
    }
    out[c0] = s0;
    if (c1 < D4) out[c1] = s1;
  }
}

// ---------------------------------------------------------------- BatchNorm
// One block per feature; x column f is contiguous ([N, F] ColMajor).  Sums
// are block reductions in a fixed order.
constexpr int BNT = 256;

__device__ float bn_block_sum(float v, float* sm) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if (lane == 0) sm[w] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < BNT / 64; ++i) r += sm[i];
  return r;  // every thread
}

// sqrt(var + eps) from var as stored: one rounding for var = sum / N, one
// for the add.  Contracting the two into an fma would give the forward a
// divisor the backward (which reads the stored var) cannot reproduce.
__device__ __forceinline__ float bn_den(float var, float eps) {
#pragma clang fp contract(off)
  return sqrtf(var + eps);
}
// xhat = (x - mean) / den, the subtraction never fused with the product that
// formed mean (the backward reads mean as stored)
__device__ __forceinline__ float bn_xhat(float x, float mean, float den) {
#pragma clang fp contract(off)
  return (x - mean) / den;
}

// batch_norm.cpp:282-318 (training)
__global__ void __launch_bounds__(BNT) bn_fwd_kernel(const float* __restrict__ x,
                                                     float* __restrict__ y,
                                                     float* __restrict__ xhat,
                                                     const float* __restrict__ gamma,
                                                     const float* __restrict__ beta,
                                                     float* __restrict__ rmean,
                                                     float* __restrict__ rvar,
                                                     float* __restrict__ bmean,
                                                     float* __restrict__ bvar, int64_t N,
                                                     float momentum, float eps) {
  __shared__ float sm[BNT / 64];
  const int64_t f = blockIdx.x;
  const float* xc = x + N * f;
  const float inv_batch = 1.0f / (float)N;
  float s = 0.f;
  for (int64_t n = threadIdx.x; n < N; n += BNT) s += xc[n];
  const float mean = bn_block_sum(s, sm) * inv_batch;
  float s2 = 0.f;
  for (int64_t n = threadIdx.x; n < N; n += BNT) {
    const float diff = xc[n] - mean;
    s2 += diff * diff;
  }
  const float var = bn_block_sum(s2, sm) * inv_batch;
  const float den = bn_den(var, eps);
  const float g = gamma[f], b = beta[f];
  for (int64_t n = threadIdx.x; n < N; n += BNT) {
    const float xh = bn_xhat(xc[n], mean, den);
    if (xhat) xhat[n + N * f] = xh;
    y[n + N * f] = g * xh + b;
  }
  if (threadIdx.x == 0) {
    bmean[f] = mean;
    bvar[f] = var;
    rmean[f] = (1.0f - momentum) * rmean[f] + momentum * mean;
    rvar[f] = (1.0f - momentum) * rvar[f] + momentum * var;
  }
}

// bn_fwd_kernel for N <= BNT * PER: the column is read once into registers
// (thread t holds rows t, t + BNT, ..); same sums in the same order as the
// looping kernel, so the results are identical.
template <int PER>
__global__ void __launch_bounds__(BNT) bn_fwd_reg_kernel(const float* __restrict__ x,
                                                         float* __restrict__ y,
                                                         float* __restrict__ xhat,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta,
                                                         float* __restrict__ rmean,
                                                         float* __restrict__ rvar,
                                                         float* __restrict__ bmean,
                                                         float* __restrict__ bvar, int64_t N,
                                                         float momentum, float eps) {
  __shared__ float sm[BNT / 64];
  const int64_t f = blockIdx.x;
  const float* xc = x + N * f;
  const float inv_batch = 1.0f / (float)N;
  float v[PER];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t n = threadIdx.x + (int64_t)BNT * i;
    v[i] = n < N ? xc[n] : 0.f;
    if (n < N) s += v[i];
  }
  const float mean = bn_block_sum(s, sm) * inv_batch;
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t n = threadIdx.x + (int64_t)BNT * i;
    if (n < N) {
      const float diff = v[i] - mean;
      s2 += diff * diff;
    }
  }
  const float var = bn_block_sum(s2, sm) * inv_batch;
  const float den = bn_den(var, eps);
  const float g = gamma[f], b = beta[f];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t n = threadIdx.x + (int64_t)BNT * i;
    if (n < N) {
      const float xh = bn_xhat(v[i], mean, den);
      if (xhat) xhat[n + N * f] = xh;
      y[n + N * f] = g * xh + b;
    }
  }
  if (threadIdx.x == 0) {
    bmean[f] = mean;
    bvar[f] = var;
    rmean[f] = (1.0f - momentum) * rmean[f] + momentum * mean;
    rvar[f] = (1.0f - momentum) * rvar[f] + momentum * var;
  }
}

// eval mode (batch_norm.cpp:320-327): running statistics
__global__ void __launch_bounds__(256) bn_eval_kernel(const float* __restrict__ x,
                                                      float* __restrict__ y,
                                                      float* __restrict__ xhat,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ beta,
                                                      const float* __restrict__ rmean,
                                                      const float* __restrict__ rvar, int64_t N,
                                                      int64_t F, float eps) {
  const int64_t total = N * F;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = i / N;
    const float xh = (x[i] - rmean[f]) / sqrtf(rvar[f] + eps);
    xhat[i] = xh;
    y[i] = gamma[f] * xh + beta[f];
  }
}

// batch_norm.cpp:353-385
__global__ void __launch_bounds__(BNT) bn_bwd_kernel(const float* __restrict__ dY,
                                                     const float* __restrict__ x,
                                                     const float* __restrict__ xhat,
                                                     const float* __restrict__ gamma,
                                                     const float* __restrict__ bmean,
                                                     const float* __restrict__ bvar,
                                                     float* __restrict__ ggamma,
                                                     float* __restrict__ gbeta,
                                                     float* __restrict__ dX, int64_t N, float eps) {
  __shared__ float sm[BNT / 64];
  const int64_t f = blockIdx.x;
  const float* dyc = dY + N * f;
  const float* xc = x + N * f;
  const float* xhc = xhat ? xhat + N * f : nullptr;
  const float g = gamma[f], mean = bmean[f];
  const float den = bn_den(bvar[f], eps);  // the forward's divisor: xhat recomputed bit for bit
  const float inv_std = 1.0f / den;
  const float inv_batch = 1.0f / (float)N;
  float sgg = 0.f, sgb = 0.f, sdv = 0.f, sdm = 0.f;
  for (int64_t n = threadIdx.x; n < N; n += BNT) {
    const float dy = dyc[n];
    sgg += dy * (xhc ? xhc[n] : bn_xhat(xc[n], mean, den));
    sgb += dy;
    const float dxh = dy * g;
    const float xmu = xc[n] - mean;
    sdv += dxh * xmu * (-0.5f) * inv_std * inv_std * inv_std;
    sdm += dxh * (-inv_std);
  }
  const float tgg = bn_block_sum(sgg, sm);
  const float tgb = bn_block_sum(sgb, sm);
  const float dvar = bn_block_sum(sdv, sm);
  const float dmean = bn_block_sum(sdm, sm);
  if (threadIdx.x == 0) {
    ggamma[f] = tgg;
    gbeta[f] = tgb;
  }
  for (int64_t n = threadIdx.x; n < N; n += BNT) {
    const float dxh = dyc[n] * g;
    const float xmu = xc[n] - mean;
    dX[n + N * f] = dxh * inv_std + dvar * 2.0f * xmu * inv_batch + dmean * inv_batch;
  }
}

// bn_bwd_kernel for N <= BNT * PER: dY, x and xhat read once into registers,
// the four column sums reduced together; same arithmetic and order.
template <int PER>
__global__ void __launch_bounds__(BNT) bn_bwd_reg_kernel(const float* __restrict__ dY,
                                                         const float* __restrict__ x,
                                                         const float* __restrict__ xhat,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ bmean,
                                                         const float* __restrict__ bvar,
                                                         float* __restrict__ ggamma,
                                                         float* __restrict__ gbeta,
                                                         float* __restrict__ dX, int64_t N,
                                                         float eps) {
  __shared__ float sm[4][BNT / 64];
  const int64_t f = blockIdx.x;
  const float* dyc = dY + N * f;
  const float* xc = x + N * f;
  const float* xhc = xhat ? xhat + N * f : nullptr;
  const float g = gamma[f], mean = bmean[f];
  const float den = bn_den(bvar[f], eps);  // the forward's divisor: xhat recomputed bit for bit
  const float inv_std = 1.0f / den;
  const float inv_batch = 1.0f / (float)N;
  float dy[PER], xm[PER];
  float sgg = 0.f, sgb = 0.f, sdv = 0.f, sdm = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t n = threadIdx.x + (int64_t)BNT * i;
    dy[i] = 0.f;
    xm[i] = 0.f;
    if (n < N) {
      dy[i] = dyc[n];
      xm[i] = xc[n] - mean;
      sgg += dy[i] * (xhc ? xhc[n] : bn_xhat(xc[n], mean, den));
      sgb += dy[i];
      const float dxh = dy[i] * g;
      sdv += dxh * xm[i] * (-0.5f) * inv_std * inv_std * inv_std;
      sdm += dxh * (-inv_std);
    }
  }
  // the four block sums of bn_block_sum, in one exchange
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sgg += __shfl_xor(sgg, off, 64);
    sgb += __shfl_xor(sgb, off, 64);
    sdv += __shfl_xor(sdv, off, 64);
    sdm += __shfl_xor(sdm, off, 64);
  }
  if (lane == 0) {
    sm[0][w] = sgg;
    sm[1][w] = sgb;
    sm[2][w] = sdv;
    sm[3][w] = sdm;
  }
  __syncthreads();
  float tgg = 0.f, tgb = 0.f, dvar = 0.f, dmean = 0.f;
#pragma unroll
  for (int i = 0; i < BNT / 64; ++i) {
    tgg += sm[0][i];
    tgb += sm[1][i];
    dvar += sm[2][i];
    dmean += sm[3][i];
  }
  if (threadIdx.x == 0) {
    ggamma[f] = tgg;
    gbeta[f] = tgb;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t n = threadIdx.x + (int64_t)BNT * i;
    if (n < N)
      dX[n + N * f] = dy[i] * g * inv_std + dvar * 2.0f * xm[i] * inv_batch + dmean * inv_batch;
  }
}

// ---------------------------------------------------------------- GELU / pool / add
// BatchNorm for columns of N = 4k rows (16-byte aligned): T threads per
// feature, thread t holds float4s t, t + T, .. of the column in registers
// (V4 of them), so every element is read once and written once.  Columns of
// up to 8192 rows take 512 threads x 4 float4s: every column of a [8192, 512]
// batch is in flight at once with a quarter of the waves a 1024 x 2 shape
// dispatches (measured on MI355X at [8192, 512]: forward 7.9 -> 7.0 us,
// backward 12.4 -> 9.7 us).  Sums: per-thread float4 partials, then waves,
// then the T/64 wave sums in order; fixed for a given launch shape.
template <int T>
__device__ __forceinline__ void wave_sums(float* v, int k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    for (int j = 0; j < k; ++j) v[j] += __shfl_xor(v[j], off, 64);
}

template <int T, int V4>
__global__ void __launch_bounds__(T) bn_fwd_vec_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y,
                                                       float* __restrict__ xhat,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta,
                                                       float* __restrict__ rmean,
                                                       float* __restrict__ rvar,
                                                       float* __restrict__ bmean,
                                                       float* __restrict__ bvar, int64_t N,
                                                       float momentum, float eps) {
  __shared__ float sm[2][T / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t f = blockIdx.x, n4 = N >> 2;
  const f32x4* xc = reinterpret_cast<const f32x4*>(x + N * f);
  const float inv_batch = 1.0f / (float)N;
  f32x4 v[V4];
  float s[1] = {0.f};
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    const int64_t q = threadIdx.x + (int64_t)T * i;
    v[i] = q < n4 ? xc[q] : f32x4{0.f, 0.f, 0.f, 0.f};
    s[0] += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
  }
  wave_sums<T>(s, 1);
  if (lane == 0) sm[0][w] = s[0];
  __syncthreads();
  float mean = 0.f;
#pragma unroll
  for (int i = 0; i < T / 64; ++i) mean += sm[0][i];
  mean *= inv_batch;
  float s2[1] = {0.f};
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    const int64_t q = threadIdx.x + (int64_t)T * i;
    if (q < n4) {
      const f32x4 d = v[i] - mean;
      s2[0] += (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]);
    }
  }
  wave_sums<T>(s2, 1);
  if (lane == 0) sm[1][w] = s2[0];
  __syncthreads();
  float var = 0.f;
#pragma unroll
  for (int i = 0; i < T / 64; ++i) var += sm[1][i];
  var *= inv_batch;
  const float den = bn_den(var, eps);
  const float g = gamma[f], b = beta[f];
  f32x4* yc = reinterpret_cast<f32x4*>(y + N * f);
  f32x4* hc = xhat ? reinterpret_cast<f32x4*>(xhat + N * f) : nullptr;
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    const int64_t q = threadIdx.x + (int64_t)T * i;
    if (q < n4) {
      f32x4 xh, o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xh[e] = bn_xhat(v[i][e], mean, den);
        o[e] = g * xh[e] + b;
      }
      if (hc) hc[q] = xh;
      yc[q] = o;
    }
  }
  if (threadIdx.x == 0) {
    bmean[f] = mean;
    bvar[f] = var;
    rmean[f] = (1.0f - momentum) * rmean[f] + momentum * mean;
    rvar[f] = (1.0f - momentum) * rvar[f] + momentum * var;
  }
}

// batch_norm.cpp:353-385 with the layout of bn_fwd_vec_kernel: dY, x and
// xhat read once as float4s, the four column sums reduced together.
template <int T, int V4>
__global__ void __launch_bounds__(T) bn_bwd_vec_kernel(const float* __restrict__ dY,
                                                       const float* __restrict__ x,
                                                       const float* __restrict__ xhat,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ bmean,
                                                       const float* __restrict__ bvar,
                                                       float* __restrict__ ggamma,
                                                       float* __restrict__ gbeta,
                                                       float* __restrict__ dX, int64_t N, float eps) {
  __shared__ float sm[4][T / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t f = blockIdx.x, n4 = N >> 2;
  const f32x4* dyc = reinterpret_cast<const f32x4*>(dY + N * f);
  const f32x4* xc = reinterpret_cast<const f32x4*>(x + N * f);
  const f32x4* hc = xhat ? reinterpret_cast<const f32x4*>(xhat + N * f) : nullptr;
  const float g = gamma[f], mean = bmean[f];
  const float den = bn_den(bvar[f], eps);  // the forward's divisor: xhat recomputed bit for bit
  const float inv_std = 1.0f / den;
  const float inv_batch = 1.0f / (float)N;
  const float c3 = (-0.5f) * inv_std * inv_std * inv_std;
  f32x4 dy[V4], xm[V4];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // grad_gamma, grad_beta, dvar, dmean
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    const int64_t q = threadIdx.x + (int64_t)T * i;
    dy[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    xm[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (q < n4) {
      dy[i] = dyc[q];
      xm[i] = xc[q] - mean;
      f32x4 xh;
      if (hc) {
        xh = hc[q];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) xh[e] = xm[i][e] / den;
      }
      f32x4 pg, pv, pm;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dxh = dy[i][e] * g;
        pg[e] = dy[i][e] * xh[e];
        pv[e] = dxh * xm[i][e] * c3;
        pm[e] = dxh * (-inv_std);
      }
      acc[0] += (pg[0] + pg[1]) + (pg[2] + pg[3]);
      acc[1] += (dy[i][0] + dy[i][1]) + (dy[i][2] + dy[i][3]);
      acc[2] += (pv[0] + pv[1]) + (pv[2] + pv[3]);
      acc[3] += (pm[0] + pm[1]) + (pm[2] + pm[3]);
    }
  }
  wave_sums<T>(acc, 4);
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) sm[j][w] = acc[j];
  }
  __syncthreads();
  float tot[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < T / 64; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) tot[j] += sm[j][i];
  if (threadIdx.x == 0) {
    ggamma[f] = tot[0];
    gbeta[f] = tot[1];
  }
  const float dvar = tot[2], dmean = tot[3];
  f32x4* dxc = reinterpret_cast<f32x4*>(dX + N * f);
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    const int64_t q = threadIdx.x + (int64_t)T * i;
    if (q < n4) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = dy[i][e] * g * inv_std + dvar * 2.0f * xm[i][e] * inv_batch + dmean * inv_batch;
      dxc[q] = o;
    }
  }
}

// GELU over n elements; vec: all pointers 16-byte aligned, so the first
// n/4*4 elements move as float4s (per-element math unchanged).
__global__ void __launch_bounds__(256) gelu_fwd_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t n, int vec) {
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t done = 0;
  if (vec) {
    const int64_t n4 = n >> 2;
    for (int64_t i = t0; i < n4; i += stride) {
      const f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = gelu_f(v[e]);
      reinterpret_cast<f32x4*>(y)[i] = o;
    }
    done = n4 << 2;
  }
  for (int64_t i = done + t0; i < n; i += stride) y[i] = gelu_f(x[i]);
}
__global__ void __launch_bounds__(256) gelu_bwd_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ dy,
                                                       float* __restrict__ dx, int64_t n, int vec) {
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t done = 0;
  if (vec) {
    const int64_t n4 = n >> 2;
    for (int64_t i = t0; i < n4; i += stride) {
      const f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
      const f32x4 g = reinterpret_cast<const f32x4*>(dy)[i];
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = g[e] * gelu_grad_f(v[e]);
      reinterpret_cast<f32x4*>(dx)[i] = o;
    }
    done = n4 << 2;
  }
  for (int64_t i = done + t0; i < n; i += stride) dx[i] = dy[i] * gelu_grad_f(x[i]);
}

// mean over s of [B,S,D].  For one feature d the [B, S] slab is contiguous
// (b + B*s), so a block owns (d, up to 64 consecutive b) and its threads
// split s into CHUNKS contiguous ranges: thread (b, chunk) sums its range in
// order, then the chunk sums are added in chunk order (a fixed order for
// any launch) and divided by S.
__global__ void __launch_bounds__(256) meanpool_fwd_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, int64_t B,
                                                           int64_t S, int64_t D, int bw) {
  __shared__ float part[256];
  const int chunks = 256 / bw;
  const int bl = threadIdx.x % bw, ch = threadIdx.x / bw;
  const int64_t d = blockIdx.x;
  const int64_t b = (int64_t)blockIdx.y * bw + bl;
  const int64_t per = (S + chunks - 1) / chunks;
  const int64_t t0 = ch * per, t1 = min(S, t0 + per);
  float s = 0.f;
  if (ch < chunks && b < B) {
    const float* xs = x + B * S * d + b;
    for (int64_t t = t0; t < t1; ++t) s += xs[B * t];
  }
  part[threadIdx.x] = s;
  __syncthreads();
  if (ch == 0 && b < B) {
    float tot = part[bl];
    for (int c = 1; c < chunks; ++c) tot += part[bl + bw * c];
    y[b + B * d] = tot / (float)S;
  }
}
// By sample, sample b's S rows of feature d are contiguous at S*b + B*S*d:
// one wave per (b, d), lane l summing s = l, l + 64, ... in order, then a
// butterfly over the 64 lane sums (a fixed order for any launch).
__global__ void __launch_bounds__(256) meanpool_fwd_by_sample_kernel(const float* __restrict__ x,
                                                                     float* __restrict__ y,
                                                                     int64_t B, int64_t S,
                                                                     int64_t D) {
  const int lane = threadIdx.x & 63;
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // b + B*d
  if (pair >= B * D) return;
  const int64_t b = pair % B, d = pair / B;
  const float* xs = x + S * b + B * S * d;
  float s = 0.f;
  for (int64_t t = lane; t < S; t += 64) s += xs[t];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) y[pair] = s / (float)S;
}
__global__ void __launch_bounds__(256) meanpool_bwd_kernel(const float* __restrict__ dy,
                                                           float* __restrict__ dx, int64_t B,
                                                           int64_t S, int64_t D, float inv_S,
                                                           int by_sample) {
  const int64_t total = B * S * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = by_sample ? (i / S) % B : i % B, d = i / (B * S);
    dx[i] = dy[b + B * d] * inv_S;
  }
}

// meanpool_bwd_kernel by sample when S % 4 == 0: a wave per (b, d) fills the
// S contiguous values of dx at S b + B S d with float4 stores of dy(b, d) / S
__global__ void __launch_bounds__(256) meanpool_bwd_by_sample_vec_kernel(const float* __restrict__ dy,
                                                                         float* __restrict__ dx, int B,
                                                                         int S, int pairs, float inv_S) {
  const int lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);  // b + B d
  if (pair >= pairs) return;
  const int b = pair % B, d = pair / B;
  const float v = dy[pair] * inv_S;
  const f32x4 v4 = {v, v, v, v};
  f32x4* out = reinterpret_cast<f32x4*>(dx + (int64_t)S * b + (int64_t)B * S * d);
  for (int t = lane; t < S / 4; t += 64) out[t] = v4;
}

// meanpool_bwd_kernel in the reference row order when B % 4 == 0: column s of
// feature d, dx[b + B s + B S d] = dy(b, d) / S, as float4s along b
__global__ void __launch_bounds__(256) meanpool_bwd_vec_kernel(const float* __restrict__ dy,
                                                               float* __restrict__ dx, int B, int S,
                                                               int D, float inv_S) {
  const int B4 = B / 4;
  const int64_t total4 = (int64_t)B4 * S * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total4;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int b4 = (int)(i % B4);
    const int d = (int)(i / ((int64_t)B4 * S));
    f32x4 v = reinterpret_cast<const f32x4*>(dy + (int64_t)B * d)[b4];
    reinterpret_cast<f32x4*>(dx)[i] = v * inv_S;
  }
}

__global__ void __launch_bounds__(256) add_kernel(const float* __restrict__ a,
                                                  const float* __restrict__ b,
                                                  float* __restrict__ y, int64_t n, int vec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    for (int64_t i = t0; i < n / 4; i += stride) {
      const f32x4 u = reinterpret_cast<const f32x4*>(a)[i];
      const f32x4 v = reinterpret_cast<const f32x4*>(b)[i];
      reinterpret_cast<f32x4*>(y)[i] = u + v;
    }
  } else {
    for (int64_t i = t0; i < n; i += stride) y[i] = a[i] + b[i];
  }
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

int cnhip_transpose(const float* in, float* out, int64_t rows, int64_t cols, cnhip_stream_t s) {
  const char* who = "cnhip_transpose";
  CNHIP_REQUIRE(rows >= 0 && cols >= 0, "%s: negative size", who);
  if (rows == 0 || cols == 0) return CNHIP_OK;
  CNHIP_REQUIRE(in && out && in != out, "%s: NULL or aliased pointers", who);
  return cnhip::transpose(in, out, rows, cols, as_stream(s), who);
}

int64_t cnhip_mha_cache_floats(int64_t B, int64_t S, int64_t D) {
  // Projections Qp | Kp | Vp, A^T per sample, context.  Reference row order:
  // sample b's Qp_b, Kp_b, Vp_b (each [S, D] ColMajor) at b*3SD, b*3SD + SD,
  // b*3SD + 2SD; by sample: the [B*S, 3D] projection matrix itself.  Then
  // A^T_b at 3BSD + b*SS with A[i][j] at j + S*i, and the context [B*S, D]
  // at 3BSD + B*SS.
  return 4 * B * S * D + B * S * S;
}

int cnhip_mha_forward_rows(const float* q, const float* k, const float* v, const float* Wq,
                           const float* Wk, const float* Wv, const float* Wo, const float* residual,
                           float* out, float* cache, int64_t B, int64_t S, int64_t D, int64_t heads,
                           int rows, cnhip_stream_t stream) {
  const char* who = residual ? "cnhip_mha_forward_residual" : "cnhip_mha_forward";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0 && heads > 0 && D % heads == 0,
                "%s: bad shape B=%lld S=%lld D=%lld heads=%lld (D %% heads must be 0)", who,
                (long long)B, (long long)S, (long long)D, (long long)heads);
  CNHIP_REQUIRE(rows == CNHIP_ROWS_REF || rows == CNHIP_ROWS_BY_SAMPLE, "%s: bad row order %d", who, rows);
  CNHIP_REQUIRE(q && k && v && Wq && Wk && Wv && Wo && out && cache, "%s: NULL pointer", who);
  CNHIP_REQUIRE(B <= 65535, "%s: batch %lld exceeds 65535", who, (long long)B);
  hipStream_t st = as_stream(stream);
  const int64_t BS = B * S, SD = S * D, SS = S * S, DD = D * D;
  const float scale = 1.0f / sqrtf((float)(D / heads));  // attention.cpp:83
  const bool by_sample = rows == CNHIP_ROWS_BY_SAMPLE;
  float* Qs = cache;            // the projections (layout above)
  float* At = Qs + 3 * BS * D;  // per-sample A^T: (j, i) at j + S*i
  float* ctx = At + B * SS;     // [B*S, D]
  cnhip::Workspace ws(st);
  float* proj = Qs;  // [B*S, 3D]: Qp | Kp | Vp
  if (!by_sample) {
    CNHIP_TRY(ws.alloc((size_t)(3 * BS * D) * sizeof(float), who));
    proj = static_cast<float*>(ws.p);
  }
  // Self-attention with W_q, W_k, W_v adjacent in memory: one GEMM X [Wq Wk Wv].
  if (q == k && k == v && Wk == Wq + DD && Wv == Wk + DD) {
    CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, 3 * D, D, 1.f, q, BS, Wq, D, 0.f, proj, BS, nullptr, 0, st, who));
  } else {
    const float* src[3] = {q, k, v};
    const float* W[3] = {Wq, Wk, Wv};
    for (int i = 0; i < 3; ++i)
      CNHIP_TRY(cnhip::gemm_f32(0, 0, BS, D, D, 1.f, src[i], BS, W[i], D, 0.f, proj + i * BS * D, BS,
                                nullptr, 0, st, who));
  }
  // Per-sample operands: sample b's Qp_b at Qb + b*ps, each [S, D] with
  // leading dimension ld.  By sample they are rows S*b.. of the projections;
  // in the reference order the [B*S, 3D] matrix is [B, 3SD] with row b + B*s,
  // and its transpose [3SD, B] holds sample b's Qp_b, Kp_b, Vp_b at b*3SD,
  // b*3SD + SD and b*3SD + 2SD.
  const float *Qb = Qs, *Kb = Qs + SD, *Vb = Qs + 2 * SD;
  int64_t ld = S, ps = 3 * SD;
  if (by_sample) {
    Kb = Qs + BS * D;
    Vb = Qs + 2 * BS * D;
    ld = BS;
    ps = S;
  } else {
    CNHIP_TRY(cnhip::transpose(proj, Qs, B, 3 * SD, st, who));
  }
  // A^T_b = (Kp_b Qp_b^T) * scale (scores transposed, 187-189), then row softmax (191-205)
  CNHIP_TRY(cnhip::gemm_f32_batched(0, 1, S, S, D, scale, Kb, ld, ps, Qb, ld, ps, 0.f, At, S, SS, B,
                                    nullptr, 0, st, who));
  CNHIP_TRY(cnhip::softmax_rows(At, At, BS, S, st, who));
  // context_b = A_b Vp_b = (A^T_b)^T Vp_b (211), in the row order of the input
  if (by_sample) {
    CNHIP_TRY(cnhip::gemm_f32_batched(1, 0, S, D, S, 1.f, At, S, SS, Vb, ld, ps, 0.f, ctx, BS, S, B,
                                      nullptr, 0, st, who));
  } else {
    CNHIP_TRY(cnhip::gemm_f32_batched(1, 0, S, D, S, 1.f, At, S, SS, Vb, ld, ps, 0.f, proj, S, SD, B,
                                      nullptr, 0, st, who));
    CNHIP_TRY(cnhip::transpose(proj, ctx, SD, B, st, who));
  }
  // out = context W_o (212), plus the skip branch when fused
  if (residual)
    return cnhip::gemm_f32_act(0, 0, BS, D, D, ctx, BS, Wo, D, out, BS, nullptr, cnhip::EPI_ADD, residual,
                               nullptr, BS, st, who);
  return cnhip::gemm_f32(0, 0, BS, D, D, 1.f, ctx, BS, Wo, D, 0.f, out, BS, nullptr, 0, st, who);
}

int cnhip_mha_forward_residual(const float* q, const float* k, const float* v, const float* Wq,
                               const float* Wk, const float* Wv, const float* Wo, const float* residual,
                               float* out, float* cache, int64_t B, int64_t S, int64_t D, int64_t heads,
                               cnhip_stream_t stream) {
  return cnhip_mha_forward_rows(q, k, v, Wq, Wk, Wv, Wo, residual, out, cache, B, S, D, heads,
                                CNHIP_ROWS_REF, stream);
}

int cnhip_mha_forward(const float* q, const float* k, const float* v, const float* Wq,
                      const float* Wk, const float* Wv, const float* Wo, float* out, float* cache,
                      int64_t B, int64_t S, int64_t D, int64_t heads, cnhip_stream_t stream) {
  return cnhip_mha_forward_rows(q, k, v, Wq, Wk, Wv, Wo, nullptr, out, cache, B, S, D, heads,
                                CNHIP_ROWS_REF, stream);
}

int cnhip_mha_backward_rows(const float* q, const float* k, const float* v, const float* Wq,
                            const float* Wk, const float* Wv, const float* Wo, const float* cache,
                            const float* dY, const float* residual_grad, float* gWq, float* gWk,
                            float* gWv, float* gWo, float* dX, int64_t B, int64_t S, int64_t D,
                            int64_t heads, int rows, cnhip_stream_t stream) {
  const char* who = residual_grad ? "cnhip_mha_backward_residual" : "cnhip_mha_backward";
  CNHIP_REQUIRE(!residual_grad || dX, "%s: the residual gradient needs dX", who);
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0 && heads > 0 && D % heads == 0, "%s: bad shape", who);
  CNHIP_REQUIRE(rows == CNHIP_ROWS_REF || rows == CNHIP_ROWS_BY_SAMPLE, "%s: bad row order %d", who, rows);
  CNHIP_REQUIRE(q && k && v && Wq && Wk && Wv && Wo && cache && dY && gWq && gWk && gWv && gWo,
                "%s: NULL pointer", who);
  CNHIP_REQUIRE(B <= 65535, "%s: batch %lld exceeds 65535", who, (long long)B);
  hipStream_t st = as_stream(stream);
  const int64_t BS = B * S, SD = S * D, SS = S * S, DD = D * D;
  const float scale = 1.0f / sqrtf((float)(D / heads));
  const bool by_sample = rows == CNHIP_ROWS_BY_SAMPLE;
  const float* Ps = cache;  // the projections (layout in cnhip_mha_cache_floats)
  const float* At = Ps + 3 * BS * D;
  const float* ctx = At + B * SS;
  cnhip::Workspace ws(st);
  const int64_t extra = by_sample ? 0 : 4 * BS * D;  // per-sample copies of gctx and gQp | gKp | gVp
  CNHIP_TRY(ws.alloc((size_t)(4 * BS * D + extra + 2 * B * SS) * sizeof(float), who));
  float* gctx = static_cast<float*>(ws.p);  // [B*S, D]
  float* G = gctx + BS * D;                 // [B*S, 3D]: gQp | gKp | gVp
  float* gAT = G + 3 * BS * D;              // per-sample (j, i)
  float* gST = gAT + B * SS;
  float* gcs = gST + B * SS;                // reference order: per-sample gctx
  float* gPs = gcs + BS * D;                // reference order: per sample b: gQp_b, gKp_b, gVp_b at b*3SD
  // per-sample operands (as in the forward): Qp_b, Kp_b, Vp_b with leading
  // dimension ld at sample stride ps; gctx_b, gQp_b, gKp_b, gVp_b likewise
  const float *Qb = Ps, *Kb = Ps + SD, *Vb = Ps + 2 * SD;
  const float* gcb = gcs;
  float *gQb = gPs, *gKb = gPs + SD, *gVb = gPs + 2 * SD;
  int64_t ld = S, ps = 3 * SD, gps = SD;
  if (by_sample) {
    Kb = Ps + BS * D;
    Vb = Ps + 2 * BS * D;
    gcb = gctx;
    gQb = G;
    gKb = G + BS * D;
    gVb = G + 2 * BS * D;
    ld = BS;
    ps = gps = S;
  }
  // grad_context = dY W_o^T (535); grad_W_o = context^T dY (536)
  CNHIP_TRY(cnhip::gemm_f32_pair(
      cnhip::GemmSpec{0, 1, BS, D, D, 1.f, dY, BS, 0, Wo, D, 0, 0.f, gctx, BS, 0, 1, nullptr, 0, nullptr, nullptr, 0},
      cnhip::GemmSpec{1, 0, D, D, BS, 1.f, ctx, BS, 0, dY, BS, 0, 0.f, gWo, D, 0, 1, nullptr, 0, nullptr, nullptr, 0},
      st, who));
  if (!by_sample) CNHIP_TRY(cnhip::transpose(gctx, gcs, B, SD, st, who));
  // grad_A^T_b = Vp_b grad_ctx_b^T (538); grad_Vp_b = A_b^T grad_ctx_b (539)
  CNHIP_TRY(cnhip::gemm_f32_batched(0, 1, S, S, D, 1.f, Vb, ld, ps, gcb, ld, gps, 0.f, gAT, S, SS, B,
                                    nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32_batched(0, 0, S, D, S, 1.f, At, S, SS, gcb, ld, gps, 0.f, gVb, ld, ps, B,
                                    nullptr, 0, st, who));
  // softmax Jacobian rows, times scale (541-551)
  CNHIP_TRY(cnhip::softmax_rows_bwd(At, gAT, gST, BS, S, scale, st, who));
  // grad_Qp_b = gS_b Kp_b ; grad_Kp_b = gS_b^T Qp_b (553-554)
  CNHIP_TRY(cnhip::gemm_f32_pair(
      cnhip::GemmSpec{1, 0, S, D, S, 1.f, gST, S, SS, Kb, ld, ps, 0.f, gQb, ld, ps, B, nullptr, 0, nullptr, nullptr, 0},
      cnhip::GemmSpec{0, 0, S, D, S, 1.f, gST, S, SS, Qb, ld, ps, 0.f, gKb, ld, ps, B, nullptr, 0, nullptr, nullptr, 0},
      st, who));
  // reference order: per-sample [3SD, B] -> [B, 3SD] = [B*S, 3D]
  if (!by_sample) CNHIP_TRY(cnhip::transpose(gPs, G, 3 * SD, B, st, who));
  const float* gQp = G;
  const float* gKp = G + BS * D;
  const float* gVp = G + 2 * BS * D;
  const bool packed = q == k && k == v && Wk == Wq + DD && Wv == Wk + DD && gWk == gWq + DD &&
                      gWv == gWk + DD;
  if (packed) {
    // [gW_q gW_k gW_v] = X^T [gQp gKp gVp]; grad_input = [gQp gKp gVp] [Wq Wk Wv]^T
    const cnhip::GemmSpec wgrad{1, 0, D, 3 * D, BS, 1.f, q, BS, 0, G, BS, 0, 0.f, gWq, D, 0, 1, nullptr, 0,
                                nullptr, nullptr, 0};
    if (!dX) return cnhip::gemm_f32(1, 0, D, 3 * D, BS, 1.f, q, BS, G, BS, 0.f, gWq, D, nullptr, 0, st, who);
    // the input gradient and the weight gradient in one launch
    return cnhip::gemm_f32_pair(cnhip::GemmSpec{0, 1, BS, D, 3 * D, 1.f, G, BS, 0, Wq, D, 0, 0.f, dX, BS, 0, 1,
                                                nullptr, residual_grad ? cnhip::EPI_ADD : 0, residual_grad,
                                                nullptr, residual_grad ? BS : 0},
                                wgrad, st, who);
  }
  // weight grads over all B*S rows (556-563)
  CNHIP_TRY(cnhip::gemm_f32(1, 0, D, D, BS, 1.f, q, BS, gQp, BS, 0.f, gWq, D, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, D, D, BS, 1.f, k, BS, gKp, BS, 0.f, gWk, D, nullptr, 0, st, who));
  CNHIP_TRY(cnhip::gemm_f32(1, 0, D, D, BS, 1.f, v, BS, gVp, BS, 0.f, gWv, D, nullptr, 0, st, who));
  // grad_input = dQ + dK + dV (565-567)
  if (dX) {
    CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, D, D, 1.f, gQp, BS, Wq, D, 0.f, dX, BS, nullptr, 0, st, who));
    CNHIP_TRY(cnhip::gemm_f32(0, 1, BS, D, D, 1.f, gKp, BS, Wk, D, 1.f, dX, BS, nullptr, 0, st, who));
    // the last term adds the skip branch's gradient after dQ + dK + dV
    CNHIP_TRY(cnhip::gemm_f32_core(0, 1, BS, D, D, 1.f, gVp, BS, 0, Wv, D, 0, 1.f, dX, BS, 0, 1, nullptr,
                                   residual_grad ? cnhip::EPI_ADD : 0, residual_grad, nullptr, BS, st, who));
  }
  return CNHIP_OK;
}

int cnhip_mha_backward_residual(const float* q, const float* k, const float* v, const float* Wq,
                                const float* Wk, const float* Wv, const float* Wo, const float* cache,
                                const float* dY, const float* residual_grad, float* gWq, float* gWk,
                                float* gWv, float* gWo, float* dX, int64_t B, int64_t S, int64_t D,
                                int64_t heads, cnhip_stream_t stream) {
  return cnhip_mha_backward_rows(q, k, v, Wq, Wk, Wv, Wo, cache, dY, residual_grad, gWq, gWk, gWv, gWo, dX,
                                 B, S, D, heads, CNHIP_ROWS_REF, stream);
}

int cnhip_mha_backward(const float* q, const float* k, const float* v, const float* Wq,
                       const float* Wk, const float* Wv, const float* Wo, const float* cache,
                       const float* dY, float* gWq, float* gWk, float* gWv, float* gWo, float* dX,
                       int64_t B, int64_t S, int64_t D, int64_t heads, cnhip_stream_t stream) {
  return cnhip_mha_backward_rows(q, k, v, Wq, Wk, Wv, Wo, cache, dY, nullptr, gWq, gWk, gWv, gWo, dX, B, S,
                                 D, heads, CNHIP_ROWS_REF, stream);
}

int cnhip_embedding_forward_rows(const int32_t* ids, const float* Wt, float* out, int64_t B, int64_t S,
                                 int64_t V, int64_t D, int32_t* oob_count, int rows, cnhip_stream_t stream) {
  const char* who = "cnhip_embedding_forward";
  CNHIP_REQUIRE(B > 0 && S > 0 && V > 0 && D > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(rows == CNHIP_ROWS_REF || rows == CNHIP_ROWS_BY_SAMPLE, "%s: bad row order %d", who, rows);
  CNHIP_REQUIRE(ids && Wt && out, "%s: NULL pointer", who);
  const int64_t BS = B * S;
  CNHIP_REQUIRE((D + cnhip::TT - 1) / cnhip::TT <= 65535, "%s: embed_dim too large", who);
  // ids read, one table row read and one output row written per token
  cnhip::HbmTimer timer("embedding_fwd_kernel", 4.0 * (double)BS + 8.0 * (double)BS * (double)D,
                        as_stream(stream));
  hipLaunchKernelGGL(cnhip::embedding_fwd_kernel,
                     dim3((unsigned)((BS + cnhip::TT - 1) / cnhip::TT), (unsigned)((D + cnhip::TT - 1) / cnhip::TT)),
                     dim3(256), 0, as_stream(stream), ids, Wt, out, B, S, V, D, rows, oob_count);
  return cnhip::check_launch(who);
}

int cnhip_embedding_forward(const int32_t* ids, const float* Wt, float* out, int64_t B, int64_t S,
                            int64_t V, int64_t D, int32_t* oob_count, cnhip_stream_t stream) {
  return cnhip_embedding_forward_rows(ids, Wt, out, B, S, V, D, oob_count, CNHIP_ROWS_REF, stream);
}

int cnhip_embedding_backward_rows(const int32_t* ids, const float* dY, float* gWt, int64_t B, int64_t S,
                                  int64_t V, int64_t D, int rows, cnhip_stream_t stream) {
  const char* who = "cnhip_embedding_backward";
  CNHIP_REQUIRE(B > 0 && S > 0 && V > 0 && D > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(rows == CNHIP_ROWS_REF || rows == CNHIP_ROWS_BY_SAMPLE, "%s: bad row order %d", who, rows);
  CNHIP_REQUIRE(ids && dY && gWt, "%s: NULL pointer", who);
  CNHIP_REQUIRE(V < ((int64_t)1 << 31) && B * S < ((int64_t)1 << 31), "%s: too large", who);
  hipStream_t st = as_stream(stream);
  const int64_t BS = B * S;
  cnhip::Workspace ws(st);
  const size_t ibytes = (size_t)(2 * V + (V + 1) + BS) * sizeof(int32_t);
  CNHIP_TRY(ws.alloc(ibytes + (size_t)(BS * D) * sizeof(float) + 16, who));
  int32_t* counts = static_cast<int32_t*>(ws.p);
  int32_t* cursor = counts + V;
  int32_t* offsets = cursor + V;
  int32_t* pos = offsets + (V + 1);
  float* dYt = reinterpret_cast<float*>(reinterpret_cast<char*>(ws.p) + ((ibytes + 15) & ~size_t(15)));
  CNHIP_TRY(cnhip::transpose(dY, dYt, BS, D, st, who));
  if (V <= cnhip::kEmbSmall && BS <= cnhip::kEmbSmall) {
    hipLaunchKernelGGL(cnhip::emb_bucket_small_kernel, dim3(1), dim3(1024), 0, st, ids, offsets, pos, (int)B,
                       (int)S, (int)V);
    CNHIP_TRY(cnhip::check_launch(who));
  } else {
    CNHIP_TRY(cnhip::fill_bytes(counts, 0, (size_t)(2 * V) * sizeof(int32_t), st, who));
    const unsigned g = cnhip::elementwise_grid(BS, 256);
    hipLaunchKernelGGL(cnhip::emb_count_kernel, dim3(g), dim3(256), 0, st, ids, counts, BS, V);
    CNHIP_TRY(cnhip::check_launch(who));
    hipLaunchKernelGGL(cnhip::emb_scan_kernel, dim3(1), dim3(1024), 0, st, counts, offsets, V);
    CNHIP_TRY(cnhip::check_launch(who));
    hipLaunchKernelGGL(cnhip::emb_fill_kernel, dim3(g), dim3(256), 0, st, ids, offsets, cursor, pos, B, S, V);
    CNHIP_TRY(cnhip::check_launch(who));
    hipLaunchKernelGGL(cnhip::emb_sort_kernel, dim3(cnhip::elementwise_grid(V, 256)), dim3(256), 0, st,
                       offsets, pos, V);
    CNHIP_TRY(cnhip::check_launch(who));
  }
  // every token's gradient row read once, every table row written
  cnhip::HbmTimer timer("emb_sum_kernel", 4.0 * (double)BS * (double)D + 4.0 * (double)V * (double)D, st);
  if (D % 4 == 0 && D < ((int64_t)1 << 31) && cnhip::aligned16(gWt))
    hipLaunchKernelGGL(cnhip::emb_sum_vec_kernel, dim3((unsigned)((V + 3) / 4)), dim3(256), 0, st, offsets, pos,
                       dYt, gWt, (int)B, (int)S, (int)D, (int)V, rows);
  else
    hipLaunchKernelGGL(cnhip::emb_sum_kernel, dim3((unsigned)V), dim3(128), 0, st, offsets, pos, dYt,
                       gWt, B, S, D, rows);
  return cnhip::check_launch(who);
}

int cnhip_embedding_backward(const int32_t* ids, const float* dY, float* gWt, int64_t B, int64_t S,
                             int64_t V, int64_t D, cnhip_stream_t stream) {
  return cnhip_embedding_backward_rows(ids, dY, gWt, B, S, V, D, CNHIP_ROWS_REF, stream);
}

int cnhip_batchnorm_forward(const float* x, float* y, float* xhat, const float* gamma,
                            const float* beta, float* running_mean, float* running_var,
                            float* batch_mean, float* batch_var, int64_t N, int64_t F,
                            float momentum, float eps, cnhip_stream_t stream) {
  const char* who = "cnhip_batchnorm_forward";
  CNHIP_REQUIRE(N > 0 && F > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(x && y && gamma && beta && running_mean && running_var && batch_mean && batch_var,
                "%s: NULL pointer", who);
  // x read once; y (and xhat when asked for) written
  cnhip::HbmTimer timer("bn_fwd_kernel", (xhat ? 12.0 : 8.0) * (double)N * (double)F, as_stream(stream));
  const bool vec =
      N % 4 == 0 && cnhip::aligned16(x) && cnhip::aligned16(y) && (!xhat || cnhip::aligned16(xhat));
  if (vec && N <= 4 * 256)
    hipLaunchKernelGGL((cnhip::bn_fwd_vec_kernel<256, 1>), dim3((unsigned)F), dim3(256), 0, as_stream(stream),
                       x, y, xhat, gamma, beta, running_mean, running_var, batch_mean, batch_var, N,
                       momentum, eps);
  else if (vec && N <= 4 * 512 * 4)
    hipLaunchKernelGGL((cnhip::bn_fwd_vec_kernel<512, 4>), dim3((unsigned)F), dim3(512), 0,
                       as_stream(stream), x, y, xhat, gamma, beta, running_mean, running_var, batch_mean,
                       batch_var, N, momentum, eps);
  else if (vec && N <= 4 * 1024 * 8)
    hipLaunchKernelGGL((cnhip::bn_fwd_vec_kernel<1024, 8>), dim3((unsigned)F), dim3(1024), 0,
                       as_stream(stream), x, y, xhat, gamma, beta, running_mean, running_var, batch_mean,
                       batch_var, N, momentum, eps);
  else if (N <= (int64_t)cnhip::BNT * 32)  // whole column in registers
    hipLaunchKernelGGL(cnhip::bn_fwd_reg_kernel<32>, dim3((unsigned)F), dim3(cnhip::BNT), 0,
                       as_stream(stream), x, y, xhat, gamma, beta, running_mean, running_var,
                       batch_mean, batch_var, N, momentum, eps);
  else
    hipLaunchKernelGGL(cnhip::bn_fwd_kernel, dim3((unsigned)F), dim3(cnhip::BNT), 0,
                       as_stream(stream), x, y, xhat, gamma, beta, running_mean, running_var,
                       batch_mean, batch_var, N, momentum, eps);
  return cnhip::check_launch(who);
}

int cnhip_batchnorm_forward_eval(const float* x, float* y, float* xhat, const float* gamma,
                                 const float* beta, const float* running_mean,
                                 const float* running_var, int64_t N, int64_t F, float eps,
                                 cnhip_stream_t stream) {
  const char* who = "cnhip_batchnorm_forward_eval";
  CNHIP_REQUIRE(N > 0 && F > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(x && y && xhat && gamma && beta && running_mean && running_var, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("bn_eval_kernel", 12.0 * (double)N * (double)F, as_stream(stream));
  hipLaunchKernelGGL(cnhip::bn_eval_kernel, dim3(cnhip::elementwise_grid(N * F, 256)), dim3(256), 0,
                     as_stream(stream), x, y, xhat, gamma, beta, running_mean, running_var, N, F, eps);
  return cnhip::check_launch(who);
}

int cnhip_batchnorm_backward(const float* dY, const float* x, const float* xhat, const float* gamma,
                             const float* batch_mean, const float* batch_var, float* grad_gamma,
                             float* grad_beta, float* dX, int64_t N, int64_t F, float eps,
                             cnhip_stream_t stream) {
  const char* who = "cnhip_batchnorm_backward";
  CNHIP_REQUIRE(N > 0 && F > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(dY && x && gamma && batch_mean && batch_var && grad_gamma && grad_beta && dX,
                "%s: NULL pointer", who);
  // dY and x (and xhat when given) read once; dX written
  cnhip::HbmTimer timer("bn_bwd_kernel", (xhat ? 16.0 : 12.0) * (double)N * (double)F, as_stream(stream));
  const bool vec = N % 4 == 0 && cnhip::aligned16(dY) && cnhip::aligned16(x) &&
                   (!xhat || cnhip::aligned16(xhat)) && cnhip::aligned16(dX);
  if (vec && N <= 4 * 256)
    hipLaunchKernelGGL((cnhip::bn_bwd_vec_kernel<256, 1>), dim3((unsigned)F), dim3(256), 0, as_stream(stream),
                       dY, x, xhat, gamma, batch_mean, batch_var, grad_gamma, grad_beta, dX, N, eps);
  else if (vec && N <= 4 * 512 * 4)
    hipLaunchKernelGGL((cnhip::bn_bwd_vec_kernel<512, 4>), dim3((unsigned)F), dim3(512), 0,
                       as_stream(stream), dY, x, xhat, gamma, batch_mean, batch_var, grad_gamma, grad_beta,
                       dX, N, eps);
  else if (vec && N <= 4 * 1024 * 8)
    hipLaunchKernelGGL((cnhip::bn_bwd_vec_kernel<1024, 8>), dim3((unsigned)F), dim3(1024), 0,
                       as_stream(stream), dY, x, xhat, gamma, batch_mean, batch_var, grad_gamma, grad_beta,
                       dX, N, eps);
  else if (N <= (int64_t)cnhip::BNT * 32)
    hipLaunchKernelGGL(cnhip::bn_bwd_reg_kernel<32>, dim3((unsigned)F), dim3(cnhip::BNT), 0,
                       as_stream(stream), dY, x, xhat, gamma, batch_mean, batch_var, grad_gamma,
                       grad_beta, dX, N, eps);
  else
    hipLaunchKernelGGL(cnhip::bn_bwd_kernel, dim3((unsigned)F), dim3(cnhip::BNT), 0,
                       as_stream(stream), dY, x, xhat, gamma, batch_mean, batch_var, grad_gamma,
                       grad_beta, dX, N, eps);
  return cnhip::check_launch(who);
}

int cnhip_gelu_forward(const float* x, float* y, int64_t n, cnhip_stream_t s) {
  const char* who = "cnhip_gelu_forward";
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(x && y, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("gelu_fwd_kernel", 8.0 * (double)n, as_stream(s));
  const int vec = cnhip::aligned16(x) && cnhip::aligned16(y);
  hipLaunchKernelGGL(cnhip::gelu_fwd_kernel, dim3(cnhip::elementwise_grid(vec ? (n + 3) / 4 : n, 256)),
                     dim3(256), 0, as_stream(s), x, y, n, vec);
  return cnhip::check_launch(who);
}

int cnhip_gelu_backward(const float* x, const float* dy, float* dx, int64_t n, cnhip_stream_t s) {
  const char* who = "cnhip_gelu_backward";
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(x && dy && dx, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("gelu_bwd_kernel", 12.0 * (double)n, as_stream(s));
  const int vec = cnhip::aligned16(x) && cnhip::aligned16(dy) && cnhip::aligned16(dx);
  hipLaunchKernelGGL(cnhip::gelu_bwd_kernel, dim3(cnhip::elementwise_grid(vec ? (n + 3) / 4 : n, 256)),
                     dim3(256), 0, as_stream(s), x, dy, dx, n, vec);
  return cnhip::check_launch(who);
}

int cnhip_meanpool1d_forward_rows(const float* x, float* y, int64_t B, int64_t S, int64_t D, int rows,
                                  cnhip_stream_t s) {
  const char* who = "cnhip_meanpool1d_forward";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(rows == CNHIP_ROWS_REF || rows == CNHIP_ROWS_BY_SAMPLE, "%s: bad row order %d", who, rows);
  CNHIP_REQUIRE(x && y, "%s: NULL pointer", who);
  CNHIP_REQUIRE(D <= 0x7fffffff, "%s: D too large", who);
  if (rows == CNHIP_ROWS_BY_SAMPLE) {
    CNHIP_REQUIRE((B * D + 3) / 4 <= 0x7fffffff, "%s: B*D too large", who);
    cnhip::HbmTimer timer("meanpool_fwd_by_sample_kernel", 4.0 * (double)B * (double)D * (double)(S + 1),
                          as_stream(s));
    hipLaunchKernelGGL(cnhip::meanpool_fwd_by_sample_kernel, dim3((unsigned)((B * D + 3) / 4)), dim3(256), 0,
                       as_stream(s), x, y, B, S, D);
    return cnhip::check_launch(who);
  }
  const int bw = B < 64 ? (int)B : 64;
  cnhip::HbmTimer timer("meanpool_fwd_kernel", 4.0 * (double)B * (double)D * (double)(S + 1), as_stream(s));
  hipLaunchKernelGGL(cnhip::meanpool_fwd_kernel, dim3((unsigned)D, (unsigned)((B + bw - 1) / bw)),
                     dim3(256), 0, as_stream(s), x, y, B, S, D, bw);
  return cnhip::check_launch(who);
}

int cnhip_meanpool1d_forward(const float* x, float* y, int64_t B, int64_t S, int64_t D,
                             cnhip_stream_t s) {
  return cnhip_meanpool1d_forward_rows(x, y, B, S, D, CNHIP_ROWS_REF, s);
}

int cnhip_meanpool1d_backward_rows(const float* dy, float* dx, int64_t B, int64_t S, int64_t D, int rows,
                                   cnhip_stream_t s) {
  const char* who = "cnhip_meanpool1d_backward";
  CNHIP_REQUIRE(B > 0 && S > 0 && D > 0, "%s: bad shape", who);
  CNHIP_REQUIRE(rows == CNHIP_ROWS_REF || rows == CNHIP_ROWS_BY_SAMPLE, "%s: bad row order %d", who, rows);
  CNHIP_REQUIRE(dy && dx, "%s: NULL pointer", who);
  cnhip::HbmTimer timer("meanpool_bwd_kernel", 4.0 * (double)B * (double)D * (double)(S + 1), as_stream(s));
  const float inv_S = 1.0f / (float)S;
  // the float4 kernels index (b, s, d) and their pair count in 32-bit integers
  const bool fits32 = B * D < ((int64_t)1 << 31) && S < ((int64_t)1 << 31);
  if (fits32 && rows == CNHIP_ROWS_BY_SAMPLE && S % 4 == 0 && cnhip::aligned16(dx)) {
    const int pairs = (int)(B * D);
    hipLaunchKernelGGL(cnhip::meanpool_bwd_by_sample_vec_kernel, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0,
                       as_stream(s), dy, dx, (int)B, (int)S, pairs, inv_S);
  } else if (fits32 && rows == CNHIP_ROWS_REF && B % 4 == 0 && cnhip::aligned16(dx) && cnhip::aligned16(dy)) {
    hipLaunchKernelGGL(cnhip::meanpool_bwd_vec_kernel, dim3(cnhip::elementwise_grid(B * S * D / 4, 256)),
                       dim3(256), 0, as_stream(s), dy, dx, (int)B, (int)S, (int)D, inv_S);
  } else {
    hipLaunchKernelGGL(cnhip::meanpool_bwd_kernel, dim3(cnhip::elementwise_grid(B * S * D, 256)),
                       dim3(256), 0, as_stream(s), dy, dx, B, S, D, inv_S, rows);
  }
  return cnhip::check_launch(who);
}

int cnhip_meanpool1d_backward(const float* dy, float* dx, int64_t B, int64_t S, int64_t D,
                              cnhip_stream_t s) {
  return cnhip_meanpool1d_backward_rows(dy, dx, B, S, D, CNHIP_ROWS_REF, s);
}

int cnhip_add(const float* a, const float* b, float* y, int64_t n, cnhip_stream_t s) {
  const char* who = "cnhip_add";
  CNHIP_REQUIRE(n >= 0, "%s: negative size", who);
  if (n == 0) return CNHIP_OK;
  CNHIP_REQUIRE(a && b && y, "%s: NULL pointer", who);
  const int vec = (n % 4 == 0) && cnhip::aligned16(a) && cnhip::aligned16(b) && cnhip::aligned16(y);
  cnhip::HbmTimer timer("add_kernel", 12.0 * (double)n, as_stream(s));
  hipLaunchKernelGGL(cnhip::add_kernel, dim3(cnhip::elementwise_grid(vec ? n / 4 : n, 256)), dim3(256),
                     0, as_stream(s), a, b, y, n, vec);
  return cnhip::check_launch(who);
}

}  // extern "C"
