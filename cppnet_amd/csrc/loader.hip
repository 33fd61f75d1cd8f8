// Batch assembly for the DataLoader's resident mode (ref: the row copy loop
// of src/CppNet/utils/dataloader.cpp:68-88, get_batch).
//
// The dataset lives in HBM sample-major: sample n's F values are contiguous
// at src + n*F (the transpose of the reference's ColMajor [N, F]).  A batch
// is written ColMajor [B, F] (the layers' layout): dst[b + B*f] =
// src[idx[b]*F + f].  One block moves a 64-sample x 64-value tile through
// LDS: reads are whole contiguous sample segments (float4 where F and the
// pointer allow), writes are 64 consecutive b of one f (256-byte rows), so
// both sides coalesce whatever order the indices come in (small batches take
// gather_small_kernel below).  An index outside [0, N) reads nothing and
// yields zeros.  HBM-bound: the
// algorithmic traffic is 2*B*F*4 bytes (+ 4*B for the indices).
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace cnhip {
namespace {

constexpr int kTile = 64;

// Tiles with blockIdx.y < ty0 gather the first matrix (src0 -> dst0, F0
// values per sample), the others the second (src1 -> dst1, F1 values), so a
// batch's features and labels take one launch.
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ src0,
                                                          float* __restrict__ dst0, int64_t F0,
                                                          const float* __restrict__ src1,
                                                          float* __restrict__ dst1, int64_t F1,
                                                          int ty0, const int32_t* __restrict__ idx,
                                                          int64_t N, int64_t B) {
  __shared__ float tile[kTile][kTile + 1];  // [sample][value], padded
  // value tiles vary fastest across the grid, so blocks that run together read
  // neighbouring segments of the same 64 samples (DRAM row locality)
  const bool first = (int)blockIdx.x < ty0;
  const float* __restrict__ src = first ? src0 : src1;
  float* __restrict__ dst = first ? dst0 : dst1;
  const int64_t F = first ? F0 : F1;
  const int64_t b0 = (int64_t)blockIdx.y * kTile;
  const int64_t f0 = (int64_t)(first ? blockIdx.x : blockIdx.x - ty0) * kTile;
  const int t = threadIdx.x;
  // float4 reads need every sample segment 16-byte aligned
  const bool vec = (F % 4 == 0) && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
  if (vec) {
    // 16 lanes cover one sample's 64 values; 16 samples per pass
    const int lane = t & 15, srow = t >> 4;
    for (int r = srow; r < kTile; r += 16) {
      const int64_t b = b0 + r;
      const int64_t f = f0 + 4 * lane;
      const int64_t n = b < B ? (int64_t)idx[b] : -1;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (n >= 0 && n < N && f < F)  // F % 4 == 0, so f < F covers f..f+3
        v = *reinterpret_cast<const float4*>(src + n * F + f);
      tile[r][4 * lane + 0] = v.x;
      tile[r][4 * lane + 1] = v.y;
      tile[r][4 * lane + 2] = v.z;
      tile[r][4 * lane + 3] = v.w;
    }
  } else {
    const int lane = t & 63, srow = t >> 6;
    for (int r = srow; r < kTile; r += 4) {
      const int64_t b = b0 + r;
      const int64_t f = f0 + lane;
      const int64_t n = b < B ? (int64_t)idx[b] : -1;
      tile[r][lane] = (n >= 0 && n < N && f < F) ? src[n * F + f] : 0.f;
    }
  }
  __syncthreads();
  if ((B % 4) == 0 && ((reinterpret_cast<uintptr_t>(dst) & 15) == 0)) {
    // 16 lanes write one value's 64 samples as float4s; 16 values per pass
    const int q = t & 15, frow = t >> 4;
    const int64_t b = b0 + 4 * q;
    if (b < B)  // B % 4 == 0, so b < B covers b..b+3
      for (int c = frow; c < kTile; c += 16) {
        const int64_t f = f0 + c;
        if (f < F)
          *reinterpret_cast<float4*>(dst + b + B * f) =
              make_float4(tile[4 * q][c], tile[4 * q + 1][c], tile[4 * q + 2][c], tile[4 * q + 3][c]);
      }
  } else {
    const int lane = t & 63, frow = t >> 6;
    const int64_t b = b0 + lane;
    if (b < B)
      for (int c = frow; c < kTile; c += 4) {
        const int64_t f = f0 + c;
        if (f < F) dst[b + B * f] = tile[lane][c];
      }
  }
}

// Small batches (B (F0 + F1) <= kSmallGather values, e.g. 512 samples of 31):
// a thread per output value, consecutive threads on consecutive samples of
// one value, so the stores coalesce; each thread loads its sample's index and
// then the value.  Two dependent loads instead of the tile kernel's staged
// passes; the same values land in the same places.
constexpr int64_t kSmallGather = 65536;

__global__ __launch_bounds__(256) void gather_small_kernel(const float* __restrict__ src0,
                                                           float* __restrict__ dst0, int64_t F0,
                                                           const float* __restrict__ src1,
                                                           float* __restrict__ dst1, int64_t F1,
                                                           const int32_t* __restrict__ idx, int64_t N,
                                                           int64_t B) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= B * (F0 + F1)) return;
  const int64_t f = e / B, b = e - f * B;
  const int64_t n = idx[b];
  const bool ok = n >= 0 && n < N;
  if (f < F0)
    dst0[b + B * f] = ok ? src0[n * F0 + f] : 0.f;
  else
    dst1[b + B * (f - F0)] = ok ? src1[n * F1 + (f - F0)] : 0.f;
}

}  // namespace
}  // namespace cnhip

using cnhip::as_stream;

extern "C" {

static int gather_launch(const char* who, const float* src0, float* dst0, int64_t F0, const float* src1,
                         float* dst1, int64_t F1, const int32_t* idx, int64_t N, int64_t B, cnhip_stream_t s) {
  CNHIP_REQUIRE(N >= 0 && F0 >= 0 && F1 >= 0 && B >= 0, "%s: negative size", who);
  if (B == 0 || F0 + F1 == 0) return CNHIP_OK;
  CNHIP_REQUIRE(idx && (F0 == 0 || (src0 && dst0)) && (F1 == 0 || (src1 && dst1)), "%s: NULL pointer", who);
  CNHIP_REQUIRE(N > 0, "%s: gathering from an empty dataset", who);
  const int64_t gx = (B + cnhip::kTile - 1) / cnhip::kTile;
  const int64_t ty0 = (F0 + cnhip::kTile - 1) / cnhip::kTile, ty1 = (F1 + cnhip::kTile - 1) / cnhip::kTile;
  CNHIP_REQUIRE(gx <= 65535 && ty0 + ty1 <= INT32_MAX, "%s: batch %lld x %lld values is too large", who,
                (long long)B, (long long)(F0 + F1));
  cnhip::HbmTimer timer("gather_rows_kernel", 8.0 * (double)B * (double)(F0 + F1) + 4.0 * (double)B,
                        as_stream(s));
  if (B * (F0 + F1) <= cnhip::kSmallGather) {
    hipLaunchKernelGGL(cnhip::gather_small_kernel, dim3((unsigned)((B * (F0 + F1) + 255) / 256)), dim3(256), 0,
                       as_stream(s), src0, dst0, F0, src1, dst1, F1, idx, N, B);
    return cnhip::check_launch(who);
  }
  hipLaunchKernelGGL(cnhip::gather_rows_kernel, dim3((unsigned)(ty0 + ty1), (unsigned)gx), dim3(256), 0,
                     as_stream(s), src0, dst0, F0, src1, dst1, F1, (int)ty0, idx, N, B);
  return cnhip::check_launch(who);
}

int cnhip_gather_rows(const float* src, const int32_t* idx, float* dst, int64_t N, int64_t F, int64_t B,
                      cnhip_stream_t s) {
  return gather_launch("cnhip_gather_rows", src, dst, F, nullptr, nullptr, 0, idx, N, B, s);
}

int cnhip_gather_batch(const float* xs, const float* ys, const int32_t* idx, float* x, float* y, int64_t N,
                       int64_t F, int64_t L, int64_t B, cnhip_stream_t s) {
  return gather_launch("cnhip_gather_batch", xs, x, F, ys, y, L, idx, N, B, s);
}

}  // extern "C"
