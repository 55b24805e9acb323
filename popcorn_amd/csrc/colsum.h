// Deterministic column sums of a [parts, cols] fp32 array of per-block partial
// rows (weight gradients), in a fixed order so repeated runs give identical
// bits. Stage one: block (cx, s) sums parts [s*kColSplit, (s+1)*kColSplit) of
// 256 columns into stage[s]; stage two sums the stage rows and rounds to T.
#pragma once

#include "common.h"

namespace pk {
namespace {

constexpr int kColThreads = 256;
constexpr int kColSplit = 32;  // partial rows summed per block in the first stage

// v[p0 * ld] + ... + v[(p1 - 1) * ld], added in index order; loads are issued
// eight at a time so their latencies overlap.
__device__ __forceinline__ float ordered_sum(const float* __restrict__ v, int64_t ld, int64_t p0, int64_t p1) {
  float s = 0.f;
  int64_t p = p0;
  for (; p + 8 <= p1; p += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = v[(p + u) * ld];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += t[u];
  }
  for (; p < p1; ++p) s += v[p * ld];
  return s;
}

__global__ __launch_bounds__(kColThreads) void column_sum_stage(const float* __restrict__ part,
                                                               float* __restrict__ stage, int64_t parts, int cols) {
  const int c = blockIdx.x * kColThreads + threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.y * kColSplit;
  const int64_t p1 = p0 + kColSplit < parts ? p0 + kColSplit : parts;
  if (c >= cols) return;
  stage[(int64_t)blockIdx.y * cols + c] = ordered_sum(part + c, cols, p0, p1);
}

// A block takes kFinalCols columns with kFinalLanes row lanes each: lane l sums
// stage rows l, l + kFinalLanes, ... in order, then lane 0 adds the lanes in
// order, so the result is the same on every run.
constexpr int kFinalCols = 32;
constexpr int kFinalLanes = kColThreads / kFinalCols;

template <typename T>
__global__ __launch_bounds__(kColThreads) void column_sum_final(const float* __restrict__ stage, T* __restrict__ out,
                                                               int64_t n, int cols) {
  __shared__ float acc[kFinalLanes][kFinalCols];
  const int cl = threadIdx.x % kFinalCols, rl = threadIdx.x / kFinalCols;
  const int c = blockIdx.x * kFinalCols + cl;
  float s = 0.f;
  if (c < cols && rl < n) s = ordered_sum(stage + rl * (int64_t)cols + c, (int64_t)kFinalLanes * cols, 0,
                                          (n - rl + kFinalLanes - 1) / kFinalLanes);
  acc[rl][cl] = s;
  __syncthreads();
  if (rl == 0 && c < cols) {
    float t = acc[0][cl];
#pragma unroll
    for (int r = 1; r < kFinalLanes; ++r) t += acc[r][cl];
    out[c] = from_f32<T>(t);
  }
}

// Rows of the first-stage array for `parts` partial rows.
inline int64_t stage_rows(int64_t parts) { return (parts + kColSplit - 1) / kColSplit; }

// out[c] = sum over p of part[p * cols + c], rounded once to T; stage holds
// stage_rows(parts) * cols floats.
template <typename T> void column_sums(const float* part, float* stage, T* out, int64_t parts, int cols,
                                       hipStream_t s) {
  const int64_t n = stage_rows(parts);
  const int cx = (cols + kColThreads - 1) / kColThreads;
  hipLaunchKernelGGL(column_sum_stage, dim3(cx, (unsigned)n), dim3(kColThreads), 0, s, part, stage, parts, cols);
  hipLaunchKernelGGL(column_sum_final<T>, dim3((cols + kFinalCols - 1) / kFinalCols), dim3(kColThreads), 0, s, stage,
                     out, n, cols);
}

}  // namespace
}  // namespace pk
