// Column slices shared by the column-sliced SpMM and attention.
//
// The column space [0, N) of a square graph is cut into kSlices = 8 equal
// ranges, one per XCD of an MI355X.  With columns ascending inside every row,
// the edges of row r in slice s form the contiguous range
// [crow[r] + off[r·7 + s-1], crow[r] + off[r·7 + s]) (off of slice 0 = 0, of
// slice 8 = the degree), found once per call by a binary search per
// (row, boundary).
#pragma once

#include "as_device.h"
#include "as_internal.h"

namespace as {
namespace {

constexpr int kSlices = 8;                 // one column slice per XCD
constexpr int kSliceBounds = kSlices - 1;  // inner slice points per row
constexpr int64_t kGridStrideBlocks = 65536;

// First column of slice b for an N-column space.
__device__ __forceinline__ int64_t slice_start(int64_t n_cols, int b) {
  return (n_cols * b + kSlices - 1) / kSlices;
}

// Rows shorter than `min_degree` are never sliced and keep no slice points.
__global__ __launch_bounds__(kBlock) void slice_points_kernel(const int64_t* __restrict__ crow,
                                                              const int64_t* __restrict__ col, int64_t n,
                                                              int64_t min_degree, int32_t* __restrict__ off) {
  const int64_t total = n * kSliceBounds;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int64_t r = t / kSliceBounds;
    const int b = static_cast<int>(t - r * kSliceBounds) + 1;
    const int64_t rs = crow[r];
    int64_t lo = rs;
    int64_t hi = crow[r + 1];
    if (hi - lo < min_degree) continue;
    const int64_t start = slice_start(n, b);
    while (lo < hi) {
      const int64_t mid = lo + ((hi - lo) >> 1);
      if (col[mid] < start) lo = mid + 1;
      else hi = mid;
    }
    off[t] = static_cast<int32_t>(lo - rs);
  }
}

inline void launch_slice_points(const int64_t* crow, const int64_t* col, int64_t n, int64_t min_degree,
                                int32_t* off, hipStream_t s) {
  int64_t blocks = (n * kSliceBounds + kBlock - 1) / kBlock;
  if (blocks > kGridStrideBlocks) blocks = kGridStrideBlocks;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(slice_points_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, crow, col, n,
                     min_degree, off);
}

// Edge range [a, b) of `slice` in a row of `deg` edges, relative to the row
// start; clamped to [0, deg] so that no access leaves the row.
__device__ __forceinline__ void slice_range(const int32_t* __restrict__ off, int64_t row, int slice, int64_t deg,
                                            int64_t& a, int64_t& b) {
  a = slice == 0 ? 0 : static_cast<int64_t>(off[row * kSliceBounds + slice - 1]);
  b = slice == kSlices - 1 ? deg : static_cast<int64_t>(off[row * kSliceBounds + slice]);
  a = a < 0 ? 0 : (a > deg ? deg : a);
  b = b < a ? a : (b > deg ? deg : b);
}

}  // namespace
}  // namespace as
