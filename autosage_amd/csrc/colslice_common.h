// Column slices shared by the column-sliced SpMM and attention.
//
// The column space [0, N) of a square graph (or of the graph a row shard was
// cut from) is cut into S equal ranges (S a
// multiple of kSlices = 8, the XCD count of an MI355X; slice s runs on XCD
// s % 8).  With columns ascending inside every row, the edges of row r in
// slice s form the contiguous range
// [crow[r] + off[r·(S-1) + s-1], crow[r] + off[r·(S-1) + s]) (off of slice 0
// = 0, of slice S = the degree), found once per call by a binary search per
// (row, boundary).
#pragma once

#include "as_device.h"
#include "as_internal.h"

namespace as {
namespace {

constexpr int kSlices = 8;                 // XCDs, and the slices of the attention
constexpr int kSliceBounds = kSlices - 1;  // inner slice points per row at 8 slices
constexpr int64_t kGridStrideBlocks = 65536;

// First column of slice b of S for an N-column space.
template <int S>
__device__ __forceinline__ int64_t slice_start(int64_t n_cols, int b) {
  return (n_cols * b + S - 1) / S;
}

// Rows shorter than `min_degree` are never sliced and keep no slice points.
// by_edges: slice b of a row of d edges starts at edge floor(d·b / S) (equal
// runs of edges, for graphs whose columns do not ascend).  n_cols: the
// column space the slices cut (n for a square graph; the full graph's N for
// a shard of its rows).
template <int S>
__global__ __launch_bounds__(kBlock) void slice_points_kernel(const int64_t* __restrict__ crow,
                                                              const int64_t* __restrict__ col, int64_t n,
                                                              int64_t n_cols, int64_t min_degree,
                                                              int32_t* __restrict__ off, bool by_edges) {
  constexpr int kBounds = S - 1;
  const int64_t total = n * kBounds;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int64_t r = t / kBounds;
    const int b = static_cast<int>(t - r * kBounds) + 1;
    const int64_t rs = crow[r];
    int64_t lo = rs;
    int64_t hi = crow[r + 1];
    if (hi - lo < min_degree) continue;
    if (by_edges) {
      off[t] = static_cast<int32_t>((hi - lo) * b / S);
      continue;
    }
    const int64_t start = slice_start<S>(n_cols, b);
    while (lo < hi) {
      const int64_t mid = lo + ((hi - lo) >> 1);
      if (col[mid] < start) lo = mid + 1;
      else hi = mid;
    }
    off[t] = static_cast<int32_t>(lo - rs);
  }
}

template <int S = kSlices>
inline void launch_slice_points(const int64_t* crow, const int64_t* col, int64_t n, int64_t min_degree,
                                int32_t* off, hipStream_t s, bool by_edges = false, int64_t n_cols = -1) {
  int64_t blocks = (n * (S - 1) + kBlock - 1) / kBlock;
  if (blocks > kGridStrideBlocks) blocks = kGridStrideBlocks;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(slice_points_kernel<S>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, crow, col, n,
                     n_cols < 0 ? n : n_cols, min_degree, off, by_edges);
}

// Edge range [a, b) of `slice` (of S) in a row of `deg` edges, relative to
// the row start; clamped to [0, deg] so that no access leaves the row.
template <int S = kSlices>
__device__ __forceinline__ void slice_range(const int32_t* __restrict__ off, int64_t row, int slice, int64_t deg,
                                            int64_t& a, int64_t& b) {
  a = slice == 0 ? 0 : static_cast<int64_t>(off[row * (S - 1) + slice - 1]);
  b = slice == S - 1 ? deg : static_cast<int64_t>(off[row * (S - 1) + slice]);
  a = a < 0 ? 0 : (a > deg ? deg : a);
  b = b < a ? a : (b > deg ? deg : b);
}

// A slice plan: the per-graph part of a column-sliced call, which depends on
// the graph, the slicing degree and the number of light buckets only (not on
// the features): the slice points of every row of slicing degree
// (off[n·(S-1)]), the degree-binned row order (order[n]), the bucket counts
// and the binning tables.  The tag packs the two settings, so that a call can
// check that it was given a plan built for its own.
struct SlicePlan {
  int32_t* off;
  int32_t* order;
  int32_t* counts;
  void* bin_ws;
};

template <int S = kSlices>
inline size_t slice_plan_bytes(int64_t n) {
  const size_t rows = static_cast<size_t>(n > 0 ? n : 1);
  return align_up(rows * (S - 1) * sizeof(int32_t), 256) + align_up(rows * sizeof(int32_t), 256) + 256 +
         bin_workspace_bytes(n);
}

template <int S = kSlices>
inline SlicePlan slice_plan_view(void* base, int64_t n) {
  char* p = static_cast<char*>(base);
  const size_t rows = static_cast<size_t>(n > 0 ? n : 1);
  SlicePlan v;
  v.off = reinterpret_cast<int32_t*>(p);
  p += align_up(rows * (S - 1) * sizeof(int32_t), 256);
  v.order = reinterpret_cast<int32_t*>(p);
  p += align_up(rows * sizeof(int32_t), 256);
  v.counts = reinterpret_cast<int32_t*>(p);
  p += 256;
  v.bin_ws = p;
  return v;
}

// What a plan was built for, checked by the calls that read it: the plan's
// kind (the SpMM's row-block layout or the attention's whole-graph order),
// the row blocks of an SpMM plan, the light buckets, whether it is a row
// shard's plan (columns cut over another row count) and the slicing degree.
enum : int64_t { kPlanKindSpmm = 1, kPlanKindAttention = 2 };
inline int64_t slice_plan_tag(int64_t min_degree, int light_buckets, int64_t kind = kPlanKindAttention,
                              int64_t blocks = 1, bool rect = false) {
  return (int64_t(1) << 62) | (kind << 56) | ((blocks & 0xff) << 48) |
         (static_cast<int64_t>(light_buckets & 0xff) << 40) | (static_cast<int64_t>(rect) << 39) |
         (min_degree & ((int64_t(1) << 39) - 1));
}

// order: rows of degree >= min_degree in 8 log2-degree buckets, longest
// first, then the shorter rows in `light_buckets` log2-degree buckets.
// n_cols < 0: a square graph (n columns).
template <int S = kSlices>
inline int build_slice_plan(const int64_t* crow, const int64_t* col, int64_t n, int64_t min_degree,
                            int light_buckets, bool by_edges, const SlicePlan& plan, hipStream_t s,
                            int64_t n_cols = -1) {
  launch_slice_points<S>(crow, col, n, min_degree, plan.off, s, by_edges, n_cols);
  return launch_bin_rows(crow, n, min_degree, kMaxHeavyBuckets, light_buckets, plan.order, plan.counts, plan.bin_ws,
                         s);
}

}  // namespace
}  // namespace as
