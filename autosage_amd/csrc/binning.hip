// Degree binning: stable partition of the rows into heavy (degree >= T) and
// light rows, both ascending — the integer work of the reference split
// launcher (csrc/launcher_spmm.cu:13-18 degrees, :49-59 nonzero lists),
// done on the device without a host synchronisation.
//
// Three small kernels over tiles of kBinTile rows:
//   count   — heavy rows per tile;
//   scan    — one workgroup turns tile counts into tile offsets and writes
//             counts[0] = H, counts[1] = n - H;
//   scatter — each row goes to order[heavy_before(r)] if heavy, else to
//             order[H + r - heavy_before(r)].
#include "as_device.h"
#include "as_internal.h"

namespace as {

namespace {

// Exclusive prefix sum over a workgroup of up to 1024 threads.
// `lds` needs blockDim.x / 64 ints.  Returns the exclusive prefix; *total
// receives the workgroup sum.
__device__ __forceinline__ int block_excl_scan(int v, int* lds, int* total) {
  const int lane = lane_id();
  const int wave = wave_in_block();
  const int waves = static_cast<int>(blockDim.x >> 6);
  const int incl = wave_incl_scan_i32(v);
  if (lane == 63) lds[wave] = incl;
  __syncthreads();
  int before = 0;
  int sum = 0;
  for (int w = 0; w < waves; ++w) {
    const int t = lds[w];
    before += (w < wave) ? t : 0;
    sum += t;
  }
  __syncthreads();
  *total = sum;
  return before + incl - v;
}

__device__ __forceinline__ int heavy_flags(const int64_t* __restrict__ crow, int64_t n,
                                           int64_t threshold, int64_t first, bool (&flag)[kBinRowsPerThread]) {
  int count = 0;
#pragma unroll
  for (int i = 0; i < kBinRowsPerThread; ++i) {
    const int64_t r = first + i;
    flag[i] = false;
    if (r < n) flag[i] = (crow[r + 1] - crow[r]) >= threshold;
    count += flag[i] ? 1 : 0;
  }
  return count;
}

__global__ __launch_bounds__(kBlock) void bin_count_kernel(const int64_t* __restrict__ crow, int64_t n,
                                                           int64_t threshold,
                                                           int32_t* __restrict__ tile_counts) {
  __shared__ int lds[kBlock / kWave];
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBinTile + threadIdx.x * kBinRowsPerThread;
  bool flag[kBinRowsPerThread];
  const int count = heavy_flags(crow, n, threshold, first, flag);
  int total = 0;
  block_excl_scan(count, lds, &total);
  if (threadIdx.x == 0) tile_counts[blockIdx.x] = total;
}

constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void bin_scan_kernel(const int32_t* __restrict__ tile_counts,
                                                                int64_t tiles, int64_t n,
                                                                int32_t* __restrict__ tile_offsets,
                                                                int32_t* __restrict__ counts) {
  __shared__ int lds[kScanThreads / kWave];
  const int64_t per = (tiles + kScanThreads - 1) / kScanThreads;
  const int64_t begin = static_cast<int64_t>(threadIdx.x) * per;
  const int64_t end = begin + per < tiles ? begin + per : tiles;
  int local = 0;
  for (int64_t t = begin; t < end; ++t) local += tile_counts[t];
  int total = 0;
  int running = block_excl_scan(local, lds, &total);
  for (int64_t t = begin; t < end; ++t) {
    tile_offsets[t] = running;
    running += tile_counts[t];
  }
  if (threadIdx.x == 0) {
    counts[0] = total;
    counts[1] = static_cast<int32_t>(n - total);
  }
}

__global__ __launch_bounds__(kBlock) void bin_scatter_kernel(const int64_t* __restrict__ crow, int64_t n,
                                                             int64_t threshold,
                                                             const int32_t* __restrict__ tile_offsets,
                                                             const int32_t* __restrict__ counts,
                                                             int32_t* __restrict__ order) {
  __shared__ int lds[kBlock / kWave];
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBinTile + threadIdx.x * kBinRowsPerThread;
  bool flag[kBinRowsPerThread];
  const int count = heavy_flags(crow, n, threshold, first, flag);
  int total = 0;
  const int excl = block_excl_scan(count, lds, &total);
  const int64_t heavy_total = counts[0];
  int64_t heavy_before = static_cast<int64_t>(tile_offsets[blockIdx.x]) + excl;
#pragma unroll
  for (int i = 0; i < kBinRowsPerThread; ++i) {
    const int64_t r = first + i;
    if (r < n) {
      if (flag[i]) {
        order[heavy_before] = static_cast<int32_t>(r);
        ++heavy_before;
      } else {
        order[heavy_total + (r - heavy_before)] = static_cast<int32_t>(r);
      }
    }
  }
}

}  // namespace

size_t bin_workspace_bytes(int64_t n) {
  const int64_t tiles = bin_tiles(n);
  return 2 * align_up(static_cast<size_t>(tiles > 0 ? tiles : 1) * sizeof(int32_t), 256);
}

int launch_bin_rows(const int64_t* crow, int64_t n, int64_t threshold, int32_t* order, int32_t* counts,
                    void* workspace, hipStream_t stream) {
  const int64_t tiles = bin_tiles(n);
  int32_t* tile_counts = static_cast<int32_t*>(workspace);
  int32_t* tile_offsets = reinterpret_cast<int32_t*>(
      static_cast<char*>(workspace) + align_up(static_cast<size_t>(tiles > 0 ? tiles : 1) * sizeof(int32_t), 256));
  if (tiles > 0) {
    hipLaunchKernelGGL(bin_count_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0, stream, crow, n,
                       threshold, tile_counts);
  }
  hipLaunchKernelGGL(bin_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, tile_counts, tiles, n, tile_offsets,
                     counts);
  if (tiles > 0) {
    hipLaunchKernelGGL(bin_scatter_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0, stream, crow, n,
                       threshold, tile_offsets, counts, order);
  }
  return check_launch("bin_rows_by_degree");
}

}  // namespace as

extern "C" {

size_t as_bin_workspace_bytes(int64_t n) { return as::bin_workspace_bytes(n < 0 ? 0 : n); }

int as_bin_rows_by_degree(const int64_t* crow, int64_t n, int64_t threshold, int32_t* order, int32_t* counts,
                          void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "row count %lld out of range", (long long)n);
  if (threshold <= 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "hub_threshold must be positive");
  if (crow == nullptr || counts == nullptr || (n > 0 && order == nullptr))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (workspace == nullptr || workspace_bytes < as::bin_workspace_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "binning needs %zu workspace bytes, got %zu", as::bin_workspace_bytes(n),
                    workspace_bytes);
  return as::launch_bin_rows(crow, n, threshold, order, counts, workspace, static_cast<hipStream_t>(stream));
}

}  // extern "C"
