// Degree binning on the device, without a host synchronisation.
//
// Reference integer work: csrc/launcher_spmm.cu:13-18 (degrees) and :49-59
// (heavy = degree >= T, heavy and light row lists ascending via at::nonzero).
//
// Generalised to K heavy and L light buckets (1 <= K, L <= kMaxHeavyBuckets):
// a heavy row of degree d goes to bucket K-1-min(K-1, floor(log2(d / T))), so
// bucket 0 holds the longest rows; a light row (d < T) goes to bucket
// K + min(L-1, floor(log2((T-1) / d))) (empty rows to the last bucket), so
// light rows are also ordered from long to short.  The output is one
// permutation
//   order = [bucket 0 rows, ..., bucket K+L-1 rows]
// with each bucket ascending by row id, plus counts[0] = H (heavy rows) and
// counts[1] = n - H.  With K = L = 1 this is exactly the reference's heavy
// list followed by its light list.
//
// Three kernels over tiles of kBinTile rows:
//   hist    — per-tile count of every bin (bin-major table);
//   scan    — one workgroup: exclusive prefix over the bin-major table, which
//             yields each (bin, tile) output offset; writes counts[];
//   scatter — each row is written at its (bin, tile) offset plus its rank
//             among the tile's earlier rows of the same bin.
#include "as_device.h"
#include "as_internal.h"

namespace as {

namespace {

__device__ __forceinline__ int bin_of(int64_t deg, int64_t threshold, int buckets, int light_buckets) {
  if (deg < threshold) {
    if (deg == 0) return buckets + light_buckets - 1;
    const uint64_t q = static_cast<uint64_t>((threshold - 1) / deg);  // >= 1
    int level = 63 - __clzll(static_cast<long long>(q));
    if (level > light_buckets - 1) level = light_buckets - 1;
    return buckets + level;
  }
  const uint64_t q = static_cast<uint64_t>(deg / threshold);  // >= 1
  int level = 63 - __clzll(static_cast<long long>(q));
  if (level > buckets - 1) level = buckets - 1;
  return buckets - 1 - level;
}

// Exclusive prefix sum over a workgroup of up to 1024 threads; `lds` needs
// blockDim.x / 64 ints; *total receives the workgroup sum.
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

__device__ __forceinline__ void row_bins(const int64_t* __restrict__ crow, int64_t n, int64_t threshold,
                                         int buckets, int light_buckets, int64_t first,
                                         int (&bin)[kBinRowsPerThread]) {
#pragma unroll
  for (int i = 0; i < kBinRowsPerThread; ++i) {
    const int64_t r = first + i;
    bin[i] = r < n ? bin_of(crow[r + 1] - crow[r], threshold, buckets, light_buckets) : -1;
  }
}

__global__ __launch_bounds__(kBlock) void bin_hist_kernel(const int64_t* __restrict__ crow, int64_t n,
                                                          int64_t threshold, int buckets, int light_buckets,
                                                          int64_t tiles, int32_t* __restrict__ table) {
  __shared__ int lds[kBlock / kWave];
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBinTile + threadIdx.x * kBinRowsPerThread;
  int bin[kBinRowsPerThread];
  row_bins(crow, n, threshold, buckets, light_buckets, first, bin);
  for (int b = 0; b < buckets + light_buckets; ++b) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < kBinRowsPerThread; ++i) c += bin[i] == b ? 1 : 0;
    int total = 0;
    block_excl_scan(c, lds, &total);
    if (threadIdx.x == 0) table[b * tiles + blockIdx.x] = total;
  }
}

constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void bin_scan_kernel(const int32_t* __restrict__ table, int64_t entries,
                                                                int64_t heavy_entries, int64_t n,
                                                                int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ counts) {
  __shared__ int lds[kScanThreads / kWave];
  __shared__ int heavy_part[kScanThreads / kWave];
  const int64_t per = (entries + kScanThreads - 1) / kScanThreads;
  const int64_t begin = static_cast<int64_t>(threadIdx.x) * per;
  const int64_t end = begin + per < entries ? begin + per : entries;
  // each thread's entries are read once, 8 loads in flight at a time
  int local = 0;
  int local_heavy = 0;
#pragma unroll 8
  for (int64_t t = begin; t < end; ++t) {
    const int v = table[t];
    local += v;
    if (t < heavy_entries) local_heavy += v;
  }
  int total = 0;
  int running = block_excl_scan(local, lds, &total);
#pragma unroll 8
  for (int64_t t = begin; t < end; ++t) {
    offsets[t] = running;
    running += table[t];
  }
  int heavy_total = 0;
  block_excl_scan(local_heavy, heavy_part, &heavy_total);
  if (threadIdx.x == 0) {
    counts[0] = heavy_total;
    counts[1] = static_cast<int32_t>(n - heavy_total);
  }
}

__global__ __launch_bounds__(kBlock) void bin_scatter_kernel(const int64_t* __restrict__ crow, int64_t n,
                                                             int64_t threshold, int buckets, int light_buckets,
                                                             int64_t tiles, const int32_t* __restrict__ offsets,
                                                             int32_t* __restrict__ order) {
  __shared__ int lds[kBlock / kWave];
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBinTile + threadIdx.x * kBinRowsPerThread;
  int bin[kBinRowsPerThread];
  row_bins(crow, n, threshold, buckets, light_buckets, first, bin);
  for (int b = 0; b < buckets + light_buckets; ++b) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < kBinRowsPerThread; ++i) c += bin[i] == b ? 1 : 0;
    int total = 0;
    const int excl = block_excl_scan(c, lds, &total);
    if (total == 0) continue;  // workgroup-uniform
    int64_t pos = static_cast<int64_t>(offsets[b * tiles + blockIdx.x]) + excl;
#pragma unroll
    for (int i = 0; i < kBinRowsPerThread; ++i) {
      if (bin[i] == b) order[pos++] = static_cast<int32_t>(first + i);
    }
  }
}

}  // namespace

size_t bin_workspace_bytes(int64_t n) {
  const int64_t tiles = bin_tiles(n) > 0 ? bin_tiles(n) : 1;
  return 2 * align_up(static_cast<size_t>(tiles) * (2 * kMaxHeavyBuckets) * sizeof(int32_t), 256);
}

const int32_t* bin_bucket_start(const void* workspace, int64_t n, int bucket) {
  const int64_t tiles = bin_tiles(n);
  if (tiles <= 0) return nullptr;
  const int32_t* offsets =
      reinterpret_cast<const int32_t*>(static_cast<const char*>(workspace) + bin_workspace_bytes(n) / 2);
  return offsets + static_cast<int64_t>(bucket) * tiles;
}

int launch_bin_rows(const int64_t* crow, int64_t n, int64_t threshold, int buckets, int light_buckets,
                    int32_t* order, int32_t* counts, void* workspace, hipStream_t stream) {
  if (buckets < 1 || buckets > kMaxHeavyBuckets || light_buckets < 1 || light_buckets > kMaxHeavyBuckets)
    return fail(AS_ERR_INVALID_ARGUMENT, "bad bucket counts %d/%d", buckets, light_buckets);
  const int64_t tiles = bin_tiles(n);
  const size_t half = bin_workspace_bytes(n) / 2;
  int32_t* table = static_cast<int32_t*>(workspace);
  int32_t* offsets = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + half);
  const int64_t entries = (buckets + light_buckets) * tiles;
  if (tiles > 0) {
    hipLaunchKernelGGL(bin_hist_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0, stream, crow, n,
                       threshold, buckets, light_buckets, tiles, table);
  }
  hipLaunchKernelGGL(bin_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, table, entries, buckets * tiles, n,
                     offsets, counts);
  if (tiles > 0) {
    hipLaunchKernelGGL(bin_scatter_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kBlock), 0, stream, crow, n,
                       threshold, buckets, light_buckets, tiles, offsets, order);
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
  return as::launch_bin_rows(crow, n, threshold, 1, 1, order, counts, workspace, static_cast<hipStream_t>(stream));
}

}  // extern "C"
