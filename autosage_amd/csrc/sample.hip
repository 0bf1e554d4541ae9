// Induced sub-graph of a row sample, on the device.
//
// Reference behaviour: autosage/_auto.py:95-154 (_induced_sample_csr), a
// composition of about fifteen torch ops with two host syncs.  Given the
// sorted sample `selected` (the caller draws it with the reference's seeded
// randperm), sampled row i keeps the edges of row selected[i] whose column
// is also sampled, in CSR order, with the column renamed to its sample index.
// Here that is two passes of one wave per sampled row:
//   count:  remap[] (-1, or the sample index of a sampled row), then per row
//           the number of kept edges (wave ballots), an in-place scan gives
//           new_crow;
//   fill:   the same walk writes the kept edges at new_crow[i] + (kept
//           edges before this one in the row): order-preserving compaction.
// The outputs are the reference's, bit for bit.  A column outside [0, n)
// (invalid input, where the reference's index_select fails) is dropped here
// rather than read out of bounds.
#include "as_device.h"
#include "as_internal.h"

namespace as {

namespace {

constexpr int kSampleScanThreads = 1024;
constexpr int64_t kSampleBlocks = 8192;

__global__ __launch_bounds__(kBlock) void remap_fill_kernel(int32_t* __restrict__ remap, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) remap[i] = -1;
}

__global__ __launch_bounds__(kBlock) void remap_scatter_kernel(const int64_t* __restrict__ selected, int64_t s,
                                                               int64_t n, int32_t* __restrict__ remap) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < s; i += stride) {
    const int64_t r = selected[i];
    if (r >= 0 && r < n) remap[r] = static_cast<int32_t>(i);
  }
}

// Kept-edge flag and renamed column of edge e of a sampled row.
__device__ __forceinline__ bool kept_edge(const int64_t* __restrict__ col, const int32_t* __restrict__ remap,
                                          int64_t n, int64_t e, int32_t& mapped) {
  const int64_t c = col[e];
  mapped = (c >= 0 && c < n) ? remap[c] : -1;
  return mapped >= 0;
}

// new_crow[1 + i] = kept edges of sampled row i.
__global__ __launch_bounds__(kBlock) void sample_count_kernel(const int64_t* __restrict__ crow,
                                                              const int64_t* __restrict__ col,
                                                              const int64_t* __restrict__ selected, int64_t s,
                                                              int64_t n, const int32_t* __restrict__ remap,
                                                              int64_t* __restrict__ new_crow) {
  const int lane = lane_id();
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block(); i < s; i += waves) {
    const int64_t r = uniform_i64(selected[i]);
    const int64_t rs = uniform_i64(crow[r]);
    const int64_t re = uniform_i64(crow[r + 1]);
    int64_t kept = 0;
    for (int64_t base = rs; base < re; base += kWave) {
      const int64_t e = base + lane;
      int32_t mapped = -1;
      const bool keep = e < re && kept_edge(col, remap, n, e, mapped);
      kept += __popcll(__ballot(keep));
    }
    if (lane == 0) new_crow[1 + i] = kept;
  }
}

// In-place inclusive scan of new_crow[1 .. s] (one workgroup): each thread
// owns a contiguous segment; segment totals are scanned in LDS.
__global__ __launch_bounds__(kSampleScanThreads) void sample_scan_kernel(int64_t* __restrict__ new_crow, int64_t s) {
  __shared__ int64_t totals[kSampleScanThreads];
  const int64_t seg = (s + kSampleScanThreads - 1) / kSampleScanThreads;
  const int64_t first = 1 + static_cast<int64_t>(threadIdx.x) * seg;
  const int64_t last = first + seg < s + 1 ? first + seg : s + 1;
  int64_t sum = 0;
  for (int64_t j = first; j < last; ++j) sum += new_crow[j];
  totals[threadIdx.x] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t run = 0;
    for (int t = 0; t < kSampleScanThreads; ++t) {
      const int64_t v = totals[t];
      totals[t] = run;
      run += v;
    }
    new_crow[0] = 0;
  }
  __syncthreads();
  int64_t run = totals[threadIdx.x];
  for (int64_t j = first; j < last; ++j) {
    run += new_crow[j];
    new_crow[j] = run;
  }
}

__global__ __launch_bounds__(kBlock) void sample_fill_kernel(const int64_t* __restrict__ crow,
                                                             const int64_t* __restrict__ col,
                                                             const float* __restrict__ val,
                                                             const int64_t* __restrict__ selected, int64_t s,
                                                             int64_t n, const int32_t* __restrict__ remap,
                                                             const int64_t* __restrict__ new_crow,
                                                             int64_t* __restrict__ new_col,
                                                             float* __restrict__ new_val) {
  const int lane = lane_id();
  const uint64_t below = (uint64_t(1) << lane) - 1;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block(); i < s; i += waves) {
    const int64_t r = uniform_i64(selected[i]);
    const int64_t rs = uniform_i64(crow[r]);
    const int64_t re = uniform_i64(crow[r + 1]);
    int64_t out = uniform_i64(new_crow[i]);
    for (int64_t base = rs; base < re; base += kWave) {
      const int64_t e = base + lane;
      int32_t mapped = -1;
      const bool keep = e < re && kept_edge(col, remap, n, e, mapped);
      const uint64_t mask = __ballot(keep);
      if (keep) {
        const int64_t at = out + __popcll(mask & below);
        new_col[at] = mapped;
        if (new_val != nullptr) new_val[at] = val[e];
      }
      out += __popcll(mask);
    }
  }
}

int64_t grid_for(int64_t work, int64_t per_block) {
  int64_t blocks = (work + per_block - 1) / per_block;
  if (blocks < 1) blocks = 1;
  return blocks > kSampleBlocks ? kSampleBlocks : blocks;
}

int validate_sample(const int64_t* crow, const int64_t* selected, int64_t n, int64_t s, const void* ws) {
  if (n < 0 || n > INT32_MAX) return fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (s < 0 || s > n) return fail(AS_ERR_INVALID_ARGUMENT, "sample size must lie in [0, N]");
  if (crow == nullptr || (s > 0 && selected == nullptr) || ws == nullptr)
    return fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  return AS_OK;
}

}  // namespace

}  // namespace as

extern "C" {

size_t as_induced_sample_workspace_bytes(int64_t n) {
  return as::align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(int32_t), 256);
}

int as_induced_sample_count(const int64_t* crow, const int64_t* col, int64_t n, const int64_t* selected, int64_t s,
                            int64_t* new_crow, void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  int st = as::validate_sample(crow, selected, n, s, workspace);
  if (st != AS_OK) return st;
  if (new_crow == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (workspace_bytes < as_induced_sample_workspace_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "induced sample needs %zu workspace bytes, got %zu",
                    as_induced_sample_workspace_bytes(n), workspace_bytes);
  const hipStream_t h = static_cast<hipStream_t>(stream);
  int32_t* remap = static_cast<int32_t*>(workspace);
  hipLaunchKernelGGL(as::remap_fill_kernel, dim3(static_cast<unsigned>(as::grid_for(n, as::kBlock))),
                     dim3(as::kBlock), 0, h, remap, n);
  if (s > 0) {
    hipLaunchKernelGGL(as::remap_scatter_kernel, dim3(static_cast<unsigned>(as::grid_for(s, as::kBlock))),
                       dim3(as::kBlock), 0, h, selected, s, n, remap);
    hipLaunchKernelGGL(as::sample_count_kernel,
                       dim3(static_cast<unsigned>(as::grid_for(s, as::kWavesPerBlock))), dim3(as::kBlock), 0, h,
                       crow, col, selected, s, n, remap, new_crow);
  }
  hipLaunchKernelGGL(as::sample_scan_kernel, dim3(1), dim3(as::kSampleScanThreads), 0, h, new_crow, s);
  return as::check_launch("induced_sample_count");
}

int as_induced_sample_fill(const int64_t* crow, const int64_t* col, const float* val, int64_t n,
                           const int64_t* selected, int64_t s, const int64_t* new_crow, int64_t* new_col,
                           float* new_val, const void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  int st = as::validate_sample(crow, selected, n, s, workspace);
  if (st != AS_OK) return st;
  if (new_crow == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if ((val == nullptr) != (new_val == nullptr))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "val and new_val must both be given or both be null");
  if (workspace_bytes < as_induced_sample_workspace_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "induced sample needs %zu workspace bytes, got %zu",
                    as_induced_sample_workspace_bytes(n), workspace_bytes);
  if (s == 0) return AS_OK;
  hipLaunchKernelGGL(as::sample_fill_kernel, dim3(static_cast<unsigned>(as::grid_for(s, as::kWavesPerBlock))),
                     dim3(as::kBlock), 0, static_cast<hipStream_t>(stream), crow, col, val, selected, s, n,
                     static_cast<const int32_t*>(workspace), new_crow, new_col, new_val);
  return as::check_launch("induced_sample_fill");
}

}  // extern "C"
