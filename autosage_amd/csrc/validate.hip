// CSR structure check on the device.
//
// The reference kernels trust their inputs (an out-of-range column reads
// out of bounds).  This pass lets a caller reject a malformed graph before
// any gather runs: crow[0] == 0, crow non-decreasing, crow[n] == nnz and
// 0 <= col[e] < n_cols.  It writes a bit mask of the violated rules to a
// caller-provided int32, plus bit 16 when columns are not ascending within
// some row (allowed, but the column-sliced SpMM needs ascending columns);
// it never reads col or crow out of bounds.
#include "as_device.h"
#include "as_internal.h"

namespace as {

namespace {

enum : int32_t {
  kBadFirst = 1,      // crow[0] != 0
  kBadOrder = 2,      // crow[r+1] < crow[r] for some r
  kBadLast = 4,       // crow[n] != nnz
  kBadColumn = 8,     // a column index outside [0, n_cols)
  kUnsorted = 16,     // columns descend somewhere inside a row (not an error)
};

__global__ __launch_bounds__(kBlock) void csr_validate_kernel(const int64_t* __restrict__ crow,
                                                              const int64_t* __restrict__ col, int64_t n,
                                                              int64_t nnz, int64_t n_cols,
                                                              int32_t* __restrict__ flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int32_t bad = 0;
  if (tid == 0) {
    if (crow[0] != 0) bad |= kBadFirst;
    if (crow[n] != nnz) bad |= kBadLast;
  }
  for (int64_t r = tid; r < n; r += stride) {
    if (crow[r + 1] < crow[r]) bad |= kBadOrder;
  }
  for (int64_t e = tid; e < nnz; e += stride) {
    const int64_t c = col[e];
    if (c < 0 || c >= n_cols) bad |= kBadColumn;
  }
  if (bad != 0) atomicOr(flags, bad);
}

// Wave per row: does any edge have a smaller column than its predecessor in
// the same row?  Row bounds are clamped to [0, nnz] so that a malformed crow
// (reported by the kernel above) cannot lead this one out of bounds.
__global__ __launch_bounds__(kBlock) void csr_sorted_kernel(const int64_t* __restrict__ crow,
                                                            const int64_t* __restrict__ col, int64_t n,
                                                            int64_t nnz, int32_t* __restrict__ flags) {
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
  bool unsorted = false;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block(); r < n; r += waves) {
    int64_t rs = crow[r];
    int64_t re = crow[r + 1];
    rs = rs < 0 ? 0 : (rs > nnz ? nnz : rs);
    re = re < rs ? rs : (re > nnz ? nnz : re);
    for (int64_t e = rs + 1 + lane_id(); e < re; e += kWave) {
      if (col[e] < col[e - 1]) unsorted = true;
    }
  }
  if (unsorted) atomicOr(flags, static_cast<int32_t>(kUnsorted));
}

}  // namespace

}  // namespace as

extern "C" {

int as_csr_validate(const int64_t* crow, const int64_t* col, int64_t n, int64_t nnz, int64_t n_cols,
                    int32_t* flags, void* stream) {
  as::clear_error();
  if (n < 0 || nnz < 0 || n_cols < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "sizes must be non-negative");
  if (crow == nullptr || flags == nullptr || (nnz > 0 && col == nullptr))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int64_t work = n > nnz ? n : nnz;
  int64_t blocks = (work + as::kBlock - 1) / as::kBlock;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(as::csr_validate_kernel, dim3(static_cast<unsigned>(blocks)), dim3(as::kBlock), 0,
                     static_cast<hipStream_t>(stream), crow, col, n, nnz, n_cols, flags);
  if (n > 0 && nnz > 0) {
    int64_t row_blocks = (n + as::kWavesPerBlock - 1) / as::kWavesPerBlock;
    if (row_blocks > 4096) row_blocks = 4096;
    hipLaunchKernelGGL(as::csr_sorted_kernel, dim3(static_cast<unsigned>(row_blocks)), dim3(as::kBlock), 0,
                       static_cast<hipStream_t>(stream), crow, col, n, nnz, flags);
  }
  return as::check_launch("csr_validate");
}

}  // extern "C"
