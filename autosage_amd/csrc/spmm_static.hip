// Allocation-free variant of the degree-split SpMM (as_spmm_csr_split_f32).
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc): the split
// SpMM's workspace — the row order, the two counts and the binning tables —
// lives in a file-scope device array instead of a caller buffer.  Every GPU
// the library runs on holds its own copy of the array (about 18 MiB) until the
// process ends.  The kernels are those of as_spmm_csr_split_f32; nothing in
// the scratch has to start at zero, because the binning kernels rewrite the
// tables, the order and counts[0..1] in full on every call.
//
// The array's name is a host-side stand-in in host code: its device address
// comes from hipGetSymbolAddress, looked up once per device (with that device
// current) on the first call there, and only that address is ever passed to
// kernels.
#include <mutex>

#include "as_internal.h"

namespace as {

size_t spmm_split_workspace_bytes(int64_t n);

namespace {

constexpr size_t kScratchBytes = size_t(18) << 20;
static_assert(AS_STATIC_MAX_ROWS == (1 << 22), "the scratch size below assumes 2^22 rows");

__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device.
int device_scratch(void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(AS_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return fail(AS_ERR_UNSUPPORTED, "device %d is beyond the static scratch table (%d devices)", device, kMaxDevices);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(AS_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                  hipGetErrorString(err));
    g_scratch[device] = ptr;
  }
  *out = g_scratch[device];
  return AS_OK;
}

}  // namespace
}  // namespace as

extern "C" {

int as_spmm_csr_split_f32_static(const int64_t* crow, const int64_t* col, const float* val, const float* x,
                                 float* y, int64_t n, int64_t nnz, int64_t f, int feature_tile,
                                 int waves_per_block, int64_t hub_threshold, int vec4, int hub_mode,
                                 void* stream) {
  as::clear_error();
  if (n > AS_STATIC_MAX_ROWS)
    return as::fail(AS_ERR_WORKSPACE, "the allocation-free split SpMM takes at most %d rows, got %lld",
                    AS_STATIC_MAX_ROWS, static_cast<long long>(n));
  if (n <= 0 || f <= 0) {
    // nothing to launch; the argument checks of the allocating entry point
    return as_spmm_csr_split_f32(crow, col, val, x, y, n, nnz, f, feature_tile, waves_per_block, hub_threshold,
                                 vec4, hub_mode, nullptr, 0, stream);
  }
  const size_t needed = as::spmm_split_workspace_bytes(n);
  if (needed > as::kScratchBytes)
    return as::fail(AS_ERR_WORKSPACE, "static scratch of %zu bytes is short of %zu", as::kScratchBytes, needed);
  if (stream != nullptr) {
    int current = -1;
    hipDevice_t owner = -1;
    if (hipGetDevice(&current) != hipSuccess || hipStreamGetDevice(static_cast<hipStream_t>(stream), &owner) !=
                                                    hipSuccess)
      return as::fail(AS_ERR_LAUNCH, "cannot tell the device of the stream");
    if (owner != current)
      return as::fail(AS_ERR_INVALID_ARGUMENT, "the stream belongs to device %d, the current device is %d",
                      static_cast<int>(owner), current);
  }
  void* ws = nullptr;
  const int st = as::device_scratch(&ws);
  if (st != AS_OK) return st;
  return as_spmm_csr_split_f32(crow, col, val, x, y, n, nnz, f, feature_tile, waves_per_block, hub_threshold, vec4,
                               hub_mode, ws, needed, stream);
}

}  // extern "C"
