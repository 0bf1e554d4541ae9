// Host-side internals shared by the kernel translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/autosage_hip.h"

namespace as {

constexpr int kWave = 64;        // CDNA wavefront width
constexpr int kBlock = 256;      // default workgroup: 4 waves
constexpr int kWavesPerBlock = kBlock / kWave;

// Largest number of workgroups one launch may use along x (grid work-items
// must stay below 2^32 on AMD hardware).
constexpr int64_t kMaxBlocksPerLaunch = int64_t(1) << 22;

// Error reporting: format into the thread-local message and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Converts the last HIP launch error (if any) into an as_status.
int check_launch(const char* what);
// Clears the thread-local message (called at the start of every entry point).
void clear_error();

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Feature widths must stay below 2^28: the kernels form a lane's byte offset
// inside a feature row as a 32-bit value (F · 8 bytes at most < 2^31).
constexpr int64_t kMaxFeatures = int64_t(1) << 28;

// Argument checks shared by the SpMM entry points (n < 2^31: kernels use
// 32-bit row indices; F below kMaxFeatures).
inline int validate_spmm(const int64_t* crow, const int64_t* col, const void* x, const void* y, int64_t n,
                         int64_t nnz, int64_t f) {
  if (n < 0 || n > INT32_MAX) return fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (f < 0) return fail(AS_ERR_INVALID_ARGUMENT, "F must be non-negative");
  if (f >= kMaxFeatures) return fail(AS_ERR_UNSUPPORTED, "F must be below 2^28 (32-bit lane offsets)");
  if (nnz < 0) return fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (n > 0 && f > 0 && (crow == nullptr || x == nullptr || y == nullptr))
    return fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (nnz > 0 && col == nullptr) return fail(AS_ERR_INVALID_ARGUMENT, "null col pointer");
  return AS_OK;
}

// Degree binning (binning.hip).
constexpr int kBinRowsPerThread = 4;
constexpr int kBinTile = kBlock * kBinRowsPerThread;
inline int64_t bin_tiles(int64_t n) { return (n + kBinTile - 1) / kBinTile; }
constexpr int kMaxHeavyBuckets = 8;
size_t bin_workspace_bytes(int64_t n);
// Writes order[n] = heavy rows (degree >= threshold) in `buckets` log2
// degree buckets, longest bucket first, then light rows in `light_buckets`
// buckets, longest first; rows ascending inside a bucket.  counts[0] = heavy,
// counts[1] = light (counts[2..3] are left to callers).  The workspace holds
// the per-tile bin table and offsets.  buckets = light_buckets = 1 gives the
// reference's two ascending lists.
int launch_bin_rows(const int64_t* crow, int64_t n, int64_t threshold,
                    int buckets, int light_buckets, int32_t* order,
                    int32_t* counts, void* workspace, hipStream_t stream);
// After launch_bin_rows on `workspace`: device address of the order index at
// which bucket `bucket` (heavy buckets first, then light ones) starts; null
// for n = 0.
const int32_t* bin_bucket_start(const void* workspace, int64_t n, int bucket);

}  // namespace as
