// Device-side helpers for gfx950 (wave64) kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace as {

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & 63u); }
__device__ __forceinline__ int wave_in_block() { return static_cast<int>(threadIdx.x >> 6); }

// Broadcast lane `src` (wave-uniform) of v to the whole wave through an SGPR.
__device__ __forceinline__ int bcast_i32(int v, int src) {
  return __builtin_amdgcn_readlane(v, src);
}
__device__ __forceinline__ float bcast_f32(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ __forceinline__ int uniform_i32(int v) {
  return __builtin_amdgcn_readfirstlane(v);
}
// A 64-bit value every lane holds identically, moved to SGPRs so that
// control flow and address arithmetic on it stay scalar.
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
// Element offset of row c in a row-major [*, F] matrix, for c < 2^31 and
// F < 2^31 (one 32x32->64 multiply).
__device__ __forceinline__ int64_t row_offset(int c, int64_t F) {
  return static_cast<int64_t>(static_cast<uint64_t>(static_cast<uint32_t>(c)) *
                              static_cast<uint64_t>(static_cast<uint32_t>(F)));
}

// V consecutive floats owned by one lane.  Component-wise arithmetic is
// written out so that no packed-fp32 instruction is needed.
template <int V>
struct alignas(4 * V) FVec {
  float v[V];
};

template <int V>
__device__ __forceinline__ FVec<V> load_vec(const float* p) {
  return *reinterpret_cast<const FVec<V>*>(p);
}
// Load from a wave-uniform base plus a per-lane byte offset below 2^32, the
// shape of the SGPR-base global load.
template <int V>
__device__ __forceinline__ FVec<V> load_vec_off(const float* base, uint32_t byte_offset) {
  return *reinterpret_cast<const FVec<V>*>(reinterpret_cast<const char*>(base) + byte_offset);
}
template <int V>
__device__ __forceinline__ void store_vec(float* p, const FVec<V>& a) {
  *reinterpret_cast<FVec<V>*>(p) = a;
}

// Butterfly reductions over the 64 lanes: every lane ends with the same bits
// (each step adds a pair in both lanes, and fp32 addition is commutative).
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Inclusive prefix sum over the wave (Hillis-Steele with shfl_up).
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

}  // namespace as
