// bf16 / fp16 elements for the 16-bit SpMM and SDDMM: raw 16-bit words,
// exact conversions to fp32 / fp64, and fp32 -> 16-bit rounding (round to
// nearest even) written as integer work on the fp32 bits.
#pragma once

#include <cstdint>

#include "as_device.h"

namespace as {
namespace {

// Inputs and outputs of an op share one element type.  bf16 and fp16 values
// are held as raw 16-bit words; every element converts exactly to fp32 and
// fp64.
struct Bf16 {
  uint16_t bits;
};
struct Fp16 {
  uint16_t bits;
};

// fp32 -> bf16, round to nearest even; NaN -> the quiet NaN 0x7fc0.
__device__ __forceinline__ uint16_t bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// fp32 -> fp16, round to nearest even, from the IEEE formats: 16 bits of
// integer work on the fp32 bits.  Written out because the compiler merges a
// float -> half conversion that follows a double -> float one into a single
// double -> half rounding, which decides ties differently.
__device__ __forceinline__ uint16_t f16_bits(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u);  // NaN
  if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // >= 65520 rounds to inf
  if (ax < 0x38800000u) {
    // below 2^-14: a multiple of 2^-24; the scaling by 2^24 is exact and
    // rintf rounds half to even (1024 encodes 2^-14, the smallest normal)
    const float units = __uint_as_float(ax) * 16777216.0f;
    return static_cast<uint16_t>(sign | static_cast<uint32_t>(__builtin_rintf(units)));
  }
  uint32_t r = ax - (112u << 23);    // exponent bias 127 -> 15
  r += 0x0fffu + ((r >> 13) & 1u);   // round the 13 dropped bits half to even
  return static_cast<uint16_t>(sign | (r >> 13));
}

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  // element p of consecutive raw little-endian 32-bit words
  __device__ static float get(const uint32_t* w, int p) { return __uint_as_float(w[p]); }
  __device__ static float at(const float* p, int64_t i) { return p[i]; }
  __device__ static void put(float* p, double v) { *p = static_cast<float>(v); }
};
template <>
struct Elem<Bf16> {
  __device__ static float get(const uint32_t* w, int p) {
    const uint32_t x = w[p >> 1];
    return __uint_as_float((p & 1) ? (x & 0xffff0000u) : (x << 16));
  }
  __device__ static float at(const Bf16* p, int64_t i) { return __uint_as_float(uint32_t(p[i].bits) << 16); }
  __device__ static uint16_t bits(double v) { return bf16_bits(static_cast<float>(v)); }
  __device__ static void put(Bf16* p, double v) { p->bits = bits(v); }
};
template <>
struct Elem<Fp16> {
  __device__ static float get(const uint32_t* w, int p) {
    const uint32_t x = w[p >> 1];
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>((p & 1) ? (x >> 16) : x)));
  }
  __device__ static float at(const Fp16* p, int64_t i) {
    return static_cast<float>(__builtin_bit_cast(_Float16, p[i].bits));
  }
  __device__ static uint16_t bits(double v) { return f16_bits(static_cast<float>(v)); }
  __device__ static void put(Fp16* p, double v) { p->bits = bits(v); }
};

// BYTES consecutive bytes (2, 4, 8 or 16, naturally aligned) as 32-bit words;
// a 2-byte load fills the low half of w[0].
template <int BYTES>
struct RawVec {
  uint32_t w[BYTES >= 4 ? BYTES / 4 : 1];
};
template <int BYTES>
__device__ __forceinline__ RawVec<BYTES> load_raw(const char* p) {
  RawVec<BYTES> r;
  if constexpr (BYTES == 2) {
    r.w[0] = *reinterpret_cast<const uint16_t*>(p);
  } else {
    const FVec<BYTES / 4> v = *reinterpret_cast<const FVec<BYTES / 4>*>(p);
#pragma unroll
    for (int i = 0; i < BYTES / 4; ++i) r.w[i] = __float_as_uint(v.v[i]);
  }
  return r;
}

}  // namespace
}  // namespace as
