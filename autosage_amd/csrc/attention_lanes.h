// Lane layout shared by the column-sliced attention and its backward: a lane
// holds one 16-byte piece of a feature row (4 fp32 or 8 bf16 / fp16
// elements), converted exactly to fp32; results are rounded once to the
// element type when stored.
#pragma once

#include "as_device.h"
#include "elem16.h"

namespace as {
namespace {

// Rows of at least this degree are cut into column slices; shorter rows run
// whole (one wave each for fp32, several to a wave for 16-bit elements).
// On the 2.4M-row, 124M-edge benchmark attention (Fqk 64, Fv 128, median
// degree 16) fp32 is fastest from 128 (forward 11.17 ms, forward + backward
// 35.86; 512: 11.27 / 36.29) and bf16 from 512 (forward 5.68 against 6.07 at
// 128, forward + backward 19.63 against 21.23; 1024: 5.69 / 19.54): K and V
// do not fit the caches there, and the grouped short-row kernels run longer
// rows at the fabric rate without the partial states.  The forward and the
// backward share the per-graph plans built with it.
#ifndef AS_ATT_SLICE_MIN_DEGREE
#define AS_ATT_SLICE_MIN_DEGREE 128
#endif
#ifndef AS_ATT_SLICE_MIN_DEGREE_16
#define AS_ATT_SLICE_MIN_DEGREE_16 512
#endif
template <typename T>
constexpr int64_t att_slice_degree() {
  return sizeof(T) == 2 ? AS_ATT_SLICE_MIN_DEGREE_16 : AS_ATT_SLICE_MIN_DEGREE;
}

// Elements of type T in one 16-byte lane.
template <typename T>
constexpr int lane_elems() {
  return 16 / static_cast<int>(sizeof(T));
}

template <int P>
__device__ __forceinline__ void merge_softmax(float& m, float& l, float (&acc)[P], float mo, float lo,
                                              const float (&ao)[P]) {
  const float mn = fmaxf(m, mo);
  if (mn == -INFINITY) return;  // both sides saw no edge
  const float c1 = m == -INFINITY ? 0.f : expf(m - mn);
  const float c2 = mo == -INFINITY ? 0.f : expf(mo - mn);
  l = l * c1 + lo * c2;
#pragma unroll
  for (int v = 0; v < P; ++v) acc[v] = acc[v] * c1 + ao[v] * c2;
  m = mn;
}

// The P elements of a 16-byte lane as exact fp32 values.
template <typename T>
__device__ __forceinline__ void lane_values(const RawVec<16>& r, float (&out)[lane_elems<T>()]) {
#pragma unroll
  for (int v = 0; v < lane_elems<T>(); ++v) out[v] = Elem<T>::get(r.w, v);
}

template <typename T, int GK>
__device__ __forceinline__ void load_query_lanes(const T* __restrict__ query, int64_t row, int64_t fqk,
                                                 float (&q)[lane_elems<T>()]) {
  constexpr int P = lane_elems<T>();
  const int kl = lane_id() % GK;
  if (P * kl < fqk) {
    lane_values<T>(load_raw<16>(reinterpret_cast<const char*>(query + row * fqk + P * kl)), q);
  } else {
#pragma unroll
    for (int v = 0; v < P; ++v) q[v] = 0.f;
  }
}

// N consecutive outputs (N = 4 or 8, 4·N-byte aligned for fp32, 2·N-byte
// for 16-bit), each rounded once to T.
template <typename T, int N>
__device__ __forceinline__ void store_out(T* p, const float (&v)[N]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      FVec<4> o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o.v[k] = v[i + k];
      store_vec<4>(reinterpret_cast<float*>(p) + i, o);
    }
  } else {
    uint32_t w[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i)
      w[i] = uint32_t(Elem<T>::bits(v[2 * i])) | (uint32_t(Elem<T>::bits(v[2 * i + 1])) << 16);
    if constexpr (N == 8) {
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    }
  }
}

// Lanes per K (or V) row: one 16-byte lane per P elements, a power of two;
// fp32 keeps at least 16 lanes (4 edges per gather), 16-bit at least 8.
template <typename T>
int lane_group(int64_t f) {
  if constexpr (sizeof(T) == 4) {
    return f <= 64 ? 16 : (f <= 128 ? 32 : 64);
  } else {
    return f <= 64 ? 8 : (f <= 128 ? 16 : (f <= 256 ? 32 : 64));
  }
}

}  // namespace
}  // namespace as
