// Column-sliced SpMM Y = A·X (fp32, bf16 or fp16 in and out, fp64
// accumulation).
//
// Why.  An MI355X has 8 XCDs, each with its own 4 MB L2; the X-row gathers
// that miss it cross the fabric to the 256 MB MALL or HBM.  When one kernel
// walks whole rows, every XCD gathers from all of X and the eight L2s hold
// the same hot rows.  Here the column space [0, N) is cut into kSlices = 8
// equal ranges and workgroup g works only on slice g % 8.  The hardware
// dispatches the workgroups of a launch round-robin over the XCDs, so each
// XCD gathers only from its own eighth of X and the eight L2s cache eight
// times as many distinct rows.  (If the dispatch order were different the
// results would not change; only the cache benefit would be lost.)
//
// Steps.
//   1. Slice points: off[r·7 + b-1] = index, relative to crow[r], of the first
//      edge of row r whose column is >= the first column of slice b (a binary
//      search, valid because columns ascend within the row).  For 16-bit
//      features on graphs whose columns do not ascend, the slices are instead
//      8 equal runs of edges (no cache benefit, but long rows still spread
//      over 8 waves).
//   2. Degree order: rows of degree >= the slicing threshold in log2-degree
//      buckets, longest first (the binning kernel of the split SpMM), then
//      the shorter rows.
//   3. For each chunk of rows of that order: the slice kernel, one wave per
//      (row, slice), writes the fp64 partial sum of the row's edges in the
//      slice; the reduction kernel adds the non-empty partials of each row in
//      slice order in fp64 and rounds once.  A shorter row is summed whole by
//      one wave (in fp64, rounded once) that writes Y: its 8 partials would
//      cost more traffic than slicing saves.
//
// Arithmetic.  Products w·x of fp32 values are exact in fp64 and every
// partial and the final sum are fp64 additions, so each output is within
// about one fp32 rounding of the exact sum (tighter than a sequential fp32
// sum), and the result is deterministic.  It is not bit-identical to the
// sequential CSR product: that order is kept by spmm.hip.  With bf16 or fp16
// elements (weights rounded to the same type) the products are exact and
// the result is the fp64 sum rounded to fp32 and then to the element type
// (round to nearest even both times).  When the fp64 sum is exact (the
// products' bits span at most 53 places) it does not depend on the order of
// the additions, and every schedule here gives the bits of an fp64 sum in
// CSR order rounded the same way; otherwise the sums differ by less than
// 2^-52 of the largest partial, which changes the rounded result only for a
// sum that close to a tie.
#include <type_traits>
#include <vector>

#include "as_device.h"
#include "as_internal.h"
#include "colslice_common.h"
#include "elem16.h"

namespace as {

namespace {

constexpr int kColsliceLongRow = 1024;     // slice length from which U = 16
// Rows shorter than this are not sliced: 8 fp64 partial rows (128·F bytes
// written and read) cost more than the cache gain on their few gathers.
#ifndef AS_COLSLICE_MIN_DEGREE
#define AS_COLSLICE_MIN_DEGREE 128
#endif
constexpr int64_t kColsliceMinDegree = AS_COLSLICE_MIN_DEGREE;
// With fp32 rows of at most 64 features (256 bytes) a row's 8 partial rows
// weigh twice as much against its gathers, and rows of 128-255 edges are
// left whole: on the skewed 115M-edge benchmark graph at F = 64 that is
// 1.92 ms against 2.00 (thresholds 192-320 all within 1 %); at F >= 128 the
// same change costs 1-2 %.
// With 2-byte elements a row's fp64 partials weigh four times as much
// against its gathers as with fp32 (8·8·F bytes against 2·F a gathered row),
// and rows are sliced from degree 512: the skewed graph in bf16 takes 1.900
// ms at F = 128 and 4.290 at F = 256 with column slices from 512, against
// 2.160 / 4.497 from 128 and 1.922 / 4.466 with edge slices (F = 64: 1.056
// against 1.347 and 1.007; the scheduler times both).
inline int64_t column_slice_degree(int64_t f, int64_t elem_bytes) {
  if (elem_bytes == 2) return 4 * kColsliceMinDegree;
  return elem_bytes == 4 && f <= 64 ? 2 * kColsliceMinDegree : kColsliceMinDegree;
}
// With slices by edge count there is no cache gain, only the spread of long
// rows over 8 waves.
constexpr int64_t kEdgeSliceMinDegree = 1024;
#ifndef AS_COLSLICE_OVERLAP
#define AS_COLSLICE_OVERLAP 1
#endif
// Column slices per XCD, worked one after the other: 8·P slices in all, XCD x
// taking slices x, x + 8, ... in that order, so that at any time an XCD
// gathers from 1/(8·P) of X.
#ifndef AS_COLSLICE_PHASES
#define AS_COLSLICE_PHASES 1
#endif
constexpr int kPhases = AS_COLSLICE_PHASES;
constexpr int kSpmmSlices = kSlices * kPhases;
constexpr int kSpmmBounds = kSpmmSlices - 1;

// fp64 partials are written once and read once by the reduction: keep them
// out of the way of the X rows in the caches.  Rows that are not sliced are
// rounded once and written to Y.
__device__ __forceinline__ void store_out(double* p, double v) { __builtin_nontemporal_store(v, p); }
template <typename T>
__device__ __forceinline__ void store_out(T* p, double v) {
  Elem<T>::put(p, v);
}

// VR consecutive outputs of Y, rounded once.
template <typename T, int VR>
__device__ __forceinline__ void store_elems(T* p, const double (&v)[VR]) {
  if constexpr (std::is_same<T, float>::value) {
    FVec<VR> o;
#pragma unroll
    for (int i = 0; i < VR; ++i) o.v[i] = static_cast<float>(v[i]);
    store_vec<VR>(p, o);
  } else if constexpr (VR == 2) {
    *reinterpret_cast<uint32_t*>(p) = uint32_t(Elem<T>::bits(v[0])) | (uint32_t(Elem<T>::bits(v[1])) << 16);
  } else {
    p->bits = Elem<T>::bits(v[0]);
  }
}

// One wave sums edges [rs, re) of a row into out[0, F) in fp64 (F not a
// multiple of the wide-lane width, or X not 16-byte aligned).  Same lane
// layout as the exact wave-row kernel: lane owns V consecutive features,
// 64 column indices per coalesced load (one chunk ahead), broadcast through
// SGPRs, U gathers in flight.
template <typename T, int V, bool HAS_VAL, int U, typename OutT>
__device__ __forceinline__ void slice_row(const int64_t* __restrict__ col, const T* __restrict__ val,
                                          const T* __restrict__ x, OutT* __restrict__ out, int64_t F, int64_t rs,
                                          int64_t re) {
  constexpr int kBytes = V * static_cast<int>(sizeof(T));
  const int lane = lane_id();
  const char* __restrict__ xb = reinterpret_cast<const char*>(x);
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  for (int64_t f0 = 0; f0 < F; f0 += kWave * V) {
    const int64_t fl = f0 + static_cast<int64_t>(lane) * V;
    const bool active = fl < F;
    const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : 0) * sizeof(T));
    double acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0;
    int next_col = 0;
    float next_w = 1.f;
    if (lane < re - rs) {
      next_col = static_cast<int>(col[rs + lane]);
      if constexpr (HAS_VAL) next_w = Elem<T>::at(val, rs + lane);
    }
    auto add = [&](const RawVec<kBytes>& xv, float w) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const double xe = static_cast<double>(Elem<T>::get(xv.w, v));
        if constexpr (HAS_VAL) {
          acc[v] = __builtin_fma(static_cast<double>(w), xe, acc[v]);
        } else {
          acc[v] = acc[v] + xe;
        }
      }
    };
    for (int64_t base = rs; base < re; base += kWave) {
      const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
      const int my_col = next_col;
      const float my_w = next_w;
      const int64_t nb = base + kWave;
      if (nb < re && lane < re - nb) {
        next_col = static_cast<int>(col[nb + lane]);
        if constexpr (HAS_VAL) next_w = Elem<T>::at(val, nb + lane);
      }
      int j = 0;
      for (; j + U <= cnt; j += U) {
        RawVec<kBytes> xv[U];
        float w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = bcast_i32(my_col, j + u);
          w[u] = HAS_VAL ? bcast_f32(my_w, j + u) : 1.f;
          xv[u] = load_raw<kBytes>(xb + row_offset(c, F) * sizeof(T) + lane_bytes);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) add(xv[u], w[u]);
      }
      for (; j < cnt; ++j) {
        const int c = bcast_i32(my_col, j);
        const RawVec<kBytes> xv = load_raw<kBytes>(xb + row_offset(c, F) * sizeof(T) + lane_bytes);
        add(xv, HAS_VAL ? bcast_f32(my_w, j) : 1.f);
      }
    }
    if (active) {
#pragma unroll
      for (int v = 0; v < V; ++v) store_out(out + fl + v, acc[v]);
    }
  }
}

// Wide form of slice_row for F a multiple of P and 16-byte aligned X: G lanes
// per edge, each lane owning P = 16 / sizeof(T) consecutive features (one
// 16-byte load: 4 fp32 or 8 bf16 / fp16), so that one gather instruction
// fetches 64/G = EPI edges.  Gathers that hit L2 run at twice the bytes per
// instruction of 8-byte lanes (four times of 4-byte lanes).  Lane group k
// takes edges j + k, j + EPI + k, ... and keeps its own fp64 sums; the groups
// are added at the end in a fixed butterfly order.  One call covers the
// feature tile [f0, f0 + P·G).
template <typename T, int G, bool HAS_VAL, int U, typename OutT>
__device__ __forceinline__ void slice_row_wide(const int64_t* __restrict__ col, const T* __restrict__ val,
                                               const T* __restrict__ x, OutT* __restrict__ out, int64_t F,
                                               int64_t rs, int64_t re, int64_t f0) {
  constexpr int P = 16 / static_cast<int>(sizeof(T));
  constexpr int EPI = kWave / G;
  const int lane = lane_id();
  const int grp = lane / G;
  const int gl = lane % G;
  const char* __restrict__ xb = reinterpret_cast<const char*>(x);
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  {
    const int64_t fl = f0 + P * static_cast<int64_t>(gl);
    const bool active = fl < F;
    const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : f0) * sizeof(T));
    double acc[P];
#pragma unroll
    for (int v = 0; v < P; ++v) acc[v] = 0.0;
    int next_col = 0;
    float next_w = 1.f;
    if (lane < re - rs) {
      next_col = static_cast<int>(col[rs + lane]);
      if constexpr (HAS_VAL) next_w = Elem<T>::at(val, rs + lane);
    }
    for (int64_t base = rs; base < re; base += kWave) {
      const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
      const int my_col = next_col;
      const float my_w = next_w;
      const int64_t nb = base + kWave;
      if (nb < re && lane < re - nb) {
        next_col = static_cast<int>(col[nb + lane]);
        if constexpr (HAS_VAL) next_w = Elem<T>::at(val, nb + lane);
      }
      for (int j = 0; j < cnt; j += U * EPI) {
        RawVec<16> xv[U];
        float w[U];
        bool live[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          // this lane group's edge; past the end, a clamped valid edge whose
          // value is not added
          live[u] = j + u * EPI + grp < cnt;
          int c = 0;
          w[u] = 1.f;
#pragma unroll
          for (int k = 0; k < EPI; ++k) {
            const int e = j + u * EPI + k < cnt ? j + u * EPI + k : cnt - 1;
            const int ck = bcast_i32(my_col, e);
            c = grp == k ? ck : c;
            if constexpr (HAS_VAL) {
              const float wk = bcast_f32(my_w, e);
              w[u] = grp == k ? wk : w[u];
            }
          }
          xv[u] = load_raw<16>(xb + row_offset(c, F) * sizeof(T) + lane_bytes);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (live[u]) {
#pragma unroll
            for (int v = 0; v < P; ++v) {
              const double xe = static_cast<double>(Elem<T>::get(xv[u].w, v));
              if constexpr (HAS_VAL) {
                acc[v] = __builtin_fma(static_cast<double>(w[u]), xe, acc[v]);
              } else {
                acc[v] = acc[v] + xe;
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (int o = G; o < kWave; o <<= 1) {
#pragma unroll
      for (int v = 0; v < P; ++v) acc[v] += __shfl_xor(acc[v], o, kWave);
    }
    if (grp == 0 && active) {
#pragma unroll
      for (int v = 0; v < P; ++v) store_out(out + fl + v, acc[v]);
    }
  }
}

// slice_row_wide for 4 or more edges per gather (16- or 8-lane groups), with
// less issue work per gather and the same sums in the same order:
//   * the lane group's column index comes from one ds_bpermute of the 64
//     indices of the block (instead of EPI readlanes and selects);
//   * with OFF32 (X smaller than 4 GiB and fewer than 2^24 rows) the X byte
//     offset is one 24-bit multiply-add and the gather uses the SGPR base
//     with a 32-bit VGPR offset;
//   * full batches carry no per-edge liveness test; only the last batch of a
//     block has one.  A lane group past the end reads the index register of
//     a lane with no edge in this block, which holds an earlier valid column
//     (or 0), and does not add what it gathers.
// On the 115M-edge skewed benchmark graph at F = 64 fp32 this takes the call
// from 2.18 to 2.00 ms; with 32-lane groups (2 edges per gather) the same
// changes cost about 1 %, so those keep slice_row_wide.
template <typename T, int G, bool HAS_VAL, int U, bool OFF32, typename OutT>
__device__ __forceinline__ void slice_row_wide_bpermute(const int64_t* __restrict__ col,
                                                        const T* __restrict__ val, const T* __restrict__ x,
                                                        OutT* __restrict__ out, int64_t F, int64_t rs, int64_t re,
                                                        int64_t f0) {
  constexpr int P = 16 / static_cast<int>(sizeof(T));
  constexpr int EPI = kWave / G;
  constexpr int B = U * EPI;
  static_assert(kWave % B == 0, "a batch must not straddle a block of 64 column indices");
  const int lane = lane_id();
  const int grp = lane / G;
  const int gl = lane % G;
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  const int64_t fl = f0 + P * static_cast<int64_t>(gl);
  const bool active = fl < F;
  const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : f0) * sizeof(T));
  const uint32_t row_bytes = static_cast<uint32_t>(F * sizeof(T));
  const char* __restrict__ xb = reinterpret_cast<const char*>(x);
  double acc[P];
#pragma unroll
  for (int v = 0; v < P; ++v) acc[v] = 0.0;
  int next_col = 0;
  float next_w = 1.f;
  if (lane < re - rs) {
    next_col = static_cast<int>(col[rs + lane]);
    if constexpr (HAS_VAL) next_w = Elem<T>::at(val, rs + lane);
  }
  // edges e0 .. e0 + EPI - 1 of the block (e0 uniform), lane group grp
  // gathers edge e0 + grp
  auto gather = [&](int my_col, float my_w, int e0, float& w) -> RawVec<16> {
    const int addr = (e0 + grp) * 4;
    const int c = __builtin_amdgcn_ds_bpermute(addr, my_col);
    if constexpr (HAS_VAL) w = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(my_w)));
    if constexpr (OFF32) {
      return load_raw<16>(xb + (__umul24(static_cast<uint32_t>(c), row_bytes) + lane_bytes));
    } else {
      return load_raw<16>(xb + row_offset(c, F) * sizeof(T) + lane_bytes);
    }
  };
  auto add = [&](const RawVec<16>& xv, float w) {
#pragma unroll
    for (int v = 0; v < P; ++v) {
      const double xe = static_cast<double>(Elem<T>::get(xv.w, v));
      if constexpr (HAS_VAL) {
        acc[v] = __builtin_fma(static_cast<double>(w), xe, acc[v]);
      } else {
        acc[v] = acc[v] + xe;
      }
    }
  };
  for (int64_t base = rs; base < re; base += kWave) {
    const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
    const int my_col = next_col;
    const float my_w = next_w;
    const int64_t nb = base + kWave;
    if (nb < re && lane < re - nb) {
      next_col = static_cast<int>(col[nb + lane]);
      if constexpr (HAS_VAL) next_w = Elem<T>::at(val, nb + lane);
    }
    int j = 0;
    for (; j + B <= cnt; j += B) {
      RawVec<16> xv[U];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) xv[u] = gather(my_col, my_w, j + u * EPI, w[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) add(xv[u], w[u]);
    }
    if (j < cnt) {
      RawVec<16> xv[U];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) xv[u] = gather(my_col, my_w, j + u * EPI, w[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u * EPI + grp < cnt) add(xv[u], w[u]);
      }
    }
  }
#pragma unroll
  for (int o = G; o < kWave; o <<= 1) {
#pragma unroll
    for (int v = 0; v < P; ++v) acc[v] += __shfl_xor(acc[v], o, kWave);
  }
  if (grp == 0 && active) {
#pragma unroll
    for (int v = 0; v < P; ++v) store_out(out + fl + v, acc[v]);
  }
}

#ifndef AS_COLSLICE_WIDE_U
#define AS_COLSLICE_WIDE_U 4
#endif
#ifndef AS_COLSLICE_WIDE_U_16
#define AS_COLSLICE_WIDE_U_16 2
#endif

template <typename T, int G, bool HAS_VAL, bool OFF32, typename OutT>
__device__ __forceinline__ void slice_wide(const int64_t* __restrict__ col, const T* __restrict__ val,
                                           const T* __restrict__ x, OutT* __restrict__ out, int64_t F, int64_t rs,
                                           int64_t re, int64_t f0) {
  if constexpr (G <= 16) {
    // 16-bit lanes carry 8 fp64 sums: 2 gathers per batch keep the wave
    // within 64 VGPRs (8 waves per SIMD)
    constexpr int U = sizeof(T) == 2 ? AS_COLSLICE_WIDE_U_16 : AS_COLSLICE_WIDE_U;
    slice_row_wide_bpermute<T, G, HAS_VAL, U, OFF32>(col, val, x, out, F, rs, re, f0);
  } else {
    slice_row_wide<T, G, HAS_VAL, AS_COLSLICE_WIDE_U>(col, val, x, out, F, rs, re, f0);
  }
}

// Short rows of 16-bit features, one lane group of G lanes per row and
// 64/G rows per wave: each group walks its own row (one edge per gather
// instruction per group, no reduction across groups), so a wave keeps 64/G
// rows' dependent loads (order, crow, columns, gathers) in flight instead of
// one.  The column indices of a block of G edges are loaded one per lane and
// handed to the group by ds_bpermute; lanes past their row's end read column
// 0 (valid) and add nothing.  Only rows of degree below 4·G take this form
// (a lane group would walk a long row alone); both forms sum the same exact
// products in fp64.
#ifndef AS_COLSLICE_GROUPED_BLOCKS
#define AS_COLSLICE_GROUPED_BLOCKS 4
#endif
constexpr int kGroupedMaxBlocks = AS_COLSLICE_GROUPED_BLOCKS;  // grouped rows have fewer than 4·G edges (0: none)

// Element types and lane widths with a grouped form: 16-bit elements with
// wide lanes, fp32 with up to AS_COLSLICE_GROUPED_F32 lanes per edge.  fp32
// short rows grouped (two rows a wave at F >= 128, four at F = 64, rows below
// 4·G edges), against one wave per short row, on the skewed 115M-edge graph:
// F = 128 3.293 against 3.366 ms, F = 256 6.752 against 6.826, F = 64 1.750
// against 1.761 (grouping F = 64 only: 1.750 / 3.351 / 6.803; the short rows
// then also run in log2-degree buckets).
#ifndef AS_COLSLICE_GROUPED_F32
#define AS_COLSLICE_GROUPED_F32 32
#endif
// Gathers in flight per lane group and step in the grouped rows (must divide
// G).  fp32: 2 on the skewed graph at F = 64 / 128 / 256 1.760 / 3.270 /
// 6.765 ms, against 1.761 / 3.298 / 6.773 with 1 and 1.761 / 3.313 / 6.830
// with 4.  16-bit: 1 (bf16 with 2: skewed graph F = 128 1.907 against 1.909
// ms, F = 256 4.204 against 4.230, the 16.8M-edge uniform graph 0.646
// against 0.624).
#ifndef AS_COLSLICE_GROUPED_U_F32
#define AS_COLSLICE_GROUPED_U_F32 2
#endif
#ifndef AS_COLSLICE_GROUPED_U_16
#define AS_COLSLICE_GROUPED_U_16 1
#endif
template <typename T, int V>
constexpr bool grouped_lanes() {
  return sizeof(T) == 2 ? V >= 8 : (AS_COLSLICE_GROUPED_F32 != 0 && V >= 8 && V <= AS_COLSLICE_GROUPED_F32);
}

template <typename T, int G, bool HAS_VAL, int U, bool OFF32>
__device__ __forceinline__ void short_rows_grouped(const int64_t* __restrict__ crow, const int64_t* __restrict__ col,
                                                   const T* __restrict__ val, const T* __restrict__ x,
                                                   T* __restrict__ y, int64_t F, const int32_t* __restrict__ order,
                                                   int64_t item0, int64_t end, int64_t f0) {
  constexpr int P = 16 / static_cast<int>(sizeof(T));
  const int lane = lane_id();
  const int grp = lane / G;
  const int gl = lane % G;
  const int64_t item = item0 + grp;
  int64_t row = -1, rs = 0;
  int deg = 0;  // below the slicing threshold, so it fits an int
  if (item < end) {
    row = order[item];
    rs = crow[row];
    deg = static_cast<int>(crow[row + 1] - rs);
  }
  int maxdeg = deg;
#pragma unroll
  for (int o = G; o < kWave; o <<= 1) maxdeg = max(maxdeg, __shfl_xor(maxdeg, o, kWave));
  maxdeg = uniform_i32(maxdeg);
  const int64_t fl = f0 + P * static_cast<int64_t>(gl);
  const bool active = fl < F;
  const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : f0) * sizeof(T));
  const uint32_t row_bytes = static_cast<uint32_t>(F * sizeof(T));
  const char* __restrict__ xb = reinterpret_cast<const char*>(x);
  double acc[P];
#pragma unroll
  for (int v = 0; v < P; ++v) acc[v] = 0.0;
  for (int base = 0; base < maxdeg; base += G) {
    int my_col = 0;
    float my_w = 1.f;
    if (base + gl < deg) {
      my_col = static_cast<int>(col[rs + base + gl]);
      if constexpr (HAS_VAL) my_w = Elem<T>::at(val, rs + base + gl);
    }
    const int lim = maxdeg - base < G ? maxdeg - base : G;
    for (int j = 0; j < lim; j += U) {
      RawVec<16> xv[U];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int addr = (grp * G + j + u) * 4;
        const int c = __builtin_amdgcn_ds_bpermute(addr, my_col);
        w[u] = 1.f;
        if constexpr (HAS_VAL) w[u] = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(my_w)));
        if constexpr (OFF32) {
          xv[u] = load_raw<16>(xb + (__umul24(static_cast<uint32_t>(c), row_bytes) + lane_bytes));
        } else {
          xv[u] = load_raw<16>(xb + row_offset(c, F) * sizeof(T) + lane_bytes);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (base + j + u < deg) {
#pragma unroll
          for (int v = 0; v < P; ++v) {
            const double xe = static_cast<double>(Elem<T>::get(xv[u].w, v));
            if constexpr (HAS_VAL) {
              acc[v] = __builtin_fma(static_cast<double>(w[u]), xe, acc[v]);
            } else {
              acc[v] = acc[v] + xe;
            }
          }
        }
      }
    }
  }
  if (row >= 0 && active) {
#pragma unroll
    for (int v = 0; v < P; ++v) store_out(y + row * F + fl + v, acc[v]);
  }
}

// One chunk of the work: rows order[item_begin, item_begin + items); the
// first counts[0] rows of the order are sliced (at most `capacity` of them in
// a chunk: with 16-bit elements the rest are summed whole), the rest are
// short.  A launch
// is made of groups of 8 workgroups (one per XCD, by blockIdx % 8):
//   * slice groups, Gs per (feature tile, phase): block mb takes slice
//     8·p + mb % 8 and its 4 waves stride over the chunk's sliced rows; the
//     wave for (row, slice) writes the partial of chunk row `local` to
//     partial[(slice·chunk_stride + local)·F ..];
//   * short groups, Gh per feature tile: every wave sums whole short rows,
//     striding over them, and writes Y;
//   * reduce groups (colslice_reduce_block).
// Gs and Gh are capped, so a chunk of short rows does not launch 8 waves per
// row; the row counts come from counts[0] on the device, so the host needs no
// copy of it.  V in {1, 2}: narrow lanes (slice_row, all features); V = 8,
// 16, 32: wide lanes with G = V lanes per edge (slice_row_wide), one feature
// tile of 16·G / sizeof(T) features per wave.  Feature tiles are the
// outermost index: every (slice, row) of tile 0 comes before tile 1, so that
// while a tile runs each XCD gathers only 16·G bytes of the X rows of its
// slice (for wider rows this keeps the per-XCD working set of 512-byte rows).
struct SliceChunk {
  int64_t item_begin;
  int64_t items;
  double* partial;
  int64_t slice_groups;  // Gs: slice groups per (tile, phase)
  int64_t short_groups;  // Gh: short groups per tile
  int64_t sliced;        // the caller's count of sliced rows in the chunk, < 0 if unknown
  // partial rows of the buffer: sliced rows past them are summed whole
  // (16-bit elements only, whose results do not depend on the order)
  int64_t capacity = INT64_MAX;
};

// Where the grouped short rows (16-bit, degree below 4·G) start in the order:
// the start of a light degree bucket of the binning, read on the device.
// Device-side bucket boundaries of the binned order, read by the step
// kernels: where the grouped short rows start, and where the rows of the
// cooperative ("mega") degree end.
struct GroupedRows {
  const int32_t* start;  // null: no grouped rows
  const int32_t* mega_end = nullptr;  // null: no cooperative rows
};

// Rows of degree >= T·2^kMegaLevel (T the slicing degree; 8192 at T = 128)
// are the first heavy buckets of the order.  On graphs of at most
// kMegaMaxNnz edges all waves of a slice workgroup share one (row, slice) of
// such a row, each summing an equal run of its edges; the fp64 partials are
// added in wave order through LDS, so a hub row's slice no longer rests on
// one wave.  Wide lanes only (V >= 8).  The reference's hub sweep (20,000
// rows, one row of 12,000 edges, the others 32) takes 74.7 against 152.5 us;
// on larger graphs the other rows fill the GPU beside the hub slices and the
// workgroup's waiting costs more than it saves (the skewed 115M-edge graph at
// F = 128: 3.494 against 3.449 ms), so it stays off there.  Which rows
// cooperate depends only on N, nnz and the degrees, never on a launch hint.
#ifndef AS_COLSLICE_MEGA_LEVEL
#define AS_COLSLICE_MEGA_LEVEL 6
#endif
constexpr int kMegaLevel = AS_COLSLICE_MEGA_LEVEL;
constexpr int64_t kMegaMaxNnz = int64_t(1) << 24;

// An fp64 sum kept in LDS (plain stores, where partial rows in memory take
// non-temporal ones).
struct LdsSum {
  double v;
};
__device__ __forceinline__ void store_out(LdsSum* p, double v) { p->v = v; }

#ifndef AS_COLSLICE_SLICE_GROUPS
#define AS_COLSLICE_SLICE_GROUPS 4096
#endif
#ifndef AS_COLSLICE_SHORT_GROUPS
#define AS_COLSLICE_SHORT_GROUPS 8192
#endif
constexpr int64_t kSliceGroupsMax = AS_COLSLICE_SLICE_GROUPS;  // without a hint
constexpr int64_t kShortGroupsMax = AS_COLSLICE_SHORT_GROUPS;
constexpr int64_t kMaxSliceGroupsHinted = 65536;

// Group counts of a chunk of `items` rows of which `sliced` are expected to
// be sliced (the caller's hint; < 0 if unknown).  Any counts >= 1 cover all
// rows, since the waves stride; the hint only avoids looping waves (too few
// groups) and idle ones (too many).
inline void chunk_groups(SliceChunk& c, int64_t sliced, int64_t grouped, int64_t rows_per_wave) {
  int64_t gs, gh;
  if (sliced < 0) {
    gs = (c.items + kWavesPerBlock - 1) / kWavesPerBlock;
    gh = (c.items + kSlices * kWavesPerBlock - 1) / (kSlices * kWavesPerBlock);
    if (gs > kSliceGroupsMax) gs = kSliceGroupsMax;
  } else {
    if (sliced > c.items) sliced = c.items;
    // short waves: one per other short row, one per rows_per_wave grouped rows
    if (grouped < 0) grouped = 0;
    if (grouped > c.items - sliced) grouped = c.items - sliced;
    const int64_t waves = c.items - sliced - grouped + (grouped + rows_per_wave - 1) / rows_per_wave;
    gs = (sliced + kWavesPerBlock - 1) / kWavesPerBlock;
    gh = (waves + kSlices * kWavesPerBlock - 1) / (kSlices * kWavesPerBlock);
    if (gs > kMaxSliceGroupsHinted) gs = kMaxSliceGroupsHinted;
  }
  if (gh > kShortGroupsMax) gh = kShortGroupsMax;
  c.slice_groups = gs > 0 ? gs : 1;
  c.short_groups = gh > 0 ? gh : 1;
  c.sliced = sliced;
}

// Sliced rows of the chunk: [item_begin, fs), fs = counts[0] clamped.
__device__ __forceinline__ int64_t first_short(const int32_t* __restrict__ counts, const SliceChunk& c) {
  const int64_t h = counts[0];
  const int64_t end = c.item_begin + c.items;
  const int64_t cap_end = c.capacity < c.items ? c.item_begin + c.capacity : end;
  return h < c.item_begin ? c.item_begin : (h > cap_end ? cap_end : h);
}

template <typename T, int V, bool HAS_VAL, bool OFF32>
__device__ __forceinline__ void colslice_slice_block(int64_t mb, const int64_t* __restrict__ crow,
                                                     const int64_t* __restrict__ col, const T* __restrict__ val,
                                                     const T* __restrict__ x, int64_t F,
                                                     const int32_t* __restrict__ order,
                                                     const int32_t* __restrict__ counts,
                                                     const int32_t* __restrict__ off, const SliceChunk& c,
                                                     int64_t chunk_stride, const int32_t* __restrict__ mega_end) {
  constexpr int64_t kTile = 16 * V / static_cast<int64_t>(sizeof(T));  // features of a wide tile
  const int64_t gs = c.slice_groups;
  const int64_t phase_blocks = kSlices * gs;
  const int64_t tile_blocks = kPhases * phase_blocks;
  const int64_t tile = mb / tile_blocks;
  const int64_t in_tile = mb - tile * tile_blocks;
  const int64_t phase = in_tile / phase_blocks;
  const int64_t in_phase = in_tile - phase * phase_blocks;
  const int slice = static_cast<int>(phase * kSlices + in_phase % kSlices);
  const int64_t sliced = first_short(counts, c) - c.item_begin;
  int64_t mega = 0;
  if constexpr (V >= 8) {
    if (mega_end != nullptr) {
      mega = uniform_i64(static_cast<int64_t>(*mega_end)) - c.item_begin;
      mega = mega < 0 ? 0 : (mega > sliced ? sliced : mega);
    }
    // cooperative rows: the whole workgroup on one (row, slice), block-strided
    __shared__ LdsSum sums[kWavesPerBlock * kTile];
    const int w = wave_in_block();
    for (int64_t local = in_phase / kSlices; local < mega; local += gs) {
      const int64_t row = uniform_i64(order[c.item_begin + local]);
      const int64_t rs = uniform_i64(crow[row]);
      const int64_t deg = uniform_i64(crow[row + 1]) - rs;
      int64_t a, b;
      slice_range<kSpmmSlices>(off, row, slice, deg, a, b);
      a = uniform_i64(a);
      b = uniform_i64(b);
      if (a >= b) continue;  // the same for the whole workgroup
      const int64_t pa = a + (b - a) * w / kWavesPerBlock;
      const int64_t pb = a + (b - a) * (w + 1) / kWavesPerBlock;
      // this wave's sums of the tile, addressed by absolute feature index
      slice_wide<T, V, HAS_VAL, OFF32>(col, val, x, sums + w * kTile - tile * kTile, F, rs + pa, rs + pb,
                                       tile * kTile);
      __syncthreads();
      const int64_t width = F - tile * kTile < kTile ? F - tile * kTile : kTile;
      double* out = c.partial + (slice * chunk_stride + local) * F + tile * kTile;
      for (int64_t f = threadIdx.x; f < width; f += kBlock) {
        double total = sums[f].v;
#pragma unroll
        for (int k = 1; k < kWavesPerBlock; ++k) total += sums[k * kTile + f].v;
        store_out(out + f, total);
      }
      __syncthreads();
    }
  }
  for (int64_t local = mega + (in_phase / kSlices) * kWavesPerBlock + wave_in_block(); local < sliced;
       local += gs * kWavesPerBlock) {
    const int64_t row = uniform_i64(order[c.item_begin + local]);
    const int64_t rs = uniform_i64(crow[row]);
    const int64_t deg = uniform_i64(crow[row + 1]) - rs;
    int64_t a, b;
    slice_range<kSpmmSlices>(off, row, slice, deg, a, b);
    a = uniform_i64(a);
    b = uniform_i64(b);
    if (a >= b) continue;
    double* out = c.partial + (slice * chunk_stride + local) * F;
    if constexpr (V >= 8) {
      slice_wide<T, V, HAS_VAL, OFF32>(col, val, x, out, F, rs + a, rs + b, tile * kTile);
    } else {
      if (b - a >= kColsliceLongRow) slice_row<T, V, HAS_VAL, 16>(col, val, x, out, F, rs + a, rs + b);
      else slice_row<T, V, HAS_VAL, 8>(col, val, x, out, F, rs + a, rs + b);
    }
  }
}

// Orders one wave's LDS stores before its later loads (lanes read what other
// lanes of the same wave wrote).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A sliced fp32 row that found no partial rows in the buffer (the workspace
// was sized for fewer sliced rows than a chunk has): one wave computes each
// non-empty slice's fp64 sum with the slice work's own code (slice_wide, into
// LDS instead of a partial row) and adds them in slice order from 0.0 as the
// reduction does, then rounds once.  The same operations in the same order,
// so the same bits as when the row is sliced across waves.  Rows of the
// cooperative degree never get here (the host keeps chunks within the
// buffers on graphs that have them).  Called from colslice_overflow_kernel,
// a launch of its own, so that the step kernel keeps its register budget.  `sums`: this wave's 2·kTile LDS slots,
// the slice's sum and the running total (kept in LDS, not in registers, so
// that the slice work around it keeps its register budget).
template <typename T, int V, bool HAS_VAL, bool OFF32>
__device__ __forceinline__ void overflow_row_exact(const int64_t* __restrict__ crow, const int64_t* __restrict__ col,
                                                   const T* __restrict__ val, const T* __restrict__ x,
                                                   T* __restrict__ y, int64_t F, const int32_t* __restrict__ off,
                                                   int64_t row, int64_t tile, LdsSum* sums) {
  constexpr int64_t kTile = 16 * V / static_cast<int64_t>(sizeof(T));
  const int lane = lane_id();
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t deg = uniform_i64(crow[row + 1]) - rs;
  const int64_t f0 = tile * kTile;
  const int64_t width = F - f0 < kTile ? F - f0 : kTile;
  LdsSum* total = sums + kTile;
  for (int64_t f = lane; f < width; f += kWave) total[f].v = 0.0;
  for (int s = 0; s < kSpmmSlices; ++s) {
    int64_t a, b;
    slice_range<kSpmmSlices>(off, row, s, deg, a, b);
    a = uniform_i64(a);
    b = uniform_i64(b);
    if (a >= b) continue;
    // addressed by absolute feature index, as for a partial row
    slice_wide<T, V, HAS_VAL, OFF32>(col, val, x, sums - f0, F, rs + a, rs + b, f0);
    wave_lds_sync();
    for (int64_t f = lane; f < width; f += kWave) total[f].v = total[f].v + sums[f].v;
    wave_lds_sync();
  }
  for (int64_t f = lane; f < width; f += kWave) Elem<T>::put(y + row * F + f0 + f, total[f].v);
}

template <typename T, int V, bool HAS_VAL, bool OFF32>
__device__ __forceinline__ void colslice_short_block(int64_t hb, const int64_t* __restrict__ crow,
                                                     const int64_t* __restrict__ col, const T* __restrict__ val,
                                                     const T* __restrict__ x, T* __restrict__ y, int64_t F,
                                                     const int32_t* __restrict__ order,
                                                     const int32_t* __restrict__ counts, const SliceChunk& c,
                                                     GroupedRows grouped) {
  constexpr int64_t kTile = 16 * V / static_cast<int64_t>(sizeof(T));
  const int64_t tile_blocks = kSlices * c.short_groups;
  const int64_t tile = hb / tile_blocks;
  const int64_t k = hb - tile * tile_blocks;
  const int64_t waves = tile_blocks * kWavesPerBlock;  // short waves per tile
  const int64_t w = k * kWavesPerBlock + wave_in_block();
  // fp32 wide lanes: sliced rows past the partial buffers' capacity, from fs
  // to counts[0], are left to colslice_overflow_kernel; 16-bit elements sum
  // them whole here with the short rows (the same bits for their rule)
  int64_t fs = first_short(counts, c);
  const int64_t end = c.item_begin + c.items;
  if constexpr (sizeof(T) == 4 && V >= 8) {
    const int64_t h = counts[0];
    fs = h < fs ? fs : (h > end ? end : h);
  }
  int64_t split = end;  // grouped rows: [split, end)
  if constexpr (grouped_lanes<T, V>()) {
    if (grouped.start != nullptr) {
      split = *grouped.start;
      split = split < fs ? fs : (split > end ? end : split);
    }
  }
  // one wave per short row
  for (int64_t item = fs + w; item < split; item += waves) {
    const int64_t row = uniform_i64(order[item]);
    const int64_t rs = uniform_i64(crow[row]);
    const int64_t deg = uniform_i64(crow[row + 1]) - rs;
    if constexpr (V >= 8) {
      slice_wide<T, V, HAS_VAL, OFF32>(col, val, x, y + row * F, F, rs, rs + deg, tile * kTile);
    } else {
      slice_row<T, V, HAS_VAL, 8>(col, val, x, y + row * F, F, rs, rs + deg);
    }
  }
  // grouped rows: 64/V per wave
  if constexpr (grouped_lanes<T, V>()) {
    constexpr int64_t kRows = kWave / V;
    constexpr int kU = sizeof(T) == 2 ? AS_COLSLICE_GROUPED_U_16 : AS_COLSLICE_GROUPED_U_F32;
    for (int64_t item0 = split + w * kRows; item0 < end; item0 += waves * kRows) {
      short_rows_grouped<T, V, HAS_VAL, kU, OFF32>(crow, col, val, x, y, F, order, item0, end, tile * kTile);
    }
  }
}

// Reduction of one chunk, block rb of R: Y[row, f..f+VR) = sum over the
// non-empty slices, in slice order, in fp64, rounded once, for the sliced
// rows (short rows wrote Y themselves).
template <typename T, int VR>
__device__ __forceinline__ void colslice_reduce_block(int64_t rb, int64_t R, const int64_t* __restrict__ crow,
                                                      const int32_t* __restrict__ off,
                                                      const int32_t* __restrict__ order,
                                                      const int32_t* __restrict__ counts, T* __restrict__ y,
                                                      int64_t F, const SliceChunk& c, int64_t chunk_stride) {
  const int64_t FV = F / VR;
  // only the rows the slice blocks took: order[item_begin, first_short)
  const int64_t total = (first_short(counts, c) - c.item_begin) * FV;
  const int64_t stride = R * kBlock;
  for (int64_t t = rb * kBlock + threadIdx.x; t < total; t += stride) {
    const int64_t local = t / FV;
    const int64_t f = (t - local * FV) * VR;
    const int64_t row = order[c.item_begin + local];
    const int64_t deg = crow[row + 1] - crow[row];
    double acc[VR];
#pragma unroll
    for (int v = 0; v < VR; ++v) acc[v] = 0.0;
#pragma unroll
    for (int s = 0; s < kSpmmSlices; ++s) {
      int64_t a, b;
      slice_range<kSpmmSlices>(off, row, s, deg, a, b);
      if (a < b) {
        const double* p = c.partial + (s * chunk_stride + local) * F + f;
#pragma unroll
        for (int v = 0; v < VR; ++v) acc[v] += __builtin_nontemporal_load(p + v);
      }
    }
    store_elems<T, VR>(y + row * F + f, acc);
  }
}

// The rows a launch reduces: those of the previous chunk, which may belong to
// the previous row block (its CSR offset, plan view and Y rows).
struct ReduceRows {
  const int64_t* crow;
  const int32_t* off;
  const int32_t* order;
  const int32_t* counts;
  void* y;
};

// One launch of the pipeline: the slice and short work of chunk `m` and the
// reduction of the previous chunk `r`, whose partials a previous launch
// wrote.  A chunk's partial rows are `capacity` apart between slices.  Of the TG groups of 8 blocks, RG evenly spread ones reduce, so the
// HBM-streaming reduction runs beside the latency-bound gathers; the others,
// in order, are the MG slice groups and then the short groups.  Group g
// reduces iff floor((g+1)·RG/TG) > floor(g·RG/TG); floor(g·RG/TG) groups
// before it reduce, so every block keeps blockIdx % 8 as its XCD.
// 8 waves per SIMD (at most 64 VGPRs, no spills in any form): the 16-bit
// forms (8 fp64 sums per lane, the grouped short rows) otherwise take up to
// 88 VGPRs; at 8 waves cfg3 in bf16 takes 1.985 ms at F = 128 and 1.10 at
// F = 64, against 2.02 and 1.13 at 7.  The fp32 forms are unchanged.
#ifndef AS_COLSLICE_WAVES_PER_EU
#define AS_COLSLICE_WAVES_PER_EU 8
#endif
template <typename T, int V, bool HAS_VAL, int VR, bool OFF32>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(AS_COLSLICE_WAVES_PER_EU))) void colslice_step_kernel(const int64_t* __restrict__ crow,
                                                               const int64_t* __restrict__ col,
                                                               const T* __restrict__ val, const T* __restrict__ x,
                                                               T* __restrict__ y, int64_t F,
                                                               const int32_t* __restrict__ order,
                                                               const int32_t* __restrict__ counts,
                                                               const int32_t* __restrict__ off, SliceChunk m,
                                                               SliceChunk r, ReduceRows rr, int64_t TG,
                                                               int64_t RG, int64_t MG, GroupedRows grouped) {
  const int64_t g = blockIdx.x / kSlices;
  const int64_t within = blockIdx.x % kSlices;
  const int64_t before = g * RG / TG;
  if ((g + 1) * RG / TG > before) {
    colslice_reduce_block<T, VR>(before * kSlices + within, RG * kSlices, rr.crow, rr.off, rr.order, rr.counts,
                                 static_cast<T*>(rr.y), F, r, r.capacity);
    return;
  }
  const int64_t work = g - before;
  if (work < MG) {
    colslice_slice_block<T, V, HAS_VAL, OFF32>(work * kSlices + within, crow, col, val, x, F, order, counts, off, m,
                                               m.capacity, grouped.mega_end);
  } else {
    colslice_short_block<T, V, HAS_VAL, OFF32>((work - MG) * kSlices + within, crow, col, val, x, y, F, order,
                                               counts, m, grouped);
  }
}

// The sliced rows of chunks whose partial buffers held fewer rows than they
// have: positions [begin, min(counts[0], end)) of each chunk's order, one wave
// per (row, feature tile), fp32 with wide lanes.  A wave finds the range empty
// and exits when the workspace was sized for the chunk's sliced rows.
constexpr int kMaxOverflowChunks = 16;
struct OverflowChunk {
  const int64_t* crow;  // the row block's (rebased) row pointer
  const int32_t* order;
  const int32_t* counts;
  const int32_t* off;
  void* y;
  int64_t begin;  // first order position past the capacity
  int64_t end;    // end of the chunk's positions
};
struct OverflowChunks {
  OverflowChunk c[kMaxOverflowChunks];
  int count;
};

template <typename T, int V, bool HAS_VAL, bool OFF32>
__global__ __launch_bounds__(kBlock) void colslice_overflow_kernel(const int64_t* __restrict__ col,
                                                                   const T* __restrict__ val,
                                                                   const T* __restrict__ x, int64_t F,
                                                                   int64_t tiles, OverflowChunks oc) {
  constexpr int64_t kTile = 16 * V / static_cast<int64_t>(sizeof(T));
  __shared__ LdsSum sums[kWavesPerBlock * 2 * kTile];
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  LdsSum* mine = sums + wave_in_block() * 2 * kTile;
  for (int k = 0; k < oc.count; ++k) {
    const OverflowChunk c = oc.c[k];
    const int64_t h = uniform_i64(static_cast<int64_t>(c.counts[0]));
    const int64_t stop = h < c.end ? h : c.end;
    if (stop <= c.begin) continue;
    const int64_t items = (stop - c.begin) * tiles;
    for (int64_t i = wave; i < items; i += waves) {
      const int64_t pos = c.begin + i / tiles;
      const int64_t tile = i - (i / tiles) * tiles;
      const int64_t row = uniform_i64(static_cast<int64_t>(c.order[pos]));
      overflow_row_exact<T, V, HAS_VAL, OFF32>(c.crow, col, val, x, static_cast<T*>(c.y), F, c.off, row, tile,
                                               mine);
    }
  }
}

size_t colslice_row_bytes(int64_t f) {
  return static_cast<size_t>(kSpmmSlices) * static_cast<size_t>(f) * sizeof(double);
}

// Rows per chunk when the workspace allows: the pipeline overlaps the
// reduction of chunk k with the slice work of chunk k + 1, so all but the
// last chunk's reduction is hidden.  Chunks hold at least 32,768 rows: on
// smaller graphs each extra launch waits for its own longest (row, slice)
// and the chunks' rows are of one degree range each (the order is binned by
// degree), so one chunk is faster.  The reference's hub sweep (20,000 rows)
// takes 0.059 against 0.076 ms as one chunk, and an eighth of the rows of the
// skewed 115M-edge graph (29,000 rows against all 232,965 columns) 0.44
// against 0.47 ms at F = 128 fp32 and 0.27 against 0.31 ms in bf16; the
// whole skewed graph keeps its four chunks of 58,000 rows.
#ifndef AS_COLSLICE_CHUNKS
#define AS_COLSLICE_CHUNKS 4
#endif
constexpr int64_t kColsliceChunks = AS_COLSLICE_CHUNKS;
#ifndef AS_COLSLICE_MIN_CHUNK_ROWS
#define AS_COLSLICE_MIN_CHUNK_ROWS 32768
#endif
constexpr int64_t kColsliceMinChunkRows = AS_COLSLICE_MIN_CHUNK_ROWS;

int64_t preferred_chunk_rows(int64_t n) {
  int64_t c = (n + kColsliceChunks - 1) / kColsliceChunks;
  if (c < kColsliceMinChunkRows) c = n < kColsliceMinChunkRows ? n : kColsliceMinChunkRows;
  return c > 0 ? c : 1;
}

struct StepArgs {
  const int64_t* crow;
  const int64_t* col;
  const void* val;
  const void* x;
  void* y;
  int64_t f;
  const int32_t* order;
  const int32_t* counts;
  const int32_t* off;
  GroupedRows grouped;
};

struct GroupCounts {
  int64_t TG, RG, MG;
};

template <typename T, int V, bool HAS_VAL, int VR, bool OFF32>
void launch_one(dim3 grid, hipStream_t s, const StepArgs& a, const SliceChunk& m, const SliceChunk& r,
                const ReduceRows& rr, const GroupCounts& n) {
  hipLaunchKernelGGL((colslice_step_kernel<T, V, HAS_VAL, VR, OFF32>), grid, dim3(kBlock), 0, s, a.crow, a.col,
                     static_cast<const T*>(a.val), static_cast<const T*>(a.x), static_cast<T*>(a.y), a.f, a.order,
                     a.counts, a.off, m, r, rr, n.TG, n.RG, n.MG, a.grouped);
}

// OFF32 only matters for the ds_bpermute form of the wide lanes (V <= 16);
// V = 8 exists for 16-bit elements and V = 2 for fp32 only.
template <typename T, bool HAS_VAL, int VR>
void launch_step_v(int v, bool off32, dim3 grid, hipStream_t s, const StepArgs& a, const SliceChunk& m,
                   const SliceChunk& r, const ReduceRows& rr, const GroupCounts& n) {
  constexpr bool kHalf = sizeof(T) == 2;
  switch (v) {
    case 32:
      launch_one<T, 32, HAS_VAL, VR, false>(grid, s, a, m, r, rr, n);
      break;
    case 16:
      if (off32) launch_one<T, 16, HAS_VAL, VR, true>(grid, s, a, m, r, rr, n);
      else launch_one<T, 16, HAS_VAL, VR, false>(grid, s, a, m, r, rr, n);
      break;
    case 8:
      if constexpr (kHalf) {
        if (off32) launch_one<T, 8, HAS_VAL, VR, true>(grid, s, a, m, r, rr, n);
        else launch_one<T, 8, HAS_VAL, VR, false>(grid, s, a, m, r, rr, n);
      }
      break;
    case 2:
      if constexpr (!kHalf) launch_one<T, 2, HAS_VAL, VR, false>(grid, s, a, m, r, rr, n);
      break;
    default:
      launch_one<T, 1, HAS_VAL, VR, false>(grid, s, a, m, r, rr, n);
      break;
  }
}

// Launch of slice work `m` (items may be 0) beside the reduction of `r`
// (items may be 0) over the rows `rr` names.
template <typename T>
void launch_step(int v, bool off32, int vr, bool has_val, int64_t tiles, hipStream_t s, const StepArgs& a,
                 const SliceChunk& m, const SliceChunk& r, const ReduceRows& rr) {
  // groups of 8 blocks: slice groups per (tile, phase), short groups per tile
  const int64_t MG = m.items > 0 ? tiles * kPhases * m.slice_groups : 0;
  const int64_t SG = m.items > 0 ? tiles * m.short_groups : 0;
  int64_t RG = 0;
  if (r.items > 0) {
    // enough reduce blocks for one element per thread of the (expected)
    // sliced rows, at most a fifth of the groups when they run beside other
    // work; the blocks stride, so any count >= 1 covers them
    const int64_t rows = r.sliced >= 0 && r.sliced < r.items ? r.sliced : r.items;
    RG = (rows * (a.f / vr) + kSlices * kBlock - 1) / (kSlices * kBlock);
    const int64_t cap = MG + SG > 0 ? (MG + SG + 3) / 4 : kGridStrideBlocks / kSlices;
    if (RG > cap) RG = cap;
    if (RG < 1) RG = 1;
  }
  const GroupCounts n{MG + SG + RG, RG, MG};
  if (n.TG == 0) return;
  const dim3 grid(static_cast<unsigned>(n.TG * kSlices));
  if (has_val) {
    if (vr == 2) launch_step_v<T, true, 2>(v, off32, grid, s, a, m, r, rr, n);
    else launch_step_v<T, true, 1>(v, off32, grid, s, a, m, r, rr, n);
  } else {
    if (vr == 2) launch_step_v<T, false, 2>(v, off32, grid, s, a, m, r, rr, n);
    else launch_step_v<T, false, 1>(v, off32, grid, s, a, m, r, rr, n);
  }
}

enum Slicing { kSliceColumns = 0, kSliceEdges = 1 };

// 16-bit SpMM without slicing: one launch, no workspace.  Wave w of feature
// tile t sums rows w, w + W, ... whole (the short-row forms above, rounded
// once into Y).  For small graphs, where the slice points, the binning and the
// chunk launches of the sliced schedule cost more than the product.
template <typename T, int V, bool HAS_VAL, bool OFF32>
__global__ __launch_bounds__(kBlock) void rows16_kernel(const int64_t* __restrict__ crow,
                                                        const int64_t* __restrict__ col, const T* __restrict__ val,
                                                        const T* __restrict__ x, T* __restrict__ y, int64_t n,
                                                        int64_t F, int64_t tile_blocks) {
  constexpr int64_t kTile = 16 * V / static_cast<int64_t>(sizeof(T));
  const int64_t tile = blockIdx.x / tile_blocks;
  const int64_t waves = tile_blocks * kWavesPerBlock;
  const int64_t w = (blockIdx.x - tile * tile_blocks) * kWavesPerBlock + wave_in_block();
  for (int64_t row = w; row < n; row += waves) {
    const int64_t rs = uniform_i64(crow[row]);
    const int64_t re = uniform_i64(crow[row + 1]);
    if constexpr (V >= 8) {
      slice_wide<T, V, HAS_VAL, OFF32>(col, val, x, y + row * F, F, rs, re, tile * kTile);
    } else {
      slice_row<T, V, HAS_VAL, 8>(col, val, x, y + row * F, F, rs, re);
    }
  }
}

template <typename T, bool HAS_VAL>
int rows16_run(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y, int64_t n,
               int64_t f, hipStream_t s) {
  constexpr int64_t P = 8;  // 16-bit elements per 16-byte lane
  int v = 1;
  if (f % P == 0 && aligned(x, 16)) v = f <= 64 ? 8 : (f <= 128 ? 16 : 32);
  const int64_t tiles = v >= 8 ? (f + P * v - 1) / (P * v) : 1;
  const bool off32 = n <= (int64_t(1) << 24) && f * 2 < (int64_t(1) << 24) && n * f * 2 <= (int64_t(1) << 32);
  int64_t tile_blocks = (n + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t cap = kMaxBlocksPerLaunch / tiles;
  if (tile_blocks > cap) tile_blocks = cap;
  if (tile_blocks < 1) tile_blocks = 1;
  const dim3 grid(static_cast<unsigned>(tiles * tile_blocks));
  const T* vp = static_cast<const T*>(val);
  const T* xp = static_cast<const T*>(x);
  T* yp = static_cast<T*>(y);
#define AS_ROWS16(V_, O_) \
  hipLaunchKernelGGL((rows16_kernel<T, V_, HAS_VAL, O_>), grid, dim3(kBlock), 0, s, crow, col, vp, xp, yp, n, f, tile_blocks)
  switch (v) {
    case 32: if (off32) AS_ROWS16(32, true); else AS_ROWS16(32, false); break;
    case 16: if (off32) AS_ROWS16(16, true); else AS_ROWS16(16, false); break;
    case 8: if (off32) AS_ROWS16(8, true); else AS_ROWS16(8, false); break;
    default: AS_ROWS16(1, false); break;
  }
#undef AS_ROWS16
  return AS_OK;
}

// Degree limit of the grouped short rows (16-byte lanes): 4·G for the G lanes
// per edge that F takes; 0 when rows are not grouped.
inline int64_t grouped_degree(int64_t f, int64_t elem_bytes) {
  if (elem_bytes == 4) {
    if (f <= 0 || f % 4 != 0) return 0;
    const int64_t g = f <= 64 ? 16 : 32;
    return g <= AS_COLSLICE_GROUPED_F32 ? kGroupedMaxBlocks * g : 0;
  }
  if (elem_bytes != 2 || f <= 0 || f % 8 != 0) return 0;
  const int64_t g = f <= 64 ? 8 : (f <= 128 ? 16 : 32);
  return kGroupedMaxBlocks * g;
}

// Row blocks (fp32).  The rows of a graph of at least 2·kColsliceMinChunkRows
// rows run as B blocks of consecutive rows (B = min(kColsliceRowBlocks,
// n / kColsliceMinChunkRows)), one block after the other, each with its own
// degree-binned order and as one chunk where the workspace allows.  A launch
// then mixes long and short rows of its block, where chunks of one
// degree-binned order are each one degree range (the longest rows first, the
// shortest last).  Which rows a block holds changes no result: a row's sums
// depend only on its own edges and slice points.  On the skewed 115M-edge
// graph, one block against 4: F = 128 3.426 against 3.360 ms, F = 256 6.957
// against 6.820, F = 64 1.776 against 1.771 (2 blocks: 3.376, 6.819, 1.761;
// 3: 3.405, 6.784, 1.787; 6: 3.378, 6.858, 1.806).  16-bit elements keep one
// block: bf16 F = 128 1.908 against 1.916 ms with 4, F = 256 4.243 against
// 4.275.
#ifndef AS_COLSLICE_ROW_BLOCKS
#define AS_COLSLICE_ROW_BLOCKS 4
#endif
constexpr int64_t kColsliceRowBlocks = AS_COLSLICE_ROW_BLOCKS;

// 16-bit elements keep one block (of 4 chunks): on the skewed 115M-edge graph
// in bf16, 4 row blocks took 1.080 / 1.927 / 4.363 ms at F = 64 / 128 / 256,
// and 1.068 / 1.902 / 4.325 as one pipeline,
// against 1.061 / 1.909 / 4.314 with one block.
#ifndef AS_COLSLICE_ROW_BLOCKS_16
#define AS_COLSLICE_ROW_BLOCKS_16 1
#endif
static_assert(AS_COLSLICE_ROW_BLOCKS_16 >= 1 && AS_COLSLICE_ROW_BLOCKS_16 <= AS_COLSLICE_ROW_BLOCKS,
              "the plan holds the tables of at most AS_COLSLICE_ROW_BLOCKS blocks");
inline int64_t row_blocks(int64_t n, int64_t elem_bytes) {
  const int64_t most = elem_bytes == 4 ? kColsliceRowBlocks : AS_COLSLICE_ROW_BLOCKS_16;
  int64_t b = n / kColsliceMinChunkRows;
  if (b > most) b = most;
  return b < 1 ? 1 : b;
}
inline int64_t block_begin(int64_t n, int64_t blocks, int64_t b) { return n * b / blocks; }
inline int64_t block_rows_max(int64_t n, int64_t blocks) { return (n + blocks - 1) / blocks; }

// The column-sliced SpMM's plan over kSpmmSlices slices: the slice points of
// every row (off[n·(S-1)], as in colslice_common.h) and the order (order[n]),
// block b's rows at [r_b, r_{b+1}) of it, as row indices relative to r_b;
// then per block its bucket counts (256 bytes) and binning tables.  One size
// serves both block counts (fp32 and 16-bit plans).
using PlanView = SlicePlan;

inline size_t block_tables_bytes(int64_t n, int64_t blocks) {
  return static_cast<size_t>(blocks) * (256 + bin_workspace_bytes(block_rows_max(n, blocks)));
}

size_t colslice_fixed_bytes(int64_t n) {
  const size_t rows = static_cast<size_t>(n > 0 ? n : 1);
  const size_t one = block_tables_bytes(n, 1);
  const size_t many = block_tables_bytes(n, row_blocks(n, 4));
  return align_up(rows * kSpmmBounds * sizeof(int32_t), 256) + align_up(rows * sizeof(int32_t), 256) +
         (one > many ? one : many);
}

// Block b (of row_blocks(n, elem_bytes)) of the plan: off and order start at
// its first row.
inline PlanView block_view(void* base, int64_t n, int64_t elem_bytes, int64_t b) {
  char* p = static_cast<char*>(base);
  const size_t rows = static_cast<size_t>(n > 0 ? n : 1);
  const int64_t blocks = row_blocks(n, elem_bytes);
  const int64_t r0 = block_begin(n, blocks, b);
  PlanView v;
  v.off = reinterpret_cast<int32_t*>(p) + r0 * kSpmmBounds;
  p += align_up(rows * kSpmmBounds * sizeof(int32_t), 256);
  v.order = reinterpret_cast<int32_t*>(p) + r0;
  p += align_up(rows * sizeof(int32_t), 256);
  p += static_cast<size_t>(b) * (256 + bin_workspace_bytes(block_rows_max(n, blocks)));
  v.counts = reinterpret_cast<int32_t*>(p);
  v.bin_ws = p + 256;
  return v;
}

inline int64_t slicing_degree(Slicing slicing, int64_t f, int64_t elem_bytes) {
  return slicing == kSliceColumns ? column_slice_degree(f, elem_bytes) : kEdgeSliceMinDegree;
}

// rows of degree >= the slicing degree in 8 log2-degree buckets, longest
// first; then the short rows, for 16-bit elements also in 8 log2-degree
// buckets (a wave of grouped short rows then holds rows of similar degree)
inline int light_bucket_count(int64_t elem_bytes) {
  return elem_bytes == 2 || AS_COLSLICE_GROUPED_F32 != 0 ? kMaxHeavyBuckets : 1;
}

inline int64_t plan_tag_of(int64_t min_degree, int light_buckets, int64_t n, int64_t n_cols, int64_t elem_bytes) {
  return slice_plan_tag(min_degree, light_buckets, kPlanKindSpmm, row_blocks(n, elem_bytes), n_cols != n);
}

// n_cols: the column space (rows of X); n for a square graph.  The slice
// points of all rows in one launch, then the binning of each row block.
inline int build_plan(const int64_t* crow, const int64_t* col, int64_t n, int64_t n_cols, int64_t min_degree,
                      int light_buckets, Slicing slicing, int64_t elem_bytes, void* plan, hipStream_t s) {
  launch_slice_points<kSpmmSlices>(crow, col, n, min_degree, block_view(plan, n, elem_bytes, 0).off, s,
                                   slicing == kSliceEdges, n_cols);
  const int64_t blocks = row_blocks(n, elem_bytes);
  for (int64_t b = 0; b < blocks; ++b) {
    const int64_t r0 = block_begin(n, blocks, b);
    const PlanView v = block_view(plan, n, elem_bytes, b);
    const int st = launch_bin_rows(crow + r0, block_begin(n, blocks, b + 1) - r0, min_degree, kMaxHeavyBuckets,
                                   light_buckets, v.order, v.counts, v.bin_ws, s);
    if (st != AS_OK) return st;
  }
  return AS_OK;
}

// One row block (or a whole graph of one block): `plan` is its view of a
// plan that build_plan built for this graph, min_degree and light bucket
// count (the caller's duty); the workspace holds the partial buffers only.
// n rows of A and Y, n_cols rows of X; nnz: the whole graph's edges (an
// upper bound for a block's); chunk: preferred rows per chunk.
// How a call's chunks are launched: the lane form, the feature tiles and the
// partial rows of each of the two buffers (the same for every row block of a
// call, since they depend on F, the alignments and the workspace only).
struct StepShape {
  int v;
  bool off32;
  int vr;
  int64_t tiles;
  int64_t fits;
  bool operator==(const StepShape& o) const {
    return v == o.v && off32 == o.off32 && vr == o.vr && tiles == o.tiles && fits == o.fits;
  }
};

// A chunk of the pipeline with the pointers and plan view of its row block.
struct ChunkWork {
  StepArgs a;
  SliceChunk c;
};

// Appends the chunks of rows [0, n) of `crow` (one row block, or the graph)
// to `out`; their partial buffers are assigned when they are launched.
template <typename T>
int colslice_chunks(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y, int64_t n,
                    int64_t n_cols, int64_t nnz, int64_t f, int64_t min_degree, const PlanView& plan, void* partials,
                    size_t partial_bytes, int64_t sliced_rows, int64_t grouped_rows, int64_t chunk, StepShape& shape,
                    std::vector<ChunkWork>& out) {
  const size_t row_bytes = colslice_row_bytes(f);
  if (partials == nullptr || partial_bytes < 2 * row_bytes)
    return fail(AS_ERR_WORKSPACE, "column-sliced SpMM needs at least %zu bytes of partial buffers, got %zu",
                2 * row_bytes, partial_bytes);
  if (!aligned(partials, 256)) return fail(AS_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  constexpr int64_t E = static_cast<int64_t>(sizeof(T));
  constexpr int64_t P = 16 / E;  // elements per 16-byte lane

  // lanes: G lanes per edge with 16-byte loads when F is a multiple of P and
  // X is 16-byte aligned (fp32: G = 16 for F <= 64, else 32 in tiles of 128
  // features; 16-bit: G = 8 / 16 / 32 for F <= 64 / 128 / more, tiles of
  // 256); otherwise 8-byte (fp32, F > 64 even) or element-wide lanes with one
  // edge per gather
  int v = 1;
  if (f % P == 0 && aligned(x, 16)) {
    if (E == 4) v = f <= 64 ? 16 : 32;
    else v = f <= 64 ? 8 : (f <= 128 ? 16 : 32);
  } else if (E == 4 && f % 2 == 0 && f > 64 && aligned(x, 8)) {
    v = 2;
  }
  const int64_t tiles = v >= 8 ? (f + P * v - 1) / (P * v) : 1;
  // every X byte offset fits 32 bits, row index and row bytes fit 24 bits
  const bool off32 =
      n_cols <= (int64_t(1) << 24) && f * E < (int64_t(1) << 24) && n_cols * f * E <= (int64_t(1) << 32);
  const int vr = (f % 2 == 0 && aligned(y, static_cast<size_t>(2 * E))) ? 2 : 1;

  // two partial buffers of `capacity` rows each (chunk k writes buffer
  // k % 2).  16-bit, and fp32 with wide lanes on graphs without cooperative
  // rows: chunks of the preferred size whatever the workspace; sliced rows
  // past the capacity are summed by one wave each (16-bit: whole, fp32: slice
  // by slice in the sliced rows' order), with the same bits, so a workspace
  // sized for the sliced rows suffices.  Otherwise (fp32 narrow lanes, or
  // cooperative rows): chunks of at most `capacity` rows, so that every
  // sliced row of a chunk has partial rows.
  const int64_t fits = static_cast<int64_t>(partial_bytes / (2 * row_bytes));
  // fp32 with wide lanes on graphs without cooperative rows: a sliced row
  // past the capacity is summed by one wave with the same arithmetic
  // (overflow_row_exact), so chunks need not fit the buffers either and a
  // workspace sized for the sliced rows keeps one chunk per row block
  const bool has_mega = nnz <= kMegaMaxNnz && kMegaLevel >= 1 && kMegaLevel < kMaxHeavyBuckets;
  const bool overflow_exact = E != 4 || (v >= 8 && !has_mega);
  // a graph holds at most nnz / min_degree sliced rows; when they fit one
  // partial buffer the whole graph is one chunk (fewer launches, and short
  // rows run beside the hub rows' slices)
  const int64_t upper = min_degree > 0 && nnz / min_degree < n ? nnz / min_degree : n;
  if (upper <= chunk && (overflow_exact || upper <= fits)) chunk = n;
  if (!overflow_exact && (chunk < upper ? chunk : upper) > fits) chunk = fits;
  // blocks of a launch: 8 per group, at most tiles·(P·ceil(c/4) + ceil(c/32))
  // work groups for c rows, and reduce groups at most a quarter of those
  const int64_t max_rows = (kMaxBlocksPerLaunch * 4 / 5 / (kSlices * tiles) - 2) * 32 / (8 * kPhases + 1);
  if (chunk > max_rows) chunk = max_rows;
  if (chunk < 1) return fail(AS_ERR_UNSUPPORTED, "F = %lld is too wide for the column-sliced SpMM", (long long)f);
  // partial rows per buffer: a chunk's sliced rows are at most min(chunk, upper)
  int64_t capacity = fits < chunk ? fits : chunk;
  if (E == 4 && capacity > upper) capacity = upper > 0 ? upper : 1;

  // grouped short rows: the light buckets from level L on, L the first whose
  // rows all have degree below the limit (light bucket L holds degrees up to
  // (min_degree - 1) >> L, and bucket L - 1 none below min_degree >> L; both
  // are powers of two, so these are exactly the rows below the limit)
  const int light_buckets = light_bucket_count(E);
  GroupedRows grouped{nullptr};
  const int64_t limit = v >= 8 ? grouped_degree(f, E) : 0;
  if (limit > 0) {
    int level = 0;
    while (level < light_buckets && ((min_degree - 1) >> level) >= limit) ++level;
    if (level < light_buckets) grouped.start = bin_bucket_start(plan.bin_ws, n, kMaxHeavyBuckets + level);
  }
  // cooperative rows (wide lanes, graphs of at most kMegaMaxNnz edges):
  // heavy buckets 0 .. K-1-kMegaLevel
  if (v >= 8 && nnz <= kMegaMaxNnz && kMegaLevel >= 1 && kMegaLevel < kMaxHeavyBuckets)
    grouped.mega_end = bin_bucket_start(plan.bin_ws, n, kMaxHeavyBuckets - kMegaLevel);
  const int64_t rows_per_wave = grouped.start != nullptr ? kWave / v : 1;
  if (grouped.start == nullptr) grouped_rows = 0;

  shape = StepShape{v, off32, vr, tiles, fits};

  const StepArgs a{crow, col, val, x, y, f, plan.order, plan.counts, plan.off, grouped};
  const int64_t chunks = (n + chunk - 1) / chunk;
  for (int64_t k = 0; k < chunks; ++k) {
    SliceChunk current{k * chunk, 0, nullptr, 1, 1, -1, capacity};
    current.items = n - current.item_begin < chunk ? n - current.item_begin : chunk;
    // the sliced rows come first in the order, the grouped ones last
    const int64_t chunk_end = current.item_begin + current.items;
    const int64_t grouped_begin = grouped_rows < 0 || grouped_rows > n ? chunk_end : n - grouped_rows;
    const int64_t from = grouped_begin > current.item_begin ? grouped_begin : current.item_begin;
    int64_t sliced_here = sliced_rows < 0 ? -1 : (sliced_rows > current.item_begin ? sliced_rows - current.item_begin : 0);
    if (sliced_here > capacity) sliced_here = capacity;
    chunk_groups(current, sliced_here, chunk_end > from ? chunk_end - from : 0, rows_per_wave);
    out.push_back(ChunkWork{a, current});
  }
  return AS_OK;
}

// Launches chunks [begin, end) of `work` as a pipeline: launch k runs the slice
// and short work of chunk k beside the reduction of chunk k - 1, which may
// belong to the previous row block; chunk k writes partial buffer k % 2.
template <typename T>
void colslice_pipeline(const StepShape& sh, bool has_val, const std::vector<ChunkWork>& work, size_t begin,
                       size_t end, void* partials, size_t row_bytes, hipStream_t s) {
  if (end <= begin) return;
  double* buffers[2] = {static_cast<double*>(partials),
                        reinterpret_cast<double*>(static_cast<char*>(partials) + sh.fits * row_bytes)};
  const SliceChunk none{0, 0, nullptr, 1, 1, -1};
  for (size_t k = begin; k <= end; ++k) {
    SliceChunk m = k < end ? work[k].c : none;
    SliceChunk r = k > begin ? work[k - 1].c : none;
    if (k < end) m.partial = buffers[(k - begin) % 2];
    if (k > begin) r.partial = buffers[(k - begin - 1) % 2];
    const StepArgs& a = work[k < end ? k : end - 1].a;
    const StepArgs& ra = work[k > begin ? k - 1 : begin].a;
    const ReduceRows rr{ra.crow, ra.off, ra.order, ra.counts, ra.y};
#if AS_COLSLICE_OVERLAP
    launch_step<T>(sh.v, sh.off32, sh.vr, has_val, sh.tiles, s, a, m, r, rr);
#else
    if (k < end) {
      const ReduceRows own{a.crow, a.off, a.order, a.counts, a.y};
      launch_step<T>(sh.v, sh.off32, sh.vr, has_val, sh.tiles, s, a, m, none, own);
      launch_step<T>(sh.v, sh.off32, sh.vr, has_val, sh.tiles, s, a, none, m, own);
    }
#endif
  }
}

// Launches colslice_overflow_kernel for the chunks of `work` whose partial
// buffers hold fewer rows than the chunk (fp32 wide lanes only; elsewhere
// the chunks fit their buffers or the step kernel sums the rest).  `upper`:
// at most this many sliced rows in a chunk (nnz / slicing degree), sizing the grid.
template <typename T>
void colslice_overflow(const StepShape& sh, bool has_val, const std::vector<ChunkWork>& work, int64_t upper,
                       hipStream_t s) {
  if constexpr (sizeof(T) != 4) {
    return;
  } else {
    if (sh.v < 8 || work.empty()) return;
    const StepArgs& a0 = work[0].a;
    OverflowChunks oc{};
    int64_t potential = 0;
    auto flush = [&]() {
      if (oc.count == 0) return;
      int64_t blocks = (potential * sh.tiles + 4 * kWavesPerBlock - 1) / (4 * kWavesPerBlock);
      blocks = blocks < kSlices ? kSlices : (blocks > 2048 ? 2048 : blocks);
      const dim3 grid(static_cast<unsigned>(blocks)), block(kBlock);
      const float* v = static_cast<const float*>(a0.val);
      const float* x = static_cast<const float*>(a0.x);
#define AS_OVERFLOW(V_, HV_, O_)                                                                                    \
  hipLaunchKernelGGL((colslice_overflow_kernel<float, V_, HV_, O_>), grid, block, 0, s, a0.col, v, x, a0.f, sh.tiles, \
                     oc)
      if (sh.v == 32) {
        if (has_val) { if (sh.off32) AS_OVERFLOW(32, true, true); else AS_OVERFLOW(32, true, false); }
        else { if (sh.off32) AS_OVERFLOW(32, false, true); else AS_OVERFLOW(32, false, false); }
      } else {
        if (has_val) { if (sh.off32) AS_OVERFLOW(16, true, true); else AS_OVERFLOW(16, true, false); }
        else { if (sh.off32) AS_OVERFLOW(16, false, true); else AS_OVERFLOW(16, false, false); }
      }
#undef AS_OVERFLOW
      oc.count = 0;
      potential = 0;
    };
    for (const ChunkWork& w : work) {
      if (w.c.capacity >= w.c.items) continue;
      const int64_t most = (upper < w.c.items ? upper : w.c.items) - w.c.capacity;
      if (most <= 0) continue;
      oc.c[oc.count++] = OverflowChunk{w.a.crow, w.a.order, w.a.counts, w.a.off, w.a.y,
                                       w.c.item_begin + w.c.capacity, w.c.item_begin + w.c.items};
      potential += most;
      if (oc.count == kMaxOverflowChunks) flush();
    }
    flush();
  }
}

template <typename T>
int colslice_execute(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y, int64_t n,
                     int64_t n_cols, int64_t nnz, int64_t f, int64_t min_degree, const PlanView& plan, void* partials,
                     size_t partial_bytes, int64_t sliced_rows, int64_t grouped_rows, int64_t chunk, hipStream_t s) {
  std::vector<ChunkWork> work;
  StepShape sh{};
  const int st = colslice_chunks<T>(crow, col, val, x, y, n, n_cols, nnz, f, min_degree, plan, partials,
                                    partial_bytes, sliced_rows, grouped_rows, chunk, sh, work);
  if (st != AS_OK) return st;
  colslice_pipeline<T>(sh, val != nullptr, work, 0, work.size(), partials, colslice_row_bytes(f), s);
  colslice_overflow<T>(sh, val != nullptr, work, min_degree > 0 ? nnz / min_degree : n, s);
  return AS_OK;
}

// The whole call over the row blocks of `plan`; a block is one chunk where
// the workspace allows.  The launch-sizing hints of a block are the graph's
// scaled to its rows.  For F up to AS_COLSLICE_FUSE_BLOCKS_MAX_F the blocks'
// chunks form one pipeline (the reduction of a block's last chunk beside the
// next block's slice work; 4 blocks of one chunk: 5 launches instead of 8);
// wider rows run each block as a pipeline of its own, whose last chunk's
// reduction is a launch of its own.  Same bits either way.  On the skewed
// 115M-edge graph one pipeline measured 1.741 / 3.281 / 6.765 ms at F = 64 /
// 128 / 256 against 1.750 / 3.271 / 6.745 with one per block.
#ifndef AS_COLSLICE_FUSE_BLOCKS_MAX_F
#define AS_COLSLICE_FUSE_BLOCKS_MAX_F 64
#endif
template <typename T>
int colslice_execute_blocks(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y,
                            int64_t n, int64_t n_cols, int64_t nnz, int64_t f, int64_t min_degree, void* plan,
                            void* partials, size_t partial_bytes, int64_t sliced_rows, int64_t grouped_rows,
                            hipStream_t s) {
  constexpr int64_t E = static_cast<int64_t>(sizeof(T));
  const int64_t blocks = row_blocks(n, E);
  if (blocks == 1)
    return colslice_execute<T>(crow, col, val, x, y, n, n_cols, nnz, f, min_degree, block_view(plan, n, E, 0),
                               partials, partial_bytes, sliced_rows, grouped_rows, preferred_chunk_rows(n), s);
  std::vector<ChunkWork> work;
  std::vector<size_t> ends;
  std::vector<StepShape> shapes;
  bool same_shape = true;
  for (int64_t b = 0; b < blocks; ++b) {
    const int64_t r0 = block_begin(n, blocks, b);
    const int64_t rows = block_begin(n, blocks, b + 1) - r0;
    const int64_t sliced = sliced_rows < 0 ? -1 : (sliced_rows * rows + n - 1) / n;
    const int64_t grouped = grouped_rows < 0 ? -1 : (grouped_rows * rows + n - 1) / n;
    StepShape sh{};
    const int st = colslice_chunks<T>(crow + r0, col, val, x, static_cast<T*>(y) + r0 * f, rows, n_cols, nnz, f,
                                      min_degree, block_view(plan, n, E, b), partials, partial_bytes, sliced,
                                      grouped, rows, sh, work);
    if (st != AS_OK) return st;
    same_shape = same_shape && (b == 0 || sh == shapes[0]);
    shapes.push_back(sh);
    ends.push_back(work.size());
  }
  const size_t row_bytes = colslice_row_bytes(f);
  if (f <= AS_COLSLICE_FUSE_BLOCKS_MAX_F && same_shape) {
    colslice_pipeline<T>(shapes[0], val != nullptr, work, 0, work.size(), partials, row_bytes, s);
  } else {
    for (size_t b = 0, begin = 0; b < ends.size(); begin = ends[b++])
      colslice_pipeline<T>(shapes[b], val != nullptr, work, begin, ends[b], partials, row_bytes, s);
  }
  // every block shares the lane shape (F, alignments), so the overflow of all
  // chunks is one launch
  colslice_overflow<T>(shapes[0], val != nullptr, work, min_degree > 0 ? nnz / min_degree : n, s);
  return AS_OK;
}

// One call with its plan built in the workspace's first colslice_fixed_bytes(n).
template <typename T>
int colslice_run(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y, int64_t n,
                 int64_t nnz, int64_t f, Slicing slicing, void* workspace, size_t workspace_bytes,
                 int64_t sliced_rows, int64_t grouped_rows, void* stream) {
  int st = validate_spmm(crow, col, x, y, n, nnz, f);
  if (st != AS_OK) return st;
  if (n == 0 || f == 0) return AS_OK;
  const size_t fixed = colslice_fixed_bytes(n);
  const size_t row_bytes = colslice_row_bytes(f);
  if (workspace == nullptr || workspace_bytes < fixed + 2 * row_bytes)
    return fail(AS_ERR_WORKSPACE, "column-sliced SpMM needs at least %zu workspace bytes, got %zu",
                fixed + 2 * row_bytes, workspace_bytes);
  if (!aligned(workspace, 256)) return fail(AS_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  constexpr int64_t E = static_cast<int64_t>(sizeof(T));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t min_degree = slicing_degree(slicing, f, E);
  st = build_plan(crow, col, n, n, min_degree, light_bucket_count(E), slicing, E, workspace, s);
  if (st != AS_OK) return st;
  return colslice_execute_blocks<T>(crow, col, val, x, y, n, n, nnz, f, min_degree, workspace,
                                    static_cast<char*>(workspace) + fixed, workspace_bytes - fixed, sliced_rows,
                                    grouped_rows, s);
}

inline int elem_bytes_of(int dtype) {
  return dtype == AS_DTYPE_F32 ? 4 : (dtype == AS_DTYPE_BF16 || dtype == AS_DTYPE_F16 ? 2 : 0);
}

}  // namespace

}  // namespace as

extern "C" {

size_t as_spmm_colslice_workspace_bytes(int64_t n, int64_t f) {
  if (n < 0) n = 0;
  if (f < 1) f = 1;
  return as::colslice_fixed_bytes(n) + 2 * static_cast<size_t>(as::preferred_chunk_rows(n)) * as::colslice_row_bytes(f);
}

int64_t as_spmm_colslice_min_degree(int column_slices, int64_t f, int dtype) {
  if (!column_slices) return as::kEdgeSliceMinDegree;
  return as::column_slice_degree(f, dtype == AS_DTYPE_F32 ? 4 : 2);
}

size_t as_spmm_colslice_plan_bytes(int64_t n) { return as::colslice_fixed_bytes(n); }

int as_spmm_colslice_plan_rect(const int64_t* crow, const int64_t* col, int64_t n, int64_t n_cols, int64_t nnz,
                               int64_t f, int dtype, int column_slices, void* plan, size_t plan_bytes,
                               int64_t* plan_tag, void* stream) {
  as::clear_error();
  if (n_cols < 0 || n_cols > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "n_cols exceeds kernel index range");
  const int64_t e = as::elem_bytes_of(dtype);
  if (e == 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_F32, AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (e == 4 && !column_slices)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "float32 features take column slices only (column_slices != 0)");
  if (plan_tag == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "plan_tag must not be NULL");
  if (n < 0 || nnz < 0 || f < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "n, nnz and f must be non-negative");
  if (n > 0 && (crow == nullptr || (nnz > 0 && col == nullptr)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "crow and col must not be NULL");
  if (plan == nullptr || plan_bytes < as::colslice_fixed_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "a column-sliced plan needs %zu bytes, got %zu", as::colslice_fixed_bytes(n),
                    plan_bytes);
  if (!as::aligned(plan, 256)) return as::fail(AS_ERR_WORKSPACE, "the plan must be 256-byte aligned");
  const as::Slicing slicing = column_slices ? as::kSliceColumns : as::kSliceEdges;
  const int64_t min_degree = as::slicing_degree(slicing, f, e);
  const int light = as::light_bucket_count(e);
  *plan_tag = as::plan_tag_of(min_degree, light, n, n_cols, e);
  if (n == 0) return AS_OK;
  const int st = as::build_plan(crow, col, n, n_cols, min_degree, light, slicing, e, plan,
                                static_cast<hipStream_t>(stream));
  if (st != AS_OK) return st;
  return as::check_launch("spmm_colslice_plan");
}

int as_spmm_colslice_plan(const int64_t* crow, const int64_t* col, int64_t n, int64_t nnz, int64_t f, int dtype,
                          int column_slices, void* plan, size_t plan_bytes, int64_t* plan_tag, void* stream) {
  return as_spmm_colslice_plan_rect(crow, col, n, n < 0 ? 0 : n, nnz, f, dtype, column_slices, plan, plan_bytes,
                                    plan_tag, stream);
}

int64_t as_spmm_colslice_row_blocks(int64_t n, int dtype, int64_t* begins, int64_t capacity) {
  const int64_t e = as::elem_bytes_of(dtype);
  if (e == 0 || n < 0) return 0;
  const int64_t blocks = as::row_blocks(n, e);
  for (int64_t b = 0; b <= blocks && b < capacity && begins != nullptr; ++b) begins[b] = as::block_begin(n, blocks, b);
  return blocks;
}

size_t as_spmm_colslice_planned_workspace_bytes(int64_t n, int64_t nnz, int64_t f, int dtype,
                                                int64_t sliced_rows) {
  if (n < 0) n = 0;
  if (f < 1) f = 1;
  // a chunk's rows: the preferred chunk, or a whole row block of the plan
  // (the planned call runs each block as one chunk when the buffers allow)
  const int64_t e = as::elem_bytes_of(dtype);
  int64_t rows = as::preferred_chunk_rows(n);
  if (e != 0) {
    const int64_t block = as::block_rows_max(n, as::row_blocks(n, e));
    if (block > rows) rows = block;
  }
  // Buffers of fewer rows than a chunk keep one chunk per row block only where
  // the sliced rows past them are summed with the same bits (16-bit; fp32
  // with 16-byte lanes, F % 4 == 0 and X aligned, on graphs without
  // cooperative hub rows, i.e. of more than 2^24 edges).  Elsewhere the
  // chunks are cut to the buffers, so buffers sized for the sliced rows
  // would cut a graph of few sliced rows into as many launches as it has
  // rows: there they hold a chunk's rows.
  const bool capped = sliced_rows >= 0 && (e != 4 || (f % 4 == 0 && nnz > as::kMegaMaxNnz));
  if (capped && sliced_rows < rows) rows = sliced_rows > 0 ? sliced_rows : 1;
  return 2 * static_cast<size_t>(rows) * as::colslice_row_bytes(f);
}

int as_spmm_csr_colslice_planned_rect(const int64_t* crow, const int64_t* col, const void* val, const void* x,
                                      void* y, int64_t n, int64_t n_cols, int64_t nnz, int64_t f, int dtype,
                                      int column_slices, const void* plan, size_t plan_bytes, int64_t plan_tag,
                                      void* workspace, size_t workspace_bytes, int64_t sliced_rows,
                                      int64_t grouped_rows, void* stream) {
  as::clear_error();
  if (n_cols < 0 || n_cols > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "n_cols exceeds kernel index range");
  const int64_t e = as::elem_bytes_of(dtype);
  if (e == 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_F32, AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (e == 4 && !column_slices)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "float32 features take column slices only (column_slices != 0)");
  if (!as::aligned(x, e) || !as::aligned(y, e) || (val != nullptr && !as::aligned(val, e)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "x, y and val must be aligned to their element size");
  int st = as::validate_spmm(crow, col, x, y, n, nnz, f);
  if (st != AS_OK) return st;
  if (n == 0 || f == 0) return AS_OK;
  const as::Slicing slicing = column_slices ? as::kSliceColumns : as::kSliceEdges;
  const int64_t min_degree = as::slicing_degree(slicing, f, e);
  const int64_t want = as::plan_tag_of(min_degree, as::light_bucket_count(e), n, n_cols, e);
  if (plan_tag != want)
    return as::fail(AS_ERR_INVALID_ARGUMENT,
                    "the plan was built for other settings (plan tag %lld, this graph, F, dtype and slicing need "
                    "%lld)", (long long)plan_tag, (long long)want);
  if (plan == nullptr || plan_bytes < as::colslice_fixed_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "a column-sliced plan needs %zu bytes, got %zu", as::colslice_fixed_bytes(n),
                    plan_bytes);
  if (!as::aligned(plan, 256)) return as::fail(AS_ERR_WORKSPACE, "the plan must be 256-byte aligned");
  void* view = const_cast<void*>(plan);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == AS_DTYPE_F32)
    st = as::colslice_execute_blocks<float>(crow, col, val, x, y, n, n_cols, nnz, f, min_degree, view, workspace,
                                            workspace_bytes, sliced_rows, grouped_rows, s);
  else if (dtype == AS_DTYPE_BF16)
    st = as::colslice_execute_blocks<as::Bf16>(crow, col, val, x, y, n, n_cols, nnz, f, min_degree, view, workspace,
                                               workspace_bytes, sliced_rows, grouped_rows, s);
  else
    st = as::colslice_execute_blocks<as::Fp16>(crow, col, val, x, y, n, n_cols, nnz, f, min_degree, view, workspace,
                                               workspace_bytes, sliced_rows, grouped_rows, s);
  if (st != AS_OK) return st;
  return as::check_launch("spmm_csr_colslice_planned");
}

int as_spmm_csr_colslice_planned(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y,
                                 int64_t n, int64_t nnz, int64_t f, int dtype, int column_slices, const void* plan,
                                 size_t plan_bytes, int64_t plan_tag, void* workspace, size_t workspace_bytes,
                                 int64_t sliced_rows, int64_t grouped_rows, void* stream) {
  return as_spmm_csr_colslice_planned_rect(crow, col, val, x, y, n, n < 0 ? 0 : n, nnz, f, dtype, column_slices,
                                           plan, plan_bytes, plan_tag, workspace, workspace_bytes, sliced_rows,
                                           grouped_rows, stream);
}

int as_spmm_csr_colslice_f32(const int64_t* crow, const int64_t* col, const float* val, const float* x, float* y,
                             int64_t n, int64_t nnz, int64_t f, void* workspace, size_t workspace_bytes,
                             int64_t sliced_rows, void* stream) {
  as::clear_error();
  const int st = as::colslice_run<float>(crow, col, val, x, y, n, nnz, f, as::kSliceColumns, workspace,
                                         workspace_bytes, sliced_rows, 0, stream);
  if (st != AS_OK) return st;
  return as::check_launch("spmm_csr_colslice");
}

int64_t as_spmm_rounded_16_group_degree(int64_t f) { return as::grouped_degree(f, 2); }

int64_t as_spmm_colslice_group_degree(int64_t f, int dtype) {
  const int64_t e = as::elem_bytes_of(dtype);
  return e == 0 ? 0 : as::grouped_degree(f, e);
}

int as_spmm_csr_rows_16(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y, int64_t n,
                        int64_t nnz, int64_t f, int dtype, void* stream) {
  as::clear_error();
  if (dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (!as::aligned(x, 2) || !as::aligned(y, 2) || (val != nullptr && !as::aligned(val, 2)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "x, y and val must be 2-byte aligned");
  int st = as::validate_spmm(crow, col, x, y, n, nnz, f);
  if (st != AS_OK) return st;
  if (n == 0 || f == 0) return AS_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == AS_DTYPE_BF16)
    st = val ? as::rows16_run<as::Bf16, true>(crow, col, val, x, y, n, f, s)
             : as::rows16_run<as::Bf16, false>(crow, col, val, x, y, n, f, s);
  else
    st = val ? as::rows16_run<as::Fp16, true>(crow, col, val, x, y, n, f, s)
             : as::rows16_run<as::Fp16, false>(crow, col, val, x, y, n, f, s);
  if (st != AS_OK) return st;
  return as::check_launch("spmm_csr_rows_16");
}

size_t as_spmm_rounded_16_workspace_bytes(int64_t n, int64_t f, int64_t sliced_rows) {
  if (n < 0) n = 0;
  if (f < 1) f = 1;
  int64_t rows = as::preferred_chunk_rows(n);
  if (sliced_rows >= 0 && sliced_rows < rows) rows = sliced_rows > 0 ? sliced_rows : 1;
  return as::colslice_fixed_bytes(n) + 2 * static_cast<size_t>(rows) * as::colslice_row_bytes(f);
}

int as_spmm_csr_rounded_16(const int64_t* crow, const int64_t* col, const void* val, const void* x, void* y,
                           int64_t n, int64_t nnz, int64_t f, int dtype, int column_slices, void* workspace,
                           size_t workspace_bytes, int64_t sliced_rows, int64_t grouped_rows, void* stream) {
  as::clear_error();
  if (dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (!as::aligned(x, 2) || !as::aligned(y, 2) || (val != nullptr && !as::aligned(val, 2)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "x, y and val must be 2-byte aligned");
  const as::Slicing slicing = column_slices ? as::kSliceColumns : as::kSliceEdges;
  const int st = dtype == AS_DTYPE_BF16
                     ? as::colslice_run<as::Bf16>(crow, col, val, x, y, n, nnz, f, slicing, workspace,
                                                  workspace_bytes, sliced_rows, grouped_rows, stream)
                     : as::colslice_run<as::Fp16>(crow, col, val, x, y, n, nnz, f, slicing, workspace,
                                                  workspace_bytes, sliced_rows, grouped_rows, stream);
  if (st != AS_OK) return st;
  return as::check_launch("spmm_csr_rounded_16");
}

}  // extern "C"
