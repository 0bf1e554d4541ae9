// CSR SpMM Y = A·X for fp32 features on gfx950.
//
// Reference behaviour: csrc/spmm_csr_vec4.cu:23-176 (whole graph),
// csrc/spmm_rows.cu:11-157 (light rows), csrc/spmm_hub.cu:13-182 (hub rows),
// csrc/launcher_spmm.cu:22-72 (split launcher).
//
// Exactness.  Except in the SPLIT64 hub mode, every output element Y[r, f]
// is one fp32 accumulator updated in CSR edge order with fmaf (acc + x when
// unweighted, which is the same value).  That is the order of the
// sequential CPU CSR product, so the result is bit-identical to it whatever
// the row-to-wave mapping, feature slicing or vector width.
//
// Row layouts:
//   wave-row  one wave64 owns a row (or a feature slice of it); lane owns V in
//             {1,2,4} consecutive features; a pass covers 64·V features.
//             Column indices and weights of 64 edges are loaded with one
//             coalesced load, one chunk ahead, and broadcast with v_readlane,
//             so the X-row address is wave-uniform.  U gathers in flight.
//   sub-wave  float4 lanes, LPR in {16,32} lanes per row, 64/LPR rows per
//             wave, for short rows where a whole wave per row would idle.
//
// Split schedule (one launch after the degree binning): workgroups of W
// waves; the first H workgroups take the heavy rows, longest degree bucket
// first, and split each heavy row's FEATURES across their W waves (no
// reassociation: W times the memory parallelism on long rows without
// changing any sum); the remaining workgroups take the light rows, one (or
// 64/LPR) per wave.  Workgroups are dispatched in index order, so hub rows
// start first and light rows fill the machine behind them.
//
// SPLIT64 hub mode: the W waves split the hub row's EDGES into contiguous
// slices accumulated in fp64; the slices are added in LDS in wave order and
// rounded to fp32 once (deterministic; reassociated, within about one fp32
// rounding of the exact sum).
#include "as_device.h"
#include "as_internal.h"

namespace as {

namespace {

enum Layout : int { kWaveV1 = 0, kWaveV2 = 1, kWaveV4 = 2, kSub16 = 3, kSub32 = 4 };

template <int L>
struct LayoutInfo;
template <>
struct LayoutInfo<kWaveV1> { static constexpr int V = 1, LPR = 64; };
template <>
struct LayoutInfo<kWaveV2> { static constexpr int V = 2, LPR = 64; };
template <>
struct LayoutInfo<kWaveV4> { static constexpr int V = 4, LPR = 64; };
template <>
struct LayoutInfo<kSub16> { static constexpr int V = 4, LPR = 16; };
template <>
struct LayoutInfo<kSub32> { static constexpr int V = 4, LPR = 32; };

// Gathers in flight per wave: hub rows, ordinary rows, and the degree from
// which an ordinary row uses the hub depth.
#ifndef AS_HUB_UNROLL
#define AS_HUB_UNROLL 16
#endif
#ifndef AS_ROW_UNROLL
#define AS_ROW_UNROLL 8
#endif
#ifndef AS_NT_STREAMS
#define AS_NT_STREAMS 0
#endif
constexpr int kHubUnroll = AS_HUB_UNROLL;
constexpr int kRowUnroll = AS_ROW_UNROLL;
constexpr int kLongRow = 1024;

// Loads of data read exactly once (column indices, weights); with
// AS_NT_STREAMS they carry the non-temporal hint so they do not displace X
// rows from the caches.
template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
  if constexpr (AS_NT_STREAMS != 0) return __builtin_nontemporal_load(p);
  else return *p;
}

// One wave computes Y[row, fbeg:fend) in edge order.  V | (fend - fbeg) and
// V | F are guaranteed by the host; row, rs, re, fbeg, fend are wave-uniform.
// Lanes past fend load a valid in-row address and store nothing, so the
// gathers carry no per-lane branches; full batches of U edges run without
// bound checks and the remainder one edge at a time.
template <int V, bool HAS_VAL, int U>
__device__ __forceinline__ void wave_row_exact(const int64_t* __restrict__ col, const float* __restrict__ val,
                                               const float* __restrict__ x, float* __restrict__ y, int64_t F,
                                               int64_t row, int64_t rs, int64_t re, int64_t fbeg, int64_t fend) {
  const int lane = lane_id();
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  for (int64_t f0 = fbeg; f0 < fend; f0 += kWave * V) {
    const int64_t fl = f0 + static_cast<int64_t>(lane) * V;
    const bool active = fl < fend;
    // byte offset of this lane's features inside an X row (< 2^32 since F < 2^29)
    const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : fbeg) * 4);
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;

    int next_col = 0;
    float next_w = 1.f;
    if (rs < re && lane < re - rs) {
      next_col = static_cast<int>(stream_load(col + rs + lane));
      if constexpr (HAS_VAL) next_w = stream_load(val + rs + lane);
    }
    for (int64_t base = rs; base < re; base += kWave) {
      const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
      const int my_col = next_col;
      const float my_w = next_w;
      const int64_t nb = base + kWave;
      if (nb < re && lane < re - nb) {
        next_col = static_cast<int>(stream_load(col + nb + lane));
        if constexpr (HAS_VAL) next_w = stream_load(val + nb + lane);
      }
      int j = 0;
      for (; j + U <= cnt; j += U) {
        FVec<V> xv[U];
        float w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = bcast_i32(my_col, j + u);
          w[u] = HAS_VAL ? bcast_f32(my_w, j + u) : 1.f;
          xv[u] = load_vec_off<V>(x + row_offset(c, F), lane_bytes);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (HAS_VAL) {
              acc[v] = __builtin_fmaf(w[u], xv[u].v[v], acc[v]);
            } else {
              acc[v] = acc[v] + xv[u].v[v];
            }
          }
        }
      }
      for (; j < cnt; ++j) {
        const int c = bcast_i32(my_col, j);
        const FVec<V> xv = load_vec_off<V>(x + row_offset(c, F), lane_bytes);
        const float w = HAS_VAL ? bcast_f32(my_w, j) : 1.f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (HAS_VAL) {
            acc[v] = __builtin_fmaf(w, xv.v[v], acc[v]);
          } else {
            acc[v] = acc[v] + xv.v[v];
          }
        }
      }
    }
    if (active) {
      FVec<V> out;
#pragma unroll
      for (int v = 0; v < V; ++v) out.v[v] = acc[v];
      store_vec<V>(y + row * F + fl, out);
    }
  }
}

// Sub-wave rows: this lane group computes the whole of `row` (valid) with
// float4 lanes; rows of one wave may differ in length (the loop runs to the
// longest, shorter groups idle).
template <int LPR, bool HAS_VAL, int U>
__device__ __forceinline__ void subwave_row_exact(const int64_t* __restrict__ col, const float* __restrict__ val,
                                                  const float* __restrict__ x, float* __restrict__ y, int64_t F,
                                                  int64_t row, bool valid, int64_t rs, int64_t re) {
  constexpr int P = LPR * 4;
  const int sl = lane_id() % LPR;
  for (int64_t f0 = 0; f0 < F; f0 += P) {
    const int64_t fl = f0 + static_cast<int64_t>(sl) * 4;
    const bool active = valid && fl < F;
    const float* xf = x + fl;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t e = rs; e < re; e += U) {
      FVec<4> xv[U];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int v = 0; v < 4; ++v) xv[u].v[v] = 0.f;
        w[u] = 1.f;
        if (e + u < re) {
          const int64_t c = static_cast<int>(col[e + u]);
          if constexpr (HAS_VAL) w[u] = val[e + u];
          if (active) xv[u] = load_vec<4>(xf + c * F);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (e + u < re) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            if constexpr (HAS_VAL) {
              acc[v] = __builtin_fmaf(w[u], xv[u].v[v], acc[v]);
            } else {
              acc[v] = acc[v] + xv[u].v[v];
            }
          }
        }
      }
    }
    if (active) {
      FVec<4> out;
#pragma unroll
      for (int v = 0; v < 4; ++v) out.v[v] = acc[v];
      store_vec<4>(y + row * F + fl, out);
    }
  }
}

// Light work of one wave: entry `wave_index` (times the rows per wave) of
// `rows` (nullptr = identity); `limit` is the number of valid entries.
template <int LAYOUT, bool HAS_VAL>
__device__ __forceinline__ void light_wave(const int64_t* __restrict__ crow, const int64_t* __restrict__ col,
                                           const float* __restrict__ val, const float* __restrict__ x,
                                           float* __restrict__ y, int64_t F, const int32_t* __restrict__ rows,
                                           int64_t wave_index, int64_t limit) {
  using LI = LayoutInfo<LAYOUT>;
  if constexpr (LI::LPR == kWave) {
    if (wave_index >= limit) return;
    const int64_t row = uniform_i64(rows ? static_cast<int64_t>(rows[wave_index]) : wave_index);
    const int64_t rs = uniform_i64(crow[row]);
    const int64_t re = uniform_i64(crow[row + 1]);
    if (re - rs >= kLongRow) {
      wave_row_exact<LI::V, HAS_VAL, kHubUnroll>(col, val, x, y, F, row, rs, re, 0, F);
    } else {
      wave_row_exact<LI::V, HAS_VAL, kRowUnroll>(col, val, x, y, F, row, rs, re, 0, F);
    }
  } else {
    constexpr int RPW = kWave / LI::LPR;
    const int64_t idx = wave_index * RPW + lane_id() / LI::LPR;
    const bool valid = idx < limit;
    int64_t row = 0;
    if (valid) row = rows ? static_cast<int64_t>(rows[idx]) : idx;
    const int64_t rs = valid ? crow[row] : 0;
    const int64_t re = valid ? crow[row + 1] : 0;
    subwave_row_exact<LI::LPR, HAS_VAL, kRowUnroll>(col, val, x, y, F, row, valid, rs, re);
  }
}

// Whole graph in row order: each wave takes one row (wave-row layouts) or
// 64/LPR consecutive rows (sub-wave layouts).
template <int LAYOUT, bool HAS_VAL>
__global__ __launch_bounds__(kBlock) void spmm_rows_kernel(const int64_t* __restrict__ crow,
                                                           const int64_t* __restrict__ col,
                                                           const float* __restrict__ val,
                                                           const float* __restrict__ x, float* __restrict__ y,
                                                           int64_t n, int64_t F, int64_t wave_base) {
  const int64_t wave_index = wave_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  light_wave<LAYOUT, HAS_VAL>(crow, col, val, x, y, F, nullptr, wave_index, n);
}

// SPLIT64 hub row: W waves, contiguous edge slices, fp64 partials, LDS
// reduction in wave order, one rounding.
template <int V, bool HAS_VAL>
__device__ __forceinline__ void hub_row_split64(const int64_t* __restrict__ col, const float* __restrict__ val,
                                                const float* __restrict__ x, float* __restrict__ y, int64_t F,
                                                int64_t row, int64_t rs, int64_t re) {
  constexpr int P = kWave * V;
  constexpr int U = 8;
  __shared__ double partial[8 * P];
  const int lane = lane_id();
  const int wave = wave_in_block();
  const int W = static_cast<int>(blockDim.x >> 6);
  const int64_t slice = (re - rs + W - 1) / W;
  const int64_t ws = rs + wave * slice < re ? rs + wave * slice : re;
  const int64_t we = ws + slice < re ? ws + slice : re;
  for (int64_t f0 = 0; f0 < F; f0 += P) {
    const int64_t fl = f0 + static_cast<int64_t>(lane) * V;
    const bool active = fl < F;
    const float* xf = x + fl;
    double acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0;
    for (int64_t base = ws; base < we; base += kWave) {
      const int cnt = static_cast<int>((we - base) < kWave ? (we - base) : kWave);
      int my_col = 0;
      float my_w = 1.f;
      if (lane < cnt) {
        my_col = static_cast<int>(col[base + lane]);
        if constexpr (HAS_VAL) my_w = val[base + lane];
      }
      for (int j = 0; j < cnt; j += U) {
        FVec<V> xv[U];
        float w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
          for (int v = 0; v < V; ++v) xv[u].v[v] = 0.f;
          w[u] = 1.f;
          if (j + u < cnt) {
            const int c = bcast_i32(my_col, j + u);
            if constexpr (HAS_VAL) w[u] = bcast_f32(my_w, j + u);
            if (active) xv[u] = load_vec<V>(xf + static_cast<int64_t>(c) * F);
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (j + u < cnt) {
#pragma unroll
            for (int v = 0; v < V; ++v) {
              acc[v] = __builtin_fma(static_cast<double>(w[u]), static_cast<double>(xv[u].v[v]), acc[v]);
            }
          }
        }
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) partial[wave * P + lane * V + v] = acc[v];
    __syncthreads();
    for (int t = static_cast<int>(threadIdx.x); t < P; t += static_cast<int>(blockDim.x)) {
      if (f0 + t < F) {
        double s = partial[t];
        for (int w2 = 1; w2 < W; ++w2) s += partial[w2 * P + t];
        y[row * F + f0 + t] = static_cast<float>(s);
      }
    }
    __syncthreads();
  }
}

// Split schedule; see the file comment.  Work item = workgroup index.
template <int HV, int LAYOUT, bool HAS_VAL, bool SPLIT64>
__global__ __launch_bounds__(512) void spmm_scheduled_kernel(const int64_t* __restrict__ crow,
                                                             const int64_t* __restrict__ col,
                                                             const float* __restrict__ val,
                                                             const float* __restrict__ x, float* __restrict__ y,
                                                             int64_t n, int64_t F,
                                                             const int32_t* __restrict__ order,
                                                             const int32_t* __restrict__ counts,
                                                             int64_t item_base) {
  const int W = static_cast<int>(blockDim.x >> 6);
  const int wave = wave_in_block();
  const int64_t item = item_base + blockIdx.x;
  const int64_t heavy = counts[0];
  if (item < heavy) {
    const int64_t row = uniform_i64(order[item]);
    const int64_t rs = uniform_i64(crow[row]);
    const int64_t re = uniform_i64(crow[row + 1]);
    if constexpr (SPLIT64) {
      hub_row_split64<HV, HAS_VAL>(col, val, x, y, F, row, rs, re);
    } else {
      // feature slice of this wave, a multiple of HV
      int64_t slice = (F + W - 1) / W;
      slice = (slice + HV - 1) / HV * HV;
      const int64_t fbeg = wave * slice;
      const int64_t fend = fbeg + slice < F ? fbeg + slice : F;
      if (fbeg < F) wave_row_exact<HV, HAS_VAL, kHubUnroll>(col, val, x, y, F, row, rs, re, fbeg, fend);
    }
    return;
  }
  const int64_t light_wave_index = (item - heavy) * W + wave;
  light_wave<LAYOUT, HAS_VAL>(crow, col, val, x, y, F, order + heavy, light_wave_index, n - heavy);
}

// ----------------------------------------------------------------------------
// Host side

struct SpmmArgs {
  const int64_t* crow;
  const int64_t* col;
  const float* val;
  const float* x;
  float* y;
  int64_t n;
  int64_t f;
};

int rows_per_wave(int layout) { return layout == kSub16 ? 4 : layout == kSub32 ? 2 : 1; }

// Mean degree below which float4 sub-wave rows (16 or 32 lanes per row,
// several rows per wave) are used for short rows when vec4 is allowed; the
// same sums in the same order as one wave per row.  On graphs of a few
// edges per row a wave per row leaves most of its lanes and issue slots
// idle: the reference's Erdos-Renyi graph (200k rows, mean degree 4) takes
// 40.1 against 68.4 us at F = 64 and 72.4 against 96.8 us at F = 128.  At
// mean degree 8 (16,384 rows) both take 17.2 us; at 16 (2^20 rows,
// F = 128) one wave per row with SGPR column broadcast is faster (1.22
// against 1.26 ms), since the sub-wave form loads each column index per lane.
#ifndef AS_SUBWAVE_MAX_MEAN_DEGREE
#define AS_SUBWAVE_MAX_MEAN_DEGREE 12
#endif
constexpr int64_t kSubwaveMaxMeanDegree = AS_SUBWAVE_MAX_MEAN_DEGREE;

// Layout of the whole-graph kernel and of the light rows: float4 sub-wave
// rows when vec4 is allowed and rows are short on average, otherwise one
// wave per row (column broadcast through SGPRs).
int pick_layout(const SpmmArgs& a, int64_t nnz, int feature_tile, bool vec4) {
#ifdef AS_FORCE_LAYOUT
  return AS_FORCE_LAYOUT;
#endif
  const bool short_rows = nnz < kSubwaveMaxMeanDegree * a.n;
  const bool v4 = vec4 && a.f % 4 == 0 && aligned(a.x, 16) && aligned(a.y, 16);
  const bool v2 = a.f % 2 == 0 && aligned(a.x, 8) && aligned(a.y, 8);
  if (v4 && short_rows) {
    if (a.f <= 64 || feature_tile == 64) return kSub16;
    if (a.f <= 128) return kSub32;
  }
  if (v4 && a.f > 128 && feature_tile == 128) return kWaveV4;
  if (v2 && feature_tile == 128 && a.f > 64) return kWaveV2;
  return kWaveV1;
}

// Lane vector width for a hub row slice of `slice` features.
int pick_hub_vector(const SpmmArgs& a, int64_t slice, bool vec4) {
  if (vec4 && slice > 128 && a.f % 4 == 0 && aligned(a.x, 16) && aligned(a.y, 16)) return 4;
  if (slice > 64 && a.f % 2 == 0 && aligned(a.x, 8) && aligned(a.y, 8)) return 2;
  return 1;
}

template <int LAYOUT, bool HAS_VAL>
void launch_rows_t(const SpmmArgs& a, hipStream_t s) {
  const int64_t waves = (a.n + rows_per_wave(LAYOUT) - 1) / rows_per_wave(LAYOUT);
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    hipLaunchKernelGGL((spmm_rows_kernel<LAYOUT, HAS_VAL>), dim3(static_cast<unsigned>(nb)), dim3(kBlock), 0, s,
                       a.crow, a.col, a.val, a.x, a.y, a.n, a.f, b0 * kWavesPerBlock);
  }
}

template <bool HAS_VAL>
void launch_rows(const SpmmArgs& a, int layout, hipStream_t s) {
  switch (layout) {
    case kWaveV1: launch_rows_t<kWaveV1, HAS_VAL>(a, s); break;
    case kWaveV2: launch_rows_t<kWaveV2, HAS_VAL>(a, s); break;
    case kWaveV4: launch_rows_t<kWaveV4, HAS_VAL>(a, s); break;
    case kSub16: launch_rows_t<kSub16, HAS_VAL>(a, s); break;
    default: launch_rows_t<kSub32, HAS_VAL>(a, s); break;
  }
}

struct SchedLaunch {
  int64_t blocks;
  int waves;
  const int32_t* order;
  const int32_t* counts;
};

template <int HV, int LAYOUT, bool HAS_VAL, bool SPLIT64>
void launch_sched_t(const SpmmArgs& a, const SchedLaunch& l, hipStream_t s) {
  for (int64_t b0 = 0; b0 < l.blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = l.blocks - b0 < kMaxBlocksPerLaunch ? l.blocks - b0 : kMaxBlocksPerLaunch;
    hipLaunchKernelGGL((spmm_scheduled_kernel<HV, LAYOUT, HAS_VAL, SPLIT64>), dim3(static_cast<unsigned>(nb)),
                       dim3(static_cast<unsigned>(l.waves * kWave)), 0, s, a.crow, a.col, a.val, a.x, a.y, a.n, a.f,
                       l.order, l.counts, b0);
  }
}

template <int HV, bool HAS_VAL, bool SPLIT64>
void launch_sched_l(int layout, const SpmmArgs& a, const SchedLaunch& l, hipStream_t s) {
  switch (layout) {
    case kWaveV1: launch_sched_t<HV, kWaveV1, HAS_VAL, SPLIT64>(a, l, s); break;
    case kWaveV2: launch_sched_t<HV, kWaveV2, HAS_VAL, SPLIT64>(a, l, s); break;
    case kWaveV4: launch_sched_t<HV, kWaveV4, HAS_VAL, SPLIT64>(a, l, s); break;
    case kSub16: launch_sched_t<HV, kSub16, HAS_VAL, SPLIT64>(a, l, s); break;
    default: launch_sched_t<HV, kSub32, HAS_VAL, SPLIT64>(a, l, s); break;
  }
}

template <bool HAS_VAL, bool SPLIT64>
void launch_sched_v(int hv, int layout, const SpmmArgs& a, const SchedLaunch& l, hipStream_t s) {
  switch (hv) {
    case 4: launch_sched_l<4, HAS_VAL, SPLIT64>(layout, a, l, s); break;
    case 2: launch_sched_l<2, HAS_VAL, SPLIT64>(layout, a, l, s); break;
    default: launch_sched_l<1, HAS_VAL, SPLIT64>(layout, a, l, s); break;
  }
}

}  // namespace

constexpr int kSplitBuckets = 8;

size_t spmm_split_workspace_bytes(int64_t n) {
  const size_t order_bytes = align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(int32_t), 256);
  return order_bytes + 256 + bin_workspace_bytes(n);
}

}  // namespace as

extern "C" {

int as_spmm_csr_f32(const int64_t* crow, const int64_t* col, const float* val, const float* x, float* y, int64_t n,
                    int64_t nnz, int64_t f, int vec4, void* stream) {
  as::clear_error();
  int st = as::validate_spmm(crow, col, x, y, n, nnz, f);
  if (st != AS_OK) return st;
  if (n == 0 || f == 0) return AS_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const as::SpmmArgs a{crow, col, val, x, y, n, f};
  const int layout = as::pick_layout(a, nnz, 128, vec4 != 0);
  if (val != nullptr) as::launch_rows<true>(a, layout, s);
  else as::launch_rows<false>(a, layout, s);
  return as::check_launch("spmm_csr");
}

size_t as_spmm_split_workspace_bytes(int64_t n) { return as::spmm_split_workspace_bytes(n < 0 ? 0 : n); }

int as_spmm_csr_split_f32(const int64_t* crow, const int64_t* col, const float* val, const float* x, float* y,
                          int64_t n, int64_t nnz, int64_t f, int feature_tile, int waves_per_block,
                          int64_t hub_threshold, int vec4, int hub_mode, void* workspace, size_t workspace_bytes,
                          void* stream) {
  as::clear_error();
  if (feature_tile != 64 && feature_tile != 128)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "feature_tile must be 64 or 128");
  if (waves_per_block != 2 && waves_per_block != 4 && waves_per_block != 8)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "warps_per_block must be 2, 4, or 8");
  if (hub_threshold <= 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "hub_threshold must be positive");
  if (hub_mode != AS_HUB_EXACT && hub_mode != AS_HUB_SPLIT64)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "unknown hub mode %d", hub_mode);
  int st = as::validate_spmm(crow, col, x, y, n, nnz, f);
  if (st != AS_OK) return st;
  if (n == 0 || f == 0) return AS_OK;
  if (workspace == nullptr || workspace_bytes < as::spmm_split_workspace_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "split SpMM needs %zu workspace bytes, got %zu",
                    as::spmm_split_workspace_bytes(n), workspace_bytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* order = reinterpret_cast<int32_t*>(ws);
  const size_t order_bytes = as::align_up(static_cast<size_t>(n) * sizeof(int32_t), 256);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + order_bytes);
  void* bin_ws = ws + order_bytes + 256;
  const bool split64 = hub_mode == AS_HUB_SPLIT64;
  st = as::launch_bin_rows(crow, n, hub_threshold, split64 ? 1 : as::kSplitBuckets, as::kSplitBuckets, order,
                           counts, bin_ws, s);
  if (st != AS_OK) return st;

  const as::SpmmArgs a{crow, col, val, x, y, n, f};
  const int layout = as::pick_layout(a, nnz, feature_tile, vec4 != 0);
  const int64_t slice = split64 ? f : (f + waves_per_block - 1) / waves_per_block;
  const int hv = as::pick_hub_vector(a, slice, vec4 != 0);
  // At most min(n, nnz / T) hub rows; light rows need ceil(n / (W·rows per wave)) workgroups.
  int64_t heavy_upper = nnz / hub_threshold;
  if (heavy_upper > n) heavy_upper = n;
  const int64_t per_group = static_cast<int64_t>(waves_per_block) * as::rows_per_wave(layout);
  const as::SchedLaunch l{heavy_upper + (n + per_group - 1) / per_group, waves_per_block, order, counts};
  const bool has_val = val != nullptr;
  if (has_val) {
    if (split64) as::launch_sched_v<true, true>(hv, layout, a, l, s);
    else as::launch_sched_v<true, false>(hv, layout, a, l, s);
  } else {
    if (split64) as::launch_sched_v<false, true>(hv, layout, a, l, s);
    else as::launch_sched_v<false, false>(hv, layout, a, l, s);
  }
  return as::check_launch("spmm_csr_split");
}

}  // extern "C"
