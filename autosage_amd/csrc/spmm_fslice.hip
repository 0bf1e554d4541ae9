// Feature-sliced exact SpMM Y = A·X (fp32): every output element is one fp32
// accumulator updated in CSR edge order (fmaf with a weight, acc + x
// without), the order of the sequential CPU CSR product, so the result is
// bit-identical to it — and it runs XCD-local.
//
// Reference behaviour: the per-(row, feature) chain of
// csrc/spmm_csr_vec4.cu:42-50 and of the CPU path autosage/ops.py:124-143.
//
// Why.  An MI355X has 8 XCDs, each with its own 4 MB L2; gathers that miss
// it cross the fabric to the 256 MB MALL or HBM.  When whole rows go to
// waves, every XCD gathers from all of X and the eight L2s hold the same hot
// rows.  Cutting the column space instead (spmm_colslice.hip) splits every
// row's sum across XCDs, which reassociates it.  Here the FEATURES are cut:
// X is copied once per call into slice-major order xs[s][c][0:32] (32
// features = one 128-byte line per (column, slice)), and workgroup g works
// on slice g % 8 (folded onto the slices that exist: two XCDs per slice at
// F = 128, four at F = 64, one at F = 256, XCD x then slice x + 8 beyond).
// Workgroups are dispatched round-robin over the XCDs, so each XCD gathers
// from one slice only — 128 bytes per edge, a whole L2 line — and each
// (row, feature) chain still sees the row's edges in CSR order.  (With
// another dispatch order only the cache benefit would be lost, never a bit.)
//
// Measured on the skewed 115M-edge graph: 32-feature slices beat 16 (64-byte
// requests, 5.2 against 3.5 ms at F = 128), 64 (a twice larger L2 window,
// 4.2 ms) and whole rows (5.3 ms); the relayout alone matters because slices
// of row-major X sit 4·F bytes apart and crowd a fraction of the L2 channels.
//
// Lanes.  A (row, slice) is 8 lanes of float4; a wave holds 8 rows, a
// workgroup 4 waves = 32 consecutive rows of the plan's order.  The order
// sorts rows by degree (longest first, stable), so the 8 rows of a wave have
// nearly equal length: batches of U edges run unmasked up to the wave's
// shortest row, the last batches mask per lane, and groups of 8 edges past
// the wave's longest row are skipped (uniform branch).  Column indices (and
// weights) come from the plan as int32: lane j of a row's 8 loads edge
// k + 8v + j, and ds_swizzle hands each edge's index to the 8 lanes, one
// load per 8 edges instead of one per edge; the address unit was ~85 % busy
// with per-edge index loads.  U = 40 edges in flight per lane (2 waves per
// SIMD) beat 16-32 at 3-4 waves: long rows are latency chains.
//
// Column phases.  Each XCD still gathers from a window of N x 128 bytes
// (29.8 MB on the 233k-row graph) against its 4 MB L2.  Where the columns of
// every row ascend, the product can run as P launches: launch p takes every
// row's edges whose column lies in the p-th of P equal column ranges, and
// continues the row's fp32 chain from Y (launch 0 starts it from 0 and writes
// every row).  A row's edges in range p follow those in range p - 1 in CSR
// order, so each output is the same chain and the same bits; the gather
// window is P times smaller.  Any split point gives the same bits (a row's
// edges are cut into consecutive runs, summed in order); only the locality
// depends on the columns ascending.  On the skewed graph, two phases take
// F = 128 from 3.15 to 2.82 ms; more phases pay more than they gain (each
// launch waits for its longest chains, and every (row, phase) pays its own
// dependent start).
//
// Plan (per graph, X-independent): a header (int32 flags: bit 0 = a column
// outside [0, n_cols), clamped to 0 so no access leaves X; bit 1 = a row of
// 2^31 or more edges), the row order, the columns as int32 padded with
// kColPad zeros, and per phase one 16-byte task per position of the order
// (row, the row's edge count in the phase, the phase's first edge), so that a
// wave reaches its edges with one load.
#include <rocprim/device/device_radix_sort.hpp>

#include "as_device.h"
#include "as_internal.h"

namespace as {

namespace {

constexpr int kSliceWidth = 32;                 // features per slice: one 128-byte line
constexpr int kSliceLanes = kSliceWidth / 4;    // float4 lanes per (row, slice)
constexpr int kRowsPerWave = kWave / kSliceLanes;
constexpr int kFsliceWaves = 4;
constexpr int kRowsPerGroup = kFsliceWaves * kRowsPerWave;
constexpr int kXcds = 8;
constexpr int kFsliceUnroll = 40;               // edges in flight per lane (a multiple of 8)
// Where several XCDs share a slice, each takes runs of kSuperblock
// consecutive 32-row blocks of the order in turn (runs of 4: cfg3 F = 64
// 1.626 against 1.671 ms with single blocks, F = 128 3.157 against 3.174;
// runs of 32 or more leave the longest rows to one XCD and are slower).
constexpr int64_t kSuperblock = 4;
constexpr int64_t kColPad = 64;
constexpr int64_t kHeaderBytes = 256;
constexpr int64_t kFslicePlanTag = (int64_t(3) << 48) | 1;  // | phases << 8
constexpr int kMaxPhases = 8;
enum : int32_t { kFlagBadColumn = 1, kFlagLongRow = 2 };

struct FslicePlan {
  int32_t* flags;
  int32_t* order;
  int32_t* col;
  int4* tasks;  // [phases][n]: row, edge count in the phase, first edge (low, high words)
};

size_t fslice_order_bytes(int64_t n) { return align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(int32_t), 256); }
size_t fslice_col_bytes(int64_t nnz) { return align_up(static_cast<size_t>(nnz + kColPad) * sizeof(int32_t), 256); }
size_t fslice_task_bytes(int64_t n, int phases) {
  return align_up(static_cast<size_t>(n > 0 ? n : 1) * static_cast<size_t>(phases) * sizeof(int4), 256);
}
size_t fslice_plan_bytes(int64_t n, int64_t nnz, int phases) {
  return kHeaderBytes + fslice_order_bytes(n) + fslice_col_bytes(nnz) + fslice_task_bytes(n, phases);
}

FslicePlan fslice_plan_view(void* base, int64_t n, int64_t nnz) {
  char* p = static_cast<char*>(base);
  return FslicePlan{reinterpret_cast<int32_t*>(p), reinterpret_cast<int32_t*>(p + kHeaderBytes),
                    reinterpret_cast<int32_t*>(p + kHeaderBytes + fslice_order_bytes(n)),
                    reinterpret_cast<int4*>(p + kHeaderBytes + fslice_order_bytes(n) + fslice_col_bytes(nnz))};
}

int64_t fslice_tag(int phases) { return kFslicePlanTag | (static_cast<int64_t>(phases) << 8); }
// The phase count of a feature-sliced plan tag, or 0 if it is not one.
int fslice_tag_phases(int64_t tag) {
  const int phases = static_cast<int>((tag >> 8) & 0xff);
  if (phases < 1 || phases > kMaxPhases || tag != fslice_tag(phases)) return 0;
  return phases;
}

// Slices of F features, and the slice count the XCDs are folded onto: a
// power of two up to 8 (XCDs per slice = 8 / it), else a multiple of 8.
int fslice_count(int64_t f) { return static_cast<int>((f + kSliceWidth - 1) / kSliceWidth); }
int fslice_padded(int ns) {
  if (ns > kXcds) return (ns + kXcds - 1) / kXcds * kXcds;
  int p = 1;
  while (p < ns) p <<= 1;
  return p;
}

size_t fslice_sort_temp_bytes(int64_t n) {
  size_t bytes = 0;
  uint32_t* k = nullptr;
  int32_t* v = nullptr;
  (void)rocprim::radix_sort_pairs_desc(nullptr, bytes, k, k, v, v, static_cast<unsigned>(n > 0 ? n : 1));
  return bytes;
}

size_t fslice_build_bytes(int64_t n) {
  const size_t rows = align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(uint32_t), 256);
  return 3 * rows + align_up(fslice_sort_temp_bytes(n), 256);
}

__global__ __launch_bounds__(kBlock) void fslice_keys_kernel(const int64_t* __restrict__ crow, int64_t n,
                                                             uint32_t* __restrict__ keys, int32_t* __restrict__ rows,
                                                             int32_t* __restrict__ flags) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t d = crow[i + 1] - crow[i];
  keys[i] = d > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(d < 0 ? 0 : d);
  rows[i] = static_cast<int32_t>(i);
  if (d > 0x7fffffff) atomicOr(flags, kFlagLongRow);
}

__global__ __launch_bounds__(kBlock) void fslice_columns_kernel(const int64_t* __restrict__ col, int64_t nnz,
                                                                int64_t n_cols, int32_t* __restrict__ out,
                                                                int32_t* __restrict__ flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  bool bad = false;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nnz + kColPad; i += stride) {
    int32_t c = 0;
    if (i < nnz) {
      const int64_t v = col[i];
      if (v < 0 || v >= n_cols) bad = true;
      else c = static_cast<int32_t>(v);
    }
    out[i] = c;
  }
  if (bad) atomicOr(flags, kFlagBadColumn);
}

// The tasks of position i of the order: the row's edges cut at the first
// column >= p * n_cols / phases (a lower bound over the row's columns; for
// columns that do not ascend it is some cut, kept monotone, which changes
// the locality and not the bits).
__global__ __launch_bounds__(kBlock) void fslice_tasks_kernel(const int64_t* __restrict__ crow,
                                                              const int64_t* __restrict__ col,
                                                              const int32_t* __restrict__ order, int64_t n,
                                                              int64_t n_cols, int phases, int4* __restrict__ tasks) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t row = order[i];
  const int64_t rs = crow[row];
  const int64_t re = crow[row + 1];
  const int64_t deg = re > rs ? re - rs : 0;
  int64_t lo = 0;
  for (int p = 0; p < phases; ++p) {
    int64_t hi = deg;
    if (p + 1 < phases) {
      const int64_t bound = n_cols * (p + 1) / phases;
      int64_t a = lo, b = deg;  // first edge in [lo, deg) with col >= bound
      while (a < b) {
        const int64_t m = a + (b - a) / 2;
        if (col[rs + m] < bound) a = m + 1;
        else b = m;
      }
      hi = a;
    }
    const int64_t first = rs + lo;
    tasks[static_cast<int64_t>(p) * n + i] =
        make_int4(row, static_cast<int>(hi - lo), static_cast<int>(static_cast<uint32_t>(first)),
                  static_cast<int>(static_cast<uint64_t>(first) >> 32));
    lo = hi;
  }
}

__global__ __launch_bounds__(kBlock) void fslice_flags_clear_kernel(int32_t* __restrict__ flags) {
  if (threadIdx.x == 0) flags[0] = 0;
}

// xs[s][c][0:32] = x[c][32 s : 32 s + 32], zeros past F.
__global__ __launch_bounds__(kBlock) void fslice_relayout_kernel(const float* __restrict__ x, float* __restrict__ xs,
                                                                 int64_t n_cols, int64_t F, int ns, int vec) {
  const int64_t per_row = static_cast<int64_t>(ns) * kSliceLanes;
  const int64_t total = n_cols * per_row;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int64_t c = t / per_row;
    const int r = static_cast<int>(t - c * per_row);
    const int s = r / kSliceLanes;
    const int j = r - s * kSliceLanes;
    const int64_t f0 = static_cast<int64_t>(s) * kSliceWidth + j * 4;
    FVec<4> v;
    if (vec) {
      if (f0 < F) {
        v = load_vec<4>(x + c * F + f0);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v.v[q] = 0.f;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) v.v[q] = f0 + q < F ? x[c * F + f0 + q] : 0.f;
    }
    store_vec<4>(xs + (static_cast<int64_t>(s) * n_cols + c) * kSliceWidth + j * 4, v);
  }
}

// Lane I (0..7) of this lane's group of 8 (ds_swizzle, bit-mask mode: keep
// the group bits of the lane id, or in I).
template <int I>
__device__ __forceinline__ int group_lane(int v) {
  return __builtin_amdgcn_ds_swizzle(v, 0x18 | (I << 5));
}

// One phase: `tasks` are that phase's; `chain` = 1 continues every row that
// has edges in the phase from Y (phases after the first), 0 starts every row
// from zero and writes it (the first phase, which also writes empty rows).
template <bool HAS_VAL, bool WIDE>
__global__ __launch_bounds__(kBlock) void fslice_spmm_kernel(const int4* __restrict__ tasks,
                                                             const int32_t* __restrict__ colp,
                                                             const float* __restrict__ val,
                                                             const float* __restrict__ xs, float* __restrict__ y,
                                                             int64_t n, int64_t n_cols, int64_t F, int ns, int nsp,
                                                             int64_t blocks, int64_t group_base, int yvec,
                                                             int chain) {
  constexpr int U = kFsliceUnroll;
  constexpr int NG = U / 8;
  const int xcd = static_cast<int>(blockIdx.x & (kXcds - 1));
  const int64_t q = group_base + (blockIdx.x >> 3);
  int s;
  int64_t blk;
  if (nsp <= kXcds) {
    s = xcd & (nsp - 1);
    const int64_t xps = kXcds / nsp;  // XCDs per slice
    const int64_t sb = xps > 1 ? kSuperblock : 1;
    blk = (q / sb) * (sb * xps) + (xcd / nsp) * sb + q % sb;
  } else {
    s = xcd + kXcds * static_cast<int>(q / blocks);
    blk = q % blocks;
  }
  if (s >= ns) return;  // whole workgroup
  const int lane = lane_id();
  const int j = lane & (kSliceLanes - 1);
  const int64_t idx = blk * kRowsPerGroup + wave_in_block() * kRowsPerWave + lane / kSliceLanes;
  const bool valid = idx < n;
  int64_t row = 0;
  int64_t rs = 0;
  int deg = 0;
  if (valid) {
    const int4 t = tasks[idx];
    row = t.x;
    deg = t.y;
    rs = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(t.w)) << 32) | static_cast<uint32_t>(t.z));
  }
  int kmin = valid ? deg : 0x7fffffff;
  int kmax = deg;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int a = __shfl_xor(kmin, o, 64);
    const int b = __shfl_xor(kmax, o, 64);
    kmin = a < kmin ? a : kmin;
    kmax = b > kmax ? b : kmax;
  }
  kmin = uniform_i32(kmin);
  kmax = uniform_i32(kmax);
  const int dlast = deg > 0 ? deg - 1 : 0;
  const char* xb = reinterpret_cast<const char*>(xs + static_cast<int64_t>(s) * n_cols * kSliceWidth);
  const uint32_t lane_off = static_cast<uint32_t>(j) * 16u;
  // Empty rows read entry 0 of the arrays and never accumulate (val has no
  // entry at rs when an empty row ends the graph).
  const int64_t base = deg > 0 ? rs : 0;
  const int32_t* cp = colp + base;
  const float* vp = HAS_VAL ? val + base : nullptr;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int64_t f0 = static_cast<int64_t>(s) * kSliceWidth + j * 4;
  // a row continued from an earlier phase: its chain so far is in Y
  const bool resume = chain && valid && deg > 0 && f0 < F;
  if (resume) {
    if (yvec) {
      const FVec<4> o = load_vec<4>(y + row * F + f0);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = o.v[t];
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = f0 + t < F ? y[row * F + f0 + t] : 0.f;
    }
  }
  int cn[NG];
  float wn[NG];
#pragma unroll
  for (int v = 0; v < NG; ++v) {
    const int e0 = 8 * v + j;
    const int e = e0 < dlast ? e0 : dlast;
    cn[v] = cp[e];
    if constexpr (HAS_VAL) wn[v] = vp[e];
  }
  for (int k = 0; k < kmax; k += U) {
    FVec<4> xv[U];
    float w[U];
#pragma unroll
    for (int v = 0; v < NG; ++v) {
      if (v == 0 || k + 8 * v < kmax) {
        int c[8];
        c[0] = group_lane<0>(cn[v]);
        c[1] = group_lane<1>(cn[v]);
        c[2] = group_lane<2>(cn[v]);
        c[3] = group_lane<3>(cn[v]);
        c[4] = group_lane<4>(cn[v]);
        c[5] = group_lane<5>(cn[v]);
        c[6] = group_lane<6>(cn[v]);
        c[7] = group_lane<7>(cn[v]);
        if constexpr (HAS_VAL) {
          const int wi = __float_as_int(wn[v]);
          w[8 * v + 0] = __int_as_float(group_lane<0>(wi));
          w[8 * v + 1] = __int_as_float(group_lane<1>(wi));
          w[8 * v + 2] = __int_as_float(group_lane<2>(wi));
          w[8 * v + 3] = __int_as_float(group_lane<3>(wi));
          w[8 * v + 4] = __int_as_float(group_lane<4>(wi));
          w[8 * v + 5] = __int_as_float(group_lane<5>(wi));
          w[8 * v + 6] = __int_as_float(group_lane<6>(wi));
          w[8 * v + 7] = __int_as_float(group_lane<7>(wi));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if constexpr (WIDE) {
            xv[8 * v + i] = *reinterpret_cast<const FVec<4>*>(
                xb + static_cast<uint64_t>(static_cast<uint32_t>(c[i])) * (kSliceWidth * 4) + lane_off);
          } else {
            xv[8 * v + i] = load_vec_off<4>(reinterpret_cast<const float*>(xb),
                                            static_cast<uint32_t>(c[i]) * (kSliceWidth * 4u) + lane_off);
          }
        }
      }
    }
    if (k + U < kmax) {
#pragma unroll
      for (int v = 0; v < NG; ++v) {
        if (v == 0 || k + U + 8 * v < kmax) {
          const int e0 = k + U + 8 * v + j;
          const int e = e0 < dlast ? e0 : dlast;
          cn[v] = cp[e];
          if constexpr (HAS_VAL) wn[v] = vp[e];
        }
      }
    }
    if (k + U <= kmin) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if constexpr (HAS_VAL) acc[t] = __builtin_fmaf(w[u], xv[u].v[t], acc[t]);
          else acc[t] = acc[t] + xv[u].v[t];
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < NG; ++v) {
        if (v == 0 || k + 8 * v < kmax) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int u = 8 * v + i;
            const bool ok = k + u < deg;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              float r;
              if constexpr (HAS_VAL) r = __builtin_fmaf(w[u], xv[u].v[t], acc[t]);
              else r = acc[t] + xv[u].v[t];
              acc[t] = ok ? r : acc[t];
            }
          }
        }
      }
    }
  }
  if (valid && (!chain || deg > 0)) {
    if (yvec) {
      if (f0 < F) {
        FVec<4> o;
#pragma unroll
        for (int t = 0; t < 4; ++t) o.v[t] = acc[t];
        store_vec<4>(y + row * F + f0, o);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (f0 + t < F) y[row * F + f0 + t] = acc[t];
      }
    }
  }
}

template <bool HAS_VAL, bool WIDE>
void launch_fslice(const int4* tasks, const int32_t* colp, const float* val, const float* xs, float* y, int64_t n,
                   int64_t n_cols, int64_t f, int ns, int nsp, int yvec, int chain, hipStream_t s) {
  const int64_t blocks = (n + kRowsPerGroup - 1) / kRowsPerGroup;
  // nsp <= 8: q runs over the runs of every XCD of a slice (blocks past the
  // last one are whole workgroups of invalid rows, which store nothing)
  const int64_t xps = nsp <= kXcds ? kXcds / nsp : 1;
  const int64_t sb = xps > 1 ? kSuperblock : 1;
  const int64_t groups = nsp <= kXcds ? (blocks + sb * xps - 1) / (sb * xps) * sb : blocks * (nsp / kXcds);
  // groups of 8 workgroups (one per XCD); launches stay below the grid limit
  constexpr int64_t kMaxGroups = kMaxBlocksPerLaunch / kXcds;
  for (int64_t g0 = 0; g0 < groups; g0 += kMaxGroups) {
    const int64_t ng = groups - g0 < kMaxGroups ? groups - g0 : kMaxGroups;
    hipLaunchKernelGGL((fslice_spmm_kernel<HAS_VAL, WIDE>), dim3(static_cast<unsigned>(ng * kXcds)), dim3(kBlock),
                       0, s, tasks, colp, val, xs, y, n, n_cols, f, ns, nsp, blocks, g0, yvec, chain);
  }
}

}  // namespace

}  // namespace as

extern "C" {

size_t as_spmm_fslice_plan_bytes(int64_t n, int64_t nnz, int64_t phases) {
  if (phases < 1 || phases > as::kMaxPhases) return 0;
  return as::fslice_plan_bytes(n < 0 ? 0 : n, nnz < 0 ? 0 : nnz, static_cast<int>(phases));
}

size_t as_spmm_fslice_plan_workspace_bytes(int64_t n) { return as::fslice_build_bytes(n < 0 ? 0 : n); }

int as_spmm_fslice_plan(const int64_t* crow, const int64_t* col, int64_t n, int64_t n_cols, int64_t nnz,
                        int64_t phases, void* plan, size_t plan_bytes, void* workspace, size_t workspace_bytes,
                        int64_t* plan_tag, void* stream) {
  as::clear_error();
  if (phases < 1 || phases > as::kMaxPhases)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "phases must be in [1, %d]", as::kMaxPhases);
  const int ph = static_cast<int>(phases);
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (n_cols < 0 || n_cols > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "n_cols exceeds kernel index range");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (plan_tag == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "plan_tag must not be NULL");
  if (plan == nullptr || plan_bytes < as::fslice_plan_bytes(n, nnz, ph))
    return as::fail(AS_ERR_WORKSPACE, "feature-sliced plan needs %zu bytes, got %zu",
                    as::fslice_plan_bytes(n, nnz, ph), plan == nullptr ? size_t(0) : plan_bytes);
  if (workspace == nullptr || workspace_bytes < as::fslice_build_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "feature-sliced plan build needs %zu workspace bytes, got %zu",
                    as::fslice_build_bytes(n), workspace == nullptr ? size_t(0) : workspace_bytes);
  if (n > 0 && crow == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "null crow pointer");
  if (nnz > 0 && col == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "null col pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const as::FslicePlan p = as::fslice_plan_view(plan, n, nnz);
  hipLaunchKernelGGL(as::fslice_flags_clear_kernel, dim3(1), dim3(64), 0, s, p.flags);
  if (n > 0) {
    const size_t rows = as::align_up(static_cast<size_t>(n) * sizeof(uint32_t), 256);
    char* ws = static_cast<char*>(workspace);
    uint32_t* keys_in = reinterpret_cast<uint32_t*>(ws);
    uint32_t* keys_out = reinterpret_cast<uint32_t*>(ws + rows);
    int32_t* rows_in = reinterpret_cast<int32_t*>(ws + 2 * rows);
    void* temp = ws + 3 * rows;
    size_t temp_bytes = workspace_bytes - 3 * rows;
    hipLaunchKernelGGL(as::fslice_keys_kernel, dim3(static_cast<unsigned>((n + as::kBlock - 1) / as::kBlock)),
                       dim3(as::kBlock), 0, s, crow, n, keys_in, rows_in, p.flags);
    // stable: rows of equal degree keep ascending row order
    const hipError_t e = rocprim::radix_sort_pairs_desc(temp, temp_bytes, keys_in, keys_out, rows_in, p.order,
                                                        static_cast<unsigned>(n), 0, 32, s);
    if (e != hipSuccess) return as::fail(AS_ERR_LAUNCH, "feature-sliced plan: degree sort failed: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(as::fslice_tasks_kernel, dim3(static_cast<unsigned>((n + as::kBlock - 1) / as::kBlock)),
                       dim3(as::kBlock), 0, s, crow, col, p.order, n, n_cols, ph, p.tasks);
  }
  const int64_t total = nnz + as::kColPad;
  int64_t blocks = (total + as::kBlock - 1) / as::kBlock;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(as::fslice_columns_kernel, dim3(static_cast<unsigned>(blocks)), dim3(as::kBlock), 0, s, col,
                     nnz, n_cols, p.col, p.flags);
  *plan_tag = as::fslice_tag(ph);
  return as::check_launch("spmm_fslice_plan");
}

size_t as_spmm_fslice_workspace_bytes(int64_t n_cols, int64_t f) {
  if (n_cols <= 0 || f <= 0) return 256;
  return as::align_up(static_cast<size_t>(as::fslice_count(f)) * static_cast<size_t>(n_cols) * as::kSliceWidth *
                          sizeof(float),
                      256);
}

int as_spmm_fslice_relayout_f32(const float* x, int64_t n_cols, int64_t f, void* xs, size_t xs_bytes,
                                void* stream) {
  as::clear_error();
  if (n_cols < 0 || n_cols > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "n_cols exceeds kernel index range");
  if (f < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "F must be non-negative");
  if (f >= as::kMaxFeatures) return as::fail(AS_ERR_UNSUPPORTED, "F must be below 2^28");
  if (n_cols == 0 || f == 0) return AS_OK;
  if (x == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  const size_t need = as_spmm_fslice_workspace_bytes(n_cols, f);
  if (xs == nullptr || xs_bytes < need)
    return as::fail(AS_ERR_WORKSPACE, "feature-sliced SpMM needs %zu workspace bytes, got %zu", need,
                    xs == nullptr ? size_t(0) : xs_bytes);
  const int ns = as::fslice_count(f);
  const int vec = f % 4 == 0 && as::aligned(x, 16);
  const int64_t total = n_cols * ns * as::kSliceLanes;
  int64_t blocks = (total + as::kBlock - 1) / as::kBlock;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(as::fslice_relayout_kernel, dim3(static_cast<unsigned>(blocks)), dim3(as::kBlock), 0,
                     static_cast<hipStream_t>(stream), x, static_cast<float*>(xs), n_cols, f, ns, vec);
  return as::check_launch("spmm_fslice_relayout");
}

int as_spmm_csr_fslice_sliced_f32(const int64_t* crow, const float* val, const void* xs, size_t xs_bytes, float* y,
                                  int64_t n, int64_t n_cols, int64_t nnz, int64_t f, const void* plan,
                                  size_t plan_bytes, int64_t plan_tag, void* stream) {
  as::clear_error();
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (n_cols < 0 || n_cols > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "n_cols exceeds kernel index range");
  if (f < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "F must be non-negative");
  if (f >= as::kMaxFeatures) return as::fail(AS_ERR_UNSUPPORTED, "F must be below 2^28");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (n == 0 || f == 0) return AS_OK;
  if (crow == nullptr || y == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (nnz > 0 && n_cols == 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "edges into an empty column space");
  const int phases = as::fslice_tag_phases(plan_tag);
  if (phases == 0)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "plan tag %lld is not a feature-sliced plan",
                    static_cast<long long>(plan_tag));
  if (plan == nullptr || plan_bytes < as::fslice_plan_bytes(n, nnz, phases))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "feature-sliced plan of %zu bytes is too small for %lld rows, %lld "
                    "edges and %d phases (%zu)", plan == nullptr ? size_t(0) : plan_bytes, static_cast<long long>(n),
                    static_cast<long long>(nnz), phases, as::fslice_plan_bytes(n, nnz, phases));
  const size_t need = as_spmm_fslice_workspace_bytes(n_cols, f);
  if (xs == nullptr || xs_bytes < need)
    return as::fail(AS_ERR_WORKSPACE, "feature-sliced SpMM needs %zu workspace bytes, got %zu", need,
                    xs == nullptr ? size_t(0) : xs_bytes);
  // no edges: every row is empty and the kernel only writes zeros (it reads
  // entry 0 of the padded columns, and would read val[0], which may not exist)
  if (nnz == 0) val = nullptr;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const as::FslicePlan p = as::fslice_plan_view(const_cast<void*>(plan), n, nnz);
  const int ns = as::fslice_count(f);
  const int nsp = as::fslice_padded(ns);
  const float* xsf = static_cast<const float*>(xs);
  const int yvec = f % 4 == 0 && as::aligned(y, 16);
  const bool wide = static_cast<uint64_t>(n_cols) * as::kSliceWidth * sizeof(float) > 0xffffffffull;
  // one launch per phase, in order: phase q continues the chains phase q - 1 left in Y
  for (int q = 0; q < phases; ++q) {
    const int4* t = p.tasks + static_cast<int64_t>(q) * n;
    const int chain = q > 0;
    if (val != nullptr) {
      if (wide) as::launch_fslice<true, true>(t, p.col, val, xsf, y, n, n_cols, f, ns, nsp, yvec, chain, s);
      else as::launch_fslice<true, false>(t, p.col, val, xsf, y, n, n_cols, f, ns, nsp, yvec, chain, s);
    } else {
      if (wide) as::launch_fslice<false, true>(t, p.col, val, xsf, y, n, n_cols, f, ns, nsp, yvec, chain, s);
      else as::launch_fslice<false, false>(t, p.col, val, xsf, y, n, n_cols, f, ns, nsp, yvec, chain, s);
    }
  }
  return as::check_launch("spmm_csr_fslice");
}

int as_spmm_csr_fslice_f32(const int64_t* crow, const float* val, const float* x, float* y, int64_t n,
                           int64_t n_cols, int64_t nnz, int64_t f, const void* plan, size_t plan_bytes,
                           int64_t plan_tag, void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (n > 0 && f > 0 && nnz > 0 && n_cols > 0 && x == nullptr)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  // the checks of the sliced call first, so that no launch happens on bad arguments
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  const int phases = as::fslice_tag_phases(plan_tag);
  if (n > 0 && f > 0 && phases == 0)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "plan tag %lld is not a feature-sliced plan",
                    static_cast<long long>(plan_tag));
  if (n > 0 && f > 0 && nnz >= 0 && (plan == nullptr || plan_bytes < as::fslice_plan_bytes(n, nnz, phases)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "feature-sliced plan of %zu bytes is too small for %lld rows, %lld "
                    "edges and %d phases (%zu)", plan == nullptr ? size_t(0) : plan_bytes, static_cast<long long>(n),
                    static_cast<long long>(nnz), phases, as::fslice_plan_bytes(n, nnz, phases));
  if (n > 0 && f > 0 && nnz > 0) {
    const int st = as_spmm_fslice_relayout_f32(x, n_cols, f, workspace, workspace_bytes, stream);
    if (st != AS_OK) return st;
  }
  return as_spmm_csr_fslice_sliced_f32(crow, val, workspace, workspace_bytes, y, n, n_cols, nnz, f, plan, plan_bytes,
                                       plan_tag, stream);
}

}  // extern "C"
