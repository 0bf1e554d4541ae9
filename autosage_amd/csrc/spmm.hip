// CSR SpMM Y = A·X for fp32 features on gfx950.
//
// Reference behaviour: csrc/spmm_csr_vec4.cu:23-176 (whole graph),
// csrc/spmm_rows.cu:11-157 (light rows), csrc/spmm_hub.cu:13-182 (hub rows),
// csrc/launcher_spmm.cu:22-72 (split launcher).
//
// Every kernel except the SPLIT64 hub kernel keeps, for each output element
// Y[r, f], one fp32 accumulator updated in CSR edge order with fmaf
// (acc + x when unweighted, which is the same value).  That is the order of
// the sequential CPU CSR product, so these kernels are bit-identical to it
// whatever the row-to-wave mapping, feature tiling or vector width.
//
// Layouts (all one row per lane group, lanes own consecutive features):
//   wave-row  one wave64 per row, lane owns V in {1,2,4} consecutive
//             features, a pass covers 64·V features.  Column indices and
//             weights of 64 edges are loaded cooperatively (one coalesced
//             load) and broadcast with v_readlane, so the X-row address is
//             wave-uniform.  U gathers are in flight per wave.
//   sub-wave  float4 lanes, LPR in {16,32} lanes per row, 64/LPR rows per
//             wave; for short uniform rows where a whole wave per row idles.
//   split64   one workgroup per hub row; its W waves take contiguous slices
//             of the row's edges, accumulate in fp64 and the slices are
//             summed in LDS in wave order (deterministic, reassociated).
#include "as_device.h"
#include "as_internal.h"

namespace as {

namespace {

enum RowSource : int { kAllRows = 0, kHeavyRows = 1, kLightRows = 2 };

// Maps the idx-th work item of a launch to a CSR row.
template <int SRC>
__device__ __forceinline__ bool pick_row(int64_t idx, int64_t n, const int32_t* __restrict__ order,
                                         const int32_t* __restrict__ counts, int64_t* row) {
  if constexpr (SRC == kAllRows) {
    *row = idx;
    return idx < n;
  } else if constexpr (SRC == kHeavyRows) {
    const int64_t heavy = counts[0];
    if (idx >= heavy) return false;
    *row = order[idx];
    return true;
  } else {
    const int64_t heavy = counts[0];
    if (idx >= n - heavy) return false;
    *row = order[heavy + idx];
    return true;
  }
}

// One wave per row; see the file comment.
template <int V, bool HAS_VAL, int U, int SRC>
__global__ __launch_bounds__(kBlock) void spmm_wave_row_kernel(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const float* __restrict__ val,
    const float* __restrict__ x, float* __restrict__ y, int64_t n, int64_t F,
    const int32_t* __restrict__ order, const int32_t* __restrict__ counts, int64_t idx_base) {
  const int lane = lane_id();
  const int64_t idx = idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  int64_t row = 0;
  if (!pick_row<SRC>(idx, n, order, counts, &row)) return;
  const int64_t rs = crow[row];
  const int64_t re = crow[row + 1];
  constexpr int P = kWave * V;

  for (int64_t f0 = 0; f0 < F; f0 += P) {
    const int64_t fl = f0 + static_cast<int64_t>(lane) * V;
    const bool active = fl < F;
    const float* xf = x + fl;
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;

    // Column/weight chunk of the next 64 edges, loaded one chunk ahead.
    int next_col = 0;
    float next_w = 1.f;
    if (rs < re && lane < re - rs) {
      next_col = static_cast<int>(col[rs + lane]);
      if constexpr (HAS_VAL) next_w = val[rs + lane];
    }
    for (int64_t base = rs; base < re; base += kWave) {
      const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
      const int my_col = next_col;
      const float my_w = next_w;
      const int64_t nb = base + kWave;
      if (nb < re && lane < re - nb) {
        next_col = static_cast<int>(col[nb + lane]);
        if constexpr (HAS_VAL) next_w = val[nb + lane];
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
              if constexpr (HAS_VAL) {
                acc[v] = __builtin_fmaf(w[u], xv[u].v[v], acc[v]);
              } else {
                acc[v] = acc[v] + xv[u].v[v];
              }
            }
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

// float4 lanes, LPR lanes per row, 64/LPR rows per wave.
template <int LPR, bool HAS_VAL, int U, int SRC>
__global__ __launch_bounds__(kBlock) void spmm_subwave_kernel(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const float* __restrict__ val,
    const float* __restrict__ x, float* __restrict__ y, int64_t n, int64_t F,
    const int32_t* __restrict__ order, const int32_t* __restrict__ counts, int64_t idx_base) {
  constexpr int RPW = kWave / LPR;
  constexpr int P = LPR * 4;
  const int lane = lane_id();
  const int sub = lane / LPR;
  const int sl = lane % LPR;
  const int64_t wave_idx = idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  const int64_t idx = wave_idx * RPW + sub;
  int64_t row = 0;
  const bool valid = pick_row<SRC>(idx, n, order, counts, &row);
  const int64_t rs = valid ? crow[row] : 0;
  const int64_t re = valid ? crow[row + 1] : 0;

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

// One workgroup of W waves per heavy row.  Wave w sums the contiguous edge
// slice [rs + w·S, rs + (w+1)·S) in fp64 (S = ceil(deg / W)), the W partial
// tiles meet in LDS and are added in wave order 0..W-1 in fp64, and the
// result is rounded to fp32 once.
template <int V, bool HAS_VAL, int W>
__global__ __launch_bounds__(512) void spmm_hub_split64_kernel(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const float* __restrict__ val,
    const float* __restrict__ x, float* __restrict__ y, int64_t n, int64_t F,
    const int32_t* __restrict__ order, const int32_t* __restrict__ counts, int64_t idx_base) {
  constexpr int P = kWave * V;
  constexpr int U = 8;
  __shared__ double partial[W][P];
  const int lane = lane_id();
  const int wave = wave_in_block();
  const int64_t idx = idx_base + blockIdx.x;
  int64_t row = 0;
  if (!pick_row<kHeavyRows>(idx, n, order, counts, &row)) return;  // workgroup-uniform
  const int64_t rs = crow[row];
  const int64_t re = crow[row + 1];
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
    for (int v = 0; v < V; ++v) partial[wave][lane * V + v] = acc[v];
    __syncthreads();
    for (int t = static_cast<int>(threadIdx.x); t < P; t += static_cast<int>(blockDim.x)) {
      if (f0 + t < F) {
        double s = partial[0][t];
#pragma unroll
        for (int w2 = 1; w2 < W; ++w2) s += partial[w2][t];
        y[row * F + f0 + t] = static_cast<float>(s);
      }
    }
    __syncthreads();
  }
}

struct SpmmArgs {
  const int64_t* crow;
  const int64_t* col;
  const float* val;
  const float* x;
  float* y;
  int64_t n;
  int64_t f;
  const int32_t* order;
  const int32_t* counts;
};

enum Layout : int { kWaveV1, kWaveV2, kWaveV4, kSub16, kSub32 };

// Launches `rows` row work items (upper bound) with the given layout.
template <int SRC, int U>
int launch_rows(const SpmmArgs& a, Layout layout, int64_t rows, bool has_val, hipStream_t stream) {
  if (rows <= 0) return AS_OK;
  const int waves_per_block = kWavesPerBlock;
  int64_t waves = rows;
  if (layout == kSub16) waves = (rows + 3) / 4;
  if (layout == kSub32) waves = (rows + 1) / 2;
  const int64_t blocks = (waves + waves_per_block - 1) / waves_per_block;
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    const int64_t wave_base = b0 * waves_per_block;
    const dim3 grid(static_cast<unsigned>(nb));
    const dim3 block(kBlock);
#define AS_LAUNCH(K)                                                                                        \
  hipLaunchKernelGGL(K, grid, block, 0, stream, a.crow, a.col, a.val, a.x, a.y, a.n, a.f, a.order, a.counts, \
                     wave_base)
    switch (layout) {
      case kWaveV1:
        if (has_val) AS_LAUNCH((spmm_wave_row_kernel<1, true, U, SRC>));
        else AS_LAUNCH((spmm_wave_row_kernel<1, false, U, SRC>));
        break;
      case kWaveV2:
        if (has_val) AS_LAUNCH((spmm_wave_row_kernel<2, true, U, SRC>));
        else AS_LAUNCH((spmm_wave_row_kernel<2, false, U, SRC>));
        break;
      case kWaveV4:
        if (has_val) AS_LAUNCH((spmm_wave_row_kernel<4, true, U, SRC>));
        else AS_LAUNCH((spmm_wave_row_kernel<4, false, U, SRC>));
        break;
      case kSub16:
        if (has_val) AS_LAUNCH((spmm_subwave_kernel<16, true, 8, SRC>));
        else AS_LAUNCH((spmm_subwave_kernel<16, false, 8, SRC>));
        break;
      case kSub32:
        if (has_val) AS_LAUNCH((spmm_subwave_kernel<32, true, 8, SRC>));
        else AS_LAUNCH((spmm_subwave_kernel<32, false, 8, SRC>));
        break;
    }
#undef AS_LAUNCH
  }
  return AS_OK;
}

template <int V, bool HAS_VAL>
void launch_split64_w(int waves, const SpmmArgs& a, int64_t blocks, int64_t base, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(blocks));
  switch (waves) {
    case 2:
      hipLaunchKernelGGL((spmm_hub_split64_kernel<V, HAS_VAL, 2>), grid, dim3(2 * kWave), 0, stream, a.crow, a.col,
                         a.val, a.x, a.y, a.n, a.f, a.order, a.counts, base);
      break;
    case 4:
      hipLaunchKernelGGL((spmm_hub_split64_kernel<V, HAS_VAL, 4>), grid, dim3(4 * kWave), 0, stream, a.crow, a.col,
                         a.val, a.x, a.y, a.n, a.f, a.order, a.counts, base);
      break;
    default:
      hipLaunchKernelGGL((spmm_hub_split64_kernel<V, HAS_VAL, 8>), grid, dim3(8 * kWave), 0, stream, a.crow, a.col,
                         a.val, a.x, a.y, a.n, a.f, a.order, a.counts, base);
      break;
  }
}

int launch_hub_split64(const SpmmArgs& a, int v, int waves, int64_t rows, bool has_val, hipStream_t stream) {
  for (int64_t b0 = 0; b0 < rows; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = rows - b0 < kMaxBlocksPerLaunch ? rows - b0 : kMaxBlocksPerLaunch;
    if (v == 4) {
      if (has_val) launch_split64_w<4, true>(waves, a, nb, b0, stream);
      else launch_split64_w<4, false>(waves, a, nb, b0, stream);
    } else if (v == 2) {
      if (has_val) launch_split64_w<2, true>(waves, a, nb, b0, stream);
      else launch_split64_w<2, false>(waves, a, nb, b0, stream);
    } else {
      if (has_val) launch_split64_w<1, true>(waves, a, nb, b0, stream);
      else launch_split64_w<1, false>(waves, a, nb, b0, stream);
    }
  }
  return AS_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Widest lane vector the feature width and pointer alignment allow, capped at cap.
int lane_vector(const float* x, const float* y, int64_t F, bool vec4, int cap) {
  if (vec4 && cap >= 4 && F % 4 == 0 && aligned(x, 16) && aligned(y, 16)) return 4;
  if (cap >= 2 && F % 2 == 0 && aligned(x, 8) && aligned(y, 8)) return 2;
  return 1;
}

int validate_spmm(const int64_t* crow, const int64_t* col, const float* x, float* y, int64_t n, int64_t nnz,
                  int64_t f) {
  if (n < 0 || n > INT32_MAX) return fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (f < 0 || f > INT32_MAX) return fail(AS_ERR_INVALID_ARGUMENT, "F exceeds kernel index range");
  if (nnz < 0) return fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (n > 0 && f > 0 && (crow == nullptr || x == nullptr || y == nullptr))
    return fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (nnz > 0 && col == nullptr) return fail(AS_ERR_INVALID_ARGUMENT, "null col pointer");
  return AS_OK;
}

}  // namespace

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
  as::SpmmArgs a{crow, col, val, x, y, n, f, nullptr, nullptr};
  const int v = as::lane_vector(x, y, f, vec4 != 0, 4);
  as::Layout layout;
  if (v == 4 && f <= 64) layout = as::kSub16;
  else if (v == 4 && f <= 128) layout = as::kSub32;
  else if (v == 4) layout = as::kWaveV4;
  else if (v == 2) layout = as::kWaveV2;
  else layout = as::kWaveV1;
  st = as::launch_rows<as::kAllRows, 8>(a, layout, n, val != nullptr, s);
  if (st != AS_OK) return st;
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
  st = as::launch_bin_rows(crow, n, hub_threshold, order, counts, bin_ws, s);
  if (st != AS_OK) return st;

  as::SpmmArgs a{crow, col, val, x, y, n, f, order, counts};
  const bool has_val = val != nullptr;
  // Hub rows: at most min(n, nnz / T) of them.
  int64_t heavy_upper = nnz / hub_threshold;
  if (heavy_upper > n) heavy_upper = n;
  const int hub_v = as::lane_vector(x, y, f, vec4 != 0, f > 128 ? 4 : 2);
  if (heavy_upper > 0) {
    if (hub_mode == AS_HUB_SPLIT64) {
      st = as::launch_hub_split64(a, hub_v, waves_per_block, heavy_upper, has_val, s);
    } else {
      const as::Layout hub_layout = hub_v == 4 ? as::kWaveV4 : hub_v == 2 ? as::kWaveV2 : as::kWaveV1;
      st = as::launch_rows<as::kHeavyRows, 16>(a, hub_layout, heavy_upper, has_val, s);
    }
    if (st != AS_OK) return st;
  }
  // Light rows: feature_tile features per pass.
  as::Layout light;
  const int lv = as::lane_vector(x, y, f, vec4 != 0, 4);
  if (lv == 4) light = feature_tile == 64 ? as::kSub16 : as::kSub32;
  else if (lv == 2 && feature_tile == 128) light = as::kWaveV2;
  else light = as::kWaveV1;
  st = as::launch_rows<as::kLightRows, 8>(a, light, n, has_val, s);
  if (st != AS_OK) return st;
  return as::check_launch("spmm_csr_split");
}

}  // extern "C"
