// CSR SDDMM: out[e] = <query[row(e)], key[col[e]]> for every nonzero e.
//
// Reference behaviour: csrc/sddmm_csr_op.cu:19-50 (row kernel),
// :52-83 (hub kernel), :108-187 (launchers).
//
// Summation order (both reference kernels, :12-17 and :39-49): the 32 lanes
// of a warp each keep one fp32 partial, lane l adding features l, l+32,
// l+64, ... with fma; the 32 partials are then combined by the 16/8/4/2/1
// shfl_down tree.  Every kernel here reproduces exactly that order, so all
// SDDMM entry points give identical bits.
//
// gfx950 mapping: G lanes of a wave64 work on one edge and each lane holds
// S = 32/G of the 32 partials (partial l = S·j + s in lane j, slot s), loaded
// as one S-wide vector per 32-feature block.  64/G edges are in flight per
// wave iteration.  Tree steps with offset o >= S are lane butterflies
// (xor o/S, inside the G-lane group); steps with o < S add slots in-lane.
#include "as_device.h"
#include "as_internal.h"

namespace as {

size_t spmm_split_workspace_bytes(int64_t n);

namespace {

constexpr int kChunkEdges = 2048;  // edges per hub work item

template <int S>
__device__ __forceinline__ float ref_tree(float (&p)[S]) {
#pragma unroll
  for (int o = 16; o >= S; o >>= 1) {
#pragma unroll
    for (int s = 0; s < S; ++s) p[s] += __shfl_xor(p[s], o / S, 64);
  }
#pragma unroll
  for (int o = S / 2; o >= 1; o >>= 1) {
#pragma unroll
    for (int s = 0; s < o; ++s) p[s] += p[s + o];
  }
  return p[0];
}

// Dot products of one query row against UE·NG key rows (vector path,
// F = 32·MF features, G lanes per edge).  Writes out[e] for valid edges.
template <int G, int MF, int UE>
__device__ __forceinline__ void dot_edges_vec(const int64_t* __restrict__ col, const float* __restrict__ key,
                                              float* __restrict__ out, int64_t F, const float (&qv)[MF][32 / G],
                                              int64_t first, int64_t stride, int64_t end, int g, int j) {
  constexpr int S = 32 / G;
  FVec<S> kv[UE][MF];
  bool ok[UE];
  int64_t e[UE];
#pragma unroll
  for (int u = 0; u < UE; ++u) {
    e[u] = first + u * stride + g;
    ok[u] = e[u] < end;
    const int64_t ee = ok[u] ? e[u] : end - 1;
    const int c = static_cast<int>(col[ee]);
    const float* kr = key + row_offset(c, F) + S * j;
#pragma unroll
    for (int m = 0; m < MF; ++m) kv[u][m] = load_vec<S>(kr + 32 * m);
  }
#pragma unroll
  for (int u = 0; u < UE; ++u) {
    float p[S];
#pragma unroll
    for (int s = 0; s < S; ++s) p[s] = 0.f;
#pragma unroll
    for (int m = 0; m < MF; ++m) {
#pragma unroll
      for (int s = 0; s < S; ++s) p[s] = __builtin_fmaf(qv[m][s], kv[u][m].v[s], p[s]);
    }
    const float d = ref_tree<S>(p);
    if (ok[u] && j == 0) out[e[u]] = d;
  }
}

// Scalar path for any F: 32 lanes per edge (exactly the reference lane
// mapping), two edges per wave iteration; the query row is re-read from cache.
__device__ __forceinline__ void dot_edges_scalar(const int64_t* __restrict__ col, const float* __restrict__ qrow,
                                                 const float* __restrict__ key, float* __restrict__ out, int64_t F,
                                                 int64_t first, int64_t stride, int64_t end, int g, int j) {
  const int64_t e = first + g;
  const bool ok = e < end;
  const int64_t ee = ok ? e : end - 1;
  const int c = static_cast<int>(col[ee]);
  const float* kr = key + row_offset(c, F);
  float p[1] = {0.f};
  for (int64_t f = j; f < F; f += 32) p[0] = __builtin_fmaf(qrow[f], kr[f], p[0]);
  const float d = ref_tree<1>(p);
  if (ok && j == 0) out[e] = d;
  (void)stride;
}

template <int G, int MF>
__device__ __forceinline__ void load_query(const float* __restrict__ qrow, int j, float (&qv)[MF][32 / G]) {
  constexpr int S = 32 / G;
#pragma unroll
  for (int m = 0; m < MF; ++m) {
    const FVec<S> t = load_vec<S>(qrow + 32 * m + S * j);
#pragma unroll
    for (int s = 0; s < S; ++s) qv[m][s] = t.v[s];
  }
}

// One wave computes every edge of `row` (vector or scalar path).
template <int G, int MF, bool VEC>
__device__ __forceinline__ void sddmm_row(const int64_t* __restrict__ col, const float* __restrict__ query,
                                          const float* __restrict__ key, float* __restrict__ out, int64_t F,
                                          int64_t row, int64_t rs, int64_t re) {
  const int lane = lane_id();
  const int g = lane / G;
  const int j = lane % G;
  if constexpr (VEC) {
    constexpr int NG = kWave / G;
    constexpr int UE = MF <= 2 ? 4 : 2;
    float qv[MF][32 / G];
    load_query<G, MF>(query + row * F, j, qv);
    for (int64_t base = rs; base < re; base += NG * UE) dot_edges_vec<G, MF, UE>(col, key, out, F, qv, base, NG, re, g, j);
  } else {
    const float* qrow = query + row * F;
    for (int64_t base = rs; base < re; base += 2) dot_edges_scalar(col, qrow, key, out, F, base, 2, re, g, j);
  }
}

// One wave per row; rows of degree >= hub_threshold are left to the hub
// kernel (csrc/sddmm_csr_op.cu:35-37).
template <int G, int MF, bool VEC>
__global__ __launch_bounds__(kBlock) void sddmm_rows_kernel(const int64_t* __restrict__ crow,
                                                            const int64_t* __restrict__ col,
                                                            const float* __restrict__ query,
                                                            const float* __restrict__ key, float* __restrict__ out,
                                                            int64_t n, int64_t F, int64_t hub_threshold,
                                                            int64_t idx_base) {
  const int64_t row = idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  if (row >= n) return;
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);
  if (re - rs >= hub_threshold || re == rs) return;
  sddmm_row<G, MF, VEC>(col, query, key, out, F, row, rs, re);
}

// Work items of the hub kernel: hub h (order[h], h < counts[0]) is cut into
// ceil(deg / kChunkEdges) chunks; chunk_off[h] is the exclusive prefix and
// counts[2] the total.  One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void hub_chunk_scan_kernel(const int64_t* __restrict__ crow,
                                                              const int32_t* __restrict__ order,
                                                              int32_t* __restrict__ counts,
                                                              int32_t* __restrict__ chunk_off) {
  __shared__ int lds[1024 / kWave];
  const int64_t hubs = counts[0];
  const int64_t per = (hubs + 1023) / 1024;
  const int64_t begin = static_cast<int64_t>(threadIdx.x) * per;
  const int64_t end = begin + per < hubs ? begin + per : hubs;
  int local = 0;
  for (int64_t h = begin; h < end; ++h) {
    const int64_t r = order[h];
    local += static_cast<int>((crow[r + 1] - crow[r] + kChunkEdges - 1) / kChunkEdges);
  }
  // block exclusive scan
  const int lane = lane_id();
  const int wave = wave_in_block();
  const int incl = wave_incl_scan_i32(local);
  if (lane == 63) lds[wave] = incl;
  __syncthreads();
  int before = 0;
  int total = 0;
  for (int w = 0; w < 1024 / kWave; ++w) {
    before += (w < wave) ? lds[w] : 0;
    total += lds[w];
  }
  int running = before + incl - local;
  for (int64_t h = begin; h < end; ++h) {
    chunk_off[h] = running;
    const int64_t r = order[h];
    running += static_cast<int>((crow[r + 1] - crow[r] + kChunkEdges - 1) / kChunkEdges);
  }
  if (threadIdx.x == 0) counts[2] = total;
}

// Split SDDMM in one launch.  Workgroups [0, hub_blocks) stride over the hub
// chunk items (2048-edge pieces of hub rows; usually one each); the rest take
// the light rows in row order, one per wave, skipping hub and empty rows.
// Hub workgroups have the lowest indices, so they are dispatched first.
template <int G, int MF, bool VEC>
__global__ __launch_bounds__(512) void sddmm_scheduled_kernel(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const float* __restrict__ query,
    const float* __restrict__ key, float* __restrict__ out, int64_t n, int64_t F, int64_t hub_threshold,
    const int32_t* __restrict__ order, const int32_t* __restrict__ counts, const int32_t* __restrict__ chunk_off,
    int64_t hub_blocks, int64_t block_base) {
  constexpr int NG = VEC ? kWave / G : 2;
  const int lane = lane_id();
  const int g = lane / (VEC ? G : 32);
  const int j = lane % (VEC ? G : 32);
  const int wave = wave_in_block();
  const int waves = static_cast<int>(blockDim.x >> 6);
  const int64_t block = block_base + blockIdx.x;
  if (block < hub_blocks) {
    const int64_t hubs = counts[0];
    const int64_t items = counts[2];
    for (int64_t item = block; item < items; item += hub_blocks) {
      int64_t lo = 0;
      int64_t hi = hubs - 1;
      while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (chunk_off[mid] <= item) lo = mid;
        else hi = mid - 1;
      }
      const int64_t row = uniform_i64(order[lo]);
      const int64_t rs = uniform_i64(crow[row]);
      const int64_t re = uniform_i64(crow[row + 1]);
      const int64_t cs = rs + (item - uniform_i64(chunk_off[lo])) * kChunkEdges;
      const int64_t ce = cs + kChunkEdges < re ? cs + kChunkEdges : re;
      if constexpr (VEC) {
        float qv[MF][32 / G];
        load_query<G, MF>(query + row * F, j, qv);
        for (int64_t base = cs + static_cast<int64_t>(wave) * NG; base < ce; base += static_cast<int64_t>(waves) * NG)
          dot_edges_vec<G, MF, 1>(col, key, out, F, qv, base, NG, ce, g, j);
      } else {
        const float* qrow = query + row * F;
        for (int64_t base = cs + static_cast<int64_t>(wave) * 2; base < ce; base += static_cast<int64_t>(waves) * 2)
          dot_edges_scalar(col, qrow, key, out, F, base, 2, ce, g, j);
      }
    }
    return;
  }
  const int64_t row = (block - hub_blocks) * waves + wave;
  if (row >= n) return;
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);
  if (re - rs >= hub_threshold || re == rs) return;
  sddmm_row<G, MF, VEC>(col, query, key, out, F, row, rs, re);
}

struct SddmmArgs {
  const int64_t* crow;
  const int64_t* col;
  const float* q;
  const float* k;
  float* out;
  int64_t n;
  int64_t f;
};

bool vec_ok(const SddmmArgs& a) {
  const auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  return a.f % 32 == 0 && a.f / 32 <= 8 && a.f > 0 && al(a.q) && al(a.k);
}

int launch_sddmm_rows(const SddmmArgs& a, int64_t hub_threshold, hipStream_t stream) {
  const int64_t blocks = (a.n + kWavesPerBlock - 1) / kWavesPerBlock;
  const bool vec = vec_ok(a);
  const int mf = static_cast<int>(a.f / 32);
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    const dim3 grid(static_cast<unsigned>(nb));
    const int64_t base = b0 * kWavesPerBlock;
#define AS_ROWS(K) \
  hipLaunchKernelGGL(K, grid, dim3(kBlock), 0, stream, a.crow, a.col, a.q, a.k, a.out, a.n, a.f, hub_threshold, base)
    if (!vec) {
      AS_ROWS((sddmm_rows_kernel<32, 1, false>));
    } else {
      switch (mf) {
        case 1: AS_ROWS((sddmm_rows_kernel<8, 1, true>)); break;
        case 2: AS_ROWS((sddmm_rows_kernel<8, 2, true>)); break;
        case 3: AS_ROWS((sddmm_rows_kernel<8, 3, true>)); break;
        case 4: AS_ROWS((sddmm_rows_kernel<8, 4, true>)); break;
        case 5: AS_ROWS((sddmm_rows_kernel<8, 5, true>)); break;
        case 6: AS_ROWS((sddmm_rows_kernel<8, 6, true>)); break;
        case 7: AS_ROWS((sddmm_rows_kernel<8, 7, true>)); break;
        default: AS_ROWS((sddmm_rows_kernel<8, 8, true>)); break;
      }
    }
#undef AS_ROWS
  }
  return AS_OK;
}

// Workgroups given to the hub chunks of the scheduled kernel: one per chunk
// up to this cap (the host knows only an upper bound on the chunk count;
// workgroups past the real count exit at once).  A small fixed pool was a
// bottleneck when a low threshold makes tens of thousands of rows hub rows
// (cfg4, threshold 197: 2.96 ms with 4,096 pool waves against 1.82 ms at
// threshold 256), and a pool much smaller than the chunk count leaves the
// hub pass as a tail behind the light rows.
constexpr int64_t kHubBlocksMax = 65536;

int launch_sddmm_scheduled(const SddmmArgs& a, int waves, int64_t hub_threshold, int64_t item_upper,
                           const int32_t* order, const int32_t* counts, const int32_t* chunk_off, hipStream_t stream) {
  const int64_t hub_blocks = item_upper < kHubBlocksMax ? item_upper : kHubBlocksMax;
  const int64_t blocks = hub_blocks + (a.n + waves - 1) / waves;
  const dim3 block(static_cast<unsigned>(waves * kWave));
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    const dim3 grid(static_cast<unsigned>(nb));
#define AS_SCHED(K)                                                                                             \
  hipLaunchKernelGGL(K, grid, block, 0, stream, a.crow, a.col, a.q, a.k, a.out, a.n, a.f, hub_threshold, order, \
                     counts, chunk_off, hub_blocks, b0)
    if (!vec_ok(a)) {
      AS_SCHED((sddmm_scheduled_kernel<32, 1, false>));
    } else {
      switch (static_cast<int>(a.f / 32)) {
        case 1: AS_SCHED((sddmm_scheduled_kernel<8, 1, true>)); break;
        case 2: AS_SCHED((sddmm_scheduled_kernel<8, 2, true>)); break;
        case 3: AS_SCHED((sddmm_scheduled_kernel<8, 3, true>)); break;
        case 4: AS_SCHED((sddmm_scheduled_kernel<8, 4, true>)); break;
        case 5: AS_SCHED((sddmm_scheduled_kernel<8, 5, true>)); break;
        case 6: AS_SCHED((sddmm_scheduled_kernel<8, 6, true>)); break;
        case 7: AS_SCHED((sddmm_scheduled_kernel<8, 7, true>)); break;
        default: AS_SCHED((sddmm_scheduled_kernel<8, 8, true>)); break;
      }
    }
#undef AS_SCHED
  }
  return AS_OK;
}

int validate_sddmm(const SddmmArgs& a, int64_t nnz) {
  if (a.n < 0 || a.n > INT32_MAX || a.f < 0 || a.f > INT32_MAX)
    return fail(AS_ERR_INVALID_ARGUMENT, "SDDMM dimensions exceed the kernel index range");
  if (nnz < 0) return fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (a.n > 0 && a.crow == nullptr) return fail(AS_ERR_INVALID_ARGUMENT, "null crow pointer");
  if (nnz > 0 && (a.col == nullptr || a.q == nullptr || a.k == nullptr || a.out == nullptr))
    return fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  return AS_OK;
}

size_t sddmm_split_ws(int64_t n) {
  return spmm_split_workspace_bytes(n) + align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(int32_t), 256);
}

}  // namespace

}  // namespace as

extern "C" {

int as_sddmm_csr_f32(const int64_t* crow, const int64_t* col, const float* query, const float* key, float* out,
                     int64_t n, int64_t nnz, int64_t f, void* stream) {
  as::clear_error();
  as::SddmmArgs a{crow, col, query, key, out, n, f};
  int st = as::validate_sddmm(a, nnz);
  if (st != AS_OK) return st;
  if (n == 0 || nnz == 0) return AS_OK;
  if (f == 0) return as::fail(AS_ERR_UNSUPPORTED, "SDDMM with zero features is handled by the caller");
  st = as::launch_sddmm_rows(a, INT64_MAX, static_cast<hipStream_t>(stream));
  if (st != AS_OK) return st;
  return as::check_launch("sddmm_csr");
}

size_t as_sddmm_split_workspace_bytes(int64_t n) { return as::sddmm_split_ws(n < 0 ? 0 : n); }

int as_sddmm_csr_split_f32(const int64_t* crow, const int64_t* col, const float* query, const float* key,
                           float* out, int64_t n, int64_t nnz, int64_t f, int waves_per_block,
                           int64_t hub_threshold, void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  as::SddmmArgs a{crow, col, query, key, out, n, f};
  if (waves_per_block != 2 && waves_per_block != 4 && waves_per_block != 8)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "warps_per_block must be 2, 4, or 8");
  if (hub_threshold <= 0 || hub_threshold > INT32_MAX)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "hub_threshold must be a positive 32-bit integer");
  int st = as::validate_sddmm(a, nnz);
  if (st != AS_OK) return st;
  if (n == 0 || nnz == 0) return AS_OK;
  if (f == 0) return as::fail(AS_ERR_UNSUPPORTED, "SDDMM with zero features is handled by the caller");
  if (workspace == nullptr || workspace_bytes < as::sddmm_split_ws(n))
    return as::fail(AS_ERR_WORKSPACE, "split SDDMM needs %zu workspace bytes, got %zu", as::sddmm_split_ws(n),
                    workspace_bytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int32_t* order = reinterpret_cast<int32_t*>(ws);
  const size_t order_bytes = as::align_up(static_cast<size_t>(n) * sizeof(int32_t), 256);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + order_bytes);
  void* bin_ws = ws + order_bytes + 256;
  int32_t* chunk_off = reinterpret_cast<int32_t*>(ws + as::spmm_split_workspace_bytes(n));

  int64_t heavy_upper = nnz / hub_threshold;
  if (heavy_upper > n) heavy_upper = n;
  if (heavy_upper == 0) {
    // no row can reach the threshold: the row kernel covers everything
    st = as::launch_sddmm_rows(a, hub_threshold, s);
    if (st != AS_OK) return st;
    return as::check_launch("sddmm_csr_split");
  }
  st = as::launch_bin_rows(crow, n, hub_threshold, 1, 1, order, counts, bin_ws, s);
  if (st != AS_OK) return st;
  hipLaunchKernelGGL(as::hub_chunk_scan_kernel, dim3(1), dim3(1024), 0, s, crow, order, counts, chunk_off);
  const int64_t item_upper = nnz / as::kChunkEdges + heavy_upper;
  st = as::launch_sddmm_scheduled(a, waves_per_block, hub_threshold, item_upper, order, counts, chunk_off, s);
  if (st != AS_OK) return st;
  return as::check_launch("sddmm_csr_split");
}

}  // extern "C"
