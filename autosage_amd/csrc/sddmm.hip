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
#include "elem16.h"

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

// ---- bf16 / fp16 SDDMM -------------------------------------------------------
// out[e] = the fp64 sum of the exact products q[row(e), f]·k[col(e), f],
// rounded to fp32 and then to the element type (round to nearest even both
// times).  Products of two 16-bit values are exact in fp64, so an exact fp64
// sum does not depend on the order of the additions, and every schedule here
// gives the same bits.  There is no reference kernel for these types (its op
// takes float32 only, csrc/sddmm_csr_op.cu:94; its scheduler runs the
// gather-dot baseline, autosage/_auto.py:575-581).
//
// Vector lanes (F a multiple of 8 up to 512, 16-byte aligned rows): a lane
// holds 8 consecutive features, chunk j + G·m of the row for m < MB; G lanes
// per edge (the power of two covering F/8, at most 32), 64/G edges per
// gather instruction.  The query row is converted to fp64 once per row and
// kept in registers.  Other shapes take element lanes: 64 lanes per edge,
// lane l adding features l, l + 64, ...
// Edges are taken in blocks of 64: one coalesced load brings the block's
// column indices (one block ahead), and ds_bpermute hands each lane group its
// edge's column, so a pass waits for one round of key gathers only; UE
// gathers per lane are in flight (all 64 edges of a block at once for G <= 8,
// else 32, 16 or 8 at a time).
template <typename T, int G, int MB, bool OFF32>
__device__ __forceinline__ void dots16_vec(const int64_t* __restrict__ col, const T* __restrict__ key,
                                           uint16_t* __restrict__ out, int64_t F, const double (&qd)[MB][8],
                                           int64_t first, int64_t end, int64_t step, int g, int j) {
  constexpr int NG = kWave / G;
  constexpr int UE = NG >= 8 ? kWave / NG : (MB == 1 ? 8 : 4);  // gathers in flight per lane
  constexpr int kSub = NG * UE;                                    // edges per sub-pass, <= 64
  static_assert(kSub <= kWave, "a sub-pass stays inside its block of 64 edges");
  const int lane = lane_id();
  const int64_t chunks = F / 8;
  const char* __restrict__ kb = reinterpret_cast<const char*>(key);
  const uint32_t row_bytes = static_cast<uint32_t>(F * sizeof(T));
  uint32_t lane_off[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) lane_off[m] = static_cast<uint32_t>((j + G * m < chunks ? j + G * m : 0) * 16);
  int next_c = first + lane < end ? static_cast<int>(col[first + lane]) : 0;
  for (int64_t base = first; base < end; base += step) {
    const int my_c = next_c;
    const int64_t nb = base + step;
    if (nb < end) next_c = nb + lane < end ? static_cast<int>(col[nb + lane]) : 0;
    const int cnt = end - base < kWave ? static_cast<int>(end - base) : kWave;
    for (int u0 = 0; u0 < cnt; u0 += kSub) {
      // edge u0 + u·NG + g; steps u with u0 + u·NG >= cnt hold no edge of
      // any group and are skipped (wave-uniform)
      RawVec<16> kv[UE][MB];
#pragma unroll
      for (int u = 0; u < UE; ++u) {
        if (u0 + u * NG < cnt) {
          const int idx = u0 + u * NG + g;  // < 64
          const int c = __builtin_amdgcn_ds_bpermute(idx * 4, my_c);
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            if constexpr (OFF32) {
              kv[u][m] = load_raw<16>(kb + (__umul24(static_cast<uint32_t>(c), row_bytes) + lane_off[m]));
            } else {
              kv[u][m] = load_raw<16>(kb + static_cast<int64_t>(c) * row_bytes + lane_off[m]);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < UE; ++u) {
        if (u0 + u * NG < cnt) {
          double acc = 0.0;
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            if (j + G * m < chunks) {
#pragma unroll
              for (int p = 0; p < 8; ++p)
                acc = __builtin_fma(qd[m][p], static_cast<double>(Elem<T>::get(kv[u][m].w, p)), acc);
            }
          }
#pragma unroll
          for (int o = 1; o < G; o <<= 1) acc += __shfl_xor(acc, o, kWave);
          const int idx = u0 + u * NG + g;
          if (j == 0 && idx < cnt) out[base + idx] = Elem<T>::bits(acc);
        }
      }
    }
  }
}

template <typename T, int G, int MB>
__device__ __forceinline__ void load_query16(const T* __restrict__ qrow, int64_t F, int j, double (&qd)[MB][8]) {
  const int64_t chunks = F / 8;
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    const int64_t chunk = j + G * m;
    const RawVec<16> v = load_raw<16>(reinterpret_cast<const char*>(qrow + (chunk < chunks ? chunk : 0) * 8));
#pragma unroll
    for (int p = 0; p < 8; ++p) qd[m][p] = chunk < chunks ? static_cast<double>(Elem<T>::get(v.w, p)) : 0.0;
  }
}

template <typename T>
__device__ __forceinline__ void dots16_scalar(const int64_t* __restrict__ col, const T* __restrict__ qrow,
                                              const T* __restrict__ key, uint16_t* __restrict__ out, int64_t F,
                                              int64_t first, int64_t end, int64_t step) {
  const int lane = lane_id();
  for (int64_t e = first; e < end; e += step) {
    const int64_t c = uniform_i64(col[e]);
    const T* __restrict__ kr = key + c * F;
    double acc = 0.0;
    for (int64_t f = lane; f < F; f += kWave)
      acc = __builtin_fma(static_cast<double>(Elem<T>::at(qrow, f)), static_cast<double>(Elem<T>::at(kr, f)), acc);
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) acc += __shfl_xor(acc, o, kWave);
    if (lane == 0) out[e] = Elem<T>::bits(acc);
  }
}

// Edges [cs, ce) of `row`, taken by `waves` waves (this one is `wave`).
template <typename T, int G, int MB, bool VEC, bool OFF32>
__device__ __forceinline__ void sddmm16_edges(const int64_t* __restrict__ col, const T* __restrict__ query,
                                              const T* __restrict__ key, uint16_t* __restrict__ out, int64_t F,
                                              int64_t row, int64_t cs, int64_t ce, int wave, int waves) {
  if constexpr (VEC) {
    const int lane = lane_id();
    const int g = lane / G;
    const int j = lane % G;
    double qd[MB][8];
    load_query16<T, G, MB>(query + row * F, F, j, qd);
    dots16_vec<T, G, MB, OFF32>(col, key, out, F, qd, cs + static_cast<int64_t>(wave) * kWave, ce,
                         static_cast<int64_t>(waves) * kWave, g, j);
  } else {
    dots16_scalar<T>(col, query + row * F, key, out, F, cs + wave, ce, waves);
  }
}

// The split schedule of sddmm_scheduled_kernel for 16-bit elements:
// workgroups [0, hub_blocks) stride over the 2048-edge chunks of the rows of
// degree >= hub_threshold, the rest take the other rows one per wave.
template <typename T, int G, int MB, bool VEC, bool OFF32>
__device__ __forceinline__ void sddmm16_scheduled_body(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const T* __restrict__ query,
    const T* __restrict__ key, uint16_t* __restrict__ out, int64_t n, int64_t F, int64_t hub_threshold,
    const int32_t* __restrict__ order, const int32_t* __restrict__ counts, const int32_t* __restrict__ chunk_off,
    int64_t hub_blocks, int64_t block_base) {
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
      sddmm16_edges<T, G, MB, VEC, OFF32>(col, query, key, out, F, row, cs, ce, wave, waves);
    }
    return;
  }
  const int64_t row = (block - hub_blocks) * waves + wave;
  if (row >= n) return;
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);
  if (re - rs >= hub_threshold || re == rs) return;
  sddmm16_edges<T, G, MB, VEC, OFF32>(col, query, key, out, F, row, rs, re, 0, 1);
}

// The kernel, and the same with at most 80 VGPRs (6 waves per SIMD, a few
// bytes spilled) for 16 lanes per edge: F = 128 in bf16 on cfg4 takes 1.97 ms
// with it against 2.21 at 89 VGPRs (5 waves), while F = 64 (8 lanes) gains
// nothing (1.163 against 1.155).
#define AS_SDDMM16_PARAMS                                                                                    \
  const int64_t *__restrict__ crow, const int64_t *__restrict__ col, const T *__restrict__ query,          \
      const T *__restrict__ key, uint16_t *__restrict__ out, int64_t n, int64_t F, int64_t hub_threshold, \
      const int32_t *__restrict__ order, const int32_t *__restrict__ counts,                              \
      const int32_t *__restrict__ chunk_off, int64_t hub_blocks, int64_t block_base
#define AS_SDDMM16_ARGS crow, col, query, key, out, n, F, hub_threshold, order, counts, chunk_off, hub_blocks, block_base
template <typename T, int G, int MB, bool VEC, bool OFF32>
__global__ __launch_bounds__(512) void sddmm16_scheduled_kernel(AS_SDDMM16_PARAMS) {
  sddmm16_scheduled_body<T, G, MB, VEC, OFF32>(AS_SDDMM16_ARGS);
}
template <typename T, int G, int MB, bool VEC, bool OFF32>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(6))) void sddmm16_scheduled_kernel_w6(
    AS_SDDMM16_PARAMS) {
  sddmm16_scheduled_body<T, G, MB, VEC, OFF32>(AS_SDDMM16_ARGS);
}
#undef AS_SDDMM16_PARAMS
#undef AS_SDDMM16_ARGS

struct Sddmm16Args {
  const int64_t* crow;
  const int64_t* col;
  const void* q;
  const void* k;
  void* out;
  int64_t n;       // rows of the graph and of the query
  int64_t f;
  int64_t n_keys;  // rows of the key (n for a square graph)
};

// Every query and key byte offset fits 32 bits, and every row index 24 bits.
inline bool sddmm16_off32(const Sddmm16Args& a) {
  const int64_t rows = a.n > a.n_keys ? a.n : a.n_keys;
  return rows <= (int64_t(1) << 24) && rows * a.f * 2 <= (int64_t(1) << 32);
}

template <typename T, int G, int MB, bool VEC, bool OFF32>
void launch_sddmm16_v(const Sddmm16Args& a, dim3 grid, dim3 block, int64_t hub_threshold, const int32_t* order,
                      const int32_t* counts, const int32_t* chunk_off, int64_t hub_blocks, int64_t b0,
                      hipStream_t s) {
  if constexpr (VEC && G == 16) {
    hipLaunchKernelGGL((sddmm16_scheduled_kernel_w6<T, G, MB, VEC, OFF32>), grid, block, 0, s, a.crow, a.col,
                       static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<uint16_t*>(a.out), a.n,
                       a.f, hub_threshold, order, counts, chunk_off, hub_blocks, b0);
  } else {
    hipLaunchKernelGGL((sddmm16_scheduled_kernel<T, G, MB, VEC, OFF32>), grid, block, 0, s, a.crow, a.col,
                       static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<uint16_t*>(a.out), a.n,
                       a.f, hub_threshold, order, counts, chunk_off, hub_blocks, b0);
  }
}

// Lanes per edge G and chunks per lane MB for F features (vector lanes), or
// G = 0 for element lanes.
inline void sddmm16_shape(const Sddmm16Args& a, int& g, int& mb) {
  g = 0;
  mb = 1;
  if (a.f % 8 != 0 || a.f > 512 || !aligned(a.q, 16) || !aligned(a.k, 16)) return;
  const int64_t chunks = a.f / 8;
  if (chunks > 32) {
    g = 32;
    mb = 2;
    return;
  }
  g = 1;
  while (g < chunks) g <<= 1;
}

template <typename T>
void launch_sddmm16(const Sddmm16Args& a, int waves, int64_t hub_threshold, int64_t item_upper,
                    const int32_t* order, const int32_t* counts, const int32_t* chunk_off, hipStream_t s) {
  const int64_t hub_blocks = item_upper < kHubBlocksMax ? item_upper : kHubBlocksMax;
  const int64_t blocks = hub_blocks + (a.n + waves - 1) / waves;
  const dim3 block(static_cast<unsigned>(waves * kWave));
  int g, mb;
  sddmm16_shape(a, g, mb);
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    const dim3 grid(static_cast<unsigned>(nb));
  const bool off32 = sddmm16_off32(a);
#define AS_S16(G, MB, VEC)                                                                                      \
  do {                                                                                                         \
    if (off32)                                                                                                 \
      launch_sddmm16_v<T, G, MB, VEC, true>(a, grid, block, hub_threshold, order, counts, chunk_off, hub_blocks, \
                                            b0, s);                                                            \
    else                                                                                                       \
      launch_sddmm16_v<T, G, MB, VEC, false>(a, grid, block, hub_threshold, order, counts, chunk_off,          \
                                             hub_blocks, b0, s);                                               \
  } while (0)
    if (mb == 2) {
      AS_S16(32, 2, true);
    } else {
      switch (g) {
        case 1: AS_S16(1, 1, true); break;
        case 2: AS_S16(2, 1, true); break;
        case 4: AS_S16(4, 1, true); break;
        case 8: AS_S16(8, 1, true); break;
        case 16: AS_S16(16, 1, true); break;
        case 32: AS_S16(32, 1, true); break;
        default:
          launch_sddmm16_v<T, 64, 1, false, false>(a, grid, block, hub_threshold, order, counts, chunk_off,
                                                   hub_blocks, b0, s);
          break;
      }
    }
#undef AS_S16
  }
}

// ---- 16-bit SDDMM by blocks of edges ---------------------------------------
// The same dot products as above (the same lane layout, fp64 sums and
// butterfly: the same bits) over the edges in CSR order, 64 at a time, with
// no regard to rows: wave w takes blocks [w·B, w·B + B) of 64 edges.  Every
// gather instruction then carries 64/G edges however short the rows are (a
// wave per row issues one partly filled gather for a row of a few edges and
// waits for it), and long rows need no schedule of their own.  The query row
// is gathered per edge (consecutive edges share it, so those gathers hit
// the caches).
//
// Rows of the edges: the wave loads the ends of the 64 rows from r, the row
// of the block's first edge, and lane i finds the row of edge b + i by a
// binary search over them (ds_bpermute).  A block spanning more than 64 rows
// (empty rows) takes further rounds of 64.  r comes from a table for the
// wave's first block (edge_wave_rows_kernel, one binary search over crow per
// wave) and is the row of the previous block's last edge after that.
// 2 blocks a wave: cfg4 (50M edges, median degree 8) bf16 F = 64 takes
// 0.975 ms against 0.986 at 4 and 1.000 at 8 (the split schedule: 1.133);
// the 2.4M-row, 124M-edge attention graph at F = 64 1.988 against 2.000 and
// 2.032 (split: 2.756); the skewed 115M-edge graph at F = 128 2.890 against
// 2.930 and 3.011 (split: 3.257).
#ifndef AS_SDDMM16_EDGE_BLOCKS
#define AS_SDDMM16_EDGE_BLOCKS 2
#endif
constexpr int64_t kEdgeBlocksPerWave = AS_SDDMM16_EDGE_BLOCKS;
constexpr int64_t kEdgesPerWave = kWave * kEdgeBlocksPerWave;
constexpr int kEdgeWaves = 4;  // waves per workgroup

int64_t edge_waves(int64_t nnz) { return (nnz + kEdgesPerWave - 1) / kEdgesPerWave; }

size_t sddmm_edges_ws(int64_t nnz) {
  return align_up(static_cast<size_t>(edge_waves(nnz) > 0 ? edge_waves(nnz) : 1) * sizeof(int32_t), 256);
}

// rows[w] = the row holding edge w·kEdgesPerWave: the last r < n with
// crow[r] <= e (rows before it that are empty end at or before e).
__global__ __launch_bounds__(256) void edge_wave_rows_kernel(const int64_t* __restrict__ crow, int64_t n,
                                                             int64_t waves, int32_t* __restrict__ rows) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (w >= waves) return;
  const int64_t e = w * kEdgesPerWave;
  int64_t lo = 0;
  int64_t hi = n - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (crow[mid] <= e) lo = mid;
    else hi = mid - 1;
  }
  rows[w] = static_cast<int32_t>(lo);
}

// Lane i: the row of edge b + min(i, cnt - 1), given r, the row of edge b.
// Every lane of the wave must be active.  The rounds end at the last row
// whatever crow holds, and the result is clamped to [0, n).
__device__ __forceinline__ int block_edge_rows(const int64_t* __restrict__ crow, int64_t n, int64_t b, int cnt,
                                               int64_t r) {
  const int lane = lane_id();
  const int i = lane < cnt ? lane : cnt - 1;
  int row = -1;
  for (int64_t rr = r;; rr += kWave) {
    // rel: where row rr + lane ends (row n - 1 for lanes past it), relative
    // to b, clamped to [0, 64]
    const int64_t left = n - 1 - rr;  // >= 0
    const int lim = left < kWave ? static_cast<int>(left) : kWave;
    const int64_t d = crow[rr + 1 + (lane < lim ? lane : lim)] - b;
    const int rel = d < 0 ? 0 : (d > kWave ? kWave : static_cast<int>(d));
    // pos = #{l : rel_l <= i}, the ends being non-decreasing in l
    int pos = 0;
#pragma unroll
    for (int s = kWave / 2; s >= 1; s >>= 1) {
      const int v = __builtin_amdgcn_ds_bpermute((pos + s - 1) * 4, rel);
      pos = v <= i ? pos + s : pos;
    }
    const int rel_last = __builtin_amdgcn_readlane(rel, kWave - 1);
    if (pos == kWave - 1 && rel_last <= i) pos = kWave;
    if (row < 0 && pos < kWave) row = static_cast<int>(rr + pos);
    if (rel_last >= cnt || rr + kWave >= n) break;
  }
  const int last = static_cast<int>(n - 1);
  return row < 0 || row > last ? last : row;
}

// Byte offset of 16-byte chunk lane_off of row `row` of a [*, F] matrix.
template <bool OFF32>
__device__ __forceinline__ const char* chunk_at(const char* base, int row, uint32_t row_bytes, uint32_t lane_off) {
  if constexpr (OFF32) {
    return base + (__umul24(static_cast<uint32_t>(row), row_bytes) + lane_off);
  } else {
    return base + static_cast<int64_t>(row) * row_bytes + lane_off;
  }
}

// The dot products of one block of cnt <= 64 edges starting at edge b,
// vector lanes: lane j of lane group g holds chunks j + G·m of the edge's
// query and key rows.  my_c / my_row: lane i holds the column / row of edge
// b + i.
template <typename T, int G, int MB, bool OFF32>
__device__ __forceinline__ void edge_block16_vec(const char* __restrict__ kb, const char* __restrict__ qb,
                                                 uint16_t* __restrict__ out, int64_t F, int64_t b, int cnt, int my_c,
                                                 int my_row) {
  constexpr int NG = kWave / G;  // edges per gather instruction
  // key (and query) gathers in flight per lane and chunk; fewer at 32 lanes
  // an edge, which would spill at 4
  constexpr int UE = MB == 1 ? (G >= 32 ? 2 : (4 < G ? 4 : G)) : 1;
  constexpr int kSub = NG * UE;  // edges per sub-pass, divides 64
  static_assert(kWave % kSub == 0, "a sub-pass stays inside its block of 64 edges");
  const int lane = lane_id();
  const int g = lane / G;
  const int j = lane % G;
  const int64_t chunks = F / 8;
  const uint32_t row_bytes = static_cast<uint32_t>(F * sizeof(T));
  uint32_t lane_off[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) lane_off[m] = static_cast<uint32_t>((j + G * m < chunks ? j + G * m : 0) * 16);
  for (int u0 = 0; u0 < cnt; u0 += kSub) {
    RawVec<16> kv[UE][MB];
    RawVec<16> qv[UE][MB];
#pragma unroll
    for (int u = 0; u < UE; ++u) {
      if (u0 + u * NG < cnt) {
        const int addr = (u0 + u * NG + g) * 4;  // an edge of this block (< 64)
        const int c = __builtin_amdgcn_ds_bpermute(addr, my_c);
        const int rw = __builtin_amdgcn_ds_bpermute(addr, my_row);
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          kv[u][m] = load_raw<16>(chunk_at<OFF32>(kb, c, row_bytes, lane_off[m]));
          qv[u][m] = load_raw<16>(chunk_at<OFF32>(qb, rw, row_bytes, lane_off[m]));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UE; ++u) {
      if (u0 + u * NG < cnt) {
        double acc = 0.0;
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          if (j + G * m < chunks) {
#pragma unroll
            for (int p = 0; p < 8; ++p)
              acc = __builtin_fma(static_cast<double>(Elem<T>::get(qv[u][m].w, p)),
                                  static_cast<double>(Elem<T>::get(kv[u][m].w, p)), acc);
          }
        }
#pragma unroll
        for (int o = 1; o < G; o <<= 1) acc += __shfl_xor(acc, o, kWave);
        const int idx = u0 + u * NG + g;
        if (j == 0 && idx < cnt) out[b + idx] = Elem<T>::bits(acc);
      }
    }
  }
}

// A wave whose edges [b0, b1) all lie in row `row` (long rows): the lane's
// query chunks are loaded once and the blocks need no row lookup.  The same
// products, sums and butterfly.
template <typename T, int G, int MB, bool OFF32>
__device__ __forceinline__ void one_row_edges16_vec(const int64_t* __restrict__ col, const char* __restrict__ kb,
                                                    const char* __restrict__ qb, uint16_t* __restrict__ out,
                                                    int64_t F, int64_t b0, int64_t b1, int row) {
  constexpr int NG = kWave / G;
  constexpr int UE = MB == 1 ? (4 < G ? 4 : G) : 1;
  constexpr int kSub = NG * UE;
  static_assert(kWave % kSub == 0, "a sub-pass stays inside its block of 64 edges");
  const int lane = lane_id();
  const int g = lane / G;
  const int j = lane % G;
  const int64_t chunks = F / 8;
  const uint32_t row_bytes = static_cast<uint32_t>(F * sizeof(T));
  uint32_t lane_off[MB];
  RawVec<16> q[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    lane_off[m] = static_cast<uint32_t>((j + G * m < chunks ? j + G * m : 0) * 16);
    q[m] = load_raw<16>(chunk_at<OFF32>(qb, row, row_bytes, lane_off[m]));
  }
  int next_c = b0 + lane < b1 ? static_cast<int>(col[b0 + lane]) : 0;
  for (int64_t b = b0; b < b1; b += kWave) {
    const int cnt = b1 - b < kWave ? static_cast<int>(b1 - b) : kWave;
    const int my_c = next_c;
    if (b + kWave < b1) next_c = b + kWave + lane < b1 ? static_cast<int>(col[b + kWave + lane]) : 0;
    for (int u0 = 0; u0 < cnt; u0 += kSub) {
      RawVec<16> kv[UE][MB];
#pragma unroll
      for (int u = 0; u < UE; ++u) {
        if (u0 + u * NG < cnt) {
          const int c = __builtin_amdgcn_ds_bpermute((u0 + u * NG + g) * 4, my_c);
#pragma unroll
          for (int m = 0; m < MB; ++m) kv[u][m] = load_raw<16>(chunk_at<OFF32>(kb, c, row_bytes, lane_off[m]));
        }
      }
#pragma unroll
      for (int u = 0; u < UE; ++u) {
        if (u0 + u * NG < cnt) {
          double acc = 0.0;
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            if (j + G * m < chunks) {
#pragma unroll
              for (int p = 0; p < 8; ++p)
                acc = __builtin_fma(static_cast<double>(Elem<T>::get(q[m].w, p)),
                                    static_cast<double>(Elem<T>::get(kv[u][m].w, p)), acc);
            }
          }
#pragma unroll
          for (int o = 1; o < G; o <<= 1) acc += __shfl_xor(acc, o, kWave);
          const int idx = u0 + u * NG + g;
          if (j == 0 && idx < cnt) out[b + idx] = Elem<T>::bits(acc);
        }
      }
    }
  }
}

template <typename T, int G, int MB, bool VEC, bool OFF32>
__global__ __launch_bounds__(kEdgeWaves * kWave) __attribute__((amdgpu_waves_per_eu(8))) void sddmm16_edges_kernel(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const T* __restrict__ query,
    const T* __restrict__ key, uint16_t* __restrict__ out, int64_t n, int64_t nnz, int64_t F,
    const int32_t* __restrict__ wave_rows, int64_t waves, int64_t wave_base) {
  const int64_t w = wave_base + static_cast<int64_t>(blockIdx.x) * kEdgeWaves + wave_in_block();
  if (w >= waves) return;  // wave-uniform
  const int lane = lane_id();
  const int64_t b0 = uniform_i64(w * kEdgesPerWave);
  const int64_t b1 = uniform_i64(b0 + kEdgesPerWave < nnz ? b0 + kEdgesPerWave : nnz);
  int64_t r = uniform_i64(wave_rows[w]);
  const char* __restrict__ kb = reinterpret_cast<const char*>(key);
  const char* __restrict__ qb = reinterpret_cast<const char*>(query);
  if constexpr (VEC) {
    if (uniform_i64(crow[r + 1]) >= b1) {  // every edge of the wave is in row r
      one_row_edges16_vec<T, G, MB, OFF32>(col, kb, qb, out, F, b0, b1, static_cast<int>(r));
      return;
    }
  }
  int next_c = b0 + lane < b1 ? static_cast<int>(col[b0 + lane]) : 0;
  for (int64_t b = b0; b < b1; b += kWave) {
    const int cnt = b1 - b < kWave ? static_cast<int>(b1 - b) : kWave;
    const int my_c = next_c;
    if (b + kWave < b1) next_c = b + kWave + lane < b1 ? static_cast<int>(col[b + kWave + lane]) : 0;
    const int my_row = block_edge_rows(crow, n, b, cnt, r);
    r = __builtin_amdgcn_readlane(my_row, cnt - 1);
    if constexpr (VEC) {
      edge_block16_vec<T, G, MB, OFF32>(kb, qb, out, F, b, cnt, my_c, my_row);
    } else {
      // element lanes: lane l adds features l, l + 64, ... of each edge in
      // turn (the order of dots16_scalar)
      for (int idx = 0; idx < cnt; ++idx) {
        const int64_t c = __builtin_amdgcn_readlane(my_c, idx);
        const int64_t rw = __builtin_amdgcn_readlane(my_row, idx);
        const T* __restrict__ kr = key + c * F;
        const T* __restrict__ qr = query + rw * F;
        double acc = 0.0;
        for (int64_t f = lane; f < F; f += kWave)
          acc = __builtin_fma(static_cast<double>(Elem<T>::at(qr, f)), static_cast<double>(Elem<T>::at(kr, f)), acc);
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) acc += __shfl_xor(acc, o, kWave);
        if (lane == 0) out[b + idx] = Elem<T>::bits(acc);
      }
    }
  }
}

template <typename T>
void launch_sddmm16_edges(const Sddmm16Args& a, int64_t nnz, int32_t* wave_rows, hipStream_t s) {
  const int64_t waves = edge_waves(nnz);
  hipLaunchKernelGGL(edge_wave_rows_kernel, dim3(static_cast<unsigned>((waves + 255) / 256)), dim3(256), 0, s,
                     a.crow, a.n, waves, wave_rows);
  int g, mb;
  sddmm16_shape(a, g, mb);
  const bool off32 = sddmm16_off32(a);
  const int64_t blocks = (waves + kEdgeWaves - 1) / kEdgeWaves;
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    const dim3 grid(static_cast<unsigned>(nb));
    const dim3 block(kEdgeWaves * kWave);
#define AS_E16(G, MB, VEC, OFF)                                                                              \
  hipLaunchKernelGGL((sddmm16_edges_kernel<T, G, MB, VEC, OFF>), grid, block, 0, s, a.crow, a.col,           \
                     static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<uint16_t*>(a.out), a.n, \
                     nnz, a.f, wave_rows, waves, b0 * kEdgeWaves)
#define AS_E16_V(G, MB)                  \
  do {                                   \
    if (off32) AS_E16(G, MB, true, true); \
    else AS_E16(G, MB, true, false);      \
  } while (0)
    if (mb == 2) {
      AS_E16_V(32, 2);
    } else {
      switch (g) {
        case 1: AS_E16_V(1, 1); break;
        case 2: AS_E16_V(2, 1); break;
        case 4: AS_E16_V(4, 1); break;
        case 8: AS_E16_V(8, 1); break;
        case 16: AS_E16_V(16, 1); break;
        case 32: AS_E16_V(32, 1); break;
        default: AS_E16(64, 1, false, false); break;
      }
    }
#undef AS_E16_V
#undef AS_E16
  }
}

int validate_sddmm(const SddmmArgs& a, int64_t nnz) {
  if (a.n < 0 || a.n > INT32_MAX || a.f < 0)
    return fail(AS_ERR_INVALID_ARGUMENT, "SDDMM dimensions exceed the kernel index range");
  if (a.f >= as::kMaxFeatures) return fail(AS_ERR_UNSUPPORTED, "F must be below 2^28 (32-bit lane offsets)");
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

int as_sddmm_csr_rounded_16(const int64_t* crow, const int64_t* col, const void* query, const void* key, void* out,
                            int64_t n, int64_t nnz, int64_t f, int dtype, int waves_per_block, int64_t hub_threshold,
                            void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (waves_per_block != 2 && waves_per_block != 4 && waves_per_block != 8)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "warps_per_block must be 2, 4, or 8");
  if (hub_threshold <= 0 || hub_threshold > INT32_MAX)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "hub_threshold must be a positive 32-bit integer");
  if (!as::aligned(query, 2) || !as::aligned(key, 2) || !as::aligned(out, 2))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "query, key and out must be 2-byte aligned");
  // the fp32 argument check covers the shapes and null pointers
  const as::SddmmArgs shape{crow, col, static_cast<const float*>(query), static_cast<const float*>(key),
                            static_cast<float*>(out), n, f};
  int st = as::validate_sddmm(shape, nnz);
  if (st != AS_OK) return st;
  if (n == 0 || nnz == 0) return AS_OK;
  if (f == 0) return as::fail(AS_ERR_UNSUPPORTED, "SDDMM with zero features is handled by the caller");
  if (workspace == nullptr || workspace_bytes < as::sddmm_split_ws(n))
    return as::fail(AS_ERR_WORKSPACE, "16-bit SDDMM needs %zu workspace bytes, got %zu", as::sddmm_split_ws(n),
                    workspace_bytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const as::Sddmm16Args a{crow, col, query, key, out, n, f, n};
  char* ws = static_cast<char*>(workspace);
  int32_t* order = reinterpret_cast<int32_t*>(ws);
  const size_t order_bytes = as::align_up(static_cast<size_t>(n) * sizeof(int32_t), 256);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + order_bytes);
  void* bin_ws = ws + order_bytes + 256;
  int32_t* chunk_off = reinterpret_cast<int32_t*>(ws + as::spmm_split_workspace_bytes(n));
  int64_t heavy_upper = nnz / hub_threshold;
  if (heavy_upper > n) heavy_upper = n;
  int64_t item_upper = 0;
  if (heavy_upper > 0) {
    st = as::launch_bin_rows(crow, n, hub_threshold, 1, 1, order, counts, bin_ws, s);
    if (st != AS_OK) return st;
    hipLaunchKernelGGL(as::hub_chunk_scan_kernel, dim3(1), dim3(1024), 0, s, crow, order, counts, chunk_off);
    item_upper = nnz / as::kChunkEdges + heavy_upper;
  }
  // with item_upper == 0 there are no hub workgroups and no row reaches the
  // threshold, so the kernel reads neither the order nor the counts
  if (dtype == AS_DTYPE_BF16)
    as::launch_sddmm16<as::Bf16>(a, waves_per_block, hub_threshold, item_upper, order, counts, chunk_off, s);
  else
    as::launch_sddmm16<as::Fp16>(a, waves_per_block, hub_threshold, item_upper, order, counts, chunk_off, s);
  return as::check_launch("sddmm_csr_rounded_16");
}

size_t as_sddmm_edges_16_workspace_bytes(int64_t nnz) { return as::sddmm_edges_ws(nnz < 0 ? 0 : nnz); }

int as_sddmm_csr_edges_16_rect(const int64_t* crow, const int64_t* col, const void* query, const void* key,
                               void* out, int64_t n, int64_t n_keys, int64_t nnz, int64_t f, int dtype,
                               void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (n_keys < 0 || n_keys > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "n_keys exceeds kernel index range");
  if (dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (!as::aligned(query, 2) || !as::aligned(key, 2) || !as::aligned(out, 2))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "query, key and out must be 2-byte aligned");
  const as::SddmmArgs shape{crow, col, static_cast<const float*>(query), static_cast<const float*>(key),
                            static_cast<float*>(out), n, f};
  int st = as::validate_sddmm(shape, nnz);
  if (st != AS_OK) return st;
  if (n == 0 || nnz == 0) return AS_OK;
  if (f == 0) return as::fail(AS_ERR_UNSUPPORTED, "SDDMM with zero features is handled by the caller");
  if (workspace == nullptr || workspace_bytes < as::sddmm_edges_ws(nnz))
    return as::fail(AS_ERR_WORKSPACE, "16-bit SDDMM by edge blocks needs %zu workspace bytes, got %zu",
                    as::sddmm_edges_ws(nnz), workspace_bytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const as::Sddmm16Args a{crow, col, query, key, out, n, f, n_keys};
  int32_t* wave_rows = static_cast<int32_t*>(workspace);
  if (dtype == AS_DTYPE_BF16)
    as::launch_sddmm16_edges<as::Bf16>(a, nnz, wave_rows, s);
  else
    as::launch_sddmm16_edges<as::Fp16>(a, nnz, wave_rows, s);
  return as::check_launch("sddmm_csr_edges_16");
}

int as_sddmm_csr_edges_16(const int64_t* crow, const int64_t* col, const void* query, const void* key, void* out,
                          int64_t n, int64_t nnz, int64_t f, int dtype, void* workspace, size_t workspace_bytes,
                          void* stream) {
  return as_sddmm_csr_edges_16_rect(crow, col, query, key, out, n, n < 0 ? 0 : n, nnz, f, dtype, workspace,
                                    workspace_bytes, stream);
}

}  // extern "C"
