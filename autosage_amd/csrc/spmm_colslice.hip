// Column-sliced SpMM Y = A·X for graphs whose columns ascend within every
// row (fp32 in and out, fp64 accumulation).
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
//      search, valid because columns ascend within the row).
//   2. Degree order: rows of degree >= 128 in log2-degree buckets, longest
//      first (the binning kernel of the split SpMM), then the shorter rows.
//   3. For each chunk of rows of that order: the slice kernel, one wave per
//      (row, slice), writes the fp64 partial sum of the row's edges in the
//      slice; the reduction kernel adds the non-empty partials of each row in
//      slice order in fp64 and rounds once to fp32.  A row shorter than 128
//      is summed whole by one wave (in fp64, rounded once) that writes Y:
//      its 8 partials would cost more traffic than slicing saves.
//
// Arithmetic.  Products w·x of fp32 values are exact in fp64 and every
// partial and the final sum are fp64 additions, so each output is within
// about one fp32 rounding of the exact sum (tighter than a sequential fp32
// sum), and the result is deterministic.  It is not bit-identical to the
// sequential CSR product: that order is kept by spmm.hip.
#include "as_device.h"
#include "as_internal.h"
#include "colslice_common.h"

namespace as {

namespace {

constexpr int kColsliceLongRow = 1024;     // slice length from which U = 16
// Rows shorter than this are not sliced: 8 fp64 partial rows (128·F bytes
// written and read) cost more than the cache gain on their few gathers.
#ifndef AS_COLSLICE_MIN_DEGREE
#define AS_COLSLICE_MIN_DEGREE 128
#endif
constexpr int64_t kColsliceMinDegree = AS_COLSLICE_MIN_DEGREE;
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
__device__ __forceinline__ void store_out(float* p, double v) { *p = static_cast<float>(v); }

// One wave sums edges [rs, re) of a row into out[0, F) in fp64 (F not a
// multiple of 4, or X not 16-byte aligned).  Same lane layout as the exact
// wave-row kernel: lane owns V consecutive features,
// 64 column indices per coalesced load (one chunk ahead), broadcast through
// SGPRs, U gathers in flight.
template <int V, bool HAS_VAL, int U, typename OutT>
__device__ __forceinline__ void slice_row(const int64_t* __restrict__ col, const float* __restrict__ val,
                                          const float* __restrict__ x, OutT* __restrict__ out, int64_t F,
                                          int64_t rs, int64_t re) {
  const int lane = lane_id();
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  for (int64_t f0 = 0; f0 < F; f0 += kWave * V) {
    const int64_t fl = f0 + static_cast<int64_t>(lane) * V;
    const bool active = fl < F;
    const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : 0) * 4);
    double acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0;
    int next_col = 0;
    float next_w = 1.f;
    if (lane < re - rs) {
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
              acc[v] = __builtin_fma(static_cast<double>(w[u]), static_cast<double>(xv[u].v[v]), acc[v]);
            } else {
              acc[v] = acc[v] + static_cast<double>(xv[u].v[v]);
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
            acc[v] = __builtin_fma(static_cast<double>(w), static_cast<double>(xv.v[v]), acc[v]);
          } else {
            acc[v] = acc[v] + static_cast<double>(xv.v[v]);
          }
        }
      }
    }
    if (active) {
#pragma unroll
      for (int v = 0; v < V; ++v) store_out(out + fl + v, acc[v]);
    }
  }
}

// Wide form of slice_row for F % 4 == 0 and 16-byte aligned X: G lanes per
// edge, each lane owning 4 consecutive features (a float4 load), so that one
// gather instruction fetches 64/G = EPI edges.  Gathers that hit L2 run at
// twice the bytes per instruction of 8-byte lanes (four times of 4-byte
// lanes).  Lane group k takes edges j + k, j + EPI + k, ... and keeps its own
// fp64 sums; the groups are added at the end in a fixed butterfly order.
// One call covers the feature tile [f0, f0 + 4·G).
template <int G, bool HAS_VAL, int U, typename OutT>
__device__ __forceinline__ void slice_row_wide(const int64_t* __restrict__ col, const float* __restrict__ val,
                                               const float* __restrict__ x, OutT* __restrict__ out, int64_t F,
                                               int64_t rs, int64_t re, int64_t f0) {
  constexpr int EPI = kWave / G;
  const int lane = lane_id();
  const int grp = lane / G;
  const int gl = lane % G;
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  {
    const int64_t fl = f0 + 4 * static_cast<int64_t>(gl);
    const bool active = fl < F;
    const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : f0) * 4);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    int next_col = 0;
    float next_w = 1.f;
    if (lane < re - rs) {
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
      for (int j = 0; j < cnt; j += U * EPI) {
        FVec<4> xv[U];
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
          xv[u] = load_vec_off<4>(x + row_offset(c, F), lane_bytes);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (live[u]) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              if constexpr (HAS_VAL) {
                acc[v] = __builtin_fma(static_cast<double>(w[u]), static_cast<double>(xv[u].v[v]), acc[v]);
              } else {
                acc[v] = acc[v] + static_cast<double>(xv[u].v[v]);
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (int o = G; o < kWave; o <<= 1) {
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] += __shfl_xor(acc[v], o, kWave);
    }
    if (grp == 0 && active) {
#pragma unroll
      for (int v = 0; v < 4; ++v) store_out(out + fl + v, acc[v]);
    }
  }
}

// slice_row_wide for 16-lane groups (F <= 64, 4 edges per gather), with
// less issue work per gather and the same sums in the same order:
//   * the lane group's column index comes from one ds_bpermute of the 64
//     indices of the block (instead of 4 readlanes and selects);
//   * with OFF32 (X smaller than 4 GiB and fewer than 2^24 rows) the X byte
//     offset is one 24-bit multiply-add and the gather uses the SGPR base
//     with a 32-bit VGPR offset;
//   * full batches carry no per-edge liveness test; only the last batch of a
//     block has one.  A lane group past the end reads the index register of
//     a lane with no edge in this block, which holds an earlier valid column
//     (or 0), and does not add what it gathers.
// On the 115M-edge skewed benchmark graph at F = 64 this takes the call from
// 2.18 to 2.00 ms; with 32-lane groups (2 edges per gather) the same changes
// cost about 1 %, so those keep slice_row_wide.
template <int G, bool HAS_VAL, int U, bool OFF32, typename OutT>
__device__ __forceinline__ void slice_row_wide_bpermute(const int64_t* __restrict__ col,
                                                        const float* __restrict__ val, const float* __restrict__ x,
                                                        OutT* __restrict__ out, int64_t F, int64_t rs, int64_t re,
                                                        int64_t f0) {
  constexpr int EPI = kWave / G;
  constexpr int B = U * EPI;
  static_assert(kWave % B == 0, "a batch must not straddle a block of 64 column indices");
  const int lane = lane_id();
  const int grp = lane / G;
  const int gl = lane % G;
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  const int64_t fl = f0 + 4 * static_cast<int64_t>(gl);
  const bool active = fl < F;
  const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : f0) * 4);
  const uint32_t row_bytes = static_cast<uint32_t>(F * 4);
  const char* __restrict__ xb = reinterpret_cast<const char*>(x);
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  int next_col = 0;
  float next_w = 1.f;
  if (lane < re - rs) {
    next_col = static_cast<int>(col[rs + lane]);
    if constexpr (HAS_VAL) next_w = val[rs + lane];
  }
  // edges e0 .. e0 + EPI - 1 of the block (e0 uniform), lane group grp
  // gathers edge e0 + grp
  auto gather = [&](int my_col, float my_w, int e0, float& w) -> FVec<4> {
    const int addr = (e0 + grp) * 4;
    const int c = __builtin_amdgcn_ds_bpermute(addr, my_col);
    if constexpr (HAS_VAL) w = __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(my_w)));
    if constexpr (OFF32) {
      const uint32_t off = __umul24(static_cast<uint32_t>(c), row_bytes) + lane_bytes;
      return *reinterpret_cast<const FVec<4>*>(xb + off);
    } else {
      return load_vec_off<4>(x + row_offset(c, F), lane_bytes);
    }
  };
  auto add = [&](const FVec<4>& xv, float w) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (HAS_VAL) {
        acc[v] = __builtin_fma(static_cast<double>(w), static_cast<double>(xv.v[v]), acc[v]);
      } else {
        acc[v] = acc[v] + static_cast<double>(xv.v[v]);
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
      if constexpr (HAS_VAL) next_w = val[nb + lane];
    }
    int j = 0;
    for (; j + B <= cnt; j += B) {
      FVec<4> xv[U];
      float w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) xv[u] = gather(my_col, my_w, j + u * EPI, w[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) add(xv[u], w[u]);
    }
    if (j < cnt) {
      FVec<4> xv[U];
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
    for (int v = 0; v < 4; ++v) acc[v] += __shfl_xor(acc[v], o, kWave);
  }
  if (grp == 0 && active) {
#pragma unroll
    for (int v = 0; v < 4; ++v) store_out(out + fl + v, acc[v]);
  }
}

#ifndef AS_COLSLICE_WIDE_U
#define AS_COLSLICE_WIDE_U 4
#endif

template <int G, bool HAS_VAL, bool OFF32, typename OutT>
__device__ __forceinline__ void slice_wide(const int64_t* __restrict__ col, const float* __restrict__ val,
                                           const float* __restrict__ x, OutT* __restrict__ out, int64_t F,
                                           int64_t rs, int64_t re, int64_t f0) {
  if constexpr (G <= 16) {
    slice_row_wide_bpermute<G, HAS_VAL, AS_COLSLICE_WIDE_U, OFF32>(col, val, x, out, F, rs, re, f0);
  } else {
    slice_row_wide<G, HAS_VAL, AS_COLSLICE_WIDE_U>(col, val, x, out, F, rs, re, f0);
  }
}

// One chunk of the slice work: rows order[item_begin, item_begin + items),
// main block mb of 8·P·ceil(items / 4)·tiles (P = kPhases).  Within a tile,
// the blocks of phase p come before those of phase p + 1; a block takes slice
// 8·p + mb % 8 (so its XCD is mb % 8) and 4 waves of the chunk; the wave for
// (row, slice) writes the partial of chunk row `local` to
// partial[(slice·chunk_stride + local)·F ..].
// V in {1, 2}: narrow lanes (slice_row, all features); V = 16, 32: wide
// lanes with G = V lanes per edge (slice_row_wide), one feature tile of 4·G
// features per wave.  Feature tiles are the outermost index: every
// (slice, row) of tile 0 comes before tile 1, so that while a tile runs each
// XCD gathers only 4·G features of the X rows of its slice (for F > 128 this
// keeps the per-XCD working set of F = 128).
struct SliceChunk {
  int64_t item_begin;
  int64_t items;
  double* partial;
};

template <int V, bool HAS_VAL, bool OFF32>
__device__ __forceinline__ void colslice_main_block(int64_t mb, const int64_t* __restrict__ crow,
                                                    const int64_t* __restrict__ col, const float* __restrict__ val,
                                                    const float* __restrict__ x, float* __restrict__ y, int64_t F,
                                                    const int32_t* __restrict__ order,
                                                    const int32_t* __restrict__ counts,
                                                    const int32_t* __restrict__ off, const SliceChunk& c,
                                                    int64_t chunk_stride) {
  const int64_t phase_blocks = kSlices * ((c.items + kWavesPerBlock - 1) / kWavesPerBlock);
  const int64_t tile_blocks = kPhases * phase_blocks;
  const int64_t tile = mb / tile_blocks;
  const int64_t in_tile = mb - tile * tile_blocks;
  const int64_t phase = in_tile / phase_blocks;
  const int64_t in_phase = in_tile - phase * phase_blocks;
  const int slice = static_cast<int>(phase * kSlices + in_phase % kSlices);
  const int64_t local = (in_phase / kSlices) * kWavesPerBlock + wave_in_block();
  if (local >= c.items) return;
  const int64_t item = c.item_begin + local;
  const int64_t row = uniform_i64(order[item]);
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t deg = uniform_i64(crow[row + 1]) - rs;
  if (item >= counts[0]) {
    // short row: one wave (of the slice item % 8, to spread them over the
    // XCDs) sums the whole row and writes Y
    if (item % kSpmmSlices != slice) return;
    if constexpr (V >= 16) {
      slice_wide<V, HAS_VAL, OFF32>(col, val, x, y + row * F, F, rs, rs + deg, tile * 4 * V);
    } else {
      slice_row<V, HAS_VAL, 8>(col, val, x, y + row * F, F, rs, rs + deg);
    }
    return;
  }
  int64_t a, b;
  slice_range<kSpmmSlices>(off, row, slice, deg, a, b);
  a = uniform_i64(a);
  b = uniform_i64(b);
  if (a >= b) return;
  double* out = c.partial + (slice * chunk_stride + local) * F;
  if constexpr (V >= 16) {
    slice_wide<V, HAS_VAL, OFF32>(col, val, x, out, F, rs + a, rs + b, tile * 4 * V);
  } else {
    if (b - a >= kColsliceLongRow) slice_row<V, HAS_VAL, 16>(col, val, x, out, F, rs + a, rs + b);
    else slice_row<V, HAS_VAL, 8>(col, val, x, out, F, rs + a, rs + b);
  }
}

// Reduction of one chunk, block rb of R: Y[row, f..f+VR) = sum over the
// non-empty slices, in slice order, in fp64, rounded once, for the sliced
// rows (short rows wrote Y themselves).
template <int VR>
__device__ __forceinline__ void colslice_reduce_block(int64_t rb, int64_t R, const int64_t* __restrict__ crow,
                                                      const int32_t* __restrict__ off,
                                                      const int32_t* __restrict__ order,
                                                      const int32_t* __restrict__ counts, float* __restrict__ y,
                                                      int64_t F, const SliceChunk& c, int64_t chunk_stride) {
  const int64_t FV = F / VR;
  // only the sliced rows: order[0, counts[0])
  const int64_t sliced = counts[0] - c.item_begin;
  const int64_t total = (sliced < c.items ? (sliced > 0 ? sliced : 0) : c.items) * FV;
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
    FVec<VR> out;
#pragma unroll
    for (int v = 0; v < VR; ++v) out.v[v] = static_cast<float>(acc[v]);
    store_vec<VR>(y + row * F + f, out);
  }
}

// One launch of the pipeline: the slice work of chunk `m` and the reduction
// of the previous chunk `r`, whose partials a previous launch wrote.  The
// blocks come in groups of 8 (one per XCD); of the TG groups, RG evenly
// spread ones reduce and the others do slice work, so the HBM-streaming
// reduction runs beside the latency-bound gathers.  Group g reduces iff
// floor((g+1)·RG/TG) > floor(g·RG/TG); floor(g·RG/TG) groups before it
// reduce, so a slice block keeps blockIdx % 8 as its slice.
template <int V, bool HAS_VAL, int VR, bool OFF32>
__global__ __launch_bounds__(kBlock) void colslice_step_kernel(const int64_t* __restrict__ crow,
                                                               const int64_t* __restrict__ col,
                                                               const float* __restrict__ val,
                                                               const float* __restrict__ x, float* __restrict__ y,
                                                               int64_t F, const int32_t* __restrict__ order,
                                                               const int32_t* __restrict__ counts,
                                                               const int32_t* __restrict__ off, SliceChunk m,
                                                               SliceChunk r, int64_t chunk_stride, int64_t TG,
                                                               int64_t RG) {
  const int64_t g = blockIdx.x / kSlices;
  const int64_t within = blockIdx.x % kSlices;
  const int64_t before = g * RG / TG;
  if ((g + 1) * RG / TG > before) {
    colslice_reduce_block<VR>(before * kSlices + within, RG * kSlices, crow, off, order, counts, y, F, r,
                              chunk_stride);
  } else {
    colslice_main_block<V, HAS_VAL, OFF32>((g - before) * kSlices + within, crow, col, val, x, y, F, order, counts, off,
                                    m, chunk_stride);
  }
}

size_t colslice_fixed_bytes(int64_t n) {
  const size_t rows = static_cast<size_t>(n > 0 ? n : 1);
  return align_up(rows * kSpmmBounds * sizeof(int32_t), 256) + align_up(rows * sizeof(int32_t), 256) + 256 +
         bin_workspace_bytes(n);
}

size_t colslice_row_bytes(int64_t f) {
  return static_cast<size_t>(kSpmmSlices) * static_cast<size_t>(f) * sizeof(double);
}

// Rows per chunk when the workspace allows: the pipeline overlaps the
// reduction of chunk k with the slice work of chunk k + 1, so all but the
// last chunk's reduction is hidden.
#ifndef AS_COLSLICE_CHUNKS
#define AS_COLSLICE_CHUNKS 4
#endif
constexpr int64_t kColsliceChunks = AS_COLSLICE_CHUNKS;
constexpr int64_t kColsliceMinChunkRows = 4096;

int64_t preferred_chunk_rows(int64_t n) {
  int64_t c = (n + kColsliceChunks - 1) / kColsliceChunks;
  if (c < kColsliceMinChunkRows) c = n < kColsliceMinChunkRows ? n : kColsliceMinChunkRows;
  return c > 0 ? c : 1;
}

template <int V, bool HAS_VAL, int VR, bool OFF32>
void launch_one(dim3 grid, hipStream_t s, const int64_t* crow, const int64_t* col, const float* val, const float* x,
                float* y, int64_t f, const int32_t* order, const int32_t* counts, const int32_t* off,
                const SliceChunk& m, const SliceChunk& r, int64_t stride, int64_t TG, int64_t RG) {
  hipLaunchKernelGGL((colslice_step_kernel<V, HAS_VAL, VR, OFF32>), grid, dim3(kBlock), 0, s, crow, col, val, x, y, f,
                     order, counts, off, m, r, stride, TG, RG);
}

// OFF32 only matters for the wide lanes (V = 16, 32).
template <bool HAS_VAL, int VR>
void launch_step_v(int v, bool off32, dim3 grid, hipStream_t s, const int64_t* crow, const int64_t* col,
                   const float* val, const float* x, float* y, int64_t f, const int32_t* order, const int32_t* counts,
                   const int32_t* off, const SliceChunk& m, const SliceChunk& r, int64_t stride, int64_t TG,
                   int64_t RG) {
  switch (v) {
    case 32:
      if (off32) launch_one<32, HAS_VAL, VR, true>(grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
      else launch_one<32, HAS_VAL, VR, false>(grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
      break;
    case 16:
      if (off32) launch_one<16, HAS_VAL, VR, true>(grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
      else launch_one<16, HAS_VAL, VR, false>(grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
      break;
    case 2:
      launch_one<2, HAS_VAL, VR, false>(grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
      break;
    default:
      launch_one<1, HAS_VAL, VR, false>(grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
      break;
  }
}

// Launch of slice work `m` (items may be 0) beside the reduction of `r`
// (items may be 0).
void launch_step(int v, bool off32, int vr, bool has_val, int64_t tiles, hipStream_t s, const int64_t* crow, const int64_t* col,
                 const float* val, const float* x, float* y, int64_t f, const int32_t* order, const int32_t* counts,
                 const int32_t* off, const SliceChunk& m, const SliceChunk& r, int64_t stride) {
  const int64_t MG = tiles * kPhases * ((m.items + kWavesPerBlock - 1) / kWavesPerBlock);  // groups of 8 slice blocks
  int64_t RG = 0;
  if (r.items > 0) {
    // enough reduce blocks for one element per thread, at most a fifth of
    // the groups when they run beside slice work
    RG = (r.items * (f / vr) + kSlices * kBlock - 1) / (kSlices * kBlock);
    const int64_t cap = MG > 0 ? (MG + 3) / 4 : kGridStrideBlocks / kSlices;
    if (RG > cap) RG = cap;
    if (RG < 1) RG = 1;
  }
  const int64_t TG = MG + RG;
  if (TG == 0) return;
  const dim3 grid(static_cast<unsigned>(TG * kSlices));
  if (has_val) {
    if (vr == 2) launch_step_v<true, 2>(v, off32, grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
    else launch_step_v<true, 1>(v, off32, grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
  } else {
    if (vr == 2) launch_step_v<false, 2>(v, off32, grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
    else launch_step_v<false, 1>(v, off32, grid, s, crow, col, val, x, y, f, order, counts, off, m, r, stride, TG, RG);
  }
}

}  // namespace

}  // namespace as

extern "C" {

size_t as_spmm_colslice_workspace_bytes(int64_t n, int64_t f) {
  if (n < 0) n = 0;
  if (f < 1) f = 1;
  return as::colslice_fixed_bytes(n) + 2 * static_cast<size_t>(as::preferred_chunk_rows(n)) * as::colslice_row_bytes(f);
}

int as_spmm_csr_colslice_f32(const int64_t* crow, const int64_t* col, const float* val, const float* x, float* y,
                             int64_t n, int64_t nnz, int64_t f, void* workspace, size_t workspace_bytes,
                             void* stream) {
  as::clear_error();
  int st = as::validate_spmm(crow, col, x, y, n, nnz, f);
  if (st != AS_OK) return st;
  if (n == 0 || f == 0) return AS_OK;
  const size_t fixed = as::colslice_fixed_bytes(n);
  const size_t row_bytes = as::colslice_row_bytes(f);
  if (workspace == nullptr || workspace_bytes < fixed + 2 * row_bytes)
    return as::fail(AS_ERR_WORKSPACE, "column-sliced SpMM needs at least %zu workspace bytes, got %zu",
                    fixed + 2 * row_bytes, workspace_bytes);
  if (!as::aligned(workspace, 256)) return as::fail(AS_ERR_WORKSPACE, "workspace must be 256-byte aligned");

  // lanes: G = 16 lanes per edge with float4 loads for F <= 64, else G = 32
  // in tiles of 128 features; 8- or 4-byte lanes with one edge per gather
  // when F is not a multiple of 4 or X is not 16-byte aligned
  int v = 1;
  if (f % 4 == 0 && as::aligned(x, 16)) v = f <= 64 ? 16 : 32;
  else if (f % 2 == 0 && f > 64 && as::aligned(x, 8)) v = 2;
  const int64_t tiles = v >= 16 ? (f + 4 * v - 1) / (4 * v) : 1;
  // every X byte offset fits 32 bits, row index and row bytes fit 24 bits
  const bool off32 = n <= (int64_t(1) << 24) && f * 4 < (int64_t(1) << 24) && n * f * 4 <= (int64_t(1) << 32);
  const int vr = (f % 2 == 0 && as::aligned(y, 8)) ? 2 : 1;

  // two partial buffers of `chunk` rows each (chunk k writes buffer k % 2)
  int64_t chunk = static_cast<int64_t>((workspace_bytes - fixed) / (2 * row_bytes));
  const int64_t preferred = as::preferred_chunk_rows(n);
  if (chunk > preferred) chunk = preferred;
  // a launch holds at most 5/4 of the slice groups of a chunk
  const int64_t max_rows = as::kMaxBlocksPerLaunch * 4 / 5 / as::kSpmmSlices * as::kWavesPerBlock / tiles;
  if (chunk > max_rows) chunk = max_rows;
  if (chunk < 1) return as::fail(AS_ERR_UNSUPPORTED, "F = %lld is too wide for the column-sliced SpMM", (long long)f);

  const hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const size_t rows = static_cast<size_t>(n);
  int32_t* off = reinterpret_cast<int32_t*>(ws);
  ws += as::align_up(rows * as::kSpmmBounds * sizeof(int32_t), 256);
  int32_t* order = reinterpret_cast<int32_t*>(ws);
  ws += as::align_up(rows * sizeof(int32_t), 256);
  int32_t* counts = reinterpret_cast<int32_t*>(ws);
  ws += 256;
  void* bin_ws = ws;
  double* buffers[2] = {reinterpret_cast<double*>(static_cast<char*>(workspace) + fixed),
                        reinterpret_cast<double*>(static_cast<char*>(workspace) + fixed + chunk * row_bytes)};

  as::launch_slice_points<as::kSpmmSlices>(crow, col, n, as::kColsliceMinDegree, off, s);
  // order: rows of degree >= kColsliceMinDegree (sliced) in 8 log2-degree
  // buckets, longest first; then the short rows in row order
  st = as::launch_bin_rows(crow, n, as::kColsliceMinDegree, as::kMaxHeavyBuckets, 1, order, counts, bin_ws, s);
  if (st != AS_OK) return st;

  // launch k: slice work of chunk k beside the reduction of chunk k - 1
  const int64_t chunks = (n + chunk - 1) / chunk;
  as::SliceChunk previous{0, 0, buffers[1]};
  for (int64_t k = 0; k <= chunks; ++k) {
    as::SliceChunk current{k * chunk, 0, buffers[k % 2]};
    if (k < chunks) current.items = n - current.item_begin < chunk ? n - current.item_begin : chunk;
#if AS_COLSLICE_OVERLAP
    as::launch_step(v, off32, vr, val != nullptr, tiles, s, crow, col, val, x, y, f, order, counts, off, current, previous,
                    chunk);
#else
    as::launch_step(v, off32, vr, val != nullptr, tiles, s, crow, col, val, x, y, f, order, counts, off, current,
                    as::SliceChunk{0, 0, nullptr}, chunk);
    as::launch_step(v, off32, vr, val != nullptr, tiles, s, crow, col, val, x, y, f, order, counts, off,
                    as::SliceChunk{0, 0, nullptr}, current, chunk);
#endif
    previous = current;
  }
  return as::check_launch("spmm_csr_colslice");
}

}  // extern "C"
