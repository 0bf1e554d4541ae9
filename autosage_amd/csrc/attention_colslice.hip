// Column-sliced CSR attention: out[r] = softmax_r(scale · <Q[r], K[c]>) · V,
// an alternative schedule for the fused attention (attention.hip) on graphs
// whose columns ascend within every row.
//
// Rows of degree >= D (att_slice_degree: 128 for fp32, 512 for 16-bit
// elements) are cut into the 8 column slices of colslice_common.h;
// workgroup g works on slice g % 8, so each XCD gathers K and V rows only
// from its eighth of the columns and its L2 caches eight times as many
// distinct rows as when every XCD gathers from all of them.  One wave per
// (row, slice) keeps an online softmax over the slice's edges (running max m,
// sum l = Σ exp(s - m), acc = Σ exp(s - m)·V[c]) and writes (m, l, acc) as
// fp32 partials; the reduction merges the 8 partials of a row
// (m = max m_s, out = Σ e^(m_s - m)·acc_s / Σ e^(m_s - m)·l_s).  Shorter rows
// run the same online softmax in one wave and write out directly.
//
// Gathers use float4 lanes: G lanes per edge for K (G = 16/32/64 for
// F_qk <= 64/128/256) and for V, 64/G edges per gather instruction.  A batch
// of 8 edges (16 with 16-bit elements) issues all its K and V gathers first;
// the scores are reduced
// inside each K lane group, broadcast through SGPRs and picked up by the V
// lane group that holds the same edge; each V lane group keeps its own
// online-softmax state, merged in a fixed butterfly order at the end.
//
// Not bit-identical to the fused kernel (that one keeps the reference's
// stage order); deterministic, and within about 0.2 of the 1e-5 relative /
// 1e-6 absolute bar against fp64 on the benchmark graph, as is the fused one.
//
// bf16 / fp16 inputs run the same kernels: a 16-byte lane holds 8 elements
// (4 for fp32), converted exactly to fp32; the online softmax and the partial
// states are fp32 and each output is rounded once to the element type (round
// to nearest even).  Scores and probabilities never leave registers, so a
// 16-bit attention is one pass over K and V instead of three stages, and it
// is more accurate than the stages, which round every score and probability
// to 16 bits.
#include "as_device.h"
#include "as_internal.h"
#include "colslice_common.h"
#include "elem16.h"
#include "attention_lanes.h"

namespace as {

namespace {

constexpr int64_t kAttChunkRows = 131072;    // sliced rows per partial chunk
constexpr int64_t kAttSliceBlocks = 4096;    // slice-kernel workgroups per slice
constexpr int64_t kAttReduceBlocks = 8192;   // reduction workgroups

// Edges per online-softmax step of a wave that walks one row or (row, slice)
// alone.  fp32: 8.  16-bit: 16, which keeps as many gathered bytes in flight
// per wave as fp32 with 8; with 16-bit elements the short rows run grouped
// (attend_rows_grouped, its own step), so this step serves the sliced rows:
// the benchmark attention (Fqk 64, Fv 128, 2.4M rows, rows sliced from
// degree 512) takes 5.63 against 5.78 ms in bf16.  (Before the short rows were
// grouped, 16 and 32 edges per step took it from 7.84 to 8.85 and 9.93 ms.)
#ifndef AS_ATT_BATCH_16
#define AS_ATT_BATCH_16 16
#endif
template <typename T>
constexpr int att_batch() {
  return sizeof(T) == 2 ? AS_ATT_BATCH_16 : 8;
}

// Online softmax of one wave over edges [rs, re) of a row.  On return every
// lane holds the merged state of the whole range; lane vl of a V group owns
// features P·vl .. P·vl + P-1 of acc.
// FQK / FV > 0: the feature widths as compile-time constants (the row stride
// of each gather becomes a shift instead of a per-lane 64-bit multiply).
template <typename T, int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void attend_edges(const int64_t* __restrict__ col, const T* __restrict__ key,
                                             const T* __restrict__ value, int64_t fqk_rt, int64_t fv_rt,
                                             const float (&q)[lane_elems<T>()], float scale, int64_t rs,
                                             int64_t re, float& m, float& l, float (&acc)[lane_elems<T>()]) {
  constexpr int P = lane_elems<T>();
  constexpr int EK = kWave / GK;  // edges per K gather instruction
  constexpr int EV = kWave / GV;  // edges per V gather instruction
  constexpr int E = att_batch<T>();
  static_assert(E % EK == 0 && E % EV == 0, "a batch holds whole gather instructions");
  const int64_t fqk = FQK > 0 ? FQK : fqk_rt;
  const int64_t fv = FV > 0 ? FV : fv_rt;
  const int lane = lane_id();
  const int gk = lane / GK;
  const int kl = lane % GK;
  const int gv = lane / GV;
  const int vl = lane % GV;
  const char* __restrict__ kb = reinterpret_cast<const char*>(key);
  const char* __restrict__ vb = reinterpret_cast<const char*>(value);
  // lanes past the feature end read feature 0 (their q is 0 / their output
  // is not stored)
  const uint32_t kbytes = static_cast<uint32_t>((P * kl < fqk ? P * kl : 0) * sizeof(T));
  const uint32_t vbytes = static_cast<uint32_t>((P * vl < fv ? P * vl : 0) * sizeof(T));
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  m = -INFINITY;
  l = 0.f;
#pragma unroll
  for (int v = 0; v < P; ++v) acc[v] = 0.f;
  int next_col = 0;
  if (lane < re - rs) next_col = static_cast<int>(col[rs + lane]);
  for (int64_t base = rs; base < re; base += kWave) {
    const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
    const int my_col = next_col;
    const int64_t nb = base + kWave;
    if (nb < re && lane < re - nb) next_col = static_cast<int>(col[nb + lane]);
    for (int j = 0; j < cnt; j += E) {
      RawVec<16> kv[E / EK];
      RawVec<16> vv[E / EV];
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        int c = 0;
#pragma unroll
        for (int g = 0; g < EK; ++g) {
          const int e = j + i * EK + g;
          const int cg = bcast_i32(my_col, e < cnt ? e : cnt - 1);
          c = gk == g ? cg : c;
        }
        kv[i] = load_raw<16>(kb + row_offset(c, fqk) * sizeof(T) + kbytes);
      }
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        int c = 0;
#pragma unroll
        for (int g = 0; g < EV; ++g) {
          const int e = j + i * EV + g;
          const int cg = bcast_i32(my_col, e < cnt ? e : cnt - 1);
          c = gv == g ? cg : c;
        }
        vv[i] = load_raw<16>(vb + row_offset(c, fv) * sizeof(T) + vbytes);
      }
      // scores: K instruction i, group g holds edge j + i·EK + g
      float sk[E / EK];
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        float k[P];
        lane_values<T>(kv[i], k);
        float d = q[0] * k[0];
#pragma unroll
        for (int v = 1; v < P; ++v) d = __builtin_fmaf(q[v], k[v], d);
#pragma unroll
        for (int o = GK / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
        sk[i] = d * scale;
      }
      float s[E / EV];
      float mb = -INFINITY;
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        float si = 0.f;
#pragma unroll
        for (int g = 0; g < EV; ++g) {
          const int e = i * EV + g;  // edge of the batch
          const float se = bcast_f32(sk[e / EK], GK * (e % EK));
          si = gv == g ? se : si;
        }
        s[i] = j + i * EV + gv < cnt ? si : -INFINITY;
        mb = fmaxf(mb, s[i]);
      }
      const float mn = fmaxf(m, mb);
      if (mn != -INFINITY) {
        const float corr = m == -INFINITY ? 0.f : expf(m - mn);
        l *= corr;
#pragma unroll
        for (int v = 0; v < P; ++v) acc[v] *= corr;
#pragma unroll
        for (int i = 0; i < E / EV; ++i) {
          const float p = s[i] == -INFINITY ? 0.f : expf(s[i] - mn);
          l += p;
          float x[P];
          lane_values<T>(vv[i], x);
#pragma unroll
          for (int v = 0; v < P; ++v) acc[v] = __builtin_fmaf(p, x[v], acc[v]);
        }
        m = mn;
      }
    }
  }
#pragma unroll
  for (int o = GV; o < kWave; o <<= 1) {
    const float mo = __shfl_xor(m, o, kWave);
    const float lo = __shfl_xor(l, o, kWave);
    float ao[P];
#pragma unroll
    for (int v = 0; v < P; ++v) ao[v] = __shfl_xor(acc[v], o, kWave);
    merge_softmax<P>(m, l, acc, mo, lo, ao);
  }
}

template <typename T>
struct AttArgs {
  const int64_t* crow;
  const int64_t* col;
  const T* q;
  const T* k;
  const T* v;
  T* out;
  int64_t n;
  int64_t fqk;
  int64_t fv;
  float scale;
  const int32_t* order;
  const int32_t* counts;
  const int32_t* off;
};

// Short rows several to a wavefront: the wave is cut into segments of
// L = GV lanes, one row each (64 / L rows per wave), so that a wave keeps
// several rows' dependent chains (row order, row bounds, column block,
// gathers) in flight instead of one.  Inside a segment, sub-groups of GK
// lanes (GK <= GV) gather K rows, L / GK edges per instruction, and the whole
// segment gathers one V row per instruction.  Each segment runs its own online
// softmax over E edges per step; the column indices of a block of L edges are
// loaded one per lane and handed out by ds_bpermute.  Lanes past a row's end
// gather row 0 (valid) and get score -inf.
#ifndef AS_ATT_GROUPED_BATCH
#define AS_ATT_GROUPED_BATCH 4
#endif
constexpr int kGroupedBatch = AS_ATT_GROUPED_BATCH;  // edges per online-softmax step per row

template <typename T, int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void attend_rows_grouped(const AttArgs<T>& a, int64_t item0, int64_t end) {
  constexpr int P = lane_elems<T>();
  constexpr int L = GV;
  constexpr int EKS = L / GK;  // K edges per instruction per row
  constexpr int E = kGroupedBatch;
  static_assert(GK <= GV && GV <= 16 && L % E == 0 && E % EKS == 0, "grouped rows need GK <= GV <= 16");
  const int64_t fqk = FQK > 0 ? FQK : a.fqk;
  const int64_t fv = FV > 0 ? FV : a.fv;
  const int lane = lane_id();
  const int seg = lane / L;
  const int sl = lane % L;
  const int kg = sl / GK;
  const int kl = sl % GK;
  const int64_t item = item0 + seg;
  int64_t row = -1;
  int64_t rs = 0;
  int deg = 0;  // below the slicing degree
  if (item < end) {
    row = a.order[item];
    rs = a.crow[row];
    deg = static_cast<int>(a.crow[row + 1] - rs);
  }
  int maxdeg = deg;
#pragma unroll
  for (int o = L; o < kWave; o <<= 1) maxdeg = max(maxdeg, __shfl_xor(maxdeg, o, kWave));
  maxdeg = uniform_i32(maxdeg);
  float q[P];
  if (row >= 0 && P * kl < fqk) {
    lane_values<T>(load_raw<16>(reinterpret_cast<const char*>(a.q + row * fqk + P * kl)), q);
  } else {
#pragma unroll
    for (int v = 0; v < P; ++v) q[v] = 0.f;
  }
  const char* __restrict__ kb = reinterpret_cast<const char*>(a.k);
  const char* __restrict__ vb = reinterpret_cast<const char*>(a.v);
  const uint32_t kbytes = static_cast<uint32_t>((P * kl < fqk ? P * kl : 0) * sizeof(T));
  const uint32_t vbytes = static_cast<uint32_t>((P * sl < fv ? P * sl : 0) * sizeof(T));
  float m = -INFINITY;
  float l = 0.f;
  float acc[P];
#pragma unroll
  for (int v = 0; v < P; ++v) acc[v] = 0.f;
  for (int base = 0; base < maxdeg; base += L) {
    int my_col = 0;
    if (base + sl < deg) my_col = static_cast<int>(a.col[rs + base + sl]);
    const int cnt = deg - base;  // edges of this segment's row in the block (may be <= 0)
    const int lim = maxdeg - base < L ? maxdeg - base : L;
    for (int j = 0; j < lim; j += E) {
      RawVec<16> kv[E / EKS];
      RawVec<16> vv[E];
#pragma unroll
      for (int i = 0; i < E / EKS; ++i) {
        const int c = __builtin_amdgcn_ds_bpermute((seg * L + j + i * EKS + kg) * 4, my_col);
        kv[i] = load_raw<16>(kb + row_offset(c, fqk) * sizeof(T) + kbytes);
      }
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int c = __builtin_amdgcn_ds_bpermute((seg * L + j + i) * 4, my_col);
        vv[i] = load_raw<16>(vb + row_offset(c, fv) * sizeof(T) + vbytes);
      }
      float sk[E / EKS];
#pragma unroll
      for (int i = 0; i < E / EKS; ++i) {
        float k[P];
        lane_values<T>(kv[i], k);
        float d = q[0] * k[0];
#pragma unroll
        for (int v = 1; v < P; ++v) d = __builtin_fmaf(q[v], k[v], d);
#pragma unroll
        for (int o = GK / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
        sk[i] = d * a.scale;
      }
      float s[E];
      float mb = -INFINITY;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        // edge j + i sits in K instruction i / EKS, sub-group i % EKS
        const float se = __shfl(sk[i / EKS], seg * L + (i % EKS) * GK, kWave);
        s[i] = j + i < cnt ? se : -INFINITY;
        mb = fmaxf(mb, s[i]);
      }
      const float mn = fmaxf(m, mb);
      if (mn != -INFINITY) {
        const float corr = m == -INFINITY ? 0.f : expf(m - mn);
        l *= corr;
#pragma unroll
        for (int v = 0; v < P; ++v) acc[v] *= corr;
#pragma unroll
        for (int i = 0; i < E; ++i) {
          const float p = s[i] == -INFINITY ? 0.f : expf(s[i] - mn);
          l += p;
          float x[P];
          lane_values<T>(vv[i], x);
#pragma unroll
          for (int v = 0; v < P; ++v) acc[v] = __builtin_fmaf(p, x[v], acc[v]);
        }
        m = mn;
      }
    }
  }
  if (row >= 0 && P * sl < fv) {
    float o[P];
#pragma unroll
    for (int v = 0; v < P; ++v) o[v] = l > 0.f ? acc[v] / l : 0.f;
    store_out<T, P>(a.out + row * fv + P * sl, o);
  }
}

// Rows of 16-bit elements with GK <= GV <= 16 (at least 4 rows per wave) run
// grouped; other element types and widths one row per wave.
template <typename T, int GK, int GV>
constexpr bool grouped_rows() {
  return sizeof(T) == 2 && GK <= GV && GV <= 16;
}

// Short rows order[H, n), H = counts[0] (known on the device only): a
// grid-stride over them, 64 / GV rows per wave when grouped_rows, else one.
// On the benchmark attention in bf16 (2.4M rows, median degree 16) grouping
// every short row takes the call from 8.04 to 6.42 ms; grouping only rows
// below 64, 32 or 16 edges (the rest one per wave, in the same kernel) gave
// 6.82, 7.05 and 7.67 ms, 2 or 8 edges per step 6.70 / 7.43 ms, and capping
// the grouped kernel at 80 / 72 / 64 VGPRs (6 / 7 / 8 waves per SIMD, the last
// two spilling) 6.44 / 6.68 / 7.01 ms.
template <typename T, int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void att_rows_kernel(AttArgs<T> a) {
  constexpr int P = lane_elems<T>();
  const int64_t first = a.counts[0];
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
  if constexpr (grouped_rows<T, GK, GV>()) {
    constexpr int64_t kRows = kWave / GV;
    for (int64_t item0 = first + w * kRows; item0 < a.n; item0 += waves * kRows) {
      attend_rows_grouped<T, GK, GV, FQK, FV>(a, item0, a.n);
    }
    return;
  }
  for (int64_t item = first + w; item < a.n; item += waves) {
    const int64_t row = uniform_i64(a.order[item]);
    float q[P];
    load_query_lanes<T, GK>(a.q, row, a.fqk, q);
    float m, l, acc[P];
    attend_edges<T, GK, GV, FQK, FV>(a.col, a.k, a.v, a.fqk, a.fv, q, a.scale, a.crow[row], a.crow[row + 1], m, l,
                                     acc);
    const int lane = lane_id();
    if (lane < GV && P * lane < a.fv) {
      float o[P];
#pragma unroll
      for (int v = 0; v < P; ++v) o[v] = l > 0.f ? acc[v] / l : 0.f;
      store_out<T, P>(a.out + row * a.fv + P * lane, o);
    }
  }
}

// Sliced rows order[begin, begin + items) (those below H): wave per
// (row, slice) writes the partial state at index slice·stride + local.  The
// host knows only an upper bound on H, so a chunk may be empty: the grid is
// capped and the waves of a slice stride over the chunk, which keeps the
// launch of an empty chunk short.
template <typename T, int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void att_slice_kernel(AttArgs<T> a, int64_t begin, int64_t items,
                                                           int64_t stride, float* __restrict__ pm,
                                                           float* __restrict__ pl, float* __restrict__ pacc) {
  constexpr int P = lane_elems<T>();
  const int slice = static_cast<int>(blockIdx.x % kSlices);
  const int64_t waves = static_cast<int64_t>(gridDim.x / kSlices) * kWavesPerBlock;
  int64_t end = a.counts[0] - begin;
  end = end < items ? end : items;
  const int lane = lane_id();
  for (int64_t local = static_cast<int64_t>(blockIdx.x / kSlices) * kWavesPerBlock + wave_in_block(); local < end;
       local += waves) {
    const int64_t row = uniform_i64(a.order[begin + local]);
    const int64_t rs = uniform_i64(a.crow[row]);
    const int64_t deg = uniform_i64(a.crow[row + 1]) - rs;
    int64_t lo, hi;
    slice_range(a.off, row, slice, deg, lo, hi);
    lo = uniform_i64(lo);
    hi = uniform_i64(hi);
    float q[P];
    load_query_lanes<T, GK>(a.q, row, a.fqk, q);
    float m, l, acc[P];
    attend_edges<T, GK, GV, FQK, FV>(a.col, a.k, a.v, a.fqk, a.fv, q, a.scale, rs + lo, rs + hi, m, l, acc);
    const int64_t at = slice * stride + local;
    if (lane < GV && P * lane < a.fv) {
#pragma unroll
      for (int i = 0; i < P; i += 4) {
        FVec<4> o;
#pragma unroll
        for (int v = 0; v < 4; ++v) o.v[v] = acc[i + v];
        store_vec<4>(pacc + at * a.fv + P * lane + i, o);
      }
    }
    if (lane == 0) {
      pm[at] = m;
      pl[at] = l;
    }
  }
}

// Merge of the 8 partial states of each sliced row of the chunk; thread per
// (row, 4 features).
template <typename T>
__global__ __launch_bounds__(kBlock) void att_reduce_kernel(AttArgs<T> a, int64_t begin, int64_t items,
                                                            int64_t stride, const float* __restrict__ pm,
                                                            const float* __restrict__ pl,
                                                            const float* __restrict__ pacc) {
  const int64_t F4 = a.fv / 4;
  const int64_t total = items * F4;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += step) {
    const int64_t local = t / F4;
    const int64_t f = (t - local * F4) * 4;
    if (begin + local >= a.counts[0]) continue;
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < kSlices; ++s) m = fmaxf(m, pm[s * stride + local]);
    float l = 0.f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (m != -INFINITY) {
#pragma unroll
      for (int s = 0; s < kSlices; ++s) {
        const float ms = pm[s * stride + local];
        if (ms == -INFINITY) continue;
        const float c = expf(ms - m);
        l = __builtin_fmaf(c, pl[s * stride + local], l);
        const FVec<4> p = load_vec<4>(pacc + (s * stride + local) * a.fv + f);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(c, p.v[v], acc[v]);
      }
    }
    const int64_t row = a.order[begin + local];
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) o[v] = l > 0.f ? acc[v] / l : 0.f;
    store_out<T, 4>(a.out + row * a.fv + f, o);
  }
}


template <typename T, int GK, int GV, int FQK = 0, int FV = 0>
void launch_attention_t(const AttArgs<T>& a, int64_t upper, int64_t chunk, float* pm, float* pl, float* pacc,
                        hipStream_t s) {
  // short rows: a grid-stride over order[H, n), sized for all n rows
  const int64_t rows_per_wave = grouped_rows<T, GK, GV>() ? kWave / GV : 1;
  int64_t row_blocks = (a.n + kWavesPerBlock * rows_per_wave - 1) / (kWavesPerBlock * rows_per_wave);
  if (row_blocks > kMaxBlocksPerLaunch) row_blocks = kMaxBlocksPerLaunch;
  hipLaunchKernelGGL((att_rows_kernel<T, GK, GV, FQK, FV>), dim3(static_cast<unsigned>(row_blocks)), dim3(kBlock),
                     0, s, a);
  for (int64_t begin = 0; begin < upper; begin += chunk) {
    const int64_t items = upper - begin < chunk ? upper - begin : chunk;
    int64_t per_slice = (items + kWavesPerBlock - 1) / kWavesPerBlock;
    if (per_slice > kAttSliceBlocks) per_slice = kAttSliceBlocks;
    hipLaunchKernelGGL((att_slice_kernel<T, GK, GV, FQK, FV>), dim3(static_cast<unsigned>(kSlices * per_slice)),
                       dim3(kBlock), 0, s, a, begin, items, chunk, pm, pl, pacc);
    int64_t blocks = (items * (a.fv / 4) + kBlock - 1) / kBlock;
    if (blocks > kAttReduceBlocks) blocks = kAttReduceBlocks;
    hipLaunchKernelGGL((att_reduce_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, a, begin,
                       items, chunk, pm, pl, pacc);
  }
}

template <typename T, int GK>
void launch_attention_k(int gv, const AttArgs<T>& a, int64_t upper, int64_t chunk, float* pm, float* pl,
                        float* pacc, hipStream_t s) {
  switch (gv) {
    case 8:
      if constexpr (sizeof(T) == 2) launch_attention_t<T, GK, 8>(a, upper, chunk, pm, pl, pacc, s);
      break;
    case 16: launch_attention_t<T, GK, 16>(a, upper, chunk, pm, pl, pacc, s); break;
    case 32: launch_attention_t<T, GK, 32>(a, upper, chunk, pm, pl, pacc, s); break;
    default: launch_attention_t<T, GK, 64>(a, upper, chunk, pm, pl, pacc, s); break;
  }
}

size_t att_fixed_bytes(int64_t n) { return slice_plan_bytes(n); }

// The plan settings of the attention on element type T: rows of degree >=
// att_slice_degree<T>() are sliced; short rows in 8 log2-degree buckets for 16-bit elements (the
// grouped rows), in one for fp32.
template <typename T>
constexpr int att_light_buckets() {
  return sizeof(T) == 2 ? kMaxHeavyBuckets : 1;
}

// Per sliced row of a chunk: 8 x (m, l, F_v accumulators), fp32.
size_t att_row_bytes(int64_t fv) { return static_cast<size_t>(kSlices) * (static_cast<size_t>(fv) + 2) * sizeof(float); }

// Upper bound on the rows of degree >= `degree` (the sliced rows).
int64_t att_sliced_upper(int64_t n, int64_t nnz, int64_t degree) {
  const int64_t u = nnz / degree;
  return u < n ? u : n;
}

// Both entry points after their element-specific checks: carves the
// workspace, computes the slice points and the row order, launches.
template <typename T>
int attention_run(const int64_t* crow, const int64_t* col, const T* query, const T* key, const T* value, T* out,
                  int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v, float scale, const void* plan, int64_t plan_tag,
                  void* workspace, size_t workspace_bytes, void* stream, const char* what) {
  constexpr int64_t kDegree = att_slice_degree<T>();
  if (plan != nullptr && plan_tag != slice_plan_tag(kDegree, att_light_buckets<T>()))
    return fail(AS_ERR_INVALID_ARGUMENT, "the plan was built for other settings (plan tag %lld, this call needs %lld)",
                (long long)plan_tag, (long long)slice_plan_tag(kDegree, att_light_buckets<T>()));
  if (plan != nullptr && !aligned(plan, 256)) return fail(AS_ERR_WORKSPACE, "the plan must be 256-byte aligned");
  if (n == 0) return AS_OK;
  if (crow == nullptr || query == nullptr || key == nullptr || value == nullptr || out == nullptr ||
      (nnz > 0 && col == nullptr))
    return fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (!aligned(query, 16) || !aligned(key, 16) || !aligned(value, 16) || !aligned(out, 16))
    return fail(AS_ERR_UNSUPPORTED, "column-sliced attention needs 16-byte aligned Q, K, V and out");
  // with a plan the workspace holds the partial states only
  const size_t fixed = plan != nullptr ? 0 : att_fixed_bytes(n);
  const size_t row_bytes = att_row_bytes(f_v);
  if (workspace == nullptr || workspace_bytes < fixed + row_bytes + 3 * 256)
    return fail(AS_ERR_WORKSPACE, "column-sliced attention needs at least %zu workspace bytes, got %zu",
                fixed + row_bytes + 3 * 256, workspace_bytes);
  if (!aligned(workspace, 256)) return fail(AS_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  const int64_t upper = att_sliced_upper(n, nnz, kDegree);
  int64_t chunk = static_cast<int64_t>((workspace_bytes - fixed - 3 * 256) / row_bytes);
  if (chunk > kAttChunkRows) chunk = kAttChunkRows;
  if (chunk > upper) chunk = upper;
  if (chunk < 1) chunk = 1;

  const hipStream_t s = static_cast<hipStream_t>(stream);
  const SlicePlan view = slice_plan_view(plan != nullptr ? const_cast<void*>(plan) : workspace, n);
  char* ws = static_cast<char*>(workspace) + fixed;
  const size_t states = static_cast<size_t>(kSlices) * static_cast<size_t>(chunk);
  float* pm = reinterpret_cast<float*>(ws);
  ws += align_up(states * sizeof(float), 256);
  float* pl = reinterpret_cast<float*>(ws);
  ws += align_up(states * sizeof(float), 256);
  float* pacc = reinterpret_cast<float*>(ws);

  // order: rows of degree >= D = kDegree (sliced) longest first, then the
  // others; for 16-bit elements in 8 log2-degree buckets, longest first (light
  // bucket b holds degrees [D / 2^(b+1), D / 2^b), the last one the empty rows)
  // (grouped rows take similar degrees together)
  constexpr bool kHalf = sizeof(T) == 2;
  if (plan == nullptr) {
    const int st = build_slice_plan(crow, col, n, kDegree, att_light_buckets<T>(), false, view, s);
    if (st != AS_OK) return st;
  }
  const AttArgs<T> a{crow, col, query, key, value, out, n, f_qk, f_v, scale, view.order, view.counts, view.off};
  // common widths with compile-time strides
  if (f_qk == 64 && f_v == 128) {
    launch_attention_t<T, kHalf ? 8 : 16, kHalf ? 16 : 32, 64, 128>(a, upper, chunk, pm, pl, pacc, s);
  } else if (f_qk == 64 && f_v == 64) {
    launch_attention_t<T, kHalf ? 8 : 16, kHalf ? 8 : 16, 64, 64>(a, upper, chunk, pm, pl, pacc, s);
  } else if (f_qk == 128 && f_v == 128) {
    launch_attention_t<T, kHalf ? 16 : 32, kHalf ? 16 : 32, 128, 128>(a, upper, chunk, pm, pl, pacc, s);
  } else {
    const int gv = lane_group<T>(f_v);
    switch (lane_group<T>(f_qk)) {
      case 8:
        if constexpr (kHalf) launch_attention_k<T, 8>(gv, a, upper, chunk, pm, pl, pacc, s);
        break;
      case 16: launch_attention_k<T, 16>(gv, a, upper, chunk, pm, pl, pacc, s); break;
      case 32: launch_attention_k<T, 32>(gv, a, upper, chunk, pm, pl, pacc, s); break;
      default: launch_attention_k<T, 64>(gv, a, upper, chunk, pm, pl, pacc, s); break;
    }
  }
  return check_launch(what);
}

}  // namespace

}  // namespace as

extern "C" {

size_t as_csr_attention_colslice_workspace_bytes(int64_t n, int64_t nnz, int64_t f_v) {
  if (n < 0) n = 0;
  if (nnz < 0) nnz = 0;
  if (f_v < 4) f_v = 4;
  // the fp32 slicing degree, the lowest: enough for every element type
  int64_t rows = as::att_sliced_upper(n, nnz, as::att_slice_degree<float>());
  if (rows > as::kAttChunkRows) rows = as::kAttChunkRows;
  if (rows < 1) rows = 1;
  // + 256 bytes per partial array for alignment
  return as::att_fixed_bytes(n) + static_cast<size_t>(rows) * as::att_row_bytes(f_v) + 3 * 256;
}

size_t as_csr_attention_plan_bytes(int64_t n) { return as::slice_plan_bytes(n); }

int as_csr_attention_plan_rect(const int64_t* crow, const int64_t* col, int64_t n, int64_t n_cols, int64_t nnz,
                               int dtype, void* plan, size_t plan_bytes, int64_t* plan_tag, void* stream) {
  as::clear_error();
  if (n_cols < 0 || n_cols > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "n_cols exceeds kernel index range");
  if (dtype != AS_DTYPE_F32 && dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_F32, AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (plan_tag == nullptr) return as::fail(AS_ERR_INVALID_ARGUMENT, "plan_tag must not be NULL");
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (n > 0 && (crow == nullptr || (nnz > 0 && col == nullptr)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "crow and col must not be NULL");
  if (plan == nullptr || plan_bytes < as::slice_plan_bytes(n))
    return as::fail(AS_ERR_WORKSPACE, "an attention plan needs %zu bytes, got %zu", as::slice_plan_bytes(n),
                    plan_bytes);
  if (!as::aligned(plan, 256)) return as::fail(AS_ERR_WORKSPACE, "the plan must be 256-byte aligned");
  const bool f32 = dtype == AS_DTYPE_F32;
  const int light = f32 ? as::att_light_buckets<float>() : as::att_light_buckets<as::Bf16>();
  const int64_t degree = f32 ? as::att_slice_degree<float>() : as::att_slice_degree<as::Bf16>();
  *plan_tag = as::slice_plan_tag(degree, light);
  if (n == 0) return AS_OK;
  const int st = as::build_slice_plan(crow, col, n, degree, light, false, as::slice_plan_view(plan, n),
                                      static_cast<hipStream_t>(stream), n_cols);
  if (st != AS_OK) return st;
  return as::check_launch("csr_attention_plan");
}

int as_csr_attention_plan(const int64_t* crow, const int64_t* col, int64_t n, int64_t nnz, int dtype, void* plan,
                          size_t plan_bytes, int64_t* plan_tag, void* stream) {
  return as_csr_attention_plan_rect(crow, col, n, n < 0 ? 0 : n, nnz, dtype, plan, plan_bytes, plan_tag, stream);
}

int as_csr_attention_colslice_f32(const int64_t* crow, const int64_t* col, const float* query, const float* key,
                                  const float* value, float* out, int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v,
                                  float scale, const void* plan, int64_t plan_tag, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (f_qk < 4 || f_qk > 256 || f_qk % 4 != 0 || f_v < 4 || f_v > 256 || f_v % 4 != 0)
    return as::fail(AS_ERR_UNSUPPORTED, "column-sliced attention needs F_qk and F_v in [4, 256], multiples of 4");
  return as::attention_run<float>(crow, col, query, key, value, out, n, nnz, f_qk, f_v, scale, plan, plan_tag,
                                  workspace, workspace_bytes, stream, "csr_attention_colslice");
}

int as_csr_attention_colslice_16(const int64_t* crow, const int64_t* col, const void* query, const void* key,
                                 const void* value, void* out, int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v,
                                 float scale, int dtype, const void* plan, int64_t plan_tag, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (f_qk < 8 || f_qk > 512 || f_qk % 8 != 0 || f_v < 8 || f_v > 512 || f_v % 8 != 0)
    return as::fail(AS_ERR_UNSUPPORTED, "16-bit attention needs F_qk and F_v in [8, 512], multiples of 8");
  if (dtype == AS_DTYPE_BF16)
    return as::attention_run<as::Bf16>(crow, col, static_cast<const as::Bf16*>(query),
                                       static_cast<const as::Bf16*>(key), static_cast<const as::Bf16*>(value),
                                       static_cast<as::Bf16*>(out), n, nnz, f_qk, f_v, scale, plan, plan_tag,
                                       workspace, workspace_bytes, stream, "csr_attention_colslice (bf16)");
  return as::attention_run<as::Fp16>(crow, col, static_cast<const as::Fp16*>(query), static_cast<const as::Fp16*>(key),
                                     static_cast<const as::Fp16*>(value), static_cast<as::Fp16*>(out), n, nnz, f_qk,
                                     f_v, scale, plan, plan_tag, workspace, workspace_bytes, stream,
                                     "csr_attention_colslice (fp16)");
}

}  // extern "C"
