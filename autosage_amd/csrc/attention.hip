// CSR row softmax and the fused SDDMM -> row softmax -> SpMM attention.
//
// Reference behaviour: _csr_row_softmax (autosage/_auto.py:744-759) and
// csr_attention_forward (autosage/_auto.py:762-780), which run as separate
// torch / native stages there.
//
// Row softmax, one wave per row (defines this library's denominator order):
//   m = max_e s_e                      (exact, order-free)
//   d = sum_e exp(s_e - m): lane l adds e = rs+l, rs+l+64, ... in order,
//       then a 32/16/8/4/2/1 butterfly (identical bits in every lane)
//   p_e = exp(s_e - m) / d             (IEEE division)
//
// The fused kernel computes, per row, the same scores as the SDDMM kernels
// (reference dot order) times `scale`, stores them in the workspace's
// nnz-float scratch, derives m and d exactly as above and then accumulates
// out[r, :] = sum_e p_e · V[col_e, :] in edge order with fmaf, as the SpMM
// kernels do.  With scale 1 (or a power of two) it is therefore
// bit-identical to the three unfused stages.  Rows of degree >= 1024 are
// binned (longest bucket first, as for the split SpMM) and each gets a
// workgroup whose waves share the scoring and split the value features.
#include <type_traits>

#include "as_device.h"
#include "as_internal.h"
#include "elem16.h"

namespace as {

namespace {

__global__ __launch_bounds__(kBlock) void csr_row_softmax_kernel(const int64_t* __restrict__ crow,
                                                                 const float* __restrict__ scores,
                                                                 float* __restrict__ probs, int64_t n,
                                                                 int64_t idx_base) {
  const int lane = lane_id();
  const int64_t row = idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  if (row >= n) return;
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);
  if (rs == re) return;
  float m = -INFINITY;
  for (int64_t e = rs + lane; e < re; e += kWave) m = fmaxf(m, scores[e]);
  m = wave_max_f32(m);
  float d = 0.f;
  for (int64_t e = rs + lane; e < re; e += kWave) d += expf(scores[e] - m);
  d = wave_sum_f32(d);
  for (int64_t e = rs + lane; e < re; e += kWave) probs[e] = expf(scores[e] - m) / d;
}

// The same row softmax on bf16 / fp16 scores: each score converts exactly to
// fp32, m, d and p_e are computed in fp32 and p_e is rounded to the 16-bit
// type (round to nearest even) once.  Rows of at most kSm16GroupDegree edges
// take a group of 16 lanes (4 rows per wave, csr_row_softmax16_grouped_kernel),
// longer rows a wave each with a running max and sum (csr_row_softmax16_kernel);
// the sums of d differ in order from the fp32 kernel's, which can move a
// result by one 16-bit unit near a tie.
constexpr int64_t kSm16GroupDegree = 64;
constexpr int kSm16Group = 16;

template <typename T>
__global__ __launch_bounds__(kBlock) void csr_row_softmax16_grouped_kernel(const int64_t* __restrict__ crow,
                                                                           const T* __restrict__ scores,
                                                                           uint16_t* __restrict__ probs, int64_t n,
                                                                           int64_t idx_base) {
  constexpr int kRowsPerWave = kWave / kSm16Group;
  const int lane = lane_id();
  const int g = lane / kSm16Group;
  const int gl = lane % kSm16Group;
  const int64_t row =
      (idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block()) * kRowsPerWave + g;
  int64_t rs = 0, re = 0;
  if (row < n) {
    rs = crow[row];
    re = crow[row + 1];
    if (re - rs > kSm16GroupDegree) re = rs;  // a whole wave takes it
  }
  // a lane holds its <= 4 scores: one read of the row, one exp per score
  constexpr int kPer = static_cast<int>(kSm16GroupDegree / kSm16Group);
  float v[kPer];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int64_t e = rs + gl + i * kSm16Group;
    v[i] = e < re ? Elem<T>::at(scores, e) : -INFINITY;
    m = fmaxf(m, v[i]);
  }
#pragma unroll
  for (int o = 1; o < kSm16Group; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int64_t e = rs + gl + i * kSm16Group;
    v[i] = e < re ? expf(v[i] - m) : 0.f;
    d += v[i];
  }
#pragma unroll
  for (int o = 1; o < kSm16Group; o <<= 1) d += __shfl_xor(d, o, kWave);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int64_t e = rs + gl + i * kSm16Group;
    if (e < re) probs[e] = Elem<T>::bits(static_cast<double>(v[i] / d));
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void csr_row_softmax16_kernel(const int64_t* __restrict__ crow,
                                                                   const T* __restrict__ scores,
                                                                   uint16_t* __restrict__ probs, int64_t n,
                                                                   int64_t idx_base) {
  const int lane = lane_id();
  const int64_t row = idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  if (row >= n) return;
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);
  if (re - rs <= kSm16GroupDegree) return;  // the grouped kernel takes it
  // one read for m and d: each lane keeps a running max and the sum of
  // exp(s - max), rescaled when the max grows; the lanes then merge
  float m = -INFINITY;
  float d = 0.f;
  for (int64_t e = rs + lane; e < re; e += kWave) {
    const float v = Elem<T>::at(scores, e);
    if (v > m) {
      d = d * expf(m - v) + 1.f;
      m = v;
    } else if (v != -INFINITY) {  // -inf adds nothing (and -inf - -inf is NaN)
      d += expf(v - m);
    }
  }
  const float mw = wave_max_f32(m);
  d = m == -INFINITY ? 0.f : d * expf(m - mw);
  d = wave_sum_f32(d);
  for (int64_t e = rs + lane; e < re; e += kWave)
    probs[e] = Elem<T>::bits(static_cast<double>(expf(Elem<T>::at(scores, e) - mw) / d));
}

// Backward of the row softmax: given p = softmax(s) and dp = dL/dp,
//   t = sum_e dp_e · p_e   (lane l: e = rs+l, rs+l+64, ... with fmaf, in
//                           order; then the 32/16/8/4/2/1 butterfly)
//   ds_e = p_e · (dp_e - t)
// in fp32 (16-bit inputs convert exactly; each ds_e is rounded once).
template <typename T>
__device__ __forceinline__ float sm_load(const T* __restrict__ p, int64_t e) {
  if constexpr (std::is_same<T, float>::value) return p[e];
  else return Elem<T>::at(p, e);
}
template <typename T>
__device__ __forceinline__ void sm_store(T* __restrict__ p, int64_t e, float v) {
  if constexpr (std::is_same<T, float>::value) p[e] = v;
  else p[e].bits = Elem<T>::bits(static_cast<double>(v));
}

template <typename T>
__global__ __launch_bounds__(kBlock) void csr_row_softmax_backward_kernel(const int64_t* __restrict__ crow,
                                                                          const T* __restrict__ probs,
                                                                          const T* __restrict__ grad,
                                                                          T* __restrict__ grad_scores, int64_t n,
                                                                          int64_t idx_base) {
  const int lane = lane_id();
  const int64_t row = idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  if (row >= n) return;
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);
  if (rs == re) return;
  float t = 0.f;
  for (int64_t e = rs + lane; e < re; e += kWave) t = __builtin_fmaf(sm_load(grad, e), sm_load(probs, e), t);
  t = wave_sum_f32(t);
  for (int64_t e = rs + lane; e < re; e += kWave) {
    const float p = sm_load(probs, e);
    sm_store(grad_scores, e, p * (sm_load(grad, e) - t));
  }
}

template <typename T>
int launch_softmax_backward(const int64_t* crow, const void* probs, const void* grad, void* grad_scores, int64_t n,
                            hipStream_t s) {
  const int64_t blocks = (n + kWavesPerBlock - 1) / kWavesPerBlock;
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    hipLaunchKernelGGL(csr_row_softmax_backward_kernel<T>, dim3(static_cast<unsigned>(nb)), dim3(kBlock), 0, s, crow,
                       static_cast<const T*>(probs), static_cast<const T*>(grad), static_cast<T*>(grad_scores), n,
                       b0 * kWavesPerBlock);
  }
  return check_launch("csr_row_softmax_backward");
}

template <int S>
__device__ __forceinline__ float ref_tree_a(float (&p)[S]) {
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

// Rows at least this long are hub rows of the fused kernel: a workgroup of
// kAttWaves waves takes each of them, longest degree bucket first.
#ifndef AS_ATT_HUB_DEGREE
#define AS_ATT_HUB_DEGREE 1024
#endif
constexpr int64_t kAttHubDegree = AS_ATT_HUB_DEGREE;
constexpr int kAttWaves = 4;
constexpr int kAttBuckets = 8;

// Pass A for one wave: scores of the edge groups starting at `first`,
// `first + step`, ... (each group = UE·NG consecutive edges) into scratch,
// returning this wave's running max over the edges it scored.
// QVEC: 8 lanes × float4 per 32 query/key features (MF blocks); otherwise
// 32 lanes per edge with scalar loads (any F_qk).
template <bool QVEC, int MF>
__device__ __forceinline__ float att_scores(const int64_t* __restrict__ col, const float* __restrict__ key,
                                            float* __restrict__ scratch, const float* __restrict__ qrow,
                                            int64_t Fqk, float scale, int64_t first, int64_t step, int64_t re) {
  constexpr int G = QVEC ? 8 : 32;
  constexpr int S = 32 / G;
  constexpr int NG = kWave / G;
  constexpr int UE = QVEC ? (MF <= 2 ? 4 : 2) : 1;
  const int lane = lane_id();
  const int g = lane / G;
  const int j = lane % G;
  float qv[QVEC ? MF : 1][S];
  if constexpr (QVEC) {
#pragma unroll
    for (int mm = 0; mm < MF; ++mm) {
      const FVec<S> t = load_vec<S>(qrow + 32 * mm + S * j);
#pragma unroll
      for (int s = 0; s < S; ++s) qv[mm][s] = t.v[s];
    }
  }
  float mloc = -INFINITY;
  for (int64_t base = first; base < re; base += step) {
    if constexpr (QVEC) {
      FVec<S> kv[UE][MF];
      bool ok[UE];
      int64_t e[UE];
#pragma unroll
      for (int u = 0; u < UE; ++u) {
        e[u] = base + u * NG + g;
        ok[u] = e[u] < re;
        const int64_t ee = ok[u] ? e[u] : re - 1;
        const int c = static_cast<int>(col[ee]);
        const float* kr = key + row_offset(c, Fqk) + S * j;
#pragma unroll
        for (int mm = 0; mm < MF; ++mm) kv[u][mm] = load_vec<S>(kr + 32 * mm);
      }
#pragma unroll
      for (int u = 0; u < UE; ++u) {
        float p[S];
#pragma unroll
        for (int s = 0; s < S; ++s) p[s] = 0.f;
#pragma unroll
        for (int mm = 0; mm < MF; ++mm) {
#pragma unroll
          for (int s = 0; s < S; ++s) p[s] = __builtin_fmaf(qv[mm][s], kv[u][mm].v[s], p[s]);
        }
        const float sc = ref_tree_a<S>(p) * scale;
        if (ok[u]) {
          mloc = fmaxf(mloc, sc);
          if (j == 0) scratch[e[u]] = sc;
        }
      }
    } else {
      const int64_t e = base + g;
      const bool ok = e < re;
      const int64_t ee = ok ? e : re - 1;
      const int c = static_cast<int>(col[ee]);
      const float* kr = key + row_offset(c, Fqk);
      float p[1] = {0.f};
      for (int64_t f = j; f < Fqk; f += 32) p[0] = __builtin_fmaf(qrow[f], kr[f], p[0]);
      const float sc = ref_tree_a<1>(p) * scale;
      if (ok) {
        mloc = fmaxf(mloc, sc);
        if (j == 0) scratch[e] = sc;
      }
    }
  }
  return mloc;
}

template <bool QVEC, int MF>
constexpr int64_t att_group_edges() {
  return QVEC ? (kWave / 8) * (MF <= 2 ? 4 : 2) : 2;
}

// Pass B: the row softmax denominator in the canonical order.
__device__ __forceinline__ float att_denominator(const float* __restrict__ scratch, float m, int64_t rs, int64_t re) {
  float d = 0.f;
  for (int64_t e = rs + lane_id(); e < re; e += kWave) d += expf(scratch[e] - m);
  return wave_sum_f32(d);
}

// Pass C for one wave: out[row, fbeg:fend) = sum_e p_e · V[col_e, fbeg:fend)
// in edge order (wave-row SpMM layout: unchecked full batches of U edges,
// then the remainder; lanes past fend load a valid address and store
// nothing).  VV | (fend - fbeg).
template <int VV>
__device__ __forceinline__ void att_accumulate(const int64_t* __restrict__ col, const float* __restrict__ value,
                                               const float* __restrict__ scratch, float* __restrict__ out,
                                               int64_t Fv, int64_t row, int64_t rs, int64_t re, float m, float d,
                                               int64_t fbeg, int64_t fend) {
  constexpr int U = 8;
  const int lane = lane_id();
  for (int64_t f0 = fbeg; f0 < fend; f0 += kWave * VV) {
    const int64_t fl = f0 + static_cast<int64_t>(lane) * VV;
    const bool active = fl < fend;
    const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : fbeg) * 4);
    float acc[VV];
#pragma unroll
    for (int v = 0; v < VV; ++v) acc[v] = 0.f;
    for (int64_t base = rs; base < re; base += kWave) {
      const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
      int my_col = 0;
      float my_p = 0.f;
      if (lane < cnt) {
        my_col = static_cast<int>(col[base + lane]);
        my_p = expf(scratch[base + lane] - m) / d;
      }
      int jj = 0;
      for (; jj + U <= cnt; jj += U) {
        FVec<VV> xv[U];
        float w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = bcast_i32(my_col, jj + u);
          w[u] = bcast_f32(my_p, jj + u);
          xv[u] = load_vec_off<VV>(value + row_offset(c, Fv), lane_bytes);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
          for (int v = 0; v < VV; ++v) acc[v] = __builtin_fmaf(w[u], xv[u].v[v], acc[v]);
        }
      }
      for (; jj < cnt; ++jj) {
        const int c = bcast_i32(my_col, jj);
        const float w = bcast_f32(my_p, jj);
        const FVec<VV> xv = load_vec_off<VV>(value + row_offset(c, Fv), lane_bytes);
#pragma unroll
        for (int v = 0; v < VV; ++v) acc[v] = __builtin_fmaf(w, xv.v[v], acc[v]);
      }
    }
    if (active) {
      FVec<VV> o;
#pragma unroll
      for (int v = 0; v < VV; ++v) o.v[v] = acc[v];
      store_vec<VV>(out + row * Fv + fl, o);
    }
  }
}

// Fused attention.  Workgroups of kAttWaves waves; work item = workgroup
// index.  Items [0, H): hub row order[item] — the waves split the row's
// edges for the scores, combine their maxima in LDS, each computes the
// denominator in the canonical order, and they split the value features
// for the weighted sum.  Items >= H: groups of kAttWaves light rows, one per
// wave, all passes on that wave.  Both give the same bits as the unfused
// SDDMM -> softmax -> SpMM stages.
template <bool QVEC, int MF, int VV, int HV>
__global__ __launch_bounds__(kAttWaves * kWave) void csr_attention_kernel(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const float* __restrict__ query,
    const float* __restrict__ key, const float* __restrict__ value, float* __restrict__ out,
    float* __restrict__ scratch, int64_t n, int64_t Fqk, int64_t Fv, float scale,
    const int32_t* __restrict__ order, const int32_t* __restrict__ counts, int64_t item_base) {
  __shared__ float wave_max[kAttWaves];
  constexpr int64_t GE = att_group_edges<QVEC, MF>();
  const int wave = wave_in_block();
  const int64_t item = item_base + blockIdx.x;
  const int64_t heavy = counts[0];
  if (item < heavy) {
    const int64_t row = uniform_i64(order[item]);
    const int64_t rs = uniform_i64(crow[row]);
    const int64_t re = uniform_i64(crow[row + 1]);
    const float mw = att_scores<QVEC, MF>(col, key, scratch, query + row * Fqk, Fqk, scale, rs + wave * GE,
                                          kAttWaves * GE, re);
    const float mwave = wave_max_f32(mw);
    if (lane_id() == 0) wave_max[wave] = mwave;
    __threadfence_block();
    __syncthreads();
    float m = wave_max[0];
#pragma unroll
    for (int w = 1; w < kAttWaves; ++w) m = fmaxf(m, wave_max[w]);
    const float d = att_denominator(scratch, m, rs, re);
    int64_t slice = (Fv + kAttWaves - 1) / kAttWaves;
    slice = (slice + HV - 1) / HV * HV;
    const int64_t fbeg = wave * slice;
    const int64_t fend = fbeg + slice < Fv ? fbeg + slice : Fv;
    if (fbeg < Fv) att_accumulate<HV>(col, value, scratch, out, Fv, row, rs, re, m, d, fbeg, fend);
    return;
  }
  const int64_t light_index = (item - heavy) * kAttWaves + wave;
  if (light_index >= n - heavy) return;
  const int64_t row = uniform_i64(order[heavy + light_index]);
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);
  float m = -INFINITY;
  float d = 0.f;
  if (rs < re) {
    m = wave_max_f32(att_scores<QVEC, MF>(col, key, scratch, query + row * Fqk, Fqk, scale, rs, GE, re));
    // The scratch scores were written by other lanes of this wave.
    __threadfence_block();
    d = att_denominator(scratch, m, rs, re);
  }
  att_accumulate<VV>(col, value, scratch, out, Fv, row, rs, re, m, d, 0, Fv);
}

bool al(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

struct AttArgs {
  const int64_t* crow;
  const int64_t* col;
  const float* q;
  const float* k;
  const float* v;
  float* out;
  float* scratch;
  int64_t n;
  int64_t fqk;
  int64_t fv;
  float scale;
  const int32_t* order;
  const int32_t* counts;
};

template <bool QVEC, int MF, int VV, int HV>
void launch_att_t(const AttArgs& a, int64_t blocks, hipStream_t s) {
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < kMaxBlocksPerLaunch ? blocks - b0 : kMaxBlocksPerLaunch;
    hipLaunchKernelGGL((csr_attention_kernel<QVEC, MF, VV, HV>), dim3(static_cast<unsigned>(nb)),
                       dim3(kAttWaves * kWave), 0, s, a.crow, a.col, a.q, a.k, a.v, a.out, a.scratch, a.n, a.fqk,
                       a.fv, a.scale, a.order, a.counts, b0);
  }
}

template <bool QVEC, int MF>
void launch_att_vv(int vv, int hv, const AttArgs& a, int64_t blocks, hipStream_t s) {
  if (vv == 4) {
    if (hv == 4) launch_att_t<QVEC, MF, 4, 4>(a, blocks, s);
    else if (hv == 2) launch_att_t<QVEC, MF, 4, 2>(a, blocks, s);
    else launch_att_t<QVEC, MF, 4, 1>(a, blocks, s);
  } else if (vv == 2) {
    if (hv == 2) launch_att_t<QVEC, MF, 2, 2>(a, blocks, s);
    else launch_att_t<QVEC, MF, 2, 1>(a, blocks, s);
  } else {
    launch_att_t<QVEC, MF, 1, 1>(a, blocks, s);
  }
}

// Lane vector width for `width` value features per wave.
int value_vector(const float* v, const float* out, int64_t fv, int64_t width) {
  if (fv % 4 == 0 && width > 128 && al(v, 16) && al(out, 16)) return 4;
  if (fv % 2 == 0 && width > 64 && al(v, 8) && al(out, 8)) return 2;
  return 1;
}

size_t attention_workspace(int64_t n, int64_t nnz) {
  const size_t scratch = align_up(static_cast<size_t>(nnz > 0 ? nnz : 1) * sizeof(float), 256);
  const size_t order = align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(int32_t), 256);
  return scratch + order + 256 + bin_workspace_bytes(n);
}

}  // namespace

}  // namespace as

extern "C" {

int as_csr_row_softmax_f32(const int64_t* crow, const float* scores, float* probs, int64_t n, int64_t nnz,
                           void* stream) {
  as::clear_error();
  if (n < 0 || n > INT32_MAX || nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "softmax sizes out of range");
  if (n == 0 || nnz == 0) return AS_OK;
  if (crow == nullptr || scores == nullptr || probs == nullptr)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t blocks = (n + as::kWavesPerBlock - 1) / as::kWavesPerBlock;
  for (int64_t b0 = 0; b0 < blocks; b0 += as::kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < as::kMaxBlocksPerLaunch ? blocks - b0 : as::kMaxBlocksPerLaunch;
    hipLaunchKernelGGL(as::csr_row_softmax_kernel, dim3(static_cast<unsigned>(nb)), dim3(as::kBlock), 0, s, crow,
                       scores, probs, n, b0 * as::kWavesPerBlock);
  }
  return as::check_launch("csr_row_softmax");
}

int as_csr_row_softmax_backward(const int64_t* crow, const void* probs, const void* grad, void* grad_scores,
                                int64_t n, int64_t nnz, int dtype, void* stream) {
  as::clear_error();
  if (dtype != AS_DTYPE_F32 && dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_F32, AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (n < 0 || n > INT32_MAX || nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "softmax sizes out of range");
  const size_t align = dtype == AS_DTYPE_F32 ? 4 : 2;
  if (!as::aligned(probs, align) || !as::aligned(grad, align) || !as::aligned(grad_scores, align))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "probs, grad and grad_scores must be aligned to their element size");
  if (n == 0 || nnz == 0) return AS_OK;
  if (crow == nullptr || probs == nullptr || grad == nullptr || grad_scores == nullptr)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == AS_DTYPE_F32) return as::launch_softmax_backward<float>(crow, probs, grad, grad_scores, n, s);
  if (dtype == AS_DTYPE_BF16) return as::launch_softmax_backward<as::Bf16>(crow, probs, grad, grad_scores, n, s);
  return as::launch_softmax_backward<as::Fp16>(crow, probs, grad, grad_scores, n, s);
}

int as_csr_row_softmax_16(const int64_t* crow, const void* scores, void* probs, int64_t n, int64_t nnz, int dtype,
                          void* stream) {
  as::clear_error();
  if (dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (n < 0 || n > INT32_MAX || nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "softmax sizes out of range");
  if (!as::aligned(scores, 2) || !as::aligned(probs, 2))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "scores and probs must be 2-byte aligned");
  if (n == 0 || nnz == 0) return AS_OK;
  if (crow == nullptr || scores == nullptr || probs == nullptr)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // short rows: 4 per wave
  const int64_t group_waves = (n + 3) / 4;
  const int64_t gblocks = (group_waves + as::kWavesPerBlock - 1) / as::kWavesPerBlock;
  for (int64_t b0 = 0; b0 < gblocks; b0 += as::kMaxBlocksPerLaunch) {
    const int64_t nb = gblocks - b0 < as::kMaxBlocksPerLaunch ? gblocks - b0 : as::kMaxBlocksPerLaunch;
    const dim3 grid(static_cast<unsigned>(nb));
    if (dtype == AS_DTYPE_BF16)
      hipLaunchKernelGGL(as::csr_row_softmax16_grouped_kernel<as::Bf16>, grid, dim3(as::kBlock), 0, s, crow,
                         static_cast<const as::Bf16*>(scores), static_cast<uint16_t*>(probs), n,
                         b0 * as::kWavesPerBlock);
    else
      hipLaunchKernelGGL(as::csr_row_softmax16_grouped_kernel<as::Fp16>, grid, dim3(as::kBlock), 0, s, crow,
                         static_cast<const as::Fp16*>(scores), static_cast<uint16_t*>(probs), n,
                         b0 * as::kWavesPerBlock);
  }
  // long rows: a wave each
  const int64_t blocks = (n + as::kWavesPerBlock - 1) / as::kWavesPerBlock;
  for (int64_t b0 = 0; b0 < blocks; b0 += as::kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < as::kMaxBlocksPerLaunch ? blocks - b0 : as::kMaxBlocksPerLaunch;
    const dim3 grid(static_cast<unsigned>(nb));
    if (dtype == AS_DTYPE_BF16)
      hipLaunchKernelGGL(as::csr_row_softmax16_kernel<as::Bf16>, grid, dim3(as::kBlock), 0, s, crow,
                         static_cast<const as::Bf16*>(scores), static_cast<uint16_t*>(probs), n,
                         b0 * as::kWavesPerBlock);
    else
      hipLaunchKernelGGL(as::csr_row_softmax16_kernel<as::Fp16>, grid, dim3(as::kBlock), 0, s, crow,
                         static_cast<const as::Fp16*>(scores), static_cast<uint16_t*>(probs), n,
                         b0 * as::kWavesPerBlock);
  }
  return as::check_launch("csr_row_softmax_16");
}

size_t as_csr_attention_workspace_bytes(int64_t n, int64_t nnz) {
  return as::attention_workspace(n < 0 ? 0 : n, nnz < 0 ? 0 : nnz);
}

int as_csr_attention_f32(const int64_t* crow, const int64_t* col, const float* query, const float* key,
                         const float* value, float* out, int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v,
                         float scale, void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (n < 0 || n > INT32_MAX || nnz < 0 || f_qk < 0 || f_v < 0)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "attention sizes out of range");
  if (f_qk >= as::kMaxFeatures || f_v >= as::kMaxFeatures)
    return as::fail(AS_ERR_UNSUPPORTED, "F_qk and F_v must be below 2^28 (32-bit lane offsets)");
  if (n == 0 || f_v == 0) return AS_OK;
  if (crow == nullptr || value == nullptr || out == nullptr || (nnz > 0 && (col == nullptr || query == nullptr ||
                                                                           key == nullptr)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (f_qk == 0 && nnz > 0)
    return as::fail(AS_ERR_UNSUPPORTED, "attention with zero query/key features is handled by the caller");
  if (workspace == nullptr || workspace_bytes < as::attention_workspace(n, nnz))
    return as::fail(AS_ERR_WORKSPACE, "attention needs %zu workspace bytes, got %zu", as::attention_workspace(n, nnz),
                    workspace_bytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* scratch = reinterpret_cast<float*>(ws);
  ws += as::align_up(static_cast<size_t>(nnz > 0 ? nnz : 1) * sizeof(float), 256);
  int32_t* order = reinterpret_cast<int32_t*>(ws);
  ws += as::align_up(static_cast<size_t>(n) * sizeof(int32_t), 256);
  int32_t* counts = reinterpret_cast<int32_t*>(ws);
  void* bin_ws = ws + 256;
  // Light rows stay in row order (one bucket): ordering them by degree measured
  // slower here (13.4 vs 12.8 ms on the 124M-nnz attention graph).
  int st = as::launch_bin_rows(crow, n, as::kAttHubDegree, as::kAttBuckets, 1, order, counts, bin_ws, s);
  if (st != AS_OK) return st;

  const bool qvec = f_qk > 0 && f_qk % 32 == 0 && f_qk / 32 <= 8 && as::al(query, 16) && as::al(key, 16);
  const int vv = as::value_vector(value, out, f_v, f_v);
  const int hv = as::value_vector(value, out, f_v, (f_v + as::kAttWaves - 1) / as::kAttWaves);
  int64_t heavy_upper = nnz / as::kAttHubDegree;
  if (heavy_upper > n) heavy_upper = n;
  const int64_t blocks = heavy_upper + (n + as::kAttWaves - 1) / as::kAttWaves;
  const as::AttArgs a{crow, col, query, key, value, out, scratch, n, f_qk, f_v, scale, order, counts};
  if (!qvec) {
    as::launch_att_vv<false, 1>(vv, hv, a, blocks, s);
  } else {
    switch (static_cast<int>(f_qk / 32)) {
      case 1: as::launch_att_vv<true, 1>(vv, hv, a, blocks, s); break;
      case 2: as::launch_att_vv<true, 2>(vv, hv, a, blocks, s); break;
      case 3: as::launch_att_vv<true, 3>(vv, hv, a, blocks, s); break;
      case 4: as::launch_att_vv<true, 4>(vv, hv, a, blocks, s); break;
      case 5: as::launch_att_vv<true, 5>(vv, hv, a, blocks, s); break;
      case 6: as::launch_att_vv<true, 6>(vv, hv, a, blocks, s); break;
      case 7: as::launch_att_vv<true, 7>(vv, hv, a, blocks, s); break;
      default: as::launch_att_vv<true, 8>(vv, hv, a, blocks, s); break;
    }
  }
  return as::check_launch("csr_attention");
}

}  // extern "C"
