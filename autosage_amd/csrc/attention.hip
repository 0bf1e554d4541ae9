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
// (reference dot order) times `scale`, stores them in a caller-provided
// nnz-float scratch, derives m and d exactly as above and then accumulates
// out[r, :] = sum_e p_e · V[col_e, :] in edge order with fmaf, as the SpMM
// kernels do.  With scale 1 (or a power of two) it is therefore
// bit-identical to the three unfused stages.
#include "as_device.h"
#include "as_internal.h"

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

// QVEC: query/key rows as 8 lanes × float4 per 32 features (MF blocks);
// otherwise 32 lanes per edge with scalar loads (any F_qk).
// VV: value floats per lane, a pass covers 64·VV value features.
template <bool QVEC, int MF, int VV>
__global__ __launch_bounds__(kBlock) void csr_attention_kernel(
    const int64_t* __restrict__ crow, const int64_t* __restrict__ col, const float* __restrict__ query,
    const float* __restrict__ key, const float* __restrict__ value, float* __restrict__ out,
    float* __restrict__ scratch, int64_t n, int64_t Fqk, int64_t Fv, float scale, int64_t idx_base) {
  constexpr int G = QVEC ? 8 : 32;
  constexpr int S = 32 / G;
  constexpr int NG = kWave / G;
  constexpr int UE = QVEC ? (MF <= 2 ? 4 : 2) : 1;
  constexpr int U = 8;
  const int lane = lane_id();
  const int g = lane / G;
  const int j = lane % G;
  const int64_t row = idx_base + static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wave_in_block();
  if (row >= n) return;
  const int64_t rs = uniform_i64(crow[row]);
  const int64_t re = uniform_i64(crow[row + 1]);

  float m = -INFINITY;
  float d = 0.f;
  if (rs < re) {
    // Pass A: scores (reference SDDMM order) into scratch, running max.
    float qv[QVEC ? MF : 1][S];
    const float* qrow = query + row * Fqk;
    if constexpr (QVEC) {
#pragma unroll
      for (int mm = 0; mm < MF; ++mm) {
        const FVec<S> t = load_vec<S>(qrow + 32 * mm + S * j);
#pragma unroll
        for (int s = 0; s < S; ++s) qv[mm][s] = t.v[s];
      }
    }
    float mloc = -INFINITY;
    for (int64_t base = rs; base < re; base += NG * UE) {
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
    m = wave_max_f32(mloc);
    // The scratch scores were written by other lanes of this wave.
    __threadfence_block();
    // Pass B: denominator in the row-softmax order.
    for (int64_t e = rs + lane; e < re; e += kWave) d += expf(scratch[e] - m);
    d = wave_sum_f32(d);
  }

  // Pass C: out = sum_e p_e · V[col_e] in edge order (wave-row SpMM layout:
  // unchecked full batches of U edges, then the remainder; lanes past Fv load
  // a valid address and store nothing).
  constexpr int P = kWave * VV;
  for (int64_t f0 = 0; f0 < Fv; f0 += P) {
    const int64_t fl = f0 + static_cast<int64_t>(lane) * VV;
    const bool active = fl < Fv;
    const uint32_t lane_bytes = static_cast<uint32_t>((active ? fl : 0) * 4);
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

bool al(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

template <bool QVEC, int MF>
void launch_attention_vv(int vv, dim3 grid, hipStream_t s, const int64_t* crow, const int64_t* col, const float* q,
                         const float* k, const float* v, float* out, float* scratch, int64_t n, int64_t fqk,
                         int64_t fv, float scale, int64_t base) {
  switch (vv) {
    case 4:
      hipLaunchKernelGGL((csr_attention_kernel<QVEC, MF, 4>), grid, dim3(kBlock), 0, s, crow, col, q, k, v, out,
                         scratch, n, fqk, fv, scale, base);
      break;
    case 2:
      hipLaunchKernelGGL((csr_attention_kernel<QVEC, MF, 2>), grid, dim3(kBlock), 0, s, crow, col, q, k, v, out,
                         scratch, n, fqk, fv, scale, base);
      break;
    default:
      hipLaunchKernelGGL((csr_attention_kernel<QVEC, MF, 1>), grid, dim3(kBlock), 0, s, crow, col, q, k, v, out,
                         scratch, n, fqk, fv, scale, base);
      break;
  }
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

size_t as_csr_attention_workspace_bytes(int64_t n, int64_t nnz) {
  (void)n;
  return as::align_up(static_cast<size_t>(nnz > 0 ? nnz : 1) * sizeof(float), 256);
}

int as_csr_attention_f32(const int64_t* crow, const int64_t* col, const float* query, const float* key,
                         const float* value, float* out, int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v,
                         float scale, void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (n < 0 || n > INT32_MAX || nnz < 0 || f_qk < 0 || f_qk > INT32_MAX || f_v < 0 || f_v > INT32_MAX)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "attention sizes out of range");
  if (n == 0 || f_v == 0) return AS_OK;
  if (crow == nullptr || value == nullptr || out == nullptr || (nnz > 0 && (col == nullptr || query == nullptr ||
                                                                           key == nullptr)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (f_qk == 0 && nnz > 0)
    return as::fail(AS_ERR_UNSUPPORTED, "attention with zero query/key features is handled by the caller");
  if (workspace == nullptr || workspace_bytes < as_csr_attention_workspace_bytes(n, nnz))
    return as::fail(AS_ERR_WORKSPACE, "attention needs %zu workspace bytes, got %zu",
                    as_csr_attention_workspace_bytes(n, nnz), workspace_bytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  float* scratch = static_cast<float*>(workspace);
  const bool qvec = f_qk > 0 && f_qk % 32 == 0 && f_qk / 32 <= 8 && as::al(query, 16) && as::al(key, 16);
  int vv = 1;
  if (f_v % 4 == 0 && f_v > 128 && as::al(value, 16) && as::al(out, 16)) vv = 4;
  else if (f_v % 2 == 0 && f_v > 64 && as::al(value, 8) && as::al(out, 8)) vv = 2;
  const int64_t blocks = (n + as::kWavesPerBlock - 1) / as::kWavesPerBlock;
  for (int64_t b0 = 0; b0 < blocks; b0 += as::kMaxBlocksPerLaunch) {
    const int64_t nb = blocks - b0 < as::kMaxBlocksPerLaunch ? blocks - b0 : as::kMaxBlocksPerLaunch;
    const dim3 grid(static_cast<unsigned>(nb));
    const int64_t base = b0 * as::kWavesPerBlock;
#define AS_ATT(QV, MF) \
  as::launch_attention_vv<QV, MF>(vv, grid, s, crow, col, query, key, value, out, scratch, n, f_qk, f_v, scale, base)
    if (!qvec) {
      AS_ATT(false, 1);
    } else {
      switch (static_cast<int>(f_qk / 32)) {
        case 1: AS_ATT(true, 1); break;
        case 2: AS_ATT(true, 2); break;
        case 3: AS_ATT(true, 3); break;
        case 4: AS_ATT(true, 4); break;
        case 5: AS_ATT(true, 5); break;
        case 6: AS_ATT(true, 6); break;
        case 7: AS_ATT(true, 7); break;
        default: AS_ATT(true, 8); break;
      }
    }
#undef AS_ATT
  }
  return as::check_launch("csr_attention");
}

}  // extern "C"
