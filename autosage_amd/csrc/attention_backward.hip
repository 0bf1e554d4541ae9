// Backward of the CSR attention out = P·V, P = softmax_row(scale · <Q[r], K[c]>),
// in two gather passes and no nnz-sized intermediate (fp32).
//
// With p_e = exp(s_e − lse_r) for edge e = (r, c), dP_e = <dOut[r], V[c]> and
// t_r = Σ_e p_e dP_e = <dOut[r], out[r]>:
//   ds_e = scale · p_e · (dP_e − t_r)
//   dQ[r] = Σ_{e in row r} ds_e K[c]        dK[c] = Σ_{e in column c} ds_e Q[r]
//   dV[c] = Σ_{e in column c} p_e dOut[r]
// Pass 1 walks the rows of A (gathers K and V): it recomputes the scores with
// an online maximum and sum, as the forward does, and accumulates
// Σ exp(s_e − m)·(dP_e − t_r)·K[c] with the same rescaling, so that dQ[r] =
// scale · acc / l and lse_r = m + log l come out of one pass.  Pass 2 walks
// the rows of Aᵀ (the columns of A; gathers Q and dOut): K[c] and V[c] are
// constants of the row, lse_r and t_r are gathered per edge, and dK[c], dV[c]
// are plain sums.  Pass 1 also computes t_r from the forward's output row and
// stores (lse_r, t_r) as one 8-byte pair, which pass 2 gathers per edge.
//
// Both passes use the column slices of colslice_common.h for rows of degree
// >= 128 (one wave per (row, slice), partial states merged per row: pass 1
// like the forward's online softmax, pass 2 by addition in slice order), and
// one wave per row below.  Lanes as in the forward (attention_colslice.hip):
// float4 lanes, G lanes per row of K / Q (GK) and of V / dOut (GV), 8 edges per
// step.  Deterministic.
#include "as_device.h"
#include "as_internal.h"
#include "colslice_common.h"

namespace as {

namespace {

constexpr int64_t kBwdSliceMinDegree = 128;
constexpr int kBwdBatch = 8;
constexpr int64_t kBwdChunkRows = 131072;
constexpr int64_t kBwdSliceBlocks = 4096;
constexpr int64_t kBwdReduceBlocks = 8192;

struct BwdArgs {
  const int64_t* crow;  // the pass's CSR (A for pass 1, Aᵀ for pass 2)
  const int64_t* col;
  const float* q;
  const float* k;
  const float* v;
  const float* g;    // dOut
  const float* out;  // the forward's output
  float2* lt;        // (lse_r, t_r = <dOut[r], out[r]>): written by pass 1, read by pass 2
  float* dq;
  float* dk;
  float* dv;
  int64_t n;
  int64_t fqk;
  int64_t fv;
  float scale;
  const int32_t* order;
  const int32_t* counts;
  const int32_t* off;
};

__device__ __forceinline__ void merge_state(float& m, float& l, float (&acc)[4], float mo, float lo,
                                            const float (&ao)[4]) {
  const float mn = fmaxf(m, mo);
  if (mn == -INFINITY) return;
  const float c1 = m == -INFINITY ? 0.f : expf(m - mn);
  const float c2 = mo == -INFINITY ? 0.f : expf(mo - mn);
  l = l * c1 + lo * c2;
#pragma unroll
  for (int v = 0; v < 4; ++v) acc[v] = acc[v] * c1 + ao[v] * c2;
  m = mn;
}

// Lanes group `width` of a float4 row owned by lane % width, zero past the
// feature end.
template <int W>
__device__ __forceinline__ FVec<4> lane_row(const float* __restrict__ base, int64_t row, int64_t f) {
  const int kl = lane_id() % W;
  FVec<4> r;
  if (4 * kl < f) {
    r = load_vec<4>(base + row * f + 4 * kl);
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) r.v[v] = 0.f;
  }
  return r;
}

// <a, b> over the W lanes of a group holding one float4 each (every lane of
// the group ends with the same value).
template <int W>
__device__ __forceinline__ float row_dot(const FVec<4>& a, const FVec<4>& b) {
  float d = a.v[0] * b.v[0];
#pragma unroll
  for (int v = 1; v < 4; ++v) d = __builtin_fmaf(a.v[v], b.v[v], d);
#pragma unroll
  for (int o = W / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
  return d;
}

// Pass 1 over edges [rs, re) of row r of A: q = Q[r] (K lanes), g = dOut[r]
// (V lanes).  Each K lane group keeps (m, l, acc) over its own edges:
// acc = Σ exp(s − m)·(dP − t)·K[c] (K lanes own 4 features of F_qk); the
// groups are merged at the end, so every lane holds the row's state.
template <int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void bwd_q_edges(const int64_t* __restrict__ col, const float* __restrict__ key,
                                            const float* __restrict__ value, int64_t fqk_rt, int64_t fv_rt,
                                            const FVec<4>& q, const FVec<4>& g, float t, float scale, int64_t rs,
                                            int64_t re, float& m, float& l, float (&acc)[4]) {
  constexpr int EK = kWave / GK;
  constexpr int EV = kWave / GV;
  constexpr int E = kBwdBatch;
  const int64_t fqk = FQK > 0 ? FQK : fqk_rt;
  const int64_t fv = FV > 0 ? FV : fv_rt;
  const int lane = lane_id();
  const int gk = lane / GK;
  const int kl = lane % GK;
  const int gv = lane / GV;
  const int vl = lane % GV;
  const uint32_t kbytes = static_cast<uint32_t>((4 * kl < fqk ? 4 * kl : 0) * 4);
  const uint32_t vbytes = static_cast<uint32_t>((4 * vl < fv ? 4 * vl : 0) * 4);
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  m = -INFINITY;
  l = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) acc[v] = 0.f;
  int next_col = 0;
  if (lane < re - rs) next_col = static_cast<int>(col[rs + lane]);
  for (int64_t base = rs; base < re; base += kWave) {
    const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
    const int my_col = next_col;
    const int64_t nb = base + kWave;
    if (nb < re && lane < re - nb) next_col = static_cast<int>(col[nb + lane]);
    for (int j = 0; j < cnt; j += E) {
      FVec<4> kv[E / EK];
      FVec<4> vv[E / EV];
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        int c = 0;
#pragma unroll
        for (int gg = 0; gg < EK; ++gg) {
          const int e = j + i * EK + gg;
          const int cg = bcast_i32(my_col, e < cnt ? e : cnt - 1);
          c = gk == gg ? cg : c;
        }
        kv[i] = load_vec_off<4>(key + row_offset(c, fqk), kbytes);
      }
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        int c = 0;
#pragma unroll
        for (int gg = 0; gg < EV; ++gg) {
          const int e = j + i * EV + gg;
          const int cg = bcast_i32(my_col, e < cnt ? e : cnt - 1);
          c = gv == gg ? cg : c;
        }
        vv[i] = load_vec_off<4>(value + row_offset(c, fv), vbytes);
      }
      // dP in the V groups: V instruction i, group gv holds batch edge i·EV + gv
      float dpv[E / EV];
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        float d = g.v[0] * vv[i].v[0];
#pragma unroll
        for (int v = 1; v < 4; ++v) d = __builtin_fmaf(g.v[v], vv[i].v[v], d);
#pragma unroll
        for (int o = GV / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
        dpv[i] = d;
      }
      // scores in the K groups, and the dP of each K group's edge
      float s[E / EK];
      float dp[E / EK];
      float mb = -INFINITY;
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        float d = q.v[0] * kv[i].v[0];
#pragma unroll
        for (int v = 1; v < 4; ++v) d = __builtin_fmaf(q.v[v], kv[i].v[v], d);
#pragma unroll
        for (int o = GK / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
        s[i] = j + i * EK + gk < cnt ? d * scale : -INFINITY;
        float di = 0.f;
#pragma unroll
        for (int gg = 0; gg < EK; ++gg) {
          const int e = i * EK + gg;  // batch edge of K group gg
          const float de = bcast_f32(dpv[e / EV], GV * (e % EV));
          di = gk == gg ? de : di;
        }
        dp[i] = di;
        mb = fmaxf(mb, s[i]);
      }
      const float mn = fmaxf(m, mb);
      if (mn != -INFINITY) {
        const float corr = m == -INFINITY ? 0.f : expf(m - mn);
        l *= corr;
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] *= corr;
#pragma unroll
        for (int i = 0; i < E / EK; ++i) {
          const float p = s[i] == -INFINITY ? 0.f : expf(s[i] - mn);
          l += p;
          const float w = p * (dp[i] - t);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(w, kv[i].v[v], acc[v]);
        }
        m = mn;
      }
    }
  }
#pragma unroll
  for (int o = GK; o < kWave; o <<= 1) {
    const float mo = __shfl_xor(m, o, kWave);
    const float lo = __shfl_xor(l, o, kWave);
    float ao[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) ao[v] = __shfl_xor(acc[v], o, kWave);
    merge_state(m, l, acc, mo, lo, ao);
  }
}

// Pass 2 over edges [rs, re) of row c of Aᵀ (edge = source row r of A):
// kc = K[c] (K lanes), vc = V[c] (V lanes).  dk (K lanes) += ds·Q[r],
// dv (V lanes) += p·dOut[r]; summed over the lane groups at the end.
template <int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void bwd_kv_edges(const int64_t* __restrict__ src, const float* __restrict__ query,
                                             const float* __restrict__ grad_out, const float2* __restrict__ lt,
                                             int64_t fqk_rt, int64_t fv_rt,
                                             const FVec<4>& kc, const FVec<4>& vc, float scale, int64_t rs,
                                             int64_t re, float (&dk)[4], float (&dv)[4]) {
  constexpr int EK = kWave / GK;
  constexpr int EV = kWave / GV;
  constexpr int E = kBwdBatch;
  const int64_t fqk = FQK > 0 ? FQK : fqk_rt;
  const int64_t fv = FV > 0 ? FV : fv_rt;
  const int lane = lane_id();
  const int gk = lane / GK;
  const int kl = lane % GK;
  const int gv = lane / GV;
  const int vl = lane % GV;
  const uint32_t kbytes = static_cast<uint32_t>((4 * kl < fqk ? 4 * kl : 0) * 4);
  const uint32_t vbytes = static_cast<uint32_t>((4 * vl < fv ? 4 * vl : 0) * 4);
  rs = uniform_i64(rs);
  re = uniform_i64(re);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    dk[v] = 0.f;
    dv[v] = 0.f;
  }
  int next_src = 0;
  if (lane < re - rs) next_src = static_cast<int>(src[rs + lane]);
  for (int64_t base = rs; base < re; base += kWave) {
    const int cnt = static_cast<int>((re - base) < kWave ? (re - base) : kWave);
    const int my_src = next_src;
    const int64_t nb = base + kWave;
    if (nb < re && lane < re - nb) next_src = static_cast<int>(src[nb + lane]);
    for (int j = 0; j < cnt; j += E) {
      FVec<4> qv[E / EK];
      FVec<4> gvv[E / EV];
      float lk[E / EK];
      float tk[E / EK];
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        int r = 0;
#pragma unroll
        for (int gg = 0; gg < EK; ++gg) {
          const int e = j + i * EK + gg;
          const int rg = bcast_i32(my_src, e < cnt ? e : cnt - 1);
          r = gk == gg ? rg : r;
        }
        qv[i] = load_vec_off<4>(query + row_offset(r, fqk), kbytes);
        const float2 w = lt[r];  // one 8-byte gather for both row scalars
        lk[i] = w.x;
        tk[i] = w.y;
      }
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        int r = 0;
#pragma unroll
        for (int gg = 0; gg < EV; ++gg) {
          const int e = j + i * EV + gg;
          const int rg = bcast_i32(my_src, e < cnt ? e : cnt - 1);
          r = gv == gg ? rg : r;
        }
        gvv[i] = load_vec_off<4>(grad_out + row_offset(r, fv), vbytes);
      }
      // dP in the V groups
      float dpv[E / EV];
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        float d = vc.v[0] * gvv[i].v[0];
#pragma unroll
        for (int v = 1; v < 4; ++v) d = __builtin_fmaf(vc.v[v], gvv[i].v[v], d);
#pragma unroll
        for (int o = GV / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
        dpv[i] = d;
      }
      // p and ds in the K groups; dK
      float pk[E / EK];
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        float d = kc.v[0] * qv[i].v[0];
#pragma unroll
        for (int v = 1; v < 4; ++v) d = __builtin_fmaf(kc.v[v], qv[i].v[v], d);
#pragma unroll
        for (int o = GK / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
        const bool valid = j + i * EK + gk < cnt;
        const float p = valid ? expf(d * scale - lk[i]) : 0.f;
        float di = 0.f;
#pragma unroll
        for (int gg = 0; gg < EK; ++gg) {
          const int e = i * EK + gg;
          const float de = bcast_f32(dpv[e / EV], GV * (e % EV));
          di = gk == gg ? de : di;
        }
        const float ds = scale * p * (di - tk[i]);
        pk[i] = p;
#pragma unroll
        for (int v = 0; v < 4; ++v) dk[v] = __builtin_fmaf(ds, qv[i].v[v], dk[v]);
      }
      // dV: the p of each V group's edge
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        float pi = 0.f;
#pragma unroll
        for (int gg = 0; gg < EV; ++gg) {
          const int e = i * EV + gg;
          const float pe = bcast_f32(pk[e / EK], GK * (e % EK));
          pi = gv == gg ? pe : pi;
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) dv[v] = __builtin_fmaf(pi, gvv[i].v[v], dv[v]);
      }
    }
  }
#pragma unroll
  for (int o = GK; o < kWave; o <<= 1) {
#pragma unroll
    for (int v = 0; v < 4; ++v) dk[v] += __shfl_xor(dk[v], o, kWave);
  }
#pragma unroll
  for (int o = GV; o < kWave; o <<= 1) {
#pragma unroll
    for (int v = 0; v < 4; ++v) dv[v] += __shfl_xor(dv[v], o, kWave);
  }
}

// ---- pass 1: dQ and lse over the rows of A ----

template <int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdq_rows_kernel(BwdArgs a) {
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const int lane = lane_id();
  for (int64_t item = a.counts[0] + static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block(); item < a.n;
       item += waves) {
    const int64_t row = uniform_i64(a.order[item]);
    const FVec<4> q = lane_row<GK>(a.q, row, a.fqk);
    const FVec<4> g = lane_row<GV>(a.g, row, a.fv);
    const float t = row_dot<GV>(g, lane_row<GV>(a.out, row, a.fv));
    float m, l, acc[4];
    bwd_q_edges<GK, GV, FQK, FV>(a.col, a.k, a.v, a.fqk, a.fv, q, g, t, a.scale, a.crow[row], a.crow[row + 1], m, l,
                                 acc);
    if (lane < GK && 4 * lane < a.fqk) {
      FVec<4> o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o.v[v] = l > 0.f ? a.scale * acc[v] / l : 0.f;
      store_vec<4>(a.dq + row * a.fqk + 4 * lane, o);
    }
    if (lane == 0) a.lt[row] = make_float2(l > 0.f ? m + logf(l) : -INFINITY, t);
  }
}

template <int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdq_slice_kernel(BwdArgs a, int64_t begin, int64_t items, int64_t stride,
                                                            float* __restrict__ pm, float* __restrict__ pl,
                                                            float* __restrict__ pacc) {
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
    const FVec<4> q = lane_row<GK>(a.q, row, a.fqk);
    const FVec<4> g = lane_row<GV>(a.g, row, a.fv);
    const float t = row_dot<GV>(g, lane_row<GV>(a.out, row, a.fv));
    float m, l, acc[4];
    bwd_q_edges<GK, GV, FQK, FV>(a.col, a.k, a.v, a.fqk, a.fv, q, g, t, a.scale, rs + lo, rs + hi, m, l, acc);
    const int64_t at = slice * stride + local;
    // the row's t, once (the reduction writes its lse)
    if (slice == 0 && lane == 0) a.lt[row].y = t;
    if (lane < GK && 4 * lane < a.fqk) {
      FVec<4> o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o.v[v] = acc[v];
      store_vec<4>(pacc + at * a.fqk + 4 * lane, o);
    }
    if (lane == 0) {
      pm[at] = m;
      pl[at] = l;
    }
  }
}

// Merge of the 8 partial states of each sliced row; thread per (row, 4
// features); the thread of features 0-3 also writes lse.
__global__ __launch_bounds__(kBlock) void bwdq_reduce_kernel(BwdArgs a, int64_t begin, int64_t items, int64_t stride,
                                                             const float* __restrict__ pm,
                                                             const float* __restrict__ pl,
                                                             const float* __restrict__ pacc) {
  const int64_t F4 = a.fqk / 4;
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
        const FVec<4> p = load_vec<4>(pacc + (s * stride + local) * a.fqk + f);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(c, p.v[v], acc[v]);
      }
    }
    const int64_t row = a.order[begin + local];
    FVec<4> o;
#pragma unroll
    for (int v = 0; v < 4; ++v) o.v[v] = l > 0.f ? a.scale * acc[v] / l : 0.f;
    store_vec<4>(a.dq + row * a.fqk + f, o);
    if (f == 0) a.lt[row].x = l > 0.f ? m + logf(l) : -INFINITY;
  }
}

// ---- pass 2: dK and dV over the rows of Aᵀ ----

template <int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdkv_rows_kernel(BwdArgs a) {
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const int lane = lane_id();
  for (int64_t item = a.counts[0] + static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block(); item < a.n;
       item += waves) {
    const int64_t row = uniform_i64(a.order[item]);
    const FVec<4> kc = lane_row<GK>(a.k, row, a.fqk);
    const FVec<4> vc = lane_row<GV>(a.v, row, a.fv);
    float dk[4], dv[4];
    bwd_kv_edges<GK, GV, FQK, FV>(a.col, a.q, a.g, a.lt, a.fqk, a.fv, kc, vc, a.scale, a.crow[row], a.crow[row + 1],
                                  dk, dv);
    if (lane < GK && 4 * lane < a.fqk) {
      FVec<4> o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o.v[v] = dk[v];
      store_vec<4>(a.dk + row * a.fqk + 4 * lane, o);
    }
    if (lane < GV && 4 * lane < a.fv) {
      FVec<4> o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o.v[v] = dv[v];
      store_vec<4>(a.dv + row * a.fv + 4 * lane, o);
    }
  }
}

template <int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdkv_slice_kernel(BwdArgs a, int64_t begin, int64_t items, int64_t stride,
                                                             float* __restrict__ pk, float* __restrict__ pv) {
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
    const FVec<4> kc = lane_row<GK>(a.k, row, a.fqk);
    const FVec<4> vc = lane_row<GV>(a.v, row, a.fv);
    float dk[4], dv[4];
    bwd_kv_edges<GK, GV, FQK, FV>(a.col, a.q, a.g, a.lt, a.fqk, a.fv, kc, vc, a.scale, rs + lo, rs + hi, dk, dv);
    const int64_t at = slice * stride + local;
    if (lane < GK && 4 * lane < a.fqk) {
      FVec<4> o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o.v[v] = dk[v];
      store_vec<4>(pk + at * a.fqk + 4 * lane, o);
    }
    if (lane < GV && 4 * lane < a.fv) {
      FVec<4> o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o.v[v] = dv[v];
      store_vec<4>(pv + at * a.fv + 4 * lane, o);
    }
  }
}

// Sums of the 8 partials of each sliced row of Aᵀ, in slice order; thread per
// (row, 4 features) over the F_qk + F_v features of dK and dV.
__global__ __launch_bounds__(kBlock) void bwdkv_reduce_kernel(BwdArgs a, int64_t begin, int64_t items,
                                                              int64_t stride, const float* __restrict__ pk,
                                                              const float* __restrict__ pv) {
  const int64_t K4 = a.fqk / 4;
  const int64_t F4 = K4 + a.fv / 4;
  const int64_t total = items * F4;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += step) {
    const int64_t local = t / F4;
    const int64_t q4 = t - local * F4;
    if (begin + local >= a.counts[0]) continue;
    const bool is_k = q4 < K4;
    const int64_t f = (is_k ? q4 : q4 - K4) * 4;
    const int64_t width = is_k ? a.fqk : a.fv;
    const float* part = is_k ? pk : pv;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kSlices; ++s) {
      const FVec<4> p = load_vec<4>(part + (s * stride + local) * width + f);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] += p.v[v];
    }
    const int64_t row = a.order[begin + local];
    FVec<4> o;
#pragma unroll
    for (int v = 0; v < 4; ++v) o.v[v] = acc[v];
    store_vec<4>((is_k ? a.dk : a.dv) + row * width + f, o);
  }
}

int bwd_lane_group(int64_t f) { return f <= 64 ? 16 : (f <= 128 ? 32 : 64); }

// Per sliced row of a chunk: pass 1 keeps 8 x (m, l, F_qk), pass 2 8 x
// (F_qk + F_v) floats.
size_t bwd_row_bytes(int64_t fqk, int64_t fv) {
  const size_t p1 = static_cast<size_t>(fqk) + 2;
  const size_t p2 = static_cast<size_t>(fqk) + static_cast<size_t>(fv);
  return static_cast<size_t>(kSlices) * (p1 > p2 ? p1 : p2) * sizeof(float);
}

// (lse, t) pairs, then a slice plan region for passes called without a plan
size_t bwd_pairs_bytes(int64_t n) { return align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(float2), 256); }
size_t bwd_fixed_bytes(int64_t n) { return bwd_pairs_bytes(n) + slice_plan_bytes(n); }

int64_t bwd_sliced_upper(int64_t n, int64_t nnz) {
  const int64_t u = nnz / kBwdSliceMinDegree;
  return u < n ? u : n;
}

template <int GK, int GV, int FQK = 0, int FV = 0>
void launch_pass1(const BwdArgs& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  int64_t row_blocks = (a.n + kWavesPerBlock - 1) / kWavesPerBlock;
  if (row_blocks > kMaxBlocksPerLaunch) row_blocks = kMaxBlocksPerLaunch;
  hipLaunchKernelGGL((bwdq_rows_kernel<GK, GV, FQK, FV>), dim3(static_cast<unsigned>(row_blocks)), dim3(kBlock), 0, s,
                     a);
  const size_t states = static_cast<size_t>(kSlices) * static_cast<size_t>(chunk);
  float* pm = part;
  float* pl = part + align_up(states, 64);
  float* pacc = pl + align_up(states, 64);
  for (int64_t begin = 0; begin < upper; begin += chunk) {
    const int64_t items = upper - begin < chunk ? upper - begin : chunk;
    int64_t per_slice = (items + kWavesPerBlock - 1) / kWavesPerBlock;
    if (per_slice > kBwdSliceBlocks) per_slice = kBwdSliceBlocks;
    hipLaunchKernelGGL((bwdq_slice_kernel<GK, GV, FQK, FV>), dim3(static_cast<unsigned>(kSlices * per_slice)),
                       dim3(kBlock), 0, s, a, begin, items, chunk, pm, pl, pacc);
    int64_t blocks = (items * (a.fqk / 4) + kBlock - 1) / kBlock;
    if (blocks > kBwdReduceBlocks) blocks = kBwdReduceBlocks;
    hipLaunchKernelGGL(bwdq_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, a, begin, items,
                       chunk, pm, pl, pacc);
  }
}

template <int GK, int GV, int FQK = 0, int FV = 0>
void launch_pass2(const BwdArgs& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  int64_t row_blocks = (a.n + kWavesPerBlock - 1) / kWavesPerBlock;
  if (row_blocks > kMaxBlocksPerLaunch) row_blocks = kMaxBlocksPerLaunch;
  hipLaunchKernelGGL((bwdkv_rows_kernel<GK, GV, FQK, FV>), dim3(static_cast<unsigned>(row_blocks)), dim3(kBlock), 0,
                     s, a);
  const size_t states = static_cast<size_t>(kSlices) * static_cast<size_t>(chunk);
  float* pk = part;
  float* pv = part + align_up(states * static_cast<size_t>(a.fqk), 64);
  for (int64_t begin = 0; begin < upper; begin += chunk) {
    const int64_t items = upper - begin < chunk ? upper - begin : chunk;
    int64_t per_slice = (items + kWavesPerBlock - 1) / kWavesPerBlock;
    if (per_slice > kBwdSliceBlocks) per_slice = kBwdSliceBlocks;
    hipLaunchKernelGGL((bwdkv_slice_kernel<GK, GV, FQK, FV>), dim3(static_cast<unsigned>(kSlices * per_slice)),
                       dim3(kBlock), 0, s, a, begin, items, chunk, pk, pv);
    int64_t blocks = (items * ((a.fqk + a.fv) / 4) + kBlock - 1) / kBlock;
    if (blocks > kBwdReduceBlocks) blocks = kBwdReduceBlocks;
    hipLaunchKernelGGL(bwdkv_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, a, begin, items,
                       chunk, pk, pv);
  }
}

template <int PASS, int GK, int GV, int FQK = 0, int FV = 0>
void launch_pass(const BwdArgs& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  if constexpr (PASS == 1) launch_pass1<GK, GV, FQK, FV>(a, upper, chunk, part, s);
  else launch_pass2<GK, GV, FQK, FV>(a, upper, chunk, part, s);
}

template <int PASS>
void dispatch_pass(const BwdArgs& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  if (a.fqk == 64 && a.fv == 128) return launch_pass<PASS, 16, 32, 64, 128>(a, upper, chunk, part, s);
  if (a.fqk == 64 && a.fv == 64) return launch_pass<PASS, 16, 16, 64, 64>(a, upper, chunk, part, s);
  if (a.fqk == 128 && a.fv == 128) return launch_pass<PASS, 32, 32, 128, 128>(a, upper, chunk, part, s);
  const int gk = bwd_lane_group(a.fqk);
  const int gv = bwd_lane_group(a.fv);
#define AS_BWD_GV(GK_)                                                                    \
  switch (gv) {                                                                           \
    case 16: launch_pass<PASS, GK_, 16>(a, upper, chunk, part, s); break;                 \
    case 32: launch_pass<PASS, GK_, 32>(a, upper, chunk, part, s); break;                 \
    default: launch_pass<PASS, GK_, 64>(a, upper, chunk, part, s); break;                 \
  }
  switch (gk) {
    case 16: AS_BWD_GV(16) break;
    case 32: AS_BWD_GV(32) break;
    default: AS_BWD_GV(64) break;
  }
#undef AS_BWD_GV
}

}  // namespace

}  // namespace as

extern "C" {

size_t as_csr_attention_backward_workspace_bytes(int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v) {
  if (n < 0) n = 0;
  if (nnz < 0) nnz = 0;
  if (f_qk < 4) f_qk = 4;
  if (f_v < 4) f_v = 4;
  int64_t rows = as::bwd_sliced_upper(n, nnz);
  if (rows > as::kBwdChunkRows) rows = as::kBwdChunkRows;
  if (rows < 1) rows = 1;
  return as::bwd_fixed_bytes(n) + static_cast<size_t>(rows) * as::bwd_row_bytes(f_qk, f_v) + 3 * 256;
}

int as_csr_attention_backward_f32(const int64_t* crow, const int64_t* col, const int64_t* crow_t,
                                  const int64_t* col_t, const float* query, const float* key, const float* value,
                                  const float* out, const float* grad_out, float* grad_q, float* grad_k,
                                  float* grad_v, int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v, float scale,
                                  const void* plan, int64_t plan_tag, const void* plan_t, int64_t plan_t_tag,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  const int64_t want = as::slice_plan_tag(as::kBwdSliceMinDegree, 1);
  if ((plan != nullptr && plan_tag != want) || (plan_t != nullptr && plan_t_tag != want))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "a plan was built for other settings (this call needs plan tag %lld)",
                    (long long)want);
  if ((plan != nullptr && !as::aligned(plan, 256)) || (plan_t != nullptr && !as::aligned(plan_t, 256)))
    return as::fail(AS_ERR_WORKSPACE, "plans must be 256-byte aligned");
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (f_qk < 4 || f_qk > 256 || f_qk % 4 != 0 || f_v < 4 || f_v > 256 || f_v % 4 != 0)
    return as::fail(AS_ERR_UNSUPPORTED, "attention backward needs F_qk and F_v in [4, 256], multiples of 4");
  if (n == 0) return AS_OK;
  if (crow == nullptr || crow_t == nullptr || query == nullptr || key == nullptr || value == nullptr ||
      out == nullptr || grad_out == nullptr || grad_q == nullptr || grad_k == nullptr || grad_v == nullptr ||
      (nnz > 0 && (col == nullptr || col_t == nullptr)))
    return as::fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  for (const void* p : {static_cast<const void*>(query), static_cast<const void*>(key),
                        static_cast<const void*>(value), static_cast<const void*>(out),
                        static_cast<const void*>(grad_out), static_cast<const void*>(grad_q),
                        static_cast<const void*>(grad_k), static_cast<const void*>(grad_v)})
    if (!as::aligned(p, 16)) return as::fail(AS_ERR_UNSUPPORTED, "attention backward needs 16-byte aligned tensors");
  // the workspace holds a plan region only for a pass called without a plan
  const bool own_plan = plan == nullptr || plan_t == nullptr;
  const size_t fixed = own_plan ? as::bwd_fixed_bytes(n) : as::bwd_pairs_bytes(n);
  const size_t row_bytes = as::bwd_row_bytes(f_qk, f_v);
  if (workspace == nullptr || workspace_bytes < fixed + row_bytes + 3 * 256)
    return as::fail(AS_ERR_WORKSPACE, "attention backward needs at least %zu workspace bytes, got %zu",
                    fixed + row_bytes + 3 * 256, workspace_bytes);
  if (!as::aligned(workspace, 256)) return as::fail(AS_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  const int64_t upper = as::bwd_sliced_upper(n, nnz);
  int64_t chunk = static_cast<int64_t>((workspace_bytes - fixed - 3 * 256) / row_bytes);
  if (chunk > as::kBwdChunkRows) chunk = as::kBwdChunkRows;
  if (chunk > upper) chunk = upper;
  if (chunk < 1) chunk = 1;

  const hipStream_t s = static_cast<hipStream_t>(stream);
  float2* lt = static_cast<float2*>(workspace);
  void* own = static_cast<char*>(workspace) + as::bwd_pairs_bytes(n);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + fixed);

  // pass 1 over A; then pass 2 over Aᵀ.  A pass without a plan builds one in
  // the workspace's plan region (pass 2 after pass 1 in stream order)
  for (int pass = 1; pass <= 2; ++pass) {
    const int64_t* pc = pass == 1 ? crow : crow_t;
    const int64_t* pcol = pass == 1 ? col : col_t;
    const void* given = pass == 1 ? plan : plan_t;
    const as::SlicePlan view = as::slice_plan_view(given != nullptr ? const_cast<void*>(given) : own, n);
    if (given == nullptr) {
      const int st = as::build_slice_plan(pc, pcol, n, as::kBwdSliceMinDegree, 1, false, view, s);
      if (st != AS_OK) return st;
    }
    const as::BwdArgs a{pc,     pcol,   query, key,  value, grad_out,   out,         lt,      grad_q,
                        grad_k, grad_v, n,     f_qk, f_v,   scale,      view.order, view.counts, view.off};
    if (pass == 1) as::dispatch_pass<1>(a, upper, chunk, part, s);
    else as::dispatch_pass<2>(a, upper, chunk, part, s);
  }
  return as::check_launch("csr_attention_backward");
}

}  // extern "C"
