// Backward of the CSR attention out = P·V, P = softmax_row(scale · <Q[r], K[c]>),
// in two gather passes and no nnz-sized intermediate; fp32, bf16 or fp16
// inputs (16-bit elements converted exactly to fp32, every sum in fp32, each
// gradient rounded once to the element type).
//
// With p_e = exp(s_e − lse_r) for edge e = (r, c), dP_e = <dOut[r], V[c]> and
// t_r = Σ_e p_e dP_e (= <dOut[r], out[r]>):
//   ds_e = scale · p_e · (dP_e − t_r)
//   dQ[r] = Σ_{e in row r} ds_e K[c]        dK[c] = Σ_{e in column c} ds_e Q[r]
//   dV[c] = Σ_{e in column c} p_e dOut[r]
// Pass 1 walks the rows of A (gathers K and V): it recomputes the scores with
// an online maximum and sum, as the forward does, and accumulates with the
// same rescaling (w = exp(s − m)):
//   fp32:   t_r from the forward's output row, acc = Σ w·(dP − t)·K[c],
//           dQ[r] = scale · acc / l;
//   16-bit: the output is rounded (bf16 keeps 8 bits), so t_r is summed here,
//           tsum = Σ w·dP, with acc = Σ w·dP·K[c] and acc2 = Σ w·K[c] apart:
//           t = tsum / l, dQ[r] = scale · (acc − t·acc2) / l.
// lse_r = m + log l comes out of the same pass; (lse_r, t_r) is stored as one
// 8-byte pair.  Pass 2 walks the rows of Aᵀ (the columns of A; gathers Q,
// dOut and the pair): K[c] and V[c] are constants of the row, and dK[c],
// dV[c] are plain sums.
//
// Both passes use the column slices of colslice_common.h for rows of degree
// >= 128 (one wave per (row, slice), partial states merged per row: pass 1
// like the forward's online softmax, pass 2 by addition in slice order), and
// one wave per row below.  Lanes as in the forward (attention_lanes.h):
// 16-byte lanes (4 fp32 or 8 16-bit elements), G lanes per row of K / Q (GK)
// and of V / dOut (GV), 8 edges per step.  Deterministic.
#include "as_device.h"
#include "as_internal.h"
#include "attention_lanes.h"
#include "colslice_common.h"
#include "elem16.h"

namespace as {

namespace {

constexpr int kBwdBatch = 8;
// Edges per step of a wave that walks one (row, slice) or row with 16-bit
// elements.  Pass 2 (dK, dV): 8, as fp32 (16 in both passes gave the
// benchmark attention's bf16 forward + backward 19.73 against 19.62 ms).
// Pass 1 (dQ): 16, as the forward takes, 19.55-19.57 against 19.69-19.73 ms.
#ifndef AS_BWD_BATCH_16
#define AS_BWD_BATCH_16 8
#endif
template <typename T>
constexpr int bwd_batch() {
  return sizeof(T) == 2 ? AS_BWD_BATCH_16 : kBwdBatch;
}
#ifndef AS_BWD_Q_BATCH_16
#define AS_BWD_Q_BATCH_16 16
#endif
template <typename T>
constexpr int bwd_q_batch() {
  return sizeof(T) == 2 ? AS_BWD_Q_BATCH_16 : kBwdBatch;
}
constexpr int64_t kBwdChunkRows = 131072;
constexpr int64_t kBwdSliceBlocks = 4096;
constexpr int64_t kBwdReduceBlocks = 8192;

// Pass 1 sums t itself (16-bit elements) instead of reading the output row.
template <typename T>
constexpr bool sums_t() {
  return sizeof(T) == 2;
}

template <typename T>
struct BwdArgs {
  const int64_t* crow;  // the pass's CSR (A for pass 1, Aᵀ for pass 2)
  const int64_t* col;
  const T* q;
  const T* k;
  const T* v;
  const T* g;    // dOut
  const T* out;  // the forward's output (read for fp32 only)
  float2* lt;    // (lse_r, t_r): written by pass 1, read by pass 2
  T* dq;
  T* dk;
  T* dv;
  int64_t n;
  int64_t fqk;
  int64_t fv;
  float scale;
  const int32_t* order;
  const int32_t* counts;
  const int32_t* off;
};

// Pass-1 state of a lane over the edges it has seen: running max m,
// l = Σ w, acc (and for 16-bit tsum = Σ w·dP and acc2 = Σ w·K).
template <int P, bool TWO>
struct QState {
  float m;
  float l;
  float tsum;
  float acc[P];
  float acc2[TWO ? P : 1];
};

template <int P, bool TWO>
__device__ __forceinline__ void q_init(QState<P, TWO>& s) {
  s.m = -INFINITY;
  s.l = 0.f;
  s.tsum = 0.f;
#pragma unroll
  for (int v = 0; v < P; ++v) s.acc[v] = 0.f;
  if constexpr (TWO) {
#pragma unroll
    for (int v = 0; v < P; ++v) s.acc2[v] = 0.f;
  }
}

// s ← merge(s, o): both rescaled to the larger maximum, then added.
template <int P, bool TWO>
__device__ __forceinline__ void q_merge(QState<P, TWO>& s, float mo, float lo, float to, const float (&ao)[P],
                                        const float (&a2o)[TWO ? P : 1]) {
  const float mn = fmaxf(s.m, mo);
  if (mn == -INFINITY) return;  // neither side saw an edge
  const float c1 = s.m == -INFINITY ? 0.f : expf(s.m - mn);
  const float c2 = mo == -INFINITY ? 0.f : expf(mo - mn);
  s.l = s.l * c1 + lo * c2;
#pragma unroll
  for (int v = 0; v < P; ++v) s.acc[v] = s.acc[v] * c1 + ao[v] * c2;
  if constexpr (TWO) {
    s.tsum = s.tsum * c1 + to * c2;
#pragma unroll
    for (int v = 0; v < P; ++v) s.acc2[v] = s.acc2[v] * c1 + a2o[v] * c2;
  }
  s.m = mn;
}

// <a, b> over the W lanes of a group holding P elements each (every lane of
// the group ends with the same value).
template <int W, int P>
__device__ __forceinline__ float row_dot(const float (&a)[P], const float (&b)[P]) {
  float d = a[0] * b[0];
#pragma unroll
  for (int v = 1; v < P; ++v) d = __builtin_fmaf(a[v], b[v], d);
#pragma unroll
  for (int o = W / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
  return d;
}

// Pass 1 over edges [rs, re) of row r of A: q = Q[r] (K lanes), g = dOut[r]
// (V lanes), t = t_r (fp32 only).  Each K lane group keeps its state over its
// own edges; the groups are merged at the end, so every lane holds the row's
// state.
template <typename T, int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void bwd_q_edges(const int64_t* __restrict__ col, const T* __restrict__ key,
                                            const T* __restrict__ value, int64_t fqk_rt, int64_t fv_rt,
                                            const float (&q)[lane_elems<T>()], const float (&g)[lane_elems<T>()],
                                            float t, float scale, int64_t rs, int64_t re,
                                            QState<lane_elems<T>(), sums_t<T>()>& st) {
  constexpr int P = lane_elems<T>();
  constexpr bool TWO = sums_t<T>();
  constexpr int EK = kWave / GK;
  constexpr int EV = kWave / GV;
  constexpr int E = bwd_q_batch<T>();
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
  // lanes past the feature end read feature 0 (their q and g are 0)
  const uint32_t kbytes = static_cast<uint32_t>((P * kl < fqk ? P * kl : 0) * sizeof(T));
  const uint32_t vbytes = static_cast<uint32_t>((P * vl < fv ? P * vl : 0) * sizeof(T));
  rs = uniform_i64(rs);
  re = uniform_i64(re);
  q_init(st);
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
        for (int gg = 0; gg < EK; ++gg) {
          const int e = j + i * EK + gg;
          const int cg = bcast_i32(my_col, e < cnt ? e : cnt - 1);
          c = gk == gg ? cg : c;
        }
        kv[i] = load_raw<16>(kb + row_offset(c, fqk) * sizeof(T) + kbytes);
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
        vv[i] = load_raw<16>(vb + row_offset(c, fv) * sizeof(T) + vbytes);
      }
      // dP in the V groups: V instruction i, group gv holds batch edge i·EV + gv
      float dpv[E / EV];
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        float x[P];
        lane_values<T>(vv[i], x);
        dpv[i] = row_dot<GV, P>(g, x);
      }
      // scores in the K groups, and the dP of each K group's edge
      float s[E / EK];
      float dp[E / EK];
      float mb = -INFINITY;
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        float x[P];
        lane_values<T>(kv[i], x);
        const float d = row_dot<GK, P>(q, x);
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
      const float mn = fmaxf(st.m, mb);
      if (mn != -INFINITY) {
        const float corr = st.m == -INFINITY ? 0.f : expf(st.m - mn);
        st.l *= corr;
#pragma unroll
        for (int v = 0; v < P; ++v) st.acc[v] *= corr;
        if constexpr (TWO) {
          st.tsum *= corr;
#pragma unroll
          for (int v = 0; v < P; ++v) st.acc2[v] *= corr;
        }
#pragma unroll
        for (int i = 0; i < E / EK; ++i) {
          const float p = s[i] == -INFINITY ? 0.f : expf(s[i] - mn);
          st.l += p;
          float x[P];
          lane_values<T>(kv[i], x);
          if constexpr (TWO) {
            const float w = p * dp[i];
            st.tsum += w;
#pragma unroll
            for (int v = 0; v < P; ++v) {
              st.acc[v] = __builtin_fmaf(w, x[v], st.acc[v]);
              st.acc2[v] = __builtin_fmaf(p, x[v], st.acc2[v]);
            }
          } else {
            const float w = p * (dp[i] - t);
#pragma unroll
            for (int v = 0; v < P; ++v) st.acc[v] = __builtin_fmaf(w, x[v], st.acc[v]);
          }
        }
        st.m = mn;
      }
    }
  }
#pragma unroll
  for (int o = GK; o < kWave; o <<= 1) {
    const float mo = __shfl_xor(st.m, o, kWave);
    const float lo = __shfl_xor(st.l, o, kWave);
    const float to = TWO ? __shfl_xor(st.tsum, o, kWave) : 0.f;
    float ao[P];
    float a2o[TWO ? P : 1];
#pragma unroll
    for (int v = 0; v < P; ++v) ao[v] = __shfl_xor(st.acc[v], o, kWave);
    if constexpr (TWO) {
#pragma unroll
      for (int v = 0; v < P; ++v) a2o[v] = __shfl_xor(st.acc2[v], o, kWave);
    } else {
      a2o[0] = 0.f;
    }
    q_merge(st, mo, lo, to, ao, a2o);
  }
}

// Pass 2 over edges [rs, re) of row c of Aᵀ (edge = source row r of A):
// kc = K[c] (K lanes), vc = V[c] (V lanes).  dk (K lanes) += ds·Q[r],
// dv (V lanes) += p·dOut[r]; summed over the lane groups at the end.
template <typename T, int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void bwd_kv_edges(const int64_t* __restrict__ src, const T* __restrict__ query,
                                             const T* __restrict__ grad_out, const float2* __restrict__ lt,
                                             int64_t fqk_rt, int64_t fv_rt, const float (&kc)[lane_elems<T>()],
                                             const float (&vc)[lane_elems<T>()], float scale, int64_t rs, int64_t re,
                                             float (&dk)[lane_elems<T>()], float (&dv)[lane_elems<T>()]) {
  constexpr int P = lane_elems<T>();
  constexpr int EK = kWave / GK;
  constexpr int EV = kWave / GV;
  constexpr int E = bwd_batch<T>();
  static_assert(E % EK == 0 && E % EV == 0, "a batch holds whole gather instructions");
  const int64_t fqk = FQK > 0 ? FQK : fqk_rt;
  const int64_t fv = FV > 0 ? FV : fv_rt;
  const int lane = lane_id();
  const int gk = lane / GK;
  const int kl = lane % GK;
  const int gv = lane / GV;
  const int vl = lane % GV;
  const char* __restrict__ qb = reinterpret_cast<const char*>(query);
  const char* __restrict__ gb = reinterpret_cast<const char*>(grad_out);
  const uint32_t kbytes = static_cast<uint32_t>((P * kl < fqk ? P * kl : 0) * sizeof(T));
  const uint32_t vbytes = static_cast<uint32_t>((P * vl < fv ? P * vl : 0) * sizeof(T));
  rs = uniform_i64(rs);
  re = uniform_i64(re);
#pragma unroll
  for (int v = 0; v < P; ++v) {
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
      RawVec<16> qv[E / EK];
      RawVec<16> gvv[E / EV];
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
        qv[i] = load_raw<16>(qb + row_offset(r, fqk) * sizeof(T) + kbytes);
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
        gvv[i] = load_raw<16>(gb + row_offset(r, fv) * sizeof(T) + vbytes);
      }
      // dP in the V groups
      float dpv[E / EV];
#pragma unroll
      for (int i = 0; i < E / EV; ++i) {
        float x[P];
        lane_values<T>(gvv[i], x);
        dpv[i] = row_dot<GV, P>(vc, x);
      }
      // p and ds in the K groups; dK
      float pk[E / EK];
#pragma unroll
      for (int i = 0; i < E / EK; ++i) {
        float x[P];
        lane_values<T>(qv[i], x);
        const float d = row_dot<GK, P>(kc, x);
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
        for (int v = 0; v < P; ++v) dk[v] = __builtin_fmaf(ds, x[v], dk[v]);
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
        float x[P];
        lane_values<T>(gvv[i], x);
#pragma unroll
        for (int v = 0; v < P; ++v) dv[v] = __builtin_fmaf(pi, x[v], dv[v]);
      }
    }
  }
#pragma unroll
  for (int o = GK; o < kWave; o <<= 1) {
#pragma unroll
    for (int v = 0; v < P; ++v) dk[v] += __shfl_xor(dk[v], o, kWave);
  }
#pragma unroll
  for (int o = GV; o < kWave; o <<= 1) {
#pragma unroll
    for (int v = 0; v < P; ++v) dv[v] += __shfl_xor(dv[v], o, kWave);
  }
}

// ---- short rows of 16-bit elements, several to a wave ----
//
// As in the forward (attention_colslice.hip): the wave is cut into segments of
// L = GV lanes, one row each (64 / L rows per wave); inside a segment,
// sub-groups of GK lanes (GK <= GV) gather K (pass 1) or Q (pass 2) rows,
// L / GK edges per instruction, and the whole segment gathers one V (pass 1)
// or dOut (pass 2) row per instruction, E edges per step.  The indices of a
// block of L edges are loaded one per lane and handed out by ds_bpermute.
// The scores are broadcast to the whole segment, so the running maximum and
// sum are segment-wide and the sub-groups' K-side sums merge by addition.
// Lanes past a row's end gather row 0 (valid) and get weight 0.  The binning
// keeps rows of similar degree together (8 log2-degree light buckets).
#ifndef AS_BWD_GROUPED_BATCH_Q
#define AS_BWD_GROUPED_BATCH_Q 4
#endif
#ifndef AS_BWD_GROUPED_BATCH_KV
#define AS_BWD_GROUPED_BATCH_KV 4
#endif

template <typename T, int GK, int GV>
constexpr bool bwd_grouped() {
  return sizeof(T) == 2 && GK <= GV && GV <= 16;
}

// Row, start and degree of this lane's segment of a wave starting at item0,
// and the largest degree over the wave's segments (wave-uniform).
struct SegRow {
  int64_t row;
  int64_t rs;
  int deg;
  int maxdeg;
};

template <int L>
__device__ __forceinline__ SegRow segment_row(const int32_t* __restrict__ order, const int64_t* __restrict__ crow,
                                              int64_t item0, int64_t end) {
  const int seg = lane_id() / L;
  SegRow r{-1, 0, 0, 0};
  const int64_t item = item0 + seg;
  if (item < end) {
    r.row = order[item];
    r.rs = crow[r.row];
    r.deg = static_cast<int>(crow[r.row + 1] - r.rs);  // below the slicing degree
  }
  int maxdeg = r.deg;
#pragma unroll
  for (int o = L; o < kWave; o <<= 1) maxdeg = max(maxdeg, __shfl_xor(maxdeg, o, kWave));
  r.maxdeg = uniform_i32(maxdeg);
  return r;
}

// P elements of row `row` at feature P·idx as fp32, zero for no row or past
// the feature end.
template <typename T>
__device__ __forceinline__ void seg_lane_row(const T* __restrict__ base, int64_t row, int64_t f, int idx,
                                             float (&out)[lane_elems<T>()]) {
  constexpr int P = lane_elems<T>();
  if (row >= 0 && P * idx < f) {
    lane_values<T>(load_raw<16>(reinterpret_cast<const char*>(base + row * f + P * idx)), out);
  } else {
#pragma unroll
    for (int v = 0; v < P; ++v) out[v] = 0.f;
  }
}

// Pass 1 for the rows order[item0, item0 + 64 / GV) (16-bit, t summed).
template <typename T, int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void bwd_q_rows_grouped(const BwdArgs<T>& a, int64_t item0, int64_t end) {
  constexpr int P = lane_elems<T>();
  constexpr int L = GV;
  constexpr int EKS = L / GK;  // K edges per instruction per row
  constexpr int E = AS_BWD_GROUPED_BATCH_Q;
  static_assert(sums_t<T>() && GK <= GV && GV <= 16 && L % E == 0 && E % EKS == 0, "grouped 16-bit rows");
  const int64_t fqk = FQK > 0 ? FQK : a.fqk;
  const int64_t fv = FV > 0 ? FV : a.fv;
  const int lane = lane_id();
  const int seg = lane / L;
  const int sl = lane % L;
  const int kg = sl / GK;
  const int kl = sl % GK;
  const SegRow sr = segment_row<L>(a.order, a.crow, item0, end);
  float q[P], g[P];
  seg_lane_row<T>(a.q, sr.row, fqk, kl, q);
  seg_lane_row<T>(a.g, sr.row, fv, sl, g);
  const char* __restrict__ kb = reinterpret_cast<const char*>(a.k);
  const char* __restrict__ vb = reinterpret_cast<const char*>(a.v);
  const uint32_t kbytes = static_cast<uint32_t>((P * kl < fqk ? P * kl : 0) * sizeof(T));
  const uint32_t vbytes = static_cast<uint32_t>((P * sl < fv ? P * sl : 0) * sizeof(T));
  float m = -INFINITY, l = 0.f, tsum = 0.f;
  float acc[P], acc2[P];
#pragma unroll
  for (int v = 0; v < P; ++v) {
    acc[v] = 0.f;
    acc2[v] = 0.f;
  }
  for (int base = 0; base < sr.maxdeg; base += L) {
    int my_col = 0;
    if (base + sl < sr.deg) my_col = static_cast<int>(a.col[sr.rs + base + sl]);
    const int cnt = sr.deg - base;  // edges of this segment's row in the block (may be <= 0)
    const int lim = sr.maxdeg - base < L ? sr.maxdeg - base : L;
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
        float x[P];
        lane_values<T>(kv[i], x);
        sk[i] = row_dot<GK, P>(q, x) * a.scale;
      }
      float s[E], dp[E];
      float mb = -INFINITY;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        float x[P];
        lane_values<T>(vv[i], x);
        dp[i] = row_dot<L, P>(g, x);
        // edge j + i sits in K instruction i / EKS, sub-group i % EKS
        const float se = __shfl(sk[i / EKS], seg * L + (i % EKS) * GK, kWave);
        s[i] = j + i < cnt ? se : -INFINITY;
        mb = fmaxf(mb, s[i]);
      }
      const float mn = fmaxf(m, mb);
      if (mn != -INFINITY) {
        const float corr = m == -INFINITY ? 0.f : expf(m - mn);
        l *= corr;
        tsum *= corr;
#pragma unroll
        for (int v = 0; v < P; ++v) {
          acc[v] *= corr;
          acc2[v] *= corr;
        }
        float p[E];
#pragma unroll
        for (int i = 0; i < E; ++i) {
          p[i] = s[i] == -INFINITY ? 0.f : expf(s[i] - mn);
          l += p[i];
          tsum = __builtin_fmaf(p[i], dp[i], tsum);
        }
        // K instruction i holds edge i·EKS + kg in sub-group kg
#pragma unroll
        for (int i = 0; i < E / EKS; ++i) {
          float pe = 0.f, de = 0.f;
#pragma unroll
          for (int gg = 0; gg < EKS; ++gg) {
            pe = kg == gg ? p[i * EKS + gg] : pe;
            de = kg == gg ? dp[i * EKS + gg] : de;
          }
          const float w = pe * de;
          float x[P];
          lane_values<T>(kv[i], x);
#pragma unroll
          for (int v = 0; v < P; ++v) {
            acc[v] = __builtin_fmaf(w, x[v], acc[v]);
            acc2[v] = __builtin_fmaf(pe, x[v], acc2[v]);
          }
        }
        m = mn;
      }
    }
  }
  // the sub-groups' K-side sums (one maximum across the segment)
#pragma unroll
  for (int o = GK; o < L; o <<= 1) {
#pragma unroll
    for (int v = 0; v < P; ++v) {
      acc[v] += __shfl_xor(acc[v], o, kWave);
      acc2[v] += __shfl_xor(acc2[v], o, kWave);
    }
  }
  if (sr.row < 0) return;
  const float t = l > 0.f ? tsum / l : 0.f;
  if (kg == 0 && P * kl < fqk) {
    float o[P];
#pragma unroll
    for (int v = 0; v < P; ++v) o[v] = l > 0.f ? a.scale * (acc[v] - t * acc2[v]) / l : 0.f;
    store_out<T, P>(a.dq + sr.row * fqk + P * kl, o);
  }
  if (sl == 0) a.lt[sr.row] = make_float2(l > 0.f ? m + logf(l) : -INFINITY, t);
}

// Pass 2 for the rows order[item0, item0 + 64 / GV) of Aᵀ (16-bit).
template <typename T, int GK, int GV, int FQK, int FV>
__device__ __forceinline__ void bwd_kv_rows_grouped(const BwdArgs<T>& a, int64_t item0, int64_t end) {
  constexpr int P = lane_elems<T>();
  constexpr int L = GV;
  constexpr int EKS = L / GK;
  constexpr int E = AS_BWD_GROUPED_BATCH_KV;
  static_assert(GK <= GV && GV <= 16 && L % E == 0 && E % EKS == 0, "grouped 16-bit rows");
  const int64_t fqk = FQK > 0 ? FQK : a.fqk;
  const int64_t fv = FV > 0 ? FV : a.fv;
  const int lane = lane_id();
  const int seg = lane / L;
  const int sl = lane % L;
  const int kg = sl / GK;
  const int kl = sl % GK;
  const SegRow sr = segment_row<L>(a.order, a.crow, item0, end);
  float kc[P], vc[P];
  seg_lane_row<T>(a.k, sr.row, fqk, kl, kc);
  seg_lane_row<T>(a.v, sr.row, fv, sl, vc);
  const char* __restrict__ qb = reinterpret_cast<const char*>(a.q);
  const char* __restrict__ gb = reinterpret_cast<const char*>(a.g);
  const uint32_t kbytes = static_cast<uint32_t>((P * kl < fqk ? P * kl : 0) * sizeof(T));
  const uint32_t vbytes = static_cast<uint32_t>((P * sl < fv ? P * sl : 0) * sizeof(T));
  float dk[P], dv[P];
#pragma unroll
  for (int v = 0; v < P; ++v) {
    dk[v] = 0.f;
    dv[v] = 0.f;
  }
  for (int base = 0; base < sr.maxdeg; base += L) {
    // the block's sources and their (lse, t), one edge per lane
    int my_src = 0;
    float my_lse = 0.f, my_t = 0.f;
    if (base + sl < sr.deg) {
      my_src = static_cast<int>(a.col[sr.rs + base + sl]);
      const float2 w = a.lt[my_src];
      my_lse = w.x;
      my_t = w.y;
    }
    const int cnt = sr.deg - base;
    const int lim = sr.maxdeg - base < L ? sr.maxdeg - base : L;
    for (int j = 0; j < lim; j += E) {
      RawVec<16> qv[E / EKS];
      RawVec<16> gv[E];
#pragma unroll
      for (int i = 0; i < E / EKS; ++i) {
        const int r = __builtin_amdgcn_ds_bpermute((seg * L + j + i * EKS + kg) * 4, my_src);
        qv[i] = load_raw<16>(qb + row_offset(r, fqk) * sizeof(T) + kbytes);
      }
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int r = __builtin_amdgcn_ds_bpermute((seg * L + j + i) * 4, my_src);
        gv[i] = load_raw<16>(gb + row_offset(r, fv) * sizeof(T) + vbytes);
      }
      // per edge of the step (segment-wide): dP, lse, t
      float dp[E], lse[E], tt[E];
#pragma unroll
      for (int i = 0; i < E; ++i) {
        float x[P];
        lane_values<T>(gv[i], x);
        dp[i] = row_dot<L, P>(vc, x);
        const int from = (seg * L + j + i) * 4;
        lse[i] = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(my_lse)));
        tt[i] = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(my_t)));
      }
      // scores in the K sub-groups, broadcast to the segment
      float sk[E / EKS];
#pragma unroll
      for (int i = 0; i < E / EKS; ++i) {
        float x[P];
        lane_values<T>(qv[i], x);
        sk[i] = row_dot<GK, P>(kc, x) * a.scale;
      }
      float p[E];
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float se = __shfl(sk[i / EKS], seg * L + (i % EKS) * GK, kWave);
        p[i] = j + i < cnt ? expf(se - lse[i]) : 0.f;
      }
      // dK: K instruction i holds edge i·EKS + kg in sub-group kg
#pragma unroll
      for (int i = 0; i < E / EKS; ++i) {
        float ds = 0.f;
#pragma unroll
        for (int gg = 0; gg < EKS; ++gg) {
          const int e = i * EKS + gg;
          ds = kg == gg ? a.scale * p[e] * (dp[e] - tt[e]) : ds;
        }
        float x[P];
        lane_values<T>(qv[i], x);
#pragma unroll
        for (int v = 0; v < P; ++v) dk[v] = __builtin_fmaf(ds, x[v], dk[v]);
      }
      // dV: every edge of the step over the whole segment
#pragma unroll
      for (int i = 0; i < E; ++i) {
        float x[P];
        lane_values<T>(gv[i], x);
#pragma unroll
        for (int v = 0; v < P; ++v) dv[v] = __builtin_fmaf(p[i], x[v], dv[v]);
      }
    }
  }
#pragma unroll
  for (int o = GK; o < L; o <<= 1) {
#pragma unroll
    for (int v = 0; v < P; ++v) dk[v] += __shfl_xor(dk[v], o, kWave);
  }
  if (sr.row < 0) return;
  if (kg == 0 && P * kl < fqk) store_out<T, P>(a.dk + sr.row * fqk + P * kl, dk);
  if (P * sl < fv) store_out<T, P>(a.dv + sr.row * fv + P * sl, dv);
}

// ---- pass 1: dQ and (lse, t) over the rows of A ----

// t of a row for fp32 (from the output row); 0 for 16-bit (summed in the pass)
template <typename T, int GV>
__device__ __forceinline__ float output_t(const BwdArgs<T>& a, int64_t row, const float (&g)[lane_elems<T>()]) {
  if constexpr (sums_t<T>()) {
    return 0.f;
  } else {
    float o[lane_elems<T>()];
    load_query_lanes<T, GV>(a.out, row, a.fv, o);
    return row_dot<GV, lane_elems<T>()>(g, o);
  }
}

template <typename T, int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdq_rows_kernel(BwdArgs<T> a) {
  constexpr int P = lane_elems<T>();
  constexpr bool TWO = sums_t<T>();
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  if constexpr (bwd_grouped<T, GK, GV>()) {
    constexpr int64_t kRows = kWave / GV;
    const int64_t w = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    for (int64_t item0 = a.counts[0] + w * kRows; item0 < a.n; item0 += waves * kRows)
      bwd_q_rows_grouped<T, GK, GV, FQK, FV>(a, item0, a.n);
    return;
  }
  const int lane = lane_id();
  for (int64_t item = a.counts[0] + static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block(); item < a.n;
       item += waves) {
    const int64_t row = uniform_i64(a.order[item]);
    float q[P], g[P];
    load_query_lanes<T, GK>(a.q, row, a.fqk, q);
    load_query_lanes<T, GV>(a.g, row, a.fv, g);
    float t = output_t<T, GV>(a, row, g);
    QState<P, TWO> st;
    bwd_q_edges<T, GK, GV, FQK, FV>(a.col, a.k, a.v, a.fqk, a.fv, q, g, t, a.scale, a.crow[row], a.crow[row + 1],
                                    st);
    if constexpr (TWO) t = st.l > 0.f ? st.tsum / st.l : 0.f;
    if (lane < GK && P * lane < a.fqk) {
      float o[P];
#pragma unroll
      for (int v = 0; v < P; ++v) {
        const float num = TWO ? st.acc[v] - t * st.acc2[TWO ? v : 0] : st.acc[v];
        o[v] = st.l > 0.f ? a.scale * num / st.l : 0.f;
      }
      store_out<T, P>(a.dq + row * a.fqk + P * lane, o);
    }
    if (lane == 0) a.lt[row] = make_float2(st.l > 0.f ? st.m + logf(st.l) : -INFINITY, t);
  }
}

// Partial states of pass 1: m, l, tsum per (slice, row), then acc (and acc2)
// rows of F_qk floats.
struct QParts {
  float* m;
  float* l;
  float* t;
  float* acc;
  float* acc2;
};

template <typename T, int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdq_slice_kernel(BwdArgs<T> a, int64_t begin, int64_t items,
                                                            int64_t stride, QParts pp) {
  constexpr int P = lane_elems<T>();
  constexpr bool TWO = sums_t<T>();
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
    float q[P], g[P];
    load_query_lanes<T, GK>(a.q, row, a.fqk, q);
    load_query_lanes<T, GV>(a.g, row, a.fv, g);
    const float t = output_t<T, GV>(a, row, g);
    QState<P, TWO> st;
    bwd_q_edges<T, GK, GV, FQK, FV>(a.col, a.k, a.v, a.fqk, a.fv, q, g, t, a.scale, rs + lo, rs + hi, st);
    const int64_t at = slice * stride + local;
    // fp32: the row's t, once (the reduction writes its lse)
    if (!TWO && slice == 0 && lane == 0) a.lt[row].y = t;
    if (lane < GK && P * lane < a.fqk) {
      store_out<float, P>(pp.acc + at * a.fqk + P * lane, st.acc);
      if constexpr (TWO) store_out<float, P>(pp.acc2 + at * a.fqk + P * lane, st.acc2);
    }
    if (lane == 0) {
      pp.m[at] = st.m;
      pp.l[at] = st.l;
      if constexpr (TWO) pp.t[at] = st.tsum;
    }
  }
}

// Merge of the 8 partial states of each sliced row; thread per (row, 4
// features); the thread of features 0-3 also writes lse (and, for 16-bit, t).
template <typename T>
__global__ __launch_bounds__(kBlock) void bwdq_reduce_kernel(BwdArgs<T> a, int64_t begin, int64_t items,
                                                             int64_t stride, QParts pp) {
  constexpr bool TWO = sums_t<T>();
  const int64_t F4 = a.fqk / 4;
  const int64_t total = items * F4;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += step) {
    const int64_t local = i / F4;
    const int64_t f = (i - local * F4) * 4;
    if (begin + local >= a.counts[0]) continue;
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < kSlices; ++s) m = fmaxf(m, pp.m[s * stride + local]);
    float l = 0.f;
    float tsum = 0.f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float acc2[4] = {0.f, 0.f, 0.f, 0.f};
    if (m != -INFINITY) {
#pragma unroll
      for (int s = 0; s < kSlices; ++s) {
        const float ms = pp.m[s * stride + local];
        if (ms == -INFINITY) continue;
        const float c = expf(ms - m);
        l = __builtin_fmaf(c, pp.l[s * stride + local], l);
        const FVec<4> p = load_vec<4>(pp.acc + (s * stride + local) * a.fqk + f);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(c, p.v[v], acc[v]);
        if constexpr (TWO) {
          tsum = __builtin_fmaf(c, pp.t[s * stride + local], tsum);
          const FVec<4> p2 = load_vec<4>(pp.acc2 + (s * stride + local) * a.fqk + f);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc2[v] = __builtin_fmaf(c, p2.v[v], acc2[v]);
        }
      }
    }
    const int64_t row = a.order[begin + local];
    const float t = TWO && l > 0.f ? tsum / l : 0.f;
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float num = TWO ? acc[v] - t * acc2[v] : acc[v];
      o[v] = l > 0.f ? a.scale * num / l : 0.f;
    }
    store_out<T, 4>(a.dq + row * a.fqk + f, o);
    if (f == 0) {
      const float lse = l > 0.f ? m + logf(l) : -INFINITY;
      if constexpr (TWO) a.lt[row] = make_float2(lse, t);
      else a.lt[row].x = lse;
    }
  }
}

// ---- pass 2: dK and dV over the rows of Aᵀ ----

template <typename T, int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdkv_rows_kernel(BwdArgs<T> a) {
  constexpr int P = lane_elems<T>();
  const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  if constexpr (bwd_grouped<T, GK, GV>()) {
    constexpr int64_t kRows = kWave / GV;
    const int64_t w = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
    for (int64_t item0 = a.counts[0] + w * kRows; item0 < a.n; item0 += waves * kRows)
      bwd_kv_rows_grouped<T, GK, GV, FQK, FV>(a, item0, a.n);
    return;
  }
  const int lane = lane_id();
  for (int64_t item = a.counts[0] + static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block(); item < a.n;
       item += waves) {
    const int64_t row = uniform_i64(a.order[item]);
    float kc[P], vc[P];
    load_query_lanes<T, GK>(a.k, row, a.fqk, kc);
    load_query_lanes<T, GV>(a.v, row, a.fv, vc);
    float dk[P], dv[P];
    bwd_kv_edges<T, GK, GV, FQK, FV>(a.col, a.q, a.g, a.lt, a.fqk, a.fv, kc, vc, a.scale, a.crow[row],
                                     a.crow[row + 1], dk, dv);
    if (lane < GK && P * lane < a.fqk) store_out<T, P>(a.dk + row * a.fqk + P * lane, dk);
    if (lane < GV && P * lane < a.fv) store_out<T, P>(a.dv + row * a.fv + P * lane, dv);
  }
}

template <typename T, int GK, int GV, int FQK, int FV>
__global__ __launch_bounds__(kBlock) void bwdkv_slice_kernel(BwdArgs<T> a, int64_t begin, int64_t items,
                                                             int64_t stride, float* __restrict__ pk,
                                                             float* __restrict__ pv) {
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
    float kc[P], vc[P];
    load_query_lanes<T, GK>(a.k, row, a.fqk, kc);
    load_query_lanes<T, GV>(a.v, row, a.fv, vc);
    float dk[P], dv[P];
    bwd_kv_edges<T, GK, GV, FQK, FV>(a.col, a.q, a.g, a.lt, a.fqk, a.fv, kc, vc, a.scale, rs + lo, rs + hi, dk, dv);
    const int64_t at = slice * stride + local;
    if (lane < GK && P * lane < a.fqk) store_out<float, P>(pk + at * a.fqk + P * lane, dk);
    if (lane < GV && P * lane < a.fv) store_out<float, P>(pv + at * a.fv + P * lane, dv);
  }
}

// Sums of the 8 partials of each sliced row of Aᵀ, in slice order; thread per
// (row, 4 features) over the F_qk + F_v features of dK and dV.
template <typename T>
__global__ __launch_bounds__(kBlock) void bwdkv_reduce_kernel(BwdArgs<T> a, int64_t begin, int64_t items,
                                                              int64_t stride, const float* __restrict__ pk,
                                                              const float* __restrict__ pv) {
  const int64_t K4 = a.fqk / 4;
  const int64_t F4 = K4 + a.fv / 4;
  const int64_t total = items * F4;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += step) {
    const int64_t local = i / F4;
    const int64_t q4 = i - local * F4;
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
    store_out<T, 4>((is_k ? a.dk : a.dv) + row * width + f, acc);
  }
}

// Per sliced row of a chunk: pass 1 keeps 8 x (m, l, t, F_qk or 2·F_qk
// accumulators), pass 2 8 x (F_qk + F_v) floats.
size_t bwd_row_bytes(int64_t fqk, int64_t fv, bool two) {
  const size_t p1 = static_cast<size_t>(fqk) * (two ? 2 : 1) + 3;
  const size_t p2 = static_cast<size_t>(fqk) + static_cast<size_t>(fv);
  return static_cast<size_t>(kSlices) * (p1 > p2 ? p1 : p2) * sizeof(float);
}

// (lse, t) pairs, then a slice plan region for passes called without a plan
size_t bwd_pairs_bytes(int64_t n) { return align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(float2), 256); }
size_t bwd_fixed_bytes(int64_t n) { return bwd_pairs_bytes(n) + slice_plan_bytes(n); }

// Upper bound on the rows of degree >= `degree` (the sliced rows).
int64_t bwd_sliced_upper(int64_t n, int64_t nnz, int64_t degree) {
  const int64_t u = nnz / degree;
  return u < n ? u : n;
}

// Slack for the alignment of the partial arrays within a chunk's buffer.
constexpr size_t kBwdPartSlack = 5 * 256;

// Workgroups of a rows kernel: one wave per row, or per 64 / GV grouped rows.
template <typename T, int GK, int GV>
int64_t rows_blocks(int64_t n) {
  const int64_t rows_per_wave = bwd_grouped<T, GK, GV>() ? kWave / GV : 1;
  const int64_t per_block = kWavesPerBlock * rows_per_wave;
  const int64_t b = (n + per_block - 1) / per_block;
  return b > kMaxBlocksPerLaunch ? kMaxBlocksPerLaunch : b;
}

template <typename T, int GK, int GV, int FQK = 0, int FV = 0>
void launch_pass1(const BwdArgs<T>& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  const int64_t row_blocks = rows_blocks<T, GK, GV>(a.n);
  hipLaunchKernelGGL((bwdq_rows_kernel<T, GK, GV, FQK, FV>), dim3(static_cast<unsigned>(row_blocks)), dim3(kBlock), 0,
                     s, a);
  const size_t states = static_cast<size_t>(kSlices) * static_cast<size_t>(chunk);
  const size_t accs = states * static_cast<size_t>(a.fqk);
  QParts pp;
  pp.m = part;
  pp.l = pp.m + align_up(states, 64);
  pp.t = pp.l + align_up(states, 64);
  pp.acc = pp.t + align_up(states, 64);
  pp.acc2 = pp.acc + align_up(accs, 64);
  for (int64_t begin = 0; begin < upper; begin += chunk) {
    const int64_t items = upper - begin < chunk ? upper - begin : chunk;
    int64_t per_slice = (items + kWavesPerBlock - 1) / kWavesPerBlock;
    if (per_slice > kBwdSliceBlocks) per_slice = kBwdSliceBlocks;
    hipLaunchKernelGGL((bwdq_slice_kernel<T, GK, GV, FQK, FV>), dim3(static_cast<unsigned>(kSlices * per_slice)),
                       dim3(kBlock), 0, s, a, begin, items, chunk, pp);
    int64_t blocks = (items * (a.fqk / 4) + kBlock - 1) / kBlock;
    if (blocks > kBwdReduceBlocks) blocks = kBwdReduceBlocks;
    hipLaunchKernelGGL((bwdq_reduce_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, a, begin,
                       items, chunk, pp);
  }
}

template <typename T, int GK, int GV, int FQK = 0, int FV = 0>
void launch_pass2(const BwdArgs<T>& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  const int64_t row_blocks = rows_blocks<T, GK, GV>(a.n);
  hipLaunchKernelGGL((bwdkv_rows_kernel<T, GK, GV, FQK, FV>), dim3(static_cast<unsigned>(row_blocks)), dim3(kBlock),
                     0, s, a);
  const size_t states = static_cast<size_t>(kSlices) * static_cast<size_t>(chunk);
  float* pk = part;
  float* pv = part + align_up(states * static_cast<size_t>(a.fqk), 64);
  for (int64_t begin = 0; begin < upper; begin += chunk) {
    const int64_t items = upper - begin < chunk ? upper - begin : chunk;
    int64_t per_slice = (items + kWavesPerBlock - 1) / kWavesPerBlock;
    if (per_slice > kBwdSliceBlocks) per_slice = kBwdSliceBlocks;
    hipLaunchKernelGGL((bwdkv_slice_kernel<T, GK, GV, FQK, FV>), dim3(static_cast<unsigned>(kSlices * per_slice)),
                       dim3(kBlock), 0, s, a, begin, items, chunk, pk, pv);
    int64_t blocks = (items * ((a.fqk + a.fv) / 4) + kBlock - 1) / kBlock;
    if (blocks > kBwdReduceBlocks) blocks = kBwdReduceBlocks;
    hipLaunchKernelGGL((bwdkv_reduce_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, a, begin,
                       items, chunk, pk, pv);
  }
}

template <int PASS, typename T, int GK, int GV, int FQK = 0, int FV = 0>
void launch_pass(const BwdArgs<T>& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  if constexpr (PASS == 1) launch_pass1<T, GK, GV, FQK, FV>(a, upper, chunk, part, s);
  else launch_pass2<T, GK, GV, FQK, FV>(a, upper, chunk, part, s);
}

template <int PASS, typename T, int GK>
void dispatch_gv(int gv, const BwdArgs<T>& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  switch (gv) {
    case 8:
      if constexpr (sizeof(T) == 2) launch_pass<PASS, T, GK, 8>(a, upper, chunk, part, s);
      break;
    case 16: launch_pass<PASS, T, GK, 16>(a, upper, chunk, part, s); break;
    case 32: launch_pass<PASS, T, GK, 32>(a, upper, chunk, part, s); break;
    default: launch_pass<PASS, T, GK, 64>(a, upper, chunk, part, s); break;
  }
}

template <int PASS, typename T>
void dispatch_pass(const BwdArgs<T>& a, int64_t upper, int64_t chunk, float* part, hipStream_t s) {
  constexpr bool kHalf = sizeof(T) == 2;
  // common widths with compile-time strides
  if (a.fqk == 64 && a.fv == 128)
    return launch_pass<PASS, T, kHalf ? 8 : 16, kHalf ? 16 : 32, 64, 128>(a, upper, chunk, part, s);
  if (a.fqk == 64 && a.fv == 64)
    return launch_pass<PASS, T, kHalf ? 8 : 16, kHalf ? 8 : 16, 64, 64>(a, upper, chunk, part, s);
  if (a.fqk == 128 && a.fv == 128)
    return launch_pass<PASS, T, kHalf ? 16 : 32, kHalf ? 16 : 32, 128, 128>(a, upper, chunk, part, s);
  const int gv = lane_group<T>(a.fv);
  switch (lane_group<T>(a.fqk)) {
    case 8:
      if constexpr (kHalf) dispatch_gv<PASS, T, 8>(gv, a, upper, chunk, part, s);
      break;
    case 16: dispatch_gv<PASS, T, 16>(gv, a, upper, chunk, part, s); break;
    case 32: dispatch_gv<PASS, T, 32>(gv, a, upper, chunk, part, s); break;
    default: dispatch_gv<PASS, T, 64>(gv, a, upper, chunk, part, s); break;
  }
}

// Both entry points after their element-specific checks.
template <typename T>
int backward_run(const int64_t* crow, const int64_t* col, const int64_t* crow_t, const int64_t* col_t,
                 const T* query, const T* key, const T* value, const T* out, const T* grad_out, T* grad_q, T* grad_k,
                 T* grad_v, int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v, float scale, const void* plan,
                 int64_t plan_tag, const void* plan_t, int64_t plan_t_tag, void* workspace, size_t workspace_bytes,
                 void* stream) {
  // 16-bit: short rows in 8 log2-degree buckets (the grouped rows), as in the
  // forward's plan
  constexpr int kLight = sums_t<T>() ? kMaxHeavyBuckets : 1;
  // the forward's slicing degree: the two share the per-graph plans
  constexpr int64_t kDegree = att_slice_degree<T>();
  const int64_t want = slice_plan_tag(kDegree, kLight);
  if ((plan != nullptr && plan_tag != want) || (plan_t != nullptr && plan_t_tag != want))
    return fail(AS_ERR_INVALID_ARGUMENT, "a plan was built for other settings (this call needs plan tag %lld)",
                (long long)want);
  if ((plan != nullptr && !aligned(plan, 256)) || (plan_t != nullptr && !aligned(plan_t, 256)))
    return fail(AS_ERR_WORKSPACE, "plans must be 256-byte aligned");
  if (n == 0) return AS_OK;
  // the output row is read for fp32 only (16-bit sums t in pass 1)
  if (crow == nullptr || crow_t == nullptr || query == nullptr || key == nullptr || value == nullptr ||
      (!sums_t<T>() && out == nullptr) || grad_out == nullptr || grad_q == nullptr || grad_k == nullptr ||
      grad_v == nullptr || (nnz > 0 && (col == nullptr || col_t == nullptr)))
    return fail(AS_ERR_INVALID_ARGUMENT, "null pointer argument");
  for (const void* p : {static_cast<const void*>(query), static_cast<const void*>(key), static_cast<const void*>(value),
                        static_cast<const void*>(out), static_cast<const void*>(grad_out),
                        static_cast<const void*>(grad_q), static_cast<const void*>(grad_k),
                        static_cast<const void*>(grad_v)})
    if (!aligned(p, 16)) return fail(AS_ERR_UNSUPPORTED, "attention backward needs 16-byte aligned tensors");
  // the workspace holds a plan region only for a pass called without a plan
  const bool own_plan = plan == nullptr || plan_t == nullptr;
  const size_t fixed = own_plan ? bwd_fixed_bytes(n) : bwd_pairs_bytes(n);
  const size_t row_bytes = bwd_row_bytes(f_qk, f_v, sums_t<T>());
  if (workspace == nullptr || workspace_bytes < fixed + row_bytes + kBwdPartSlack)
    return fail(AS_ERR_WORKSPACE, "attention backward needs at least %zu workspace bytes, got %zu",
                fixed + row_bytes + kBwdPartSlack, workspace_bytes);
  if (!aligned(workspace, 256)) return fail(AS_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  const int64_t upper = bwd_sliced_upper(n, nnz, kDegree);
  int64_t chunk = static_cast<int64_t>((workspace_bytes - fixed - kBwdPartSlack) / row_bytes);
  if (chunk > kBwdChunkRows) chunk = kBwdChunkRows;
  if (chunk > upper) chunk = upper;
  if (chunk < 1) chunk = 1;

  const hipStream_t s = static_cast<hipStream_t>(stream);
  float2* lt = static_cast<float2*>(workspace);
  void* own = static_cast<char*>(workspace) + bwd_pairs_bytes(n);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + fixed);

  // pass 1 over A; then pass 2 over Aᵀ.  A pass without a plan builds one in
  // the workspace's plan region (pass 2 after pass 1 in stream order)
  for (int pass = 1; pass <= 2; ++pass) {
    const int64_t* pc = pass == 1 ? crow : crow_t;
    const int64_t* pcol = pass == 1 ? col : col_t;
    const void* given = pass == 1 ? plan : plan_t;
    const SlicePlan view = slice_plan_view(given != nullptr ? const_cast<void*>(given) : own, n);
    if (given == nullptr) {
      const int st = build_slice_plan(pc, pcol, n, kDegree, kLight, false, view, s);
      if (st != AS_OK) return st;
    }
    const BwdArgs<T> a{pc,     pcol,   query, key,  value, grad_out, out,        lt,          grad_q,
                       grad_k, grad_v, n,     f_qk, f_v,   scale,    view.order, view.counts, view.off};
    if (pass == 1) dispatch_pass<1, T>(a, upper, chunk, part, s);
    else dispatch_pass<2, T>(a, upper, chunk, part, s);
  }
  return check_launch(sums_t<T>() ? "csr_attention_backward (16-bit)" : "csr_attention_backward");
}

}  // namespace

}  // namespace as

extern "C" {

size_t as_csr_attention_backward_workspace_bytes(int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v, int dtype) {
  if (n < 0) n = 0;
  if (nnz < 0) nnz = 0;
  if (f_qk < 4) f_qk = 4;
  if (f_v < 4) f_v = 4;
  int64_t rows = as::bwd_sliced_upper(
      n, nnz, dtype == AS_DTYPE_F32 ? as::att_slice_degree<float>() : as::att_slice_degree<as::Bf16>());
  if (rows > as::kBwdChunkRows) rows = as::kBwdChunkRows;
  if (rows < 1) rows = 1;
  return as::bwd_fixed_bytes(n) + static_cast<size_t>(rows) * as::bwd_row_bytes(f_qk, f_v, dtype != AS_DTYPE_F32) +
         as::kBwdPartSlack;
}

int as_csr_attention_backward_f32(const int64_t* crow, const int64_t* col, const int64_t* crow_t,
                                  const int64_t* col_t, const float* query, const float* key, const float* value,
                                  const float* out, const float* grad_out, float* grad_q, float* grad_k,
                                  float* grad_v, int64_t n, int64_t nnz, int64_t f_qk, int64_t f_v, float scale,
                                  const void* plan, int64_t plan_tag, const void* plan_t, int64_t plan_t_tag,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  as::clear_error();
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (f_qk < 4 || f_qk > 256 || f_qk % 4 != 0 || f_v < 4 || f_v > 256 || f_v % 4 != 0)
    return as::fail(AS_ERR_UNSUPPORTED, "attention backward needs F_qk and F_v in [4, 256], multiples of 4");
  return as::backward_run<float>(crow, col, crow_t, col_t, query, key, value, out, grad_out, grad_q, grad_k, grad_v,
                                 n, nnz, f_qk, f_v, scale, plan, plan_tag, plan_t, plan_t_tag, workspace,
                                 workspace_bytes, stream);
}

int as_csr_attention_backward_16(const int64_t* crow, const int64_t* col, const int64_t* crow_t, const int64_t* col_t,
                                 const void* query, const void* key, const void* value, const void* grad_out,
                                 void* grad_q, void* grad_k, void* grad_v, int64_t n, int64_t nnz, int64_t f_qk,
                                 int64_t f_v, float scale, int dtype, const void* plan, int64_t plan_tag,
                                 const void* plan_t, int64_t plan_t_tag, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  as::clear_error();
  if (dtype != AS_DTYPE_BF16 && dtype != AS_DTYPE_F16)
    return as::fail(AS_ERR_INVALID_ARGUMENT, "dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16");
  if (n < 0 || n > INT32_MAX) return as::fail(AS_ERR_INVALID_ARGUMENT, "N exceeds kernel index range");
  if (nnz < 0) return as::fail(AS_ERR_INVALID_ARGUMENT, "nnz must be non-negative");
  if (f_qk < 8 || f_qk > 512 || f_qk % 8 != 0 || f_v < 8 || f_v > 512 || f_v % 8 != 0)
    return as::fail(AS_ERR_UNSUPPORTED, "16-bit attention backward needs F_qk and F_v in [8, 512], multiples of 8");
  // 16-bit: t is summed in pass 1 and the output row is never read (query
  // stands in for it in the pointer checks)
  if (dtype == AS_DTYPE_BF16)
    return as::backward_run<as::Bf16>(
        crow, col, crow_t, col_t, static_cast<const as::Bf16*>(query), static_cast<const as::Bf16*>(key),
        static_cast<const as::Bf16*>(value), static_cast<const as::Bf16*>(query),
        static_cast<const as::Bf16*>(grad_out), static_cast<as::Bf16*>(grad_q), static_cast<as::Bf16*>(grad_k),
        static_cast<as::Bf16*>(grad_v), n, nnz, f_qk, f_v, scale, plan, plan_tag, plan_t, plan_t_tag, workspace,
        workspace_bytes, stream);
  return as::backward_run<as::Fp16>(
      crow, col, crow_t, col_t, static_cast<const as::Fp16*>(query), static_cast<const as::Fp16*>(key),
      static_cast<const as::Fp16*>(value), static_cast<const as::Fp16*>(query), static_cast<const as::Fp16*>(grad_out),
      static_cast<as::Fp16*>(grad_q), static_cast<as::Fp16*>(grad_k), static_cast<as::Fp16*>(grad_v), n, nnz, f_qk,
      f_v, scale, plan, plan_tag, plan_t, plan_t_tag, workspace, workspace_bytes, stream);
}

}  // extern "C"
