/*
 * CPU oracle for the AutoSAGE sparse hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Plain C restatement of the reference arithmetic, used as the checker by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in
 * the product (autosage_amd/) may link or call it.
 *
 * Every output element is computed independently in a fixed, documented
 * order; citations are to the AutoSAGE reference tree.
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf/fma call.  Built with OpenMP: the loops over rows run in parallel,
 * one row per thread at a time, so every element is computed by one thread
 * in the order stated and the results do not depend on the thread count.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

/* Y[r, f] = sum over edges e of row r, in CSR order, of w_e * X[col_e, f]
 * as one fp32 chain acc = fmaf(w, x, acc) from acc = 0 (w = 1 when val is
 * NULL).  This is the per-(row, feature) loop of the reference kernels
 * (csrc/spmm_csr_vec4.cu:42-50 and :75-88, csrc/spmm_rows.cu:58-69) and the
 * order of the reference CPU path torch.sparse.mm (autosage/ops.py:124-143).
 * rows == NULL: all n rows into y[n, f]; otherwise rows[0..nrows) into
 * y[nrows, f]. */
void or_spmm_seq_f32(const int64_t* crow, const int64_t* col, const float* val, const float* x, const int64_t* rows,
                     int64_t nrows, int64_t f, float* y) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t i = 0; i < nrows; ++i) {
    const int64_t r = rows ? rows[i] : i;
    float* out = y + i * f;
    for (int64_t k = 0; k < f; ++k) out[k] = 0.0f;
    for (int64_t e = crow[r]; e < crow[r + 1]; ++e) {
      const float* xr = x + col[e] * f;
      const float w = val ? val[e] : 1.0f;
      for (int64_t k = 0; k < f; ++k) out[k] = fmaf(w, xr[k], out[k]);
    }
  }
}

/* Same sums in fp64 (products and additions in double): the near-exact value
 * used to bound reassociating kernels. */
void or_spmm_f64(const int64_t* crow, const int64_t* col, const float* val, const float* x, const int64_t* rows,
                 int64_t nrows, int64_t f, double* y) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t i = 0; i < nrows; ++i) {
    const int64_t r = rows ? rows[i] : i;
    double* out = y + i * f;
    for (int64_t k = 0; k < f; ++k) out[k] = 0.0;
    for (int64_t e = crow[r]; e < crow[r + 1]; ++e) {
      const float* xr = x + col[e] * f;
      const double w = val ? (double)val[e] : 1.0;
      for (int64_t k = 0; k < f; ++k) out[k] += w * (double)xr[k];
    }
  }
}

/* Degree binning of csrc/launcher_spmm.cu:13-18,49-59: deg = crow[r+1]-crow[r];
 * heavy rows (deg >= threshold) and light rows, each ascending, as int32
 * (at::nonzero(...).flatten().toType(kInt)).  counts[0] = #heavy,
 * counts[1] = #light. */
void or_bin_rows(const int64_t* crow, int64_t n, int64_t threshold, int32_t* heavy, int32_t* light,
                 int64_t* counts) {
  int64_t h = 0, l = 0;
  for (int64_t r = 0; r < n; ++r) {
    if (crow[r + 1] - crow[r] >= threshold) heavy[h++] = (int32_t)r;
    else light[l++] = (int32_t)r;
  }
  counts[0] = h;
  counts[1] = l;
}

/* SDDMM dot in the reference kernel order (csrc/sddmm_csr_op.cu:39-49 and the
 * shuffle tree :12-17): 32 lane partials p_l = fmaf chain over features
 * l, l+32, l+64, ... (< F) from 0, then for o = 16, 8, 4, 2, 1:
 * p_l = p_l + p_{l+o} for l < o; the result is p_0. */
static float ref_dot(const float* q, const float* k, int64_t f) {
  float p[32];
  for (int l = 0; l < 32; ++l) {
    float s = 0.0f;
    for (int64_t j = l; j < f; j += 32) s = fmaf(q[j], k[j], s);
    p[l] = s;
  }
  for (int o = 16; o >= 1; o >>= 1)
    for (int l = 0; l < o; ++l) p[l] = p[l] + p[l + o];
  return p[0];
}

/* out[e] = <query[r], key[col[e]]> for every edge e of every row r
 * (csrc/sddmm_csr_op.cu:19-50 row kernel, :52-83 hub kernel: same dot). */
void or_sddmm_ref_f32(const int64_t* crow, const int64_t* col, const float* query, const float* key, int64_t n,
                      int64_t f, float* out) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < n; ++r)
    for (int64_t e = crow[r]; e < crow[r + 1]; ++e) out[e] = ref_dot(query + r * f, key + col[e] * f, f);
}

void or_sddmm_f64(const int64_t* crow, const int64_t* col, const float* query, const float* key, int64_t n,
                  int64_t f, double* out) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < n; ++r)
    for (int64_t e = crow[r]; e < crow[r + 1]; ++e) {
      const float* a = query + r * f;
      const float* b = key + col[e] * f;
      double s = 0.0;
      for (int64_t j = 0; j < f; ++j) s += (double)a[j] * (double)b[j];
      out[e] = s;
    }
}

/* Row softmax of autosage/_auto.py:744-759: m = max of the row's scores
 * (scatter_reduce amax), e_i = exp(s_i - m), d = sum of e_i in CSR order
 * (scatter_add), p_i = e_i / d.  Empty rows produce nothing. */
void or_row_softmax_f32(const int64_t* crow, const float* scores, int64_t n, float* probs) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < n; ++r) {
    const int64_t s0 = crow[r], s1 = crow[r + 1];
    if (s0 == s1) continue;
    float m = -INFINITY;
    for (int64_t e = s0; e < s1; ++e) m = scores[e] > m ? scores[e] : m;
    float d = 0.0f;
    for (int64_t e = s0; e < s1; ++e) d += expf(scores[e] - m);
    for (int64_t e = s0; e < s1; ++e) probs[e] = expf(scores[e] - m) / d;
  }
}

void or_row_softmax_f64(const int64_t* crow, const double* scores, int64_t n, double* probs) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < n; ++r) {
    const int64_t s0 = crow[r], s1 = crow[r + 1];
    if (s0 == s1) continue;
    double m = -INFINITY;
    for (int64_t e = s0; e < s1; ++e) m = scores[e] > m ? scores[e] : m;
    double d = 0.0;
    for (int64_t e = s0; e < s1; ++e) d += exp(scores[e] - m);
    for (int64_t e = s0; e < s1; ++e) probs[e] = exp(scores[e] - m) / d;
  }
}

/* Backward of the row softmax in the order the GPU kernel defines (the
 * reference registers no autograd; its torch composition,
 * autosage/_auto.py:744-759, has the same mathematical gradient):
 *   t = sum_e grad_e * p_e  as 64 lane partials (edge e of the row goes to
 *       lane (e - row start) mod 64, each lane an fmaf chain in edge order),
 *       then the butterfly v_l += v_{l xor o} for o = 32, 16, 8, 4, 2, 1;
 *   out_e = p_e * (grad_e - t). */
void or_row_softmax_backward_f32(const int64_t* crow, const float* probs, const float* grad, int64_t n,
                                 float* out) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < n; ++r) {
    const int64_t s0 = crow[r], s1 = crow[r + 1];
    if (s0 == s1) continue;
    float lane[64];
    for (int l = 0; l < 64; ++l) lane[l] = 0.0f;
    for (int64_t e = s0; e < s1; ++e) {
      const int l = (int)((e - s0) % 64);
      lane[l] = fmaf(grad[e], probs[e], lane[l]);
    }
    for (int o = 32; o > 0; o >>= 1) {
      float next[64];
      for (int l = 0; l < 64; ++l) next[l] = lane[l] + lane[l ^ o];
      for (int l = 0; l < 64; ++l) lane[l] = next[l];
    }
    const float t = lane[0];
    for (int64_t e = s0; e < s1; ++e) out[e] = probs[e] * (grad[e] - t);
  }
}

/* CSR attention in fp64 (autosage/_auto.py:762-780 with the scores scaled):
 * per row r, s_e = scale * <query[r], key[col_e]> (products and sums in
 * double, features in order), m = max s_e, p_e = exp(s_e - m) / sum exp,
 * out[r, j] = sum over the row's edges in CSR order of p_e * value[col_e, j].
 * Empty rows give zeros.  The near-exact value that bounds the fp32
 * attention kernels. */
void or_attention_f64(const int64_t* crow, const int64_t* col, const float* query, const float* key,
                      const float* value, int64_t n, int64_t f_qk, int64_t f_v, double scale, double* out) {
#pragma omp parallel
  {
    double* scores = NULL;
    int64_t cap = 0;
#pragma omp for schedule(dynamic, 64)
    for (int64_t r = 0; r < n; ++r) {
      const int64_t s0 = crow[r], s1 = crow[r + 1];
      double* o = out + r * f_v;
      for (int64_t j = 0; j < f_v; ++j) o[j] = 0.0;
      if (s0 == s1) continue;
      if (s1 - s0 > cap) {
        free(scores);
        cap = s1 - s0;
        scores = (double*)malloc((size_t)cap * sizeof(double));
      }
      const float* q = query + r * f_qk;
      double m = -INFINITY;
      for (int64_t e = s0; e < s1; ++e) {
        const float* k = key + col[e] * f_qk;
        double dot = 0.0;
        for (int64_t j = 0; j < f_qk; ++j) dot += (double)q[j] * (double)k[j];
        const double s = scale * dot;
        scores[e - s0] = s;
        m = s > m ? s : m;
      }
      double d = 0.0;
      for (int64_t e = s0; e < s1; ++e) d += exp(scores[e - s0] - m);
      for (int64_t e = s0; e < s1; ++e) {
        const double p = exp(scores[e - s0] - m) / d;
        const float* v = value + col[e] * f_v;
        for (int64_t j = 0; j < f_v; ++j) o[j] += p * (double)v[j];
      }
    }
    free(scores);
  }
}
