// Seeded synthetic CSR generators for the benchmark and test workloads.
//
// Host-only C++ (OpenMP).  Every row draws from its own counter-seeded
// xoshiro256** stream, so the output does not depend on the thread count.
#include <algorithm>
#include <cstdint>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct Xoshiro {
  uint64_t s[4];
  Xoshiro(uint64_t seed, uint64_t stream) {
    uint64_t x = seed * 0xD1B54A32D192ED03ull + stream * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull;
    for (auto& v : s) v = splitmix64(x);
  }
  static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  uint64_t next() {
    const uint64_t result = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return result;
  }
  // uniform in [0, bound) (Lemire's multiply-shift; bias < 2^-32 for our sizes)
  uint64_t below(uint64_t bound) {
    return static_cast<uint64_t>((static_cast<unsigned __int128>(next()) * bound) >> 64);
  }
};

// Column j drawn with probability (cum[j+1]-cum[j]) / cum[n_cols].
inline int64_t draw(Xoshiro& rng, int mode, int64_t n_cols, const int64_t* cum) {
  if (mode == 0) return static_cast<int64_t>(rng.below(static_cast<uint64_t>(n_cols)));
  const uint64_t t = rng.below(static_cast<uint64_t>(cum[n_cols]));
  // largest j with cum[j] <= t
  const int64_t* it = std::upper_bound(cum, cum + n_cols + 1, static_cast<int64_t>(t));
  return static_cast<int64_t>(it - cum) - 1;
}

}  // namespace

extern "C" {

// Fills col[crow[r]..crow[r+1]) for every row with distinct columns in
// ascending order.  mode 0: uniform over [0, n_cols); mode 1: column j with
// probability proportional to cum[j+1] - cum[j].  Rows whose degree exceeds
// n_cols are an error (returns -1).
int synth_fill_columns(const int64_t* crow, int64_t n_rows, int64_t n_cols, int mode, const int64_t* cum,
                       uint64_t seed, int64_t* col) {
  for (int64_t r = 0; r < n_rows; ++r)
    if (crow[r + 1] - crow[r] > n_cols) return -1;
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < n_rows; ++r) {
    const int64_t begin = crow[r];
    const int64_t deg = crow[r + 1] - begin;
    if (deg == 0) continue;
    Xoshiro rng(seed, static_cast<uint64_t>(r));
    std::vector<int64_t> picked;
    picked.reserve(static_cast<size_t>(deg));
    while (static_cast<int64_t>(picked.size()) < deg) {
      const int64_t need = deg - static_cast<int64_t>(picked.size());
      for (int64_t i = 0; i < need; ++i) picked.push_back(draw(rng, mode, n_cols, cum));
      std::sort(picked.begin(), picked.end());
      picked.erase(std::unique(picked.begin(), picked.end()), picked.end());
    }
    std::copy(picked.begin(), picked.end(), col + begin);
  }
  return 0;
}

// Row-wise union of A and its transpose for a square CSR A (rows sorted,
// unique).  Pass out_col = nullptr to get only out_crow; then call again with
// out_col sized out_crow[n].  Uses t_crow/t_col = transpose of A (sorted).
int synth_union_rows(const int64_t* crow, const int64_t* col, const int64_t* t_crow, const int64_t* t_col,
                     int64_t n, int64_t* out_crow, int64_t* out_col) {
  if (out_col == nullptr) {
    out_crow[0] = 0;
#pragma omp parallel for schedule(dynamic, 256)
    for (int64_t r = 0; r < n; ++r) {
      int64_t i = crow[r], ie = crow[r + 1], j = t_crow[r], je = t_crow[r + 1], c = 0;
      while (i < ie || j < je) {
        if (j >= je || (i < ie && col[i] < t_col[j])) ++i;
        else if (i >= ie || t_col[j] < col[i]) ++j;
        else { ++i; ++j; }
        ++c;
      }
      out_crow[r + 1] = c;
    }
    for (int64_t r = 0; r < n; ++r) out_crow[r + 1] += out_crow[r];
    return 0;
  }
#pragma omp parallel for schedule(dynamic, 256)
  for (int64_t r = 0; r < n; ++r) {
    int64_t i = crow[r], ie = crow[r + 1], j = t_crow[r], je = t_crow[r + 1], o = out_crow[r];
    while (i < ie || j < je) {
      if (j >= je || (i < ie && col[i] < t_col[j])) out_col[o++] = col[i++];
      else if (i >= ie || t_col[j] < col[i]) out_col[o++] = t_col[j++];
      else { out_col[o++] = col[i]; ++i; ++j; }
    }
  }
  return 0;
}

// Transpose of a square CSR A: t_crow[n+1], t_col[nnz]; rows of the
// transpose list their columns in ascending order.  Threads own contiguous
// source-row ranges; per-thread column histograms give each thread its write
// offsets, so the output is the same for every thread count.
int synth_transpose(const int64_t* crow, const int64_t* col, int64_t n, int64_t* t_crow, int64_t* t_col) {
  const int parts = 16;
  std::vector<std::vector<int64_t>> hist(parts, std::vector<int64_t>(static_cast<size_t>(n), 0));
  auto range = [&](int p, int64_t* b, int64_t* e) {
    *b = n * p / parts;
    *e = n * (p + 1) / parts;
  };
#pragma omp parallel for schedule(static, 1)
  for (int p = 0; p < parts; ++p) {
    int64_t b, e;
    range(p, &b, &e);
    auto& h = hist[p];
    for (int64_t k = crow[b]; k < crow[e]; ++k) ++h[static_cast<size_t>(col[k])];
  }
  t_crow[0] = 0;
  for (int64_t c = 0; c < n; ++c) {
    int64_t total = 0;
    for (int p = 0; p < parts; ++p) {
      const int64_t v = hist[p][c];
      hist[p][c] = total;  // exclusive offset of part p inside column c
      total += v;
    }
    t_crow[c + 1] = t_crow[c] + total;
  }
#pragma omp parallel for schedule(static, 1)
  for (int p = 0; p < parts; ++p) {
    int64_t b, e;
    range(p, &b, &e);
    auto& h = hist[p];
    for (int64_t r = b; r < e; ++r)
      for (int64_t k = crow[r]; k < crow[r + 1]; ++k) {
        const int64_t c = col[k];
        t_col[t_crow[c] + h[static_cast<size_t>(c)]++] = r;
      }
  }
  return 0;
}

}  // extern "C"
