// Deterministic synthetic CSR / dense generators (include/csrspmm_gen.h).
// Host-only C++, built with g++ -fopenmp into libcsrspmm.so.

#include "csrspmm_gen.h"

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <parallel/algorithm>
#include <vector>

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ULL;

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
inline uint64_t rnd(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGamma); }
inline float u11(uint64_t r) { return (float)(r >> 40) * (1.0f / 8388608.0f) - 1.0f; }
inline double u01(uint64_t r) { return (double)(r >> 11) * (1.0 / 9007199254740992.0); }
inline uint32_t below(uint64_t r, uint32_t n) { return (uint32_t)(((r >> 32) * (uint64_t)n) >> 32); }

}  // namespace

struct csrspmm_gen_csr {
  int M = 0, K = 0;
  long long nnz = 0;
  int max_row = 0;
  std::vector<int> rowptr, colidx;
  std::vector<float> vals;
};

namespace {

// Columns of every row by Floyd's sampling without replacement (Bentley &
// Floyd, CACM 1987), sorted; then values by CSR position.
void fill_columns_and_values(csrspmm_gen_csr* g, const std::vector<int>& len, uint64_t seed) {
  const int M = g->M, K = g->K;
  g->rowptr.assign((size_t)M + 1, 0);
  for (int r = 0; r < M; ++r) g->rowptr[r + 1] = g->rowptr[r] + len[r];
  g->nnz = g->rowptr[M];
  g->colidx.resize((size_t)g->nnz);
  g->vals.resize((size_t)g->nnz);
  int mx = 0;
  for (int r = 0; r < M; ++r) mx = std::max(mx, len[r]);
  g->max_row = mx;
  const uint64_t kc = csrspmm_gen_key(seed, CSRSPMM_TAG_COLS);
  const uint64_t kv = csrspmm_gen_key(seed, CSRSPMM_TAG_VALS);
#pragma omp parallel
  {
    std::vector<uint64_t> bitmap(((size_t)K + 63) / 64, 0);
#pragma omp for schedule(dynamic, 256)
    for (int r = 0; r < M; ++r) {
      const int L = len[r];
      int* out = g->colidx.data() + g->rowptr[r];
      const uint64_t rk = rnd(kc, (uint64_t)r);
      int n = 0;
      uint64_t draw = 0;
      for (int j = K - L; j < K; ++j) {
        const int t = (int)below(rnd(rk, draw++), (uint32_t)j + 1u);
        const int pick = (bitmap[(size_t)t >> 6] >> (t & 63)) & 1ULL ? j : t;
        bitmap[(size_t)pick >> 6] |= 1ULL << (pick & 63);
        out[n++] = pick;
      }
      for (int i = 0; i < n; ++i) bitmap[(size_t)out[i] >> 6] &= ~(1ULL << (out[i] & 63));
      std::sort(out, out + n);
    }
#pragma omp for schedule(static)
    for (long long p = 0; p < g->nnz; ++p) g->vals[(size_t)p] = u11(rnd(kv, (uint64_t)p));
  }
}

}  // namespace

extern "C" {

uint64_t csrspmm_gen_key(uint64_t seed, int tag) { return mix64(seed * kGamma + (uint64_t)tag); }
uint64_t csrspmm_gen_rand(uint64_t key, uint64_t i) { return rnd(key, i); }

void csrspmm_gen_dense(uint64_t seed, int tag, uint64_t first, size_t count, float* out) {
  const uint64_t k = csrspmm_gen_key(seed, tag);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)count; ++i) out[i] = u11(rnd(k, first + (uint64_t)i));
}

csrspmm_gen_csr* csrspmm_gen_uniform(int M, int K, int per_row, uint64_t seed) {
  if (M < 0 || K <= 0 || per_row < 0 || per_row > K) return nullptr;
  auto* g = new csrspmm_gen_csr();
  g->M = M;
  g->K = K;
  std::vector<int> len((size_t)M, per_row);
  fill_columns_and_values(g, len, seed);
  return g;
}

csrspmm_gen_csr* csrspmm_gen_powerlaw(int M, int K, double exponent, double shift, int cap,
                                      uint64_t seed) {
  if (M < 0 || K <= 0 || cap < 1 || cap > K || shift >= 1.0) return nullptr;
  std::vector<double> cdf((size_t)cap);
  double acc = 0.0;
  for (int k = 1; k <= cap; ++k) {
    acc += std::pow((double)k - shift, -exponent);
    cdf[(size_t)k - 1] = acc;
  }
  for (double& c : cdf) c /= acc;
  auto* g = new csrspmm_gen_csr();
  g->M = M;
  g->K = K;
  std::vector<int> len((size_t)M);
  const uint64_t kl = csrspmm_gen_key(seed, CSRSPMM_TAG_ROWLEN);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < M; ++r) {
    const double u = u01(rnd(kl, (uint64_t)r));
    const long long idx = std::upper_bound(cdf.begin(), cdf.end(), u) - cdf.begin();
    len[(size_t)r] = (int)std::min<long long>(idx + 1, cap);
  }
  fill_columns_and_values(g, len, seed);
  return g;
}

csrspmm_gen_csr* csrspmm_gen_ragged(int M, int K, int min_len, int max_len, uint64_t seed) {
  if (M < 0 || K <= 0 || min_len < 0 || max_len < min_len || max_len > K) return nullptr;
  auto* g = new csrspmm_gen_csr();
  g->M = M;
  g->K = K;
  std::vector<int> len((size_t)M);
  const uint64_t kl = csrspmm_gen_key(seed, CSRSPMM_TAG_ROWLEN);
  for (int r = 0; r < M; ++r)
    len[(size_t)r] = min_len + (int)below(rnd(kl, (uint64_t)r), (uint32_t)(max_len - min_len + 1));
  fill_columns_and_values(g, len, seed);
  return g;
}

csrspmm_gen_csr* csrspmm_gen_rmat(int scale, long long samples, double a, double b, double c,
                                  uint64_t seed) {
  if (scale < 1 || scale > 30 || samples < 0) return nullptr;
  const int n = 1 << scale;
  const uint64_t kc = csrspmm_gen_key(seed, CSRSPMM_TAG_COLS);
  std::vector<uint64_t> edges((size_t)samples);
  const double ab = a + b, abc = a + b + c;
#pragma omp parallel for schedule(static)
  for (long long s = 0; s < samples; ++s) {
    uint64_t r = 0, col = 0;
    const uint64_t base = (uint64_t)s * (uint64_t)scale;
    for (int l = 0; l < scale; ++l) {
      const double u = u01(rnd(kc, base + (uint64_t)l));
      const uint64_t rb = u >= ab ? 1 : 0;
      const uint64_t cb = (u >= a && u < ab) || u >= abc ? 1 : 0;
      r = (r << 1) | rb;
      col = (col << 1) | cb;
    }
    edges[(size_t)s] = (r << 32) | col;
  }
  __gnu_parallel::sort(edges.begin(), edges.end());
  edges.erase(std::unique(edges.begin(), edges.end()), edges.end());
  auto* g = new csrspmm_gen_csr();
  g->M = n;
  g->K = n;
  g->nnz = (long long)edges.size();
  g->rowptr.assign((size_t)n + 1, 0);
  g->colidx.resize(edges.size());
  g->vals.resize(edges.size());
  for (size_t p = 0; p < edges.size(); ++p) {
    g->rowptr[(size_t)(edges[p] >> 32) + 1]++;
    g->colidx[p] = (int)(edges[p] & 0xffffffffULL);
  }
  int mx = 0;
  for (int r = 0; r < n; ++r) {
    mx = std::max(mx, g->rowptr[(size_t)r + 1]);
    g->rowptr[(size_t)r + 1] += g->rowptr[(size_t)r];
  }
  g->max_row = mx;
  const uint64_t kv = csrspmm_gen_key(seed, CSRSPMM_TAG_VALS);
#pragma omp parallel for schedule(static)
  for (long long p = 0; p < g->nnz; ++p) g->vals[(size_t)p] = u11(rnd(kv, (uint64_t)p));
  return g;
}

int csrspmm_gen_shape(const csrspmm_gen_csr* g, int* M, int* K, long long* nnz, int* max_row_nnz) {
  if (!g) return -1;
  if (M) *M = g->M;
  if (K) *K = g->K;
  if (nnz) *nnz = g->nnz;
  if (max_row_nnz) *max_row_nnz = g->max_row;
  return 0;
}

int csrspmm_gen_copy(const csrspmm_gen_csr* g, int* rowptr, int* colidx, float* values) {
  if (!g) return -1;
  if (rowptr) std::memcpy(rowptr, g->rowptr.data(), g->rowptr.size() * sizeof(int));
  if (colidx && g->nnz) std::memcpy(colidx, g->colidx.data(), g->colidx.size() * sizeof(int));
  if (values && g->nnz) std::memcpy(values, g->vals.data(), g->vals.size() * sizeof(float));
  return 0;
}

void csrspmm_gen_free(csrspmm_gen_csr* g) { delete g; }

uint64_t csrspmm_fnv1a64(uint64_t h, const void* data, size_t bytes) {
  const unsigned char* p = static_cast<const unsigned char*>(data);
  for (size_t i = 0; i < bytes; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ULL;
  }
  return h;
}

}  // extern "C"
