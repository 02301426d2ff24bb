/*
 * csrspmm_gen.h -- deterministic synthetic inputs for tests and benchmarks
 * (C ABI, host only, built with g++ into libcsrspmm.so).
 *
 * No counterpart in the reference, whose generator re-seeds rand_r inside its
 * loop and so fills every element with the same value
 * (src/host/dense_utils.cpp:54-64).  These generators are counter based:
 * element i of a stream keyed by (seed, tag) is a function of (key, i) only,
 * so results do not depend on thread count and numpy can recompute them.
 *
 *   splitmix64 output:  r(key, i) = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)
 *   mix64 (Stafford variant 13, as in SplitMix64, Steele/Lea/Flood 2014):
 *       z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9
 *       z = (z ^ (z >> 27)) * 0x94D049BB133111EB
 *       z ^= z >> 31
 *   stream key:         key(seed, tag) = mix64(seed * 0x9E3779B97F4A7C15 + tag)
 *   U(-1, 1) fp32:      ((r >> 40) * 2^-23) - 1     (exact in fp32)
 *   U[0, 1) fp64:       (r >> 11) * 2^-53
 *   uniform int [0, n): (uint32)(((r >> 32) * n) >> 32)
 */
#ifndef CSRSPMM_GEN_H_
#define CSRSPMM_GEN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Stream tags. */
enum {
    CSRSPMM_TAG_ROWLEN = 1,  /* row lengths (power-law configs) */
    CSRSPMM_TAG_COLS = 2,    /* column sampling / RMAT quadrant draws */
    CSRSPMM_TAG_VALS = 3,    /* A values, indexed by CSR position */
    CSRSPMM_TAG_B = 4,       /* dense B, indexed row-major */
    CSRSPMM_TAG_C0 = 5       /* dense C0, indexed row-major */
};

uint64_t csrspmm_gen_key(uint64_t seed, int tag);
uint64_t csrspmm_gen_rand(uint64_t key, uint64_t i);

/* out[i] = U(-1,1) of stream key(seed, tag) at index first + i, i < count.
 * Multithreaded. */
void csrspmm_gen_dense(uint64_t seed, int tag, uint64_t first, size_t count, float* out);

/* A generated CSR matrix owned by the library (opaque handle). */
typedef struct csrspmm_gen_csr csrspmm_gen_csr;

/* Every row has exactly per_row distinct columns drawn uniformly from [0, K)
 * by Floyd's algorithm, sorted ascending. */
csrspmm_gen_csr* csrspmm_gen_uniform(int M, int K, int per_row, uint64_t seed);

/* Row length L in {1..cap} with P(L = k) proportional to (k - shift)^-exponent
 * (Zipf-Mandelbrot; shift = 0 is the truncated Zipf law), drawn by inverse
 * CDF over an fp64 table; columns as in csrspmm_gen_uniform (cap <= K). */
csrspmm_gen_csr* csrspmm_gen_powerlaw(int M, int K, double exponent, double shift, int cap,
                                      uint64_t seed);

/* Row lengths uniform in [min_len, max_len] (small parity cases with empty
 * and ragged rows); columns as in csrspmm_gen_uniform. */
csrspmm_gen_csr* csrspmm_gen_ragged(int M, int K, int min_len, int max_len, uint64_t seed);

/* R-MAT graph on 2^scale vertices: `samples` edges, each placed by `scale`
 * quadrant choices with probabilities (a, b, c, 1-a-b-c); duplicates removed,
 * self loops kept, no vertex permutation, columns sorted in each row. */
csrspmm_gen_csr* csrspmm_gen_rmat(int scale, long long samples, double a, double b, double c,
                                  uint64_t seed);

/* Shape of a generated matrix; returns 0, or -1 for a NULL handle. */
int csrspmm_gen_shape(const csrspmm_gen_csr* g, int* M, int* K, long long* nnz, int* max_row_nnz);

/* Copies rowptr (M+1), colidx (nnz), values (nnz); any pointer may be NULL. */
int csrspmm_gen_copy(const csrspmm_gen_csr* g, int* rowptr, int* colidx, float* values);

void csrspmm_gen_free(csrspmm_gen_csr* g);

/* 64-bit FNV-1a over a byte range, continuing from h (start with
 * 0xcbf29ce484222325). Used to pin generated CSR arrays in tests. */
uint64_t csrspmm_fnv1a64(uint64_t h, const void* data, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* CSRSPMM_GEN_H_ */
