/*
 * spmm_oracle.c -- CPU restatement of the reference's CSR SpMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only as the checker
 * (or, for the baseline, as the thing the GPU is compared against).  The
 * product (libcsrspmm_hip.so, libcsrspmm.so, the torch extension) never
 * links or calls it.
 *
 * Built strictly (-O2 -ffp-contract=off, no fast-math) by oracle/Makefile
 * into oracle/build/liboracle.so.  Each function cites the reference
 * (anh-thh/csrspmm) file:line it restates.  Pinning of every function is in
 * tests/test_oracle.py; a function without such a check would be marked
 * "parity unpinned" here (none is).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/*
 * fp64-accumulated definition of the path:
 *   R[i,j] = alpha * sum_{p in row i} val[p] * B[col[p], j]  +  beta * C0[i,j]
 * where C0 is not read when beta == 0 (reference src/device/csrspmm_naive.cu:38,
 * csrspmm_warp_per_row.cu:45-46, csrspmm_warp_per_row_fp4.cu:48-63), and the
 * condition magnitude
 *   S[i,j] = |alpha| * sum |val[p] * B[col[p], j]|  +  |beta * C0[i,j]|
 * used by the correctness metric.  rows (optional, nrows entries) restricts
 * the computation to a subset; output row r of R/S then holds rows[r].
 * c0_zero != 0 reads C0 as +0 (the torch forwards' zeros() C,
 * torch_csrspmm/torch_csrspmm_naive.cpp:32-34).  S may be NULL.
 */
EXPORT void oracle_spmm_f64(int M, int N, const int* rowptr, const int* colidx, const float* vals,
                            const float* B, long long ldb, const float* C0, long long ldc0,
                            double alpha, double beta, int c0_zero, const int* rows, int nrows,
                            double* R, double* S) {
    const int n_out = rows ? nrows : M;
#pragma omp parallel for schedule(dynamic, 16)
    for (int r = 0; r < n_out; ++r) {
        const int i = rows ? rows[r] : r;
        double* rr = R + (size_t)r * N;
        double* ss = S ? S + (size_t)r * N : NULL;
        for (int j = 0; j < N; ++j) {
            rr[j] = 0.0;
            if (ss) ss[j] = 0.0;
        }
        for (int p = rowptr[i]; p < rowptr[i + 1]; ++p) {
            const double a = (double)vals[p];
            const float* brow = B + (size_t)colidx[p] * (size_t)ldb;
            for (int j = 0; j < N; ++j) {
                const double t = a * (double)brow[j];
                rr[j] += t;
                if (ss) ss[j] += fabs(t);
            }
        }
        for (int j = 0; j < N; ++j) {
            double c = 0.0;
            if (beta != 0.0) c = c0_zero ? 0.0 : (double)C0[(size_t)i * ldc0 + j];
            const double bc = beta != 0.0 ? beta * c : 0.0;
            rr[j] = alpha * rr[j] + bc;
            if (ss) ss[j] = fabs(alpha) * ss[j] + fabs(bc);
        }
    }
}

/*
 * fp32 restatement of the reference kernels' arithmetic: one fp32
 * accumulator per output, products added sequentially in CSR order with a
 * fused multiply-add (nvcc contracts `sum += a * b` to fma by default,
 * reference csrspmm_warp_per_row.cu:37-43, csrspmm_naive.cu:31-35,
 * csrspmm_warp_per_row_fp4.cu:35-45), then the epilogue
 *   beta == 0 : out = alpha * sum                  (C not read)
 *   else      : out = fma(alpha, sum, beta * c0)    (c0 = +0 when c0_zero)
 * (csrspmm_warp_per_row.cu:45-46).  Writes out[r * ldo + j] for the row
 * subset / all rows as oracle_spmm_f64 does.
 */
EXPORT void oracle_spmm_f32_seq(int M, int N, const int* rowptr, const int* colidx,
                                const float* vals, const float* B, long long ldb, const float* C0,
                                long long ldc0, float alpha, float beta, int c0_zero,
                                const int* rows, int nrows, float* out, long long ldo) {
    const int n_out = rows ? nrows : M;
#pragma omp parallel for schedule(dynamic, 16)
    for (int r = 0; r < n_out; ++r) {
        const int i = rows ? rows[r] : r;
        float* o = out + (size_t)r * (size_t)ldo;
        for (int j = 0; j < N; ++j) o[j] = 0.0f;
        for (int p = rowptr[i]; p < rowptr[i + 1]; ++p) {
            const float a = vals[p];
            const float* brow = B + (size_t)colidx[p] * (size_t)ldb;
            for (int j = 0; j < N; ++j) o[j] = fmaf(a, brow[j], o[j]);
        }
        for (int j = 0; j < N; ++j) {
            if (beta == 0.0f) {
                o[j] = alpha * o[j];
            } else {
                const float c = c0_zero ? 0.0f : C0[(size_t)i * ldc0 + j];
                o[j] = fmaf(alpha, o[j], beta * c);
            }
        }
    }
}

/*
 * Correctness metric: element (r, j) passes iff
 *   |C - R| <= tol * max(|R|, S)
 * (both sides finite or both the same non-finite class).  Returns the number
 * of failing elements; *max_ratio = max |C-R| / max(|R|, S) over finite
 * elements, *max_rel_plain = max|C-R| / max|R|; *worst = first index of the
 * largest ratio.
 */
EXPORT long long oracle_check(long long n, const float* C, long long ldc, int ncols,
                              const double* R, const double* S, double tol, double* max_ratio,
                              double* max_rel_plain, long long* worst) {
    long long bad = 0;
    double mr = 0.0, maxdiff = 0.0, maxabs = 0.0;
    long long w = -1;
    for (long long e = 0; e < n; ++e) {
        const long long r = e / ncols, j = e % ncols;
        const double c = (double)C[r * ldc + j];
        const double ref = R[e];
        if (!isfinite(ref) || !isfinite(c)) {
            const int same = (isnan(ref) && isnan(c)) || (isinf(ref) && isinf(c) && (ref > 0) == (c > 0));
            if (!same) {
                ++bad;
                if (w < 0) w = e;
            }
            continue;
        }
        const double d = fabs(c - ref);
        const double scale = fmax(fabs(ref), S ? S[e] : fabs(ref));
        const double ratio = scale > 0.0 ? d / scale : (d > 0.0 ? INFINITY : 0.0);
        if (ratio > mr) {
            mr = ratio;
            w = e;
        }
        if (!(d <= tol * scale)) ++bad;
        if (d > maxdiff) maxdiff = d;
        if (fabs(ref) > maxabs) maxabs = fabs(ref);
    }
    if (max_ratio) *max_ratio = mr;
    if (max_rel_plain) *max_rel_plain = maxabs > 0.0 ? maxdiff / maxabs : maxdiff;
    if (worst) *worst = w;
    return bad;
}

/*
 * dense2csr (reference src/host/csr_utils.cpp:70-111): row-major scan keeping
 * entries with fabs(v) > tol (so +-0 and NaN are dropped), rowptr/colidx/
 * values written in scan order, *max_row_nnz the longest row.  Pass NULL
 * arrays to count only; returns nnz.
 */
EXPORT long long oracle_dense2csr(const float* dense, int H, int W, float tol, int* rowptr,
                                  int* colidx, float* vals, int* max_row_nnz) {
    long long idx = 0;
    int mx = 0;
    if (rowptr) rowptr[0] = 0;
    for (int i = 0; i < H; ++i) {
        const long long start = idx;
        for (int j = 0; j < W; ++j) {
            const float v = dense[(size_t)i * W + j];
            if (fabsf(v) > tol) {
                if (colidx) colidx[idx] = j;
                if (vals) vals[idx] = v;
                ++idx;
            }
        }
        if (rowptr) rowptr[i + 1] = (int)idx;
        if (idx - start > mx) mx = (int)(idx - start);
    }
    if (max_row_nnz) *max_row_nnz = mx;
    return idx;
}

/* csr2dense (reference src/host/csr_utils.cpp:114-145): zero fill, then
 * dense[i, col[p]] = val[p] in CSR order (a later duplicate wins). */
EXPORT void oracle_csr2dense(int H, int W, const int* rowptr, const int* colidx, const float* vals,
                             float* dense) {
    memset(dense, 0, (size_t)H * (size_t)W * sizeof(float));
    for (int i = 0; i < H; ++i)
        for (int p = rowptr[i]; p < rowptr[i + 1]; ++p) dense[(size_t)i * W + colidx[p]] = vals[p];
}

/*
 * dense_gemm_cpu (reference src/host/dense_utils.cpp:109-126), reference
 * naming: A is M x N, B is N x K, C is M x K; fp32 sum over all N in order,
 * zeros included, then C = alpha*sum + beta*C.  The reference builds it with
 * -ffast-math (CMakeLists.txt:23), which leaves its rounding unspecified;
 * this restatement rounds each operation.  With the integer inputs the
 * reference's own test uses, every ordering gives the same exact result.
 */
EXPORT void oracle_dense_gemm_cpu(int M, int N, int K, float alpha, float beta, const float* A,
                                  const float* B, float* C) {
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < K; ++j) {
            float sum = 0.0f;
            for (int k = 0; k < N; ++k) {
                const float prod = A[(size_t)i * N + k] * B[(size_t)k * K + j];
                sum = sum + prod;
            }
            const float t1 = alpha * sum;
            const float t2 = beta * C[(size_t)i * K + j];
            C[(size_t)i * K + j] = t1 + t2;
        }
    }
}

/*
 * dense_init_random as the reference writes it (src/host/dense_utils.cpp:46-65):
 * the rand_r seed is reset to 1234 inside the loop, so every element gets the
 * same draw.  Kept only to pin the reference's own test inputs (its default
 * test_csrspmm run).
 */
EXPORT void oracle_dense_init_random_ref(float* A, int height, int width, float low, float high,
                                         float sparsity, int integer_values) {
    const long long total = (long long)height * width;
    for (long long i = 0; i < total; ++i) {
        unsigned int seed = 1234;
        const float r = (float)rand_r(&seed) / RAND_MAX;
        if (r < sparsity) {
            A[i] = 0.0f;
        } else {
            const float val = (float)rand_r(&seed) / RAND_MAX * (high - low) + low;
            A[i] = integer_values ? (float)(int)val : val;
        }
    }
}
