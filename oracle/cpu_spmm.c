/*
 * cpu_spmm.c -- CPU baseline for bench.py: the fp32 CSR restatement of the
 * reference kernels' arithmetic (one fp32 accumulator per output, products
 * fused-multiply-added in CSR order; reference
 * src/device/csrspmm_warp_per_row.cu:37-46), rows spread over OpenMP threads
 * with schedule(dynamic, 64).
 *
 * Also the reference's dense CPU GEMM (src/host/dense_utils.cpp:109-126),
 * the only CPU product the reference has, timed on the host config.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it; nothing in
 * the product calls it.  Built with the reference's release flags
 * (-O3 -ffast-math, CMakeLists.txt:23) except -march=native, which is replaced
 * by x86-64-v3 because the library is built here and run on the GPU box's host.
 */
#include <math.h>
#include <omp.h>
#include <stddef.h>

#define EXPORT __attribute__((visibility("default")))

EXPORT int cpu_spmm_max_threads(void) { return omp_get_max_threads(); }

EXPORT void cpu_spmm_f32(int M, int N, const int* rowptr, const int* colidx, const float* vals,
                         const float* B, long long ldb, float* C, long long ldc, float alpha,
                         float beta, int nthreads) {
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 64) num_threads(nthreads)
    for (int i = 0; i < M; ++i) {
        float* c = C + (size_t)i * (size_t)ldc;
        float acc[N];
        for (int j = 0; j < N; ++j) acc[j] = 0.0f;
        for (int p = rowptr[i]; p < rowptr[i + 1]; ++p) {
            const float a = vals[p];
            const float* b = B + (size_t)colidx[p] * (size_t)ldb;
            for (int j = 0; j < N; ++j) acc[j] = fmaf(a, b[j], acc[j]);
        }
        if (beta == 0.0f) {
            for (int j = 0; j < N; ++j) c[j] = alpha * acc[j];
        } else {
            for (int j = 0; j < N; ++j) c[j] = fmaf(alpha, acc[j], beta * c[j]);
        }
    }
}

/*
 * dense_gemm_cpu as the reference writes it (src/host/dense_utils.cpp:109-126),
 * reference naming: A is M x N, B is N x K, C is M x K; for each output an
 * fp32 sum over all N in order, zeros included, then C = alpha*sum + beta*C.
 * Single-threaded, as the reference's.  Timed beside the GPU on the host
 * config; the strictly rounded restatement that tests pin is
 * oracle_dense_gemm_cpu in spmm_oracle.c.
 */
EXPORT void cpu_dense_gemm(int M, int N, int K, float alpha, float beta, const float* A,
                           const float* B, float* C) {
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < K; ++j) {
            float sum = 0.0f;
            for (int k = 0; k < N; ++k) sum += A[(size_t)i * N + k] * B[(size_t)k * K + j];
            C[(size_t)i * K + j] = alpha * sum + beta * C[(size_t)i * K + j];
        }
    }
}
