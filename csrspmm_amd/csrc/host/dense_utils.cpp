// Dense helpers (reference src/host/dense_utils.cpp:12-162).
#include <csrspmm/dense_utils.h>
#include <csrspmm/error_check.h>

#include "csrspmm_gen.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <iostream>

namespace csrspmm {

namespace {
[[noreturn]] void die(const char* msg) {
    std::cerr << msg << "\n";
    std::exit(1);
}
size_t elems(int h, int w) { return (size_t)(h > 0 ? h : 0) * (size_t)(w > 0 ? w : 0); }
std::atomic<unsigned long long> g_init_calls{0};
}  // namespace

void dense_alloc_host(DenseMatrix& A, int height, int width) {
    if (A.data != nullptr) die("dense_alloc_host error: already allocated host memory.");
    A.height = height;
    A.width = width;
    A.data = static_cast<float*>(std::malloc(std::max<size_t>(elems(height, width), 1) * sizeof(float)));
    if (!A.data) die("dense_alloc_host: malloc failed");
}

void dense_free_host(DenseMatrix& A) {
    std::free(A.data);
    A.data = nullptr;
    A.height = A.width = 0;
}

void dense_alloc_device(DenseMatrix& A, int height, int width) {
    if (A.data != nullptr) die("dense_alloc_device error: already allocated device memory.");
    A.height = height;
    A.width = width;
    A.data = nullptr;
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&A.data),
                                       std::max<size_t>(elems(height, width), 1) * sizeof(float)));
}

void dense_free_device(DenseMatrix& A) {
    if (A.data) csrspmmCheck(csrspmm_device_free(A.data));
    A.data = nullptr;
    A.height = A.width = 0;
}

void dense_init_random(DenseMatrix& A, float low, float high, float sparsity, bool integer_values) {
    const size_t total = elems(A.height, A.width);
    const unsigned long long call = g_init_calls.fetch_add(1);
    const uint64_t key_keep = csrspmm_gen_key(0x1234ULL + call, CSRSPMM_TAG_ROWLEN);
    const uint64_t key_val = csrspmm_gen_key(0x1234ULL + call, CSRSPMM_TAG_VALS);
    for (size_t i = 0; i < total; ++i) {
        const double r = (double)(csrspmm_gen_rand(key_keep, i) >> 11) * (1.0 / 9007199254740992.0);
        if (r < sparsity) {
            A.data[i] = 0.0f;
        } else {
            const double u = (double)(csrspmm_gen_rand(key_val, i) >> 11) * (1.0 / 9007199254740992.0);
            const float val = (float)(u * ((double)high - (double)low) + (double)low);
            A.data[i] = integer_values ? (float)(int)val : val;
        }
    }
}

void print_dense(const DenseMatrix& A) {
    std::cout << "DenseMatrix (" << A.height << "x" << A.width << "):\n";
    for (int i = 0; i < A.height; ++i) {
        std::cout << "  [ ";
        for (int j = 0; j < A.width; ++j) {
            std::cout << A.data[(size_t)i * A.width + j];
            if (j < A.width - 1) std::cout << ", ";
        }
        std::cout << " ]\n";
    }
    std::cout << std::endl;
}

bool dense_compare(const DenseMatrix& A, const DenseMatrix& B, float tol) {
    if (A.height != B.height || A.width != B.width) {
        std::cout << "Dense compare failed: shape mismatch\n";
        return false;
    }
    const size_t total = elems(A.height, A.width);
    for (size_t i = 0; i < total; ++i) {
        const float a = A.data[i], b = B.data[i];
        // Written so that a NaN on either side counts as a mismatch.
        if (!(std::fabs(a - b) <= tol)) {
            std::cout << "Mismatch at index " << i << ": " << a << " vs " << b << "\n";
            return false;
        }
    }
    return true;
}

void dense_gemm_cpu(int M, int N, int K, float alpha, float beta, const DenseMatrix& A,
                    const DenseMatrix& B, DenseMatrix& C) {
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < K; ++j) {
            float sum = 0.0f;
            for (int k = 0; k < N; ++k) sum += A.data[(size_t)i * N + k] * B.data[(size_t)k * K + j];
            C.data[(size_t)i * K + j] = alpha * sum + beta * C.data[(size_t)i * K + j];
        }
    }
}

void dense_host2device(const DenseMatrix& hA, DenseMatrix& dA) {
    if (!hA.data) die("dense_host2device: host data is null");
    if (dA.data != nullptr) die("dense_host2device error: Only accept null destination.");
    dense_alloc_device(dA, hA.height, hA.width);
    csrspmmCheck(csrspmm_memcpy_h2d(dA.data, hA.data, elems(hA.height, hA.width) * sizeof(float)));
}

void dense_device2host(const DenseMatrix& dA, DenseMatrix& hA) {
    if (!dA.data) die("dense_device2host: device data is null");
    if (hA.data != nullptr) die("dense_device2host error: only accept null destination.");
    dense_alloc_host(hA, dA.height, dA.width);
    csrspmmCheck(csrspmm_memcpy_d2h(hA.data, dA.data, elems(dA.height, dA.width) * sizeof(float)));
}

}  // namespace csrspmm
