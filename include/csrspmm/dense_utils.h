// Dense helpers (reference include/csrspmm/dense_utils.h:7-32).
#pragma once
#include <csrspmm/matrix.h>

namespace csrspmm {

void dense_alloc_host(DenseMatrix& A, int height, int width);
void dense_alloc_device(DenseMatrix& A, int height, int width);

void dense_free_host(DenseMatrix& A);
void dense_free_device(DenseMatrix& A);

// Allocate the destination (which must be empty) and copy.
void dense_host2device(const DenseMatrix& hA, DenseMatrix& dA);
void dense_device2host(const DenseMatrix& dA, DenseMatrix& hA);

// Fills A with values uniform in [low, high); an element is zero with
// probability `sparsity`; integer_values truncates toward zero.  Unlike the
// reference (which re-seeds rand_r inside its loop and writes one value
// everywhere, src/host/dense_utils.cpp:54-64) every element is drawn from
// the counter-based stream of csrspmm_gen.h, keyed by a per-process call
// counter so successive calls give different, reproducible matrices.
void dense_init_random(DenseMatrix& A,
                       float low = -1.0f,
                       float hight = 1.0f,
                       float sparsity = 0.0f,
                       bool integer_values = false);

void print_dense(const DenseMatrix& A);

// True iff shapes match and |A - B| <= tol elementwise (prints the first
// mismatch), as the reference's absolute-tolerance compare.
bool dense_compare(const DenseMatrix& A,
                   const DenseMatrix& B,
                   float tol = 1e-4f);

// Dense fp32 C = alpha * A * B + beta * C with A M x N, B N x K, C M x K
// (the reference's naming: its N is the inner dimension).
void dense_gemm_cpu(int M, int N, int K,
                    float alpha, float beta,
                    const DenseMatrix& A,
                    const DenseMatrix& B,
                    DenseMatrix& C);

}  // namespace csrspmm
