// Per-variant launchers (reference include/csrspmm/spmm_launcher.cuh:8-43).
// The file keeps the reference's name so existing #include lines resolve; its
// contents are plain C++ (the kernels live in libcsrspmm_hip.so behind
// include/csrspmm_c.h).  Each launcher enqueues the variant on the default
// stream and returns without synchronising, like the reference; an argument
// or launch error prints a message and exits (the reference leaves it for the
// next cudaGetLastError).
#pragma once

#include <csrspmm/config.h>
#include <csrspmm/matrix.h>

namespace csrspmm {

void launch_naive(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C,
                  float alpha, float beta);

void launch_naive_smem(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C,
                       float alpha, float beta);

void launch_warp_per_row(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C,
                         float alpha, float beta);

void launch_warp_per_row_fp4(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C,
                             float alpha, float beta);

void launch_warp_per_row_smem(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C,
                              float alpha, float beta);

void launch_warp_per_row_smem_fp4(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C,
                                  float alpha, float beta);

}  // namespace csrspmm
