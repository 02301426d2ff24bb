// The reference's kernel declarations (reference include/csrspmm/kernels.h:6-71),
// for HIP translation units that launch the kernels themselves:
//
//   csrspmm::kernel::csrspmm_warp_per_row<<<grid, block>>>(M, N, K, alpha, beta,
//       A.values, A.col_idx, A.row_ptr, B.data, C.data);
//
// Reference naming: A is M x N, B is N x K, C is M x K, row-major.  The
// definitions live in libcsrspmm_hip.so (csrc/device/kernels_direct.hip):
// any launch shape computes the whole product, no LDS is used (so the smem
// forms accept any dynamic LDS size that launches), and the Fp4 forms compute
// every column.  Code that does not launch kernels itself should call
// csrspmm::spmm / launch_* (csrspmm.h, spmm_launcher.cuh), which run the
// planned gfx950 kernels and are much faster on large or skewed matrices.
//
// Only HIP code (hipcc) can include this header: it declares __global__
// functions.  C++ built by another compiler uses csrspmm.h, which includes
// this header only under hipcc.
#pragma once

#if !defined(__HIPCC__) && !defined(__HIP__)
#error "csrspmm/kernels.h declares __global__ kernels: include it from HIP code built by hipcc"
#endif

#include <hip/hip_runtime.h>

#include <csrspmm/matrix.h>

namespace csrspmm::kernel {

__global__ void csrspmm_naive(int M, int N, int K, float alpha, float beta,
                              const float* __restrict__ A_values,
                              const int* __restrict__ A_col_idx,
                              const int* __restrict__ A_row_ptr,
                              const float* __restrict__ B, float* __restrict__ C);

__global__ void csrspmm_naive_smem(int M, int N, int K, float alpha, float beta,
                                   const float* __restrict__ A_values,
                                   const int* __restrict__ A_col_idx,
                                   const int* __restrict__ A_row_ptr,
                                   const float* __restrict__ B, float* __restrict__ C);

__global__ void csrspmm_warp_per_row(int M, int N, int K, float alpha, float beta,
                                     const float* __restrict__ A_values,
                                     const int* __restrict__ A_col_idx,
                                     const int* __restrict__ A_row_ptr,
                                     const float* __restrict__ B, float* __restrict__ C);

// B and C rows 16-byte aligned and K % 4 == 0 give float4 loads; otherwise
// scalar ones (the result is the same).
__global__ void csrspmm_warp_per_row_fp4(int M, int N, int K, float alpha, float beta,
                                         const float* __restrict__ A_values,
                                         const int* __restrict__ A_col_idx,
                                         const int* __restrict__ A_row_ptr,
                                         const float* __restrict__ B, float* __restrict__ C);

// A_max_row_nnz sized the reference's LDS stage; here it is ignored.
__global__ void csrspmm_warp_per_row_smem(int M, int N, int K, float alpha, float beta,
                                          const float* __restrict__ A_values,
                                          const int* __restrict__ A_col_idx,
                                          const int* __restrict__ A_row_ptr,
                                          const int A_max_row_nnz,
                                          const float* __restrict__ B, float* __restrict__ C);

__global__ void csrspmm_warp_per_row_smem_fp4(int M, int N, int K, float alpha, float beta,
                                              const float* __restrict__ A_values,
                                              const int* __restrict__ A_col_idx,
                                              const int* __restrict__ A_row_ptr,
                                              const int A_max_row_nnz,
                                              const float* __restrict__ B,
                                              float* __restrict__ C);

}  // namespace csrspmm::kernel
