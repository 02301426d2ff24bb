// The reference's six __global__ kernels under their own names and
// signatures (reference include/csrspmm/kernels.h:6-71, declared here in
// include/csrspmm/kernels.h), for HIP code that launches them itself with
// <<<grid, block, lds>>> instead of going through csrspmm::spmm or the C ABI.
//
// Arguments follow the reference's naming: A is M x N (M rows, N columns),
// B is N x K and C is M x K, both row-major with leading dimension K
// (reference src/device/csrspmm_naive.cu:11-39).  C = alpha*A*B + beta*C,
// with C read only when beta != 0.
//
// A caller picks the launch shape, usually the reference launcher's
// (src/host/spmm_launcher.cu: 32 x 32 threads per block over a 2-D grid for
// the naive pair, ceil(M / 4) blocks of 128 threads with dynamic LDS for the
// warp-per-row family).  These kernels therefore depend on no launch shape:
// the launch's waves walk the rows grid-strided, a wave summing one row at a
// time with its active lanes spread over the columns, and they use no LDS, so
// any dynamic LDS size that launches is accepted.  Per output element the
// products are fma-accumulated in CSR order, the order of the reference
// kernels, and the epilogue is fma(alpha, sum, beta * C).  The Fp4 forms use
// 16-byte loads and stores where B, C and K allow them and compute every
// column (the reference drops the last K % 4, csrspmm_warp_per_row_fp4.cu:29-32).
// The planned kernels behind csrspmm::spmm are the fast path; these exist so
// that code written against the reference's kernel declarations compiles and
// computes the same result.

#include <csrspmm/kernels.h>

#include "common.hpp"

namespace csrspmm {
namespace kernel {

namespace {

using csrspmm_hip::f4;

struct WaveSlot {
  int lane, active, first, stride;
};

// This wave's place in the launch: its lane, how many of its lanes exist
// (a block of, say, 32 threads fills half a wave), its first row and the
// grid-stride over rows.
__device__ __forceinline__ WaveSlot wave_slot() {
  const int bt = blockDim.x * blockDim.y * blockDim.z;
  const int tid = threadIdx.x + blockDim.x * (threadIdx.y + blockDim.y * threadIdx.z);
  const int wpb = (bt + 63) / 64;
  const int bid = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int nb = gridDim.x * gridDim.y * gridDim.z;
  const int wib = tid / 64;
  WaveSlot s;
  s.lane = tid % 64;
  s.active = min(64, bt - wib * 64);
  s.first = bid * wpb + wib;
  s.stride = nb * wpb;
  return s;
}

__device__ __forceinline__ float epilogue(float alpha, float beta, float sum, const float* c) {
  return beta != 0.0f ? __builtin_fmaf(alpha, sum, beta * *c) : alpha * sum;
}

// Scalar columns: lane l of the wave's `active` lanes owns columns
// l, l + active, ...
__device__ void rows_scalar(int M, int K, float alpha, float beta, const float* vals,
                            const int* cols, const int* rowptr, const float* B, float* C) {
  const WaveSlot s = wave_slot();
  for (int row = s.first; row < M; row += s.stride) {
    const int rs = rowptr[row];
    const int re = rowptr[row + 1];
    float* crow = C + (long long)row * K;
    for (int c = s.lane; c < K; c += s.active) {
      float sum = 0.0f;
      for (int j = rs; j < re; ++j) sum = __builtin_fmaf(vals[j], B[(long long)cols[j] * K + c], sum);
      crow[c] = epilogue(alpha, beta, sum, crow + c);
    }
  }
}

// float4 columns: lane l owns column chunks l, l + active, ... of K / 4.
__device__ void rows_vec4(int M, int K, float alpha, float beta, const float* vals,
                          const int* cols, const int* rowptr, const float* B, float* C) {
  const WaveSlot s = wave_slot();
  const int K4 = K / 4;
  for (int row = s.first; row < M; row += s.stride) {
    const int rs = rowptr[row];
    const int re = rowptr[row + 1];
    float* crow = C + (long long)row * K;
    for (int c = s.lane; c < K4; c += s.active) {
      f4 sum = f4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int j = rs; j < re; ++j)
        sum = csrspmm_hip::fma4(vals[j], *reinterpret_cast<const f4*>(B + (long long)cols[j] * K + 4 * c), sum);
      f4* cp = reinterpret_cast<f4*>(crow + 4 * c);
      f4 out;
      if (beta != 0.0f) {
        const f4 c0 = *cp;
        out = f4{__builtin_fmaf(alpha, sum.x, beta * c0.x), __builtin_fmaf(alpha, sum.y, beta * c0.y),
                 __builtin_fmaf(alpha, sum.z, beta * c0.z), __builtin_fmaf(alpha, sum.w, beta * c0.w)};
      } else {
        out = f4{alpha * sum.x, alpha * sum.y, alpha * sum.z, alpha * sum.w};
      }
      *cp = out;
    }
  }
}

__device__ __forceinline__ bool vec4_ok(int K, const float* B, const float* C) {
  return K % 4 == 0 && ((reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) & 15) == 0;
}

}  // namespace

__global__ void csrspmm_naive(int M, int N, int K, float alpha, float beta, const float* A_values,
                              const int* A_col_idx, const int* A_row_ptr, const float* B, float* C) {
  (void)N;
  rows_scalar(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
}

__global__ void csrspmm_naive_smem(int M, int N, int K, float alpha, float beta,
                                   const float* A_values, const int* A_col_idx,
                                   const int* A_row_ptr, const float* B, float* C) {
  (void)N;
  rows_scalar(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
}

__global__ void csrspmm_warp_per_row(int M, int N, int K, float alpha, float beta,
                                     const float* A_values, const int* A_col_idx,
                                     const int* A_row_ptr, const float* B, float* C) {
  (void)N;
  rows_scalar(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
}

__global__ void csrspmm_warp_per_row_fp4(int M, int N, int K, float alpha, float beta,
                                         const float* A_values, const int* A_col_idx,
                                         const int* A_row_ptr, const float* B, float* C) {
  (void)N;
  if (vec4_ok(K, B, C))
    rows_vec4(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
  else
    rows_scalar(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
}

__global__ void csrspmm_warp_per_row_smem(int M, int N, int K, float alpha, float beta,
                                          const float* A_values, const int* A_col_idx,
                                          const int* A_row_ptr, const int A_max_row_nnz,
                                          const float* B, float* C) {
  (void)N;
  (void)A_max_row_nnz;  // a hint in the reference's launcher (its LDS size); unused here
  rows_scalar(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
}

__global__ void csrspmm_warp_per_row_smem_fp4(int M, int N, int K, float alpha, float beta,
                                              const float* A_values, const int* A_col_idx,
                                              const int* A_row_ptr, const int A_max_row_nnz,
                                              const float* B, float* C) {
  (void)N;
  (void)A_max_row_nnz;
  if (vec4_ok(K, B, C))
    rows_vec4(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
  else
    rows_scalar(M, K, alpha, beta, A_values, A_col_idx, A_row_ptr, B, C);
}

}  // namespace kernel
}  // namespace csrspmm
