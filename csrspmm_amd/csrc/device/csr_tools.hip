// Device-side CSR tooling: dense -> CSR, the longest row, and int64 -> int32
// index narrowing, all on the caller's stream with no host synchronisation.
//
// dense -> CSR follows the reference's host dense2csr (src/host/csr_utils.cpp
// :70-111): an element is kept when fabsf(v) > tol (so +-0 and NaN are
// dropped), in row-major order.  It runs in two steps because the output
// size is data-dependent: csrspmm_dense2csr_count_f32 writes rowptr and the
// nonzero count (both in device memory); the caller allocates colidx/vals
// from the count and calls csrspmm_dense2csr_fill_f32.

#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../../include/csrspmm_c.h"
#include "common.hpp"
#include "spmm_internal.h"

namespace csrspmm_hip {
namespace {

constexpr int kToolBlock = 256;
constexpr int kToolMaxBlocks = 8192;
constexpr int kScanThreads = 1024;
constexpr int kScanItems = 4;

__device__ __forceinline__ bool keep(float v, float tol) { return fabsf(v) > tol; }

// One wave per row: rowptr[row + 1] = kept elements of the row.
__global__ __launch_bounds__(kToolBlock) void d2c_count_kernel(int M, int K, const float* A,
                                                               long long lda, float tol,
                                                               int* rowptr) {
  const int lane = lane_id();
  const int nw = blockDim.x >> 6;
  for (int row = blockIdx.x * nw + (threadIdx.x >> 6); row < M; row += gridDim.x * nw) {
    const float* a = A + (long long)row * lda;
    int cnt = 0;
    for (int c = lane; c < K; c += 64) cnt += keep(a[c], tol) ? 1 : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off);
    if (lane == 0) rowptr[row + 1] = cnt;
  }
}

// In-place inclusive scan of rowptr[1..M] by one workgroup, 4096 entries per
// step with the running total carried between steps; rowptr[0] = 0 and the
// 64-bit total goes to *total.
__global__ __launch_bounds__(kScanThreads) void scan_rowptr_kernel(int* rowptr, int M,
                                                                   long long* total) {
  __shared__ long long wave_tot[kScanThreads / 64];
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  long long carry = 0;
  for (int base = 1; base <= M; base += kScanThreads * kScanItems) {
    const int i0 = base + threadIdx.x * kScanItems;
    long long v[kScanItems];
    long long t = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      v[i] = (i0 + i <= M) ? rowptr[i0 + i] : 0;
      t += v[i];
      v[i] = t;  // inclusive within the thread
    }
    // inclusive scan of the thread totals across the wave
    long long x = t;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const long long y = __shfl_up(x, off);
      if (lane >= off) x += y;
    }
    if (lane == 63) wave_tot[wave] = x;
    __syncthreads();
    long long before = carry;
    long long step = 0;
    for (int w = 0; w < kScanThreads / 64; ++w) {
      if (w < wave) before += wave_tot[w];
      step += wave_tot[w];
    }
    before += x - t;  // exclusive prefix of this thread
#pragma unroll
    for (int i = 0; i < kScanItems; ++i)
      if (i0 + i <= M) rowptr[i0 + i] = static_cast<int>(before + v[i]);
    carry += step;
    __syncthreads();  // wave_tot is rewritten by the next step
  }
  if (threadIdx.x == 0) {
    rowptr[0] = 0;
    *total = carry;
  }
}

// One wave per row: the kept elements of 64 columns at a time, placed by a
// ballot prefix so the row's order is the column order.
__global__ __launch_bounds__(kToolBlock) void d2c_fill_kernel(int M, int K, const float* A,
                                                              long long lda, float tol,
                                                              const int* rowptr, int* colidx,
                                                              float* vals) {
  const int lane = lane_id();
  const int nw = blockDim.x >> 6;
  const unsigned long long below = (1ULL << lane) - 1ULL;
  for (int row = blockIdx.x * nw + (threadIdx.x >> 6); row < M; row += gridDim.x * nw) {
    const float* a = A + (long long)row * lda;
    int pos = rowptr[row];
    for (int c0 = 0; c0 < K; c0 += 64) {
      const int c = c0 + lane;
      const float v = c < K ? a[c] : 0.0f;
      const bool k = c < K && keep(v, tol);
      const unsigned long long m = __ballot(k);
      if (k) {
        const int at = pos + __popcll(m & below);
        colidx[at] = c;
        vals[at] = v;
      }
      pos += __popcll(m);
    }
  }
}

__global__ void zero_int_kernel(int* p) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *p = 0;
}

// *out = max over rows of rowptr[r + 1] - rowptr[r] (0 when M == 0).
__global__ __launch_bounds__(kToolBlock) void max_row_kernel(int M, const int* rowptr, int* out) {
  __shared__ int s_max;
  if (threadIdx.x == 0) s_max = 0;
  __syncthreads();
  int mx = 0;
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < M; r += gridDim.x * blockDim.x)
    mx = max(mx, rowptr[r + 1] - rowptr[r]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off));
  if (lane_id() == 0 && mx > 0) atomicMax(&s_max, mx);
  __syncthreads();
  if (threadIdx.x == 0 && s_max > 0) atomicMax(out, s_max);
}

// dst[i] = src[i] for values that fit int32; *overflow = 1 if any does not
// (dst then holds the low 32 bits there).
__global__ __launch_bounds__(kToolBlock) void narrow_kernel(const long long* src, int* dst,
                                                            long long n, int* overflow) {
  bool bad = false;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x) {
    const long long v = src[i];
    bad |= v < INT32_MIN || v > INT32_MAX;
    dst[i] = static_cast<int>(v);
  }
  if (overflow && __ballot(bad) && lane_id() == 0) *overflow = 1;
}

int tool_blocks(long long work, int per_block) {
  return static_cast<int>(std::max<long long>(1, std::min<long long>(kToolMaxBlocks, (work + per_block - 1) / per_block)));
}

int status_of(hipError_t e) { return e == hipSuccess ? CSRSPMM_STATUS_SUCCESS : static_cast<int>(e); }

}  // namespace
}  // namespace csrspmm_hip

using namespace csrspmm_hip;

extern "C" {

int csrspmm_dense2csr_count_f32(int M, int K, const float* dense, long long ld, float tol,
                                int* rowptr, long long* nnz_out, void* stream) {
  if (M < 0 || K < 0 || !rowptr || !nnz_out || (M > 0 && K > 0 && (!dense || ld < K)))
    return CSRSPMM_STATUS_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  if (M > 0) {  // K == 0 leaves every count 0 without touching dense
    hipLaunchKernelGGL(d2c_count_kernel, dim3(tool_blocks(M, kToolBlock / 64)), dim3(kToolBlock), 0,
                       s, M, K, dense, ld, tol, rowptr);
  }
  hipLaunchKernelGGL(scan_rowptr_kernel, dim3(1), dim3(kScanThreads), 0, s, rowptr, M, nnz_out);
  return status_of(hipGetLastError());
}

int csrspmm_dense2csr_fill_f32(int M, int K, const float* dense, long long ld, float tol,
                               const int* rowptr, int* colidx, float* vals, void* stream) {
  if (M < 0 || K < 0 || !rowptr || (M > 0 && K > 0 && (!dense || ld < K)))
    return CSRSPMM_STATUS_INVALID_VALUE;
  if (M == 0 || K == 0) return CSRSPMM_STATUS_SUCCESS;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  hipLaunchKernelGGL(d2c_fill_kernel, dim3(tool_blocks(M, kToolBlock / 64)), dim3(kToolBlock), 0,
                     s, M, K, dense, ld, tol, rowptr, colidx, vals);
  return status_of(hipGetLastError());
}

int csrspmm_csr_max_row_nnz(int M, const int* rowptr, int* max_out, void* stream) {
  if (M < 0 || !max_out || (M > 0 && !rowptr)) return CSRSPMM_STATUS_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  hipLaunchKernelGGL(zero_int_kernel, dim3(1), dim3(64), 0, s, max_out);
  if (M > 0)
    hipLaunchKernelGGL(max_row_kernel, dim3(tool_blocks(M, kToolBlock)), dim3(kToolBlock), 0, s, M,
                       rowptr, max_out);
  return status_of(hipGetLastError());
}

int csrspmm_indices_i64_to_i32(const long long* src, int* dst, long long n, int* overflow_out,
                               void* stream) {
  if (n < 0 || (n > 0 && (!src || !dst))) return CSRSPMM_STATUS_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  if (overflow_out) hipLaunchKernelGGL(zero_int_kernel, dim3(1), dim3(64), 0, s, overflow_out);
  if (n > 0)
    hipLaunchKernelGGL(narrow_kernel, dim3(tool_blocks(n, kToolBlock)), dim3(kToolBlock), 0, s, src,
                       dst, n, overflow_out);
  return status_of(hipGetLastError());
}

}  // extern "C"
