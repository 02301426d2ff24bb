// Naive and NaiveSmem for gfx950 (reference src/device/csrspmm_naive.cu:11-39,
// src/device/csrspmm_naive_smem.cu:5-44).
//
// Both keep the reference's "one thread per output element C[row, col]"
// decomposition and its sequential CSR-order accumulation, laid out for
// wave64: a wave covers 64 consecutive columns of one row, so the row index,
// its rowptr bounds and every (col, val) pair are wave-uniform and come in
// through the scalar cache (s_load), while each lane gathers one float of the
// B row (256 B per wave per nonzero, coalesced).
//
// NaiveSmem: a block covers up to 256 columns of one row and stages the row's
// (col, val) pairs through LDS in 256-entry chunks, so each pair is read from
// global memory once per block instead of once per wave.  Barriers sit at
// block-uniform trip counts (the reference places __syncthreads inside a
// per-row loop after an early return, csrspmm_naive_smem.cu:19,37,40).

#include "common.hpp"

namespace csrspmm_hip {

namespace {

constexpr int kNaiveWaves = 4;
constexpr int kNaiveUnroll = 8;
// A long row is one wave's (or block's) chain of dependent batches: batches
// of kNaiveLongUnroll gathers in flight come before the 8-wide ones and the
// tail.  Measured on MI355X per call against 8 throughout: Naive XL 1878 ->
// 1380 us, R-MAT N = 64 4593 -> 3130 us, medium 63.7 -> 57.8 us; NaiveSmem
// XL 1792 -> 1451 us, R-MAT 3858 -> 2913 us (16 or 64 in flight: slower).
#ifndef CSRSPMM_NAIVE_LONG_UNROLL
#define CSRSPMM_NAIVE_LONG_UNROLL 32
#endif
constexpr int kNaiveLongUnroll = CSRSPMM_NAIVE_LONG_UNROLL;

__global__ __launch_bounds__(kNaiveWaves * 64) void naive_kernel(Problem p, int ntile) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id();
  const int tile = blockIdx.x % ntile;
  const int row = (blockIdx.x / ntile) * kNaiveWaves + wave;
  if (row >= p.M) return;
  const int col = tile * 64 + lane;
  const bool valid = col < p.N;
  const int start = p.rowptr[row];
  const int end = p.rowptr[row + 1];
  const float* bc = p.B + col;
  float sum = 0.0f;
  int j = start;
  // U gathers of the row in flight, then the next U, in CSR order
  auto batch = [&](auto u_const) {
    constexpr int U = decltype(u_const)::value;
    int c[U];
    float v[U];
    float b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      c[u] = p.colidx[j + u];
      v[u] = p.vals[j + u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) b[u] = valid ? bc[(long long)c[u] * p.ldb] : 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) sum = __builtin_fmaf(v[u], b[u], sum);
    j += U;
  };
  while (j + kNaiveLongUnroll <= end) batch(std::integral_constant<int, kNaiveLongUnroll>{});
  while (j + kNaiveUnroll <= end) batch(std::integral_constant<int, kNaiveUnroll>{});
  for (; j < end; ++j) {
    const int c = p.colidx[j];
    const float v = p.vals[j];
    const float b = valid ? bc[(long long)c * p.ldb] : 0.0f;
    sum = __builtin_fmaf(v, b, sum);
  }
  if (valid) {
    float* cp = p.C + (long long)row * p.ldc + col;
    st_c(cp, epi1(p.epi, p.alpha, p.beta, sum, cp));
  }
}

constexpr int kSmemChunk = 256;

__global__ __launch_bounds__(256) void naive_smem_kernel(Problem p, int ntile, int cols_per_block) {
  __shared__ int s_col[kSmemChunk];
  __shared__ float s_val[kSmemChunk];
  const int tile = blockIdx.x % ntile;
  const int row = blockIdx.x / ntile;  // block-uniform: every barrier below is reached by all threads
  const int t = threadIdx.x;
  const int col = tile * cols_per_block + t;
  const bool valid = col < p.N;
  const int start = p.rowptr[row];
  const int end = p.rowptr[row + 1];
  const float* bc = p.B + col;
  float sum = 0.0f;
  const int nthreads = blockDim.x;
  for (int base = start; base < end; base += kSmemChunk) {
    const int cnt = min(kSmemChunk, end - base);
    for (int i = t; i < cnt; i += nthreads) {
      s_col[i] = ld_stream(p.colidx + base + i);
      s_val[i] = ld_stream(p.vals + base + i);
    }
    __syncthreads();
    int k = 0;
    auto batch = [&](auto u_const) {
      constexpr int U = decltype(u_const)::value;
      float b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = valid ? bc[(long long)s_col[k + u] * p.ldb] : 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) sum = __builtin_fmaf(s_val[k + u], b[u], sum);
      k += U;
    };
    while (k + kNaiveLongUnroll <= cnt) batch(std::integral_constant<int, kNaiveLongUnroll>{});
    while (k + kNaiveUnroll <= cnt) batch(std::integral_constant<int, kNaiveUnroll>{});
    for (; k < cnt; ++k) {
      const float b = valid ? bc[(long long)s_col[k] * p.ldb] : 0.0f;
      sum = __builtin_fmaf(s_val[k], b, sum);
    }
    __syncthreads();  // chunk fully consumed before the next overwrite
  }
  if (valid) {
    float* cp = p.C + (long long)row * p.ldc + col;
    st_c(cp, epi1(p.epi, p.alpha, p.beta, sum, cp));
  }
}

}  // namespace

hipError_t launch_naive(const Problem& p, hipStream_t s) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  const int ntile = div_up_host(p.N, 64);
  const long long blocks = (long long)div_up_host(p.M, kNaiveWaves) * ntile;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  timing_before_main(s);
  hipLaunchKernelGGL(naive_kernel, dim3((unsigned)blocks), dim3(kNaiveWaves * 64), 0, s, p, ntile);
  const hipError_t e = hipGetLastError();
  timing_after_main(s);
  return e;
}

hipError_t launch_naive_smem(const Problem& p, hipStream_t s) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  const int cols_per_block = p.N >= 256 ? 256 : ((p.N + 63) / 64) * 64;
  const int ntile = div_up_host(p.N, cols_per_block);
  const long long blocks = (long long)p.M * ntile;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  timing_before_main(s);
  hipLaunchKernelGGL(naive_smem_kernel, dim3((unsigned)blocks), dim3(cols_per_block), 0, s, p, ntile,
                     cols_per_block);
  const hipError_t e = hipGetLastError();
  timing_after_main(s);
  return e;
}

}  // namespace csrspmm_hip
