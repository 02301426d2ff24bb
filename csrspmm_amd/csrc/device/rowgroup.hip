// Warp-per-row family for gfx950: WarpPerRow, WarpPerRowFp4, WarpPerRowSmem,
// WarpPerRowSmemFp4 (reference src/device/csrspmm_warp_per_row*.cu).
//
// Mapping (wave64): a group of G lanes owns one CSR row; lane l of the group
// owns column chunks l, l+G, ..., each VEC floats wide (VEC = 4 is the
// float4 "Fp4" form, 16-byte global_load_dwordx4 gathers of B rows).  With
// N = 128 and VEC = 4 a group is 32 lanes and a wave carries two rows; with
// N = 256 one row fills the wave.  Each lane keeps T chunk accumulators in
// registers so A is read once per row (the reference re-reads A once per
// 32-column pass, csrspmm_warp_per_row.cu:34-43).
//
// Per output element the products are summed sequentially in CSR order with
// fma, the same order as the reference kernels (csrspmm_warp_per_row.cu:37-43),
// so rows processed whole reproduce its accumulation.  The (col, val) pairs
// of a chunk of G nonzeros are loaded coalesced (one per lane) and broadcast
// to the group: by v_readlane / ds_bpermute in the register variants, through
// a per-wave LDS stage in the Smem variants.  U independent B-row gathers are
// issued before their fmas to keep U x 16 B per lane in flight.
//
// Skew: rows longer than kSplitLen nonzeros are cut into kSplitLen segments.
// A plan kernel lists them; a persistent phase of the main kernel computes
// each segment's partial sum into the workspace; a combine kernel adds the
// partials of a row in segment order and applies the epilogue.  Every step is
// deterministic (no float atomics), so results repeat bit for bit.

#include "common.hpp"

namespace csrspmm_hip {

namespace {

constexpr int kWaves = 4;  // waves per block (256 threads)

__device__ __forceinline__ void wave_lds_sync() {
  // LDS stage is private to the wave: order its writes against the group's
  // reads (and the next chunk's overwrite) without a block barrier.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum of val[j] * B[col[j], cols of this lane] over j in [start, end).
template <int VEC, int G, int T, int U, bool LDS>
__device__ __forceinline__ void accumulate_range(const Problem& p, int start, int end, int gl,
                                                 int gbase, int2* stage,
                                                 const float* const (&bcol)[T],
                                                 const bool (&cval)[T],
                                                 typename Vec<VEC>::T (&acc)[T]) {
  using VT = typename Vec<VEC>::T;
  int j = start + gl;
  int cj = 0;
  float vj = 0.0f;
  if (j < end) {
    cj = ld_stream(p.colidx + j);
    vj = ld_stream(p.vals + j);
  }
  for (int base = start; base < end; base += G) {
    // Prefetch the next chunk's (col, val) while this chunk's gathers run.
    const int jn = base + G + gl;
    int cn = 0;
    float vn = 0.0f;
    if (jn < end) {
      cn = ld_stream(p.colidx + jn);
      vn = ld_stream(p.vals + jn);
    }
    const int cnt = min(G, end - base);
    if constexpr (LDS) {
      stage[gbase + gl] = make_int2(cj, __float_as_int(vj));
      wave_lds_sync();
    }
    for (int k = 0; k < cnt; k += U) {
      int c[U];
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kk = (k + u) & (G - 1);
        if constexpr (LDS) {
          const int2 e = stage[gbase + kk];
          c[u] = e.x;
          v[u] = __int_as_float(e.y);
        } else {
          c[u] = group_bcast<G>(cj, gbase, kk);
          v[u] = group_bcast<G>(vj, gbase, kk);
        }
      }
      VT b[U][T];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = (k + u) < cnt;
        const long long roff = (long long)c[u] * p.ldb;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          b[u][t] = Vec<VEC>::zero();
          if (ok && cval[t]) b[u][t] = ld_b<VEC>(bcol[t] + roff);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if ((k + u) < cnt) {
#pragma unroll
          for (int t = 0; t < T; ++t) acc[t] = fma_v(v[u], b[u][t], acc[t]);
        }
      }
    }
    if constexpr (LDS) wave_lds_sync();
    cj = cn;
    vj = vn;
  }
}

template <int VEC, int G, int T>
__device__ __forceinline__ void panel_setup(const Problem& p, int c0, int gl, const float* (&bcol)[T],
                                            bool (&cval)[T], int (&col)[T]) {
#pragma unroll
  for (int t = 0; t < T; ++t) {
    col[t] = c0 + (gl + G * t) * VEC;
    cval[t] = col[t] < p.N;  // VEC == 4 requires N % 4 == 0 (host-checked)
    bcol[t] = p.B + col[t];
  }
}

template <int VEC, int G, int T, int U, bool LDS>
__global__ __launch_bounds__(kWaves * 64) void rowgroup_kernel(Problem p, int seg_blocks) {
  using VT = typename Vec<VEC>::T;
  constexpr int GPW = 64 / G;          // groups (rows) per wave
  constexpr int GPB = kWaves * GPW;    // groups per block
  constexpr int PW = G * VEC * T;      // columns per panel
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gl = lane & (G - 1);
  const int gbase = lane & ~(G - 1);
  const int gid = wave * GPW + lane / G;  // group index within block

  __shared__ int2 stage_all[LDS ? kWaves * 64 : 1];
  int2* stage = stage_all + (LDS ? wave * 64 : 0);

  const float* bcol[T];
  bool cval[T];
  int col[T];

  if ((int)blockIdx.x < seg_blocks) {
    // Persistent phase: segments of split rows, grid-strided.  Exits at once
    // when the plan found no long rows (or flagged an overflow, which only a
    // malformed CSR can cause).
    if (p.counters[2] != 0) return;
    const int nseg = min(p.counters[0], p.seg_cap);
    for (int s = blockIdx.x * GPB + gid; s < nseg; s += seg_blocks * GPB) {
      const int2 si = p.seg_info[s];
      const int rs = p.rowptr[si.x];
      const int re = p.rowptr[si.x + 1];
      const int start = rs + si.y * kSplitLen;
      const int end = min(re, start + kSplitLen);
      for (int c0 = 0; c0 < p.N; c0 += PW) {
        panel_setup<VEC, G, T>(p, c0, gl, bcol, cval, col);
        VT acc[T];
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = Vec<VEC>::zero();
        accumulate_range<VEC, G, T, U, LDS>(p, start, end, gl, gbase, stage, bcol, cval, acc);
        float* prow = p.partials + (long long)s * p.ldp;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if (cval[t]) *reinterpret_cast<VT*>(prow + col[t]) = acc[t];
        }
      }
    }
    return;
  }

  const int row = ((int)blockIdx.x - seg_blocks) * GPB + gid;
  if (row >= p.M) return;
  const int start = p.rowptr[row];
  const int end = p.rowptr[row + 1];
  if (p.plan && end - start > kSplitLen) return;  // handled by segments + combine
  float* crow = p.C + (long long)row * p.ldc;
  for (int c0 = 0; c0 < p.N; c0 += PW) {
    panel_setup<VEC, G, T>(p, c0, gl, bcol, cval, col);
    VT acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = Vec<VEC>::zero();
    accumulate_range<VEC, G, T, U, LDS>(p, start, end, gl, gbase, stage, bcol, cval, acc);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (cval[t]) store_epi<VEC>(p, crow + col[t], acc[t]);
    }
  }
}

__global__ void zero_counters_kernel(int* counters) {
  if (threadIdx.x < 4) counters[threadIdx.x] = 0;
}

// Lists rows longer than kSplitLen and gives each a contiguous range of
// segment slots.  Slot order depends on atomic arrival, but every segment's
// nonzero range and the combine order depend only on (row, segment index),
// so the arithmetic does not.
__global__ __launch_bounds__(256) void plan_kernel(Problem p) {
  const int stride = gridDim.x * blockDim.x;
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < p.M; r += stride) {
    const int len = p.rowptr[r + 1] - p.rowptr[r];
    if (len > kSplitLen) {
      const int nseg = div_up(len, kSplitLen);
      const int base = atomicAdd(&p.counters[0], nseg);
      const int li = atomicAdd(&p.counters[1], 1);
      if (base + nseg <= p.seg_cap && li < p.long_cap && base >= 0) {
        p.long_rows[li] = make_int4(r, base, nseg, 0);
        for (int k = 0; k < nseg; ++k) p.seg_info[base + k] = make_int2(r, k);
      } else {
        atomicOr(&p.counters[2], 1);
      }
    }
  }
}

// One wave per split row: C[row] = epilogue(sum over segments, in order, of partials).
template <int VEC>
__global__ __launch_bounds__(256) void combine_kernel(Problem p) {
  using VT = typename Vec<VEC>::T;
  if (p.counters[2] != 0) return;
  const int nlong = min(p.counters[1], p.long_cap);
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  for (int l = blockIdx.x * nw + wave; l < nlong; l += gridDim.x * nw) {
    const int4 lr = p.long_rows[l];
    float* crow = p.C + (long long)lr.x * p.ldc;
    for (int c = lane * VEC; c < p.N; c += 64 * VEC) {
      const float* src = p.partials + (long long)lr.y * p.ldp + c;
      VT acc = Vec<VEC>::zero();
      int k = 0;
      for (; k + 4 <= lr.z; k += 4) {
        const VT a0 = *reinterpret_cast<const VT*>(src + (long long)(k + 0) * p.ldp);
        const VT a1 = *reinterpret_cast<const VT*>(src + (long long)(k + 1) * p.ldp);
        const VT a2 = *reinterpret_cast<const VT*>(src + (long long)(k + 2) * p.ldp);
        const VT a3 = *reinterpret_cast<const VT*>(src + (long long)(k + 3) * p.ldp);
        acc = add_v(add_v(add_v(add_v(acc, a0), a1), a2), a3);
      }
      for (; k < lr.z; ++k) acc = add_v(acc, *reinterpret_cast<const VT*>(src + (long long)k * p.ldp));
      store_epi<VEC>(p, crow + c, acc);
    }
  }
}

template <int VEC, int G, int T, int U, bool LDS>
hipError_t launch_rg(const Problem& p, hipStream_t s) {
  constexpr int GPB = kWaves * (64 / G);
  const int row_blocks = div_up_host(p.M, GPB);
  const int seg_blocks = p.plan ? kPersistentBlocks : 0;
  const long long blocks = (long long)row_blocks + seg_blocks;
  if (blocks == 0) return hipSuccess;
  timing_before_main(s);
  hipLaunchKernelGGL((rowgroup_kernel<VEC, G, T, U, LDS>), dim3((unsigned)blocks), dim3(kWaves * 64),
                     0, s, p, seg_blocks);
  const hipError_t e = hipGetLastError();
  timing_after_main(s);
  return e;
}

}  // namespace

static inline int pow2_ceil(int x) {
  int v = 1;
  while (v < x) v <<= 1;
  return v;
}

template <bool LDS>
static hipError_t dispatch_vec4(const Problem& p, hipStream_t s) {
  const int nv = p.N / 4;
  const int G = nv >= 64 ? 64 : (pow2_ceil(nv) < 4 ? 4 : pow2_ceil(nv));
  if (G < 64) {
    switch (G) {
      case 4: return launch_rg<4, 4, 1, 8, LDS>(p, s);
      case 8: return launch_rg<4, 8, 1, 8, LDS>(p, s);
      case 16: return launch_rg<4, 16, 1, 8, LDS>(p, s);
      default: return launch_rg<4, 32, 1, 8, LDS>(p, s);
    }
  }
  const int t = (nv + 63) / 64;
  if (t <= 1) return launch_rg<4, 64, 1, 8, LDS>(p, s);
  if (t <= 2) return launch_rg<4, 64, 2, 4, LDS>(p, s);
  return launch_rg<4, 64, 4, 2, LDS>(p, s);  // N > 1024 loops over 1024-column panels
}

template <bool LDS>
static hipError_t dispatch_vec1(const Problem& p, hipStream_t s) {
  const int n = p.N;
  const int G = n >= 64 ? 64 : (pow2_ceil(n) < 4 ? 4 : pow2_ceil(n));
  if (G < 64) {
    switch (G) {
      case 4: return launch_rg<1, 4, 1, 8, LDS>(p, s);
      case 8: return launch_rg<1, 8, 1, 8, LDS>(p, s);
      case 16: return launch_rg<1, 16, 1, 8, LDS>(p, s);
      default: return launch_rg<1, 32, 1, 8, LDS>(p, s);
    }
  }
  const int t = (n + 63) / 64;
  if (t <= 1) return launch_rg<1, 64, 1, 8, LDS>(p, s);
  if (t <= 2) return launch_rg<1, 64, 2, 8, LDS>(p, s);
  if (t <= 4) return launch_rg<1, 64, 4, 8, LDS>(p, s);
  return launch_rg<1, 64, 8, 4, LDS>(p, s);  // N > 512 loops over 512-column panels
}

hipError_t launch_rowgroup(const Problem& p, int vec, bool lds, hipStream_t s) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  if (p.plan) {
    hipLaunchKernelGGL(zero_counters_kernel, dim3(1), dim3(64), 0, s, p.counters);
    const int pblocks = std::min(div_up_host(p.M, 256), 2048);
    hipLaunchKernelGGL(plan_kernel, dim3(pblocks), dim3(256), 0, s, p);
  }
  hipError_t e;
  if (vec == 4) {
    e = lds ? dispatch_vec4<true>(p, s) : dispatch_vec4<false>(p, s);
  } else {
    e = lds ? dispatch_vec1<true>(p, s) : dispatch_vec1<false>(p, s);
  }
  if (e != hipSuccess) return e;
  if (p.plan) {
    if (vec == 4) {
      hipLaunchKernelGGL(combine_kernel<4>, dim3(kPersistentBlocks / 2), dim3(256), 0, s, p);
    } else {
      hipLaunchKernelGGL(combine_kernel<1>, dim3(kPersistentBlocks / 2), dim3(256), 0, s, p);
    }
    e = hipGetLastError();
  }
  return e;
}

}  // namespace csrspmm_hip
