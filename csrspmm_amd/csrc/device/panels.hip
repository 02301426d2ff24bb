// Per-call column panels: the schedule of the panelized long rows, built on
// the device from the CSR on every call, with no host synchronisation.
//
// A stored plan (plan.hip) cuts rows of >= kPanelMinLen nonzeros at column
// panel boundaries on the host, once.  This file builds the same kind of
// schedule inside each SpMM call, in two launches after plan_kernel:
//
//  1. panel_window_kernel, one wave per window of kPanelMinLen nonzero
//     positions.  A long row covering part of window w is the row of win[w]
//     or of win[w + 1] (a row that starts inside the window also holds the
//     start of the next one), so each wave checks at most two rows.  Over its
//     share of a long row it checks that the columns are in range and
//     non-decreasing (any violation clears dp_flag[id]), and records where
//     each panel starts: bnd[id][q] = the first position whose column lies
//     in panel q or later (the row end when there is none).  With sorted
//     columns every q in [0, P] is written exactly once, by the wave that
//     holds the position where the panel index first reaches q.
//     Every (nwin / kDevPanelSample)-th window's wave also samples the long
//     row holding its first position: 1024 positions spread over the row,
//     added to the call's panel loads per panel (integer atomics into a
//     table that plan_kernel zeroes).
//  2. panel_sched_kernel, 64 workgroups that share nothing.  Workgroup s
//     counts the flags before its equal range of windows (its first list
//     position) and compacts the flagged rows of the range into list[] in
//     row order (at most nl_max in all; pidx[id] = their index, -1
//     elsewhere).  The last one also turns panels off for this call when the
//     heaviest sampled panel load exceeds kPanelSkewMax times the mean (hot
//     columns, as in R-MAT, already give L2 reuse) or the heaviest XCD range
//     1.5 times the mean, and gives XCD x the panels [x P / 8, (x + 1) P / 8).
//
// The pieces kernel (rowgroup.hip) then lets the workgroups of XCD x walk
// the pieces (panel, row) of range x in panel order; the main kernel and the
// combine pass skip the segments of panelized rows, and the combine adds each
// panelized row's P partials in column order.  Every table entry a launch
// reads is written earlier in the same call (or is bounds-checked before
// use), so the workspace may come uninitialised.

#include "common.hpp"

namespace csrspmm_hip {

namespace {

constexpr int kXcdSkewMax2 = 3;  // heaviest XCD range at most 1.5 (= 3 / 2) x the mean
constexpr int kSamplePos = 1024;  // positions sampled per sampled row
static_assert(kSamplePos <= kPanelMinLen, "a sampled row has kSamplePos distinct positions");

__device__ __forceinline__ int clampi(int x, int lo, int hi) { return min(max(x, lo), hi); }

__global__ __launch_bounds__(256) void panel_window_kernel(Problem p) {
  const DevPanels& d = p.dp;
  const int lane = lane_id();
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= d.nwin) return;
  const int pos0 = w * kPanelMinLen;
  const int pos1 = min(pos0 + kPanelMinLen, p.nnz);
  const int4 wa = d.win[w];
  const int4 wb = w + 1 < d.nwin ? d.win[w + 1] : make_int4(-1, 0, 0, 0);
  // Every stride-th window samples the panel loads of the long row holding
  // its first position: kSamplePos positions spread evenly over the whole
  // row (a window alone would cover only a few adjacent panels of a very
  // long row), counted run by run into the call's panel-load table (integer
  // atomics; plan_kernel zeroes the table).  Runs of equal panels are counted
  // exactly whatever the column order, and out-of-range columns are skipped.
  const int stride = max(d.nwin / kDevPanelSample, 1);
  if (w % stride == 0) {
    const int x0 = clampi(wa.y, 0, p.nnz);
    const int x1 = clampi(wa.z, x0, p.nnz);
    if (wa.x >= 0 && wa.x < p.M && x1 - x0 >= kPanelMinLen) {
      constexpr int kS = kSamplePos / 64;
      const long long len = x1 - x0;
      int qv[kS];
#pragma unroll
      for (int u = 0; u < kS; ++u) {
        const int pos = x0 + (int)((long long)(u * 64 + lane) * len / kSamplePos);
        const int cj = p.colidx[pos];
        qv[u] = cj >= 0 && cj < p.K ? cj >> d.wshift : -1;
      }
      int* hist = d.sched + kPanelHist;
#pragma unroll
      for (int u = 0; u < kS; ++u) {
        const int q = qv[u];
        const int qp = __shfl_up(q, 1);
        const unsigned long long bm = __ballot(lane == 0 || qp != q);  // run starts
        if (q >= 0 && (lane == 0 || qp != q)) {
          const unsigned long long above = lane == 63 ? 0ull : bm >> (lane + 1);
          const int next = above ? lane + 1 + __builtin_ctzll(above) : 64;
          atomicAdd(&hist[q], next - lane);
        }
      }
    }
  }
  for (int c = 0; c < 2; ++c) {
    const int4 wi = c == 0 ? wa : wb;
    const int r = wi.x;
    if (r < 0 || r >= p.M || (c == 1 && r == wa.x)) continue;
    const int x0 = clampi(wi.y, 0, p.nnz);
    const int x1 = clampi(wi.z, x0, p.nnz);
    if (x1 - x0 < kPanelMinLen) continue;
    const int id = (x0 + kPanelMinLen - 1) / kPanelMinLen;
    const int lo = max(pos0, x0);
    const int hi = min(pos1, x1);
    if (id >= d.nwin || lo >= hi) continue;
    int* bnd = d.bnd + (long long)id * (d.P + 1);
    // this row's columns in the window, all loads in flight at once; the
    // previous column of lane l is lane l-1's (lane 0: the carry)
    constexpr int kC = kPanelMinLen / 64;
    int cv[kC];
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      const int j = lo + u * 64 + lane;
      cv[u] = j < hi ? p.colidx[j] : 0;
    }
    int carry = lo > x0 ? p.colidx[lo - 1] : -1;
    bool bad = false;
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      const int j = lo + u * 64 + lane;
      int prev = __shfl_up(cv[u], 1);
      const int last = __shfl(cv[u], 63);
      if (lane == 0) prev = carry;
      carry = last;
      if (j < hi) {
        const int cj = cv[u];
        const bool first = j == x0;
        if (cj < 0 || cj >= p.K || (!first && prev > cj)) {
          bad = true;
        } else {
          const int q1 = cj >> d.wshift;                                // panel of this column
          const int q0 = first ? -1 : clampi(prev >> d.wshift, 0, q1);  // panel of the previous one
          for (int q = q0 + 1; q <= q1; ++q) bnd[q] = j;
          if (j == x1 - 1)
            for (int q = q1 + 1; q <= d.P; ++q) bnd[q] = x1;
        }
      }
    }
    if (__ballot(bad) && lane == 0) p.dp_flag[id] = 0;
  }
}

// Inclusive sum over the wave's lanes.
template <class T>
__device__ __forceinline__ T wave_incl_scan(T v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T o = __shfl_up(v, off);
    if (lane >= off) v += o;
  }
  return v;
}

constexpr int kSchedBlocks = 64;  // compaction blocks, one per equal range of windows
constexpr int kSchedThreads = 256;
constexpr int kSchedWaves = kSchedThreads / 64;
constexpr int kSchedPer = 16;  // windows per thread per pass: 16 flag bytes, one aligned load
constexpr int kSchedPass = kSchedThreads * kSchedPer;
static_assert(kPanelMaxPanels <= kSchedThreads, "one thread per panel");
static_assert(kPanelMaxPanels == 4 * 64, "the skew rules give each lane of a wave 4 panels");

// First window of range s: equal ranges, starts rounded down to a multiple
// of 16 so that a thread's 16 flags are one aligned 16-byte load.
__device__ __forceinline__ int sched_lo(int nwin, int s) {
  return s >= kSchedBlocks ? nwin : (int)(((long long)nwin * s / kSchedBlocks) & ~15LL);
}

// Set flag bytes (each 0 or 1) of a 16-byte load, as bits 0..15.
__device__ __forceinline__ unsigned flag_bits(uint4 x) {
  const unsigned w[4] = {x.x, x.y, x.z, x.w};
  unsigned m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int b = 0; b < 4; ++b) m |= ((w[j] >> (8 * b)) & 1u) << (4 * j + b);
  return m;
}

// Block s compacts the flagged windows of its range; the blocks share
// nothing.  The last block, which counts almost every flag anyway, also
// takes the decision for the call: nl, and the skew rules on the sampled
// panel loads.
__global__ __launch_bounds__(kSchedThreads) void panel_sched_kernel(Problem p) {
  const DevPanels& d = p.dp;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wave = t >> 6;
  const int s = blockIdx.x;
  const int lo = sched_lo(d.nwin, s);
  const int hi = sched_lo(d.nwin, s + 1);
  const int P = d.P;
  const bool decide = s == kSchedBlocks - 1;
  const uint4* fl4 = reinterpret_cast<const uint4*>(p.dp_flag);
  __shared__ int s_red[kSchedWaves];
  __shared__ int s_w[kPanelMaxPanels];

  // 1. This block's first list position: the flags before lo, counted by
  // the block itself (a flag byte is 0 or 1, so a word's popcount counts its
  // set bytes).  The first pass's own flags, and in the last block the
  // sampled panel loads, load alongside.
  uint4 own = make_uint4(0, 0, 0, 0);
  if (lo + kSchedPer * t < hi) own = fl4[(lo >> 4) + t];
  const int load = decide && t < P ? d.sched[kPanelHist + t] : 0;
  int before = 0;
#pragma unroll 8
  for (int v = t; v < (lo >> 4); v += kSchedThreads) {
    const uint4 x = fl4[v];
    before += __builtin_popcount(x.x) + __builtin_popcount(x.y) + __builtin_popcount(x.z) +
              __builtin_popcount(x.w);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) before += __shfl_xor(before, off);
  if (lane == 0) s_red[wave] = before;
  __syncthreads();
  int base = 0;
#pragma unroll
  for (int v = 0; v < kSchedWaves; ++v) base += s_red[v];
  __syncthreads();

  // 2. Compaction of the flagged windows of [lo, hi), in window (= row)
  // order: thread t holds windows kt .. kt + 15 of the pass and a block scan
  // gives its first list position.
  for (int k0 = lo; k0 < hi; k0 += kSchedPass) {
    const int kt = k0 + kSchedPer * t;
    uint4 x = own;
    if (k0 != lo) x = kt < hi ? fl4[kt >> 4] : make_uint4(0, 0, 0, 0);
    const int nval = min(max(hi - kt, 0), kSchedPer);
    const unsigned mask = flag_bits(x) & ((1u << nval) - 1u);
    const int cnt = __builtin_popcount(mask);
    const int incl = wave_incl_scan(cnt, lane);
    if (lane == 63) s_red[wave] = incl;
    __syncthreads();
    int excl = base + incl - cnt;
#pragma unroll
    for (int v = 0; v < kSchedWaves; ++v) {
      if (v < wave) excl += s_red[v];
      base += s_red[v];
    }
    __syncthreads();
    if (kt < hi) {
      int pv[kSchedPer];
#pragma unroll
      for (int u = 0; u < kSchedPer; ++u) {
        const int i = excl + __builtin_popcount(mask & ((1u << u) - 1u));
        const bool take = ((mask >> u) & 1u) && i < d.nl_max;
        pv[u] = take ? i : -1;
        if (take) d.list[i] = kt + u;
      }
      // pidx + kt is 16-byte aligned; past hi only in the last range, into
      // the table's padding
      int4* dst = reinterpret_cast<int4*>(d.pidx + kt);
#pragma unroll
      for (int j = 0; j < kSchedPer / 4; ++j)
        if (kt + 4 * j < hi) dst[j] = make_int4(pv[4 * j], pv[4 * j + 1], pv[4 * j + 2], pv[4 * j + 3]);
    }
  }
  if (!decide) return;

  // 3. The decision (base now counts every flag).  Panels stay off for this
  // call when the heaviest sampled panel load exceeds kPanelSkewMax times
  // the mean (hot columns, as in R-MAT, already give L2 reuse), or the
  // heaviest XCD range kXcdSkewMax times the mean.  XCD x takes the panels
  // [x P / kXcds, (x + 1) P / kXcds): equal ranges, so the host can size the
  // pieces grid.
  s_w[t] = load;
  __syncthreads();
  if (wave != 0) return;
  long long wq[4];
  long long total = 0, mx = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    wq[u] = s_w[4 * lane + u];
    total += wq[u];
    mx = max(mx, wq[u]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    total += __shfl_xor(total, off);
    mx = max(mx, __shfl_xor(mx, off));
  }
  long long xmax = 0;
  for (int x = 0; x < kXcds; ++x) {
    const int q0 = (int)((long long)P * x / kXcds), q1 = (int)((long long)P * (x + 1) / kXcds);
    long long lx = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q = 4 * lane + u;
      if (q >= q0 && q < q1) lx += wq[u];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) lx += __shfl_xor(lx, off);
    xmax = max(xmax, lx);
  }
  const bool skewed = total > 0 && (mx * P > (long long)kPanelSkewMax * total ||
                                    xmax * kXcds * 2 > (long long)kXcdSkewMax2 * total);
  if (lane <= kXcds) d.sched[1 + lane] = (int)((long long)P * lane / kXcds);
  if (lane == 0) d.sched[0] = skewed ? 0 : min(base, d.nl_max);
}

}  // namespace

hipError_t launch_panel_schedule(const Problem& p, hipStream_t s) {
  if (p.dp.P <= 0 || p.dp.nwin <= 0) return hipSuccess;
  hipLaunchKernelGGL(panel_window_kernel, dim3(div_up_host(p.dp.nwin, 4)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(panel_sched_kernel, dim3(kSchedBlocks), dim3(kSchedThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace csrspmm_hip
