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
//     non-decreasing (any violation clears the flag of win[id]), and records where each
//     panel starts: bnd[id][q] = the first position whose column lies in
//     panel q or later (the row end when there is none).  With sorted
//     columns every q in [0, P] is written exactly once, by the wave that
//     holds the position where the panel index first reaches q.
//  2. panel_sched_kernel, one workgroup: compacts the flagged rows into
//     list[] in row order (at most nl_max of them; pidx[id] = their index,
//     -1 elsewhere), gives XCD x the panels [x P / 8, (x + 1) P / 8), and
//     estimates the panel loads from up to kDevPanelSample rows (the first
//     listed row in each of that many equal ranges of windows) to turn panels off for this call when the heaviest panel carries more
//     than kPanelSkewMax times the mean (hot columns, as in R-MAT, already
//     give L2 reuse) or the heaviest XCD range more than 1.5 times the mean.
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

constexpr int kSchedThreads = 1024;
constexpr int kXcdSkewMax2 = 3;  // heaviest XCD range at most 1.5 (= 3 / 2) x the mean

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
    if (__ballot(bad) && lane == 0) reinterpret_cast<int*>(d.win + id)[3] = 0;
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

__global__ __launch_bounds__(kSchedThreads) void panel_sched_kernel(Problem p) {
  const DevPanels& d = p.dp;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wave = t >> 6;
  constexpr int kWavesS = kSchedThreads / 64;
  constexpr int kPer = 16;  // windows per thread per pass
  constexpr int kPass = kSchedThreads * kPer;
  __shared__ int s_wsum[kWavesS];
  __shared__ int s_base;
  __shared__ int s_id[kDevPanelSample];
  __shared__ int s_w[kPanelMaxPanels];
  __shared__ unsigned char s_flag[kPass];
  __shared__ int s_excl[kSchedThreads];
  __shared__ unsigned s_mask[kSchedThreads];
  const int P = d.P;

  // 1. Compaction of the flagged ids, in id (= row) order, kPass windows per
  // pass.  The flags are read coalesced into LDS (window k0 + u * 1024 + t),
  // thread t counts windows [k0 + kPer t, k0 + kPer (t + 1)) there, a block
  // scan gives each thread its first list position, and pidx / list are
  // written coalesced again, each window's position being its thread's
  // start plus the flags before it in that thread's mask.  The sample for the
  // panel loads is found on the way: the first listed id of each of
  // kDevPanelSample equal ranges of window ids (LDS atomicMin, so the choice
  // does not depend on timing).
  if (t == 0) s_base = 0;
  for (int q = t; q < P; q += kSchedThreads) s_w[q] = 0;
  if (t < kDevPanelSample) s_id[t] = 0x7fffffff;
  for (int k0 = 0; k0 < d.nwin; k0 += kPass) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int k = k0 + u * kSchedThreads + t;
      s_flag[u * kSchedThreads + t] = k < d.nwin && reinterpret_cast<const int*>(d.win + k)[3] == 1;
    }
    __syncthreads();
    unsigned mask = 0;
#pragma unroll
    for (int u = 0; u < kPer; ++u) mask |= (unsigned)s_flag[kPer * t + u] << u;
    const int cnt = __builtin_popcount(mask);
    const int incl = wave_incl_scan(cnt, lane);
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    int excl = s_base + incl - cnt;
    for (int v = 0; v < wave; ++v) excl += s_wsum[v];
    s_excl[t] = excl;
    s_mask[t] = mask;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int j = u * kSchedThreads + t;  // window k0 + j, counted by thread j / kPer
      const int k = k0 + j;
      if (k < d.nwin) {
        const unsigned m = s_mask[j / kPer];
        const int bit = j % kPer;
        const int i = s_excl[j / kPer] + __builtin_popcount(m & ((1u << bit) - 1u));
        const bool take = ((m >> bit) & 1u) && i < d.nl_max;
        d.pidx[k] = take ? i : -1;
        if (take) {
          d.list[i] = k;
          atomicMin(&s_id[(int)(((long long)k * kDevPanelSample) / d.nwin)], k);
        }
      }
    }
    if (t == 0) {
      int tot = 0;
      for (int v = 0; v < kWavesS; ++v) tot += s_wsum[v];
      s_base += tot;
    }
    __syncthreads();
  }
  const int nl = min(s_base, d.nl_max);

  // 2. Panel loads of the sampled rows: pair m = (sample m / P, panel m % P),
  // all loads of a thread in flight at once (empty ranges have no sample).
  constexpr int kPairs = kDevPanelSample * kPanelMaxPanels / kSchedThreads;
  const int npairs = kDevPanelSample * P;
  int b0[kPairs], b1[kPairs];
#pragma unroll
  for (int u = 0; u < kPairs; ++u) {
    const int m = t + u * kSchedThreads;
    b0[u] = b1[u] = 0;
    const int id = m < npairs ? s_id[m / P] : 0x7fffffff;
    if (id != 0x7fffffff) {
      const int* b = d.bnd + (long long)id * (P + 1) + (m % P);
      b0[u] = b[0];
      b1[u] = b[1];
    }
  }
#pragma unroll
  for (int u = 0; u < kPairs; ++u) {
    const int m = t + u * kSchedThreads;
    if (m < npairs) atomicAdd(&s_w[m % P], max(b1[u] - b0[u], 0));
  }
  __syncthreads();

  // 3. XCD ranges and the skew rules (wave 0; lane l holds panels 4l .. 4l+3).
  // XCD x takes the panels [x P / kXcds, (x + 1) P / kXcds): equal ranges, so
  // the host can size the pieces grid.  Panels stay off for this call when
  // the heaviest panel carries more than kPanelSkewMax times the mean panel
  // load, or the heaviest XCD range more than kXcdSkewMax times the mean.
  if (wave != 0) return;
  long long wq[4];
  long long total = 0, mx = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int q = 4 * lane + u;
    wq[u] = q < P ? s_w[q] : 0;
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
  if (lane == 0) d.sched[0] = skewed ? 0 : nl;
}

}  // namespace

hipError_t launch_panel_schedule(const Problem& p, hipStream_t s) {
  if (p.dp.P <= 0 || p.dp.nwin <= 0) return hipSuccess;
  hipLaunchKernelGGL(panel_window_kernel, dim3(div_up_host(p.dp.nwin, 4)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(panel_sched_kernel, dim3(1), dim3(kSchedThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace csrspmm_hip
