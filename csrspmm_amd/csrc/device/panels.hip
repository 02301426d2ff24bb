// Per-call column panels: the schedule of the panelized long rows, built on
// the device from the CSR on every call, with no host synchronisation.
//
// A stored plan (plan.hip) cuts rows of >= kPanelMinLen nonzeros at column
// panel boundaries on the host, once.  This file builds the same kind of
// schedule inside each SpMM call, in two launches after plan_kernel:
//
//  1. panel_window_kernel, one wave per window of kPanelMinLen nonzero
//     positions.  A long row covering part of window w is win_row[w] or
//     win_row[w + 1] (a row that starts inside the window also holds the
//     start of the next one), so each wave checks at most two rows.  Over its
//     share of a long row it checks that the columns are in range and
//     non-decreasing (any violation clears flag[id]), and records where each
//     panel starts: bnd[id][q] = the first position whose column lies in
//     panel q or later (the row end when there is none).  With sorted
//     columns every q in [0, P] is written exactly once, by the wave that
//     holds the position where the panel index first reaches q.
//  2. panel_sched_kernel, one workgroup: compacts the flagged rows into
//     list[] in row order (at most nl_max of them; pidx[id] = their index,
//     -1 elsewhere), estimates the load of each panel from up to
//     kDevPanelSample evenly spaced rows, turns panels off for this call when
//     the heaviest panel carries more than kPanelSkewMax times the mean (hot
//     columns, as in R-MAT, already give L2 reuse), and cuts the panels into
//     kXcds contiguous ranges of near-equal load.
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

__device__ __forceinline__ int clampi(int x, int lo, int hi) { return min(max(x, lo), hi); }

__global__ __launch_bounds__(256) void panel_window_kernel(Problem p) {
  const DevPanels& d = p.dp;
  const int lane = lane_id();
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= d.nwin) return;
  const int pos0 = w * kPanelMinLen;
  const int pos1 = min(pos0 + kPanelMinLen, p.nnz);
  const int cand[2] = {d.win_row[w], w + 1 < d.nwin ? d.win_row[w + 1] : -1};
  for (int c = 0; c < 2; ++c) {
    const int r = cand[c];
    if (r < 0 || r >= p.M || (c == 1 && r == cand[0])) continue;
    const int x0 = clampi(p.rowptr[r], 0, p.nnz);
    const int x1 = clampi(p.rowptr[r + 1], x0, p.nnz);
    if (x1 - x0 < kPanelMinLen) continue;
    const int id = (x0 + kPanelMinLen - 1) / kPanelMinLen;
    if (id >= d.nwin || d.win_row[id] != r) continue;  // only for a malformed rowptr
    const int lo = max(pos0, x0);
    const int hi = min(pos1, x1);
    int* bnd = d.bnd + (long long)id * (d.P + 1);
    bool bad = false;
    for (int j0 = lo; j0 < hi; j0 += 8 * 64) {
      int cj[8], pv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {  // 16 loads in flight per lane
        const int j = j0 + u * 64 + lane;
        cj[u] = j < hi ? p.colidx[j] : 0;
        pv[u] = (j < hi && j > x0) ? p.colidx[j - 1] : -1;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u * 64 + lane;
        if (j >= hi) continue;
        if (cj[u] < 0 || cj[u] >= p.K || pv[u] > cj[u]) {
          bad = true;
          continue;
        }
        const int q1 = cj[u] / d.width;                                 // panel of this column
        const int q0 = j > x0 ? clampi(pv[u] / d.width, 0, q1) : -1;  // panel of the previous one
        for (int q = q0 + 1; q <= q1; ++q) bnd[q] = j;
        if (j == x1 - 1)
          for (int q = q1 + 1; q <= d.P; ++q) bnd[q] = x1;
      }
    }
    if (__ballot(bad) && lane == 0) d.flag[id] = 0;
  }
}

__global__ __launch_bounds__(kSchedThreads) void panel_sched_kernel(Problem p) {
  const DevPanels& d = p.dp;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wave = t >> 6;
  constexpr int kWavesS = kSchedThreads / 64;
  __shared__ int s_wave[kWavesS];
  __shared__ int s_base;
  __shared__ long long s_w[kPanelMaxPanels];

  // 1. Compaction of the flagged ids, in id (= row) order.
  if (t == 0) s_base = 0;
  __syncthreads();
  for (int k0 = 0; k0 < d.nwin; k0 += kSchedThreads) {
    const int k = k0 + t;
    const bool f = k < d.nwin && d.flag[k] == 1;
    const unsigned long long m = __ballot(f);
    const int before = __popcll(m & ((1ULL << lane) - 1ULL));
    if (lane == 0) s_wave[wave] = __popcll(m);
    __syncthreads();
    int off = s_base;
    for (int v = 0; v < wave; ++v) off += s_wave[v];
    const int i = off + before;
    if (k < d.nwin) {
      const bool take = f && i < d.nl_max;
      d.pidx[k] = take ? i : -1;
      if (take) d.list[i] = k;
    }
    __syncthreads();
    if (t == 0) {
      int tot = 0;
      for (int v = 0; v < kWavesS; ++v) tot += s_wave[v];
      s_base += tot;
    }
    __syncthreads();
  }
  const int nl = min(s_base, d.nl_max);

  // 2. Panel loads from up to kDevPanelSample evenly spaced rows.
  const int P = d.P;
  const int ns = min(nl, kDevPanelSample);
  for (int q = t; q < P; q += kSchedThreads) s_w[q] = 0;
  __syncthreads();
  if (ns > 0) {
    // thread t: panel q = t % P, samples t / P, t / P + stride, ...
    const int per = kSchedThreads / P > 0 ? kSchedThreads / P : 1;
    const int q = t % P;
    const int s0 = t / P;
    if (s0 < per) {
      long long acc = 0;
      for (int sidx = s0; sidx < ns; sidx += per) {
        const int i = (int)(((long long)sidx * nl) / ns);
        const int* b = d.bnd + (long long)d.list[i] * (P + 1);
        acc += (long long)max(b[q + 1] - b[q], 0);
      }
      atomicAdd(reinterpret_cast<unsigned long long*>(&s_w[q]), (unsigned long long)acc);
    }
  }
  __syncthreads();

  // 3. Skew rule and the XCD ranges: range x ends at the last panel whose
  // load prefix stays within x / kXcds of the total.
  if (t == 0) {
    long long total = 0, mx = 0;
    for (int q = 0; q < P; ++q) {
      total += s_w[q];
      mx = max(mx, s_w[q]);
    }
    const bool skewed = total > 0 && mx * P > (long long)kPanelSkewMax * total;
    d.sched[0] = skewed ? 0 : nl;
    d.sched[1] = 0;
    long long pre = 0;
    int q = 0;
    for (int x = 1; x < kXcds; ++x) {
      if (total > 0) {
        const long long target = total * x / kXcds;
        while (q < P && pre + s_w[q] <= target) pre += s_w[q++];
        d.sched[1 + x] = q;
      } else {
        d.sched[1 + x] = (int)((long long)P * x / kXcds);
      }
    }
    d.sched[1 + kXcds] = P;
  }
}

}  // namespace

hipError_t launch_panel_schedule(const Problem& p, hipStream_t s) {
  if (p.dp.P <= 0 || p.dp.nwin <= 0) return hipSuccess;
  hipLaunchKernelGGL(panel_window_kernel, dim3(div_up_host(p.dp.nwin, 4)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(panel_sched_kernel, dim3(1), dim3(kSchedThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace csrspmm_hip
