// C ABI (include/csrspmm_c.h) over the gfx950 kernels: argument checks,
// variant dispatch, workspace management, CSR validation and the memory
// helpers the g++-built C++ layer uses.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <string.h>
#include <utility>
#include <vector>

#include "../../../include/csrspmm_c.h"
#include "common.hpp"
#include "spmm_internal.h"

namespace csrspmm_hip {

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

WorkspaceLayout workspace_layout(int M, int K, int N, int nnz, int P, bool shares) {
  WorkspaceLayout L{};
  const SegGeom g = seg_geom(nnz);
  L.nslots = nnz >> g.slot_shift;
  // capacity for the merge blocks of either column width, sliced or not
  L.nblocks = merge_blocks(
      M, nnz, std::min({merge_block(1, M, nnz), merge_block(4, M, nnz), sliced_merge_block(M, nnz)}));
  L.ldp = ((long long)N + 3) & ~3LL;
  size_t off = 0;
  L.block_start_off = off;
  off = align256(off + ((size_t)L.nblocks + 1) * sizeof(int));
  L.seg_info_off = off;
  off = align256(off + (size_t)L.nslots * sizeof(int2));
  L.partials_off = off;
  off = align256(off + (size_t)(nnz >> g.seg_shift) * (size_t)L.ldp * sizeof(float));
  L.need_off = off;
  off = align256(off + (size_t)plan_row_blocks(M));
  L.segcnt_off = off;
  off = align256(off + (size_t)L.nslots * sizeof(int));
  L.base_total = off;
  if (P > 0 && K > 0) {
    const long long w = ((long long)K + P - 1) / P;
    L.wshift = 0;
    while ((1LL << L.wshift) < w) ++L.wshift;
    L.P = (int)(((long long)K + (1LL << L.wshift) - 1) >> L.wshift);
    P = L.P;
    L.nwin = (int)(((long long)nnz + kPanelMinLen - 1) / kPanelMinLen);
    const long long per_row = (long long)P * L.ldp * (long long)sizeof(float);
    L.nl_max = (int)std::min<long long>(
        {(long long)L.nwin, std::max<long long>(1, kDevPanelPartialBudget / per_row),
         std::max<long long>(1, ((long long)nnz + kPanelRowCapLen - 1) / kPanelRowCapLen)});
    const size_t nw = (size_t)L.nwin;
    L.win_off = off;
    off = align256(off + nw * sizeof(int4));
    L.flag_off = off;
    off = align256(off + nw);
    L.pidx_off = off;
    off = align256(off + nw * sizeof(int));
    L.list_off = off;
    off = align256(off + (size_t)L.nl_max * sizeof(int));
    L.bnd_off = off;
    off = align256(off + nw * ((size_t)P + 1) * sizeof(int));
    L.sched_off = off;
    off = align256(off + (size_t)(kPanelHist + P) * sizeof(int));
    L.part_off = off;
    off = align256(off + (size_t)L.nl_max * (size_t)P * (size_t)L.ldp * sizeof(float));
  } else if (shares) {
    L.shares = true;
    L.shr_cb_off = off;
    off = align256(off + (size_t)kXcds * sizeof(int));
    L.shr_pb_off = off;
    off = align256(off + (size_t)L.nslots * 2 * sizeof(int4));  // 8 ints per slot
    L.shr_part_off = off;
    off = align256(off + ((size_t)(nnz >> kShareIdxShift) + 1) * (size_t)L.ldp * sizeof(float));
  }
  L.total = off;
  return L;
}

void bind_workspace(Problem& p, void* ws, const WorkspaceLayout& L, int mblk) {
  char* b = static_cast<char*>(ws);
  p.block_start = reinterpret_cast<int*>(b + L.block_start_off);
  p.seg_info = reinterpret_cast<int2*>(b + L.seg_info_off);
  p.partials = reinterpret_cast<float*>(b + L.partials_off);
  p.need = reinterpret_cast<unsigned char*>(b + L.need_off);
  p.need_blocks = plan_row_blocks(p.M);
  p.seg_cnt = reinterpret_cast<int*>(b + L.segcnt_off);
  p.ldp = L.ldp;
  p.nslots = L.nslots;
  p.mblk = mblk;
  p.nblocks = merge_blocks(p.M, p.nnz, mblk);

  p.dp = DevPanels{};
  p.dp_flag = nullptr;
  if (L.P > 0) {
    p.dp.P = L.P;
    p.dp.wshift = L.wshift;
    p.dp.nwin = L.nwin;
    p.dp.nl_max = L.nl_max;
    p.dp.win = reinterpret_cast<int4*>(b + L.win_off);
    p.dp.pidx = reinterpret_cast<int*>(b + L.pidx_off);
    p.dp.list = reinterpret_cast<int*>(b + L.list_off);
    p.dp.bnd = reinterpret_cast<int*>(b + L.bnd_off);
    p.dp.sched = reinterpret_cast<int*>(b + L.sched_off);
    p.dp.part = reinterpret_cast<float*>(b + L.part_off);
    p.dp_flag = reinterpret_cast<unsigned char*>(b + L.flag_off);
  }
  p.shares = L.shares;
  p.shr_cb = L.shares ? reinterpret_cast<int*>(b + L.shr_cb_off) : nullptr;
  p.shr_pb = L.shares ? reinterpret_cast<int4*>(b + L.shr_pb_off) : nullptr;
  p.shr_part = L.shares ? reinterpret_cast<float*>(b + L.shr_part_off) : nullptr;
}

int per_call_panels(int vec, bool plan, int K, int N, int nnz, int hint) {
  if ((vec != 4 && N < kPanelMinScalarN) || !plan || nnz < kPanelMinLen) return 0;
  if (hint >= 0 && hint < kPanelMinLen) return 0;
  const int P = panel_count(K, N);
  return P >= kDevPanelMinPanels ? P : 0;
}

namespace {

bool is_rowgroup(int algo) {
  return algo == CSRSPMM_ALGO_WARP_PER_ROW || algo == CSRSPMM_ALGO_WARP_PER_ROW_FP4 ||
         algo == CSRSPMM_ALGO_WARP_PER_ROW_SMEM || algo == CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4;
}

// The plan pays for itself on large matrices (short rows are streamed,
// long rows split); small ones with no row above kSegLen run as one launch,
// and so do mid-sized ones whose hint rules out long rows (plan_skips).
bool wants_plan(int algo, int M, int K, int N, int nnz, int hint) {
  if (!is_rowgroup(algo)) return false;
  if (plan_skips(M, K, N, nnz, hint)) return false;
  if ((long long)M + nnz >= kPlanMinItems) return true;
  return (hint < 0 || hint > kSegLen) && nnz > kSegLen;
}

int to_status(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

// Library-owned workspaces, one per (device, stream).  hipStreamPerThread
// names a different stream in every host thread, so its workspaces are kept
// per thread as well.  The map holds at most kMaxOwnedWorkspaces entries; a
// new key beyond that evicts the least recently used one.
//
// Threading: every workspace has its own lock, held from the moment a call
// takes it until the call's kernels are enqueued (spmm_impl), so a buffer is
// never freed or regrown between a call taking it and its kernels being
// queued behind it.  Calls on different streams or devices share only
// g_ws_mutex, for the map lookup, not across the enqueue.  Growing a buffer
// synchronises its stream first (the stream is alive: its caller is using
// it); evicting or releasing one takes its lock and synchronises the whole
// device, since the stream it was keyed on may have been destroyed since.
struct WsKey {
  int dev;
  void* stream;
  std::thread::id tid;  // set only for hipStreamPerThread
  bool operator<(const WsKey& o) const {
    if (dev != o.dev) return dev < o.dev;
    if (stream != o.stream) return stream < o.stream;
    return tid < o.tid;
  }
};

struct OwnedWorkspace {
  std::mutex m;
  void* ptr = nullptr;     // ptr, bytes, dead: under m
  size_t bytes = 0;
  bool dead = false;       // released or evicted: look it up again
  unsigned long long last_use = 0;  // under g_ws_mutex
};

constexpr size_t kMaxOwnedWorkspaces = 16;

std::mutex g_ws_mutex;
std::map<WsKey, std::shared_ptr<OwnedWorkspace>> g_ws;
unsigned long long g_ws_clock = 0;

WsKey ws_key(int dev, void* stream) {
  WsKey k{dev, stream, std::thread::id()};
  if (static_cast<hipStream_t>(stream) == hipStreamPerThread) k.tid = std::this_thread::get_id();
  return k;
}

// Frees one workspace after all work on its device has finished.  Caller
// holds w.m.
int free_owned_device_synced(int dev, OwnedWorkspace& w) {
  w.dead = true;
  if (!w.ptr) return 0;
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return (int)e;
  if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
  e = hipDeviceSynchronize();
  hipError_t e2 = hipFree(w.ptr);
  w.ptr = nullptr;
  w.bytes = 0;
  hipError_t e3 = cur != dev ? hipSetDevice(cur) : hipSuccess;
  if (e != hipSuccess) return (int)e;
  if (e2 != hipSuccess) return (int)e2;
  return (int)e3;
}

// Grows w to at least `bytes` (caller holds w.m).
int grow_locked(OwnedWorkspace& w, void* stream, size_t bytes) {
  if (w.bytes >= bytes) return 0;
  if (w.ptr) {
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return (int)e;
    e = hipFree(w.ptr);
    w.ptr = nullptr;
    w.bytes = 0;
    if (e != hipSuccess) return (int)e;
  }
  const size_t want = bytes + bytes / 4;  // headroom against repeated small growth
  if (hipMalloc(&w.ptr, want) != hipSuccess) {
    w.ptr = nullptr;
    (void)hipGetLastError();
    return CSRSPMM_STATUS_ALLOC_FAILED;
  }
  w.bytes = want;
  return 0;
}

// The workspace of (current device, stream), grown to at least `bytes`, in
// *out; on success it stays locked through `lock` (and alive through `held`)
// until the caller has enqueued the kernels that use it, on failure it is
// unlocked.
int owned_workspace(void* stream, size_t bytes, void** out, std::shared_ptr<OwnedWorkspace>& held,
                    std::unique_lock<std::mutex>& lock) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  const WsKey key = ws_key(dev, stream);
  for (;;) {
    {
      std::lock_guard<std::mutex> g(g_ws_mutex);
      auto it = g_ws.find(key);
      if (it == g_ws.end()) {
        if (g_ws.size() >= kMaxOwnedWorkspaces) {
          auto lru = g_ws.begin();
          for (auto j = g_ws.begin(); j != g_ws.end(); ++j)
            if (j->second->last_use < lru->second->last_use) lru = j;
          const std::shared_ptr<OwnedWorkspace> victim = lru->second;
          const int vdev = lru->first.dev;
          g_ws.erase(lru);
          // a call holding the victim's lock never waits for g_ws_mutex
          std::lock_guard<std::mutex> vl(victim->m);
          const int st = free_owned_device_synced(vdev, *victim);
          if (st != 0) return st;
        }
        it = g_ws.emplace(key, std::make_shared<OwnedWorkspace>()).first;
      }
      held = it->second;
      held->last_use = ++g_ws_clock;
    }
    lock = std::unique_lock<std::mutex>(held->m);
    if (!held->dead) break;
    lock.unlock();  // evicted or released between the lookup and the lock
  }
  OwnedWorkspace& w = *held;
  const int st = grow_locked(w, stream, bytes);
  if (st != 0) {
    // unlocked on failure: the caller may retry with a smaller size
    lock.unlock();
    return st;
  }
  *out = w.ptr;
  return 0;
}

}  // namespace

// A float4 call from N = 128 whose column slices would be swept (the plan,
// slice_width and sweep_applies as spmm_impl and the dispatch decide them).
static bool sliced_sweep(int M, int K, int N, int nnz, int hint) {
  const bool plan = wants_plan(CSRSPMM_ALGO_WARP_PER_ROW_FP4, M, K, N, nnz, hint);
  if (!plan) return false;
  const int P = per_call_panels(4, plan, K, N, nnz, hint);
  return slice_width(K, N, P > 0, wide_sweep(4, plan, M, K, nnz)) > 0 &&
         sweep_applies(plan, M, K, nnz, kSliceWidth);
}

// A call from N = 128 that would be cut into column slices (the plan and
// slice_width as spmm_impl decides them).
static bool sliced(int M, int K, int N, int nnz, int hint) {
  const bool plan = wants_plan(CSRSPMM_ALGO_WARP_PER_ROW_FP4, M, K, N, nnz, hint);
  if (!plan) return false;
  const int P = per_call_panels(4, plan, K, N, nnz, hint);
  return slice_width(K, N, P > 0, wide_sweep(4, plan, M, K, nnz)) > 0;
}

// A float4 call from N = 128 cut into column slices that are not swept, or
// swept with fewer than kSweepWideMinPerBand nonzeros per band and row, and
// whose long rows are split by XCD (share_applies).
static bool sliced_shares(int M, int K, int N, int nnz, int hint) {
  const bool plan = wants_plan(CSRSPMM_ALGO_WARP_PER_ROW_FP4, M, K, N, nnz, hint);
  if (!plan) return false;
  const int P = per_call_panels(4, plan, K, N, nnz, hint);
  const int sw = slice_width(K, N, P > 0, wide_sweep(4, plan, M, K, nnz));
  return sw > 0 && !sweep_applies(plan, M, K, nnz, sw, kSweepWideMinPerBand) &&
         share_applies(plan, K, N, nnz, sw, 0, hint);
}

int resolve_algorithm(int algo, int M, int K, int N, int nnz, int hint) {
  if (algo == CSRSPMM_ALGO_AUTO && N % 4 == 0 && N >= 128 && sliced_shares(M, K, N, nnz, hint)) {
    // Column slices that are not swept (or swept with under 4 nonzeros per
    // band), of a matrix whose long rows are split by XCD: the scalar
    // LDS-staged form's 64-lane groups (a slice's 64 columns, one per lane)
    // run four times the waves of the float4 16-lane groups over the short
    // rows and the parts.  Measured on MI355X per call without a hint: R-MAT
    // N = 512 4218 -> 3832 us, N = 256 2156 -> 1886; uniform rows of 16
    // (524288 x 262144) at N = 512 2614 -> 2592; swept with 2 per band,
    // power-law rows (mean 32, 262144^2) at N = 1024 7021 -> 5197 and uniform
    // rows of 32 (262144^2) at N = 1024 5811 -> 4874.
    return CSRSPMM_ALGO_WARP_PER_ROW_SMEM;
  }
  if (algo == CSRSPMM_ALGO_AUTO && N % 4 == 0 && N >= 128 && M > 0 && hint > kLongRow &&
      (long long)hint > 4LL * nnz / M && sliced(M, K, N, nnz, hint)) {
    // Column slices of skewed rows (the hint above both long_row and 4x the
    // mean): the scalar LDS-staged form's 64-lane groups run each slice's
    // long-row chains with four times the waves of the float4 16-lane
    // groups.  Measured on MI355X per call with the hint: power-law rows
    // (mean 32) at K = 65536, N = 256 307 -> 269 us (swept by the float4
    // form) and K = 32768, N = 512 579 -> 337; mean 98 at K = 131072, N = 512
    // 3855 -> 3536; R-MAT N = 256 2303 -> 2186, N = 512 4876 -> 4726.
    // Uniform rows of 200 at K = 65536, N = 256 (the hint within 4x the mean)
    // keep the float4 sweep: 1248 against 1351 us.
    return CSRSPMM_ALGO_WARP_PER_ROW_SMEM;
  }
  if (algo == CSRSPMM_ALGO_AUTO && N % 4 == 0 && N >= 128 && sliced_sweep(M, K, N, nnz, hint)) {
    // Swept column slices run 0-5% faster with the chunks through LDS than
    // broadcast across lanes.  Measured on MI355X per call: large 299 ->
    // 286 us, 65536^2 x 256 with 128 per row 490 -> 465, 65536^2 x 512 with
    // 66 per row 591 -> 564; 16 per row and power-law rows within 0.4%.
    return CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4;
  }
  if (algo == CSRSPMM_ALGO_AUTO && N % 4 == 0 && N >= 128 && M > 0 && sliced(M, K, N, nnz, hint)) {
    // Column slices that do not sweep, of rows averaging 64-511 nonzeros or
    // with the hint at 129-511: a row is one long chain of gathers per
    // slice, and the scalar 64-lane groups run four times the waves of the
    // float4 16-lane ones.  Measured on MI355X per call, bit-identical:
    // uniform rows of 128 at M = 4096, K = 65536, N = 128-1024 1.6-1.9x
    // faster, of 64 at N = 256 1.3x; at M = K = 32768, N = 256 rows of 128
    // 357 -> 289 us and of 300 798 -> 632; 4096^2 x 2048 with 300 per row
    // 1368 -> 607 us, 2048 x 16384 x 1024 with 400 per row 388 -> 275.  On
    // a 64-column band above kSliceCapBand (8 MiB), from 4096 rows, the
    // float4 segments, 8 gathers deep under the residency cap, lead as soon
    // as rows exceed long_row (with the hint: 8192 x 65536 x 256 with 300 per
    // row 241 against 314 us, 16384 x 65536 x 256 with 200 per row 278
    // against 342, 32768 x 65536 x 256 with 132 per row 356 against 442;
    // 4096 x 65536 with 300 per row, since the float4 slices gather through
    // a buffer resource: N = 128 73.2 against 86.3 us, 256 140.9 against
    // 165.7, 1024 563 against 667).  Rows
    // of 512 or more are split into segments (1024 x 65536 x 512 with 1000
    // per row: float4 13% faster).
    const bool mid_rows = (nnz >= 64LL * M && nnz < 512LL * M) || (hint > kLongRow && hint < 2 * kSegLen);
    const bool long_rows = hint > kLongRow || (hint < 0 && nnz > (long long)kLongRow * M);
    const bool wide_band = (long long)K * kSliceWidth * 4 > kSliceCapBand;
    if (mid_rows && !(wide_band && long_rows && M >= 4096)) return CSRSPMM_ALGO_WARP_PER_ROW_SMEM;
  }
  if (algo == CSRSPMM_ALGO_AUTO && N % 4 == 0 && N < 128 && (long long)nnz >= 24LL * M &&
      per_call_panels(4, wants_plan(CSRSPMM_ALGO_WARP_PER_ROW_FP4, M, K, N, nnz, hint), K, N, nnz, hint) > 0) {
    // Below N = 128 the float4 form has the per-call column panels from a
    // 64 MiB B, the scalar form none.  Measured on MI355X per call with the
    // hint: power-law rows at K = 262144 (mean 32) N = 64 320.5 -> 227.4 us,
    // N = 96 470.0 -> 295.9; mean 98 N = 64 896.9 -> 612.3.  R-MAT (15 per
    // row, its panels turned off by the skew) stays scalar: 564 against 599 us
    // at N = 64.
    return CSRSPMM_ALGO_WARP_PER_ROW_FP4;
  }
  if (algo == CSRSPMM_ALGO_AUTO && N % 4 == 0 && N == 128 &&
      (M >= 4096 || (M >= 1024 && plan_skips(M, K, N, nnz, hint))) &&
      (long long)K * N * 4 <= (4LL << 20) && (long long)nnz >= 96LL * M) {
    // A B that stays in the L2s and rows of 96 nonzeros or more on average:
    // the rows are long-row segments, and the scalar LDS-staged form keeps
    // more gathers in flight per row.  Measured on MI355X per call, uniform
    // rows at N = 128 with max_row_nnz given: M = 4096, K = 4096, 205 per row
    // 33.2 -> 23.0 us, 600 per row 81.8 -> 66.8; M = 16384, K = 2048, 205
    // per row 90.7 -> 68.8; but 64 per row, M = 1024, an 8 MiB B (K = 16384)
    // or N = 256 keep float4 within 0-21%.  From M = 1024 when the hint runs
    // the call as one launch (plan_skips), rows summed whole by one group
    // each: M = 1024, K = 2048, 200 per row 13.0 -> 10.5 us; M = 1536, K =
    // 8192, 220 per row 23.1 -> 16.4; M = 2048, K = 2048, 200 per row 13.6 ->
    // 11.2; M = 1024, K = 1024, 160 per row 10.9 -> 10.0.  Rows of 96-159
    // without a hint, M = 4096, K = 4096: 112 per row 23.9 -> 18.2 us, 128
    // per row 29.9 -> 22.1, 144 per row 22.0 -> 21.5; M = 16384, K = 8192,
    // 128 per row 77.0 -> 55.1; M = 8192, K = 8192, 120 per row 43.6 -> 36.5;
    // 64 per row stays even (15.8 against 16.0 us).
    return CSRSPMM_ALGO_WARP_PER_ROW_SMEM;
  }
  return resolve_algorithm(algo, N);
}

int resolve_algorithm(int algo, int N) {
  if (algo == CSRSPMM_ALGO_AUTO) {
    // Measured on MI355X: float4 columns win from N = 128 up, scalar columns
    // below (64-lane groups instead of 16-lane float4 groups), where the
    // LDS-staged form leads.  From N = 128 the broadcast form is ahead on the
    // power-law configs (XL 341.1 -> 333.9 us, the mean-98 config 988 ->
    // 957 us), 1.7% behind on power-law rows at K = 131072, and within 0.3%
    // on the uniform and R-MAT configs.
    return (N % 4 == 0 && N >= 128) ? CSRSPMM_ALGO_WARP_PER_ROW_FP4 : CSRSPMM_ALGO_WARP_PER_ROW_SMEM;
  }
  if (algo < 0 || algo >= CSRSPMM_ALGO_COUNT) return -1;
  return algo;
}

bool is_rowgroup_algorithm(int algo) { return is_rowgroup(algo); }

bool uses_lds(int algo) {
  return algo == CSRSPMM_ALGO_WARP_PER_ROW_SMEM || algo == CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4;
}

int vector_width(int algo, const Problem& p) {
  if (algo != CSRSPMM_ALGO_WARP_PER_ROW_FP4 && algo != CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4) return 1;
  // The float4 forms need 16-byte aligned rows of B and C; otherwise the
  // scalar-column kernel of the same family runs (the reference instead drops
  // the last N % 4 columns, csrspmm_warp_per_row_fp4.cu:29-32).
  const bool ok = (p.N % 4 == 0) && (p.ldc % 4 == 0) &&
                  ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0) &&
                  (p.nnz == 0 || ((p.ldb % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.B) & 15) == 0)));
  return ok ? 4 : 1;
}

int fill_problem(Problem& p, int algo, int M, int K, int N, int nnz, const int* rowptr,
                 const int* colidx, const float* vals, const float* B, long long ldb, float* C,
                 long long ldc, float alpha, float beta, unsigned flags) {
  if (algo < 0 || algo >= CSRSPMM_ALGO_COUNT) return CSRSPMM_STATUS_INVALID_VALUE;
  if (M < 0 || K < 0 || N < 0 || nnz < 0) return CSRSPMM_STATUS_INVALID_VALUE;
  p = Problem{};
  p.row_hint = -1;
  p.M = M;
  p.K = K;
  p.N = N;
  p.nnz = nnz;
  const SegGeom g = seg_geom(nnz);
  p.seg_shift = g.seg_shift;
  p.slot_shift = g.slot_shift;
  p.long_row = g.long_row;
  if (M == 0 || N == 0) return 0;
  if (!rowptr || !C) return CSRSPMM_STATUS_INVALID_VALUE;
  if (nnz > 0 && (!colidx || !vals || !B || K == 0)) return CSRSPMM_STATUS_INVALID_VALUE;
  if (ldc < N || (nnz > 0 && ldb < N)) return CSRSPMM_STATUS_INVALID_VALUE;
  // Merge coordinates (row + nonzero index) and grid sizes must fit int32.
  if ((long long)M + nnz + 1 > 0x7fffffffLL - kMergeBlockMax) return CSRSPMM_STATUS_NOT_SUPPORTED;
  p.rowptr = rowptr;
  p.colidx = colidx;
  p.vals = vals;
  p.B = B;
  p.ldb = ldb;
  p.C = C;
  p.ldc = ldc;
  p.alpha = alpha;
  p.beta = beta;
  if (flags & CSRSPMM_FLAG_C_IS_ZERO)
    p.epi = kEpiZeroC;
  else
    p.epi = (beta == 0.0f) ? kEpiOverwrite : kEpiAccumulate;
  return 0;
}

hipError_t launch_algorithm(int algo, const Problem& p, hipStream_t s) {
  const int vec = vector_width(algo, p);
  switch (algo) {
    case CSRSPMM_ALGO_NAIVE: return launch_naive(p, s);
    case CSRSPMM_ALGO_NAIVE_SMEM: return launch_naive_smem(p, s);
    case CSRSPMM_ALGO_WARP_PER_ROW:
    case CSRSPMM_ALGO_WARP_PER_ROW_FP4:
    case CSRSPMM_ALGO_WARP_PER_ROW_SMEM:
    case CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4: return launch_rowgroup(p, vec, uses_lds(algo), s);
    default: return hipErrorInvalidValue;
  }
}

namespace {

// Device scratch of csrspmm_spmm_f32_noalloc: the workspace of its calls,
// CSRSPMM_NOALLOC_SCRATCH_BYTES per GPU, held by every GPU the library runs
// on until the process ends.  In host code `scratch` names a host-side
// stand-in, not device memory: the device address of each GPU's copy comes
// from hipGetSymbolAddress, taken once per device (with that device
// current) on its first no-allocation call and kept in g_scratch_ptr; only
// that address is handed to kernels.  No kernel needs any of it to start at
// zero: every entry a call reads is written earlier in the same call.
static __device__ __align__(256) unsigned char scratch[CSRSPMM_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return CSRSPMM_STATUS_NOT_SUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr || (reinterpret_cast<uintptr_t>(ptr) & 255)) return CSRSPMM_STATUS_NOT_SUPPORTED;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

int spmm_impl(int algo_in, int M, int K, int N, int nnz, const int* rowptr, const int* colidx,
              const float* vals, int hint, const float* B, long long ldb, float* C, long long ldc,
              float alpha, float beta, unsigned flags, void* ws, size_t ws_bytes, bool owned,
              void* stream) {
  const int algo = resolve_algorithm(algo_in, M, K, N, nnz, hint);
  Problem p;
  int st = fill_problem(p, algo, M, K, N, nnz, rowptr, colidx, vals, B, ldb, C, ldc, alpha, beta, flags);
  if (st != 0) return st;
  if (M == 0 || N == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // an owned workspace stays locked until the kernels are enqueued
  std::shared_ptr<OwnedWorkspace> held;
  std::unique_lock<std::mutex> lock;
  p.plan = wants_plan(algo, M, K, N, nnz, hint);
  if (p.plan) {
    const int vec = vector_width(algo, p);
    int P = per_call_panels(vec, true, K, N, nnz, hint);
    p.sw = slice_width(K, N, P > 0, wide_sweep(vec, true, M, K, nnz));
    p.slice_launch = slice_launches(M, nnz);
    if (p.sw == 0 && P == 0 && vec == 4 && xcd_slices(K, N) > 0) {
      p.sw = kSliceWidth;
      p.slice_launch = false;
      p.xslice = true;
    }
    if (p.sw > 0) P = 0;  // a sliced call gathers band by band instead
    WorkspaceLayout L = workspace_layout(M, K, N, nnz, P, share_applies(true, K, N, nnz, p.sw, P, hint));
    if (owned) {
      st = owned_workspace(stream, L.total, &ws, held, lock);
      if (st == CSRSPMM_STATUS_ALLOC_FAILED && L.total > L.base_total) {
        // no room for the panel or share tables: run without them
        L = workspace_layout(M, K, N, nnz, 0);
        st = owned_workspace(stream, L.total, &ws, held, lock);
      }
      if (st != 0) return st;
    } else {
      if (!ws || ws_bytes < L.base_total) return CSRSPMM_STATUS_WORKSPACE_TOO_SMALL;
      if (reinterpret_cast<uintptr_t>(ws) & 255) return CSRSPMM_STATUS_INVALID_VALUE;
      // a workspace sized without the panel or share tables runs without them
      if (ws_bytes < L.total) L = workspace_layout(M, K, N, nnz, 0);
    }
    // XCD slices keep the unsliced merge blocks (each launch holds every slice)
    bind_workspace(p, ws, L, call_merge_block(vec, M, nnz, p.sw > 0 && !p.xslice));
    set_row_hint(p, hint);
  }
  return to_status(launch_algorithm(algo, p, s));
}

// One wave per row: rowptr monotonicity and row length (lane 0), column
// range and in-row order (all lanes).  Reads are clamped to [0, nnz) so a
// malformed rowptr cannot send the validator out of bounds.
__global__ __launch_bounds__(256) void validate_kernel(int M, int K, int nnz, const int* rowptr,
                                                       const int* colidx, int* out) {
  __shared__ int s_flags;
  __shared__ int s_max;
  if (threadIdx.x == 0) {
    s_flags = 0;
    s_max = 0;
  }
  __syncthreads();
  const int lane = lane_id();
  const int nw = blockDim.x >> 6;
  int flags = 0;
  int mx = 0;
  for (int row = blockIdx.x * nw + (threadIdx.x >> 6); row < M; row += gridDim.x * nw) {
    const int rs = rowptr[row];
    const int re = rowptr[row + 1];
    if (lane == 0) {
      if (re < rs) flags |= CSRSPMM_CSR_NON_MONOTONE;
      mx = max(mx, re - rs);
      if (row == 0 && rs != 0) flags |= CSRSPMM_CSR_BAD_ROWPTR0;
      if (row == M - 1 && re != nnz) flags |= CSRSPMM_CSR_BAD_ROWPTR_END;
    }
    const int lo = max(rs, 0);
    const int hi = min(re, nnz);
    for (int j = lo + lane; j < hi; j += 64) {
      const int c = colidx[j];
      if (c < 0 || c >= K) flags |= CSRSPMM_CSR_COL_OUT_OF_RANGE;
      if (j + 1 < hi && colidx[j + 1] <= c) flags |= CSRSPMM_CSR_UNSORTED;
    }
  }
  if (flags) atomicOr(&s_flags, flags);
  if (mx) atomicMax(&s_max, mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (s_flags) atomicOr(&out[0], s_flags);
    atomicMax(&out[1], s_max);
  }
}

__global__ void zero2_kernel(int* out) {
  if (threadIdx.x < 2) out[threadIdx.x] = 0;
}

// Timing hook state: a pool of event pairs; pairs [0, g_t_used) hold
// recordings not yet read.
std::mutex g_t_mutex;                // the event pool
std::atomic<bool> g_t_on{false};     // read without the lock on every call
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_t_events;
size_t g_t_used = 0;

}  // namespace

thread_local int t_timing_depth = 0;
thread_local bool t_timing_recorded = false;  // the outermost call recorded a start event

void timing_before_main(hipStream_t s) {
  if (t_timing_depth++ > 0) return;
  t_timing_recorded = false;
  if (!g_t_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_t_mutex);
  if (g_t_used == g_t_events.size()) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess) return;
    if (hipEventCreate(&b) != hipSuccess) {
      (void)hipEventDestroy(a);
      return;
    }
    g_t_events.emplace_back(a, b);
  }
  t_timing_recorded = hipEventRecord(g_t_events[g_t_used].first, s) == hipSuccess;
}

void timing_after_main(hipStream_t s) {
  if (--t_timing_depth > 0 || !t_timing_recorded) return;
  t_timing_recorded = false;
  std::lock_guard<std::mutex> lock(g_t_mutex);
  if (g_t_used == g_t_events.size()) return;
  (void)hipEventRecord(g_t_events[g_t_used].second, s);
  ++g_t_used;
}

hipError_t launch_validate(int M, int K, int nnz, const int* rowptr, const int* colidx, int* d_out,
                           hipStream_t s) {
  hipLaunchKernelGGL(zero2_kernel, dim3(1), dim3(64), 0, s, d_out);
  if (M > 0) {
    const int blocks = std::min(div_up_host(M, 4), 65536);
    hipLaunchKernelGGL(validate_kernel, dim3(blocks), dim3(256), 0, s, M, K, nnz, rowptr, colidx, d_out);
  }
  return hipGetLastError();
}

}  // namespace csrspmm_hip

using namespace csrspmm_hip;

extern "C" {

int csrspmm_version(void) { return 100; }

const char* csrspmm_status_string(int status) {
  switch (status) {
    case CSRSPMM_STATUS_SUCCESS: return "success";
    case CSRSPMM_STATUS_INVALID_VALUE: return "invalid value";
    case CSRSPMM_STATUS_NOT_SUPPORTED: return "not supported";
    case CSRSPMM_STATUS_ALLOC_FAILED: return "workspace allocation failed";
    case CSRSPMM_STATUS_INVALID_CSR: return "invalid CSR matrix";
    case CSRSPMM_STATUS_WORKSPACE_TOO_SMALL: return "workspace too small";
    case CSRSPMM_STATUS_SCRATCH_TOO_SMALL:
      return "problem needs a larger workspace than the no-allocation scratch holds "
             "(CSRSPMM_NOALLOC_SCRATCH_BYTES, 128 MiB per GPU)";
    default:
      if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
      return "unknown status";
  }
}

static const char* const kAlgoNames[CSRSPMM_ALGO_COUNT + 1] = {
    "Naive", "NaiveSmem", "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4",
    "Auto"};

int csrspmm_parse_algorithm(const char* name) {
  if (!name) return -1;
  for (int i = 0; i <= CSRSPMM_ALGO_COUNT; ++i)
    if (strcmp(name, kAlgoNames[i]) == 0) return i;
  return -1;
}

const char* csrspmm_algorithm_name(int algo) {
  if (algo < 0 || algo > CSRSPMM_ALGO_COUNT) return nullptr;
  return kAlgoNames[algo];
}

int csrspmm_resolve_algorithm(int algo, int N) { return resolve_algorithm(algo, N); }
int csrspmm_resolve_algorithm_ex(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint) {
  return resolve_algorithm(algo, M, K, N, nnz, max_row_nnz_hint);
}

size_t csrspmm_workspace_bytes(int algo, int M, int N, int nnz) {
  algo = resolve_algorithm(algo, N);
  if (M <= 0 || N <= 0 || nnz < 0 || !wants_plan(algo, M, 0, N, nnz, -1)) return 0;
  return workspace_layout(M, 0, N, nnz, 0).base_total;
}

// The panels of a per-call product as far as the shape tells (pointer
// alignment is checked per call), as spmm_impl decides them; -1 when the
// call makes no plan.  *shares: the call splits its long rows by XCD.
static int shape_panels(int algo, int M, int K, int N, int nnz, int hint, bool* shares = nullptr) {
  if (shares) *shares = false;
  algo = resolve_algorithm(algo, M, K, N, nnz, hint);
  if (M <= 0 || N <= 0 || nnz < 0 || K < 0 || !wants_plan(algo, M, K, N, nnz, hint)) return -1;
  const bool fp4 = (algo == CSRSPMM_ALGO_WARP_PER_ROW_FP4 || algo == CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4) &&
                   N % 4 == 0;
  const int vec = fp4 ? 4 : 1;
  int P = per_call_panels(vec, true, K, N, nnz, hint);
  const int sw = slice_width(K, N, P > 0, wide_sweep(vec, true, M, K, nnz));
  if (sw > 0) P = 0;
  if (shares) *shares = share_applies(true, K, N, nnz, sw, P, hint);
  return P;
}

size_t csrspmm_workspace_bytes_ex(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint) {
  bool shares = false;
  const int P = shape_panels(algo, M, K, N, nnz, max_row_nnz_hint, &shares);
  return P < 0 ? 0 : workspace_layout(M, K, N, nnz, P, shares).total;
}

int csrspmm_call_shares(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint) {
  bool shares = false;
  const int P = shape_panels(algo, M, K, N, nnz, max_row_nnz_hint, &shares);
  return P >= 0 && shares ? 1 : 0;
}

int csrspmm_workspace_panel_info(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint,
                                 long long* nl_offset) {
  const int P = shape_panels(algo, M, K, N, nnz, max_row_nnz_hint);
  if (P <= 0) return 0;
  const WorkspaceLayout L = workspace_layout(M, K, N, nnz, P);
  if (nl_offset) *nl_offset = (long long)L.sched_off;  // sched[0] = nl
  return L.P;
}

int csrspmm_spmm_f32(int algo, int M, int K, int N, int nnz, const int* rowptr, const int* colidx,
                     const float* vals, int max_row_nnz_hint, const float* B, long long ldb, float* C,
                     long long ldc, float alpha, float beta, void* stream) {
  return spmm_impl(algo, M, K, N, nnz, rowptr, colidx, vals, max_row_nnz_hint, B, ldb, C, ldc, alpha,
                   beta, 0u, nullptr, 0, true, stream);
}

int csrspmm_spmm_f32_ex(int algo, int M, int K, int N, int nnz, const int* rowptr, const int* colidx,
                        const float* vals, int max_row_nnz_hint, const float* B, long long ldb,
                        float* C, long long ldc, float alpha, float beta, unsigned flags,
                        void* workspace, size_t workspace_bytes, void* stream) {
  return spmm_impl(algo, M, K, N, nnz, rowptr, colidx, vals, max_row_nnz_hint, B, ldb, C, ldc, alpha,
                   beta, flags, workspace, workspace_bytes, false, stream);
}

int csrspmm_spmm_f32_noalloc(int algo, int M, int K, int N, int nnz, const int* rowptr,
                             const int* colidx, const float* vals, int max_row_nnz_hint,
                             const float* B, long long ldb, float* C, long long ldc, float alpha,
                             float beta, unsigned flags, void* stream) {
  // The base workspace (block starts, segment slots, partials) of the call's
  // own plan must fit, none when it runs without one (a hint can make a
  // mid-sized call one launch); the per-call panel and share tables are
  // optional: spmm_impl runs without them when the scratch cannot hold them,
  // as for any workspace of base size.
  const int ralgo = resolve_algorithm(algo, M, K, N, nnz, max_row_nnz_hint);
  if (ralgo >= 0 && M > 0 && N > 0 && nnz >= 0 && K >= 0 &&
      wants_plan(ralgo, M, K, N, nnz, max_row_nnz_hint) &&
      workspace_layout(M, K, N, nnz, 0).base_total > CSRSPMM_NOALLOC_SCRATCH_BYTES)
    return CSRSPMM_STATUS_SCRATCH_TOO_SMALL;
  void* ws = nullptr;
  const int st = scratch_on_current_device(&ws);
  if (st != 0) return st;
  return spmm_impl(algo, M, K, N, nnz, rowptr, colidx, vals, max_row_nnz_hint, B, ldb, C, ldc, alpha,
                   beta, flags, ws, CSRSPMM_NOALLOC_SCRATCH_BYTES, false, stream);
}

int csrspmm_release_workspace(void* stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::shared_ptr<OwnedWorkspace> w;
  {
    std::lock_guard<std::mutex> g(g_ws_mutex);
    auto it = g_ws.find(ws_key(dev, stream));
    if (it == g_ws.end()) return 0;
    w = it->second;
    g_ws.erase(it);
  }
  std::lock_guard<std::mutex> l(w->m);  // after any call still enqueuing on it
  w->dead = true;
  e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  hipError_t e2 = w->ptr ? hipFree(w->ptr) : hipSuccess;
  w->ptr = nullptr;
  w->bytes = 0;
  if (e != hipSuccess) return (int)e;
  return to_status(e2);
}

int csrspmm_release_all_workspaces(void) {
  std::map<WsKey, std::shared_ptr<OwnedWorkspace>> all;
  {
    std::lock_guard<std::mutex> g(g_ws_mutex);
    all.swap(g_ws);
  }
  int st = 0;
  for (auto& kv : all) {
    std::lock_guard<std::mutex> l(kv.second->m);
    const int s1 = free_owned_device_synced(kv.first.dev, *kv.second);
    if (st == 0) st = s1;
  }
  return st;
}

int csrspmm_owned_workspaces(size_t* bytes_out) {
  std::lock_guard<std::mutex> g(g_ws_mutex);
  size_t total = 0;
  for (const auto& kv : g_ws) {
    std::lock_guard<std::mutex> l(kv.second->m);
    total += kv.second->bytes;
  }
  if (bytes_out) *bytes_out = total;
  return (int)g_ws.size();
}

int csrspmm_validate_csr(int M, int K, int nnz, const int* rowptr, const int* colidx, int* flags_out,
                         int* max_row_nnz_out, void* stream) {
  if (M < 0 || K < 0 || nnz < 0 || (!rowptr && M > 0) || (!colidx && nnz > 0))
    return CSRSPMM_STATUS_INVALID_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int* d_out = nullptr;
  hipError_t e = hipMalloc(&d_out, 2 * sizeof(int));
  if (e != hipSuccess) return (int)e;
  int h_out[2] = {0, 0};
  e = launch_validate(M, K, nnz, rowptr, colidx, d_out, s);
  if (e == hipSuccess) e = hipMemcpyAsync(h_out, d_out, sizeof(h_out), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  hipError_t e2 = hipFree(d_out);
  if (e != hipSuccess) return (int)e;
  if (e2 != hipSuccess) return (int)e2;
  if (M == 0 && nnz != 0) h_out[0] |= CSRSPMM_CSR_BAD_ROWPTR_END;
  if (flags_out) *flags_out = h_out[0];
  if (max_row_nnz_out) *max_row_nnz_out = h_out[1];
  return 0;
}

int csrspmm_device_malloc(void** ptr, size_t bytes) {
  if (!ptr) return CSRSPMM_STATUS_INVALID_VALUE;
  return to_status(hipMalloc(ptr, bytes));
}
int csrspmm_device_free(void* ptr) { return to_status(hipFree(ptr)); }
int csrspmm_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return to_status(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
}
int csrspmm_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return to_status(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
}
int csrspmm_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  return to_status(
      hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
}
int csrspmm_device_synchronize(void) { return to_status(hipDeviceSynchronize()); }
int csrspmm_stream_synchronize(void* stream) {
  return to_status(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
}
int csrspmm_get_last_error(void) { return to_status(hipGetLastError()); }
int csrspmm_timing_enable(int on) {
  g_t_on.store(on != 0, std::memory_order_relaxed);
  return 0;
}

int csrspmm_timing_read(double* main_kernel_ms, int* calls) {
  std::lock_guard<std::mutex> lock(g_t_mutex);
  double total = 0.0;
  for (size_t i = 0; i < g_t_used; ++i) {
    hipError_t e = hipEventSynchronize(g_t_events[i].second);
    if (e != hipSuccess) return (int)e;
    float ms = 0.0f;
    e = hipEventElapsedTime(&ms, g_t_events[i].first, g_t_events[i].second);
    if (e != hipSuccess) return (int)e;
    total += ms;
  }
  if (main_kernel_ms) *main_kernel_ms = total;
  if (calls) *calls = (int)g_t_used;
  g_t_used = 0;
  return 0;
}

int csrspmm_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

}  // extern "C"
