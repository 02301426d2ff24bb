// Stored SpMM plans (csrspmm_plan_* in include/csrspmm_c.h).
//
// A plan analyses A once: it picks the variant (CSRSPMM_ALGO_AUTO), builds
// the merge-block starts and long-row segment slots that plan_kernel would
// otherwise rebuild on every call, and "panelizes" very long rows on a large
// B.  That last step is what a per-call path cannot afford.
//
// Panelized rows.  A row of at least kPanelMinLen nonzeros with sorted
// columns is cut at column-panel boundaries (P panels of K/P columns, the
// B band of a panel is ~kPanelBandBytes) into pieces of at most kPieceMaxLen
// nonzeros.  Panels are dealt to the 8 XCDs in column order, each to the
// least-loaded XCD; the pieces of an XCD's panels, in panel order, form its
// list, and each list is cut into units of ~kPanelUnitItems
// (nonzeros + pieces), and the units are laid out in chunks of one
// workgroup's worth (GPB units) taking the XCD lists in turn.  Chunk c is
// workgroup c, which the hardware dispatches to XCD c mod 8, so every XCD
// works through its own panels in order and the B rows it gathers at any
// time fit in its L2.  The pieces are copied into a derived CSR (one row per
// piece, rows in unit order) and streamed by the ordinary short-row kernel
// into a partial buffer; the combine pass adds a row's pieces in column
// order.  Measured on the XL config, in isolation, this cut the long-row
// part from 562 us to 352 us.
//
// Device tables.  Where the per-call path itself cuts long rows into column
// panels for the plan's N (B >= 64 MiB, at least kDevPanelMinPanels panels;
// XL), the plan instead keeps that path's own tables: it runs plan_kernel and
// the panel schedule once into a workspace of its own, and each call
// launches only the main kernel, whose panel pieces interleave with the other
// roles, and the combine pass.  Measured on MI355X for XL (Auto, N = 128):
// 352 us per call through the derived CSR (its pieces launch ahead of the
// rest, which the device-side schedule's single grid overlaps), against the
// per-call path's 339 us; the tables are rebuilt when a call's N, column
// width or alignment no longer matches them.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "../../../include/csrspmm_c.h"
#include "common.hpp"
#include "spmm_internal.h"

#ifndef CSRSPMM_PANEL_UNIT_ITEMS
#define CSRSPMM_PANEL_UNIT_ITEMS 64
#endif

namespace csrspmm_hip {
namespace {

constexpr int kPanelUnitItems = CSRSPMM_PANEL_UNIT_ITEMS;

// Groups (rows) per workgroup of the kernel launch_rowgroup picks for N.
int groups_per_block(int vec, int N) {
  const int chunks = vec == 4 ? N / 4 : N;
  int g = 4;
  while (g < chunks && g < 64) g <<= 1;
  return 4 * (64 / g);
}

struct Dev {
  std::vector<void*> ptrs;
  size_t bytes = 0;
  template <class T>
  hipError_t alloc_copy(T** out, const std::vector<T>& host) {
    *out = nullptr;
    if (host.empty()) return hipSuccess;
    const size_t b = host.size() * sizeof(T);
    hipError_t e = hipMalloc(reinterpret_cast<void**>(out), b);
    if (e != hipSuccess) return e;
    ptrs.push_back(*out);
    bytes += b;
    return hipMemcpy(*out, host.data(), b, hipMemcpyHostToDevice);
  }
};

}  // namespace
}  // namespace csrspmm_hip

using namespace csrspmm_hip;

struct csrspmm_plan_s {
  int algo = 0;
  int M = 0, K = 0, nnz = 0;
  const int* rowptr = nullptr;
  const int* colidx = nullptr;
  const float* vals = nullptr;
  bool use_plan = false;
  int maxlen = 0;
  int nslots = 0, mblk = kMergeBlock, nblocks = 0;
  int* d_block_start = nullptr;
  int2* d_seg_info = nullptr;
  // panelized rows
  int npan = 0, npieces = 0, nunits = 0;
  int* d_pan_rows = nullptr;
  int* d_pan_ptr = nullptr;
  int* d_pan_piece = nullptr;
  int* d_drowptr = nullptr;
  int* d_dcolidx = nullptr;
  float* d_dvals = nullptr;
  int* d_unit_start = nullptr;
  // device tables (per-call path's tables, built once): the workspace and the
  // N, column width and layout they were built for
  bool dev_mode = false;
  void* d_ws = nullptr;
  size_t ws_bytes = 0;
  int tab_n = 0, tab_vec = 0, tab_P = -1;
  bool tab_sliced = false, tab_shares = false;
  WorkspaceLayout tab_L{};
  int dev_nl = 0;  // rows the device schedule panelized
  // partial buffers, grown with N
  long long ldp_cap = 0;
  float* d_partials = nullptr;
  float* d_pan_part = nullptr;
  Dev dev;
  size_t partial_bytes = 0;
};

namespace {

void plan_free(csrspmm_plan_s* p) {
  for (void* q : p->dev.ptrs) (void)hipFree(q);
  if (p->d_ws) (void)hipFree(p->d_ws);
  if (p->d_partials) (void)hipFree(p->d_partials);
  if (p->d_pan_part) (void)hipFree(p->d_pan_part);
  delete p;
}

hipError_t ensure_partials(csrspmm_plan_s* p, int N, hipStream_t s) {
  const long long ldp = ((long long)N + 3) & ~3LL;
  if (ldp <= p->ldp_cap) return hipSuccess;
  hipError_t e = hipStreamSynchronize(s);  // earlier calls may still read the old buffers
  if (e != hipSuccess) return e;
  if (p->d_partials) (void)hipFree(p->d_partials);
  if (p->d_pan_part) (void)hipFree(p->d_pan_part);
  p->d_partials = p->d_pan_part = nullptr;
  p->ldp_cap = 0;
  p->partial_bytes = 0;
  // partials only for rows of two segments or more
  const SegGeom g = seg_geom(p->nnz);
  const size_t nparts = p->maxlen < (2 << g.seg_shift) ? 0 : (size_t)(p->nnz >> g.seg_shift);
  if (nparts > 0) {
    e = hipMalloc(reinterpret_cast<void**>(&p->d_partials), nparts * ldp * sizeof(float));
    if (e != hipSuccess) return e;
  }
  if (p->npieces > 0) {
    e = hipMalloc(reinterpret_cast<void**>(&p->d_pan_part), (size_t)p->npieces * ldp * sizeof(float));
    if (e != hipSuccess) return e;
  }
  p->ldp_cap = ldp;
  p->partial_bytes = (nparts + (size_t)p->npieces) * ldp * sizeof(float);
  return hipSuccess;
}

int to_status(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

// Host analysis of a rowgroup-family plan (rowptr already on the host).
int build_rowgroup_plan(csrspmm_plan_s* p, const std::vector<int>& rp, int n_hint, int vec) {
  const int M = p->M, K = p->K, nnz = p->nnz;
  int maxlen = 0;
  for (int r = 0; r < M; ++r) maxlen = std::max(maxlen, rp[r + 1] - rp[r]);
  p->maxlen = maxlen;
  p->use_plan = ((long long)M + nnz >= kPlanMinItems) || maxlen > kSegLen;
  if (!p->use_plan) return 0;
  const SegGeom g = seg_geom(nnz);
  p->nslots = maxlen <= g.long_row ? 0 : nnz >> g.slot_shift;  // no long row: no segment table
  // Panelized rows: long, on a large B, with non-decreasing columns; for
  // scalar columns from N = kPanelMinScalarN (measured on XL through a stored
  // plan: WarpPerRowSmem 625 -> 412 us, WarpPerRow 636 -> 513).
  const int P = (vec == 4 || n_hint >= kPanelMinScalarN) ? panel_count(K, n_hint) : 0;
  std::vector<int> pan_rows;
  std::vector<int> hcol;
  std::vector<float> hval;
  if (P > 0 && maxlen >= kPanelMinLen) {
    hcol.resize((size_t)nnz);
    hval.resize((size_t)nnz);
    hipError_t e = hipMemcpy(hcol.data(), p->colidx, (size_t)nnz * sizeof(int), hipMemcpyDeviceToHost);
    if (e == hipSuccess)
      e = hipMemcpy(hval.data(), p->vals, (size_t)nnz * sizeof(float), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return (int)e;
    for (int r = 0; r < M; ++r) {
      if (rp[r + 1] - rp[r] < kPanelMinLen) continue;
      bool sorted = true;
      for (int j = rp[r] + 1; j < rp[r + 1] && sorted; ++j) sorted = hcol[j - 1] <= hcol[j];
      if (sorted) pan_rows.push_back(r);
    }
  }
  // Pieces: (row index i, panel, [a, b)) with b - a <= kPieceMaxLen.
  struct Piece {
    int i, a, b;
  };
  const long long width = P > 0 ? ((long long)K + P - 1) / P : 1;
  std::vector<std::vector<Piece>> by_panel((size_t)P);
  for (int i = 0; i < (int)pan_rows.size(); ++i) {
    const int r = pan_rows[(size_t)i];
    int a = rp[r];
    for (int pn = 0; pn < P; ++pn) {
      const long long hi_col = (pn + 1) * width;
      const int b = (int)(std::lower_bound(hcol.begin() + a, hcol.begin() + rp[r + 1], (int)std::min<long long>(hi_col, 0x7fffffff)) - hcol.begin());
      for (int x = a; x < b; x += kPieceMaxLen)
        by_panel[(size_t)pn].push_back({i, x, std::min(b, x + kPieceMaxLen)});
      a = b;
    }
  }
  // Skewed columns (a few hot panels, as in R-MAT graphs) already give L2
  // reuse without panels, and panels there only add partial traffic: keep
  // such rows on the ordinary segment path.
  std::vector<long long> weight((size_t)P, 0);
  long long total = 0;
  for (int pn = 0; pn < P; ++pn) {
    for (const Piece& pc : by_panel[(size_t)pn]) weight[(size_t)pn] += pc.b - pc.a + 1;
    total += weight[(size_t)pn];
  }
  if (total > 0 && *std::max_element(weight.begin(), weight.end()) * P > kPanelSkewMax * total)
    pan_rows.clear();  // back to segments, before the merge blocks are sized
  std::vector<char> panelized((size_t)M, 0);
  for (int r : pan_rows) panelized[r] = 1;

  // Merge blocks as a per-call call of the hinted width takes them (sized to
  // the rows below 65536 of them); calls of another width run on them too.
  const int nh = n_hint > 0 ? n_hint : 128;
  const bool sliced = pan_rows.empty() && slice_width(K, nh, false, wide_sweep(vec, true, M, K, nnz)) > 0;
  p->mblk = call_merge_block(vec, M, nnz, sliced);
  p->nblocks = merge_blocks(M, nnz, p->mblk);

  // Merge-block starts and segment slots: the formulas of plan_kernel, with
  // panelized rows leaving their slots unused.
  std::vector<int> block_start((size_t)p->nblocks + 1);
  std::vector<int2> seg_info((size_t)p->nslots, make_int2(-1, 0));
  long long fprev = -1;
  for (int r = 0; r <= M; ++r) {
    const long long f = (long long)r + rp[r];
    const long long b_lo = fprev < 0 ? 0 : fprev / p->mblk + 1;
    const long long b_hi = std::min(f / p->mblk, (long long)p->nblocks - 1);
    for (long long b = b_lo; b <= b_hi; ++b) block_start[(size_t)b] = r;
    fprev = f;
    if (r == M) break;
    const int len = rp[r + 1] - rp[r];
    if (!panelized[r]) {
      const int s0 = rp[r] >> g.slot_shift;
      for (int k = 0; k < seg_count(len, g.long_row, g.seg_shift); ++k)
        seg_info[(size_t)s0 + k] = make_int2(r, k);
    }
  }
  block_start[(size_t)p->nblocks] = M;
  hipError_t e = p->dev.alloc_copy(&p->d_block_start, block_start);
  if (e == hipSuccess) e = p->dev.alloc_copy(&p->d_seg_info, seg_info);
  if (e != hipSuccess) return (int)e;
  if (pan_rows.empty()) return 0;

  // Panels go to XCDs in column order, each to the XCD with the least work so
  // far; each XCD list keeps its panels in column order and is cut into units
  // of ~kPanelUnitItems.
  std::vector<std::vector<int>> panels_of(kXcds);
  {
    std::vector<long long> load(kXcds, 0);
    for (int pn = 0; pn < P; ++pn) {
      const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
      load[(size_t)x] += weight[(size_t)pn];
      panels_of[(size_t)x].push_back(pn);
    }
  }
  std::vector<std::vector<std::vector<Piece>>> units_of(kXcds);
  for (int x = 0; x < kXcds; ++x) {
    std::vector<Piece> cur;
    int items = 0;
    for (int pn : panels_of[(size_t)x]) {
      for (const Piece& pc : by_panel[(size_t)pn]) {
        cur.push_back(pc);
        items += pc.b - pc.a + 1;
        if (items >= kPanelUnitItems) {
          units_of[x].push_back(cur);
          cur.clear();
          items = 0;
        }
      }
    }
    if (!cur.empty()) units_of[x].push_back(cur);
  }
  // Chunks of GPB units, XCD lists in turn; an exhausted list pads with
  // empty units so every chunk keeps its XCD.
  const int gpb = groups_per_block(vec, n_hint);
  std::vector<int> drowptr(1, 0), dcol, unit_start(1, 0);
  std::vector<float> dval;
  std::vector<std::vector<std::pair<int, int>>> row_pieces(pan_rows.size());  // (CSR position, derived row)
  std::vector<size_t> next(kXcds, 0);
  bool more = true;
  while (more) {
    more = false;
    for (int x = 0; x < kXcds; ++x) {
      for (int u = 0; u < gpb; ++u) {
        if (next[x] < units_of[x].size()) {
          for (const Piece& pc : units_of[x][next[x]]) {
            row_pieces[(size_t)pc.i].emplace_back(pc.a, (int)drowptr.size() - 1);
            dcol.insert(dcol.end(), hcol.begin() + pc.a, hcol.begin() + pc.b);
            dval.insert(dval.end(), hval.begin() + pc.a, hval.begin() + pc.b);
            drowptr.push_back((int)dcol.size());
          }
          ++next[x];
        }
        unit_start.push_back((int)drowptr.size() - 1);
      }
    }
    for (int x = 0; x < kXcds; ++x) more = more || next[x] < units_of[x].size();
  }
  // A row's pieces were appended XCD list by XCD list; the combine adds them
  // in CSR order (sorted by their position in the original row).
  std::vector<int> pan_ptr(1, 0), pan_piece;
  for (auto& v : row_pieces) {
    std::sort(v.begin(), v.end());
    for (const auto& pr : v) pan_piece.push_back(pr.second);
    pan_ptr.push_back((int)pan_piece.size());
  }
  p->npan = (int)pan_rows.size();
  p->npieces = (int)drowptr.size() - 1;
  p->nunits = (int)unit_start.size() - 1;
  e = p->dev.alloc_copy(&p->d_pan_rows, pan_rows);
  if (e == hipSuccess) e = p->dev.alloc_copy(&p->d_pan_ptr, pan_ptr);
  if (e == hipSuccess) e = p->dev.alloc_copy(&p->d_pan_piece, pan_piece);
  if (e == hipSuccess) e = p->dev.alloc_copy(&p->d_drowptr, drowptr);
  if (e == hipSuccess) e = p->dev.alloc_copy(&p->d_dcolidx, dcol);
  if (e == hipSuccess) e = p->dev.alloc_copy(&p->d_dvals, dval);
  if (e == hipSuccess) e = p->dev.alloc_copy(&p->d_unit_start, unit_start);
  return to_status(e);
}

// Column panels the per-call path uses for N with this column width (0: none,
// also when column slices take over).
int device_panels(const csrspmm_plan_s* p, int vec, int N) {
  const int P = per_call_panels(vec, true, p->K, N, p->nnz, p->maxlen);
  return slice_width(p->K, N, P > 0) > 0 ? 0 : P;
}

// Column slices of a call of N with P panels (npan panelized rows): the
// per-call rules, column slices or else XCD slices.
void call_slicing(const csrspmm_plan_s* p, int vec, int N, int P, int& sw, bool& xslice) {
  sw = P > 0 ? 0 : slice_width(p->K, N, false, wide_sweep(vec, true, p->M, p->K, p->nnz));
  xslice = sw == 0 && P == 0 && vec == 4 && xcd_slices(p->K, N) > 0;
  if (xslice) sw = kSliceWidth;
}

// XCD shares of a call of N without panels: the per-call rule, with the
// plan's true longest row as the hint.
bool device_shares(const csrspmm_plan_s* p, int vec, int N) {
  if (device_panels(p, vec, N) > 0) return false;
  int sw;
  bool xslice;
  call_slicing(p, vec, N, 0, sw, xslice);
  return share_applies(true, p->K, N, p->nnz, sw, 0, p->maxlen);
}

// A Problem carrying the plan's CSR and tables (B and C are the call's); the
// merge blocks are the per-call path's for the tables' slicing.
void bind_tables(const csrspmm_plan_s* p, Problem& q, int vec) {
  q.plan = true;
  bind_workspace(q, p->d_ws, p->tab_L, call_merge_block(vec, p->M, p->nnz, p->tab_sliced));
  set_row_hint(q, p->maxlen);
}

// Builds (or rebuilds) the per-call tables for N and column width vec into the
// plan's workspace: plan_kernel and the panel schedule, on stream s.
hipError_t build_device_tables(csrspmm_plan_s* p, int N, int vec, hipStream_t s) {
  const int P = device_panels(p, vec, N);
  const bool shares = P == 0 && device_shares(p, vec, N);
  const WorkspaceLayout L = workspace_layout(p->M, p->K, N, p->nnz, P, shares);
  hipError_t e = hipSuccess;
  if (L.total > p->ws_bytes) {
    e = hipStreamSynchronize(s);  // earlier calls may still use the old tables
    if (e != hipSuccess) return e;
    if (p->d_ws) (void)hipFree(p->d_ws);
    p->d_ws = nullptr;
    p->ws_bytes = 0;
    e = hipMalloc(&p->d_ws, L.total);
    if (e != hipSuccess) {
      p->d_ws = nullptr;
      return e;
    }
    p->ws_bytes = L.total;
  }
  p->tab_L = L;
  p->tab_n = N;
  p->tab_vec = vec;
  p->tab_P = P;
  int sw;
  bool xslice;
  call_slicing(p, vec, N, P, sw, xslice);
  p->tab_sliced = sw > 0 && !xslice;  // XCD slices keep the unsliced merge blocks
  p->tab_shares = shares;
  Problem q{};
  q.M = p->M;
  q.K = p->K;
  q.N = N;
  q.nnz = p->nnz;
  q.rowptr = p->rowptr;
  q.colidx = p->colidx;
  q.vals = p->vals;
  const SegGeom g = seg_geom(p->nnz);
  q.seg_shift = g.seg_shift;
  q.slot_shift = g.slot_shift;
  q.long_row = g.long_row;
  bind_tables(p, q, vec);
  e = launch_plan_tables(q, s);
  if (e != hipSuccess) return e;
  p->dev_nl = 0;
  if (P > 0) {  // rows panelized (sched[0]), for csrspmm_plan_panelized_rows
    e = hipMemcpyAsync(&p->dev_nl, q.dp.sched, sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
  }
  return e;
}

}  // namespace

extern "C" {

int csrspmm_plan_create(int algo, int M, int K, int nnz, const int* rowptr, const int* colidx,
                        const float* vals, int n_hint, void* stream, csrspmm_plan_t* out) {
  if (!out) return CSRSPMM_STATUS_INVALID_VALUE;
  *out = nullptr;
  if (M < 0 || K < 0 || nnz < 0 || !rowptr || (nnz > 0 && (!colidx || !vals || K == 0)))
    return CSRSPMM_STATUS_INVALID_VALUE;
  if ((long long)M + nnz + 1 > 0x7fffffffLL - kMergeBlockMax) return CSRSPMM_STATUS_NOT_SUPPORTED;
  const int n_eff = n_hint > 0 ? n_hint : 128;
  if (resolve_algorithm(algo, n_eff) < 0) return CSRSPMM_STATUS_INVALID_VALUE;
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));  // A must be ready
  if (e != hipSuccess) return (int)e;
  std::vector<int> rp((size_t)M + 1);
  e = hipMemcpy(rp.data(), rowptr, rp.size() * sizeof(int), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return (int)e;
  if (rp[0] != 0 || rp[(size_t)M] != nnz) return CSRSPMM_STATUS_INVALID_CSR;
  int maxlen = 0;
  for (int r = 0; r < M; ++r) {
    if (rp[(size_t)r + 1] < rp[(size_t)r]) return CSRSPMM_STATUS_INVALID_CSR;
    maxlen = std::max(maxlen, rp[(size_t)r + 1] - rp[(size_t)r]);
  }
  // Auto from the shape and the true longest row
  const int concrete = resolve_algorithm(algo, M, K, n_eff, nnz, maxlen);
  auto* p = new csrspmm_plan_s();
  p->algo = concrete;
  p->M = M;
  p->K = K;
  p->nnz = nnz;
  p->rowptr = rowptr;
  p->colidx = colidx;
  p->vals = vals;
  if (is_rowgroup_algorithm(concrete)) {
    const int vec = (concrete == CSRSPMM_ALGO_WARP_PER_ROW_FP4 ||
                     concrete == CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4) && n_eff % 4 == 0 ? 4 : 1;
    p->maxlen = maxlen;
    p->use_plan = ((long long)M + nnz >= kPlanMinItems) || maxlen > kSegLen;
    // per-call tables built once: with column panels, or with XCD shares
    // (the host-built tables have neither share entries nor boundaries)
    p->dev_mode = p->use_plan && (device_panels(p, vec, n_eff) > 0 || device_shares(p, vec, n_eff));
    if (p->dev_mode) {
      e = build_device_tables(p, n_eff, vec, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) {
        plan_free(p);
        return e == hipErrorOutOfMemory ? CSRSPMM_STATUS_ALLOC_FAILED : (int)e;
      }
      *out = p;
      return 0;
    }
    const int st = build_rowgroup_plan(p, rp, n_eff, vec);
    if (st != 0) {
      plan_free(p);
      return st;
    }
    if (p->use_plan) {
      e = ensure_partials(p, n_eff, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) {
        plan_free(p);
        return CSRSPMM_STATUS_ALLOC_FAILED;
      }
    }
  }
  *out = p;
  return 0;
}

int csrspmm_plan_spmm_f32(csrspmm_plan_t plan, int N, const float* B, long long ldb, float* C,
                          long long ldc, float alpha, float beta, unsigned flags, void* stream) {
  if (!plan) return CSRSPMM_STATUS_INVALID_VALUE;
  csrspmm_plan_s* p = plan;
  if (!p->use_plan) {
    // naive family or a small problem: the per-call path (allocates nothing)
    return csrspmm_spmm_f32_ex(p->algo, p->M, p->K, N, p->nnz, p->rowptr, p->colidx, p->vals,
                               p->maxlen, B, ldb, C, ldc, alpha, beta, flags, nullptr, 0, stream);
  }
  Problem pr{};
  int st = fill_problem(pr, p->algo, p->M, p->K, N, p->nnz, p->rowptr, p->colidx, p->vals, B, ldb, C,
                        ldc, alpha, beta, flags);
  if (st != 0 || p->M == 0 || N == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (p->dev_mode) {
    // the per-call path with its tables built once: rebuilt when this call's
    // panels, column width or partial width differ from theirs
    const int vec = vector_width(p->algo, pr);
    const int P = device_panels(p, vec, N);
    int sw;
    bool xslice;
    call_slicing(p, vec, N, P, sw, xslice);
    const bool shares = P == 0 && device_shares(p, vec, N);
    const long long ldp = ((long long)N + 3) & ~3LL;
    if (P != p->tab_P || vec != p->tab_vec || (sw > 0 && !xslice) != p->tab_sliced ||
        shares != p->tab_shares || ldp > p->tab_L.ldp) {
      const hipError_t eb = build_device_tables(p, N, vec, s);
      if (eb != hipSuccess) return eb == hipErrorOutOfMemory ? CSRSPMM_STATUS_ALLOC_FAILED : (int)eb;
    }
    bind_tables(p, pr, vec);
    pr.plan_ready = true;
    pr.dp_ready = true;
    pr.sw = sw;
    pr.slice_launch = !xslice && slice_launches(p->M, p->nnz);
    pr.xslice = xslice;
    return to_status(launch_algorithm(p->algo, pr, s));
  }
  hipError_t e = ensure_partials(p, N, s);
  if (e != hipSuccess) return CSRSPMM_STATUS_ALLOC_FAILED;
  pr.plan = true;
  pr.plan_ready = true;
  pr.nslots = p->nslots;
  set_row_hint(pr, p->maxlen);
  pr.mblk = p->mblk;
  pr.nblocks = p->nblocks;
  pr.block_start = p->d_block_start;
  pr.seg_info = p->d_seg_info;
  pr.partials = p->d_partials;
  pr.ldp = p->ldp_cap;
  pr.npan = p->npan;
  const int vec = vector_width(p->algo, pr);
  const bool lds = uses_lds(p->algo);
  // a plan with panelized rows keeps them; otherwise large B are sliced by
  // columns (or by XCD)
  bool xslice;
  call_slicing(p, vec, N, p->npan, pr.sw, xslice);
  pr.slice_launch = !xslice && slice_launches(p->M, p->nnz);
  pr.xslice = xslice;
  pr.pan_rows = p->d_pan_rows;
  pr.pan_ptr = p->d_pan_ptr;
  pr.pan_piece = p->d_pan_piece;
  pr.pan_part = p->d_pan_part;
  timing_before_main(s);
  if (p->npan > 0) {
    // the pieces of panelized rows, alone first so nothing else evicts their band
    Problem d = pr;
    d.sw = 0;
    d.M = p->npieces;
    d.rowptr = p->d_drowptr;
    d.colidx = p->d_dcolidx;
    d.vals = p->d_dvals;
    d.C = p->d_pan_part;
    d.ldc = p->ldp_cap;
    d.alpha = 1.0f;
    d.beta = 0.0f;
    d.epi = kEpiOverwrite;
    d.nblocks = p->nunits;
    d.block_start = p->d_unit_start;
    d.nslots = 0;
    d.npan = 0;
    d.rows_whole = true;  // pieces (at most kPieceMaxLen nonzeros) are summed whole
    d.no_split = true;
    e = launch_rowgroup(d, vec, lds, s);
  }
  if (e == hipSuccess) e = launch_rowgroup(pr, vec, lds, s);
  timing_after_main(s);
  return to_status(e);
}

int csrspmm_plan_algorithm(csrspmm_plan_t plan) { return plan ? plan->algo : -1; }

size_t csrspmm_plan_device_bytes(csrspmm_plan_t plan) {
  return plan ? plan->dev.bytes + plan->partial_bytes + plan->ws_bytes : 0;
}

int csrspmm_plan_shares(csrspmm_plan_t plan, int N) {
  if (!plan || N <= 0) return CSRSPMM_STATUS_INVALID_VALUE;
  const csrspmm_plan_s* p = plan;
  if (!p->dev_mode || !is_rowgroup_algorithm(p->algo)) return 0;
  const int vec = (p->algo == CSRSPMM_ALGO_WARP_PER_ROW_FP4 ||
                   p->algo == CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4) && N % 4 == 0 ? 4 : 1;
  return device_shares(p, vec, N) ? 1 : 0;
}

int csrspmm_plan_panelized_rows(csrspmm_plan_t plan) {
  if (!plan) return -1;
  return plan->dev_mode ? plan->dev_nl : plan->npan;
}

int csrspmm_plan_destroy(csrspmm_plan_t plan) {
  if (!plan) return 0;
  hipError_t e = hipDeviceSynchronize();  // no call may still use its buffers
  plan_free(plan);
  return to_status(e);
}

}  // extern "C"
