// Internal (HIP-side) interface between the C-ABI layer (capi.hip) and the
// kernel translation units.  Not installed; callers use include/csrspmm_c.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace csrspmm_hip {

// Epilogue modes.  The reference computes C = alpha*sum + (beta != 0 ? beta*C : 0)
// (src/device/csrspmm_naive.cu:38, csrspmm_warp_per_row.cu:45-46,
// csrspmm_warp_per_row_fp4.cu:48-63): C is read only when beta != 0.
enum EpilogueMode : int {
  kEpiOverwrite = 0,   // beta == 0: C = alpha*sum, prior C never read
  kEpiAccumulate = 1,  // C = fma(alpha, sum, beta*C)
  kEpiZeroC = 2,       // C = fma(alpha, sum, beta*0.0f): prior C taken as +0 without reading
                       // it (the torch forwards' zeros()+beta, torch_csrspmm_naive.cpp:32-34)
};

// Long rows.  A row of len > long_row nonzeros leaves the merge blocks of
// short rows and is cut into nseg = max(1, floor(len / seg)) segments of
// near-equal length: segment k covers nonzeros
// [seg_begin(len, nseg, k), seg_begin(len, nseg, k + 1)) of the row, so a
// row's segments differ in length by at most one (up to 2*seg-1 nonzeros for
// a single segment, at most (3/2)*seg from two on).  A row with one segment is
// summed whole and stored with the epilogue directly; otherwise segment k's
// partial sum goes to workspace partial rowptr[r] / seg + k, and a combine
// pass adds the partials of the row in segment order and applies the
// epilogue.  The segments run in the first blocks of the main launch, so
// rows above long_row, each one group's chain of dependent gathers, start
// early rather than trailing the short rows (measured on MI355X: long_row
// 128 instead of 256, 2.5% faster on XL).
//
// No counters are needed: row r owns the table slots
// [rowptr[r] / slot, rowptr[r+1] / slot), at least one for
// len > long_row >= slot and at least nseg since seg >= slot, and the
// partials [rowptr[r] / seg, rowptr[r+1] / seg), at least nseg when
// nseg >= 2; the ranges of all rows tile [0, nnz / slot) and [0, nnz / seg).
//
// The geometry (seg, slot, long_row) is (kSegLen, kSlotLen, kLongRow), or,
// for a matrix with fewer than kMinSegments * kSegLen nonzeros, seg halved
// down to kSegLenMin until there are kMinSegments segments' worth of
// nonzeros, with slot and long_row at most seg: a small matrix's long rows
// still split into enough chains to fill the GPU.
#ifndef CSRSPMM_SEG_LEN
#define CSRSPMM_SEG_LEN 256
#endif
#ifndef CSRSPMM_LONG_ROW
#define CSRSPMM_LONG_ROW 128
#endif
#ifndef CSRSPMM_SLOT_LEN
#define CSRSPMM_SLOT_LEN 128
#endif
constexpr int kSegLen = CSRSPMM_SEG_LEN;
constexpr int kLongRow = CSRSPMM_LONG_ROW;
constexpr int kSlotLen = CSRSPMM_SLOT_LEN;
constexpr int kSegLenMin = 32;
constexpr long long kMinSegments = 4096;
static_assert(kLongRow >= kSlotLen, "a long row owns at least one table slot");
static_assert(kSegLen >= kSlotLen, "a row owns a table slot for each of its segments");
static_assert((kSegLen & (kSegLen - 1)) == 0 && (kSlotLen & (kSlotLen - 1)) == 0 &&
                  kSegLenMin <= kSlotLen && kSegLenMin <= kLongRow,
              "segment geometry: powers of two, shortened down to kSegLenMin");

struct SegGeom {
  int seg_shift;   // seg = 1 << seg_shift
  int slot_shift;  // slot = 1 << slot_shift
  int long_row;
};

inline SegGeom seg_geom(int nnz) {
  int seg = kSegLen;
  while (seg > kSegLenMin && (long long)nnz / seg < kMinSegments) seg >>= 1;
  const int slot = seg < kSlotLen ? seg : kSlotLen;
  SegGeom g;
  g.seg_shift = __builtin_ctz((unsigned)seg);
  g.slot_shift = __builtin_ctz((unsigned)slot);
  g.long_row = seg < kLongRow ? seg : kLongRow;
  return g;
}

// Segments of a row of len nonzeros (0: a short row).
__host__ __device__ inline int seg_count(int len, int long_row, int seg_shift) {
  if (len <= long_row) return 0;
  const int n = len >> seg_shift;
  return n < 2 ? 1 : n;
}

__host__ __device__ inline int seg_begin(int len, int nseg, int k) {
  return static_cast<int>((static_cast<long long>(k) * len) / nseg);
}

// Pieces of a stored plan's panelized rows hold at most this many nonzeros:
// they are streamed as the short rows of a derived CSR, which has no segment
// table, so none may be a long row.
constexpr int kPieceMaxLen = kLongRow;
static_assert(kPieceMaxLen <= kLongRow, "pieces are streamed as short rows");

// Short rows (len <= kLongRow) are streamed in merge-path blocks: with the
// strictly increasing merge coordinate F(r) = r + rowptr[r], block b holds
// the rows r with F(r) in [b*kMergeBlock, (b+1)*kMergeBlock), so every block
// carries at most kMergeBlock (rows + nonzeros) of short-row work plus one
// row's tail, and runs of empty rows are spread like nonzeros.
// The block is smaller for float4 columns (measured on MI355X: 64 for
// float4, whose groups are narrower and more per wave; 128 for scalar ones).
#ifndef CSRSPMM_MERGE_BLOCK
#define CSRSPMM_MERGE_BLOCK 128
#endif
#ifndef CSRSPMM_MERGE_BLOCK_VEC4
#define CSRSPMM_MERGE_BLOCK_VEC4 64
#endif
constexpr int kMergeBlock = CSRSPMM_MERGE_BLOCK;
constexpr int kMergeBlockVec4 = CSRSPMM_MERGE_BLOCK_VEC4;
constexpr int kMergeBlockMax = kMergeBlock > kMergeBlockVec4 ? kMergeBlock : kMergeBlockVec4;
static_assert((kMergeBlock & (kMergeBlock - 1)) == 0 && (kMergeBlockVec4 & (kMergeBlockVec4 - 1)) == 0,
              "merge blocks are powers of two (plan_kernel shifts by them)");
// A small problem gets smaller merge blocks, down to one item, so that it
// still has at least kMinMergeBlocks of them to spread over the GPU's
// 256 CUs (measured on MI355X: 512 rows x N = 1024 with the full block ran
// as 7 groups, 187 us a call).
constexpr long long kMinMergeBlocks = 4096;
inline int merge_block(int vec, int M, int nnz) {
  int m = vec == 4 ? kMergeBlockVec4 : kMergeBlock;
  while (m > 1 && ((long long)M + nnz + 1) / m < kMinMergeBlocks) m >>= 1;
  return m;
}
inline int merge_blocks(int M, int nnz, int mblk) {
  return (int)(((long long)M + nnz + 1 + mblk - 1) / mblk);
}
// A per-call float4 call with column slices and fewer than
// kSlicedMergeRowsMax rows sizes its merge blocks to the rows instead: the
// largest power of two from 16 to 64 not above the mean row's items (1 + its
// nonzeros).  Such a slice launch holds a round or two of 16-lane groups,
// each on one block of whole rows, so the last round's few blocks set its
// length; smaller blocks spread that tail over more, shorter rounds, and
// rows longer than the block leave its groups idle.  Measured on MI355X per
// call (N = 256, uniform rows, bit-identical), 64 -> this rule: 32768^2 with
// 8 per row 50.8 -> 39.7 us, 16: 71.9 -> 58.4, 24: 97.9 -> 84.4, 40: 118.1
// -> 113.8, 48: 187.3 -> 150.1; 16384 x 32768 with 16 per row 47.4 -> 35.9,
// 32: 75.2 -> 56.0, 40: 87.7 -> 66.3; 8192 x 65536 x 1024 with 50 per row
// 395 -> 257.  From 65536 rows the launches hold enough blocks that their
// size hardly matters (65536 x 32768 and 131072^2 within 1%), and R-MAT's
// 2^20 rows lost 7-14% with the small blocks.  A stored plan takes the
// blocks of its hinted width.
constexpr int kSlicedMergeBlockMin = 16;
constexpr int kSlicedMergeRowsMax = 65536;
inline int sliced_merge_block(int M, int nnz) {
  if (M >= kSlicedMergeRowsMax) return merge_block(4, M, nnz);
  const long long items = M > 0 ? ((long long)M + nnz) / M : 1;
  int m = kSlicedMergeBlockMin;
  while (m * 2 <= kMergeBlockVec4 && m * 2 <= items) m *= 2;
  while (m > 1 && ((long long)M + nnz + 1) / m < kMinMergeBlocks) m >>= 1;
  return m;
}
// Unsliced per-call float4 calls take the same row-sized blocks when they
// still number at least kRowSizedMinBlocks.  Measured on MI355X per call,
// bit-identical: 32768^2 x 128 with 20 per row 48.5 -> 44.7 us, 49152 x
// 16384 x 128 with 12 per row 36.5 -> 34.4, 32768 x 16384 x 128 with 24 per
// row 41.1 -> 40.1, 32768 x 8192 x 256 with 40 per row 101.3 -> 99.4,
// 16384^2 x 64 with 16 per row 16.3 -> 15.2; with fewer blocks, 16384^2 x 128
// with 8 per row lost 15.5 -> 17.8 us (16-item blocks against 32).
constexpr int kRowSizedMinBlocks = 16384;
inline int call_merge_block(int vec, int M, int nnz, bool sliced) {
  if (vec != 4) return merge_block(vec, M, nnz);
  const int m = sliced_merge_block(M, nnz);
  if (sliced || merge_blocks(M, nnz, m) >= kRowSizedMinBlocks) return m;
  return merge_block(4, M, nnz);
}

// Below this many (rows + nonzeros) the plan is skipped and each row is
// processed whole by one group (one launch instead of three).
constexpr long long kPlanMinItems = 1 << 16;
// With a max_row_nnz hint of at most kPlanSkipMaxRow, a problem of fewer
// than kPlanSkipItems (rows + nonzeros) and kPlanSkipRows rows, without
// column slices, runs as one launch too (plan_skips): one group per row,
// every row summed whole.  The plan's and the combine's launches cost more
// than the merge blocks and the split rows save.  Measured on MI355X per
// call (Auto, the hint = the longest row): 4096^2 x 128 with 41 per row
// 14.4 -> 9.8 us, 8192 x 4096 x 256 with 41 per row 22.0 -> 17.4 us,
// 16384^2 x 128 with 20 per row 19.4 -> 16.6 us, 16384^2 x 256 with 60 per
// row 105 -> 95 us, 8192 x 131072 x 128 with 100 per row 58.4 -> 46.8 us;
// rows of 129-256 (which the plan cuts into segments of 32 on a small
// matrix): 1024 x 2048 x 128 with 200 per row 19.2 -> 13.0 us, 4096^2 x 128
// with 200 per row 24.6 -> 18.8 us, 2048 x 131072 x 128 with 250 per row
// 44.6 -> 34.4 us, 3072 x 262144 x 256 with 200 per row 87.9 -> 79.7 us.
// From 32768 rows the band sweep, which needs the plan, leads (32768^2 x
// 128 with 20 per row 31.3 us planned against 39.5 us, 65536^2 x 128 with
// 12 per row 49.1 against 56.5 us), and sliced calls keep it too (16384^2 x
// 512 with 50 per row 192 against 201 us).
constexpr long long kPlanSkipItems = 1 << 20;
constexpr int kPlanSkipRows = 32768;
constexpr int kPlanSkipMaxRow = 256;

// XCDs of an MI355X.  Workgroups are dispatched to them round-robin by
// workgroup id, which stored plans use for L2 locality (plan.hip).
constexpr int kXcds = 8;

// Column panels.  A row of at least kPanelMinLen nonzeros with sorted
// columns, on a B of at least 16 MiB (per call: at least kDevPanelMinPanels
// panels) with N <= 256 (float4 columns, or scalar ones from N = 128), is cut
// at the boundaries of P column panels (P a power of two, kXcds..256, so that
// a panel's band of B is about kPanelBandBytes).  Each XCD walks its own
// panels in column order, so the band it gathers from stays in its L2.  Stored
// plans build the schedule on the host (plan.hip); the per-call path builds
// it on the device (panels.hip).  The band is 2 MiB (measured on MI355X
// against 1 and 4 MiB: XL 3% and the mean-98 power-law config 15% faster
// per call than at 1 MiB, whose partials (P x N floats per row) cost more
// traffic and, under the partial budget, left long rows unpanelized).
#ifndef CSRSPMM_PANEL_MIN_LEN
#define CSRSPMM_PANEL_MIN_LEN 1024
#endif
#ifndef CSRSPMM_PANEL_BAND_KB
#define CSRSPMM_PANEL_BAND_KB 2048
#endif
constexpr int kPanelMinLen = CSRSPMM_PANEL_MIN_LEN;
constexpr long long kPanelBandBytes = (long long)CSRSPMM_PANEL_BAND_KB * 1024;
constexpr int kPanelMaxPanels = 256;
// Scalar-column (VEC = 1) calls use panels from N = 128 up.  Measured on
// MI355X, WarpPerRowSmem on XL: N = 128 648 -> 451 us, N = 256 1252 -> 831;
// at N = 64 the pieces lost (331 -> 350 us), and the float4 form leads there.
constexpr int kPanelMinScalarN = 128;
constexpr int kPanelSkewMax = 4;  // panels stay off when max panel load > 4 x mean
static_assert(kPanelMinLen > kLongRow, "panelized rows are long rows");

// Panels for a K x N fp32 B: a power of two (>= kXcds) giving a band of about
// kPanelBandBytes; 0 (off) when B is small enough for the L2s or N is wide.
inline int panel_count(int K, int N) {
  const long long bbytes = (long long)K * N * 4;
  if (kPanelBandBytes <= 0 || N > 256 || bbytes < 16LL * 1024 * 1024) return 0;
  long long p = kXcds;
  while (p * 2 <= kPanelMaxPanels && p * 2 * kPanelBandBytes <= bbytes) p *= 2;
  return (int)p;
}

// The per-call path takes panels only when B is wide enough for 32 of them
// (B >= 64 MiB).  Its pieces are whole (row, panel) ranges: with 8 or 16
// panels a 16k-nonzero row's pieces are dependent chains of 1-2k nonzeros.
// Measured on MI355X per call: with 16 panels, power-law rows at K = 65536,
// N = 128 took 242 us with panels against 194 without, and 278 against 191 at
// K = 131072, N = 64; with 32 (XL at N = 64, K = 131072 at N = 128) panels
// won 286 against 350 and 254 against 323.  Stored plans cut pieces at
// kPieceMaxLen and keep panels from 8 (a 16-panel plan ran 146 us there,
// 192 without).
#ifndef CSRSPMM_DEV_PANEL_MIN_PANELS
#define CSRSPMM_DEV_PANEL_MIN_PANELS 32
#endif
constexpr int kDevPanelMinPanels = CSRSPMM_DEV_PANEL_MIN_PANELS;

// Column slices.  On a B much larger than the L2s, gathering one band of sw
// columns at a time (all rows, then the next band) lets more of the B rows
// in use stay in L2; A is read once per slice.  Measured on MI355X: 64-column
// slices cut the 65536 x 256 uniform config by 25% and the R-MAT N = 512
// config by 5-13%; on XL (N = 128) the column panels win and slices lose.
constexpr int kSliceWidth = 64;
// One launch per slice separates the slices' bands completely; one launch
// for all of them lets a slice's first blocks overlap the previous slice's
// last.  Measured: the first is 16-20% faster on uniform rows (66 nonzeros
// per row), the second 7-9% faster on R-MAT (15 per row, a few huge rows).
constexpr int kSliceLaunchMinAvgRow = 32;
inline bool slice_launches(int M, int nnz) {
  return M > 0 && (long long)nnz >= (long long)kSliceLaunchMinAvgRow * M;
}
// 0 (no slices) or the slice width for a K x N B; `panels` tells that the
// per-call column panels could apply (they are kept, unsliced, for N <= 128).
#ifndef CSRSPMM_SLICE_MIN_MB
#define CSRSPMM_SLICE_MIN_MB 32
#endif
#ifndef CSRSPMM_SLICE_BAND_MAX_MB
#define CSRSPMM_SLICE_BAND_MAX_MB 16
#endif
// `sweeps`: the call would sweep its slices with rows averaging at least
// kSweepWideMinPerBand nonzeros per band (wide_sweep); with no column panels
// possible (a max_row_nnz hint below kPanelMinLen, or a stored plan without
// such rows), such a call slices bands of any width.  Measured on MI355X with
// the hint, against no slices: 131072 x 131072 x 256 with 66 per row
// 1208 -> 875 us, 32 per row 600 -> 546 us; 98304^2 x 256 with 48 per row
// 663 -> 444 us; 262144^2 x 256 with 32 per row (2 per band) 1222 -> 1409
// us, below the threshold.
#ifndef CSRSPMM_SWEEP_WIDE
#define CSRSPMM_SWEEP_WIDE 1
#endif
constexpr int kSweepWideMinPerBand = 4;
inline int slice_width(int K, int N, bool panels, bool sweeps = false) {
  const long long full = (long long)K * N * 4;
  const long long band = (long long)K * kSliceWidth * 4;
  if (N < 2 * kSliceWidth || full < ((long long)CSRSPMM_SLICE_MIN_MB << 20)) return 0;
  if (N <= 128 && panels) return 0;
  const bool wide = CSRSPMM_SWEEP_WIDE && sweeps && !panels;
  if (band > ((long long)CSRSPMM_SLICE_BAND_MAX_MB << 20) && full < (1LL << 30) && !wide) return 0;
  return kSliceWidth;
}

// plan_kernel's row blocks: 256 rows each, grid-strided beyond kPlanMaxRowBlocks.
constexpr int kPlanMaxRowBlocks = 4096;
inline int plan_row_blocks(int M) {
  const long long b = ((long long)M + 1 + 255) / 256;
  return b < kPlanMaxRowBlocks ? (int)b : kPlanMaxRowBlocks;
}

// XCD slices (Problem::xslice): a float4 call whose B exceeds one XCD's L2
// (kXcdL2Bytes) but whose kSliceWidth-column bands fit it runs 2, 4 or 8
// slices in one launch, block b on slice b mod the slice count; blocks reach
// the XCDs in turn (b mod kXcds), so each XCD gathers from one band only.
// Measured on MI355X per call (rocprofv3), medium (16384^2, 82 per row,
// N = 128, 8 MiB B): main kernel 45.5 -> 40.5 us; 4 slices of 32 columns
// took 48.9 and 8 of 16 more (narrower gathers).  Returns the slice count
// (0: none).
constexpr long long kXcdL2Bytes = 4LL << 20;
inline int xcd_slices(int K, int N) {
  const long long full = (long long)K * N * 4;
  const long long band = (long long)K * kSliceWidth * 4;
  const int ns = (N + kSliceWidth - 1) / kSliceWidth;
  if (ns < 2 || ns > kXcds || (ns & (ns - 1)) != 0) return 0;
  return full > kXcdL2Bytes && band <= kXcdL2Bytes ? ns : 0;
}

// The plan is skipped for a hinted short-row problem (kPlanSkipItems).
inline bool plan_skips(int M, int K, int N, int nnz, int hint) {
  return hint >= 0 && hint <= kPlanSkipMaxRow && M < kPlanSkipRows &&
         (long long)M + nnz < kPlanSkipItems && slice_width(K, N, false) == 0;
}

// Resident blocks per CU for slices launched one by one over a band wider
// than kSliceCapBand (0: no cap).  Such a band streams through each XCD's
// 4 MiB L2 from the MALL and HBM, and with fewer blocks in flight fewer misses
// compete for L2 lines.  Measured on MI355X (65536 x 256 uniform, 16 MiB
// band): L2 hit rate 0.40 -> 0.50, DRAM read requests -17%, 10% faster, and
// 4-10% on other K = 65536 shapes; on an 8 MiB band, which half fits in L2,
// the cap cost 22%, so it stops there.  The cap is set by padding each
// block's LDS so that only kSliceBlocksPerCu fit in the CU's kLdsPerCu.
constexpr long long kSliceCapBand = 8LL << 20;
#ifndef CSRSPMM_SLICE_BLOCKS_PER_CU
#define CSRSPMM_SLICE_BLOCKS_PER_CU 6
#endif
constexpr int kSliceBlocksPerCu = CSRSPMM_SLICE_BLOCKS_PER_CU;
constexpr int kLdsPerCu = 160 * 1024;
inline int slice_blocks_per_cu(int K, int sw, bool slice_launch) {
  if (sw <= 0 || !slice_launch || (long long)K * sw * 4 <= kSliceCapBand) return 0;
  return kSliceBlocksPerCu;
}

// Per-call column panels, built on the device each call (panels.hip) from the
// CSR alone.  Positions of A's nonzeros are cut into windows of kPanelMinLen;
// a row of len >= kPanelMinLen contains the start of window
// id(r) = ceil(rowptr[r] / kPanelMinLen), which no other such row does, so
// id(r) names the row in the per-window tables below.
#ifndef CSRSPMM_PANEL_PARTIAL_MB
#define CSRSPMM_PANEL_PARTIAL_MB 256
#endif
constexpr long long kDevPanelPartialBudget = (long long)CSRSPMM_PANEL_PARTIAL_MB << 20;  // bytes of piece partials, at most
// A call panelizes at most nnz / kPanelRowCapLen rows as well (a quarter of
// the nnz / kPanelMinLen possible): the main launch sizes its pieces grid for
// nl_max rows, since the host cannot know how many there are, and a grid for
// 8192 rows where XL has 1501 left ~25,000 blocks that exit at once, 10 us
// of dispatch.  Rows beyond the cap, in row order, stay on segments.
constexpr long long kPanelRowCapLen = 4LL * kPanelMinLen;
constexpr int kDevPanelSample = 64;  // rows sampled for the panel loads
constexpr int kPanelHist = kXcds + 2;
struct DevPanels {
  int P;           // panels, ceil(K / 2^wshift) <= panel_count(K, N); 0 = off
  int wshift;      // columns per panel = 2^wshift: ceil(K / panel_count) rounded up to a power
                   // of two, so a column's panel is a shift
  int nwin;        // windows, ceil(nnz / kPanelMinLen)
  int nl_max;      // panelized rows at most (rows of the partial buffer)
  int4* win;       // [nwin] (r, rowptr[r], rowptr[r+1], w == id(r) of a long row) for the
                   // row r holding position w * kPanelMinLen
  int* pidx;       // [nwin] compact index of the panelized row with id w, else -1
  int* list;       // [nl_max] ids of the panelized rows, in row order
  int* bnd;        // [nwin][P + 1] absolute position where panel q starts in the row with id w
  int* sched;      // [0] = nl (0: no row panelized this call), [1 .. kXcds + 1] = XCD panel
                   // ranges, [kPanelHist + q] = sampled nonzeros in panel q
  float* part;     // [nl_max][P][ldp] piece partial sums
};

// Cap on the blocks of the segment phase.  By default every segment slot
// gets its own group, so the hardware dispatcher balances segments across
// CUs; a smaller cap makes the segment blocks persistent (grid-strided).
#ifndef CSRSPMM_SEG_BLOCKS_MAX
#define CSRSPMM_SEG_BLOCKS_MAX (1 << 24)
#endif
constexpr int kSegBlocksMax = CSRSPMM_SEG_BLOCKS_MAX;

struct Problem {
  int M, K, N, nnz;
  const int* rowptr;
  const int* colidx;
  const float* vals;
  const float* B;
  long long ldb;
  float* C;
  long long ldc;
  float alpha, beta;
  int epi;  // EpilogueMode
  // Plan (all inside the workspace, all written by plan_kernel each call).
  // plan == false: every row is processed whole by its own group.
  bool plan;
  int nslots;         // table slots, nnz / slot
  int mblk;           // merge block size (rows + nonzeros)
  int nblocks;        // merge blocks
  int* block_start;   // nblocks + 1 entries: first row of each merge block, then M
  int2* seg_info;     // per slot: (row, segment index) or (-1, 0) for an unused slot
  float* partials;    // nnz / seg partial rows of ldp floats
  long long ldp;
  // Per row block of plan_kernel: 1 when a row of the block needs the
  // combine (split into segments, by XCD or into panel pieces), else 0;
  // written by plan_kernel on every call.  nullptr: the combine scans anyway.
  unsigned char* need;
  int need_blocks;
  // A stored plan (csrspmm_plan_create) filled block_start / seg_info once:
  // no plan_kernel launch per call.
  bool plan_ready;
  // Panelized rows of a stored plan: row pan_rows[i] is summed in the combine
  // pass from the partials pan_part[pan_piece[k] * ldp] of its pieces
  // k in [pan_ptr[i], pan_ptr[i+1]), in column order.
  int npan;
  const int* pan_rows;
  const int* pan_ptr;
  const int* pan_piece;
  const float* pan_part;
  // Per-call column panels (dp.P == 0: off).
  DevPanels dp;
  // Column slice width (0: every block covers all N columns).  With sw > 0 the
  // main launch runs ceil(N / sw) slices of sw columns, one after another in
  // block order; the plan and the combine are shared.
  int sw;
  // Slices as one launch each (true) or all in one launch, slice after slice
  // in block order (false).
  bool slice_launch;
  // XCD slices (with slice_launch false): block b takes slice b mod the slice
  // count instead, so a slice count dividing kXcds keeps each slice on the
  // same XCDs and its band in their L2.
  bool xslice;
  // From the caller's max_row_nnz hint (or a stored plan's true maximum):
  // rows_whole, no row above kLongRow: no segment phase (nslots = 0) and the
  // merge blocks sum every row whole, whatever its length, so a hint that is
  // too small costs time, never correctness; no_split, no row of 2 * kSegLen
  // nonzeros: a long row is one segment, so no partials and no combine.
  bool rows_whole;
  bool no_split;
  // Segment geometry (seg_geom).  New fields go here, at the end: inserting
  // them above shifted the kernel-argument offsets of the fields after them
  // and, with the same kernel code, measured 4-5% slower on the XL configs.
  int seg_shift, slot_shift, long_row;
  // A per-call panel table added after the fields above, for the same
  // reason: dp_flag[w] = 1 when window w is id(r) of a long row whose columns
  // are sorted and in range (plan_kernel sets it from rowptr,
  // panel_window_kernel clears it), else 0.
  unsigned char* dp_flag;
  // A stored plan built the per-call panel schedule (dp), or the XCD share
  // entries, once: no panel schedule or share-bounds launches per call.
  bool dp_ready;
  // Band sweep of the short rows of a column slice (sweep_geometry; bands 0:
  // merge blocks instead): bands of 2^sweep_shift B rows, sweep_bands of them.
  int sweep_shift, sweep_bands;
  // The caller's max_row_nnz hint (or a stored plan's true longest row);
  // -1 when unknown.
  int row_hint;
  // XCD shares (share_applies; false: off): long rows are summed XCD by XCD
  // (see kShareSplitSegs); shr_cb holds the column boundaries (plan_kernel),
  // shr_pb the per-slot share entries (share_bounds_kernel), both written
  // each call, shr_part the parts' partial rows.
  bool shares;
  int* shr_cb;
  int4* shr_pb;
  float* shr_part;
  // The split rows summed in the main launch (seg_fuse: a per-call plan
  // with no column panels, XCD shares or stored panels): each segment of a
  // split row counts itself in seg_cnt[the row's first slot], which
  // plan_kernel zeroes, and the last of the row's segments (in every column
  // slice) adds its partial rows, so no combine is launched.
  bool seg_fuse;
  int* seg_cnt;
};

// XCD shares.  On a B far larger than the L2s, with no column panels (hot
// columns spread over the whole index range, as in R-MAT, or rows too short
// for panels), every XCD gathers from all of B and its 4 MiB L2 keeps little.
// Instead, the columns are cut into kXcds ranges at boundaries chosen per call
// so that each range carries about 1/kXcds of a column sample, and the long
// rows' nonzeros of range x are summed on XCD x (block b runs on XCD
// b mod kXcds): each L2 then serves 1/kXcds of the columns.  Measured with an
// LRU model of the eight L2s over R-MAT N = 64 (16.1 M nonzeros): hit rate
// 0.39 -> 0.65, L2 misses 2.66 -> 1.52 GB; the model gave 0.39 for the
// unsplit call, as the hardware counters do.
//
//  * A long row of fewer than kShareSplitSegs segments (under 2048
//    nonzeros) is split: its part x, the nonzeros whose column lies in
//    range x (for a sorted row, a contiguous run), is summed on XCD x into
//    shr_part row (rowptr[r] >> kShareIdxShift) + x, written (zero when
//    empty) for every x, and the combine adds the row's kXcds consecutive
//    partial rows in order.  Such a row owns the rows
//    [rowptr[r] >> 4, rowptr[r+1] >> 4), at least floor(len / 16) >= kXcds
//    of them (len > 128), so the rows of all split rows tile the buffer
//    without a scan.
//  * A longer row keeps its segments whole, each summed on the XCD whose
//    range holds the column at the segment's middle, into the ordinary
//    segment partials: its segments are narrow in column space, and
//    splitting them would only multiply its partials by kXcds.
//
// The parts of a segment partition its positions whatever the boundaries,
// so the results never depend on them, only the locality does.
constexpr int kShareIdxShift = 4;
constexpr int kShareSplitSegs = 8;
constexpr int kShareSamples = 4096;      // columns sampled for the boundaries
constexpr int kShareBins = 1024;         // histogram bins of the sample
constexpr long long kShareMinBand = 64LL << 20;  // bytes of B (one column slice) from which to split
constexpr int kShareMinNnz = 1 << 20;
static_assert(kXcds == 8, "a slot's part offsets are 8 ints");

// The call splits its long rows by XCD: the plan on, no per-call column
// panels, a B (or column slice of it) of at least kShareMinBand, rows that
// can be long under the hint, and segments of at least 128 nonzeros (the
// partial numbering above).
inline bool share_applies(bool plan, int K, int N, int nnz, int sw, int P, int hint) {
  if (!plan || P > 0 || nnz < kShareMinNnz || K <= 0) return false;
  const SegGeom g = seg_geom(nnz);
  if (g.seg_shift < 7 || g.long_row < 128) return false;
  if (hint >= 0 && hint <= g.long_row) return false;
  return (long long)K * (sw > 0 ? sw : N) * 4 >= kShareMinBand;
}

// Band sweep (sliced float4 calls).  Each group keeps kSweepRows rows'
// accumulators in registers while all groups walk the slice's band of B in
// bands of about kSweepBandBytes, so a band stays in the L2s while every row
// takes its nonzeros in it.  Measured on MI355X, per call against the merge
// blocks (bit-identical): 65536 x 65536 x 256 with 66 per row 387 -> 286 us
// (L2 hit rate per slice 0.47 -> 0.70, fetched bytes -42%), 16 per row
// 151 -> 113 us, 128 per row 870 -> 460 us; 131072 x 131072 x 256 with 66
// per row 1247 -> 806 us; 65536 x 65536 x 512 with 66 per row 765 -> 572 us.
#ifndef CSRSPMM_SWEEP_BAND_KB
#define CSRSPMM_SWEEP_BAND_KB 4096
#endif
constexpr int kSweepRows = 2;
constexpr int kSweepMaxBands = 64;
// (shift, bands) for a K-row B swept in slices of sw columns: the smallest
// power-of-two band of at least CSRSPMM_SWEEP_BAND_KB KiB, widened until
// at most kSweepMaxBands cover K.
inline void sweep_geometry(int K, int sw, int& shift, int& bands) {
  shift = 0;
  while (((long long)sw * 4 << shift) < ((long long)CSRSPMM_SWEEP_BAND_KB << 10)) ++shift;
  while (((long long)K + (1LL << shift) - 1) >> shift > kSweepMaxBands) ++shift;
  bands = (int)(((long long)K + (1LL << shift) - 1) >> shift);
}
// The sweep pays when rows average enough nonzeros per band.  Measured on
// MI355X: 65536 x 65536 x 256 with 8 per row (2 per band) 88.7 -> 79.2 us,
// with 16 per row (4 per band) 148.5 -> 119.9 us; R-MAT N = 512 (15 per row,
// 0.24 per band) 4.86 -> 9.03 ms, so it keeps the merge blocks.
#ifndef CSRSPMM_SWEEP_MIN_PER_BAND
#define CSRSPMM_SWEEP_MIN_PER_BAND 2
#endif
// A group keeps one gather per row in flight, so the sweep also needs
// enough groups to hide latency: at least 8192 waves for 16-lane groups (64
// columns) and 4096 for 32-lane ones.  Measured on MI355X per call against
// the merge blocks, K = 65536 x 256 sliced with 66 per row: M = 8192 (1024
// waves) 74 -> 170 us, 16384 101 -> 176, 32768 (4096 waves) 183 -> 190,
// 65536 (8192 waves) 380 -> 305; unsliced K = 32768 x 128 with 100 per row:
// M = 8192 (2048 waves) 38 -> 55, 12288 55 -> 56, 16384 (4096 waves) 75 ->
// 59, 24576 115 -> 69.
inline bool sweep_applies(bool plan, int M, int K, int nnz, int sw,
                          int min_per_band = CSRSPMM_SWEEP_MIN_PER_BAND) {
  if (!plan || sw <= 0 || M <= 0 || K <= 0) return false;
  const int G = sw / 4;  // lanes per group, float4 columns
  const long long waves = (long long)M / kSweepRows * G / 64;
  if (waves < (G >= 32 ? 4096 : 8192)) return false;
  int shift, bands;
  sweep_geometry(K, sw, shift, bands);
  return (long long)nnz >= (long long)min_per_band * bands * M;
}
// The call's slices would be swept (float4 columns, vec 4, with a plan) with
// at least kSweepWideMinPerBand nonzeros per band and row: slice_width's
// `sweeps`.
inline bool wide_sweep(int vec, bool plan, int M, int K, int nnz) {
  return vec == 4 && sweep_applies(plan, M, K, nnz, kSliceWidth, kSweepWideMinPerBand);
}

// Segments of a row of len nonzeros under the problem's geometry and hint.
__host__ __device__ inline int seg_count(const Problem& p, int len) {
  const int n = seg_count(len, p.long_row, p.seg_shift);
  return p.no_split && n > 1 ? 1 : n;
}

// The hint flags for a longest row of max_row_nnz nonzeros (-1: unknown).
inline void set_row_hint(Problem& p, int max_row_nnz) {
  p.row_hint = max_row_nnz < 0 ? -1 : max_row_nnz;
  p.rows_whole = max_row_nnz >= 0 && max_row_nnz <= p.long_row;
  p.no_split = max_row_nnz >= 0 && max_row_nnz < (2 << p.seg_shift);
  if (p.rows_whole) p.nslots = 0;
}

// Workspace layout for a problem (all offsets 256-byte aligned).  P > 0 adds
// the per-call panel tables and partial buffer after the base sections.
struct WorkspaceLayout {
  size_t block_start_off, seg_info_off, partials_off, need_off, segcnt_off, base_total;
  size_t win_off, flag_off, pidx_off, list_off, bnd_off, sched_off, part_off, total;
  int nslots, nblocks;
  long long ldp;
  int P, wshift, nwin, nl_max;
  // XCD shares (after the base sections; panels and shares exclude each other)
  bool shares;
  size_t shr_cb_off, shr_pb_off, shr_part_off;
};
WorkspaceLayout workspace_layout(int M, int K, int N, int nnz, int P, bool shares = false);

// Panels the per-call path uses for this problem (0: none): float4 columns
// (or scalar ones from N = kPanelMinScalarN), the plan on, and a row of
// kPanelMinLen nonzeros possible under the hint.
int per_call_panels(int vec, bool plan, int K, int N, int nnz, int hint);

// Bind the plan pointers of p into a workspace base pointer; merge blocks of
// mblk (the layout holds block starts for any merge block size).
void bind_workspace(Problem& p, void* ws, const WorkspaceLayout& L, int mblk);

// Shared by the per-call C ABI and stored plans (capi.hip).
int resolve_algorithm(int algo, int N);  // CSRSPMM_ALGO_AUTO -> a concrete variant; -1 if invalid
int resolve_algorithm(int algo, int M, int K, int N, int nnz, int hint);  // the same, from the shape
bool is_rowgroup_algorithm(int algo);
bool uses_lds(int algo);
int vector_width(int algo, const Problem& p);
int fill_problem(Problem& p, int algo, int M, int K, int N, int nnz, const int* rowptr,
                 const int* colidx, const float* vals, const float* B, long long ldb, float* C,
                 long long ldc, float alpha, float beta, unsigned flags);
hipError_t launch_algorithm(int algo, const Problem& p, hipStream_t s);

hipError_t launch_naive(const Problem& p, hipStream_t s);
hipError_t launch_naive_smem(const Problem& p, hipStream_t s);
// vec = 1 (scalar columns) or 4 (float4 columns); lds = stage (col,val) in LDS.
hipError_t launch_rowgroup(const Problem& p, int vec, bool lds, hipStream_t s);

// Per-call panel schedule (panels.hip): after plan_kernel has filled dp.win
// and dp_flag, find the panel boundaries of the long rows, then compact the
// panelized rows and deal the panels to the XCDs.
hipError_t launch_panel_schedule(const Problem& p, hipStream_t s);

// XCD shares: after plan_kernel has written the column boundaries and the
// segment slots, record where each XCD's part of every split row begins and
// which XCD sums each segment kept whole.
hipError_t launch_share_bounds(const Problem& p, hipStream_t s);



// The tables of a planned call without the product: plan_kernel and, with
// column panels, the panel schedule (stored plans build them once).
hipError_t launch_plan_tables(const Problem& p, hipStream_t s);

// Benchmark timing hook: no-ops unless csrspmm_timing_enable(1) was called.
// Calls nest (per thread): only the outermost before/after pair records, so
// one SpMM made of several launches is timed as one.
void timing_before_main(hipStream_t s);
void timing_after_main(hipStream_t s);

hipError_t launch_validate(int M, int K, int nnz, const int* rowptr, const int* colidx,
                           int* d_out /* [0]=flags, [1]=max_row_nnz */, hipStream_t s);

}  // namespace csrspmm_hip
