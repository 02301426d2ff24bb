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

// Segment length for splitting long rows.  A row longer than kSplitLen
// nonzeros is cut into ceil(len / kSplitLen) segments of kSplitLen nonzeros
// (the last one shorter); each segment's partial sum goes to the workspace
// and a combine pass adds them in segment order.
constexpr int kSplitLen = 256;

// Blocks of the persistent segment phase / combine phase: a few per CU.
constexpr int kPersistentBlocks = 1024;

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
  // Row-split plan (all inside the workspace); plan == false means every row
  // is processed whole by its row group.
  bool plan;
  int* counters;     // [0] = #segments, [1] = #long rows, [2] = overflow flag
  int2* seg_info;    // (row, segment index within row)
  int4* long_rows;   // (row, first segment slot, #segments, 0)
  float* partials;   // seg_cap x ldp floats
  long long ldp;
  int seg_cap;
  int long_cap;
};

// Workspace layout for a problem (all offsets 256-byte aligned).
struct WorkspaceLayout {
  size_t counters_off, seg_info_off, long_rows_off, partials_off, total;
  int seg_cap, long_cap;
  long long ldp;
};
WorkspaceLayout workspace_layout(int M, int N, int nnz);

// Bind the plan pointers of p into a workspace base pointer.
void bind_workspace(Problem& p, void* ws, const WorkspaceLayout& L);

hipError_t launch_naive(const Problem& p, hipStream_t s);
hipError_t launch_naive_smem(const Problem& p, hipStream_t s);
// vec = 1 (scalar columns) or 4 (float4 columns); lds = stage (col,val) in LDS.
hipError_t launch_rowgroup(const Problem& p, int vec, bool lds, hipStream_t s);

// Benchmark timing hook: no-ops unless csrspmm_timing_enable(1) was called.
void timing_before_main(hipStream_t s);
void timing_after_main(hipStream_t s);

hipError_t launch_validate(int M, int K, int nnz, const int* rowptr, const int* colidx,
                           int* d_out /* [0]=flags, [1]=max_row_nnz */, hipStream_t s);

}  // namespace csrspmm_hip
