/*
 * csrspmm_c.h -- the C ABI of the MI355X (gfx950) CSR SpMM library.
 *
 * Computes C = alpha * A * B + beta * C for A in CSR (int32 indices, fp32
 * values, M x K, nnz nonzeros) and dense row-major fp32 B (K x N, leading
 * dimension ldb) and C (M x N, leading dimension ldc).  When beta == 0 the
 * prior contents of C are never read (NaN in C is overwritten).
 *
 * Every entry point takes plain pointers and sizes, no C++ or torch types.
 * Device pointers are caller-owned; the library never frees user memory.
 * Status convention: 0 = success, negative = CSRSPMM_STATUS_* below,
 * positive = a hipError_t value reported by the HIP runtime.
 *
 * This header is the only surface through which host C++ (libcsrspmm.so,
 * built with g++), the torch extension and ctypes reach HIP.  Each entry
 * point names the reference interface it replaces (anh-thh/csrspmm paths).
 */
#ifndef CSRSPMM_C_H_
#define CSRSPMM_C_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Algorithm ids, in the order of csrspmm::Algorithm
 * (reference include/csrspmm/csrspmm.h:10-17). */
enum {
    CSRSPMM_ALGO_NAIVE = 0,
    CSRSPMM_ALGO_NAIVE_SMEM = 1,
    CSRSPMM_ALGO_WARP_PER_ROW = 2,
    CSRSPMM_ALGO_WARP_PER_ROW_FP4 = 3,
    CSRSPMM_ALGO_WARP_PER_ROW_SMEM = 4,
    CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4 = 5,
    CSRSPMM_ALGO_COUNT = 6,   /* number of concrete variants */
    /* Pick a variant from the problem (csrspmm_resolve_algorithm).  Fills the
     * reference's "auto-selection" stub (src/csrspmm.cpp:34-40). */
    CSRSPMM_ALGO_AUTO = 6
};

enum {
    CSRSPMM_STATUS_SUCCESS = 0,
    CSRSPMM_STATUS_INVALID_VALUE = -1,     /* bad size, null pointer, bad ld, unknown algo */
    CSRSPMM_STATUS_NOT_SUPPORTED = -2,     /* shape beyond int32 index range */
    CSRSPMM_STATUS_ALLOC_FAILED = -3,      /* library-owned workspace could not grow */
    CSRSPMM_STATUS_INVALID_CSR = -4,       /* validator found a malformed CSR */
    CSRSPMM_STATUS_WORKSPACE_TOO_SMALL = -5,
    /* csrspmm_spmm_f32_noalloc: the base workspace exceeds its scratch */
    CSRSPMM_STATUS_SCRATCH_TOO_SMALL = -6
};

/* Validator result bits (csrspmm_validate_csr). */
enum {
    CSRSPMM_CSR_OK = 0,
    CSRSPMM_CSR_BAD_ROWPTR0 = 1,       /* rowptr[0] != 0 */
    CSRSPMM_CSR_BAD_ROWPTR_END = 2,    /* rowptr[M] != nnz */
    CSRSPMM_CSR_NON_MONOTONE = 4,      /* rowptr[i+1] < rowptr[i] for some i */
    CSRSPMM_CSR_COL_OUT_OF_RANGE = 8,  /* col < 0 or col >= K */
    CSRSPMM_CSR_UNSORTED = 16,         /* informational: columns not strictly increasing in a row */
    CSRSPMM_CSR_FATAL_MASK = 15        /* bits that make a kernel launch unsafe */
};

/* Library version as 10000*major + 100*minor + patch. */
int csrspmm_version(void);

/* Human-readable text for a status code (never NULL). */
const char* csrspmm_status_string(int status);

/* Name -> algorithm id by exact CamelCase match ("Naive", "NaiveSmem",
 * "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4");
 * returns -1 for an unknown name.  The C++ parse_algorithm adds the
 * reference's warn-and-fall-back-to-Naive behaviour on top
 * (reference src/csrspmm.cpp:13-25). */
int csrspmm_parse_algorithm(const char* name);

/* Algorithm id -> CamelCase name ("Auto" for CSRSPMM_ALGO_AUTO), or NULL. */
const char* csrspmm_algorithm_name(int algo);

/* The concrete variant CSRSPMM_ALGO_AUTO picks from N output columns alone
 * (a concrete id is returned unchanged; -1 for an invalid id). */
int csrspmm_resolve_algorithm(int algo, int N);
/* The concrete variant CSRSPMM_ALGO_AUTO runs for the whole shape (A is
 * M x K with nnz nonzeros, N output columns, max_row_nnz_hint as for the
 * SpMM, -1 if unknown): csrspmm_resolve_algorithm's choice, except that
 *  - from N = 128 (N % 4 == 0), a call cut into column slices that are not
 *    swept, or swept with fewer than 4 nonzeros per band and row, whose
 *    long rows are split by XCD (csrspmm_call_shares for the float4
 *    variant), takes the scalar LDS-staged variant;
 *  - below N = 128 (N % 4 == 0), rows of 24 or more nonzeros on average
 *    with per-call column panels possible for float4 columns (a B of at
 *    least 64 MiB, a row of 1024 or more not ruled out) take the float4
 *    broadcast variant, which has the panels;
 *  - at N = 128 a B of at most 4 MiB with rows of 96 or more nonzeros on
 *    average (M >= 4096, or M >= 1024 when the hint lets the call run as
 *    one launch) takes the scalar LDS-staged variant;
 *  - from N = 128, a call cut into column slices whose hint exceeds both
 *    128 and 4x the mean row length (skewed rows) takes the scalar
 *    LDS-staged variant;
 *  - otherwise, from N = 128, a call whose column slices are swept (a B of
 *    at least 32 MiB in bands, rows dense enough per band, M large enough)
 *    takes the float4 LDS-staged variant;
 *  - and a sliced call that is not swept, of rows averaging 64 to 511
 *    nonzeros or with a hint of 129 to 511, takes the scalar LDS-staged
 *    variant, unless its 64-column band exceeds 8 MiB, M is at least 4096 and
 *    rows exceed 128 (the hint, or the mean without one).
 * The SpMM entry points resolve Auto this way, and stored plans with the
 * true longest row.  No counterpart in the reference, whose Auto stub is
 * empty. */
int csrspmm_resolve_algorithm_ex(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint);

/* Bytes of device workspace csrspmm_spmm_f32_ws needs for this problem
 * (row-split plan, partial sums of split rows, counters).  No counterpart in
 * the reference, which has no long-row splitting. */
size_t csrspmm_workspace_bytes(int algo, int M, int N, int nnz);

/* As csrspmm_workspace_bytes, plus the per-call column-panel tables and
 * partial sums used for rows of >= 1024 nonzeros when B (K x N fp32) is
 * >= 64 MiB and N <= 256, with float4 columns or from N = 128 with scalar
 * ones (at most 256 MiB of partials).  A
 * max_row_nnz_hint in [0, 1024) tells that no such row exists (-1: unknown).
 * csrspmm_spmm_f32_ex given a workspace of at least
 * csrspmm_workspace_bytes but less than this size runs without panels.
 * A hint in [0, 256] on fewer than 2^20 rows + nonzeros and 32768 rows, when
 * B is not cut into column slices, gives 0: such a call runs as one launch
 * with no plan and no workspace.  It also holds the XCD share tables and
 * partial sums (csrspmm_call_shares: (nnz / 16) x N floats) of a call that
 * splits its long rows by XCD; a smaller workspace of at least
 * csrspmm_workspace_bytes runs without them. */
size_t csrspmm_workspace_bytes_ex(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint);

/* 1 when a per-call product of this shape, given a workspace of
 * csrspmm_workspace_bytes_ex bytes and 16-byte aligned B and C rows, splits
 * its long rows (above 128 nonzeros) by XCD, else 0.  Such a call cuts each
 * long-row segment at eight column ranges chosen from a sample of the
 * columns, sums the part of range x on XCD x, and adds the parts in range
 * order: within the 1e-5 bar, but no longer the CSR order of the fp32
 * restatement for those rows.  It applies with the plan on, no column
 * panels, nnz >= 2^20 and a B (or 64-column slice of it) of at least
 * 64 MiB, unless the hint rules out rows above 128.  For tests and tuning;
 * no counterpart in the reference, whose kernels sum each row on one warp. */
int csrspmm_call_shares(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint);

/* Where a per-call workspace of csrspmm_workspace_bytes_ex bytes holds the
 * call's column-panel decision, for tests and tuning: returns the number of
 * column panels such a call uses (0: none, and *nl_offset is left alone)
 * when B and C rows are 16-byte aligned, and sets *nl_offset to the byte
 * offset of an int32 that the call writes: the number of rows it panelized,
 * 0 when the panel loads were too skewed.  Reading it needs the call to have
 * finished.  No counterpart in the reference, which has no panels. */
int csrspmm_workspace_panel_info(int algo, int M, int K, int N, int nnz, int max_row_nnz_hint,
                                 long long* nl_offset);

/*
 * The SpMM.  Replaces csrspmm::spmm's dispatch to launch_<variant>
 * (reference src/csrspmm.cpp:28-71, src/host/spmm_launcher.cu:11-171) and the
 * torch forwards' launch (reference torch_csrspmm/torch_csrspmm_*.cpp).
 *   algo            CSRSPMM_ALGO_*
 *   M, K, N, nnz    A is M x K with nnz nonzeros; B is K x N; C is M x N
 *   rowptr, colidx, vals   device CSR arrays (M+1, nnz, nnz entries); as in
 *                   the reference, rowptr must run from 0 to nnz without
 *                   decreasing and every column must lie in [0, K); the
 *                   per-call path does not check (csrspmm_validate_csr does).
 *                   Columns need not be sorted within a row.
 *   max_row_nnz_hint       -1 if unknown; otherwise the caller's claim of the
 *                   longest row.  It only steers the schedule (and Auto's
 *                   variant): at most 128 drops the long-row segments and
 *                   their combine pass, below 512 the split rows and the
 *                   combine, below 1024 the column panels, and a matrix under
 *                   2^20 rows + nonzeros and 32768 rows (no column slices)
 *                   with no row above 256 runs as one launch.  Never used to
 *                   size memory or bound a loop:
 *                   a hint below the true longest row still gives the exact
 *                   result, only more slowly.
 *   B, ldb, C, ldc  row-major dense operands, ldb >= N, ldc >= N
 *   stream          hipStream_t (NULL = legacy default stream)
 * Asynchronous: returns after enqueueing.  Uses a library-owned device
 * workspace kept per (device, stream) and grown on demand; calls on one
 * stream are ordered, calls on different streams use different workspaces.
 * Thread-safe: a call holds the library's workspace lock until its kernels
 * are enqueued, so another thread growing or releasing the same workspace
 * waits for them.
 */
int csrspmm_spmm_f32(int algo, int M, int K, int N, int nnz,
                     const int* rowptr, const int* colidx, const float* vals,
                     int max_row_nnz_hint,
                     const float* B, long long ldb,
                     float* C, long long ldc,
                     float alpha, float beta,
                     void* stream);

/*
 * Library-owned workspaces (those of csrspmm_spmm_f32).  The library keeps
 * at most 16 of them (one per device and stream, and per host thread for
 * hipStreamPerThread), evicting the least recently used one beyond that.
 * No counterpart in the reference, whose kernels need no workspace.
 *
 * csrspmm_release_workspace frees the workspace of (current device, stream)
 * after synchronising that stream; 0 when there was none.  The next call on
 * the stream allocates a new one.
 * csrspmm_release_all_workspaces frees every one of them, on every device,
 * each after a device synchronise (their streams may no longer exist).
 * csrspmm_owned_workspaces returns how many are held and, in *bytes_out (may
 * be NULL), their total size.
 * All three are safe to call from any thread, concurrently with
 * csrspmm_spmm_f32 on other streams.
 */
int csrspmm_release_workspace(void* stream);
int csrspmm_release_all_workspaces(void);
int csrspmm_owned_workspaces(size_t* bytes_out);

/* Flags for csrspmm_spmm_f32_ex. */
enum {
    /* Treat the prior contents of C as +0.0 without reading them:
     * C = fma(alpha, sum, beta * 0.0f).  This is what the reference torch
     * forwards compute by allocating C with zeros() whenever beta != 0
     * (torch_csrspmm/torch_csrspmm_naive.cpp:32-34), without the memset and
     * the read of C. */
    CSRSPMM_FLAG_C_IS_ZERO = 1
};

/* As csrspmm_spmm_f32, with CSRSPMM_FLAG_* flags and a caller-provided
 * device workspace of at least csrspmm_workspace_bytes(algo, M, N, nnz)
 * bytes, 256-byte aligned (torch's caching allocator, for example; it may be
 * NULL when that size is 0).  Allocates nothing.  The torch forwards call
 * this entry point. */
int csrspmm_spmm_f32_ex(int algo, int M, int K, int N, int nnz,
                        const int* rowptr, const int* colidx, const float* vals,
                        int max_row_nnz_hint,
                        const float* B, long long ldb,
                        float* C, long long ldc,
                        float alpha, float beta,
                        unsigned flags,
                        void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * As csrspmm_spmm_f32_ex, with no workspace argument and no allocation: no
 * counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a static device array of
 * CSRSPMM_NOALLOC_SCRATCH_BYTES (128 MiB) in the library, one per GPU, which
 * each GPU the library runs on holds until the process ends.  A problem whose
 * base workspace (block starts, segment slots and partials of the call's own
 * plan; none when the call runs as one launch, as a max_row_nnz hint can
 * make it) exceeds it is rejected with CSRSPMM_STATUS_SCRATCH_TOO_SMALL
 * before anything is enqueued; one whose per-call column-panel or XCD share
 * tables do not fit as well runs without them (more slowly; without the
 * shares, rows above 128 nonzeros are summed in CSR order segment by
 * segment, a result within the same bound).  The five benchmark
 * configurations all fit, with their panels (R-MAT without its shares).
 * Calls no hipMalloc or hipFree
 * (the first call on a device looks the array's address up once).
 * All calls on one GPU share its array: calls that overlap on one GPU (on
 * different streams, or from different threads) race and give wrong
 * results; order them on one stream or synchronise between them.
 */
#define CSRSPMM_NOALLOC_SCRATCH_BYTES (128ull << 20)
int csrspmm_spmm_f32_noalloc(int algo, int M, int K, int N, int nnz,
                             const int* rowptr, const int* colidx, const float* vals,
                             int max_row_nnz_hint,
                             const float* B, long long ldb,
                             float* C, long long ldc,
                             float alpha, float beta,
                             unsigned flags,
                             void* stream);

/*
 * Stored plans: analyse A once, then multiply it by many B.  No counterpart
 * in the reference, whose spmm() re-derives nothing between calls
 * (src/csrspmm.cpp:28-75); its "auto-selection" stub (:34-40) is what
 * CSRSPMM_ALGO_AUTO fills.
 *
 * csrspmm_plan_create synchronises `stream`, reads rowptr (and, for
 * very long rows on a large B, their columns and values) to the host, and
 * keeps on the device:
 *  - the merge-block starts and long-row segment slots (no per-call plan
 *    kernel);
 *  - for rows of >= 1024 nonzeros with sorted columns when K*N*4 >= 16 MiB, a
 *    column-panel copy of the row pieces, laid out so that each of the 8 XCDs
 *    streams its own panels in order and keeps the gathered B band in its L2;
 *  - partial-sum buffers for n_hint columns (grown on a call with larger N).
 * n_hint <= 0 means 128.  The CSR arrays are referenced, not copied (except
 * the panel pieces): they must stay alive and unchanged while the plan is
 * used.  A plan serves one stream at a time (its partial buffers are shared
 * by its calls).  Creation and destruction allocate and synchronise; calls
 * allocate only when N outgrows the buffers.
 */
typedef struct csrspmm_plan_s* csrspmm_plan_t;

int csrspmm_plan_create(int algo, int M, int K, int nnz,
                        const int* rowptr, const int* colidx, const float* vals,
                        int n_hint, void* stream, csrspmm_plan_t* plan);

/* C = alpha * A * B + beta * C with the plan's A; flags as for
 * csrspmm_spmm_f32_ex.  Asynchronous on `stream`. */
int csrspmm_plan_spmm_f32(csrspmm_plan_t plan, int N,
                          const float* B, long long ldb,
                          float* C, long long ldc,
                          float alpha, float beta, unsigned flags, void* stream);

/* The concrete variant the plan runs. */
int csrspmm_plan_algorithm(csrspmm_plan_t plan);
/* Device memory the plan holds, in bytes. */
size_t csrspmm_plan_device_bytes(csrspmm_plan_t plan);
/* Rows the plan cut into column panels. */
int csrspmm_plan_panelized_rows(csrspmm_plan_t plan);
/* 1 when the plan's calls of N columns (16-byte aligned B and C rows) split
 * their long rows by XCD (as csrspmm_call_shares reports for a per-call
 * product, with the plan's true longest row as the hint): rows above 128
 * nonzeros are then summed in parts rather than in CSR order.  0 otherwise;
 * a negative status for a null plan or N <= 0.  No counterpart in the reference: a query for tests and tools,
 * like csrspmm_plan_panelized_rows. */
int csrspmm_plan_shares(csrspmm_plan_t plan, int N);
/* Waits for the device, then frees the plan (NULL is a no-op). */
int csrspmm_plan_destroy(csrspmm_plan_t plan);

/* Device-side CSR validation.  Writes the CSRSPMM_CSR_* bit set to
 * *flags_out and the true longest row to *max_row_nnz_out (host pointers,
 * either may be NULL); synchronises the stream.  Returns a status.  The
 * reference has no validator; it stands in for the max_row_nnz scan that
 * dense2csr performs on the host (reference src/host/csr_utils.cpp:106-110). */
int csrspmm_validate_csr(int M, int K, int nnz,
                         const int* rowptr, const int* colidx,
                         int* flags_out, int* max_row_nnz_out,
                         void* stream);

/*
 * Device-side CSR tooling, asynchronous on `stream` (no host sync).
 *
 * Dense -> CSR replaces the reference's host dense2csr
 * (src/host/csr_utils.cpp:70-111) with the same rule: element (r, c) of the
 * row-major M x K matrix `dense` (leading dimension ld >= K) is kept when
 * fabsf(v) > tol, so +-0 and NaN are dropped, in row-major order.  Two steps,
 * because the output size depends on the data:
 *  1. csrspmm_dense2csr_count_f32 writes rowptr[0..M] and the nonzero count
 *     as a 64-bit integer to *nnz_out (both device memory);
 *  2. after allocating colidx and vals for that count (it must fit int32),
 *     csrspmm_dense2csr_fill_f32 fills them.  Step 2 must see the same dense
 *     values, tol and rowptr as step 1.
 */
int csrspmm_dense2csr_count_f32(int M, int K, const float* dense, long long ld, float tol,
                                int* rowptr, long long* nnz_out, void* stream);
int csrspmm_dense2csr_fill_f32(int M, int K, const float* dense, long long ld, float tol,
                               const int* rowptr, int* colidx, float* vals, void* stream);

/* *max_out (device memory) = the longest row of rowptr[0..M]: the
 * max_row_nnz that the reference's dense2csr scans on the host
 * (src/host/csr_utils.cpp:106-110) and its torch benchmark fetches with a
 * host sync (torch_csrspmm/torch_benchmarks.py:39-44), here left on the device. */
int csrspmm_csr_max_row_nnz(int M, const int* rowptr, int* max_out, void* stream);

/* dst[i] = (int32)src[i] for i < n: int64 CSR indices (torch.sparse_csr's
 * default) narrowed for this library's int32 kernels.  If overflow_out
 * (device memory) is not NULL it is set to 1 when some value does not fit
 * int32, else 0.  The reference accepts int32 only
 * (torch_csrspmm/torch_csrspmm_naive.cpp:24-26). */
int csrspmm_indices_i64_to_i32(const long long* src, int* dst, long long n, int* overflow_out,
                               void* stream);

/* Memory and device helpers that let the g++-built C++ layer stay free of
 * HIP headers (they back csr_alloc_device / dense_alloc_device and the
 * host<->device copies at reference src/host/csr_utils.cpp:44-67,183-238 and
 * src/host/dense_utils.cpp:28-44,128-162). */
int csrspmm_device_malloc(void** ptr, size_t bytes);
int csrspmm_device_free(void* ptr);
int csrspmm_memcpy_h2d(void* dst, const void* src, size_t bytes);
int csrspmm_memcpy_d2h(void* dst, const void* src, size_t bytes);
int csrspmm_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int csrspmm_device_synchronize(void);
int csrspmm_stream_synchronize(void* stream);
/* Returns and clears the last HIP error of this thread (cudaGetLastError at
 * reference src/csrspmm.cpp:73). */
int csrspmm_get_last_error(void);
/* Number of visible devices (0 when no GPU); never initialises a context
 * beyond what hipGetDeviceCount does. */
int csrspmm_device_count(void);

/* Kernel timing for benchmarks (no counterpart in the reference, whose bench
 * times whole spmm() calls with cudaEvents, benchmarks/bench_csrspmm.cu:103-118).
 * While enabled (process-wide), every SpMM call records a HIP event pair
 * around its main kernel on the call's stream.  csrspmm_timing_read waits for
 * the recorded pairs, returns the summed main-kernel milliseconds and the
 * number of calls since the previous read, and recycles the events. */
int csrspmm_timing_enable(int on);
int csrspmm_timing_read(double* main_kernel_ms, int* calls);

#ifdef __cplusplus
}
#endif

#endif /* CSRSPMM_C_H_ */
