// High-level CSR SpMM API (reference include/csrspmm/csrspmm.h:10-34).
#pragma once
#include <string>

#include <csrspmm/config.h>
#include <csrspmm/csr_utils.h>
#include <csrspmm/matrix.h>
#if defined(__HIPCC__) || defined(__HIP__)
// HIP code also sees the kernel declarations, as the reference's csrspmm.h:6
// gives them (other compilers cannot parse __global__).
#include <csrspmm/kernels.h>
#endif

struct csrspmm_plan_s;  // opaque plan of the C ABI (include/csrspmm_c.h)

namespace csrspmm {

// The reference's enumerators in the reference's order (csrspmm.h:10-17),
// then Auto, which picks a variant from N (the reference's spmm() has only an
// "auto-selection" stub that always runs Naive, src/csrspmm.cpp:34-40).
enum class Algorithm {
    Naive,
    NaiveSmem,
    WarpPerRow,
    WarpPerRowFp4,
    WarpPerRowSmem,
    WarpPerRowSmemFp4,
    Auto
};

// Exact CamelCase match ("Auto" included); an unknown name prints a warning
// to stderr and returns Naive (reference src/csrspmm.cpp:13-25).
Algorithm parse_algorithm(const std::string& name);

// C = alpha * A * B + beta * C on the device.
//   A: CSR, M x K (device arrays);  B: dense K x N;  C: dense M x N.
// When beta == 0, C is not read.  Runs on the default stream and returns
// after the device has finished (reference src/csrspmm.cpp:28-75); a launch
// or runtime error prints a message and exits the process, as the
// reference's cudaCheck does.
void spmm(const CSRMatrix& A,
          const DenseMatrix& B,
          DenseMatrix& C,
          float alpha, float beta,
          Algorithm algo = Algorithm::Naive);

// A stored plan for repeated products with one device CSR matrix A
// (include/csrspmm_c.h, csrspmm_plan_*): analysed once, including the
// column-panel layout of very long rows that speeds up large, skew-free
// matrices.  A's arrays must outlive the plan and stay unchanged.  Errors
// print a message and exit, like the rest of this API.
class SpmmPlan {
public:
    explicit SpmmPlan(const CSRMatrix& A, Algorithm algo = Algorithm::Auto, int n_hint = 0);
    ~SpmmPlan();
    SpmmPlan(const SpmmPlan&) = delete;
    SpmmPlan& operator=(const SpmmPlan&) = delete;
    SpmmPlan(SpmmPlan&& other) noexcept;
    SpmmPlan& operator=(SpmmPlan&& other) noexcept;

    // C = alpha * A * B + beta * C; returns after the device has finished,
    // like spmm().
    void run(const DenseMatrix& B, DenseMatrix& C, float alpha, float beta);
    // The same, enqueued on the default stream without waiting.
    void run_async(const DenseMatrix& B, DenseMatrix& C, float alpha, float beta);

    Algorithm algorithm() const;     // the concrete variant the plan runs
    size_t device_bytes() const;     // device memory the plan holds
    int panelized_rows() const;      // rows laid out in column panels

private:
    ::csrspmm_plan_s* plan_ = nullptr;
};

}  // namespace csrspmm
