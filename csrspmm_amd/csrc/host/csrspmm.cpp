// csrspmm::parse_algorithm and csrspmm::spmm (reference src/csrspmm.cpp:13-75),
// implemented over the C ABI.
#include <csrspmm/csrspmm.h>
#include <csrspmm/error_check.h>
#include <csrspmm/spmm_launcher.cuh>

#include <iostream>

namespace csrspmm {

Algorithm parse_algorithm(const std::string& name) {
    const int id = csrspmm_parse_algorithm(name.c_str());
    if (id >= 0) return static_cast<Algorithm>(id);
    std::cerr << "[csrspmm] Unknown algorithm: " << name << ", using Naive\n";
    return Algorithm::Naive;
}

void spmm(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C, float alpha, float beta,
          Algorithm algo) {
    // The reference's "auto-selection" maps Naive to Naive in both branches
    // (src/csrspmm.cpp:34-40); the requested variant is used as given.
    switch (algo) {
        case Algorithm::Naive: launch_naive(A, B, C, alpha, beta); break;
        case Algorithm::NaiveSmem: launch_naive_smem(A, B, C, alpha, beta); break;
        case Algorithm::WarpPerRow: launch_warp_per_row(A, B, C, alpha, beta); break;
        case Algorithm::WarpPerRowFp4: launch_warp_per_row_fp4(A, B, C, alpha, beta); break;
        case Algorithm::WarpPerRowSmem: launch_warp_per_row_smem(A, B, C, alpha, beta); break;
        case Algorithm::WarpPerRowSmemFp4: launch_warp_per_row_smem_fp4(A, B, C, alpha, beta); break;
        case Algorithm::Auto:
            csrspmmCheck(csrspmm_spmm_f32(CSRSPMM_ALGO_AUTO, A.height, A.width, B.width, A.nnz,
                                          A.row_ptr, A.col_idx, A.values,
                                          A.max_row_nnz > 0 ? A.max_row_nnz : -1, B.data, B.width,
                                          C.data, C.width, alpha, beta, nullptr));
            break;
        default:
            std::printf("[csrspmm::spmm] Invalid Algorithm.\n");
            return;
    }
    csrspmmCheck(csrspmm_get_last_error());
    csrspmmCheck(csrspmm_device_synchronize());
}

SpmmPlan::SpmmPlan(const CSRMatrix& A, Algorithm algo, int n_hint) {
    csrspmmCheck(csrspmm_plan_create(static_cast<int>(algo), A.height, A.width, A.nnz, A.row_ptr,
                                     A.col_idx, A.values, n_hint, nullptr, &plan_));
}

SpmmPlan::~SpmmPlan() {
    if (plan_) (void)csrspmm_plan_destroy(plan_);
}

SpmmPlan::SpmmPlan(SpmmPlan&& other) noexcept : plan_(other.plan_) { other.plan_ = nullptr; }

SpmmPlan& SpmmPlan::operator=(SpmmPlan&& other) noexcept {
    if (this != &other) {
        if (plan_) (void)csrspmm_plan_destroy(plan_);
        plan_ = other.plan_;
        other.plan_ = nullptr;
    }
    return *this;
}

void SpmmPlan::run_async(const DenseMatrix& B, DenseMatrix& C, float alpha, float beta) {
    csrspmmCheck(csrspmm_plan_spmm_f32(plan_, B.width, B.data, B.width, C.data, C.width, alpha, beta,
                                       0u, nullptr));
}

void SpmmPlan::run(const DenseMatrix& B, DenseMatrix& C, float alpha, float beta) {
    run_async(B, C, alpha, beta);
    csrspmmCheck(csrspmm_device_synchronize());
}

Algorithm SpmmPlan::algorithm() const { return static_cast<Algorithm>(csrspmm_plan_algorithm(plan_)); }

size_t SpmmPlan::device_bytes() const { return csrspmm_plan_device_bytes(plan_); }

int SpmmPlan::panelized_rows() const { return csrspmm_plan_panelized_rows(plan_); }

}  // namespace csrspmm
