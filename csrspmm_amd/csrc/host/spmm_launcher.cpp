// launch_<variant> (reference src/host/spmm_launcher.cu:11-171): shape
// bookkeeping from the POD handles, then one C-ABI call on the default
// stream.  Grid, block and LDS sizing live with the kernels.
#include <csrspmm/error_check.h>
#include <csrspmm/spmm_launcher.cuh>

namespace csrspmm {

namespace {

void launch(int algo, const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C, float alpha,
            float beta) {
    // Shapes follow the reference launchers: M = A.height, K = A.width = B.height,
    // N = B.width; C is M x N with leading dimension C.width.
    const int hint = A.max_row_nnz > 0 ? A.max_row_nnz : -1;
    csrspmmCheck(csrspmm_spmm_f32(algo, A.height, A.width, B.width, A.nnz, A.row_ptr, A.col_idx,
                                  A.values, hint, B.data, B.width, C.data, C.width, alpha, beta,
                                  nullptr));
}

}  // namespace

void launch_naive(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C, float alpha, float beta) {
    launch(CSRSPMM_ALGO_NAIVE, A, B, C, alpha, beta);
}
void launch_naive_smem(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C, float alpha,
                       float beta) {
    launch(CSRSPMM_ALGO_NAIVE_SMEM, A, B, C, alpha, beta);
}
void launch_warp_per_row(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C, float alpha,
                         float beta) {
    launch(CSRSPMM_ALGO_WARP_PER_ROW, A, B, C, alpha, beta);
}
void launch_warp_per_row_fp4(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C, float alpha,
                             float beta) {
    launch(CSRSPMM_ALGO_WARP_PER_ROW_FP4, A, B, C, alpha, beta);
}
void launch_warp_per_row_smem(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C, float alpha,
                              float beta) {
    launch(CSRSPMM_ALGO_WARP_PER_ROW_SMEM, A, B, C, alpha, beta);
}
void launch_warp_per_row_smem_fp4(const CSRMatrix& A, const DenseMatrix& B, DenseMatrix& C,
                                  float alpha, float beta) {
    launch(CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4, A, B, C, alpha, beta);
}

}  // namespace csrspmm
