// torch_csrspmm._C for PyTorch-ROCm: the five forwards of the reference's
// torch extension (torch_csrspmm/binding.cpp:26-32 and
// torch_csrspmm/torch_csrspmm_{naive,warp_per_row,warp_per_row_fp4,
// warp_per_row_smem,warp_per_row_smem_fp4}.cpp), over the C ABI.
//
// Kept from the reference: argument order, the is_cuda / dtype checks and
// messages, M = rowptr.size(0) - 1, K = B.size(0), N = B.size(1), a new
// [M, N] output with B's options, and the result of its C = beta == 0 ?
// empty : zeros allocation (beta then scales an all-zero C, so the result is
// alpha*A*B, with beta's NaN/Inf still propagating through beta*0).
// Changed: the zero C is never materialised (CSRSPMM_FLAG_C_IS_ZERO), the
// launch goes on the current HIP stream of B's device instead of the legacy
// default stream, shapes / contiguity are checked, and a failed launch raises.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "csrspmm_c.h"

using torch::Tensor;

namespace {

void check_inputs(const Tensor& rowptr, const Tensor& colidx, const Tensor& vals, const Tensor& B) {
  TORCH_CHECK(rowptr.is_cuda(), "A_row_ptr must be a CUDA tensor");
  TORCH_CHECK(colidx.is_cuda(), "A_col_idx must be a CUDA tensor");
  TORCH_CHECK(vals.is_cuda(), "A_values must be a CUDA tensor");
  TORCH_CHECK(B.is_cuda(), "B must be a CUDA tensor");

  TORCH_CHECK(rowptr.dtype() == torch::kInt32, "A_row_ptr must be int32");
  TORCH_CHECK(colidx.dtype() == torch::kInt32, "A_col_idx must be int32");
  TORCH_CHECK(vals.dtype() == torch::kFloat32, "A_values must be float32");
  TORCH_CHECK(B.dtype() == torch::kFloat32, "B must be float32");

  TORCH_CHECK(rowptr.dim() == 1 && rowptr.size(0) >= 1, "A_row_ptr must be 1-D with M+1 >= 1 entries");
  TORCH_CHECK(colidx.dim() == 1 && vals.dim() == 1, "A_col_idx and A_values must be 1-D");
  TORCH_CHECK(colidx.size(0) == vals.size(0), "A_col_idx and A_values must have nnz entries each");
  TORCH_CHECK(B.dim() == 2, "B must be 2-D [K, N]");
  TORCH_CHECK(rowptr.is_contiguous() && colidx.is_contiguous() && vals.is_contiguous(),
              "CSR arrays must be contiguous");
  TORCH_CHECK(B.size(1) <= 1 || B.stride(1) == 1, "B must be row-major (stride(1) == 1)");
  TORCH_CHECK(rowptr.device() == B.device() && colidx.device() == B.device() &&
                  vals.device() == B.device(),
              "all tensors must be on the same device");
  TORCH_CHECK(rowptr.size(0) - 1 <= INT32_MAX && vals.size(0) <= INT32_MAX &&
                  B.size(0) <= INT32_MAX && B.size(1) <= INT32_MAX,
              "sizes must fit int32");
}

Tensor forward(int algo, const Tensor& rowptr, const Tensor& colidx, const Tensor& vals, int hint,
               const Tensor& B, double alpha_d, double beta_d) {
  check_inputs(rowptr, colidx, vals, B);
  // The reference binds alpha and beta as C++ float.
  const float alpha = static_cast<float>(alpha_d);
  const float beta = static_cast<float>(beta_d);
  c10::DeviceGuard guard(B.device());

  const int M = static_cast<int>(rowptr.size(0) - 1);
  const int K = static_cast<int>(B.size(0));
  const int N = static_cast<int>(B.size(1));
  const int nnz = static_cast<int>(vals.size(0));
  Tensor C = torch::empty({M, N}, B.options());
  if (M == 0 || N == 0) return C;

  const long long ldb = B.size(1) <= 1 ? std::max<long long>(N, 1) : B.stride(0);
  const size_t ws_bytes = csrspmm_workspace_bytes(algo, M, N, nnz);
  Tensor ws;
  void* ws_ptr = nullptr;
  if (ws_bytes > 0) {
    ws = torch::empty({static_cast<int64_t>(ws_bytes)}, B.options().dtype(torch::kUInt8));
    ws_ptr = ws.data_ptr();
  }
  const unsigned flags = beta != 0.0f ? CSRSPMM_FLAG_C_IS_ZERO : 0u;
  hipStream_t stream = c10::hip::getCurrentHIPStream(B.device().index()).stream();
  const int st = csrspmm_spmm_f32_ex(algo, M, K, N, nnz, rowptr.data_ptr<int>(),
                                     nnz ? colidx.data_ptr<int>() : nullptr,
                                     nnz ? vals.data_ptr<float>() : nullptr, hint,
                                     B.numel() ? B.data_ptr<float>() : nullptr, ldb,
                                     C.data_ptr<float>(), N, alpha, beta, flags, ws_ptr, ws_bytes,
                                     static_cast<void*>(stream));
  TORCH_CHECK(st == 0, "csrspmm ", csrspmm_algorithm_name(algo), " failed: ",
              csrspmm_status_string(st));
  return C;
}

Tensor csrspmm_naive_forward(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values, Tensor B,
                             double alpha, double beta) {
  return forward(CSRSPMM_ALGO_NAIVE, A_row_ptr, A_col_idx, A_values, -1, B, alpha, beta);
}

Tensor csrspmm_warp_per_row_forward(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values, Tensor B,
                                    double alpha, double beta) {
  return forward(CSRSPMM_ALGO_WARP_PER_ROW, A_row_ptr, A_col_idx, A_values, -1, B, alpha, beta);
}

Tensor csrspmm_warp_per_row_fp4_forward(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values,
                                        Tensor B, double alpha, double beta) {
  return forward(CSRSPMM_ALGO_WARP_PER_ROW_FP4, A_row_ptr, A_col_idx, A_values, -1, B, alpha, beta);
}

Tensor csrspmm_warp_per_row_smem_forward(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values,
                                         int64_t A_max_row_nnz, Tensor B, double alpha,
                                         double beta) {
  return forward(CSRSPMM_ALGO_WARP_PER_ROW_SMEM, A_row_ptr, A_col_idx, A_values,
                 static_cast<int>(std::min<int64_t>(A_max_row_nnz, INT32_MAX)), B, alpha, beta);
}

Tensor csrspmm_warp_per_row_smem_fp4_forward(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values,
                                             int64_t A_max_row_nnz, Tensor B, double alpha,
                                             double beta) {
  return forward(CSRSPMM_ALGO_WARP_PER_ROW_SMEM_FP4, A_row_ptr, A_col_idx, A_values,
                 static_cast<int>(std::min<int64_t>(A_max_row_nnz, INT32_MAX)), B, alpha, beta);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("csrspmm_naive", &csrspmm_naive_forward, "CSR SpMM (naive)");
  m.def("csrspmm_warp_per_row", &csrspmm_warp_per_row_forward, "CSR SpMM (warp_per_row)");
  m.def("csrspmm_warp_per_row_smem", &csrspmm_warp_per_row_smem_forward,
        "CSR SpMM (warp_per_row_smem)");
  m.def("csrspmm_warp_per_row_fp4", &csrspmm_warp_per_row_fp4_forward, "CSR SpMM (warp_per_row_fp4)");
  m.def("csrspmm_warp_per_row_smem_fp4", &csrspmm_warp_per_row_smem_fp4_forward,
        "CSR SpMM (warp_per_row_smem_fp4)");
}
