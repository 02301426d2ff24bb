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

#include <vector>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "csrspmm_c.h"

using torch::Tensor;

namespace {

// Row stride of a 2-D row-major operand X (B, C or a dense input): stride(0)
// whenever X has more than one row, whatever its width, so a one-column view
// such as X[:, k:k+1] of a wider tensor is addressed through its parent's
// rows; max(width, 1) for a single row (or none) or no columns, where
// stride(0) addresses nothing.  A row stride below the width (overlapping or
// broadcast rows) is rejected.
long long leading_dim(const Tensor& X, const char* name) {
  if (X.size(0) <= 1 || X.size(1) == 0) return std::max<int64_t>(X.size(1), 1);
  TORCH_CHECK(X.size(1) <= 1 || X.stride(1) == 1, name, " must be row-major (stride(1) == 1)");
  TORCH_CHECK(X.stride(0) >= std::max<int64_t>(X.size(1), 1), name,
              " must have a row stride (stride(0)) of at least its width");
  return X.stride(0);
}

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

  const long long ldb = leading_dim(B, "B");
  const size_t ws_bytes = csrspmm_workspace_bytes_ex(algo, M, K, N, nnz, hint);
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

// max_row_nnz: the longest row, or -1 when unknown (a scheduling hint only).
int row_hint(int64_t max_row_nnz) {
  return max_row_nnz < 0 ? -1 : static_cast<int>(std::min<int64_t>(max_row_nnz, INT32_MAX));
}

Tensor csrspmm_auto_forward(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values, Tensor B,
                            double alpha, double beta, int64_t max_row_nnz) {
  return forward(CSRSPMM_ALGO_AUTO, A_row_ptr, A_col_idx, A_values, row_hint(max_row_nnz), B, alpha,
                 beta);
}

int algo_id(const std::string& name) {
  const int a = csrspmm_parse_algorithm(name.c_str());
  TORCH_CHECK(a >= 0, "unknown algorithm '", name, "'");
  return a;
}

void check_out(const Tensor& C, const Tensor& B, int64_t M) {
  TORCH_CHECK(C.is_cuda() && C.device() == B.device(), "C must be a CUDA tensor on B's device");
  TORCH_CHECK(C.dtype() == torch::kFloat32, "C must be float32");
  TORCH_CHECK(C.dim() == 2 && C.size(0) == M && C.size(1) == B.size(1), "C must be [M, N]");
  TORCH_CHECK(C.size(1) <= 1 || C.stride(1) == 1, "C must be row-major (stride(1) == 1)");
}

// C = alpha * A * B + beta * C in place, with the prior C read when beta != 0
// (the reference's C++ spmm() semantics, src/csrspmm.cpp:28-75; its torch
// forwards always start from a fresh C).
Tensor csrspmm_spmm_out(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values, Tensor B, Tensor C,
                        double alpha_d, double beta_d, const std::string& algo, int64_t max_row_nnz) {
  check_inputs(A_row_ptr, A_col_idx, A_values, B);
  const int M = static_cast<int>(A_row_ptr.size(0) - 1);
  check_out(C, B, M);
  c10::DeviceGuard guard(B.device());
  const int K = static_cast<int>(B.size(0)), N = static_cast<int>(B.size(1));
  const int nnz = static_cast<int>(A_values.size(0));
  if (M == 0 || N == 0) return C;
  const int a = algo_id(algo);
  const int hint = row_hint(max_row_nnz);
  const size_t ws_bytes = csrspmm_workspace_bytes_ex(a, M, K, N, nnz, hint);
  Tensor ws;
  if (ws_bytes > 0) ws = torch::empty({static_cast<int64_t>(ws_bytes)}, B.options().dtype(torch::kUInt8));
  hipStream_t stream = c10::hip::getCurrentHIPStream(B.device().index()).stream();
  const int st = csrspmm_spmm_f32_ex(a, M, K, N, nnz, A_row_ptr.data_ptr<int>(),
                                     nnz ? A_col_idx.data_ptr<int>() : nullptr,
                                     nnz ? A_values.data_ptr<float>() : nullptr, hint,
                                     B.numel() ? B.data_ptr<float>() : nullptr, leading_dim(B, "B"),
                                     C.data_ptr<float>(), leading_dim(C, "C"), static_cast<float>(alpha_d),
                                     static_cast<float>(beta_d), 0u,
                                     ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream);
  TORCH_CHECK(st == 0, "csrspmm_spmm_out failed: ", csrspmm_status_string(st));
  return C;
}

// A stored plan (csrspmm_plan_*) for one CSR matrix; holds references to the
// CSR tensors, which the plan reads in place.
class CsrSpmmPlan {
 public:
  CsrSpmmPlan(Tensor rowptr, Tensor colidx, Tensor vals, int64_t K, const std::string& algo,
              int64_t n_hint)
      : rowptr_(rowptr), colidx_(colidx), vals_(vals), K_(K) {
    TORCH_CHECK(rowptr.is_cuda() && colidx.is_cuda() && vals.is_cuda(),
                "CSR tensors must be CUDA tensors");
    TORCH_CHECK(rowptr.dtype() == torch::kInt32, "A_row_ptr must be int32");
    TORCH_CHECK(colidx.dtype() == torch::kInt32, "A_col_idx must be int32");
    TORCH_CHECK(vals.dtype() == torch::kFloat32, "A_values must be float32");
    TORCH_CHECK(rowptr.dim() == 1 && rowptr.size(0) >= 1 && colidx.dim() == 1 && vals.dim() == 1 &&
                    colidx.size(0) == vals.size(0),
                "bad CSR shapes");
    TORCH_CHECK(rowptr.is_contiguous() && colidx.is_contiguous() && vals.is_contiguous(),
                "CSR arrays must be contiguous");
    TORCH_CHECK(K >= 0 && K <= INT32_MAX && vals.size(0) <= INT32_MAX, "sizes must fit int32");
    c10::DeviceGuard guard(rowptr.device());
    const int nnz = static_cast<int>(vals.size(0));
    hipStream_t stream = c10::hip::getCurrentHIPStream(rowptr.device().index()).stream();
    const int st = csrspmm_plan_create(algo_id(algo), static_cast<int>(rowptr.size(0) - 1),
                                       static_cast<int>(K), nnz, rowptr.data_ptr<int>(),
                                       nnz ? colidx.data_ptr<int>() : nullptr,
                                       nnz ? vals.data_ptr<float>() : nullptr,
                                       static_cast<int>(n_hint), stream, &plan_);
    TORCH_CHECK(st == 0, "csrspmm_plan_create failed: ", csrspmm_status_string(st));
  }
  ~CsrSpmmPlan() {
    if (plan_) (void)csrspmm_plan_destroy(plan_);
  }
  CsrSpmmPlan(const CsrSpmmPlan&) = delete;
  CsrSpmmPlan& operator=(const CsrSpmmPlan&) = delete;

  // New [M, N] output, the reference forwards' semantics (beta scales zero).
  Tensor spmm(Tensor B, double alpha, double beta) {
    check_b(B);
    Tensor C = torch::empty({rowptr_.size(0) - 1, B.size(1)}, B.options());
    run(B, C, alpha, beta, beta != 0.0 ? CSRSPMM_FLAG_C_IS_ZERO : 0u);
    return C;
  }
  // In place: C = alpha * A * B + beta * C.
  Tensor spmm_out(Tensor B, Tensor C, double alpha, double beta) {
    check_b(B);
    check_out(C, B, rowptr_.size(0) - 1);
    run(B, C, alpha, beta, 0u);
    return C;
  }
  std::string algorithm() const { return csrspmm_algorithm_name(csrspmm_plan_algorithm(plan_)); }
  int64_t device_bytes() const { return static_cast<int64_t>(csrspmm_plan_device_bytes(plan_)); }
  int64_t panelized_rows() const { return csrspmm_plan_panelized_rows(plan_); }

 private:
  void check_b(const Tensor& B) const {
    TORCH_CHECK(B.is_cuda() && B.device() == rowptr_.device(), "B must be a CUDA tensor on A's device");
    TORCH_CHECK(B.dtype() == torch::kFloat32, "B must be float32");
    TORCH_CHECK(B.dim() == 2 && B.size(0) == K_, "B must be [K, N]");
    TORCH_CHECK(B.size(1) <= 1 || B.stride(1) == 1, "B must be row-major (stride(1) == 1)");
  }
  void run(const Tensor& B, Tensor& C, double alpha, double beta, unsigned flags) {
    c10::DeviceGuard guard(B.device());
    if (C.numel() == 0) return;
    hipStream_t stream = c10::hip::getCurrentHIPStream(B.device().index()).stream();
    const int st = csrspmm_plan_spmm_f32(plan_, static_cast<int>(B.size(1)),
                                         B.numel() ? B.data_ptr<float>() : nullptr, leading_dim(B, "B"),
                                         C.data_ptr<float>(), leading_dim(C, "C"), static_cast<float>(alpha),
                                         static_cast<float>(beta), flags, stream);
    TORCH_CHECK(st == 0, "csrspmm plan spmm failed: ", csrspmm_status_string(st));
  }
  Tensor rowptr_, colidx_, vals_;
  int64_t K_;
  csrspmm_plan_t plan_ = nullptr;
};

// The forwards' semantics (new C, beta scaling zero) for a named variant.
Tensor csrspmm_forward_named(Tensor A_row_ptr, Tensor A_col_idx, Tensor A_values, Tensor B,
                             double alpha, double beta, const std::string& algo) {
  return forward(algo_id(algo), A_row_ptr, A_col_idx, A_values, -1, B, alpha, beta);
}

hipStream_t stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Device dense -> CSR: (rowptr, colidx, values).  One host sync, to size
// colidx/values from the count.
std::vector<Tensor> dense_to_csr(Tensor D, double tol) {
  TORCH_CHECK(D.is_cuda(), "dense must be a CUDA tensor");
  TORCH_CHECK(D.dtype() == torch::kFloat32, "dense must be float32");
  TORCH_CHECK(D.dim() == 2, "dense must be 2-D");
  TORCH_CHECK(D.size(1) <= 1 || D.stride(1) == 1, "dense must be row-major (stride(1) == 1)");
  TORCH_CHECK(D.size(0) < INT32_MAX && D.size(1) <= INT32_MAX, "sizes must fit int32");
  c10::DeviceGuard guard(D.device());
  const int M = static_cast<int>(D.size(0)), K = static_cast<int>(D.size(1));
  const long long ld = leading_dim(D, "dense");
  Tensor rowptr = torch::empty({M + 1}, D.options().dtype(torch::kInt32));
  Tensor nnz = torch::empty({1}, D.options().dtype(torch::kInt64));
  hipStream_t s = stream_of(D);
  const float* d = D.numel() ? D.data_ptr<float>() : nullptr;
  int st = csrspmm_dense2csr_count_f32(M, K, d, ld, static_cast<float>(tol), rowptr.data_ptr<int>(),
                                       reinterpret_cast<long long*>(nnz.data_ptr<int64_t>()), s);
  TORCH_CHECK(st == 0, "dense_to_csr failed: ", csrspmm_status_string(st));
  const int64_t n = nnz.item<int64_t>();
  TORCH_CHECK(n <= INT32_MAX, "dense_to_csr: ", n, " nonzeros exceed int32");
  Tensor colidx = torch::empty({n}, D.options().dtype(torch::kInt32));
  Tensor vals = torch::empty({n}, D.options());
  st = csrspmm_dense2csr_fill_f32(M, K, d, ld, static_cast<float>(tol), rowptr.data_ptr<int>(),
                                  n ? colidx.data_ptr<int>() : nullptr,
                                  n ? vals.data_ptr<float>() : nullptr, s);
  TORCH_CHECK(st == 0, "dense_to_csr failed: ", csrspmm_status_string(st));
  return {rowptr, colidx, vals};
}

// Longest row as a one-element int32 CUDA tensor, with no host sync.
Tensor csr_max_row_nnz(Tensor rowptr) {
  TORCH_CHECK(rowptr.is_cuda() && rowptr.dtype() == torch::kInt32 && rowptr.dim() == 1 &&
                  rowptr.size(0) >= 1 && rowptr.is_contiguous(),
              "rowptr must be a contiguous 1-D int32 CUDA tensor");
  c10::DeviceGuard guard(rowptr.device());
  Tensor out = torch::empty({1}, rowptr.options());
  const int st = csrspmm_csr_max_row_nnz(static_cast<int>(rowptr.size(0) - 1),
                                         rowptr.data_ptr<int>(), out.data_ptr<int>(),
                                         stream_of(rowptr));
  TORCH_CHECK(st == 0, "csr_max_row_nnz failed: ", csrspmm_status_string(st));
  return out;
}

// int64 -> int32 CSR indices on the device; int32 input is returned as is.
// Values beyond int32 are not checked here (no sync); callers that know
// nnz and K fit int32 need no check for a valid CSR.
Tensor indices_to_int32(Tensor idx) {
  TORCH_CHECK(idx.is_cuda() && idx.dim() == 1, "indices must be a 1-D CUDA tensor");
  if (idx.dtype() == torch::kInt32) return idx.contiguous();
  TORCH_CHECK(idx.dtype() == torch::kInt64, "indices must be int32 or int64");
  c10::DeviceGuard guard(idx.device());
  Tensor src = idx.contiguous();
  Tensor dst = torch::empty({src.size(0)}, src.options().dtype(torch::kInt32));
  const int st = csrspmm_indices_i64_to_i32(
      reinterpret_cast<const long long*>(src.numel() ? src.data_ptr<int64_t>() : nullptr),
      src.numel() ? dst.data_ptr<int>() : nullptr, src.numel(), nullptr, stream_of(src));
  TORCH_CHECK(st == 0, "indices_to_int32 failed: ", csrspmm_status_string(st));
  return dst;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("csrspmm_forward", &csrspmm_forward_named, "CSR SpMM by variant name (new C)");
  m.def("dense_to_csr", &dense_to_csr, "device dense -> CSR (rowptr, colidx, values)");
  m.def("csr_max_row_nnz", &csr_max_row_nnz, "longest row, on the device");
  m.def("indices_to_int32", &indices_to_int32, "int64 -> int32 CSR indices, on the device");
  m.def("csrspmm_auto", &csrspmm_auto_forward, "CSR SpMM (variant picked from the shape)");
  m.def("csrspmm_spmm_out", &csrspmm_spmm_out, "CSR SpMM into C in place (C = alpha*A*B + beta*C)");
  pybind11::class_<CsrSpmmPlan>(m, "CsrSpmmPlan")
      .def(pybind11::init<Tensor, Tensor, Tensor, int64_t, const std::string&, int64_t>())
      .def("spmm", &CsrSpmmPlan::spmm)
      .def("spmm_out", &CsrSpmmPlan::spmm_out)
      .def_property_readonly("algorithm", &CsrSpmmPlan::algorithm)
      .def_property_readonly("device_bytes", &CsrSpmmPlan::device_bytes)
      .def_property_readonly("panelized_rows", &CsrSpmmPlan::panelized_rows);
  m.def("csrspmm_naive", &csrspmm_naive_forward, "CSR SpMM (naive)");
  m.def("csrspmm_warp_per_row", &csrspmm_warp_per_row_forward, "CSR SpMM (warp_per_row)");
  m.def("csrspmm_warp_per_row_smem", &csrspmm_warp_per_row_smem_forward,
        "CSR SpMM (warp_per_row_smem)");
  m.def("csrspmm_warp_per_row_fp4", &csrspmm_warp_per_row_fp4_forward, "CSR SpMM (warp_per_row_fp4)");
  m.def("csrspmm_warp_per_row_smem_fp4", &csrspmm_warp_per_row_smem_fp4_forward,
        "CSR SpMM (warp_per_row_smem_fp4)");
}
