// Launches the kernels of <csrspmm/kernels.h> directly, as code written
// against the reference's kernel declarations does (reference
// src/host/spmm_launcher.cu: 32 x 32 threads over a 2-D grid for the naive
// pair; ceil(M / 4) blocks of 4 warps, with 4 * max_row_nnz * 8 bytes of
// dynamic LDS for the smem forms), plus launch shapes the reference never
// uses (one block of 32 threads; 4 waves of 64), and checks every output
// element against an fp64 host product: |C - R| <= 1e-5 * max(|R|, S), S the
// condition magnitude.  Ragged rows (empty, short, one of 3000 nonzeros),
// beta != 0, and K = 64 (float4), 130 and 1 (scalar).  Exit status 0 when
// every case passes.
#include <csrspmm/kernels.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

namespace {

struct Rng {
  uint64_t s;
  uint32_t next() {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return (uint32_t)(s >> 33);
  }
  float u11() { return (float)((next() >> 8) * (1.0 / 8388608.0)) - 1.0f; }
};

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      std::exit(2);                                                               \
    }                                                                             \
  } while (0)

}  // namespace

int main() {
  const int M = 1000, NA = 700;  // A is M x NA (reference naming: N columns)
  Rng rng{2026};
  std::vector<int> rowptr(M + 1, 0), col;
  std::vector<float> val;
  int max_row = 0;
  for (int r = 0; r < M; ++r) {
    int len = (r % 7 == 0) ? 0 : (int)(rng.next() % 40);
    if (r == 500) len = 3000;
    std::vector<int> cs;
    for (int i = 0; i < len; ++i) cs.push_back((int)(rng.next() % NA));
    for (int c : cs) {  // unsorted, duplicates allowed: any CSR the reference accepts
      col.push_back(c);
      val.push_back(rng.u11());
    }
    rowptr[r + 1] = (int)col.size();
    if (len > max_row) max_row = len;
  }
  const int nnz = (int)col.size();
  int *d_rp, *d_ci;
  float *d_va, *d_B, *d_C;
  CHECK(hipMalloc(&d_rp, (M + 1) * sizeof(int)));
  CHECK(hipMalloc(&d_ci, nnz * sizeof(int)));
  CHECK(hipMalloc(&d_va, nnz * sizeof(float)));
  CHECK(hipMemcpy(d_rp, rowptr.data(), (M + 1) * sizeof(int), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(d_ci, col.data(), nnz * sizeof(int), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(d_va, val.data(), nnz * sizeof(float), hipMemcpyHostToDevice));

  int failures = 0;
  const float alpha = 1.25f, beta = 0.5f;
  for (int K : {64, 130, 1}) {
    std::vector<float> B((size_t)NA * K), C0((size_t)M * K);
    for (auto& x : B) x = rng.u11();
    for (auto& x : C0) x = rng.u11();
    std::vector<double> R((size_t)M * K), S((size_t)M * K);
    for (int r = 0; r < M; ++r)
      for (int c = 0; c < K; ++c) {
        double acc = 0.0, mag = 0.0;
        for (int j = rowptr[r]; j < rowptr[r + 1]; ++j) {
          const double p = (double)val[j] * B[(size_t)col[j] * K + c];
          acc += p;
          mag += std::fabs(p);
        }
        const double c0 = C0[(size_t)r * K + c];
        R[(size_t)r * K + c] = alpha * acc + beta * c0;
        S[(size_t)r * K + c] = std::fabs(alpha) * mag + std::fabs(beta * c0);
      }
    CHECK(hipMalloc(&d_B, B.size() * sizeof(float)));
    CHECK(hipMalloc(&d_C, C0.size() * sizeof(float)));
    CHECK(hipMemcpy(d_B, B.data(), B.size() * sizeof(float), hipMemcpyHostToDevice));
    const size_t smem_ref = (size_t)4 * max_row * (sizeof(int) + sizeof(float));
    const int warp_blocks = (M + 3) / 4;
    struct Shape {
      const char* what;
      dim3 grid, block;
      size_t lds;
    };
    const Shape naive_shapes[] = {
        {"reference 32x32", dim3((K + 31) / 32, (M + 31) / 32), dim3(32, 32), 0},
        {"one block of 32", dim3(1), dim3(32), 0}};
    const Shape warp_shapes[] = {
        {"reference 4 warps of 32", dim3(warp_blocks), dim3(128), 0},
        {"4 waves of 64", dim3(warp_blocks), dim3(256), 0},
        {"one block of 32", dim3(1), dim3(32), 0}};
    for (int kind = 0; kind < 6; ++kind) {
      const char* names[] = {"csrspmm_naive", "csrspmm_naive_smem", "csrspmm_warp_per_row",
                             "csrspmm_warp_per_row_fp4", "csrspmm_warp_per_row_smem",
                             "csrspmm_warp_per_row_smem_fp4"};
      const bool naive = kind < 2;
      const int nshapes = naive ? 2 : 3;
      for (int si = 0; si < nshapes; ++si) {
        Shape sh = naive ? naive_shapes[si] : warp_shapes[si];
        // the smem forms get the reference launcher's LDS when it fits a workgroup
        const bool smem = kind >= 4;
        if (smem && si == 0 && smem_ref <= 64 * 1024) sh.lds = smem_ref;
        CHECK(hipMemcpy(d_C, C0.data(), C0.size() * sizeof(float), hipMemcpyHostToDevice));
        switch (kind) {
          case 0: csrspmm::kernel::csrspmm_naive<<<sh.grid, sh.block, sh.lds>>>(M, NA, K, alpha, beta, d_va, d_ci, d_rp, d_B, d_C); break;
          case 1: csrspmm::kernel::csrspmm_naive_smem<<<sh.grid, sh.block, sh.lds>>>(M, NA, K, alpha, beta, d_va, d_ci, d_rp, d_B, d_C); break;
          case 2: csrspmm::kernel::csrspmm_warp_per_row<<<sh.grid, sh.block, sh.lds>>>(M, NA, K, alpha, beta, d_va, d_ci, d_rp, d_B, d_C); break;
          case 3: csrspmm::kernel::csrspmm_warp_per_row_fp4<<<sh.grid, sh.block, sh.lds>>>(M, NA, K, alpha, beta, d_va, d_ci, d_rp, d_B, d_C); break;
          case 4: csrspmm::kernel::csrspmm_warp_per_row_smem<<<sh.grid, sh.block, sh.lds>>>(M, NA, K, alpha, beta, d_va, d_ci, d_rp, max_row, d_B, d_C); break;
          default: csrspmm::kernel::csrspmm_warp_per_row_smem_fp4<<<sh.grid, sh.block, sh.lds>>>(M, NA, K, alpha, beta, d_va, d_ci, d_rp, max_row, d_B, d_C); break;
        }
        CHECK(hipGetLastError());
        CHECK(hipDeviceSynchronize());
        std::vector<float> C(C0.size());
        CHECK(hipMemcpy(C.data(), d_C, C.size() * sizeof(float), hipMemcpyDeviceToHost));
        long long bad = 0;
        double worst = 0.0;
        for (size_t i = 0; i < C.size(); ++i) {
          const double lim = 1e-5 * std::fmax(std::fabs(R[i]), S[i]);
          const double err = std::fabs((double)C[i] - R[i]);
          if (!(err <= lim)) ++bad;
          if (lim > 0) worst = std::fmax(worst, err / lim);
        }
        std::printf("kernels.h %-30s K=%-4d %-24s lds=%-6zu %s (worst %.3f of the bound)\n",
                    names[kind], K, sh.what, sh.lds, bad ? "FAIL" : "ok", worst);
        if (bad) ++failures;
      }
    }
    CHECK(hipFree(d_B));
    CHECK(hipFree(d_C));
  }
  CHECK(hipFree(d_rp));
  CHECK(hipFree(d_ci));
  CHECK(hipFree(d_va));
  std::printf("%s\n", failures ? "FAILED" : "all kernels.h launches passed");
  return failures ? 1 : 0;
}
