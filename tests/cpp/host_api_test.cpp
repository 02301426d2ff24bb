// Host-only checks of the drop-in C++ API (include/csrspmm/*.h): no device
// call is made, so this runs on a machine without a GPU.  Driven by
// tests/test_cpp_api.py:
//   host_api_test checks
//   host_api_test dense2csr IN.bin H W TOL OUT_PREFIX
//   host_api_test death-<case>        (expected to exit(1) with a message)
#include <csrspmm/csrspmm.h>
#include <csrspmm/dense_utils.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace csrspmm;

#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      std::fprintf(stderr, "CHECK failed: %s (line %d)\n", #c, __LINE__); \
      return 2;                                                    \
    }                                                              \
  } while (0)

static int checks() {
  CHECK(parse_algorithm("Naive") == Algorithm::Naive);
  CHECK(parse_algorithm("NaiveSmem") == Algorithm::NaiveSmem);
  CHECK(parse_algorithm("WarpPerRow") == Algorithm::WarpPerRow);
  CHECK(parse_algorithm("WarpPerRowFp4") == Algorithm::WarpPerRowFp4);
  CHECK(parse_algorithm("WarpPerRowSmem") == Algorithm::WarpPerRowSmem);
  CHECK(parse_algorithm("WarpPerRowSmemFp4") == Algorithm::WarpPerRowSmemFp4);
  CHECK(parse_algorithm("Auto") == Algorithm::Auto);
  CHECK(static_cast<int>(Algorithm::WarpPerRowSmemFp4) == 5 && static_cast<int>(Algorithm::Auto) == 6);
  CHECK(parse_algorithm("adaptive") == Algorithm::Naive);  // warns on stderr, falls back
  CHECK(WARP_SIZE == 64);

  // dense <-> CSR round trip, max_row_nnz, compression ratio
  DenseMatrix d;
  dense_alloc_host(d, 3, 4);
  const float vals[12] = {0, 1.5f, 0, -2, 0, 0, 0, 0, 3, -0.0f, 4, 5};
  std::memcpy(d.data, vals, sizeof(vals));
  CSRMatrix c;
  dense2csr(d, c);
  CHECK(c.height == 3 && c.width == 4 && c.nnz == 5 && c.max_row_nnz == 3);
  const int rp[4] = {0, 2, 2, 5};
  const int ci[5] = {1, 3, 0, 2, 3};
  CHECK(std::memcmp(c.row_ptr, rp, sizeof(rp)) == 0);
  CHECK(std::memcmp(c.col_idx, ci, sizeof(ci)) == 0);
  CHECK(c.values[0] == 1.5f && c.values[4] == 5.0f);
  CHECK(std::fabs(compression_ratio(c) - 12.0f / 14.0f) < 1e-6f);
  DenseMatrix back;
  csr2dense(c, back);
  CHECK(back.height == 3 && back.width == 4);
  for (int i = 0; i < 12; ++i) CHECK(back.data[i] == (vals[i] == 0 ? 0.0f : vals[i]));
  print_csr(c);
  print_dense(back);

  // dense_compare: absolute tolerance, shape check, NaN is a mismatch
  CHECK(dense_compare(d, back, 0.0f));
  back.data[1] += 1e-3f;
  CHECK(!dense_compare(d, back, 1e-4f));
  CHECK(dense_compare(d, back, 1e-2f));
  back.data[1] = NAN;
  CHECK(!dense_compare(d, back, 1e9f));
  DenseMatrix other;
  dense_alloc_host(other, 4, 3);
  CHECK(!dense_compare(d, other, 1.0f));

  // dense_gemm_cpu on integers is exact: C = 2*A*B - C
  DenseMatrix A, B, C;
  dense_alloc_host(A, 2, 3);
  dense_alloc_host(B, 3, 2);
  dense_alloc_host(C, 2, 2);
  const float a[6] = {1, 2, 3, 4, 5, 6}, b[6] = {1, -1, 2, 0, 0, 3}, c0[4] = {1, 1, 1, 1};
  std::memcpy(A.data, a, sizeof(a));
  std::memcpy(B.data, b, sizeof(b));
  std::memcpy(C.data, c0, sizeof(c0));
  dense_gemm_cpu(2, 3, 2, 2.0f, -1.0f, A, B, C);
  CHECK(C.data[0] == 9 && C.data[1] == 15 && C.data[2] == 27 && C.data[3] == 27);

  // dense_init_random: values in range, requested sparsity, distinct values
  DenseMatrix R;
  dense_alloc_host(R, 100, 100);
  dense_init_random(R, -10.0f, 10.0f, 0.7f, false);
  int zeros = 0;
  for (int i = 0; i < 10000; ++i) {
    CHECK(R.data[i] >= -10.0f && R.data[i] <= 10.0f);
    zeros += R.data[i] == 0.0f;
  }
  CHECK(zeros > 6500 && zeros < 7500);
  CHECK(R.data[1] != R.data[2] || R.data[3] != R.data[4]);
  DenseMatrix R2;
  dense_alloc_host(R2, 100, 100);
  dense_init_random(R2, -10.0f, 10.0f, 0.0f, true);
  for (int i = 0; i < 10000; ++i) CHECK(R2.data[i] == std::trunc(R2.data[i]));

  csr_free_host(c);
  CHECK(c.row_ptr == nullptr && c.nnz == 0 && c.max_row_nnz == 0);
  for (DenseMatrix* m : {&d, &back, &other, &A, &B, &C, &R, &R2}) dense_free_host(*m);
  std::printf("OK\n");
  return 0;
}

static int run_dense2csr(int argc, char** argv) {
  if (argc < 7) return 3;
  const int H = std::atoi(argv[3]), W = std::atoi(argv[4]);
  const float tol = std::atof(argv[5]);
  DenseMatrix d;
  dense_alloc_host(d, H, W);
  FILE* f = std::fopen(argv[2], "rb");
  if (!f || std::fread(d.data, sizeof(float), (size_t)H * W, f) != (size_t)H * W) return 4;
  std::fclose(f);
  CSRMatrix c;
  dense2csr(d, c, tol);
  const std::string pre = argv[6];
  auto dump = [&](const char* suffix, const void* p, size_t bytes) {
    FILE* o = std::fopen((pre + suffix).c_str(), "wb");
    std::fwrite(p, 1, bytes, o);
    std::fclose(o);
  };
  dump(".rowptr", c.row_ptr, sizeof(int) * (H + 1));
  dump(".colidx", c.col_idx, sizeof(int) * c.nnz);
  dump(".vals", c.values, sizeof(float) * c.nnz);
  std::printf("%d %d\n", c.nnz, c.max_row_nnz);
  return 0;
}

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "checks";
  if (mode == "checks") return checks();
  if (mode == "dense2csr") return run_dense2csr(argc, argv);
  CSRMatrix c;
  DenseMatrix d;
  if (mode == "death-csr-alloc-twice") {
    csr_alloc_host(c, 2, 2, 1);
    csr_alloc_host(c, 2, 2, 1);
  } else if (mode == "death-dense2csr-nonempty") {
    dense_alloc_host(d, 2, 2);
    std::memset(d.data, 0, 16);
    csr_alloc_host(c, 2, 2, 1);
    dense2csr(d, c);
  } else if (mode == "death-dense2csr-invalid") {
    dense2csr(d, c);
  } else if (mode == "death-csr2dense-nonempty") {
    csr_alloc_host(c, 2, 2, 1);
    dense_alloc_host(d, 2, 2);
    csr2dense(c, d);
  } else if (mode == "death-dense-alloc-twice") {
    dense_alloc_host(d, 2, 2);
    dense_alloc_host(d, 2, 2);
  } else if (mode == "death-h2d-null-source") {
    CSRMatrix dev;
    csr_host2device(c, dev);
  } else if (mode == "death-dense-h2d-nonnull") {
    DenseMatrix h, dev;
    dense_alloc_host(h, 1, 1);
    dense_alloc_host(dev, 1, 1);  // a non-null destination is rejected before any copy
    dense_host2device(h, dev);
  } else {
    return 5;
  }
  return 0;  // not reached for death cases
}
