// CSR helpers (reference src/host/csr_utils.cpp:13-238).  Same contracts and
// exit(1)-on-error convention; sizes are computed in size_t (the reference's
// int products overflow for large shapes, csr_utils.cpp:175-176).
#include <csrspmm/csr_utils.h>
#include <csrspmm/error_check.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <iostream>

namespace csrspmm {

namespace {
[[noreturn]] void die(const char* msg) {
    std::cerr << msg << "\n";
    std::exit(1);
}
}  // namespace

void csr_alloc_host(CSRMatrix& csr, int height, int width, int nnz) {
    if (csr.row_ptr || csr.col_idx || csr.values)
        die("csr_alloc_host error: already allocated host memory.");
    if (height < 0 || width < 0 || nnz < 0) die("csr_alloc_host: negative size");
    csr.height = height;
    csr.width = width;
    csr.nnz = nnz;
    // malloc(0) may return NULL; allocate at least one element per array.
    csr.row_ptr = static_cast<int*>(std::malloc(((size_t)height + 1) * sizeof(int)));
    csr.col_idx = static_cast<int*>(std::malloc(std::max<size_t>(nnz, 1) * sizeof(int)));
    csr.values = static_cast<float*>(std::malloc(std::max<size_t>(nnz, 1) * sizeof(float)));
    if (!csr.row_ptr || !csr.col_idx || !csr.values) die("csr_alloc_host: malloc failed");
}

void csr_free_host(CSRMatrix& csr) {
    std::free(csr.row_ptr);
    std::free(csr.col_idx);
    std::free(csr.values);
    csr.row_ptr = nullptr;
    csr.col_idx = nullptr;
    csr.values = nullptr;
    csr.height = csr.width = csr.nnz = csr.max_row_nnz = 0;
}

void csr_alloc_device(CSRMatrix& csr, int height, int width, int nnz) {
    if (csr.row_ptr || csr.col_idx || csr.values)
        die("csr_alloc_device error: already allocated device memory.");
    if (height < 0 || width < 0 || nnz < 0) die("csr_alloc_device: negative size");
    csr.height = height;
    csr.width = width;
    csr.nnz = nnz;
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&csr.row_ptr),
                                       ((size_t)height + 1) * sizeof(int)));
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&csr.col_idx),
                                       std::max<size_t>(nnz, 1) * sizeof(int)));
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&csr.values),
                                       std::max<size_t>(nnz, 1) * sizeof(float)));
}

void csr_free_device(CSRMatrix& csr) {
    if (csr.row_ptr) csrspmmCheck(csrspmm_device_free(csr.row_ptr));
    if (csr.col_idx) csrspmmCheck(csrspmm_device_free(csr.col_idx));
    if (csr.values) csrspmmCheck(csrspmm_device_free(csr.values));
    csr.row_ptr = nullptr;
    csr.col_idx = nullptr;
    csr.values = nullptr;
    csr.height = csr.width = csr.nnz = csr.max_row_nnz = 0;
}

void dense2csr(const DenseMatrix& dense, CSRMatrix& csr, float tol) {
    if (!dense.data || dense.height <= 0 || dense.width <= 0) die("dense2csr: invalid dense matrix");
    if (csr.row_ptr || csr.col_idx || csr.values) die("dense2csr error: destination must be null.");
    const int H = dense.height, W = dense.width;
    const size_t total = (size_t)H * (size_t)W;
    // The keep rule is fabs(v) > tol, which drops +-0 and NaN
    // (reference csr_utils.cpp:87,97).
    size_t count = 0;
    for (size_t i = 0; i < total; ++i)
        if (std::fabs(dense.data[i]) > tol) ++count;
    if (count > 0x7fffffffULL) die("dense2csr: nnz exceeds int32");
    csr_alloc_host(csr, H, W, (int)count);
    int idx = 0;
    int mx = 0;
    csr.row_ptr[0] = 0;
    for (int i = 0; i < H; ++i) {
        const float* row = dense.data + (size_t)i * W;
        for (int j = 0; j < W; ++j) {
            if (std::fabs(row[j]) > tol) {
                csr.col_idx[idx] = j;
                csr.values[idx] = row[j];
                ++idx;
            }
        }
        csr.row_ptr[i + 1] = idx;
        mx = std::max(mx, csr.row_ptr[i + 1] - csr.row_ptr[i]);
    }
    csr.max_row_nnz = mx;
}

void dense2csr_device(const DenseMatrix& d_dense, CSRMatrix& d_csr, float tol) {
    if (!d_dense.data || d_dense.height <= 0 || d_dense.width <= 0)
        die("dense2csr_device: invalid dense matrix");
    if (d_csr.row_ptr || d_csr.col_idx || d_csr.values)
        die("dense2csr_device error: destination must be null.");
    const int H = d_dense.height, W = d_dense.width;
    int* rowptr = nullptr;
    long long* d_nnz = nullptr;
    int* d_max = nullptr;
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&rowptr), ((size_t)H + 1) * sizeof(int)));
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&d_nnz), sizeof(long long)));
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&d_max), sizeof(int)));
    csrspmmCheck(csrspmm_dense2csr_count_f32(H, W, d_dense.data, W, tol, rowptr, d_nnz, nullptr));
    long long nnz = 0;
    csrspmmCheck(csrspmm_memcpy_d2h(&nnz, d_nnz, sizeof(nnz)));
    if (nnz > 0x7fffffffLL) die("dense2csr_device: nnz exceeds int32");
    d_csr.height = H;
    d_csr.width = W;
    d_csr.nnz = (int)nnz;
    d_csr.row_ptr = rowptr;
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&d_csr.col_idx),
                                       std::max<size_t>((size_t)nnz, 1) * sizeof(int)));
    csrspmmCheck(csrspmm_device_malloc(reinterpret_cast<void**>(&d_csr.values),
                                       std::max<size_t>((size_t)nnz, 1) * sizeof(float)));
    csrspmmCheck(csrspmm_dense2csr_fill_f32(H, W, d_dense.data, W, tol, rowptr, d_csr.col_idx,
                                            d_csr.values, nullptr));
    csrspmmCheck(csrspmm_csr_max_row_nnz(H, rowptr, d_max, nullptr));
    csrspmmCheck(csrspmm_memcpy_d2h(&d_csr.max_row_nnz, d_max, sizeof(int)));
    csrspmmCheck(csrspmm_device_free(d_nnz));
    csrspmmCheck(csrspmm_device_free(d_max));
}

void csr2dense(const CSRMatrix& csr, DenseMatrix& dense) {
    if (!csr.row_ptr || !csr.col_idx || !csr.values || csr.height <= 0 || csr.width <= 0)
        die("csr2dense: invalid csr");
    if (dense.data != nullptr) die("csr2dense error: destination must be null.");
    const size_t bytes = (size_t)csr.height * (size_t)csr.width * sizeof(float);
    dense.data = static_cast<float*>(std::malloc(bytes));
    if (!dense.data) die("csr2dense: malloc failed");
    dense.height = csr.height;
    dense.width = csr.width;
    std::memset(dense.data, 0, bytes);
    // Later duplicates of a column overwrite earlier ones, as in the reference.
    for (int i = 0; i < csr.height; ++i)
        for (int p = csr.row_ptr[i]; p < csr.row_ptr[i + 1]; ++p)
            dense.data[(size_t)i * csr.width + csr.col_idx[p]] = csr.values[p];
}

void print_csr(const CSRMatrix& csr) {
    std::cout << "CSRMatrix (HOST): " << csr.height << "x" << csr.width << ", nnz=" << csr.nnz
              << ", max_row_nnz=" << csr.max_row_nnz << "\n";
    std::cout << "row_ptr: [ ";
    for (int i = 0; i <= csr.height; i++) std::cout << csr.row_ptr[i] << " ";
    std::cout << "]\ncol_idx: [ ";
    for (int i = 0; i < csr.nnz; i++) std::cout << csr.col_idx[i] << " ";
    std::cout << "]\nvalues:  [ ";
    for (int i = 0; i < csr.nnz; i++) std::cout << csr.values[i] << " ";
    std::cout << "]\n";
}

float compression_ratio(const CSRMatrix& csr) {
    const double dense = (double)csr.height * (double)csr.width;
    const double sparse = 2.0 * (double)csr.nnz + (double)csr.height + 1.0;
    return (float)(dense / sparse);
}

void csr_host2device(const CSRMatrix& hA, CSRMatrix& dA) {
    if (!hA.row_ptr || !hA.col_idx || !hA.values) die("csr_host2device: host CSRMatrix invalid");
    if (dA.row_ptr || dA.col_idx || dA.values) die("csr_host2device error: destination must be null.");
    csr_alloc_device(dA, hA.height, hA.width, hA.nnz);
    dA.max_row_nnz = hA.max_row_nnz;
    csrspmmCheck(csrspmm_memcpy_h2d(dA.row_ptr, hA.row_ptr, ((size_t)hA.height + 1) * sizeof(int)));
    csrspmmCheck(csrspmm_memcpy_h2d(dA.col_idx, hA.col_idx, (size_t)hA.nnz * sizeof(int)));
    csrspmmCheck(csrspmm_memcpy_h2d(dA.values, hA.values, (size_t)hA.nnz * sizeof(float)));
}

void csr_device2host(const CSRMatrix& dA, CSRMatrix& hA) {
    if (!dA.row_ptr || !dA.col_idx || !dA.values) die("csr_device2host: device pointer invalid");
    if (hA.row_ptr || hA.col_idx || hA.values) die("csr_device2host error: destination must be null.");
    csr_alloc_host(hA, dA.height, dA.width, dA.nnz);
    hA.max_row_nnz = dA.max_row_nnz;
    csrspmmCheck(csrspmm_memcpy_d2h(hA.row_ptr, dA.row_ptr, ((size_t)dA.height + 1) * sizeof(int)));
    csrspmmCheck(csrspmm_memcpy_d2h(hA.col_idx, dA.col_idx, (size_t)dA.nnz * sizeof(int)));
    csrspmmCheck(csrspmm_memcpy_d2h(hA.values, dA.values, (size_t)dA.nnz * sizeof(float)));
}

}  // namespace csrspmm
