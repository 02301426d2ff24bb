// CSR helpers (reference include/csrspmm/csr_utils.h:6-18).  Errors print a
// message and exit(1), as in the reference.
#pragma once
#include <csrspmm/matrix.h>

namespace csrspmm {

void csr_alloc_host(CSRMatrix& csr, int height, int width, int nnz);
void csr_free_host(CSRMatrix& csr);

void csr_alloc_device(CSRMatrix& csr, int height, int width, int nnz);
void csr_free_device(CSRMatrix& csr);

// Keeps entries with fabs(v) > tol (so +-0 and NaN are dropped), row-major
// order, and sets max_row_nnz.  csr must be empty.
void dense2csr(const DenseMatrix& dense, CSRMatrix& csr, float tol = 0.0f);
// As dense2csr, on the GPU: d_dense.data is device memory and d_csr (which
// must be empty) receives device arrays and max_row_nnz.  The keep rule and
// order are dense2csr's, so the arrays are identical.  No counterpart in the
// reference, whose dense2csr runs on the host only.
void dense2csr_device(const DenseMatrix& d_dense, CSRMatrix& d_csr, float tol = 0.0f);
// dense must be empty; allocates host memory.
void csr2dense(const CSRMatrix& csr, DenseMatrix& dense);
void print_csr(const CSRMatrix& csr);
// Dense element count over CSR element count (height*width / (2*nnz + height + 1)).
float compression_ratio(const CSRMatrix& csr);

// Allocate the destination (which must be empty) and copy all three arrays
// and max_row_nnz.
void csr_host2device(const CSRMatrix& hA, CSRMatrix& dA);
void csr_device2host(const CSRMatrix& dA, CSRMatrix& hA);

}  // namespace csrspmm
