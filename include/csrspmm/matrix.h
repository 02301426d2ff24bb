// Plain-old-data matrix handles (reference include/csrspmm/matrix.h:6-23).
// Same fields and defaults; no runtime header is pulled in.  Pointers may be
// host or device memory depending on who filled them (the csr_/dense_ helper
// that allocated them says which).
#pragma once

namespace csrspmm {

struct CSRMatrix {
    int height = 0;  // rows (M)
    int width = 0;   // columns (K)
    int nnz = 0;     // nonzeros

    int* row_ptr = nullptr;   // height + 1 entries
    int* col_idx = nullptr;   // nnz entries
    float* values = nullptr;  // nnz entries

    // Longest row.  Set by dense2csr and copied by csr_host2device; the
    // library uses it only as a scheduling hint, never to size memory.
    int max_row_nnz = 0;
};

// Row-major dense matrix; the leading dimension is width.
struct DenseMatrix {
    int height = 0;
    int width = 0;
    float* data = nullptr;  // height * width entries
};

}  // namespace csrspmm
