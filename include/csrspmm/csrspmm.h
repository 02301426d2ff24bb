// High-level CSR SpMM API (reference include/csrspmm/csrspmm.h:10-34).
#pragma once
#include <string>

#include <csrspmm/config.h>
#include <csrspmm/csr_utils.h>
#include <csrspmm/matrix.h>

namespace csrspmm {

// Same enumerators in the same order as the reference (csrspmm.h:10-17).
enum class Algorithm {
    Naive,
    NaiveSmem,
    WarpPerRow,
    WarpPerRowFp4,
    WarpPerRowSmem,
    WarpPerRowSmemFp4
};

// Exact CamelCase match; an unknown name prints a warning to stderr and
// returns Naive (reference src/csrspmm.cpp:13-25).
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

}  // namespace csrspmm
