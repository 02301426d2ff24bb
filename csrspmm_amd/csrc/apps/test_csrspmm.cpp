// C++ correctness driver over the drop-in API (reference tests/test_csrspmm.cu).
// Same flags: -M -N -K -s -a -b -algo, with the reference's naming (A is M x N,
// B is N x K, C is M x K).  -algo all runs every variant.  Unlike the
// reference, the exit status reports the result (0 = every variant passed).
#include <csrspmm/csrspmm.h>
#include <csrspmm/csr_utils.h>
#include <csrspmm/dense_utils.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <string>
#include <vector>

int main(int argc, char** argv) {
    int M = 1024, N = 1024, K = 1024;
    float sparsity = 0.7f, alpha = 1.0f, beta = 0.5f;
    std::string algo_str = "Naive";
    for (int i = 1; i < argc; ++i) {
        std::string arg = argv[i];
        if (arg == "-M" && i + 1 < argc) M = std::atoi(argv[++i]);
        else if (arg == "-N" && i + 1 < argc) N = std::atoi(argv[++i]);
        else if (arg == "-K" && i + 1 < argc) K = std::atoi(argv[++i]);
        else if (arg == "-s" && i + 1 < argc) sparsity = std::atof(argv[++i]);
        else if (arg == "-a" && i + 1 < argc) alpha = std::atof(argv[++i]);
        else if (arg == "-b" && i + 1 < argc) beta = std::atof(argv[++i]);
        else if (arg == "-algo" && i + 1 < argc) algo_str = argv[++i];
        else if (arg == "-h" || arg == "--help") {
            std::cout << "Usage: " << argv[0]
                      << " [-M rows] [-N cols of A] [-K cols of B] [-s sparsity] [-a alpha] [-b beta]"
                         " [-algo Naive|NaiveSmem|WarpPerRow|WarpPerRowFp4|WarpPerRowSmem|"
                         "WarpPerRowSmemFp4|Auto|all]\n";
            return 0;
        } else {
            std::cerr << "Unknown or incomplete flag: " << arg << std::endl;
            return 1;
        }
    }
    std::vector<std::string> algos;
    if (algo_str == "all")
        algos = {"Naive", "NaiveSmem", "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4",
                 "Auto"};
    else
        algos = {algo_str};

    csrspmm::DenseMatrix hA, hB, hC;
    csrspmm::dense_alloc_host(hA, M, N);
    csrspmm::dense_alloc_host(hB, N, K);
    csrspmm::dense_alloc_host(hC, M, K);
    csrspmm::dense_init_random(hA, -10.0f, 10.0f, sparsity, true);
    csrspmm::dense_init_random(hB, -10.0f, 10.0f, 0.0f, true);
    csrspmm::dense_init_random(hC, -10.0f, 10.0f, 0.0f, true);
    csrspmm::CSRMatrix hA_csr;
    csrspmm::dense2csr(hA, hA_csr, 0.0f);

    // Integer inputs with |sum| < 2^24 make every variant's fp32 result exact,
    // so the reference's absolute tolerance (1e-2) is a bit-level check here.
    csrspmm::DenseMatrix hRef;
    csrspmm::dense_alloc_host(hRef, M, K);
    std::memcpy(hRef.data, hC.data, sizeof(float) * (size_t)M * K);
    csrspmm::dense_gemm_cpu(M, N, K, alpha, beta, hA, hB, hRef);

    int failures = 0;
    for (const std::string& name : algos) {
        csrspmm::Algorithm algo = csrspmm::parse_algorithm(name);
        csrspmm::CSRMatrix dA;
        csrspmm::csr_host2device(hA_csr, dA);
        csrspmm::DenseMatrix dB, dC, hOut;
        csrspmm::dense_host2device(hB, dB);
        csrspmm::dense_host2device(hC, dC);
        csrspmm::spmm(dA, dB, dC, alpha, beta, algo);
        csrspmm::dense_device2host(dC, hOut);
        const bool ok = csrspmm::dense_compare(hOut, hRef, 1e-2f);
        std::cout << (ok ? "Pass: " : "Error: ") << name << " M=" << M << " N=" << N << " K=" << K
                  << " nnz=" << hA_csr.nnz << std::endl;
        failures += ok ? 0 : 1;
        // the same product through a stored plan, twice
        {
            csrspmm::dense_free_device(dC);
            csrspmm::dense_host2device(hC, dC);
            csrspmm::SpmmPlan plan(dA, algo, K);
            plan.run(dB, dC, alpha, beta);
            csrspmm::dense_free_host(hOut);
            csrspmm::dense_device2host(dC, hOut);
            const bool ok2 = csrspmm::dense_compare(hOut, hRef, 1e-2f);
            std::cout << (ok2 ? "Pass: " : "Error: ") << name << " (plan)" << std::endl;
            failures += ok2 ? 0 : 1;
        }
        csrspmm::dense_free_host(hOut);
        csrspmm::csr_free_device(dA);
        csrspmm::dense_free_device(dB);
        csrspmm::dense_free_device(dC);
    }
    if (algo_str == "all") {
        // the device dense -> CSR must give the host dense2csr's arrays exactly
        csrspmm::DenseMatrix dDense;
        csrspmm::dense_host2device(hA, dDense);
        csrspmm::CSRMatrix dA2, hA2;
        csrspmm::dense2csr_device(dDense, dA2, 0.0f);
        csrspmm::csr_device2host(dA2, hA2);
        const bool same =
            hA2.nnz == hA_csr.nnz && hA2.max_row_nnz == hA_csr.max_row_nnz &&
            std::memcmp(hA2.row_ptr, hA_csr.row_ptr, sizeof(int) * ((size_t)M + 1)) == 0 &&
            std::memcmp(hA2.col_idx, hA_csr.col_idx, sizeof(int) * (size_t)hA_csr.nnz) == 0 &&
            std::memcmp(hA2.values, hA_csr.values, sizeof(float) * (size_t)hA_csr.nnz) == 0;
        std::cout << (same ? "Pass: " : "Error: ") << "dense2csr_device nnz=" << hA2.nnz
                  << " max_row_nnz=" << hA2.max_row_nnz << std::endl;
        failures += same ? 0 : 1;
        csrspmm::csr_free_host(hA2);
        csrspmm::csr_free_device(dA2);
        csrspmm::dense_free_device(dDense);
    }
    csrspmm::dense_free_host(hA);
    csrspmm::dense_free_host(hB);
    csrspmm::dense_free_host(hC);
    csrspmm::dense_free_host(hRef);
    csrspmm::csr_free_host(hA_csr);
    return failures == 0 ? 0 : 1;
}
