// C++ timing driver over the drop-in API (reference benchmarks/bench_csrspmm.cu):
// warmup, then REPS calls of csrspmm::spmm (each ends in a device
// synchronisation, as in the reference), wall-clock timed.  Prints the
// reference's GFLOPS line plus the gather-model bandwidth
// 4(M+1) + 8 nnz + 4 nnz K + 4 M K (1 + [beta != 0]) bytes per call.
#include <csrspmm/csrspmm.h>
#include <csrspmm/csr_utils.h>
#include <csrspmm/dense_utils.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <iostream>
#include <string>

int main(int argc, char** argv) {
    int M = 1024, N = 1024, K = 1024, warmup = 200, reps = 1000;
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
        else if (arg == "-warmup" && i + 1 < argc) warmup = std::atoi(argv[++i]);
        else if (arg == "-reps" && i + 1 < argc) reps = std::atoi(argv[++i]);
        else if (arg == "-h" || arg == "--help") {
            std::cout << "Usage: " << argv[0]
                      << " [-M] [-N] [-K] [-s] [-a] [-b] [-algo name] [-warmup W] [-reps R]\n";
            return 0;
        } else {
            std::cerr << "Unknown or incomplete flag: " << arg << std::endl;
            return 1;
        }
    }
    csrspmm::Algorithm algo = csrspmm::parse_algorithm(algo_str);
    csrspmm::DenseMatrix hA, hB, hC;
    csrspmm::dense_alloc_host(hA, M, N);
    csrspmm::dense_alloc_host(hB, N, K);
    csrspmm::dense_alloc_host(hC, M, K);
    csrspmm::dense_init_random(hA, -10.0f, 10.0f, sparsity, false);
    csrspmm::dense_init_random(hB, -10.0f, 10.0f, 0.0f, false);
    csrspmm::dense_init_random(hC, -10.0f, 10.0f, 0.0f, false);
    csrspmm::CSRMatrix hA_csr;
    csrspmm::dense2csr(hA, hA_csr, 0.0f);
    csrspmm::CSRMatrix dA;
    csrspmm::csr_host2device(hA_csr, dA);
    csrspmm::DenseMatrix dB, dC;
    csrspmm::dense_host2device(hB, dB);
    csrspmm::dense_host2device(hC, dC);

    for (int i = 0; i < warmup + 1; ++i) csrspmm::spmm(dA, dB, dC, alpha, beta, algo);
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < reps; ++i) csrspmm::spmm(dA, dB, dC, alpha, beta, algo);
    const auto t1 = std::chrono::steady_clock::now();
    const double sec = std::chrono::duration<double>(t1 - t0).count() / reps;
    const double flops = 2.0 * hA_csr.nnz * (double)K;
    const double bytes = 4.0 * (M + 1) + 8.0 * hA_csr.nnz + 4.0 * hA_csr.nnz * (double)K +
                         4.0 * M * (double)K * (beta != 0.0f ? 2.0 : 1.0);
    std::printf("%s krnl: avg elapsed time: (%7.6f) s, performance: (%7.2f) GFLOPS, (%7.2f) GB/s "
                "gather-model. size: [%d x %d x %d] nnz=%d\n",
                algo_str.c_str(), sec, flops * 1e-9 / sec, bytes * 1e-9 / sec, M, N, K, hA_csr.nnz);
    csrspmm::dense_free_host(hA);
    csrspmm::dense_free_host(hB);
    csrspmm::dense_free_host(hC);
    csrspmm::csr_free_host(hA_csr);
    csrspmm::csr_free_device(dA);
    csrspmm::dense_free_device(dB);
    csrspmm::dense_free_device(dC);
    return 0;
}
