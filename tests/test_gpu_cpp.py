"""GPU runs of the prebuilt C++ drivers over the drop-in C++ API
(csrspmm_amd/lib/test_csrspmm, bench_csrspmm; reference tests/test_csrspmm.cu,
benchmarks/bench_csrspmm.cu).  test_csrspmm checks every variant against
dense_gemm_cpu on integer inputs (exact) and exits non-zero on a mismatch."""
import os
import re
import subprocess

import pytest

from csrspmm_amd import LIB_DIR

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("args", [
    ["-M", "256", "-N", "300", "-K", "64", "-s", "0.9", "-a", "1.5", "-b", "0.5"],
    ["-M", "100", "-N", "70", "-K", "33", "-s", "0.5", "-a", "1", "-b", "0"],
    ["-M", "64", "-N", "2000", "-K", "16", "-s", "0.0", "-a", "-1", "-b", "2"],
])
def test_cpp_test_driver_all_variants(args, gpu):
    r = subprocess.run([os.path.join(LIB_DIR, "test_csrspmm"), *args, "-algo", "all"],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    # 7 algorithms, each per call and through a plan, and the device dense2csr
    assert r.stdout.count("Pass: ") == 15
    assert "Error" not in r.stdout


def test_cpp_bench_driver(gpu):
    r = subprocess.run([os.path.join(LIB_DIR, "bench_csrspmm"), "-M", "2048", "-N", "2048", "-K",
                        "128", "-s", "0.99", "-algo", "WarpPerRowFp4", "-warmup", "5", "-reps",
                        "20"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    m = re.search(r"performance: \(\s*([0-9.]+)\) GFLOPS", r.stdout)
    assert m and float(m.group(1)) > 0


def test_kernels_h_direct_launches(gpu):
    """HIP code that includes <csrspmm/kernels.h> (reference
    include/csrspmm/kernels.h:6-71) and launches the six kernels itself, with
    the reference launcher's shapes and others, checked element by element
    against an fp64 product inside the driver."""
    r = subprocess.run([os.path.join(LIB_DIR, "test_kernels_h")], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    # 6 kernels x (2 or 3 launch shapes) x 3 column counts
    assert r.stdout.count(" ok ") == 3 * (2 * 2 + 4 * 3)
    assert "FAIL" not in r.stdout
