"""Host-side behaviour of the drop-in C++ API (include/csrspmm, libcsrspmm.so):
parse_algorithm's fallback, the CSR/dense helpers against the oracle, and the
reference's exit(1)-on-misuse contract (reference src/host/csr_utils.cpp:15-18,
72-80,116-125,185-193; src/host/dense_utils.cpp:13-16,130-137).  Compiled with
g++ here; no device call is made."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from csrspmm_amd import LIB_DIR

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("cpp") / "host_api_test")
    subprocess.run(["g++", "-O1", "-std=c++17", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "host_api_test.cpp"), "-L", LIB_DIR,
                    "-lcsrspmm", "-lcsrspmm_hip", f"-Wl,-rpath,{LIB_DIR}", "-o", out], check=True)
    return out


def test_host_checks(exe):
    r = subprocess.run([exe, "checks"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip().endswith("OK")
    assert "Unknown algorithm: adaptive, using Naive" in r.stderr


def test_dense2csr_matches_oracle_bitwise(exe, tmp_path):
    rng = np.random.default_rng(1)
    D = rng.uniform(-1, 1, (60, 90)).astype(np.float32)
    D[rng.random(D.shape) < 0.7] = 0.0
    D[1, 1] = np.nan
    D[2, 2] = -0.0
    D[3, 3] = 1e-6
    src = tmp_path / "d.bin"
    D.tofile(src)
    for tol in ("0", "0.25"):
        pre = str(tmp_path / f"o{tol}")
        r = subprocess.run([exe, "dense2csr", str(src), "60", "90", tol, pre], capture_output=True,
                           text=True, timeout=60)
        assert r.returncode == 0, r.stderr
        nnz, mx = map(int, r.stdout.split())
        rp, ci, va, omx = oracle.dense2csr(D, float(tol))
        assert nnz == ci.size and mx == omx
        assert np.array_equal(np.fromfile(pre + ".rowptr", np.int32), rp)
        assert np.array_equal(np.fromfile(pre + ".colidx", np.int32), ci)
        assert np.array_equal(np.fromfile(pre + ".vals", np.uint32), va.view(np.uint32))


@pytest.mark.parametrize("case,msg", [
    ("death-csr-alloc-twice", "already allocated host memory"),
    ("death-dense2csr-nonempty", "destination must be null"),
    ("death-dense2csr-invalid", "invalid dense matrix"),
    ("death-csr2dense-nonempty", "destination must be null"),
    ("death-dense-alloc-twice", "already allocated host memory"),
    ("death-h2d-null-source", "host CSRMatrix invalid"),
    ("death-dense-h2d-nonnull", "Only accept null destination"),
])
def test_misuse_exits_1(exe, case, msg):
    r = subprocess.run([exe, case], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1
    assert msg in r.stderr
