"""CPU oracle for the CSR SpMM path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker (or as the CPU baseline that is timed
beside the GPU).  The product never imports it.

Wraps oracle/build/liboracle.so (spmm_oracle.c, built strictly) and
oracle/build/libcpu_spmm.so (cpu_spmm.c, the timed CPU baseline).  Each C
function cites the reference file:line it restates; the pinning checks live
in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "build")

_vp, _i, _ll, _f, _d = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float, ctypes.c_double

_ORACLE_API = {
    "oracle_spmm_f64": (None, [_i, _i, _vp, _vp, _vp, _vp, _ll, _vp, _ll, _d, _d, _i, _vp, _i, _vp,
                               _vp]),
    "oracle_spmm_f32_seq": (None, [_i, _i, _vp, _vp, _vp, _vp, _ll, _vp, _ll, _f, _f, _i, _vp, _i,
                                   _vp, _ll]),
    "oracle_check": (_ll, [_ll, _vp, _ll, _i, _vp, _vp, _d, ctypes.POINTER(_d), ctypes.POINTER(_d),
                           ctypes.POINTER(_ll)]),
    "oracle_dense2csr": (_ll, [_vp, _i, _i, _f, _vp, _vp, _vp, ctypes.POINTER(_i)]),
    "oracle_csr2dense": (None, [_i, _i, _vp, _vp, _vp, _vp]),
    "oracle_dense_gemm_cpu": (None, [_i, _i, _i, _f, _f, _vp, _vp, _vp]),
    "oracle_dense_init_random_ref": (None, [_vp, _i, _i, _f, _f, _f, _i]),
}
_CPU_API = {
    "cpu_spmm_max_threads": (_i, []),
    "cpu_spmm_f32": (None, [_i, _i, _vp, _vp, _vp, _vp, _ll, _vp, _ll, _f, _f, _i]),
    "cpu_dense_gemm": (None, [_i, _i, _i, _f, _f, _vp, _vp, _vp]),
}

_lib = None
_cpu = None


def build() -> None:
    """Compile the oracle libraries (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load(name, table):
    path = os.path.join(BUILD, name)
    if not os.path.exists(path):
        build()
    lib = ctypes.CDLL(path)
    for fn, (res, args) in table.items():
        f = getattr(lib, fn)
        f.restype = res
        f.argtypes = args
    return lib


def lib():
    global _lib
    if _lib is None:
        _lib = _load("liboracle.so", _ORACLE_API)
    return _lib


def cpu():
    global _cpu
    if _cpu is None:
        _cpu = _load("libcpu_spmm.so", _CPU_API)
    return _cpu


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _c(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


def spmm_f64(rowptr, colidx, vals, B, C0=None, alpha=1.0, beta=0.0, c0_zero=False, rows=None,
             with_s=True):
    """(R, S): fp64 reference and condition magnitude, [len(rows) or M, N]."""
    rowptr, colidx, vals = _c(rowptr, np.int32), _c(colidx, np.int32), _c(vals, np.float32)
    B = _c(B, np.float32)
    C0 = _c(C0, np.float32)
    M = rowptr.size - 1
    N = B.shape[1]
    rows_a = None if rows is None else _c(rows, np.int32)
    n_out = M if rows_a is None else rows_a.size
    R = np.empty((n_out, N), dtype=np.float64)
    S = np.empty((n_out, N), dtype=np.float64) if with_s else None
    if beta != 0.0 and not c0_zero and C0 is None:
        raise ValueError("beta != 0 needs C0")
    lib().oracle_spmm_f64(M, N, _p(rowptr), _p(colidx), _p(vals), _p(B), B.shape[1], _p(C0),
                          N if C0 is None else C0.shape[1], alpha, beta, int(c0_zero), _p(rows_a),
                          0 if rows_a is None else rows_a.size, _p(R), _p(S))
    return R, S


def spmm_f32_seq(rowptr, colidx, vals, B, C0=None, alpha=1.0, beta=0.0, c0_zero=False, rows=None):
    """fp32 CSR-order fma restatement of the reference kernels, [rows or M, N]."""
    rowptr, colidx, vals = _c(rowptr, np.int32), _c(colidx, np.int32), _c(vals, np.float32)
    B = _c(B, np.float32)
    C0 = _c(C0, np.float32)
    M = rowptr.size - 1
    N = B.shape[1]
    rows_a = None if rows is None else _c(rows, np.int32)
    n_out = M if rows_a is None else rows_a.size
    out = np.empty((n_out, N), dtype=np.float32)
    lib().oracle_spmm_f32_seq(M, N, _p(rowptr), _p(colidx), _p(vals), _p(B), B.shape[1], _p(C0),
                              N if C0 is None else C0.shape[1], alpha, beta, int(c0_zero),
                              _p(rows_a), 0 if rows_a is None else rows_a.size, _p(out), N)
    return out


def check(C, R, S, tol=1e-5):
    """(n_bad, max_ratio, max_rel_plain, worst_index) under
    |C - R| <= tol * max(|R|, S)."""
    C = _c(C, np.float32)
    R = _c(R, np.float64)
    S = None if S is None else _c(S, np.float64)
    mr, mp, w = _d(), _d(), _ll()
    n = R.size
    ncols = R.shape[1] if R.ndim == 2 else max(n, 1)
    bad = lib().oracle_check(n, _p(C), ncols, ncols, _p(R), _p(S), tol, ctypes.byref(mr),
                             ctypes.byref(mp), ctypes.byref(w))
    return int(bad), mr.value, mp.value, int(w.value)


def dense2csr(dense, tol=0.0):
    dense = _c(dense, np.float32)
    H, W = dense.shape
    mx = _i()
    nnz = lib().oracle_dense2csr(_p(dense), H, W, tol, None, None, None, ctypes.byref(mx))
    rowptr = np.empty(H + 1, dtype=np.int32)
    colidx = np.empty(nnz, dtype=np.int32)
    vals = np.empty(nnz, dtype=np.float32)
    lib().oracle_dense2csr(_p(dense), H, W, tol, _p(rowptr), _p(colidx), _p(vals), ctypes.byref(mx))
    return rowptr, colidx, vals, mx.value


def csr2dense(rowptr, colidx, vals, H, W):
    rowptr, colidx, vals = _c(rowptr, np.int32), _c(colidx, np.int32), _c(vals, np.float32)
    out = np.empty((H, W), dtype=np.float32)
    lib().oracle_csr2dense(H, W, _p(rowptr), _p(colidx), _p(vals), _p(out))
    return out


def dense_gemm_cpu(A, B, C, alpha, beta):
    """In-place on a copy of C; reference naming A: M x N, B: N x K."""
    A, B = _c(A, np.float32), _c(B, np.float32)
    C = np.array(C, dtype=np.float32, copy=True)
    M, N = A.shape
    K = B.shape[1]
    lib().oracle_dense_gemm_cpu(M, N, K, alpha, beta, _p(A), _p(B), _p(C))
    return C


def dense_init_random_ref(height, width, low=-1.0, high=1.0, sparsity=0.0, integer_values=False):
    out = np.empty((height, width), dtype=np.float32)
    lib().oracle_dense_init_random_ref(_p(out), height, width, low, high, sparsity,
                                       int(integer_values))
    return out


def cpu_dense_gemm(A, B, C, alpha, beta):
    """Timed reference dense CPU GEMM (fast-math build); C updated in place."""
    M, N = A.shape
    K = B.shape[1]
    cpu().cpu_dense_gemm(M, N, K, alpha, beta, _p(A), _p(B), _p(C))
    return C


def cpu_spmm_f32(rowptr, colidx, vals, B, C, alpha, beta, nthreads=0):
    """Timed CPU baseline; C updated in place."""
    cpu().cpu_spmm_f32(rowptr.size - 1, B.shape[1], _p(rowptr), _p(colidx), _p(vals), _p(B),
                       B.shape[1], _p(C), C.shape[1], alpha, beta, nthreads)
    return C
