"""Seeded synthetic inputs (numpy arrays) from the generators of
include/csrspmm_gen.h, plus a numpy restatement of the counter-based stream
so that tests can pin the C++ implementation element by element."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import capi

TAG_ROWLEN, TAG_COLS, TAG_VALS, TAG_B, TAG_C0 = 1, 2, 3, 4, 5
_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def mix64_np(z: np.ndarray) -> np.ndarray:
    """SplitMix64's finaliser (Stafford variant 13) on a uint64 array."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def key_np(seed: int, tag: int) -> np.uint64:
    with np.errstate(over="ignore"):
        return mix64_np(np.uint64(seed) * _GAMMA + np.uint64(tag))[()]


def rand_np(key, idx: np.ndarray) -> np.ndarray:
    idx = np.asarray(idx, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix64_np(np.uint64(key) + (idx + np.uint64(1)) * _GAMMA)


def u11_np(r: np.ndarray) -> np.ndarray:
    """U(-1, 1) fp32 from 64-bit draws: (r >> 40) * 2^-23 - 1 (exact)."""
    return ((r >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -23)) - np.float32(1.0)


@dataclass
class Csr:
    M: int
    K: int
    rowptr: np.ndarray  # int32 [M+1]
    colidx: np.ndarray  # int32 [nnz]
    vals: np.ndarray    # float32 [nnz]
    max_row_nnz: int

    @property
    def nnz(self) -> int:
        return int(self.colidx.size)

    def digest(self) -> str:
        """FNV-1a 64 over rowptr, colidx, values bytes (hex)."""
        h = 0xcbf29ce484222325
        for a in (self.rowptr, self.colidx, self.vals):
            a = np.ascontiguousarray(a)
            h = capi.host().csrspmm_fnv1a64(h, a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        return f"{h:016x}"


def _take(handle) -> Csr:
    lib = capi.host()
    if not handle:
        raise ValueError("generator rejected its parameters")
    try:
        M, K, mx = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        nnz = ctypes.c_longlong()
        lib.csrspmm_gen_shape(handle, ctypes.byref(M), ctypes.byref(K), ctypes.byref(nnz),
                              ctypes.byref(mx))
        rowptr = np.empty(M.value + 1, dtype=np.int32)
        colidx = np.empty(nnz.value, dtype=np.int32)
        vals = np.empty(nnz.value, dtype=np.float32)
        lib.csrspmm_gen_copy(handle, rowptr.ctypes.data_as(ctypes.c_void_p),
                             colidx.ctypes.data_as(ctypes.c_void_p),
                             vals.ctypes.data_as(ctypes.c_void_p))
        return Csr(M.value, K.value, rowptr, colidx, vals, mx.value)
    finally:
        lib.csrspmm_gen_free(handle)


def uniform(M: int, K: int, per_row: int, seed: int) -> Csr:
    return _take(capi.host().csrspmm_gen_uniform(M, K, per_row, seed))


def powerlaw(M: int, K: int, exponent: float, shift: float, cap: int, seed: int) -> Csr:
    return _take(capi.host().csrspmm_gen_powerlaw(M, K, exponent, shift, cap, seed))


def ragged(M: int, K: int, min_len: int, max_len: int, seed: int) -> Csr:
    return _take(capi.host().csrspmm_gen_ragged(M, K, min_len, max_len, seed))


def rmat(scale: int, samples: int, a: float, b: float, c: float, seed: int) -> Csr:
    return _take(capi.host().csrspmm_gen_rmat(scale, samples, a, b, c, seed))


def dense(seed: int, tag: int, rows: int, cols: int, first: int = 0) -> np.ndarray:
    """rows x cols fp32 U(-1,1), row-major, element i = stream(seed, tag)[first + i]."""
    out = np.empty((rows, cols), dtype=np.float32)
    capi.host().csrspmm_gen_dense(seed, tag, first, out.size, out.ctypes.data_as(ctypes.c_void_p))
    return out
