"""ctypes view of the C ABI (include/csrspmm_c.h, include/csrspmm_gen.h).

Loading imports torch first so that libcsrspmm_hip.so binds to the HIP
runtime torch already loaded (both are SONAME libamdhip64.so.7): one runtime
per process, so torch's device pointers and streams are valid here.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (see module docstring)

from . import LIB_DIR

_c_int, _c_ll, _c_float, _c_void_p, _c_size_t = (ctypes.c_int, ctypes.c_longlong, ctypes.c_float,
                                                 ctypes.c_void_p, ctypes.c_size_t)
_c_u64 = ctypes.c_uint64

ALGO = {"Naive": 0, "NaiveSmem": 1, "WarpPerRow": 2, "WarpPerRowFp4": 3, "WarpPerRowSmem": 4,
        "WarpPerRowSmemFp4": 5, "Auto": 6}
FLAG_C_IS_ZERO = 1

# Every function include/csrspmm_c.h declares: name -> (restype, argtypes).
HIP_API = {
    "csrspmm_version": (_c_int, []),
    "csrspmm_status_string": (ctypes.c_char_p, [_c_int]),
    "csrspmm_parse_algorithm": (_c_int, [ctypes.c_char_p]),
    "csrspmm_algorithm_name": (ctypes.c_char_p, [_c_int]),
    "csrspmm_resolve_algorithm": (_c_int, [_c_int, _c_int]),
    "csrspmm_resolve_algorithm_ex": (_c_int, [_c_int] * 6),
    "csrspmm_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int, _c_int]),
    "csrspmm_workspace_bytes_ex": (_c_size_t, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "csrspmm_workspace_panel_info": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                              ctypes.POINTER(_c_ll)]),
    "csrspmm_call_shares": (_c_int, [_c_int] * 6),
    "csrspmm_spmm_f32": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p,
                                  _c_void_p, _c_int, _c_void_p, _c_ll, _c_void_p, _c_ll, _c_float,
                                  _c_float, _c_void_p]),
    "csrspmm_spmm_f32_ex": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p,
                                     _c_void_p, _c_int, _c_void_p, _c_ll, _c_void_p, _c_ll,
                                     _c_float, _c_float, ctypes.c_uint, _c_void_p, _c_size_t,
                                     _c_void_p]),
    "csrspmm_spmm_f32_noalloc": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p,
                                          _c_void_p, _c_void_p, _c_int, _c_void_p, _c_ll,
                                          _c_void_p, _c_ll, _c_float, _c_float, ctypes.c_uint,
                                          _c_void_p]),
    "csrspmm_plan_create": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p,
                                     _c_int, _c_void_p, ctypes.POINTER(_c_void_p)]),
    "csrspmm_plan_spmm_f32": (_c_int, [_c_void_p, _c_int, _c_void_p, _c_ll, _c_void_p, _c_ll, _c_float,
                                       _c_float, ctypes.c_uint, _c_void_p]),
    "csrspmm_plan_algorithm": (_c_int, [_c_void_p]),
    "csrspmm_plan_device_bytes": (_c_size_t, [_c_void_p]),
    "csrspmm_plan_panelized_rows": (_c_int, [_c_void_p]),
    "csrspmm_plan_shares": (_c_int, [_c_void_p, _c_int]),
    "csrspmm_plan_destroy": (_c_int, [_c_void_p]),
    "csrspmm_release_workspace": (_c_int, [_c_void_p]),
    "csrspmm_release_all_workspaces": (_c_int, []),
    "csrspmm_owned_workspaces": (_c_int, [ctypes.POINTER(_c_size_t)]),
    "csrspmm_validate_csr": (_c_int, [_c_int, _c_int, _c_int, _c_void_p, _c_void_p,
                                      ctypes.POINTER(_c_int), ctypes.POINTER(_c_int), _c_void_p]),
    "csrspmm_dense2csr_count_f32": (_c_int, [_c_int, _c_int, _c_void_p, _c_ll, _c_float, _c_void_p,
                                             _c_void_p, _c_void_p]),
    "csrspmm_dense2csr_fill_f32": (_c_int, [_c_int, _c_int, _c_void_p, _c_ll, _c_float, _c_void_p,
                                            _c_void_p, _c_void_p, _c_void_p]),
    "csrspmm_csr_max_row_nnz": (_c_int, [_c_int, _c_void_p, _c_void_p, _c_void_p]),
    "csrspmm_indices_i64_to_i32": (_c_int, [_c_void_p, _c_void_p, _c_ll, _c_void_p, _c_void_p]),
    "csrspmm_device_malloc": (_c_int, [ctypes.POINTER(_c_void_p), _c_size_t]),
    "csrspmm_device_free": (_c_int, [_c_void_p]),
    "csrspmm_memcpy_h2d": (_c_int, [_c_void_p, _c_void_p, _c_size_t]),
    "csrspmm_memcpy_d2h": (_c_int, [_c_void_p, _c_void_p, _c_size_t]),
    "csrspmm_memcpy_d2d": (_c_int, [_c_void_p, _c_void_p, _c_size_t, _c_void_p]),
    "csrspmm_device_synchronize": (_c_int, []),
    "csrspmm_stream_synchronize": (_c_int, [_c_void_p]),
    "csrspmm_get_last_error": (_c_int, []),
    "csrspmm_device_count": (_c_int, []),
    "csrspmm_timing_enable": (_c_int, [_c_int]),
    "csrspmm_timing_read": (_c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_int)]),
}

# Every function include/csrspmm_gen.h declares.
GEN_API = {
    "csrspmm_gen_key": (_c_u64, [_c_u64, _c_int]),
    "csrspmm_gen_rand": (_c_u64, [_c_u64, _c_u64]),
    "csrspmm_gen_dense": (None, [_c_u64, _c_int, _c_u64, _c_size_t, _c_void_p]),
    "csrspmm_gen_uniform": (_c_void_p, [_c_int, _c_int, _c_int, _c_u64]),
    "csrspmm_gen_powerlaw": (_c_void_p, [_c_int, _c_int, ctypes.c_double, ctypes.c_double, _c_int,
                                         _c_u64]),
    "csrspmm_gen_ragged": (_c_void_p, [_c_int, _c_int, _c_int, _c_int, _c_u64]),
    "csrspmm_gen_rmat": (_c_void_p, [_c_int, _c_ll, ctypes.c_double, ctypes.c_double,
                                     ctypes.c_double, _c_u64]),
    "csrspmm_gen_shape": (_c_int, [_c_void_p, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int),
                                   ctypes.POINTER(_c_ll), ctypes.POINTER(_c_int)]),
    "csrspmm_gen_copy": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "csrspmm_gen_free": (None, [_c_void_p]),
    "csrspmm_fnv1a64": (_c_u64, [_c_u64, _c_void_p, _c_size_t]),
}

_hip = None
_host = None


def _bind(lib, table):
    for name, (res, args) in table.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _load(name):
    path = os.path.join(LIB_DIR, name)
    if not os.path.exists(path):
        raise OSError(f"{path} is missing: build it with `python -m csrspmm_amd.build`")
    return ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)


def hip():
    """libcsrspmm_hip.so with the C ABI bound."""
    global _hip
    if _hip is None:
        _hip = _bind(_load("libcsrspmm_hip.so"), HIP_API)
    return _hip


def host():
    """libcsrspmm.so (C++ API + generators) with the generator ABI bound."""
    global _host
    if _host is None:
        hip()
        _host = _bind(_load("libcsrspmm.so"), GEN_API)
    return _host


class CsrspmmError(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        msg = hip().csrspmm_status_string(status).decode()
        super().__init__(f"{what}: status {status} ({msg})" if what else f"status {status} ({msg})")
        self.status = status


def check(status: int, what: str = "") -> None:
    if status != 0:
        raise CsrspmmError(status, what)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def leading_dim(X, name="operand") -> int:
    """Row stride of a 2-D row-major operand (B, C or a dense input):
    stride(0) whenever X has more than one row, whatever its width, so a
    one-column view X[:, k:k+1] of a wider tensor is addressed through its
    parent's rows; max(width, 1) for a single row (or none) or no columns,
    where stride(0) addresses nothing.  A row stride below the width is
    rejected."""
    rows, cols = X.shape
    if rows <= 1 or cols == 0:
        return max(cols, 1)
    if cols > 1 and X.stride(1) != 1:
        raise ValueError(f"{name} must be row-major (stride(1) == 1)")
    if X.stride(0) < max(cols, 1):
        raise ValueError(f"{name} must have a row stride (stride(0)) of at least its width")
    return X.stride(0)


def spmm(algo, rowptr, colidx, vals, B, C, alpha, beta, *, M=None, K=None, hint=-1, flags=0,
         workspace=None, stream=None, owned_workspace=False, noalloc=False):
    """C = alpha*A*B + beta*C through csrspmm_spmm_f32_ex (or csrspmm_spmm_f32
    when owned_workspace=True, csrspmm_spmm_f32_noalloc when noalloc=True).
    All tensors on one GPU; C is written in place.  Returns C.  Allocates the
    workspace with torch when none is given (not for noalloc)."""
    a = ALGO[algo] if isinstance(algo, str) else int(algo)
    M = rowptr.numel() - 1 if M is None else M
    K = B.shape[0] if K is None else K
    N = C.shape[1]
    nnz = vals.numel()
    ldb = leading_dim(B, "B")
    ldc = leading_dim(C, "C")
    if stream is None:
        stream = torch.cuda.current_stream(C.device).cuda_stream
    lib = hip()
    if noalloc:
        st = lib.csrspmm_spmm_f32_noalloc(a, M, K, N, nnz, _ptr(rowptr), _ptr(colidx), _ptr(vals),
                                          hint, _ptr(B), ldb, _ptr(C), ldc, alpha, beta, flags,
                                          ctypes.c_void_p(stream))
    elif owned_workspace:
        st = lib.csrspmm_spmm_f32(a, M, K, N, nnz, _ptr(rowptr), _ptr(colidx), _ptr(vals), hint,
                                  _ptr(B), ldb, _ptr(C), ldc, alpha, beta, ctypes.c_void_p(stream))
    else:
        need = lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, hint)
        if workspace is None and need > 0:
            workspace = torch.empty(need, dtype=torch.uint8, device=C.device)
        wsz = 0 if workspace is None else workspace.numel()
        st = lib.csrspmm_spmm_f32_ex(a, M, K, N, nnz, _ptr(rowptr), _ptr(colidx), _ptr(vals),
                                     hint, _ptr(B), ldb, _ptr(C), ldc, alpha, beta, flags,
                                     _ptr(workspace), wsz, ctypes.c_void_p(stream))
    check(st, f"csrspmm_spmm {algo}")
    return C


def call_shares(algo, M, K, N, nnz, hint=-1) -> bool:
    """Whether a per-call product of this shape (workspace of
    csrspmm_workspace_bytes_ex bytes, 16-byte aligned B and C rows) splits
    its long rows by XCD, so that rows above 128 nonzeros are summed in
    parts rather than in CSR order."""
    a = ALGO[algo] if isinstance(algo, str) else int(algo)
    return bool(hip().csrspmm_call_shares(a, M, K, N, nnz, hint))


def panelized_rows(algo, rowptr, colidx, vals, B, C, alpha=1.0, beta=0.0, *, hint=-1):
    """Runs one per-call product (as spmm, with a workspace of
    csrspmm_workspace_bytes_ex bytes) and returns how many rows it cut into
    column panels: None when a call of this shape uses no panels, 0 when the
    panel loads were too skewed.  Synchronizes the device."""
    a = ALGO[algo] if isinstance(algo, str) else int(algo)
    M, K, N, nnz = rowptr.numel() - 1, B.shape[0], C.shape[1], vals.numel()
    lib = hip()
    off = ctypes.c_longlong(-1)
    P = lib.csrspmm_workspace_panel_info(a, M, K, N, nnz, hint, ctypes.byref(off))
    need = lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, hint)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=C.device)
    spmm(algo, rowptr, colidx, vals, B, C, alpha, beta, hint=hint, workspace=ws)
    torch.cuda.synchronize(C.device)
    if P <= 0:
        return None
    return int(ws[off.value:off.value + 4].view(torch.int32).item())


class Plan:
    """A stored plan (csrspmm_plan_*) for one CSR matrix on the GPU.  Keeps
    references to the CSR tensors, which the plan uses in place."""

    def __init__(self, algo, rowptr, colidx, vals, K, n_hint=-1, stream=None):
        a = ALGO[algo] if isinstance(algo, str) else int(algo)
        self._keep = (rowptr, colidx, vals)
        self.M = rowptr.numel() - 1
        self.K = K
        if stream is None:
            stream = torch.cuda.current_stream(rowptr.device).cuda_stream
        h = _c_void_p()
        check(hip().csrspmm_plan_create(a, self.M, K, vals.numel(), _ptr(rowptr), _ptr(colidx),
                                        _ptr(vals), n_hint, ctypes.c_void_p(stream),
                                        ctypes.byref(h)), "csrspmm_plan_create")
        self._h = h

    @property
    def algorithm(self) -> str:
        return hip().csrspmm_algorithm_name(hip().csrspmm_plan_algorithm(self._h)).decode()

    @property
    def device_bytes(self) -> int:
        return hip().csrspmm_plan_device_bytes(self._h)

    @property
    def panelized_rows(self) -> int:
        return hip().csrspmm_plan_panelized_rows(self._h)

    def shares(self, N) -> bool:
        """Whether this plan's calls of N columns split long rows by XCD."""
        st = hip().csrspmm_plan_shares(self._h, int(N))
        if st < 0:
            raise RuntimeError(f"csrspmm_plan_shares: status {st}")
        return bool(st)

    def spmm(self, B, C, alpha, beta, flags=0, stream=None):
        if stream is None:
            stream = torch.cuda.current_stream(C.device).cuda_stream
        N = C.shape[1]
        ldb = leading_dim(B, "B")
        ldc = leading_dim(C, "C")
        check(hip().csrspmm_plan_spmm_f32(self._h, N, _ptr(B), ldb, _ptr(C), ldc, alpha, beta, flags,
                                          ctypes.c_void_p(stream)), "csrspmm_plan_spmm_f32")
        return C

    def close(self):
        if self._h:
            check(hip().csrspmm_plan_destroy(self._h), "csrspmm_plan_destroy")
            self._h = _c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def release_workspace(stream=None, device=None) -> None:
    """Frees the library-owned workspace of (device, stream); the current
    stream of the current device by default."""
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    check(hip().csrspmm_release_workspace(ctypes.c_void_p(stream)), "csrspmm_release_workspace")


def release_all_workspaces() -> None:
    check(hip().csrspmm_release_all_workspaces(), "csrspmm_release_all_workspaces")


def owned_workspaces():
    """(number of library-owned workspaces held, their total bytes)."""
    b = _c_size_t(0)
    n = hip().csrspmm_owned_workspaces(ctypes.byref(b))
    return n, b.value


def timing_enable(on: bool) -> None:
    check(hip().csrspmm_timing_enable(1 if on else 0), "csrspmm_timing_enable")


def timing_read():
    """(summed main-kernel ms, calls) since the previous read."""
    ms = ctypes.c_double(0.0)
    n = _c_int(0)
    check(hip().csrspmm_timing_read(ctypes.byref(ms), ctypes.byref(n)), "csrspmm_timing_read")
    return ms.value, n.value


def validate(rowptr, colidx, K, stream=None):
    """(flags, max_row_nnz) from the device validator."""
    M = rowptr.numel() - 1
    f = _c_int(0)
    m = _c_int(0)
    if stream is None:
        stream = torch.cuda.current_stream(rowptr.device).cuda_stream
    check(hip().csrspmm_validate_csr(M, K, colidx.numel(), _ptr(rowptr), _ptr(colidx),
                                     ctypes.byref(f), ctypes.byref(m), ctypes.c_void_p(stream)),
          "csrspmm_validate_csr")
    return f.value, m.value


def _stream_of(t, stream):
    return torch.cuda.current_stream(t.device).cuda_stream if stream is None else stream


def dense2csr(D, tol=0.0, stream=None):
    """Device dense -> CSR (rowptr, colidx, vals); one host sync to size the
    arrays."""
    M, K = D.shape
    s = _stream_of(D, stream)
    rowptr = torch.empty(M + 1, dtype=torch.int32, device=D.device)
    nnz = torch.empty(1, dtype=torch.int64, device=D.device)
    ld = leading_dim(D, "dense")
    check(hip().csrspmm_dense2csr_count_f32(M, K, _ptr(D), ld, tol, _ptr(rowptr), _ptr(nnz),
                                            ctypes.c_void_p(s)), "csrspmm_dense2csr_count_f32")
    n = int(nnz.item())
    colidx = torch.empty(n, dtype=torch.int32, device=D.device)
    vals = torch.empty(n, dtype=torch.float32, device=D.device)
    check(hip().csrspmm_dense2csr_fill_f32(M, K, _ptr(D), ld, tol, _ptr(rowptr), _ptr(colidx),
                                           _ptr(vals), ctypes.c_void_p(s)),
          "csrspmm_dense2csr_fill_f32")
    return rowptr, colidx, vals


def max_row_nnz(rowptr, stream=None):
    """Longest row, as a one-element int32 device tensor (no host sync)."""
    out = torch.empty(1, dtype=torch.int32, device=rowptr.device)
    check(hip().csrspmm_csr_max_row_nnz(rowptr.numel() - 1, _ptr(rowptr), _ptr(out),
                                        ctypes.c_void_p(_stream_of(rowptr, stream))),
          "csrspmm_csr_max_row_nnz")
    return out


def narrow_indices(idx64, stream=None):
    """(int32 copy, one-element int32 overflow flag), both on the device."""
    dst = torch.empty(idx64.numel(), dtype=torch.int32, device=idx64.device)
    flag = torch.empty(1, dtype=torch.int32, device=idx64.device)
    check(hip().csrspmm_indices_i64_to_i32(_ptr(idx64), _ptr(dst), idx64.numel(), _ptr(flag),
                                           ctypes.c_void_p(_stream_of(idx64, stream))),
          "csrspmm_indices_i64_to_i32")
    return dst, flag
