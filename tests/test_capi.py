"""The C ABI library loads on a machine without a GPU, exports every function
include/*.h declares, and rejects bad arguments before touching the device."""
import os
import re

import pytest

from csrspmm_amd import ALGORITHMS, LIB_DIR, capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(csrspmm_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("csrspmm_c.h", "hip"), ("csrspmm_gen.h", "host")])
def test_every_declared_symbol_is_exported(header, lib):
    names = declared_functions(header)
    assert len(names) >= 10
    handle = capi.hip() if lib == "hip" else capi.host()
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, missing
    table = capi.HIP_API if lib == "hip" else capi.GEN_API
    assert sorted(table) == names, "ctypes table out of sync with the header"


def test_libraries_are_in_tree():
    for name in ("libcsrspmm_hip.so", "libcsrspmm.so"):
        assert os.path.exists(os.path.join(LIB_DIR, name))


def test_parse_and_names():
    lib = capi.hip()
    for i, name in enumerate(ALGORITHMS):
        assert lib.csrspmm_parse_algorithm(name.encode()) == i
        assert lib.csrspmm_algorithm_name(i).decode() == name
    assert lib.csrspmm_parse_algorithm(b"naive") == -1  # exact CamelCase match only
    assert lib.csrspmm_parse_algorithm(b"Adaptive") == -1
    assert lib.csrspmm_parse_algorithm(None) == -1
    assert lib.csrspmm_parse_algorithm(b"Auto") == 6
    assert lib.csrspmm_algorithm_name(6).decode() == "Auto"
    assert lib.csrspmm_algorithm_name(7) is None
    # Auto resolves by N; concrete ids pass through
    assert lib.csrspmm_resolve_algorithm(6, 128) == 3
    assert lib.csrspmm_resolve_algorithm(6, 256) == 3
    assert lib.csrspmm_resolve_algorithm(6, 64) == 4
    assert lib.csrspmm_resolve_algorithm(6, 130) == 4
    assert lib.csrspmm_resolve_algorithm(2, 128) == 2
    assert lib.csrspmm_resolve_algorithm(9, 128) == -1
    # From the whole shape: at N = 128 an L2-sized B (<= 4 MiB) with long rows
    # (>= 96 per row on average, M >= 4096) takes WarpPerRowSmem
    def ex(a, M, K, N, nnz, hint=-1):
        return lib.csrspmm_resolve_algorithm_ex(a, M, K, N, nnz, hint)
    assert ex(6, 4096, 4096, 128, 4096 * 160) == 4
    assert ex(6, 4096, 8192, 128, 4096 * 160) == 4          # B exactly 4 MiB
    assert ex(6, 4096, 8193, 128, 4096 * 160) == 3          # B above 4 MiB
    assert ex(6, 4096, 4096, 128, 4096 * 96) == 4           # from 96 per row
    assert ex(6, 4096, 4096, 128, 4096 * 96 - 1) == 3      # rows shorter
    assert ex(6, 4095, 4096, 128, 4095 * 200) == 3          # fewer rows
    assert ex(6, 1024, 2048, 128, 1024 * 200, 250) == 4     # one launch under the hint: from 1024 rows
    assert ex(6, 1023, 2048, 128, 1023 * 200, 250) == 3
    assert ex(6, 1024, 2048, 128, 1024 * 200, 257) == 3     # a longer row: the plan
    assert ex(6, 4096, 4096, 256, 4096 * 200) == 3          # N = 256
    assert ex(6, 262144, 262144, 128, 8453223) == 3         # XL
    # below N = 128: float4 when its column panels are possible (B >= 64 MiB,
    # no hint below 1024) and rows average 24 or more
    assert ex(6, 262144, 262144, 64, 8453223) == 3          # XL at N = 64: 64 MiB
    assert ex(6, 262144, 262144, 96, 8453223) == 3
    assert ex(6, 262144, 262144, 60, 8453223) == 4          # 60 MiB: no panels
    assert ex(6, 262144, 262144, 64, 8453223, 1023) == 4    # hint rules panels out
    assert ex(6, 262144, 262144, 64, 8453223, 16315) == 3
    assert ex(6, 262144, 262144, 64, 24 * 262144 - 1) == 4  # rows shorter
    assert ex(6, 1 << 20, 1 << 20, 64, 16 << 20) == 4       # R-MAT-like: 16 per row
    assert ex(6, 262144, 262144, 66, 8453223) == 4          # N % 4 != 0
    assert ex(6, 4096, 4096, 64, 4096 * 200) == 4           # small B: scalar
    # from N = 128, sliced calls split by XCD (not swept) take the scalar
    # LDS-staged variant: R-MAT at N = 256 and 512, K = 262144 at N = 1024
    # (or swept with under 4 nonzeros per band)
    assert ex(6, 1 << 20, 1 << 20, 256, 16 << 20) == 4
    assert lib.csrspmm_call_shares(3, 1 << 20, 1 << 20, 512, 16 << 20, -1) == 1
    assert ex(6, 1 << 20, 1 << 20, 128, 16 << 20) == 3      # N = 128: panels, no slices
    assert ex(6, 262144, 262144, 1024, 8453223) == 4        # XL at N = 1024: 2 per band
    assert ex(6, 262144, 262144, 1024, 262144 * 64) == 5    # 4 per band: the sweep
    # from N = 128, swept column slices take the float4 LDS-staged variant
    assert ex(6, 65536, 65536, 256, 4325376) == 5           # large
    assert ex(6, 65536, 65536, 256, 65536 * 7) == 3         # under 2 per band: merge blocks
    assert ex(6, 32768, 65536, 256, 4325376) == 3           # too few rows to sweep: a 16 MiB
                                                            # band and rows above 128
    assert ex(6, 32768, 65536, 256, 32768 * 40) == 3         # too few rows to sweep, 40 per row
    # unswept slices of rows averaging 64..511: the scalar LDS form
    assert ex(6, 4096, 65536, 128, 4096 * 128) == 4
    assert ex(6, 32768, 32768, 256, 32768 * 300) == 4        # rows above 128 on an 8 MiB band
    assert ex(6, 4096, 65536, 256, 4096 * 300, 300) == 3     # a 16 MiB band from 4096 rows
    assert ex(6, 2048, 65536, 256, 2048 * 300, 300) == 4     # but not fewer
    assert ex(6, 8192, 65536, 256, 8192 * 300, 300) == 3
    assert ex(6, 4096, 65536, 128, 4096 * 512) == 3          # 512 per row: split rows
    assert ex(6, 4096, 65536, 128, 4096 * 63) == 3
    assert ex(6, 1 << 20, 1 << 20, 512, 16 << 20) == 4      # R-MAT N = 512: split by XCD
    # sliced calls of skewed rows (a hint above 128 and 4x the mean) take the scalar LDS form
    assert ex(6, 1 << 20, 1 << 20, 512, 16084813, 39531) == 4   # R-MAT N = 512 with its hint
    assert ex(6, 65536, 65536, 256, 65536 * 32, 16384) == 4     # power-law rows, even swept
    assert ex(6, 65536, 65536, 256, 65536 * 200, 250) == 5      # uniform long rows: the sweep
    assert ex(6, 65536, 65536, 256, 65536 * 32, 128) == 5       # no long row: the sweep
    assert ex(6, 131072, 131072, 256, 131072 * 32, 16384) == 3  # unsliced (panels): float4
    # sliced calls that do not sweep, of rows of 129..511 nonzeros, take it too
    assert ex(6, 4096, 4096, 2048, 4096 * 300, 300) == 4
    assert ex(6, 8192, 16384, 512, 8192 * 300, 300) == 4
    assert ex(6, 8192, 16384, 512, 8192 * 40, 128) == 3        # short rows
    assert ex(6, 8192, 16384, 512, 8192 * 600, 700) == 3       # rows split into segments
    assert ex(6, 8192, 16384, 512, 8192 * 300, -1) == 4        # the mean tells without a hint
    assert ex(3, 4096, 4096, 128, 4096 * 200) == 3          # concrete ids pass through
    assert ex(9, 4096, 4096, 128, 4096 * 200) == -1
    assert lib.csrspmm_version() >= 100


def test_status_strings():
    lib = capi.hip()
    for st in (0, -1, -2, -3, -4, -5, -99):
        assert lib.csrspmm_status_string(st)
    assert lib.csrspmm_status_string(-1).decode() == "invalid value"


def _call(**kw):
    args = dict(algo=3, M=4, K=4, N=4, nnz=0, rowptr=None, colidx=None, vals=None, hint=-1,
                B=None, ldb=4, C=None, ldc=4, alpha=1.0, beta=0.0, stream=None)
    args.update(kw)
    return capi.hip().csrspmm_spmm_f32(args["algo"], args["M"], args["K"], args["N"], args["nnz"],
                                       args["rowptr"], args["colidx"], args["vals"], args["hint"],
                                       args["B"], args["ldb"], args["C"], args["ldc"],
                                       args["alpha"], args["beta"], args["stream"])


def test_argument_errors_without_device():
    fake = 0x1000  # never dereferenced: every case fails validation first
    assert _call(algo=-1) == -1
    assert _call(algo=6) == -1
    assert _call(M=-1) == -1
    assert _call(nnz=-5) == -1
    assert _call(rowptr=None, C=fake) == -1          # rowptr missing
    assert _call(rowptr=fake, C=None) == -1          # C missing
    assert _call(rowptr=fake, C=fake, nnz=3) == -1   # colidx / vals / B missing
    assert _call(rowptr=fake, C=fake, ldc=3) == -1   # ldc < N
    assert _call(rowptr=fake, C=fake, nnz=3, colidx=fake, vals=fake, B=fake, ldb=2) == -1
    assert _call(rowptr=fake, C=fake, nnz=3, colidx=fake, vals=fake, B=fake, K=0) == -1
    # merge coordinates beyond int32
    assert _call(M=2**31 - 10, nnz=10, rowptr=fake, C=fake, colidx=fake, vals=fake, B=fake) == -2
    # M == 0 or N == 0 is a successful no-op
    assert _call(M=0) == 0
    assert _call(N=0, ldc=0) == 0


def test_workspace_bytes():
    lib = capi.hip()
    # Naive variants never need one; the warp family needs one for big problems.
    assert lib.csrspmm_workspace_bytes(0, 100000, 128, 10**6) == 0
    assert lib.csrspmm_workspace_bytes(1, 100000, 128, 10**6) == 0
    big = lib.csrspmm_workspace_bytes(3, 262144, 128, 8453223)
    nslots = 8453223 // 256
    assert big >= nslots * 128 * 4 + nslots * 8 + (262144 + 8453223) // 128 * 4
    assert big < 64 * 2**20
    assert lib.csrspmm_workspace_bytes(3, 0, 128, 0) == 0
    assert lib.csrspmm_workspace_bytes(3, 10, 16, 20) == 0  # tiny, no long row possible


def test_hinted_short_rows_skip_the_plan():
    """A hint of at most 256 nonzeros per row on fewer than 2^20 rows +
    nonzeros and 32768 rows, with no column slices, runs as one launch: no
    workspace.  Without the hint, with a longer row possible, from 32768 rows
    (the band sweep needs the plan) or with slices, the plan stays."""
    lib = capi.hip()
    ex = lib.csrspmm_workspace_bytes_ex
    for algo in ("Auto", "WarpPerRow", "WarpPerRowFp4", "WarpPerRowSmem", "WarpPerRowSmemFp4"):
        a = capi.ALGO[algo]
        assert ex(a, 4096, 4096, 128, 4096 * 41, 60) == 0
        assert ex(a, 4096, 4096, 128, 4096 * 41, 256) == 0
        assert ex(a, 4096, 4096, 128, 4096 * 41, -1) > 0      # no hint
        assert ex(a, 4096, 4096, 128, 4096 * 41, 257) > 0     # a row of 257 possible
        assert ex(a, 16384, 16384, 256, 16384 * 60, 70) == 0  # 999,424 items
        assert ex(a, 16384, 16384, 256, 16384 * 63, 70) > 0   # 2^20 items or more
        assert ex(a, 32768, 32768, 128, 32768 * 20, 30) > 0   # 32768 rows
        assert ex(a, 16384, 16384, 512, 16384 * 50, 60) > 0   # 64-column slices


def test_ex_rejects_small_workspace_without_device():
    lib = capi.hip()
    fake = 0x1000
    need = lib.csrspmm_workspace_bytes(3, 262144, 128, 8453223)
    st = lib.csrspmm_spmm_f32_ex(3, 262144, 262144, 128, 8453223, fake, fake, fake, -1, fake, 128,
                                 fake, 128, 1.0, 0.0, 0, fake, need - 1, None)
    assert st == -5
    st = lib.csrspmm_spmm_f32_ex(3, 262144, 262144, 128, 8453223, fake, fake, fake, -1, fake, 128,
                                 fake, 128, 1.0, 0.0, 0, fake + 8, need, None)
    assert st == -1  # misaligned workspace


def test_plan_argument_errors_without_device():
    import ctypes
    lib = capi.hip()
    h = ctypes.c_void_p()
    assert lib.csrspmm_plan_create(3, 4, 4, 0, None, None, None, 0, None, ctypes.byref(h)) == -1
    assert lib.csrspmm_plan_create(3, -1, 4, 0, 0x1000, None, None, 0, None, ctypes.byref(h)) == -1
    assert lib.csrspmm_plan_create(3, 4, 4, 5, 0x1000, None, None, 0, None, ctypes.byref(h)) == -1
    assert lib.csrspmm_plan_create(9, 4, 4, 0, 0x1000, None, None, 0, None, ctypes.byref(h)) == -1
    assert lib.csrspmm_plan_create(3, 4, 4, 0, 0x1000, None, None, 0, None, None) == -1
    assert lib.csrspmm_plan_spmm_f32(None, 4, None, 4, None, 4, 1.0, 0.0, 0, None) == -1
    assert lib.csrspmm_plan_algorithm(None) == -1
    assert lib.csrspmm_plan_device_bytes(None) == 0
    assert lib.csrspmm_plan_destroy(None) == 0


def test_validate_rejects_bad_sizes_without_device():
    lib = capi.hip()
    assert lib.csrspmm_validate_csr(-1, 4, 0, None, None, None, None, None) == -1
    assert lib.csrspmm_validate_csr(4, 4, 0, None, None, None, None, None) == -1


def test_csr_tools_argument_errors_without_device():
    lib = capi.hip()
    inv = -1  # CSRSPMM_STATUS_INVALID_VALUE
    assert lib.csrspmm_dense2csr_count_f32(-1, 4, None, 4, 0.0, None, None, None) == inv
    assert lib.csrspmm_dense2csr_count_f32(4, 4, None, 4, 0.0, None, None, None) == inv
    assert lib.csrspmm_dense2csr_fill_f32(4, 8, None, 4, 0.0, None, None, None, None) == inv
    assert lib.csrspmm_csr_max_row_nnz(3, None, None, None) == inv
    assert lib.csrspmm_indices_i64_to_i32(None, None, 5, None, None) == inv
    assert lib.csrspmm_indices_i64_to_i32(None, None, -1, None, None) == inv


def test_workspace_bytes_ex_panels():
    """The panel tables are reserved on a B of >= 16 MiB with N <= 256 (for
    scalar columns from N = 128) when a row of >= 1024 nonzeros is possible
    under the hint.  Without panels, on a B (or 64-column slice) of >= 64 MiB
    with 2^20 nonzeros and rows above 128 possible, the XCD share tables and
    partials ((nnz / 16) x N floats) are reserved instead."""
    lib = capi.hip()
    a = capi.ALGO["WarpPerRowSmemFp4"]
    M, K, N, nnz = 262144, 262144, 128, 8453223
    base = lib.csrspmm_workspace_bytes(a, M, N, nnz)
    share_part = (nnz // 16) * N * 4
    full = lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, -1)
    assert full == lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, 16384) > base
    assert lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, 1024) == full
    # partials at most 256 MiB, plus tables of a few MiB
    assert full - base <= (256 << 20) + (8 << 20)
    assert not lib.csrspmm_call_shares(a, M, K, N, nnz, -1)  # panels
    # below 1024 no panels: the long rows (above 128) are split by XCD
    assert lib.csrspmm_call_shares(a, M, K, N, nnz, 1023)
    sh = lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, 1023)
    assert share_part <= sh - base <= share_part + (8 << 20)
    assert lib.csrspmm_workspace_bytes_ex(a, M, K, N, nnz, 128) == base  # no long rows at all
    assert not lib.csrspmm_call_shares(a, M, K, N, nnz, 128)
    s = capi.ALGO["WarpPerRowSmem"]
    assert lib.csrspmm_workspace_bytes_ex(s, M, K, N, nnz, -1) > lib.csrspmm_workspace_bytes(s, M, N, nnz)
    # scalar columns below N = 128 take no panels: shares on a 64 MiB B
    assert lib.csrspmm_call_shares(s, M, K, 64, nnz, -1)
    assert lib.csrspmm_workspace_bytes_ex(s, M, K, 64, nnz, -1) > lib.csrspmm_workspace_bytes(s, M, 64, nnz)
    assert not lib.csrspmm_call_shares(s, M, K // 2, 64, nnz, -1)  # a 32 MiB B: neither
    assert lib.csrspmm_workspace_bytes_ex(s, M, K // 2, 64, nnz, -1) == lib.csrspmm_workspace_bytes(s, M, 64, nnz)
    assert lib.csrspmm_workspace_bytes_ex(a, M, K, 64, nnz, -1) > lib.csrspmm_workspace_bytes(a, M, 64, nnz)
    assert lib.csrspmm_workspace_bytes_ex(a, M, 1024, N, nnz, -1) == base  # B of 512 KiB
    assert lib.csrspmm_workspace_bytes_ex(capi.ALGO["Naive"], M, K, N, nnz, -1) == 0
    assert not lib.csrspmm_call_shares(capi.ALGO["Naive"], M, K, N, nnz, -1)
    # too few nonzeros for the shares
    assert not lib.csrspmm_call_shares(s, M, K, 64, (1 << 20) - 1, -1)


def test_panel_rules_without_device():
    """The per-call panel decision the host makes (csrspmm_workspace_panel_info):
    panels need B wide enough for 32 of them (>= 64 MiB), float4 columns or
    scalar ones from N = 128, no column slices, and a row of >= 1024 nonzeros
    possible under the hint."""
    import ctypes
    lib = capi.hip()
    A = capi.ALGO

    def panels(algo, M, K, N, nnz, hint=-1):
        off = ctypes.c_longlong(-1)
        P = lib.csrspmm_workspace_panel_info(A[algo], M, K, N, nnz, hint, ctypes.byref(off))
        if P > 0:
            # the decision word sits inside the workspace the call is sized for
            assert 0 <= off.value < lib.csrspmm_workspace_bytes_ex(A[algo], M, K, N, nnz, hint)
        return P

    M, nnz = 262144, 8453223
    assert panels("WarpPerRowSmemFp4", M, 262144, 128, nnz) == 64    # XL: 128 MiB B
    assert panels("WarpPerRowSmemFp4", M, 262144, 64, nnz) == 32     # 64 MiB: 32 panels
    assert panels("WarpPerRowSmemFp4", M, 131072, 64, nnz) == 0      # 32 MiB: 16 panels, too few
    assert panels("WarpPerRowSmemFp4", M, 65536, 128, nnz) == 0      # 32 MiB
    assert panels("WarpPerRowSmem", M, 262144, 128, nnz) == 64       # scalar columns from N = 128
    assert panels("WarpPerRowSmem", M, 262144, 64, nnz) == 0         # but not at N = 64
    assert panels("Auto", M, 262144, 64, nnz) == 32                  # Auto takes float4 for them
    assert panels("Auto", M, 262144, 64, nnz, 1023) == 0             # unless no row can use them
    assert panels("Auto", M, 262144, 128, nnz) == 64
    assert panels("WarpPerRowSmemFp4", M, 65536, 256, nnz) == 0      # 16 MiB bands: column slices
    assert panels("WarpPerRowSmemFp4", M, 131072, 256, nnz) == 64    # 32 MiB bands: panels
    assert panels("WarpPerRowSmemFp4", M, 262144, 512, nnz) == 0     # N > 256
    assert panels("WarpPerRowSmemFp4", M, 262144, 128, nnz, 1023) == 0  # no row of 1024
    assert panels("WarpPerRowSmemFp4", M, 262144, 128, nnz, 1024) == 64
    assert panels("Naive", M, 262144, 128, nnz) == 0
    # K not a power of two: fewer panels than the count, the last one partial
    assert 16 < panels("WarpPerRowSmemFp4", 3000, 150000, 128, 200000) <= 32


def test_leading_dim_rule():
    """The row stride a tensor operand is passed with: stride(0) for any
    operand of two rows or more (a one-column view of a wider tensor keeps
    its parent's row stride), the width for a single row; a row stride below
    the width, or a non-unit column stride, is rejected."""
    import torch

    X = torch.zeros(10, 4)
    assert capi.leading_dim(X) == 4
    assert capi.leading_dim(X[:, 2:3]) == 4           # one column, strides (4, 1)
    assert capi.leading_dim(X[:, :3]) == 4            # padded rows
    assert capi.leading_dim(X[3:4, :3]) == 3          # one row: the width
    assert capi.leading_dim(torch.zeros(0, 5)) == 5
    assert capi.leading_dim(torch.zeros(6, 0)) == 1   # no columns: nothing to address
    assert capi.leading_dim(torch.from_numpy(__import__("numpy").zeros((5, 0), "f4"))) == 1
    assert capi.leading_dim(torch.zeros(1, 0)) == 1
    assert capi.leading_dim(torch.zeros(7, 1)) == 1
    with pytest.raises(ValueError, match="row stride"):
        capi.leading_dim(torch.zeros(1, 4).expand(3, 4))
    with pytest.raises(ValueError, match="row-major"):
        capi.leading_dim(torch.zeros(4, 3).t())


def test_noalloc_rejects_beyond_scratch_without_device():
    """The size check runs on the host before any device call: a problem
    whose base workspace exceeds the 128 MiB scratch is rejected (null
    pointers are never reached)."""
    lib = capi.hip()
    M, K, N, nnz = 1024, 1, 1100, 8_000_000
    assert lib.csrspmm_workspace_bytes(capi.ALGO["Auto"], M, N, nnz) > 128 << 20
    st = lib.csrspmm_spmm_f32_noalloc(capi.ALGO["Auto"], M, K, N, nnz, None, None, None, -1, None,
                                      N, None, N, 1.0, 0.0, 0, None)
    assert st == -6
    assert "no-allocation scratch" in lib.csrspmm_status_string(st).decode()


def test_kernels_h_symbols_exported():
    """The reference's six kernel declarations (include/csrspmm/kernels.h)
    have their host-side launch stubs in libcsrspmm_hip.so, so HIP code that
    declares and launches them links against the library."""
    header = open(os.path.join(os.path.dirname(LIB_DIR), "..", "include", "csrspmm",
                               "kernels.h")).read()
    names = re.findall(r"__global__ void (\w+)\(", header)
    assert len(names) == 6
    out = __import__("subprocess").run(["nm", "-D", "--defined-only",
                                        os.path.join(LIB_DIR, "libcsrspmm_hip.so")],
                                       capture_output=True, text=True, check=True).stdout
    for n in names:
        assert re.search(rf"_ZN7csrspmm6kernel\d+__device_stub__{n}E", out), n
