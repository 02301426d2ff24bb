"""Drop-in for the reference's ``torch_csrspmm`` package
(reference torch_csrspmm/__init__.py:10-23): the same five entry points with
the same argument order, each returning a new ``[M, N]`` fp32 tensor with B's
options, computed by the gfx950 HIP kernels of ``libcsrspmm_hip.so``.

    import csrspmm_amd.torch_csrspmm as torch_csrspmm
    C = torch_csrspmm.csrspmm_warp_per_row_fp4(rowptr, colidx, vals, B, alpha, beta)

The launch goes on the current HIP stream of B's device and is asynchronous.
There is no CPU path: importing this module raises if the extension is not
built (``python -m csrspmm_amd.build``).
"""
import torch  # noqa: F401  (loads torch's HIP runtime before the extension binds to it)

try:
    from . import _C
except ImportError as exc:  # pragma: no cover - exercised only when the build is missing
    raise ImportError(
        "csrspmm_amd.torch_csrspmm: the HIP extension _C is not built; run "
        "`python -m csrspmm_amd.build` (needs hipcc for gfx950)") from exc

__all__ = [
    "csrspmm_naive",
    "csrspmm_warp_per_row",
    "csrspmm_warp_per_row_smem",
    "csrspmm_warp_per_row_fp4",
    "csrspmm_warp_per_row_smem_fp4",
]


def csrspmm_naive(A_rowptr, A_colidx, A_values, B, alpha, beta):
    return _C.csrspmm_naive(A_rowptr, A_colidx, A_values, B, alpha, beta)


def csrspmm_warp_per_row(A_rowptr, A_colidx, A_values, B, alpha, beta):
    return _C.csrspmm_warp_per_row(A_rowptr, A_colidx, A_values, B, alpha, beta)


def csrspmm_warp_per_row_smem(A_rowptr, A_colidx, A_values, A_max_row_nnz, B, alpha, beta):
    return _C.csrspmm_warp_per_row_smem(A_rowptr, A_colidx, A_values, A_max_row_nnz, B, alpha, beta)


def csrspmm_warp_per_row_fp4(A_rowptr, A_colidx, A_values, B, alpha, beta):
    return _C.csrspmm_warp_per_row_fp4(A_rowptr, A_colidx, A_values, B, alpha, beta)


def csrspmm_warp_per_row_smem_fp4(A_rowptr, A_colidx, A_values, A_max_row_nnz, B, alpha, beta):
    return _C.csrspmm_warp_per_row_smem_fp4(A_rowptr, A_colidx, A_values, A_max_row_nnz, B, alpha,
                                            beta)
