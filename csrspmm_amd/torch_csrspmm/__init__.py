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
# Beyond the reference's five: the variant picked from N, an in-place product
# with a real beta, and a stored plan for repeated products with one A.
EXTRAS = ["csrspmm_auto", "csrspmm_spmm_out", "CsrSpmmPlan"]


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


def csrspmm_auto(A_rowptr, A_colidx, A_values, B, alpha, beta):
    """As the five entry points, with the variant picked from N."""
    return _C.csrspmm_auto(A_rowptr, A_colidx, A_values, B, alpha, beta)


def csrspmm_spmm_out(A_rowptr, A_colidx, A_values, B, C, alpha, beta, algo="Auto"):
    """C = alpha * A @ B + beta * C in place (C is read when beta != 0); returns C."""
    return _C.csrspmm_spmm_out(A_rowptr, A_colidx, A_values, B, C, alpha, beta, algo)


class CsrSpmmPlan:
    """A stored plan for repeated products with one CSR matrix A (K columns).

        plan = CsrSpmmPlan(rowptr, colidx, values, K)        # algo="Auto"
        C = plan.spmm(B, alpha, beta)          # new C, like the entry points
        plan.spmm_out(B, C, alpha, beta)       # in place, C = alpha*A@B + beta*C

    The CSR tensors are used in place and must not be modified while the
    plan is alive; n_hint is the expected number of columns of B.
    """

    def __init__(self, A_rowptr, A_colidx, A_values, K, algo="Auto", n_hint=0):
        self._plan = _C.CsrSpmmPlan(A_rowptr, A_colidx, A_values, int(K), algo, int(n_hint))

    def spmm(self, B, alpha=1.0, beta=0.0):
        return self._plan.spmm(B, alpha, beta)

    def spmm_out(self, B, C, alpha=1.0, beta=0.0):
        return self._plan.spmm_out(B, C, alpha, beta)

    @property
    def algorithm(self):
        return self._plan.algorithm

    @property
    def device_bytes(self):
        return self._plan.device_bytes

    @property
    def panelized_rows(self):
        return self._plan.panelized_rows
