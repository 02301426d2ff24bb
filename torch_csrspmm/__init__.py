"""Drop-in for the reference's ``torch_csrspmm`` package, under its import
name (reference torch_csrspmm/__init__.py:1-23): the same five entry points
with the same argument order, each returning a new ``[M, N]`` fp32 tensor with
B's options, computed by the gfx950 HIP kernels of ``libcsrspmm_hip.so``.

    import torch_csrspmm
    C = torch_csrspmm.csrspmm_warp_per_row_fp4(rowptr, colidx, vals, B, alpha, beta)

The extension ``torch_csrspmm._C`` is built in place by
``python -m csrspmm_amd.build`` or ``python setup.py build_ext --inplace``
(after ``python -m csrspmm_amd.build hip``, which builds the kernels it
links).  The launch goes on the current HIP stream of B's device and is
asynchronous.  There is no CPU path: importing this module raises if the
extension is not built.
"""
import torch  # noqa: F401  (loads torch's HIP runtime before the extension binds to it)

try:
    from . import _C
except ImportError as exc:  # pragma: no cover - exercised only when the build is missing
    raise ImportError(
        "torch_csrspmm: the HIP extension _C is not built; run "
        "`python -m csrspmm_amd.build` (needs hipcc for gfx950)") from exc

__all__ = [
    "csrspmm_naive",
    "csrspmm_warp_per_row",
    "csrspmm_warp_per_row_smem",
    "csrspmm_warp_per_row_fp4",
    "csrspmm_warp_per_row_smem_fp4",
]
# Beyond the reference's five: the variant picked from the shape, an in-place product
# with a real beta, a stored plan for repeated products with one A, and
# device-side CSR tooling (torch.sparse_csr input, dense -> CSR, longest row).
EXTRAS = ["csrspmm_auto", "csrspmm_spmm_out", "CsrSpmmPlan", "csrspmm_sparse", "from_sparse_csr",
          "dense_to_csr", "csr_max_row_nnz"]


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


def csrspmm_auto(A_rowptr, A_colidx, A_values, B, alpha, beta, max_row_nnz=-1):
    """As the five entry points, with the variant picked from the shape
    (csrspmm_resolve_algorithm_ex).  max_row_nnz, the longest row when known
    (-1: unknown), is a scheduling hint only: with at most 256 a mid-sized
    product runs as one launch."""
    return _C.csrspmm_auto(A_rowptr, A_colidx, A_values, B, alpha, beta, max_row_nnz)


def csrspmm_spmm_out(A_rowptr, A_colidx, A_values, B, C, alpha, beta, algo="Auto", max_row_nnz=-1):
    """C = alpha * A @ B + beta * C in place (C is read when beta != 0); returns C.
    max_row_nnz as for csrspmm_auto."""
    return _C.csrspmm_spmm_out(A_rowptr, A_colidx, A_values, B, C, alpha, beta, algo, max_row_nnz)


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


def from_sparse_csr(A):
    """(rowptr, colidx, values, K) of a torch.sparse_csr CUDA tensor, ready for
    the entry points, with no host sync: int32 indices are used in place
    (zero-copy) and int64 indices are narrowed on the device.  A's shapes
    must fit int32, which makes the narrowing exact for a valid CSR."""
    if A.layout != torch.sparse_csr:
        raise RuntimeError("A must be a torch.sparse_csr tensor")
    if not A.is_cuda:
        raise RuntimeError("A must be a CUDA tensor")
    if A.dim() != 2:
        raise RuntimeError("A must be 2-D (no batch dimensions)")
    M, K = A.shape
    vals = A.values()
    if M >= 2**31 - 1 or K > 2**31 - 1 or vals.numel() > 2**31 - 1:
        raise RuntimeError("A's sizes must fit int32")
    if vals.dtype != torch.float32:
        raise RuntimeError("A_values must be float32")
    rowptr = _C.indices_to_int32(A.crow_indices())
    colidx = _C.indices_to_int32(A.col_indices())
    return rowptr, colidx, vals.contiguous(), K


def csrspmm_sparse(A, B, alpha=1.0, beta=0.0, algo="Auto"):
    """C = alpha * A @ B for a torch.sparse_csr A (a new C; beta scales a zero
    C, as in the five entry points)."""
    rowptr, colidx, vals, K = from_sparse_csr(A)
    if B.dim() != 2 or B.size(0) != K:
        raise RuntimeError("B must be [K, N] with K = A.shape[1]")
    return _C.csrspmm_forward(rowptr, colidx, vals, B, alpha, beta, algo)


def dense_to_csr(D, tol=0.0):
    """Device dense -> CSR (rowptr, colidx, values), keeping |v| > tol in
    row-major order like the reference's host dense2csr; one host sync."""
    return tuple(_C.dense_to_csr(D, float(tol)))


def csr_max_row_nnz(rowptr):
    """Longest row as a one-element int32 CUDA tensor (no host sync)."""
    return _C.csr_max_row_nnz(rowptr)
