"""Full-size checks that need no oracle: identities and closed forms over
the whole output, for every variant and config path (test_gpu_parity.py
holds the every-element fp64 oracle comparison of the BASELINE configs).

* Exact identities, bit for bit over every element of C: B scaled by 2 gives
  2 C (every product and partial sum scales by a power of two, exactly);
  B's columns permuted give C's columns permuted (each output column is
  computed on its own, in an order that does not depend on its position);
  alpha = 0.5 gives C / 2.  These hold on every path (panels, slices,
  segments, merge blocks) and catch a column mixed up with another, a lane
  reading another lane's data, results that depend on timing (a race, an
  uninitialised workspace entry) or on where B and C sit in memory.
* Column checksums against a closed form: sum_i C[i, j] = sum_k w[k] B[k, j]
  with w[k] the sum of A's values in column k, computed in fp64 on the host
  from A alone.  The 1e-5 elementwise bar implies
  |colsum error| <= 1e-5 * sum_k |w|[k] |B[k, j]| (|w| from |values|), so
  every row of the full matrix takes part: a row or a long segment dropped
  or counted twice anywhere shows (a dropped 400-nonzero row measured 27x
  the bound on a small case).  Small value errors are left to the oracle
  comparison and the identities.
"""
import functools

import numpy as np
import pytest
import torch

from csrspmm_amd import ALGORITHMS, capi, configs

pytestmark = pytest.mark.gpu

TOL = 1e-5


@functools.lru_cache(maxsize=None)
def matrix(cfg_name):
    return configs.CONFIGS[cfg_name].csr()


@functools.lru_cache(maxsize=2)
def colsum_closed_form(cfg_name):
    """(want, bound) per output column, fp64, from A's column sums and B."""
    cfg = configs.CONFIGS[cfg_name]
    a = matrix(cfg_name)
    B = cfg.B(a.K)
    vals = a.vals.astype(np.float64)
    w = np.bincount(a.colidx, weights=vals, minlength=a.K)
    w_abs = np.bincount(a.colidx, weights=np.abs(vals), minlength=a.K)
    want = np.zeros(cfg.N)
    bound = np.zeros(cfg.N)
    for k0 in range(0, a.K, 65536):  # B in fp64 a band of rows at a time
        Bk = B[k0:k0 + 65536].astype(np.float64)
        want += w[k0:k0 + 65536] @ Bk
        bound += w_abs[k0:k0 + 65536] @ np.abs(Bk)
    return want, bound


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def spmm(algo, drp, dci, dva, dB, M, alpha=1.0):
    C = torch.full((M, dB.shape[1]), float("nan"), device=dB.device)
    capi.spmm(algo, drp, dci, dva, dB, C, alpha, 0.0)
    torch.cuda.synchronize()
    return C


@pytest.mark.parametrize("algo", ("Auto",) + ALGORITHMS)
@pytest.mark.parametrize("cfg_name", ["xl", "large", "rmat512"])
def test_exact_identities(cfg_name, algo, gpu):
    cfg = configs.CONFIGS[cfg_name]
    a = matrix(cfg_name)
    print(f"[fullsize] identities {cfg_name} {algo} M={a.M} nnz={a.nnz} N={cfg.N}", flush=True)
    drp, dci, dva = dev_t(a.rowptr, gpu), dev_t(a.colidx, gpu), dev_t(a.vals, gpu)
    dB = dev_t(cfg.B(a.K), gpu)
    C = spmm(algo, drp, dci, dva, dB, a.M)
    assert not torch.isnan(C).any()
    C2 = spmm(algo, drp, dci, dva, dB * 2.0, a.M)
    assert torch.equal(C2, C * 2.0), "A (2B) != 2 (A B) bit for bit"
    del C2
    perm = torch.from_numpy(np.random.default_rng(3).permutation(cfg.N)).to(gpu)
    C3 = spmm(algo, drp, dci, dva, dB[:, perm].contiguous(), a.M)
    assert torch.equal(C3, C[:, perm]), "permuted columns of B do not permute C"
    del C3
    C4 = spmm(algo, drp, dci, dva, dB, a.M, alpha=0.5)
    assert torch.equal(C4, C * 0.5), "alpha = 0.5 is not C / 2 bit for bit"


@pytest.mark.parametrize("cfg_name", ["xl", "xl98", "rmat", "rmat512", "large"])
def test_column_checksums(cfg_name, gpu):
    """Every variant (and Auto) on the full matrix: each output column's sum
    against the closed form."""
    cfg = configs.CONFIGS[cfg_name]
    a = matrix(cfg_name)
    want, bound = colsum_closed_form(cfg_name)
    drp, dci, dva = dev_t(a.rowptr, gpu), dev_t(a.colidx, gpu), dev_t(a.vals, gpu)
    dB = dev_t(cfg.B(a.K), gpu)
    for algo in ("Auto",) + ALGORITHMS:
        print(f"[fullsize] checksums {cfg_name} {algo} M={a.M} nnz={a.nnz} N={cfg.N}", flush=True)
        C = spmm(algo, drp, dci, dva, dB, a.M)
        got = C.double().sum(0).cpu().numpy()
        del C
        err = np.abs(got - want)
        assert (err <= TOL * bound).all(), \
            f"{cfg_name} {algo}: column sums off, worst {np.max(err / bound):.3g} of the 1e-5 bound"


@pytest.mark.parametrize("cfg_name,algo,expect", [
    ("xl", "Auto", "long"), ("xl", "WarpPerRowSmem", "long"), ("xl98", "Auto", "long"),
    ("rmat", "WarpPerRowFp4", "skewed")])
def test_panel_decision(cfg_name, algo, expect, gpu):
    """The per-call schedule's decision on the bench configs: the power-law
    configs (columns uniform) panelize every row of >= 1024 nonzeros, all
    under the nnz / 4096 cap; R-MAT's hot columns read as skewed."""
    cfg = configs.CONFIGS[cfg_name]
    a = matrix(cfg_name)
    print(f"[fullsize] panel decision {cfg_name} {algo}", flush=True)
    C = torch.empty((a.M, cfg.N), device=gpu)
    nl = capi.panelized_rows(algo, dev_t(a.rowptr, gpu), dev_t(a.colidx, gpu), dev_t(a.vals, gpu),
                             dev_t(cfg.B(a.K), gpu), C)
    long_rows = int(np.count_nonzero(np.diff(a.rowptr) >= 1024))
    if expect == "long":
        assert long_rows <= -(-a.nnz // 4096)
        assert nl == long_rows
    else:
        assert nl == 0

