"""The benchmark / parity configurations (BASELINE.json "configs"), pinned.

Row-length laws and seeds are fixed here so C++ and Python regenerate the
same bits; the XL law is Zipf-Mandelbrot P(L=k) ~ (k - 0.7)^-1.5 on
{1..16384}, which keeps the exponent 1.5, the 16,384 cap and a mean of about
32 nonzeros per row (a plain truncated Zipf(1.5) on that support has mean 98;
it is kept as the secondary config "xl98").
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import gen


@dataclass(frozen=True)
class Config:
    name: str
    kind: str           # uniform | powerlaw | rmat
    N: int              # columns of B and C
    seed: int
    params: dict = field(default_factory=dict)
    description: str = ""

    def csr(self) -> gen.Csr:
        p = self.params
        if self.kind == "uniform":
            return gen.uniform(p["M"], p["K"], p["per_row"], self.seed)
        if self.kind == "powerlaw":
            return gen.powerlaw(p["M"], p["K"], p["exponent"], p["shift"], p["cap"], self.seed)
        if self.kind == "rmat":
            return gen.rmat(p["scale"], p["samples"], p["a"], p["b"], p["c"], self.seed)
        raise ValueError(self.kind)

    def K(self) -> int:
        """Columns of A (rows of B), without generating the matrix."""
        return 1 << self.params["scale"] if self.kind == "rmat" else self.params["K"]

    def B(self, K: int):
        return gen.dense(self.seed, gen.TAG_B, K, self.N)

    def C0(self, M: int):
        return gen.dense(self.seed, gen.TAG_C0, M, self.N)


CONFIGS = {
    "host": Config("host", "uniform", 32, 1, dict(M=1024, K=1024, per_row=10),
                   "1024^2, 10 nnz/row (1%), N=32"),
    "medium": Config("medium", "uniform", 128, 2, dict(M=16384, K=16384, per_row=82),
                     "16384^2, 82 nnz/row (0.5%), N=128"),
    "large": Config("large", "uniform", 256, 3, dict(M=65536, K=65536, per_row=66),
                    "65536^2, 66 nnz/row (0.1%), N=256"),
    "xl": Config("xl", "powerlaw", 128, 4,
                 dict(M=262144, K=262144, exponent=1.5, shift=0.7, cap=16384),
                 "262144^2 power-law rows (Zipf-Mandelbrot 1.5, shift 0.7, cap 16384), N=128"),
    "rmat": Config("rmat", "rmat", 64, 5,
                   dict(scale=20, samples=1 << 24, a=0.57, b=0.19, c=0.19),
                   "RMAT 2^20 (a .57, b .19, c .19), 2^24 samples deduplicated, N=64"),
    "rmat512": Config("rmat512", "rmat", 512, 5,
                      dict(scale=20, samples=1 << 24, a=0.57, b=0.19, c=0.19),
                      "same RMAT matrix, N=512"),
    "xl98": Config("xl98", "powerlaw", 128, 4,
                   dict(M=262144, K=262144, exponent=1.5, shift=0.0, cap=16384),
                   "262144^2 truncated Zipf(1.5) rows (mean ~98), N=128"),
}


def bytes_alg(M: int, nnz: int, N: int, beta_nonzero: bool = False) -> int:
    """Gather-model bytes per SpMM: rowptr + (col, val) + one fp32 B row per
    nonzero + C written (and read when beta != 0)."""
    return 4 * (M + 1) + 8 * nnz + 4 * nnz * N + 4 * M * N * (2 if beta_nonzero else 1)


def bytes_min(M: int, nnz: int, N: int, U: int, beta_nonzero: bool = False) -> int:
    """Compulsory bytes per SpMM: as bytes_alg, with each of the U distinct
    referenced B rows read once instead of once per nonzero."""
    return 4 * (M + 1) + 8 * nnz + 4 * U * N + 4 * M * N * (2 if beta_nonzero else 1)


def distinct_columns(colidx, K: int) -> int:
    """U: the number of distinct column indices of A (the B rows it reads)."""
    import numpy as np

    if colidx.size == 0:
        return 0
    return int(np.count_nonzero(np.bincount(colidx, minlength=K)))


def flops(nnz: int, N: int) -> int:
    return 2 * nnz * N
