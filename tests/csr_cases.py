"""Synthetic CSR matrices with chosen row lengths, for the GPU parity tests
of the long-row paths (column panels, column slices), and the library's
documented rule for which rows it sums whole."""
import numpy as np


def whole_row_max(nnz, shares=False):
    """Longest row the warp-per-row family sums in one piece (in CSR order,
    so bit-identical to the fp32 restatement) for a matrix of nnz nonzeros:
    rows shorter than two segments.  The segment is 256 nonzeros, halved
    (down to 32) while the matrix holds fewer than 4096 segments' worth, so
    that a small matrix's long rows still split over the GPU.  A call that
    splits its long rows by XCD (shares, capi.call_shares) sums only rows
    of at most 128 nonzeros whole."""
    if shares:
        return 128
    seg = 256
    while seg > 32 and nnz // seg < 4096:
        seg //= 2
    return 2 * seg - 1


def csr_from_lengths(lens, K, seed, narrow=None, unsorted_rows=()):
    """Rows of the given lengths, columns uniform without replacement in
    [0, K) (or in narrow[r] = (lo, hi) for chosen rows), sorted unless the
    row is in unsorted_rows; values U(-1, 1) exact in fp32."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    rowptr = np.zeros(lens.size + 1, dtype=np.int32)
    rowptr[1:] = np.cumsum(lens)
    cols = []
    for r, L in enumerate(lens):
        lo, hi = (narrow or {}).get(r, (0, K))
        c = rng.choice(hi - lo, size=int(L), replace=False).astype(np.int32) + lo
        c.sort()
        if r in unsorted_rows:
            rng.shuffle(c)
        cols.append(c)
    colidx = np.concatenate(cols) if cols else np.zeros(0, np.int32)
    vals = (rng.integers(0, 1 << 24, size=colidx.size) * 2.0 ** -23 - 1.0).astype(np.float32)
    return rowptr, colidx.astype(np.int32), vals


def mixed_lengths(seed, M=3000):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 40, size=M)
    special = [1023, 1024, 1025, 2047, 2048, 2049, 3000, 4096, 5000, 20000, 256, 257, 511, 512, 767,
               768, 0, 1, 16384]
    pos = rng.choice(M, size=len(special), replace=False)
    lens[pos] = special
    lens[-1] = 6000  # a long row at the very end
    return lens


def whole_row_limit(algo, rowptr, K, N, hint=-1, shares=None):
    """whole_row_max for a per-call product of this shape through the
    library (shares=None: as the library decides, capi.call_shares)."""
    nnz = int(rowptr[-1])
    if shares is None:
        from csrspmm_amd import capi
        shares = capi.call_shares(algo, int(rowptr.size - 1), int(K), int(N), nnz, hint)
    return whole_row_max(nnz, shares)
