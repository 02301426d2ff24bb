"""Pins the synthetic-input generators: the C++ counter-based stream equals
its numpy restatement element by element, generated CSR matrices have the
stated structure, and the BASELINE configs reproduce committed digests."""
import json
import os

import numpy as np
import pytest

from csrspmm_amd import configs, gen

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_dense_stream_matches_numpy():
    for seed, tag in [(0, 4), (5, 4), (123456789, 5)]:
        out = gen.dense(seed, tag, 37, 29, first=1000)
        key = gen.key_np(seed, tag)
        want = gen.u11_np(gen.rand_np(key, np.arange(1000, 1000 + out.size)))
        assert np.array_equal(out.ravel().view(np.uint32), want.view(np.uint32))
    assert -1.0 <= out.min() and out.max() < 1.0


def test_splitmix64_known_values():
    # SplitMix64 with state 0: the published first outputs of the generator.
    first = gen.mix64_np(np.arange(1, 4, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15))
    assert [hex(int(x)) for x in first] == ["0xe220a8397b1dcdaf", "0x6e789e6aa1b965f4",
                                            "0x6c45d188009454f"]


def check_structure(a, per_row=None, cap=None):
    lens = np.diff(a.rowptr)
    assert a.rowptr[0] == 0 and a.rowptr[-1] == a.nnz and np.all(lens >= 0)
    assert a.max_row_nnz == lens.max()
    assert np.all((a.colidx >= 0) & (a.colidx < a.K))
    # strictly increasing inside every row (sorted, no duplicates)
    d = np.diff(a.colidx.astype(np.int64))
    row_start = np.zeros(a.nnz, dtype=bool)
    row_start[a.rowptr[1:-1][a.rowptr[1:-1] < a.nnz]] = True
    assert np.all((d > 0) | row_start[1:])
    if per_row is not None:
        assert np.all(lens == per_row)
    if cap is not None:
        assert lens.max() <= cap and lens.min() >= 1
    assert np.all(np.abs(a.vals) < 1.0)
    key = gen.key_np(0, gen.TAG_VALS)
    del key


def test_uniform_and_ragged_structure():
    a = gen.uniform(500, 700, 33, seed=3)
    check_structure(a, per_row=33)
    b = gen.ragged(400, 300, 0, 300, seed=4)
    check_structure(b)
    assert np.diff(b.rowptr).min() == 0
    # values follow the documented stream (seed, VALS) by CSR position
    key = gen.key_np(4, gen.TAG_VALS)
    assert np.array_equal(b.vals.view(np.uint32),
                          gen.u11_np(gen.rand_np(key, np.arange(b.nnz))).view(np.uint32))
    # full rows (per_row == K) are every column once
    c = gen.uniform(3, 50, 50, seed=1)
    assert np.array_equal(c.colidx.reshape(3, 50), np.tile(np.arange(50), (3, 1)))


def test_uniform_columns_are_uniform():
    a = gen.uniform(4000, 100, 10, seed=9)
    counts = np.bincount(a.colidx, minlength=100)
    expected = a.nnz / 100
    chi2 = ((counts - expected) ** 2 / expected).sum()
    assert chi2 < 200  # 99 dof; a gross bias would be far above


def test_powerlaw_law():
    a = gen.powerlaw(200000, 262144, 1.5, 0.7, 16384, seed=11)
    check_structure(a, cap=16384)
    lens = np.diff(a.rowptr)
    k = np.arange(1, 16385, dtype=np.float64)
    w = (k - 0.7) ** -1.5
    w /= w.sum()
    assert abs(lens.mean() - (k * w).sum()) / (k * w).sum() < 0.1
    assert abs((lens == 1).mean() - w[0]) < 0.01
    assert abs((lens == 2).mean() - w[1]) < 0.01


def test_rmat_small():
    a = gen.rmat(10, 20000, 0.57, 0.19, 0.19, seed=2)
    check_structure(a)
    assert a.M == a.K == 1024
    # skew: row 0 (all-"a" quadrant path) is the heaviest region
    lens = np.diff(a.rowptr)
    assert lens[:64].sum() > lens[-64:].sum()


def test_generator_rejects_bad_parameters():
    with pytest.raises(ValueError):
        gen.uniform(10, 5, 6, seed=1)  # more per row than columns
    with pytest.raises(ValueError):
        gen.ragged(10, 5, 3, 2, seed=1)
    with pytest.raises(ValueError):
        gen.powerlaw(10, 100, 1.5, 1.0, 50, seed=1)


@pytest.mark.parametrize("name", ["host", "medium", "large", "xl", "rmat"])
def test_config_digests(name):
    """The BASELINE configs regenerate bit for bit (FNV-1a over rowptr, colidx,
    values), so every machine benchmarks and checks the same matrices."""
    with open(os.path.join(GOLDEN, "config_digests.json")) as f:
        pinned = json.load(f)[name]
    a = configs.CONFIGS[name].csr()
    assert (a.M, a.nnz, a.max_row_nnz) == (pinned["M"], pinned["nnz"], pinned["max_row_nnz"])
    assert a.digest() == pinned["digest"]
    B = configs.CONFIGS[name].B(a.K)
    assert gen.key_np(configs.CONFIGS[name].seed, gen.TAG_B) is not None
    first = gen.u11_np(gen.rand_np(gen.key_np(configs.CONFIGS[name].seed, gen.TAG_B),
                                   np.arange(16)))
    assert np.array_equal(B.ravel()[:16], first)
