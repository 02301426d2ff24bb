"""The host side of csrspmm_amd.reference_sweep (no GPU): per-variant means
over the 20 shapes and the summary beside the reference's published means."""
from csrspmm_amd import reference_sweep as rs


def fake_rows():
    rows = []
    for i, (name, M, N, K) in enumerate(rs.SHAPES):
        for j, d in enumerate(rs.DENSITIES):
            for algo in rs.VARIANTS:
                rows.append({"sweep": "cpp", "case": name, "M": M, "N": N, "K": K, "density": d,
                             "algo": algo, "gflops": 100.0 * (i + 1) + j})
            rows.append({"sweep": "torch", "case": name, "M": M, "N": N, "K": K, "density": d,
                         "algo": "WarpPerRowFp4", "gflops": 466.0})
    return rows


def test_sweep_grid_is_the_reference_grid():
    # 4 shapes x 5 densities, as in the reference's two benchmark scripts
    assert len(rs.SHAPES) * len(rs.DENSITIES) == 20
    assert set(rs.VARIANTS) <= set(rs.PUBLISHED_CPP) and set(rs.VARIANTS) <= set(rs.PUBLISHED_TORCH)


def test_means_over_shapes():
    m = rs.means(fake_rows(), "cpp")
    assert set(m) == set(rs.VARIANTS)
    # mean of 100*(i+1)+j over i in 0..3, j in 0..4
    assert abs(m["Naive"] - (250.0 + 2.0)) < 1e-9
    assert rs.means(fake_rows(), "torch") == {"WarpPerRowFp4": 466.0}


def test_markdown_summary():
    md = rs.markdown(fake_rows(), "test GPU", "python -m csrspmm_amd.reference_sweep")
    assert "| WarpPerRowFp4 | 252 | 727 | 0.35× |" in md
    assert "| WarpPerRowFp4 | 466 | 466 | 1.00× |" in md
    assert md.count("| cpp |") == 20 and md.count("| torch |") == 20
