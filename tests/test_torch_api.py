"""The torch_csrspmm drop-in imports on a CPU-only machine, exposes the
reference's five entry points with the reference's argument lists
(torch_csrspmm/__init__.py:10-23), and raises the reference's RuntimeError for
host tensors (torch_csrspmm/torch_csrspmm_naive.cpp:22-25)."""
import inspect

import pytest
import torch

import torch_csrspmm as tc

SIGS = {
    "csrspmm_naive": ["A_rowptr", "A_colidx", "A_values", "B", "alpha", "beta"],
    "csrspmm_warp_per_row": ["A_rowptr", "A_colidx", "A_values", "B", "alpha", "beta"],
    "csrspmm_warp_per_row_fp4": ["A_rowptr", "A_colidx", "A_values", "B", "alpha", "beta"],
    "csrspmm_warp_per_row_smem": ["A_rowptr", "A_colidx", "A_values", "A_max_row_nnz", "B",
                                  "alpha", "beta"],
    "csrspmm_warp_per_row_smem_fp4": ["A_rowptr", "A_colidx", "A_values", "A_max_row_nnz", "B",
                                      "alpha", "beta"],
}


def test_entry_points_and_signatures():
    assert sorted(tc.__all__) == sorted(SIGS)
    for name in tc.EXTRAS:
        assert hasattr(tc, name)
    for name, params in SIGS.items():
        assert list(inspect.signature(getattr(tc, name)).parameters) == params
        assert hasattr(tc._C, name)
    assert tc._C.__file__.startswith(tc.__file__.rsplit("/", 1)[0])  # in-tree extension


def cpu_inputs():
    rowptr = torch.tensor([0, 1, 2], dtype=torch.int32)
    colidx = torch.tensor([0, 1], dtype=torch.int32)
    vals = torch.ones(2)
    B = torch.ones(2, 4)
    return rowptr, colidx, vals, B


@pytest.mark.parametrize("name", sorted(SIGS))
def test_host_tensors_raise(name):
    rowptr, colidx, vals, B = cpu_inputs()
    fn = getattr(tc, name)
    args = (rowptr, colidx, vals, 1, B, 1.0, 0.0) if "smem" in name else (rowptr, colidx, vals, B, 1.0, 0.0)
    with pytest.raises(RuntimeError, match="A_row_ptr must be a CUDA tensor"):
        fn(*args)


def test_extras_raise_on_host_tensors():
    rowptr, colidx, vals, B = cpu_inputs()
    with pytest.raises(RuntimeError, match="A_row_ptr must be a CUDA tensor"):
        tc.csrspmm_auto(rowptr, colidx, vals, B, 1.0, 0.0)
    with pytest.raises(RuntimeError, match="A_row_ptr must be a CUDA tensor"):
        tc.csrspmm_spmm_out(rowptr, colidx, vals, B, torch.zeros(2, 4), 1.0, 0.0)
    with pytest.raises(RuntimeError, match="CSR tensors must be CUDA tensors"):
        tc.CsrSpmmPlan(rowptr, colidx, vals, 2)


@pytest.mark.filterwarnings("ignore:Sparse CSR tensor support")
def test_sparse_csr_entry_checks_on_host():
    A = torch.eye(3).to_sparse_csr()
    with pytest.raises(RuntimeError, match="CUDA"):
        tc.from_sparse_csr(A)
    with pytest.raises(RuntimeError, match="sparse_csr"):
        tc.from_sparse_csr(torch.eye(3))
    with pytest.raises(RuntimeError, match="CUDA"):
        tc.dense_to_csr(torch.eye(3))


def test_import_name_and_setup_extension():
    """`import torch_csrspmm` resolves to the top-level package of this tree
    (the reference's import name, torch_csrspmm/__init__.py:1-7), and
    setup.py declares its extension as the reference's setup.py does
    (setup.py:79-86: torch_csrspmm._C), built from the committed C++ source
    against the in-tree kernel library (a CppExtension: no CUDA, no hipify)."""
    import importlib.util
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    assert os.path.dirname(tc.__file__) == os.path.join(root, "torch_csrspmm")
    spec = importlib.util.spec_from_file_location("csrspmm_setup", os.path.join(root, "setup.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # the setup() call is guarded by __main__
    (ext,) = mod.ext_modules()
    assert ext.name == "torch_csrspmm._C"
    assert all(os.path.exists(os.path.join(root, s)) for s in ext.sources)
    assert "csrspmm_hip" in ext.libraries
    assert not any("cuda" in s.lower() for s in ext.sources)
