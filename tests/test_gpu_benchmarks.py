"""The reference's benchmark helpers (benchmark_spmv_case, benchmark_spmm_case,
benchmark_spmm_opt_case, benchmark_spmm_opt_alg2_case): their result-dict
keys are the reference's, the torch leg runs, the cuSPARSE leg reports
itself unavailable, and the timed operator's output matches the CPU oracle
on the same matrix (sparse_operations/benchmarks.py:343-505,
spmm_csr.py:3619-4045, spmm_csr_opt_alg2.py:1024-1149)."""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from oracle import csr_oracle as O
from tests._helpers import np_, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float64: 1e-12, torch.complex64: 1e-5, torch.complex128: 1e-12}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["f32", "f64", "c64"])
@pytest.mark.parametrize("op", ["non", "trans", "conj"])
def test_benchmark_spmv_case(device, dtype, op):
    torch.manual_seed(0)
    r = fs.benchmark_spmv_case(n_rows=700, n_cols=500, nnz=6000, value_dtype=dtype, index_dtype=torch.int32,
                               warmup=1, iters=3, op=op)
    assert set(r) == {"parameters", "performance", "verification", "backend_status", "samples"}
    assert set(r["performance"]) == {"triton_ms", "cusparse_ms", "triton_speedup_vs_cusparse"}
    assert set(r["verification"]) == {"triton_match_reference", "triton_max_error", "cusparse_match_reference",
                                      "cusparse_max_error"}
    assert r["parameters"]["op"] == op and r["parameters"]["transpose"] == (op != "non")
    assert r["performance"]["triton_ms"] > 0 and r["performance"]["cusparse_ms"] is None
    assert r["backend_status"]["cusparse_unavailable_reason"]
    assert r["verification"]["triton_match_reference"]
    y, ref = r["samples"]["triton"], r["samples"]["reference"]
    assert y.shape == ((500,) if op != "non" else (700,))
    assert rel_err(np_(y), np_(ref)) <= 10 * TOL[dtype]


def test_benchmark_spmv_case_matches_oracle(device):
    """Operator output and torch leg against the CPU oracle on the helper's
    own matrix, rebuilt from the same seed."""
    from flagsparse_amd import benchmarks as bm

    dev = torch.device("cuda")
    torch.manual_seed(9)
    d, i, p = bm._random_csr(400, 300, 3000, torch.float64, torch.int64, dev)
    x = bm._random_dense(400, torch.float64, dev)
    torch.manual_seed(9)
    r = fs.benchmark_spmv_case(n_rows=400, n_cols=300, nnz=3000, value_dtype=torch.float64,
                               index_dtype=torch.int64, warmup=0, iters=1, op="trans")
    ref = O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), (400, 300), op="trans")
    assert rel_err(np_(r["samples"]["triton"]), ref) <= 1e-12
    assert rel_err(np_(r["samples"]["reference"]), ref) <= 1e-12


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["f32", "f64", "c64"])
@pytest.mark.parametrize("op", ["non", "trans", "conj"])
def test_benchmark_spmm_case(device, dtype, op):
    torch.manual_seed(1)
    r = fs.benchmark_spmm_case(n_rows=600, n_cols=400, nnz=5000, n_dense_cols=16, value_dtype=dtype,
                               warmup=1, iters=3, op=op)
    for key in ("pytorch_ms", "triton_ms", "triton_first_call_ms", "cusparse_ms", "triton_speedup_vs_pytorch",
                "triton_speedup_vs_cusparse"):
        assert key in r["performance"]
    for key in ("triton_match_reference", "triton_max_relative_error", "triton_relative_threshold",
                "cusparse_strict_allclose_match"):
        assert key in r["verification"]
    assert r["parameters"]["format"] == "csr" and r["parameters"]["op"] == op
    assert r["performance"]["cusparse_ms"] is None and r["backend_status"]["cusparse_unavailable_reason"]
    assert r["verification"]["triton_max_relative_error"] <= TOL[dtype]
    C = r["samples"]["triton"]
    assert C.shape == ((400, 16) if op != "non" else (600, 16))


def test_benchmark_spmm_case_matches_oracle(device):
    """The helper's operator output against the CPU oracle on the same
    matrix: rebuild the helper's matrix from the same seed."""
    from flagsparse_amd import benchmarks as bm

    torch.manual_seed(5)
    d, i, p = bm._random_csr(300, 200, 2500, torch.float32, torch.int32, torch.device("cuda"))
    B = bm._random_dense((300, 8), torch.float32, torch.device("cuda"))
    torch.manual_seed(5)
    r = fs.benchmark_spmm_case(n_rows=300, n_cols=200, nnz=2500, n_dense_cols=8, warmup=0, iters=1, op="trans")
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), (300, 200), op="trans")
    assert rel_err(np_(r["samples"]["triton"]), ref) <= 1e-5
    assert rel_err(np_(r["samples"]["pytorch"]), ref) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["f32", "f64"])
def test_benchmark_spmm_opt_cases(device, dtype):
    torch.manual_seed(2)
    r = fs.benchmark_spmm_opt_case(n_rows=500, n_cols=500, nnz=6000, n_dense_cols=8, value_dtype=dtype,
                                   warmup=1, iters=2)
    assert set(r["performance"]) >= {"base_ms", "opt_ms", "pt_ms", "cu_ms", "opt_vs_base"}
    assert r["verification"]["status"] == "PASS" and r["verification"]["base_ok"]
    assert "long_row_fallback_used" in r["backend_status"]
    r2 = fs.benchmark_spmm_opt_alg2_case(n_rows=500, n_cols=500, nnz=6000, n_dense_cols=8, value_dtype=dtype,
                                         warmup=1, iters=2)
    assert set(r2["performance"]) == {"base_ms", "opt_ms", "opt_alg2_ms", "torch_ms", "cusparse_ms"}
    for k in ("base_vs_torch_err", "opt_vs_torch_err", "opt_alg2_vs_torch_err"):
        assert r2["verification"][k] <= 1.0
    assert r2["samples"]["cusparse_ref"] is None
    with pytest.raises(TypeError, match="only supports float32 and float64"):
        fs.benchmark_spmm_opt_case(value_dtype=torch.complex64)
    with pytest.raises(TypeError, match="only supports float32 and float64"):
        fs.benchmark_spmm_opt_alg2_case(value_dtype=torch.complex64)
