"""GPU: COO -> CSR conversion (bit-exact vs the oracle) and the prepared
"opt" SpMM entry points (spmm_csr.py:2586-2630, 3451-3607;
spmm_csr_opt_alg2.py:732-1013)."""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import REL_TOL, VALUE_DTYPES, VALUE_IDS, np_, rel_err

pytestmark = pytest.mark.gpu


def _random_coo(n_rows, n_cols, nnz, dtype, idx_dtype, device, seed, dups=False):
    g = np.random.default_rng(seed)
    if dups:
        flat = g.integers(0, n_rows * n_cols, nnz)
    else:
        flat = g.choice(n_rows * n_cols, nnz, replace=False)
    row = torch.from_numpy(flat // n_cols).to(idx_dtype).to(device)
    col = torch.from_numpy(flat % n_cols).to(idx_dtype).to(device)
    data = S.vector(nnz, dtype, device, seed=seed)
    return data, row, col


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
@pytest.mark.parametrize("dups", [False, True], ids=["distinct", "dups"])
@pytest.mark.parametrize("shape_nnz", [((1, 1), 1), ((300, 200), 5000), ((4000, 70000), 200000), ((1, 5000), 3000),
                                       ((5000, 1), 3000), ((3000, 9_000_000), 40000), ((300_000, 300_000), 600_000)])
def test_coo_to_csr_bit_exact(device, dtype, idx_dtype, dups, shape_nnz):
    # (one row / one column: a single sort phase; 9M columns: three column
    # passes; 300k x 300k: many workgroup tiles on both phases)
    (m, n), nnz = shape_nnz
    data, row, col = _random_coo(m, n, nnz, dtype, idx_dtype, device, seed=m + nnz, dups=dups)
    d, c, p = fs.coo_to_csr_for_spmv(data, row, col, (m, n))
    od, oc, op = O.coo_to_csr(np_(data), np_(row), np_(col), (m, n))
    assert c.dtype == torch.int32 and p.dtype == torch.int64
    assert np.array_equal(np_(p), op) and np.array_equal(np_(c), oc) and np.array_equal(np_(d), od)


@pytest.mark.parametrize("dtype", [torch.float32, torch.complex64], ids=["float32", "complex64"])
def test_coo_to_csr_workgroup_path_matches_wave_path(device, monkeypatch, dtype):
    data, row, col = _random_coo(50_000, 40_000, 400_000, dtype, torch.int32, device, seed=8, dups=True)
    monkeypatch.setenv("FLAGSPARSE_TRANSPOSE_WG", "1")
    a = fs.coo_to_csr_for_spmv(data, row, col, (50_000, 40_000))
    monkeypatch.setenv("FLAGSPARSE_TRANSPOSE_WG", "0")
    b = fs.coo_to_csr_for_spmv(data, row, col, (50_000, 40_000))
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_coo_to_csr_assume_sorted_and_empty(device):
    data, row, col = _random_coo(100, 80, 600, torch.float64, torch.int64, device, seed=2)
    d, c, p = fs.coo_to_csr_for_spmv(data, row, col, (100, 80))
    rows_sorted = torch.repeat_interleave(torch.arange(100, device=device), p[1:] - p[:-1])
    d2, c2, p2 = fs.coo_to_csr_for_spmv(d, rows_sorted, c.to(torch.int64), (100, 80), assume_sorted=True)
    assert torch.equal(d2, d) and torch.equal(c2, c) and torch.equal(p2, p)
    e = torch.empty(0, device=device)
    ei = torch.empty(0, dtype=torch.int64, device=device)
    d3, c3, p3 = fs.coo_to_csr_for_spmv(e, ei, ei, (7, 3))
    assert p3.shape == (8,) and int(p3.abs().sum()) == 0 and c3.numel() == 0


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
def test_spmv_coo_tocsr(device, dtype):
    data, row, col = _random_coo(500, 300, 4000, dtype, torch.int64, device, seed=9)
    x = S.vector(300, dtype, device, seed=1)
    y = fs.flagsparse_spmv_coo_tocsr(data, row, col, x, (500, 300))
    od, oc, op = O.coo_to_csr(np_(data), np_(row), np_(col), (500, 300))
    ref = O.spmv_csr_wide(od, oc, op, np_(x), (500, 300))
    assert rel_err(np_(y), ref) <= REL_TOL[dtype]
    prep = fs.prepare_spmv_coo_tocsr(data, row, col, (500, 300))
    assert torch.equal(fs.flagsparse_spmv_coo_tocsr(x=x, prepared=prep), y)
    with pytest.raises(ValueError, match="does not match prepared.shape"):
        fs.flagsparse_spmv_coo_tocsr(x=x, prepared=prep, shape=(300, 500))
    with pytest.raises(TypeError, match="x dtype must match data dtype"):
        other = torch.float64 if dtype != torch.float64 else torch.float32
        fs.flagsparse_spmv_coo_tocsr(data, row, col, torch.zeros(300, dtype=other, device=device), (500, 300))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["float32", "float64"])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
@pytest.mark.parametrize("api", ["opt", "alg1", "alg1_pre", "alg2", "alg2_pre"])
def test_spmm_opt_entry_points(device, dtype, index_dtype, api):
    d, i, p, sh = S.random_csr(700, 400, 0.02, dtype, index_dtype, device, seed=4, empty_row_every=5,
                               long_rows=((7, 390),))
    B = S.dense(400, 48, dtype, device, seed=5)
    prep_fn, run_fn = {
        "opt": (fs.prepare_spmm_csr_opt, fs.flagsparse_spmm_csr_opt),
        "alg1": (fs.prepare_spmm_csr_opt_alg1, fs.flagsparse_spmm_csr_opt_alg1),
        "alg1_pre": (fs.prepare_spmm_csr_opt_alg1_preprocess, fs.flagsparse_spmm_csr_opt_alg1_preprocess),
        "alg2": (fs.prepare_spmm_csr_opt_alg2, fs.flagsparse_spmm_csr_opt_alg2),
        "alg2_pre": (fs.prepare_spmm_csr_opt_alg2_preprocess, fs.flagsparse_spmm_csr_opt_alg2_preprocess),
    }[api]
    prep = prep_fn(d, i, p, sh)
    C, ms, meta = run_fn(B=B, prepared=prep, return_time=True, return_meta=True)
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)
    assert rel_err(np_(C), ref) <= REL_TOL[dtype]
    assert ms == pytest.approx(meta["op_total_ms"])
    out = torch.empty_like(C)
    assert run_fn(B=B, prepared=prep, out=out).data_ptr() == out.data_ptr()
    assert torch.equal(run_fn(d, i, p, B, sh), C)
    with pytest.raises(ValueError, match="does not match prepared.shape"):
        run_fn(B=B, prepared=prep, shape=(1, 1))
    with pytest.raises(ValueError, match="B.shape\\[0\\] must be n_cols=400"):
        run_fn(B=B[:10], prepared=prep)


def test_spmm_opt_rejects_complex(device):
    d, i, p, sh = S.random_csr(20, 20, 0.2, torch.complex64, torch.int32, device, seed=1)
    B = S.dense(20, 4, torch.complex64, device)
    with pytest.raises(TypeError, match="only supports float32 and float64"):
        fs.flagsparse_spmm_csr_opt(d, i, p, B, sh)
    with pytest.raises(TypeError, match="only supports float32 and float64"):
        fs.flagsparse_spmm_csr_opt_alg2(d, i, p, B, sh)
    with pytest.raises(TypeError, match="prepared must be a PreparedCsrSpmmOpt instance"):
        fs.flagsparse_spmm_csr_opt(B=B, prepared=object())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["float16", "bfloat16"])
@pytest.mark.parametrize("op", ["non", "trans"])
def test_half_precision_spmv_spmm(device, dtype, op):
    """f16 / bf16 are accepted and computed in f32 (reference: spmv_csr.py:124-127,
    spmm_csr.py:2716-2719); outputs keep the input dtype."""
    d32, i, p, sh = S.random_csr(300, 200, 0.05, torch.float32, torch.int32, device, seed=6, long_rows=((3, 190),))
    d = d32.to(dtype)
    m_in = 300 if op != "non" else 200
    x = S.vector(m_in, torch.float32, device, seed=7).to(dtype)
    y = fs.flagsparse_spmv_csr(d, i, p, x, sh, op=op)
    assert y.dtype == dtype
    ref = O.spmv_csr_wide(np_(d.float()), np_(i), np_(p), np_(x.float()), sh, op=op)
    assert rel_err(np_(y.float()), ref) <= REL_TOL[dtype]
    B = S.dense(m_in, 20, torch.float32, device, seed=8).to(dtype)
    C = fs.flagsparse_spmm_csr(d, i, p, B, sh, op=op)
    assert C.dtype == dtype
    refC = O.spmm_csr_wide(np_(d.float()), np_(i), np_(p), np_(B.float()), sh, op=op)
    assert rel_err(np_(C.float()), refC) <= REL_TOL[dtype]
