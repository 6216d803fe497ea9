"""GPU parity of the use_opt SpMV path (native-precision bucketed kernels).

The reference's opt path (spmv_csr.py:353-461, 870-880) accumulates
float32 in float32 and float64 in float64 over row-length buckets and
reports the number of non-empty buckets as meta["bucket_count"].  These
tests compare the HIP path with the fp64 oracle across the bucket tiers,
index widths and ops, and check bucket_count against the reference's tier
table restated here (_SPMV_OPT_BUCKET_CONFIGS / _FP64, spmv_csr.py:136-161).
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import OPS, np_, rel_err

pytestmark = pytest.mark.gpu

# upper row-length bound per tier; the first tier also holds the empty rows
_TIERS = {torch.float32: (64, 512, 4096, None), torch.float64: (64, 256, 2048, 8192, None)}
# float32 sums accumulate in float32 here, as in the reference's opt kernels
_TOL = {torch.float32: 2e-5, torch.float64: 1e-12}


def _expected_bucket_count(lengths, dtype):
    lo, n = -1, 0
    for hi in _TIERS[dtype]:
        sel = lengths > lo if hi is None else (lengths > lo) & (lengths <= hi)
        n += int(np.any(sel))
        lo = hi if hi is not None else lo
    return n


# (row, length) overrides that put rows in every tier of both tables
_LONG = ((1, 70), (2, 300), (3, 600), (5, 3000), (7, 5000), (11, 9000))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["float32", "float64"])
@pytest.mark.parametrize("ptr_dtype", [torch.int32, torch.int64], ids=["ptr32", "ptr64"])
@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape,long_rows", [((97, 10000), _LONG), ((4099, 700), ()), ((1, 5), ()), ((300, 9500), _LONG[:3])],
                         ids=["tiers", "short", "one-row", "mid"])
def test_spmv_use_opt_matches_oracle(device, dtype, ptr_dtype, op, shape, long_rows):
    m, n = shape
    d, i, p, sh = S.random_csr(m, n, 0.02, dtype, torch.int32, device, seed=m + n, empty_row_every=7,
                               long_rows=long_rows)
    p = p.to(ptr_dtype)
    x = S.vector(m if op != "non" else n, dtype, device, seed=3)
    y, meta = fs.flagsparse_spmv_csr(d, i, p, x, sh, op=op, use_opt=True, return_meta=True)
    ref = O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh, op=op)
    assert y.dtype == dtype and tuple(y.shape) == ref.shape
    err = rel_err(np_(y), ref)
    assert err <= _TOL[dtype], f"rel err {err:.3e}"
    # buckets are formed on the matrix the kernel runs: A, or A^T for trans / conj
    td, ti, tp, _ = O.materialize_op(np_(d), np_(i), np_(p), sh, op)
    assert meta["bucket_count"] == _expected_bucket_count(np.diff(tp.astype(np.int64)), dtype)
    assert meta["kernel"] == "opt"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["float32", "float64"])
def test_spmv_use_opt_prepared_reuse_deterministic(device, dtype):
    d, i, p, sh = S.powerlaw(1 << 15, dtype, torch.int32, device, seed=4)
    prep = fs.prepare_spmv_csr(d, i, p, sh)
    x = S.vector(sh[1], dtype, device, seed=5)
    y1, meta1 = fs.flagsparse_spmv_csr(x=x, prepared=prep, use_opt=True, return_meta=True)
    y2, meta2 = fs.flagsparse_spmv_csr(x=x, prepared=prep, use_opt=True, return_meta=True)
    assert torch.equal(y1, y2)
    assert meta1["bucket_count"] == meta2["bucket_count"] == _expected_bucket_count(np.diff(np_(p).astype(np.int64)), dtype)
    assert prep._opt is not None  # kept on the prepared matrix after the first call
    ref = O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh)
    assert rel_err(np_(y1), ref) <= _TOL[dtype]
    out = torch.empty_like(y1)
    res = fs.flagsparse_spmv_csr(x=x, prepared=prep, use_opt=True, out=out)
    assert res.data_ptr() == out.data_ptr() and torch.equal(out, y1)


def test_spmv_use_opt_not_supported_runs_base_path(device):
    """int64 column indices or complex values: supports_opt is False, the
    base kernels run and bucket_count is 0 (spmv_csr.py:115-118, 870-880)."""
    d, i, p, sh = S.random_csr(200, 300, 0.05, torch.float32, torch.int64, device, seed=1)
    x = S.vector(300, torch.float32, device, seed=2)
    y, meta = fs.flagsparse_spmv_csr(d, i, p, x, sh, use_opt=True, return_meta=True)
    assert meta["bucket_count"] == 0 and meta["kernel"] != "opt"
    assert rel_err(np_(y), O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh)) <= 1e-5
    d, i, p, sh = S.random_csr(200, 300, 0.05, torch.complex64, torch.int32, device, seed=1)
    x = S.vector(300, torch.complex64, device, seed=2)
    y, meta = fs.flagsparse_spmv_csr(d, i, p, x, sh, use_opt=True, return_meta=True)
    assert meta["bucket_count"] == 0
    assert rel_err(np_(y), O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh)) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["float32", "float64"])
def test_spmv_use_opt_empty_cases(device, dtype):
    # every row empty: one bucket, y = 0
    d = torch.empty(0, dtype=dtype, device=device)
    i = torch.empty(0, dtype=torch.int32, device=device)
    p = torch.zeros(6, dtype=torch.int32, device=device)
    y, meta = fs.flagsparse_spmv_csr(d, i, p, torch.ones(4, dtype=dtype, device=device), (5, 4), use_opt=True,
                                     return_meta=True)
    assert torch.count_nonzero(y).item() == 0 and meta["bucket_count"] == 1
    # no rows
    p0 = torch.zeros(1, dtype=torch.int32, device=device)
    y = fs.flagsparse_spmv_csr(d, i, p0, torch.ones(4, dtype=dtype, device=device), (0, 4), use_opt=True)
    assert y.shape == (0,)


def test_spmv_use_opt_inf_and_nan_propagate(device):
    """Each row's product is its own sum: a NaN in x reaches exactly the rows
    that reference its column."""
    d, i, p, sh = S.random_csr(500, 400, 0.02, torch.float32, torch.int32, device, seed=9, long_rows=((3, 390),))
    x = S.vector(400, torch.float32, device, seed=1)
    x[17] = float("nan")
    y = fs.flagsparse_spmv_csr(d, i, p, x, sh, use_opt=True)
    cols = np_(i)
    ptr = np_(p).astype(np.int64)
    hit = np.array([np.any(cols[ptr[r]:ptr[r + 1]] == 17) for r in range(500)])
    assert np.array_equal(np.isnan(np_(y)), hit)
