"""GPU: COO SpMV / SpMM (flagsparse_spmv_coo, prepare_spmv_coo,
flagsparse_spmm_coo) against the CPU oracle and dense references, following
the reference's tests/pytest/test_spmv_coo_accuracy.py:91-233 and
test_spmm_coo_accuracy.py:61-101."""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import spmv_coo as coo_mod
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import ELEM_TOL, REL_TOL, VALUE_DTYPES, VALUE_IDS, np_, rel_err

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (8, 10), (37, 29), (300, 200), (1000, 2500)]


def _random_coo(m, n, nnz, dtype, idx_dtype, device, seed, dups=False):
    g = np.random.default_rng(seed)
    if dups:
        flat = g.integers(0, m * n, nnz)
    else:
        flat = g.choice(m * n, min(nnz, m * n), replace=False)
    g.shuffle(flat)  # unsorted input
    row = torch.from_numpy(flat // n).to(idx_dtype).to(device)
    col = torch.from_numpy(flat % n).to(idx_dtype).to(device)
    data = S.vector(flat.size, dtype, device, seed=seed)
    return data, row, col


def _nnz_for(m, n):
    return max(1, int(0.1 * m * n))


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}" for m, n in SHAPES])
@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
@pytest.mark.parametrize("op", ["non", "trans", "conj"])
def test_spmv_coo_matches_oracle(device, shape, dtype, index_dtype, op):
    m, n = shape
    data, row, col = _random_coo(m, n, _nnz_for(m, n), dtype, index_dtype, device, seed=m * 7 + n)
    x_len = m if op != "non" else n
    x = S.vector(x_len, dtype, device, seed=3)
    y = fs.flagsparse_spmv_coo(data, row, col, x, shape=(m, n), op=op)
    ref = O.spmv_coo(np_(data), np_(row), np_(col), np_(x), (m, n), op=op)
    assert y.dtype == dtype and y.shape == (m if op == "non" else n,)
    assert rel_err(np_(y), ref) <= REL_TOL[dtype]


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("op", ["non", "trans", "conj"])
def test_spmv_coo_matches_dense_reference(device, dtype, op):
    """The reference's own check: allclose against the dense product in the
    wide dtype (test_spmv_coo_accuracy.py:91-108)."""
    m, n = 37, 29
    data, row, col = _random_coo(m, n, 200, dtype, torch.int32, device, seed=5)
    dense = torch.zeros((m, n), dtype=dtype, device=device)
    dense[row.long(), col.long()] = data
    A = {"non": dense, "trans": dense.t(), "conj": dense.conj().t()}[op]
    x = S.vector(A.shape[1], dtype, device, seed=6)
    wide = torch.complex128 if dtype.is_complex else torch.float64
    ref = (A.to(wide) @ x.to(wide)).to(dtype)
    out = fs.flagsparse_spmv_coo(data, row, col, x, shape=(m, n), op=op)
    tol = ELEM_TOL[dtype]
    assert torch.allclose(out.to(wide), ref.to(wide), rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.complex128], ids=["float32", "complex128"])
def test_spmv_coo_duplicates_and_sort_by_row_false(device, dtype):
    m, n = 300, 200
    data, row, col = _random_coo(m, n, 20000, dtype, torch.int64, device, seed=8, dups=True)
    x = S.vector(n, dtype, device, seed=9)
    ref = O.spmv_coo(np_(data), np_(row), np_(col), np_(x), (m, n))
    for sort_by_row in (True, False):
        y = fs.flagsparse_spmv_coo(data, row, col, x, shape=(m, n), sort_by_row=sort_by_row)
        assert rel_err(np_(y), ref) <= REL_TOL[dtype]
    p = fs.prepare_spmv_coo(data, row, col, (m, n), sort_by_row=False)
    assert p.seg_starts_non is None and torch.equal(p.data_non, data) and torch.equal(p.row_non, row)


def test_spmv_coo_prepared_fields_and_reuse_across_ops(device):
    """test_spmv_coo_accuracy.py:111-133: one prepared structure serves
    non / trans / conj; the sorted fields follow spmv_coo.py:357-387."""
    m, n = 8, 10
    dtype = torch.complex64
    data, row, col = _random_coo(m, n, 30, dtype, torch.int32, device, seed=12)
    p = fs.prepare_spmv_coo(data, row, col, (m, n))
    r, c = np_(p.row_non).astype(np.int64), np_(p.col_non).astype(np.int64)
    key = r * n + c
    assert np.all(np.diff(key) > 0)  # lex-sorted (row, col), distinct entries
    seg = np_(p.seg_starts_non)
    assert seg[0] == 0 and seg[-1] == p.nnz and np.all(np.diff(seg) > 0)
    assert np.all(r[seg[:-1]] != np.r_[-1, r[seg[1:-1] - 1]])  # every run starts a new row
    assert p.row_non.dtype == torch.int32 and p.col_non.dtype == torch.int32
    rt = np_(p.row_trans).astype(np.int64)
    assert np.all(np.diff(rt * m + np_(p.col_trans)) > 0)
    for op, x_len in (("non", n), ("trans", m), ("conj", m)):
        x = S.vector(x_len, dtype, device, seed=x_len)
        y = fs.flagsparse_spmv_coo(x=x, prepared=p, op=op)
        ref = O.spmv_coo(np_(data), np_(row), np_(col), np_(x), (m, n), op=op)
        assert rel_err(np_(y), ref) <= REL_TOL[dtype]
    pt = fs.prepare_spmv_coo(data, row, col, (m, n), transpose=True)
    with pytest.raises(ValueError, match="transpose conflicts with op"):
        fs.flagsparse_spmv_coo(x=S.vector(n, dtype, device, seed=1), prepared=pt, op="non", transpose=True)
    y_default = fs.flagsparse_spmv_coo(x=S.vector(m, dtype, device, seed=2), prepared=pt)
    assert y_default.shape == (n,)
    with pytest.raises(ValueError, match=r"shape \(3, 3\) does not match prepared.shape \(8, 10\)"):
        fs.flagsparse_spmv_coo(x=S.vector(n, dtype, device, seed=1), prepared=p, shape=(3, 3))


def test_spmv_coo_int64_auto_fallback_to_int32(device, monkeypatch):
    """test_spmv_coo_accuracy.py:199-233 with the HIP launcher."""
    m, n = 12, 9
    data, row, col = _random_coo(m, n, 40, torch.float32, torch.int64, device, seed=4)
    x = S.vector(n, torch.float32, device, seed=5)
    state = {"forced_once": False}
    original = coo_mod._hip_spmv_coo_kernel

    def fail_int64_once(launch, x_in, block_size, num_warps, block_inner):
        if launch.row.dtype == torch.int64 and not state["forced_once"]:
            state["forced_once"] = True
            raise RuntimeError("forced int64 launch failure")
        return original(launch, x_in, block_size, num_warps, block_inner)

    monkeypatch.setattr(coo_mod, "_hip_spmv_coo_kernel", fail_int64_once)
    out = fs.flagsparse_spmv_coo(data, row, col, x, shape=(m, n), index_fallback_policy="auto")
    assert state["forced_once"]
    ref = O.spmv_coo(np_(data), np_(row), np_(col), np_(x), (m, n))
    assert rel_err(np_(out), ref) <= REL_TOL[torch.float32]


def test_spmv_coo_edge_cases(device):
    e = torch.empty(0, device=device)
    ei = torch.empty(0, dtype=torch.int64, device=device)
    y = fs.flagsparse_spmv_coo(e, ei, ei, torch.ones(4, device=device), shape=(5, 4))
    assert y.shape == (5,) and int((y != 0).sum()) == 0
    y = fs.flagsparse_spmv_coo(e, ei, ei, torch.ones(5, device=device), shape=(5, 4), op="trans")
    assert y.shape == (4,) and int((y != 0).sum()) == 0
    data, row, col = _random_coo(50, 40, 100, torch.float64, torch.int32, device, seed=3)
    x = S.vector(40, torch.float64, device, seed=4)
    out = torch.empty(50, dtype=torch.float64, device=device)
    r = fs.flagsparse_spmv_coo(data, row, col, x, shape=(50, 40), out=out)
    assert r.data_ptr() == out.data_ptr()
    y, ms = fs.flagsparse_spmv_coo(data, row, col, x, shape=(50, 40), return_time=True)
    assert ms >= 0.0 and torch.equal(y, out)
    with pytest.raises(IndexError, match="row indices out of range"):
        fs.flagsparse_spmv_coo(data, row + 100, col, x, shape=(50, 40))
    with pytest.raises(ValueError, match="num_warps must be a power of 2"):
        fs.flagsparse_spmv_coo(data, row, col, x, shape=(50, 40), num_warps=3)
    with pytest.raises(ValueError, match="block_inner must be a positive power of 2"):
        fs.flagsparse_spmv_coo(data, row, col, x, shape=(50, 40), block_inner=96)
    with pytest.raises(ValueError, match="x length must be n_cols=40, got 50"):
        fs.flagsparse_spmv_coo(data, row, col, S.vector(50, torch.float64, device, seed=1), shape=(50, 40))


def test_spmv_coo_large_power_law_deterministic(device):
    """A power-law COO (rows up to tens of thousands of entries, shuffled) through the merge-path kernels:
    oracle parity and bit-identical repeats."""
    d, i, p, sh = S.powerlaw(200000, torch.float32, torch.int32, device, seed=21)
    rows = torch.repeat_interleave(torch.arange(sh[0], device=device, dtype=torch.int32), p[1:] - p[:-1])
    perm = torch.randperm(d.numel(), device=device)
    data, row, col = d[perm], rows[perm], i[perm]
    x = S.vector(sh[1], torch.float32, device, seed=22)
    prep = fs.prepare_spmv_coo(data, row, col, sh)
    y1 = fs.flagsparse_spmv_coo(x=x, prepared=prep)
    y2 = fs.flagsparse_spmv_coo(x=x, prepared=prep)
    assert torch.equal(y1, y2)
    ref = O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh)
    assert rel_err(np_(y1), ref) <= REL_TOL[torch.float32]


MNK = [(1, 1, 1), (8, 4, 12), (64, 33, 50), (300, 64, 200), (500, 130, 700)]


@pytest.mark.parametrize("mnk", MNK, ids=[f"{m}x{n}x{k}" for m, n, k in MNK])
@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
def test_spmm_coo_matches_oracle(device, mnk, dtype, index_dtype):
    m, n, k = mnk
    data, row, col = _random_coo(m, k, _nnz_for(m, k), dtype, index_dtype, device, seed=m + n + k)
    B = S.dense(k, n, dtype, device, seed=7)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (m, k))
    ref = O.spmm_coo(np_(data), np_(row), np_(col), np_(B), (m, k))
    assert C.dtype == dtype and C.shape == (m, n)
    assert rel_err(np_(C), ref) <= REL_TOL[dtype]


@pytest.mark.parametrize("dtype", VALUE_DTYPES + [torch.float16, torch.bfloat16],
                         ids=VALUE_IDS + ["float16", "bfloat16"])
def test_spmm_coo_matches_dense_reference_with_duplicates(device, dtype):
    """test_spmm_coo_accuracy.py:61-83, plus duplicate entries (summed)."""
    m, k, n = 64, 50, 33
    src = torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype
    data, row, col = _random_coo(m, k, 900, src, torch.int64, device, seed=31, dups=True)
    data = data.to(dtype)
    B = S.dense(k, n, src, device, seed=32).to(dtype)
    wide = torch.complex128 if dtype.is_complex else torch.float64
    dense = torch.zeros((m, k), dtype=wide, device=device)
    dense.index_put_((row, col), data.to(wide), accumulate=True)
    ref = dense @ B.to(wide)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (m, k))
    assert C.dtype == dtype
    assert rel_err(np_(C.to(wide)), np_(ref)) <= REL_TOL[dtype]


def test_spmm_coo_out_time_empty_and_determinism(device):
    data, row, col = _random_coo(300, 200, 6000, torch.float32, torch.int32, device, seed=41, dups=True)
    B = S.dense(200, 48, torch.float32, device, seed=42)
    out = torch.empty(300, 48, device=device)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (300, 200), out=out)
    assert C.data_ptr() == out.data_ptr()
    C2, ms = fs.flagsparse_spmm_coo(data, row, col, B, (300, 200), return_time=True)
    assert ms >= 0.0 and torch.equal(C2, out)  # bit-identical repeat
    with pytest.raises(ValueError, match="out shape/dtype must match result"):
        fs.flagsparse_spmm_coo(data, row, col, B, (300, 200), out=torch.empty(300, 47, device=device))
    with pytest.raises(IndexError, match="col indices out of range for n_cols"):
        fs.flagsparse_spmm_coo(data, row, col + 200, B, (300, 200))
    e = torch.empty(0, device=device)
    ei = torch.empty(0, dtype=torch.int32, device=device)
    Z = fs.flagsparse_spmm_coo(e, ei, ei, B, (7, 200))
    assert Z.shape == (7, 48) and int((Z != 0).sum()) == 0
