"""More than 2^31 - 1 columns (64-bit column indices).

The matrix is 2^16 rows x (2^31 + 2^20) columns with 64 entries per row;
each row's last entry sits in the columns above 2^31. The reference's SpMM
rejects such indices (spmm_csr.py:280-283). Here both widths run natively,
which is a deliberate superset, so these tests pin that it computes exactly.
op = trans turns the matrix into 2^31 + 2^20 mostly empty rows, which
exercises every row-indexed grid and the 64-bit row arithmetic of the
kernels. Values and x are small integers, so every sum is exact and the
checks are bit-exact against torch index_add_.
"""

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _csr

pytestmark = pytest.mark.gpu

WIDE_ROWS = 1 << 16
WIDE_COLS = (1 << 31) + (1 << 20)
WIDE_PER_ROW = 64
SLICE = 1 << 28


def _pattern(n, modulus, device):
    """(i % modulus) - modulus // 2 as f32, built in slices (n can exceed 2^31)."""
    out = torch.empty(n, dtype=torch.float32, device=device)
    for s in range(0, n, SLICE):
        e = min(n, s + SLICE)
        out[s:e] = (torch.arange(s, e, dtype=torch.int64, device=device) % modulus - modulus // 2).to(torch.float32)
    return out


@pytest.fixture(scope="module")
def wide(device):
    torch.cuda.empty_cache()  # blocks cached by earlier tests count as used below
    free, _ = torch.cuda.mem_get_info(device)
    if free < 80 * (1 << 30):
        pytest.skip(f"needs ~80 GB of free device memory, {free / 2**30:.0f} GiB free")
    nnz = WIDE_ROWS * WIDE_PER_ROW
    rid = torch.arange(WIDE_ROWS, dtype=torch.int64, device=device).repeat_interleave(WIDE_PER_ROW)
    j = torch.arange(nnz, dtype=torch.int64, device=device) % WIDE_PER_ROW
    cols = (rid * 2654435761 + j * 33554467) % WIDE_COLS
    last = j == WIDE_PER_ROW - 1
    cols[last] = WIDE_COLS - 1 - rid[last]  # one entry per row above 2^31
    assert int(cols.max()) == WIDE_COLS - 1
    data = (1 + torch.arange(nnz, device=device) % 3).to(torch.float32)
    indptr = torch.arange(0, nnz + 1, WIDE_PER_ROW, dtype=torch.int64, device=device)
    x = _pattern(WIDE_COLS, 5, device)
    xt = _pattern(WIDE_ROWS, 7, device)
    y_non = torch.zeros(WIDE_ROWS, dtype=torch.float64, device=device)
    y_non.index_add_(0, rid, data.double() * x[cols].double())
    tensors = dict(data=data, indices=cols, indptr=indptr, rid=rid, x=x, xt=xt, y_non=y_non)
    del data, cols, indptr, x, xt, y_non, j, last
    yield tensors
    tensors.clear()
    torch.cuda.empty_cache()


def test_spmv_int64_columns_above_int32(wide):
    shape = (WIDE_ROWS, WIDE_COLS)
    y = fs.flagsparse_spmv_csr(wide["data"], wide["indices"], wide["indptr"], wide["x"], shape)
    assert torch.equal(y.double(), wide["y_non"])


def test_spmv_trans_rows_above_int32(wide):
    shape = (WIDE_ROWS, WIDE_COLS)
    y = fs.flagsparse_spmv_csr(wide["data"], wide["indices"], wide["indptr"], wide["xt"], shape, op="trans")
    assert y.shape == (WIDE_COLS,)
    exp = torch.zeros(WIDE_COLS, dtype=torch.float64, device=y.device)
    exp.index_add_(0, wide["indices"], wide["data"].double() * wide["xt"][wide["rid"]].double())
    for s in range(0, WIDE_COLS, SLICE):
        e = min(WIDE_COLS, s + SLICE)
        assert torch.equal(y[s:e].double(), exp[s:e]), s


def test_transpose_rows_above_int32_dtypes(wide):
    """The reference's dtype rule: index dtype kept (n_rows <= 2^31 - 1),
    indptr dtype kept (nnz <= 2^31 - 1), for an int32 indptr input too."""
    shape = (WIDE_ROWS, WIDE_COLS)
    for ptr_dtype in (torch.int64, torch.int32):
        td, ti, tp, tsh = _csr.transpose_csr(wide["data"], wide["indices"], wide["indptr"].to(ptr_dtype), shape)
        assert tsh == (WIDE_COLS, WIDE_ROWS)
        assert ti.dtype == torch.int64 and tp.dtype == ptr_dtype
        # (torch.bincount overflows for minlength > 2^31, so count with index_add_)
        counts = torch.zeros(WIDE_COLS, dtype=torch.int64, device=ti.device)
        counts.index_add_(0, wide["indices"], torch.ones_like(wide["indices"]))
        assert torch.equal(tp[1:].to(torch.int64) - tp[:-1].to(torch.int64), counts)
        del td, ti, tp, counts


def test_spmm_int64_columns_above_int32(wide):
    shape = (WIDE_ROWS, WIDE_COLS)
    B = torch.empty((WIDE_COLS, 2), dtype=torch.float32, device=wide["x"].device)
    B[:, 0] = wide["x"]
    B[:, 1] = -wide["x"]
    C = fs.flagsparse_spmm_csr(wide["data"], wide["indices"], wide["indptr"], B, shape)
    assert torch.equal(C[:, 0].double(), wide["y_non"])
    assert torch.equal(C[:, 1].double(), -wide["y_non"])


def test_spmv_sell_int64_columns(wide, monkeypatch):
    """The SELL copy forced on this matrix stores int64 absolute columns (the
    offsets exceed int16 and n_cols - 1 exceeds int32) in the slot layout,
    and computes exactly."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
    shape = (WIDE_ROWS, WIDE_COLS)
    prep = fs.prepare_spmv_csr(wide["data"], wide["indices"], wide["indptr"], shape)
    assert prep.kernel_name == "sell"
    assert prep._sell.cols.dtype == torch.int64 and prep._sell.layout == 0
    y = fs.flagsparse_spmv_csr(x=wide["x"], prepared=prep)
    assert torch.equal(y.double(), wide["y_non"])
