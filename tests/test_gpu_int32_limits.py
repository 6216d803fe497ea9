"""Matrices with more than 2^31 - 1 stored entries (64-bit row pointers).

The reference switches index dtypes at exactly this limit: the transpose
keeps the index dtype while n_rows <= 2^31 - 1, and widens indptr to int64
when nnz > 2^31 - 1 (spmv_csr.py:482-483, 508-509). SpMM keeps int32 kernel
indices with an int64 indptr (spmm_csr.py:275-292).

The matrix is 2^22 x 2^22 with row r holding 512 + r % 33 entries:
2,214,590,448 in total, which is between 2^31 and 2^32. Values are
1 + (entry % 3) and x[c] = c % 5 - 2. Every product and every row sum is
then a small integer, exact in f32 and in the f64 accumulator whatever
the summation order. So the check is bit-exact equality with an
independent torch index_add_ over the same entries.

Device memory at peak is about 110 GB (A, A^T and the transpose
workspace), well inside one MI355X's 288 GB.
"""

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _csr

pytestmark = pytest.mark.gpu

N = 1 << 22
INT32_MAX = 2**31 - 1
CHUNK_ROWS = 1 << 18


def _lengths(r):
    return 512 + (r % 33)


def _chunk(r0, r1, start, device):
    """Row ids, columns (int32) and values (f32) of rows [r0, r1); `start`
    is the global position of row r0's first entry."""
    rows = torch.arange(r0, r1, dtype=torch.int64, device=device)
    lens = _lengths(rows)
    rid = torch.repeat_interleave(rows, lens)
    first = torch.cumsum(lens, 0) - lens  # chunk-local start of each row
    pos = torch.arange(rid.numel(), dtype=torch.int64, device=device)
    j = pos - torch.repeat_interleave(first, lens)  # position inside the row
    # 40503 is odd, so j * 40503 mod 2^22 is distinct for j < 2^22: no duplicates in a row
    cols = ((rid * 2654435761 + j * 40503) & (N - 1)).to(torch.int32)
    vals = (1 + (pos + start) % 3).to(torch.float32)
    return rid, cols, vals


@pytest.fixture(scope="module")
def big(device):
    torch.cuda.empty_cache()  # blocks cached by earlier tests count as used below
    free, _ = torch.cuda.mem_get_info(device)
    if free < 140 * (1 << 30):
        pytest.skip(f"needs ~140 GB of free device memory, {free / 2**30:.0f} GiB free")
    lens = _lengths(torch.arange(N, dtype=torch.int64, device=device))
    indptr = torch.zeros(N + 1, dtype=torch.int64, device=device)
    indptr[1:] = torch.cumsum(lens, 0)
    nnz = int(indptr[-1])
    assert INT32_MAX < nnz < 2**32
    data = torch.empty(nnz, dtype=torch.float32, device=device)
    indices = torch.empty(nnz, dtype=torch.int32, device=device)
    x = ((torch.arange(N, device=device) % 5) - 2).to(torch.float32)
    xt = ((torch.arange(N, device=device) % 7) - 3).to(torch.float32)
    y_non = torch.zeros(N, dtype=torch.float64, device=device)
    y_trans = torch.zeros(N, dtype=torch.float64, device=device)
    for r0 in range(0, N, CHUNK_ROWS):
        r1 = min(N, r0 + CHUNK_ROWS)
        s, e = int(indptr[r0]), int(indptr[r1])
        rid, cols, vals = _chunk(r0, r1, s, device)
        data[s:e] = vals
        indices[s:e] = cols
        c64 = cols.to(torch.int64)
        y_non.index_add_(0, rid, vals.double() * x[c64].double())
        y_trans.index_add_(0, c64, vals.double() * xt[rid].double())
        del rid, cols, vals, c64
    torch.cuda.synchronize()
    tensors = dict(data=data, indices=indices, indptr=indptr, nnz=nnz, x=x, xt=xt, y_non=y_non, y_trans=y_trans)
    del data, indices, indptr, x, xt, y_non, y_trans
    yield tensors
    tensors.clear()
    torch.cuda.empty_cache()  # hand the ~110 GB back before the other GPU tests


def test_spmv_nnz_above_int32(big):
    y = fs.flagsparse_spmv_csr(big["data"], big["indices"], big["indptr"], big["x"], (N, N))
    assert y.dtype == torch.float32
    assert torch.equal(y.double(), big["y_non"])


def test_transpose_nnz_above_int32_dtypes_and_order(big):
    """Output dtypes follow the reference's rule; within every column the
    rows ascend (the stable sort); column counts equal a bincount."""
    td, ti, tp, tsh = _csr.transpose_csr(big["data"], big["indices"], big["indptr"], (N, N))
    assert tsh == (N, N)
    assert ti.dtype == torch.int32 and tp.dtype == torch.int64
    assert int(tp[0]) == 0 and int(tp[-1]) == big["nnz"]
    counts = torch.bincount(big["indices"], minlength=N)
    assert torch.equal(tp[1:] - tp[:-1], counts)
    del counts
    # rows ascend inside each column: a descent may only happen at a column start
    # (torch.nonzero over > 2^31 elements is not usable, so mask and reduce)
    starts = torch.zeros(big["nnz"] + 1, dtype=torch.bool, device=ti.device)
    starts[tp] = True
    assert not bool(((ti[1:] < ti[:-1]) & ~starts[1 : big["nnz"]]).any())
    del starts
    # the values travel with their rows: entry (r, c) has value 1 + (pos % 3),
    # so the sum of values per column is checked through A^T @ 1
    ones = torch.ones(N, dtype=torch.float32, device=ti.device)
    col_sum = fs.flagsparse_spmv_csr(td, ti, tp, ones, tsh)
    ref = torch.zeros(N, dtype=torch.float64, device=ti.device)
    ref.index_add_(0, big["indices"].to(torch.int64), big["data"].double())
    assert torch.equal(col_sum.double(), ref)


def test_spmv_trans_nnz_above_int32(big):
    y = fs.flagsparse_spmv_csr(big["data"], big["indices"], big["indptr"], big["xt"], (N, N), op="trans")
    assert torch.equal(y.double(), big["y_trans"])


def test_spmm_nnz_above_int32(big):
    B = torch.stack([big["x"], -2 * big["x"]], dim=1).contiguous()
    C = fs.flagsparse_spmm_csr(big["data"], big["indices"], big["indptr"], B, (N, N))
    assert C.shape == (N, 2)
    assert torch.equal(C[:, 0].double(), big["y_non"])
    assert torch.equal(C[:, 1].double(), -2 * big["y_non"])



def test_spmv_sell_nnz_above_int32(big, monkeypatch):
    """The SELL copy forced on the matrix with more than 2^31 entries (slot
    layout, int32 columns: the column offsets exceed int16) computes exactly."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
    prep = fs.prepare_spmv_csr(big["data"], big["indices"], big["indptr"], (N, N))
    assert prep.kernel_name == "sell" and prep._sell.cols.dtype == torch.int32
    assert prep._sell.padded >= big["nnz"]
    y = fs.flagsparse_spmv_csr(x=big["x"], prepared=prep)
    assert torch.equal(y.double(), big["y_non"])
    del prep
