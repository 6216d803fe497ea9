"""GPU transpose (op=trans/conj materialisation) is bit-exact with the oracle.

The reference builds A^T with a stable argsort by column plus bincount /
cumsum (spmv_csr.py:477-515, spmm_csr.py:300-338); indices, indptr and
(conjugated) values must match exactly, including the output index dtypes.
"""

import numpy as np
import pytest
import torch

from flagsparse_amd import _csr
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import INDEX_DTYPES, INDEX_IDS, VALUE_DTYPES, VALUE_IDS, np_

pytestmark = pytest.mark.gpu


def _check(data, indices, indptr, shape, conj):
    td, ti, tp, tsh = _csr.transpose_csr(data, indices, indptr, shape, conj=conj)
    od, oi, op, osh = O.transpose_csr(np_(data), np_(indices), np_(indptr), shape, conj=conj)
    assert tsh == osh
    assert np_(ti).dtype == oi.dtype and np_(tp).dtype == op.dtype
    assert np.array_equal(np_(tp), op)
    assert np.array_equal(np_(ti), oi)
    assert np.array_equal(np_(td), od)  # bit-exact permutation (+ exact conj)


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("conj", [False, True], ids=["trans", "conj"])
@pytest.mark.parametrize("shape", [(1, 1), (1, 300), (300, 1), (257, 513), (1000, 70000), (5000, 300)])
def test_transpose_bit_exact(device, dtype, index_dtype, conj, shape):
    m, n = shape
    d, i, p, sh = S.random_csr(m, n, min(0.2, 40.0 / n), dtype, index_dtype, device, seed=m * 7 + n,
                               empty_row_every=5 if m > 5 else 0)
    _check(d, i, p, sh, conj)


def test_transpose_duplicates_stay_stable(device):
    # Unsorted columns with repeats inside a row: a stable sort keeps input order.
    indptr = torch.tensor([0, 4, 4, 7], dtype=torch.int32, device=device)
    indices = torch.tensor([3, 1, 3, 0, 1, 1, 3], dtype=torch.int32, device=device)
    data = torch.arange(1, 8, dtype=torch.float64, device=device)
    _check(data, indices, indptr, (3, 4), False)


def test_transpose_multi_pass_keys(device):
    # n_cols needing three 8-bit radix passes, power-law rows
    d, i, p, sh = S.powerlaw(1 << 17, torch.float32, torch.int32, device, seed=4)
    _check(d, i, p, sh, False)
    d, i, p, sh = S.rmat(scale=14, dtype=torch.complex64, index_dtype=torch.int64, device=device, seed=1)
    _check(d, i, p, sh, True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["float32", "float64", "complex64"])
def test_transpose_three_wide_passes(device, dtype):
    # more than 2^22 columns: three 11-bit passes of the workgroup-tile sort
    d, i, p, sh = S.random_csr(3000, 9_000_000, 25.0 / 9_000_000, dtype, torch.int64, device, seed=11)
    _check(d, i, p, sh, dtype == torch.complex64)


@pytest.mark.parametrize("rows", [255, 256, 257, 512, 1023])
def test_transpose_tile_boundaries(device, rows):
    # 32 entries per row: nnz just below, at and above multiples of the
    # 8192-entry workgroup tile (and of its 1024-entry wave sub-tiles)
    d, i, p, sh = S.uniform_rows(rows, 5000, 32, torch.float32, torch.int32, device, seed=rows)
    _check(d, i, p, sh, False)


@pytest.mark.parametrize("dtype", [torch.float32, torch.complex64], ids=["float32", "complex64"])
def test_transpose_workgroup_path_matches_wave_path(device, monkeypatch, dtype):
    # the workgroup-tile passes and the wave-tile passes give the same bits
    d, i, p, sh = S.powerlaw(1 << 17, dtype, torch.int32, device, seed=9)
    monkeypatch.setenv("FLAGSPARSE_TRANSPOSE_WG", "1")
    a = _csr.transpose_csr(d, i, p, sh, conj=True)
    monkeypatch.setenv("FLAGSPARSE_TRANSPOSE_WG", "0")
    b = _csr.transpose_csr(d, i, p, sh, conj=True)
    for x, y in zip(a[:3], b[:3]):
        assert torch.equal(x, y)


def test_transpose_empty(device):
    d = torch.empty(0, dtype=torch.float32, device=device)
    i = torch.empty(0, dtype=torch.int64, device=device)
    p = torch.zeros(4, dtype=torch.int64, device=device)
    _check(d, i, p, (3, 5), False)


def test_transpose_full_size_roundtrip(device):
    """C4-sized matrix: (A^T)^T == A exactly (sorted columns), colptr == counts."""
    d, i, p, sh = S.uniform_rows(1 << 20, 1 << 20, 32, torch.float32, torch.int32, device, seed=7)
    td, ti, tp, tsh = _csr.transpose_csr(d, i, p, sh)
    counts = torch.bincount(i.to(torch.int64), minlength=sh[1])
    assert torch.equal((tp[1:] - tp[:-1]).to(torch.int64), counts)
    d2, i2, p2, sh2 = _csr.transpose_csr(td, ti, tp, tsh)
    assert sh2 == sh
    assert torch.equal(p2, p) and torch.equal(i2, i) and torch.equal(d2, d)


def _stable_argsort_transpose(d, i, p, sh, conj):
    """The reference's transpose algorithm (spmv_csr.py:477-515) in torch on
    the device: row ids by repeat_interleave, stable argsort by column, two
    gathers, bincount + cumsum."""
    rows = torch.repeat_interleave(torch.arange(sh[0], device=d.device), (p[1:] - p[:-1]).to(torch.int64))
    perm = torch.argsort(i.to(torch.int64), stable=True)
    v = d[perm]
    if conj and v.is_complex():
        v = v.conj()
    tp = torch.zeros(sh[1] + 1, dtype=torch.int64, device=d.device)
    tp[1:] = torch.cumsum(torch.bincount(i.to(torch.int64), minlength=sh[1]), 0)
    return v, rows[perm], tp


@pytest.mark.parametrize("case", ["c4_f32_i32", "c5_c64_i64_conj", "c5_f32_i64", "powerlaw_f32_i32"])
def test_transpose_full_size_matches_stable_argsort(device, case):
    """BASELINE-sized matrices (uniform 1M x 32, R-MAT 2^21 with its many empty
    rows, power-law 4M): the HIP transpose equals the reference algorithm's
    output bit for bit, so the full-size op=trans / conj checks do not rest on
    the product's own transpose."""
    if case == "c4_f32_i32":
        (d, i, p, sh), conj = S.uniform_rows(1 << 20, 1 << 20, 32, torch.float32, torch.int32, device, seed=5), False
    elif case == "c5_c64_i64_conj":
        (d, i, p, sh), conj = S.rmat(21, dtype=torch.complex64, index_dtype=torch.int64, device=device, seed=7), True
    elif case == "c5_f32_i64":
        (d, i, p, sh), conj = S.rmat(21, dtype=torch.float32, index_dtype=torch.int64, device=device, seed=7), False
    else:
        (d, i, p, sh), conj = S.powerlaw(4194304, torch.float32, torch.int32, device, seed=3), False
    tv, tc, tp, tsh = _csr.transpose_csr(d, i, p, sh, conj=conj)
    rv, rc, rp = _stable_argsort_transpose(d, i, p, sh, conj)
    assert tsh == (sh[1], sh[0])
    assert torch.equal(tv, rv)
    assert torch.equal(tc.to(torch.int64), rc)
    assert torch.equal(tp.to(torch.int64), rp)
    del tv, tc, tp, rv, rc, rp
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["f32", "f64", "c64"])
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
def test_transpose_with_fused_check(device, dtype, index_dtype):
    """fs_csr_transpose_checked: the transpose is bit-identical to
    fs_csr_transpose, a valid matrix decodes as valid (column range [0, 0]),
    and each fault is reported with the reference's error, whether the check
    runs inside the transpose or is queued on its own (a check that no
    transpose took over is queued by finish())."""
    from flagsparse_amd.spmv_csr import _PendingCheck, _SPMV_STRUCT_MESSAGES

    d, i, p, sh = S.random_csr(3000, 5000, 0.01, dtype, index_dtype, device, seed=5, empty_row_every=7,
                               long_rows=((11, 4000),))
    ref = _csr.transpose_csr(d, i, p, sh, conj=True)
    pc = _PendingCheck(d, i, p, sh[1], _SPMV_STRUCT_MESSAGES, lazy=True)
    got = _csr.transpose_csr(d, i, p, sh, conj=True, check=pc)
    assert pc.finish() == (0, 0)
    for a, b in zip(got[:3], ref[:3]):
        assert torch.equal(a, b)
    big = (1 << 40) if index_dtype == torch.int64 else (1 << 31) - 1
    for col in (sh[1], -1, big, -big):
        c = i.clone()
        c[int(p[1500].item()) + 1] = col
        pc = _PendingCheck(d, c, p, sh[1], _SPMV_STRUCT_MESSAGES, lazy=True)
        _csr.transpose_csr(d, c, p, sh, check=pc)  # stays in bounds whatever the columns hold
        with pytest.raises(IndexError, match="indices out of range"):
            pc.finish()
    bad = p.clone()
    bad[2000] = bad[2001] + 5
    pc = _PendingCheck(d, i, bad, sh[1], _SPMV_STRUCT_MESSAGES, lazy=True)
    _csr.transpose_csr(d, i, bad, sh, check=pc)
    with pytest.raises(ValueError, match="non-decreasing"):
        pc.finish()
    pc = _PendingCheck(d, i, bad, sh[1], _SPMV_STRUCT_MESSAGES, lazy=True)  # never fused: finish() queues it
    with pytest.raises(ValueError, match="non-decreasing"):
        pc.finish()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_fused_check_half_precision_and_mixed_widths(device, dtype):
    """Half-precision values transpose through float32 and keep the fused
    check; an int64 row pointer with int32 columns (and the reverse) reads
    each width correctly in the row-tile and count passes."""
    from flagsparse_amd.spmv_csr import _PendingCheck, _SPMV_STRUCT_MESSAGES

    d, i, p, sh = S.random_csr(2000, 3000, 0.01, torch.float32, torch.int32, device, seed=8)
    d = d.to(dtype)
    for ii, pp in ((i, p.to(torch.int64)), (i.to(torch.int64), p)):
        ref = _csr.transpose_csr(d, ii, pp, sh)
        pc = _PendingCheck(d, ii, pp, sh[1], _SPMV_STRUCT_MESSAGES, lazy=True)
        got = _csr.transpose_csr(d, ii, pp, sh, check=pc)
        pc.finish()
        for a, b in zip(got[:3], ref[:3]):
            assert torch.equal(a, b)
        c = ii.clone()
        c[17] = sh[1] + 3
        pc = _PendingCheck(d, c, pp, sh[1], _SPMV_STRUCT_MESSAGES, lazy=True)
        _csr.transpose_csr(d, c, pp, sh, check=pc)
        with pytest.raises(IndexError, match="indices out of range"):
            pc.finish()


def test_transpose_checked_abi_refusals(device):
    """fs_csr_transpose_checked refuses what it cannot fuse: no entries, or a
    value type without a bounded transpose (complex128)."""
    from flagsparse_amd import _lib

    lib = _lib.lib()
    d, i, p, sh = S.random_csr(64, 64, 0.1, torch.complex128, torch.int32, device, seed=1)
    nnz = d.numel()
    td, ti, tp = torch.empty_like(d), torch.empty_like(i), torch.empty(sh[1] + 1, dtype=torch.int32, device=device)
    ws = _lib.workspace(lib.fs_csr_transpose_workspace_bytes(sh[0], sh[1], nnz), device)
    ck = _lib.workspace(lib.fs_csr_check_bytes(), device)
    words = torch.zeros(5, dtype=torch.int64, pin_memory=True)
    args = lambda vcode, n: (vcode, _lib.index_code(i.dtype), _lib.index_code(p.dtype), _lib.index_code(torch.int32),  # noqa: E731
                             _lib.index_code(torch.int32), sh[0], sh[1], n, _lib.ptr(d), _lib.ptr(i), _lib.ptr(p), 0,
                             _lib.ptr(td), _lib.ptr(ti), _lib.ptr(tp), _lib.ptr(ws), ws.numel(), _lib.ptr(ck),
                             words.data_ptr(), _lib.stream_handle(device))
    assert lib.fs_csr_transpose_bounded(_lib.value_code(d.dtype), sh[0], sh[1], nnz) == 0
    assert lib.fs_csr_transpose_checked(*args(_lib.value_code(d.dtype), nnz)) != 0
    assert "not a bounded transpose" in lib.fs_last_error().decode()
    assert lib.fs_csr_transpose_checked(*args(_lib.value_code(torch.float64), 0)) != 0
