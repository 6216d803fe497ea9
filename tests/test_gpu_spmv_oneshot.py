"""The unprepared SpMV call's one-launch path (fs_spmv_csr_oneshot): the
kernel validates the CSR structure while it computes.  Its three ways
through a 64-row block (the LDS stage with 4 lanes per row, two 32-row
halves with 8 lanes per row, the whole workgroup per long row) against the
fp64 oracle and against the prepared path, and its error contract: the
reference's errors in the reference's order (spmv_csr.py:546-558), raised
before `out` is written."""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _lib
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import INDEX_DTYPES, INDEX_IDS, REL_TOL, VALUE_DTYPES, VALUE_IDS, np_, rel_err

pytestmark = pytest.mark.gpu


def _matrix(kind, dtype, idx, device):
    if kind == "short":  # 64 x 8 entries per block: the 4-lane stage
        return S.uniform_rows(5000, 3000, 8, dtype, idx, device, seed=1)
    if kind == "halves":  # 64 x 40 > one stage (f64 accumulation): two 32-row halves
        return S.uniform_rows(3001, 2500, 40, dtype, idx, device, seed=2)
    if kind == "long":  # rows of thousands of entries: the whole workgroup per row
        return S.random_csr(700, 9000, 0.01, dtype, idx, device, seed=3, long_rows=((5, 8000), (400, 5000)))
    return S.powerlaw(20000, dtype, idx, device, seed=4, clip=6000)


@pytest.mark.parametrize("kind", ["short", "halves", "long", "powerlaw"])
@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
def test_oneshot_matches_oracle_and_prepared(device, monkeypatch, kind, dtype, index_dtype):
    monkeypatch.delenv("FLAGSPARSE_SPMV_ONESHOT", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SPMV_KERNEL", raising=False)
    data, indices, indptr, sh = _matrix(kind, dtype, index_dtype, device)
    x = S.vector(sh[1], dtype, device, seed=7)
    y, meta = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh, return_meta=True)
    assert _lib.last_kernel() == "spmv_oneshot_kernel" and meta["kernel"] == "oneshot"
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), sh)
    assert rel_err(np_(y), ref) <= REL_TOL[dtype]
    assert torch.equal(y, fs.flagsparse_spmv_csr(data, indices, indptr, x, sh))  # deterministic
    y_prep = fs.flagsparse_spmv_csr(x=x, prepared=fs.prepare_spmv_csr(data, indices, indptr, sh))
    assert rel_err(np_(y), np_(y_prep).astype(ref.dtype)) <= REL_TOL[dtype]


def test_oneshot_equals_stream_kernel_bits(device, monkeypatch):
    """Blocks that fit the stage sum exactly as the row-block kernel K3t with
    four lanes per row does, so the 27-point stencil gives the same bits
    one-shot and prepared without the SELL copy."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "0")
    data, indices, indptr, sh = S.stencil27(40, torch.float64, torch.int32, device, seed=3)
    x = S.vector(sh[1], torch.float64, device, seed=4)
    y = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep.kernel_name == "stream"
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x, prepared=prep))


def test_oneshot_errors_leave_out_untouched(device):
    n, per = 70_000, 3
    indptr = torch.arange(0, (n + 1) * per, per, dtype=torch.int64, device=device)
    cols = (torch.arange(n * per, dtype=torch.int64, device=device) * 5) % n
    data = torch.ones(n * per, dtype=torch.float64, device=device)
    x = torch.ones(n, dtype=torch.float64, device=device)
    out = torch.full((n,), 7.0, dtype=torch.float64, device=device)
    bad = indptr.clone()
    bad[1000] = bad[1001] + 2
    with pytest.raises(ValueError, match="non-decreasing"):
        fs.flagsparse_spmv_csr(data, cols, bad, x, (n, n), out=out)
    c = cols.clone()
    c[12345] = n
    with pytest.raises(IndexError, match="indices out of range for n_cols"):
        fs.flagsparse_spmv_csr(data, c, indptr, x, (n, n), out=out)
    assert torch.all(out == 7.0)
    # a malformed row pointer far past nnz is clamped inside the kernel, and reported
    bad = indptr.clone()
    bad[n // 2] = 1 << 40
    with pytest.raises(ValueError, match="non-decreasing"):
        fs.flagsparse_spmv_csr(data, cols, bad, x, (n, n))
    # structure errors come before x errors (the general path raises them)
    with pytest.raises(ValueError, match="indptr must start at zero"):
        fs.flagsparse_spmv_csr(data, cols, indptr + 1, x[:-1], (n, n))
    with pytest.raises(ValueError, match="x length"):
        fs.flagsparse_spmv_csr(data, cols, indptr, x[:-1], (n, n))
    y = fs.flagsparse_spmv_csr(data, cols, indptr, x, (n, n), out=out)
    assert y is out and torch.all(out == 3.0)


@pytest.mark.parametrize("kind", ["short", "halves", "long"])
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
def test_oneshot_column_check_on_every_block_path(device, monkeypatch, kind, index_dtype):
    """A column below 0, at n_cols or far past it is flagged on each of the
    three ways through a block (the kernel compares columns as unsigned and
    clamps them for the gather); the last column itself is valid."""
    monkeypatch.delenv("FLAGSPARSE_SPMV_ONESHOT", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SPMV_KERNEL", raising=False)
    data, indices, indptr, sh = _matrix(kind, torch.float64, index_dtype, device)
    x = S.vector(sh[1], torch.float64, device, seed=8)
    row = 400 if kind == "long" else (indptr.numel() - 1) // 2  # row 400 has 5000 entries
    k = int(indptr[row].item()) + 3
    far = (1 << 31) - 1 if index_dtype == torch.int32 else 1 << 40
    for bad in (-1, sh[1], far, -far):
        c = indices.clone()
        c[k] = bad
        with pytest.raises(IndexError, match="indices out of range for n_cols"):
            fs.flagsparse_spmv_csr(data, c, indptr, x, sh)
        assert _lib.last_kernel() == "spmv_oneshot_kernel"
    c = indices.clone()
    c[k] = sh[1] - 1
    y = fs.flagsparse_spmv_csr(data, c, indptr, x, sh)
    ref = O.spmv_csr_wide(np_(data), np_(c), np_(indptr), np_(x), sh)
    assert rel_err(np_(y), ref) <= REL_TOL[torch.float64]


def test_oneshot_switch_off_runs_general_path(device, monkeypatch):
    data, indices, indptr, sh = S.uniform_rows(3000, 3000, 8, torch.float32, torch.int32, device, seed=5)
    x = S.vector(sh[1], torch.float32, device, seed=6)
    monkeypatch.setenv("FLAGSPARSE_SPMV_ONESHOT", "0")
    y0 = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh)
    assert _lib.last_kernel() != "spmv_oneshot_kernel"
    monkeypatch.delenv("FLAGSPARSE_SPMV_ONESHOT")
    y1 = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh)
    assert _lib.last_kernel() == "spmv_oneshot_kernel"
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), sh)
    assert rel_err(np_(y0), ref) <= 1e-5 and rel_err(np_(y1), ref) <= 1e-5


def test_oneshot_launch_failure_takes_general_path_with_int32_fallback(device, monkeypatch):
    """A failed one-shot launch hands the call to the general path, which
    keeps the reference's int64 -> int32 re-run (spmv_csr.py:790-810)."""
    from flagsparse_amd import spmv_csr as spmv_mod

    d, i, p, sh = S.random_csr(40, 30, 0.2, torch.float32, torch.int64, device, seed=2)
    x = S.vector(30, torch.float32, device)
    ref = O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh)
    seen = {"oneshot": 0, "general_int64": 0}
    original = spmv_mod._hip_spmv_csr_impl_prepared

    def fail_oneshot(*args, **kwargs):
        seen["oneshot"] += 1
        return -3

    def fail_int64_once(prepared, x_in):
        if prepared.kernel_indices.dtype == torch.int64 and not seen["general_int64"]:
            seen["general_int64"] += 1
            raise RuntimeError("forced int64 launch failure")
        return original(prepared, x_in)

    monkeypatch.setattr(spmv_mod, "_oneshot_launch", fail_oneshot)
    monkeypatch.setattr(spmv_mod, "_hip_spmv_csr_impl_prepared", fail_int64_once)
    y = fs.flagsparse_spmv_csr(d, i, p, x, sh, index_fallback_policy="auto")
    assert seen == {"oneshot": 1, "general_int64": 1}
    assert rel_err(np_(y), ref) <= 1e-5


def test_oneshot_abi_rejects_unpinned_flags(device):
    """The flags must be pinned, device-mapped host memory: anything else is
    refused before a launch."""
    import ctypes

    data, indices, indptr, sh = S.uniform_rows(100, 100, 4, torch.float32, torch.int32, device, seed=1)
    x = S.vector(100, torch.float32, device, seed=2)
    y = torch.empty(100, dtype=torch.float32, device=device)
    plain = (ctypes.c_int32 * 4)()
    rc = _lib.lib().fs_spmv_csr_oneshot(0, 0, 0, 100, 100, data.numel(), _lib.ptr(data), _lib.ptr(indices),
                                        _lib.ptr(indptr), _lib.ptr(x), _lib.ptr(y), ctypes.addressof(plain),
                                        _lib.stream_handle(device))
    assert rc != 0
    # the refusal leaves no error behind for torch's next launch to report
    assert torch.equal((x * 2).cpu(), x.cpu() * 2)
    torch.cuda.synchronize()
