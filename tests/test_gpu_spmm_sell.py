"""SpMM on the SELL-64 copy (fs_spmm_sell) for stencil and banded matrices
on the prepared route: against the fp64 oracle and the lane-group kernel
(both sum a row in CSR order in the accumulator type; the lane-group kernel
splits rows that cross its sub-tiles into fragments, so the two agree to
rounding, not bit for bit), every column storage of the copy (offset codes,
int16 offsets, absolute columns), padded slices, the widths it takes and
the ones it hands back."""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _lib
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import REL_TOL, VALUE_DTYPES, VALUE_IDS, np_, rel_err

pytestmark = pytest.mark.gpu

_SELL_KERNELS = ("spmm_sell_kernel", "spmm_sell_staged_kernel")


def _run(d, i, p, sh, B, monkeypatch, sell):
    monkeypatch.setenv("FLAGSPARSE_SPMM_SELL", "1" if sell else "0")
    route = fs.prepare_spmm_csr_route(d, i, p, sh, op="non")
    C = fs.flagsparse_spmm_csr_run(route, B)
    return C, _lib.last_kernel()


def _drop(d, i, p, keep, seed):
    """The matrix with each entry kept with probability `keep` (uneven rows)."""
    g = torch.Generator(device=d.device).manual_seed(seed)
    m = torch.rand(d.numel(), generator=g, device=d.device) < keep
    rows = torch.repeat_interleave(torch.arange(p.numel() - 1, device=d.device), (p[1:] - p[:-1]).long())
    counts = torch.bincount(rows[m], minlength=p.numel() - 1)
    p2 = torch.zeros_like(p)
    p2[1:] = torch.cumsum(counts, 0).to(p.dtype)
    return d[m], i[m], p2


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("n_dense_slices", [1, 2, 4, 8, 12, 16])
def test_sell_spmm_stencil_matches_oracle_and_group_bits(device, monkeypatch, dtype, n_dense_slices):
    epl = 16 // torch.empty(0, dtype=dtype).element_size()
    n = n_dense_slices * epl
    d, i, p, sh = S.stencil27(20, dtype, torch.int32, device, seed=4)
    B = S.dense(sh[1], n, dtype, device, seed=5)
    C, kern = _run(d, i, p, sh, B, monkeypatch, True)
    assert kern in _SELL_KERNELS
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)
    assert rel_err(np_(C), ref) <= REL_TOL[dtype]
    C0, kern0 = _run(d, i, p, sh, B, monkeypatch, False)
    assert kern0 not in _SELL_KERNELS
    assert rel_err(np_(C), np_(C0).astype(ref.dtype)) <= REL_TOL[dtype]


@pytest.mark.parametrize("storage", ["codes", "int16", "int32"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["f32", "f64", "c64"])
def test_sell_spmm_column_storages_and_padding(device, monkeypatch, storage, dtype):
    if storage == "int16":
        monkeypatch.setenv("FLAGSPARSE_SELL_CODES", "0")
    elif storage == "int32":
        monkeypatch.setenv("FLAGSPARSE_SELL_DELTA", "0")
    d, i, p, sh = S.stencil27(18, dtype, torch.int64, device, seed=6)
    d, i, p = _drop(d, i, p, 0.7, seed=7)  # uneven rows: slots past a row's length are padding
    B = S.dense(sh[1], 32 if dtype == torch.float32 else 16, dtype, device, seed=8)
    C, kern = _run(d, i, p, sh, B, monkeypatch, True)
    assert kern in _SELL_KERNELS
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)
    assert rel_err(np_(C), ref) <= REL_TOL[dtype]
    C0, _ = _run(d, i, p, sh, B, monkeypatch, False)
    assert rel_err(np_(C), np_(C0).astype(ref.dtype)) <= REL_TOL[dtype]
    assert torch.equal(C, _run(d, i, p, sh, B, monkeypatch, True)[0])  # deterministic


def test_sell_spmm_padding_never_multiplied(device, monkeypatch):
    """B rows that no entry references hold inf: padding slots must not
    gather them (0 * inf would be nan)."""
    d, i, p, sh = S.stencil27(16, torch.float32, torch.int32, device, seed=1)
    d, i, p = _drop(d, i, p, 0.5, seed=2)
    B = S.dense(sh[1], 16, torch.float32, device, seed=3)
    used = torch.zeros(sh[1], dtype=torch.bool, device=device)
    used[i.long()] = True
    B[~used] = float("inf")
    C, kern = _run(d, i, p, sh, B, monkeypatch, True)
    assert kern in _SELL_KERNELS and bool(torch.isfinite(C).all())


def test_sell_spmm_chosen_by_itself_on_a_stencil(device, monkeypatch):
    """With no switch set, a prepared stencil of at least 2,048 slices gets
    the copy on its first launch; random columns do not."""
    monkeypatch.delenv("FLAGSPARSE_SPMM_SELL", raising=False)
    d, i, p, sh = S.stencil27(52, torch.float64, torch.int32, device, seed=9)
    B = S.dense(sh[1], 16, torch.float64, device, seed=10)
    route = fs.prepare_spmm_csr_route(d, i, p, sh, op="non")
    C = fs.flagsparse_spmm_csr_run(route, B)
    assert _lib.last_kernel() in _SELL_KERNELS
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)
    assert rel_err(np_(C), ref) <= 1e-12
    d, i, p, sh = S.uniform_rows(200000, 200000, 8, torch.float64, torch.int32, device, seed=11)
    route = fs.prepare_spmm_csr_route(d, i, p, sh, op="non")
    fs.flagsparse_spmm_csr_run(route, S.dense(sh[1], 16, torch.float64, device, seed=12))
    assert _lib.last_kernel() not in _SELL_KERNELS
    # an unprepared public call never builds the copy
    fs.flagsparse_spmm_csr(d, i, p, S.dense(sh[1], 16, torch.float64, device, seed=12), sh)
    assert _lib.last_kernel() not in _SELL_KERNELS


def test_sell_spmm_hands_back_what_it_cannot_take(device, monkeypatch):
    """Widths that are not whole 16-byte slices and column-major B run the
    lane-group kernel on the same prepared route, with the same results."""
    d, i, p, sh = S.stencil27(16, torch.float32, torch.int32, device, seed=1)
    ref_of = lambda B: O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)  # noqa: E731
    B = S.dense(sh[1], 6, torch.float32, device, seed=2)
    C, kern = _run(d, i, p, sh, B, monkeypatch, True)
    assert kern not in _SELL_KERNELS and rel_err(np_(C), ref_of(B)) <= 1e-5
    Bc = S.dense(sh[1], 16, torch.float32, device, seed=3).t().contiguous().t()
    monkeypatch.setenv("FLAGSPARSE_SPMM_SELL", "1")
    route = fs.prepare_spmm_csr_route(d, i, p, sh, op="non")
    C = fs.flagsparse_spmm_csr_run(route, Bc, dense_layout="col")
    assert _lib.last_kernel() not in _SELL_KERNELS and rel_err(np_(C), ref_of(Bc)) <= 1e-5


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("n_dense_slices", [1, 2, 4, 8, 12, 16])
@pytest.mark.parametrize("tl", ["4", "8"])
@pytest.mark.parametrize("keep", [1.0, 0.7], ids=["stencil", "uneven"])
def test_sell_spmm_staged_bits_match_unstaged(device, monkeypatch, dtype, n_dense_slices, tl, keep):
    """B through LDS (fs_spmm_sell_staged) against the direct kernel: same
    slot order, same bits, for both row-tile widths, several column tiles,
    and uneven rows (entries dropped at random)."""
    epl = 16 // torch.empty(0, dtype=dtype).element_size()
    d, i, p, sh = S.stencil27(20, dtype, torch.int32, device, seed=4)
    if keep < 1.0:
        d, i, p = _drop(d, i, p, keep, seed=9)
    B = S.dense(sh[1], n_dense_slices * epl, dtype, device, seed=5)
    monkeypatch.setenv("FLAGSPARSE_SPMM_SELL_STAGE_TL", tl)
    monkeypatch.setenv("FLAGSPARSE_SPMM_SELL_STAGE", "1")
    C1, k1 = _run(d, i, p, sh, B, monkeypatch, True)
    monkeypatch.setenv("FLAGSPARSE_SPMM_SELL_STAGE", "0")
    C0, k0 = _run(d, i, p, sh, B, monkeypatch, True)
    assert k0 == "spmm_sell_kernel"
    if k1 == "spmm_sell_staged_kernel":
        assert torch.equal(C1, C0)
    else:  # the copy kept other column storage (no codes): nothing staged
        assert k1 == "spmm_sell_kernel"
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)
    assert rel_err(np_(C1), ref) <= REL_TOL[dtype]


def test_sell_spmm_staged_runs_on_the_stencil(device, monkeypatch):
    d, i, p, sh = S.stencil27(20, torch.float32, torch.int32, device, seed=4)
    B = S.dense(sh[1], 32, torch.float32, device, seed=5)
    monkeypatch.setenv("FLAGSPARSE_SPMM_SELL_STAGE", "1")
    _, k = _run(d, i, p, sh, B, monkeypatch, True)
    assert k == "spmm_sell_staged_kernel"
    monkeypatch.delenv("FLAGSPARSE_SPMM_SELL_STAGE")
    _, k = _run(d, i, p, sh, B, monkeypatch, True)
    assert k == "spmm_sell_kernel"  # the default
