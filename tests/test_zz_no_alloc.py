"""fs_spmv_csr_noalloc (static scratch, no allocation) against fs_spmv_csr
(caller workspace): bit-identical outputs through the C ABI, on two calls in
a row (the second on a smaller matrix), for the kernels that use carry
scratch (merge path, entry blocks) and one that does not (row blocks); and
a clear error for a matrix whose carries exceed the static array."""

import ctypes

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _lib
from flagsparse_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _both(prep, x):
    lib = _lib.lib()
    plan = prep.hip_plan()
    dev = x.device
    y_ref = torch.full((prep.n_rows,), float("nan"), dtype=prep.compute_data().dtype, device=dev)
    y_new = torch.full_like(y_ref, float("nan"))
    carry = prep._carry
    common = (_lib.ptr(prep.compute_data()), _lib.ptr(prep.kernel_indices), _lib.ptr(prep.kernel_indptr),
              _lib.ptr(x))
    _lib.check(lib.fs_spmv_csr(plan.plan, *common, _lib.ptr(y_ref), _lib.ptr(prep._part), _lib.ptr(carry),
                               0 if carry is None else carry.numel(), _lib.stream_handle(dev)), "fs_spmv_csr")
    _lib.check(lib.fs_spmv_csr_noalloc(plan.plan, *common, _lib.ptr(y_new), _lib.ptr(prep._part),
                                       _lib.stream_handle(dev)), "fs_spmv_csr_noalloc")
    torch.cuda.synchronize()
    return y_ref, y_new


@pytest.mark.parametrize("kernel", ["merge", "nnzblock", "stream"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64, torch.complex128],
                         ids=["float32", "float64", "complex64", "complex128"])
def test_noalloc_matches_workspace_entry(device, monkeypatch, kernel, dtype):
    monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", kernel)
    monkeypatch.setenv("FLAGSPARSE_SPMV_PANELS", "0")
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "0")
    for n_rows, seed in ((1 << 17, 1), (3000, 2)):  # second call: a smaller matrix
        if kernel == "stream":  # row blocks need short rows
            d, i, p, sh = S.uniform_rows(n_rows, n_rows, 16, dtype, torch.int32, device, seed=seed)
        else:
            d, i, p, sh = S.powerlaw(n_rows, dtype, torch.int32, device, seed=seed)
        prep = fs.prepare_spmv_csr(d, i, p, sh)
        assert prep.kernel_name == kernel
        x = S.vector(sh[1], dtype, device, seed=seed + 10)
        y_ref, y_new = _both(prep, x)
        assert torch.equal(y_ref, y_new), (kernel, n_rows)
        assert not torch.isnan(y_new.real if y_new.is_complex() else y_new).any()


def test_noalloc_rejects_oversized_plan(device, monkeypatch):
    monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", "merge")
    d, i, p, sh = S.powerlaw(4096, torch.float64, torch.int32, device, seed=3)
    prep = fs.prepare_spmv_csr(d, i, p, sh)
    lib = _lib.lib()
    big = _lib.FsCsrPlan()
    ctypes.memmove(ctypes.byref(big), ctypes.byref(prep.hip_plan().plan), ctypes.sizeof(big))
    limit = int(lib.fs_spmv_noalloc_scratch_bytes())
    big.n_tiles = limit // 16 + 1  # 2 x 8-byte carries per tile: one tile too many
    y = torch.empty(sh[0], dtype=torch.float64, device=device)
    x = S.vector(sh[1], torch.float64, device, seed=1)
    rc = lib.fs_spmv_csr_noalloc(big, _lib.ptr(d), _lib.ptr(i), _lib.ptr(p), _lib.ptr(x), _lib.ptr(y),
                                 _lib.ptr(prep._part), _lib.stream_handle(device))
    assert rc == _lib.FS_E_WORKSPACE
    assert "carry scratch" in lib.fs_last_error().decode()


def test_noalloc_calls_on_two_streams_are_ordered(device, monkeypatch):
    """Back-to-back calls on two streams share the static array; the entry
    point orders the second after the first (an event per call), so both
    give fs_spmv_csr's bits with no synchronisation between them."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", "merge")
    monkeypatch.setenv("FLAGSPARSE_SPMV_PANELS", "0")
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "0")
    lib = _lib.lib()
    cases = []
    for n_rows, seed in ((1 << 18, 4), (1 << 17, 5)):
        d, i, p, sh = S.powerlaw(n_rows, torch.float64, torch.int32, device, seed=seed)
        prep = fs.prepare_spmv_csr(d, i, p, sh)
        x = S.vector(sh[1], torch.float64, device, seed=seed + 10)
        y_ref, _ = _both(prep, x)
        cases.append((prep, x, y_ref))
    streams = [torch.cuda.Stream(device=device), torch.cuda.Stream(device=device)]
    outs = []
    torch.cuda.synchronize()
    for rep in range(3):
        for (prep, x, _), st in zip(cases, streams):
            y = torch.full((prep.n_rows,), float("nan"), dtype=torch.float64, device=device)
            st.wait_stream(torch.cuda.current_stream(device))  # y's fill is done before the launch
            _lib.check(lib.fs_spmv_csr_noalloc(prep.hip_plan().plan, _lib.ptr(prep.compute_data()),
                                               _lib.ptr(prep.kernel_indices), _lib.ptr(prep.kernel_indptr),
                                               _lib.ptr(x), _lib.ptr(y), _lib.ptr(prep._part), st.cuda_stream),
                       "fs_spmv_csr_noalloc")
            outs.append((y, cases[streams.index(st)][2]))
    torch.cuda.synchronize()
    for y, y_ref in outs:
        assert torch.equal(y, y_ref)
