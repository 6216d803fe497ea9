"""CPU-only checks of the host layer and the C ABI (no GPU compute calls).

Covers what the reference's CPU CI covers (tests/ci/test_public_api.py,
tests/ci/test_runtime_policies.py): the public names, op and policy
normalisation, validation messages raised before any launch, the
fallback policy (with an injected launcher, as in
test_spmv_csr_accuracy.py:152-233), the algorithm registry, and that the
shared library loads and exports every symbol include/flagsparse_hip.h
declares.
"""

import ctypes
import os
import re

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _lib
from flagsparse_amd import spmm_csr as spmm_mod
from flagsparse_amd import spmv_csr as spmv_mod

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flagsparse_hip.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fs_[a-z0-9_]+)\s*\(", text)))


def test_public_surface():
    expected = {
        "flagsparse_spmv_csr", "prepare_spmv_csr", "PreparedCsrSpmv", "flagsparse_spmm_csr",
        "flagsparse_spmm_csr_run", "prepare_spmm_csr_route", "list_spmm_csr_algorithms",
        "resolve_spmm_csr_algorithm", "SPMM_CSR_ALGORITHMS", "SpmmCsrAlgorithm",
        "SpmmCsrAlgorithmUnavailable", "PreparedCsrSpmmRoute", "PreparedCsrSpmmOpt", "PreparedCsrSpmmOptAlg2",
        "prepare_spmm_csr_opt", "prepare_spmm_csr_opt_alg1", "prepare_spmm_csr_opt_alg1_preprocess",
        "prepare_spmm_csr_opt_alg2", "prepare_spmm_csr_opt_alg2_preprocess", "flagsparse_spmm_csr_opt",
        "flagsparse_spmm_csr_opt_alg1", "flagsparse_spmm_csr_opt_alg1_preprocess", "flagsparse_spmm_csr_opt_alg2",
        "flagsparse_spmm_csr_opt_alg2_preprocess", "coo_to_csr_for_spmv", "prepare_spmv_coo_tocsr",
        "flagsparse_spmv_coo_tocsr", "PreparedCoo", "prepare_spmv_coo", "flagsparse_spmv_coo",
        "flagsparse_spmm_coo", "PreparedAlphaSpmmAlg1", "prepare_alpha_spmm_alg1", "flagsparse_alpha_spmm_alg1",
        "flagsparse_alpha_spmm_alg1_tle", "flagsparse_alpha_spmm_alg1_tle_opt", "flagsparse_alpha_spmm_alg1_tle_opt2",
        "is_alpha_spmm_alg1_tle_available", "alpha_spmm_alg1_tle_unavailable_reason",
        "benchmark_spmv_case", "benchmark_spmm_case", "benchmark_spmm_opt_case", "benchmark_spmm_opt_alg2_case",
    }
    assert expected <= set(dir(fs)) and expected <= set(fs.__all__)


def test_library_exports_every_header_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libflagsparse_hip.so not built")
    lib = _lib.load_library()
    declared = _header_functions()
    assert declared, "no declarations parsed from the header"
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.fs_version().decode().startswith("flagsparse_hip")
    assert lib.fs_last_kernel() == b""


def test_diagnostic_lives_in_its_own_library():
    """The gather-floor probe is measurement tooling: declared in its own
    header and built into libflagsparse_diag.so, absent from the product
    library and its header."""
    if not os.path.exists(_lib.LIB_PATH) or not os.path.exists(_lib.DIAG_LIB_PATH):
        pytest.skip("libraries not built")
    assert not hasattr(_lib.load_library(), "fs_diag_gather_rows")
    text = open(os.path.join(ROOT, "flagsparse_amd", "csrc", "flagsparse_diag.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    declared = set(re.findall(r"\b(fs_[a-z0-9_]+)\s*\(", text))
    assert declared == {"fs_last_error", "fs_diag_gather_rows"}
    d = _lib.diag_lib()
    for name in declared:
        assert hasattr(d, name)
    assert d.fs_diag_gather_rows(0, None, 1, 12, None, 1, None, None) == -1
    assert b"row_bytes" in d.fs_last_error()


def test_abi_rejects_bad_arguments_without_touching_the_gpu():
    lib = _lib.load_library()
    assert lib.fs_spmv_csr(None, None, None, None, None, None, None, None, 0, None) == -1
    assert b"plan is null" in lib.fs_last_error()
    plan = _lib.FsCsrPlan()
    plan.val_t = 7
    assert lib.fs_spmv_csr(plan, None, None, None, None, None, None, None, 0, None) == -1
    assert b"bad type code" in lib.fs_last_error()
    assert lib.fs_csr_transpose(0, 0, 0, 0, 0, -1, 1, 1, None, None, None, 0, None, None, None, None, 0, None) == -1
    assert lib.fs_csr_transpose_workspace_bytes(10, 10, 0) == 0
    assert lib.fs_csr_transpose_workspace_bytes(10, 10, 100) > 100 * 8
    assert lib.fs_spmm_workspace_bytes(_lib.FS_F32, 10, 64) == 10 * 64 * 2 * 8
    assert lib.fs_spmm_tile_items(_lib.FS_F32, 64) > 0


def test_plan_struct_layout():
    # offsets must match the C struct (natural alignment, x86-64)
    assert _lib.FsCsrPlan.n_tiles.offset == 56
    assert _lib.FsCsrPlan.hist.offset == 80
    assert ctypes.sizeof(_lib.FsCsrPlan) == 80 + 8 * _lib.FS_HIST_BINS + 16


@pytest.mark.parametrize("op,expected", [(None, 0), ("non", 0), ("trans", 1), ("conj", 2), (" Trans ", 1), (2, 2)])
def test_op_normalisation(op, expected):
    assert spmv_mod._normalize_spmv_op(op) == expected
    assert spmm_mod._normalize_spmm_op(op) == expected


@pytest.mark.parametrize("bad", ["bad", 3, -1, object()])
def test_op_rejects(bad):
    with pytest.raises(ValueError, match="op must be one of: 0=non, 1=trans, 2=conj"):
        spmv_mod._normalize_spmv_op(bad)
    with pytest.raises(ValueError, match="op must be one of"):
        spmm_mod._normalize_spmm_op(bad)


@pytest.mark.parametrize("op", ["non", "trans", "conj"])
def test_op_transpose_contract(op):
    assert spmv_mod._spmv_op_transposes(spmv_mod._normalize_spmv_op(op)) is (op != "non")


@pytest.mark.parametrize("policy", ["auto", "strict", "AUTO"])
def test_index_fallback_policy(policy):
    assert spmv_mod._normalize_spmv_index_fallback_policy(policy) == policy.lower()
    with pytest.raises(ValueError, match="index_fallback_policy must be 'auto' or 'strict'"):
        spmv_mod._normalize_spmv_index_fallback_policy("never")


def test_validation_before_launch_on_cpu_tensors():
    data = torch.ones(3)
    idx = torch.tensor([0, 1, 1], dtype=torch.int32)
    ptr = torch.tensor([0, 2, 3], dtype=torch.int32)
    with pytest.raises(ValueError, match="data, indices, indptr must be CUDA tensors"):
        fs.prepare_spmv_csr(data, idx, ptr, (2, 2))
    with pytest.raises(TypeError, match="must all be torch.Tensor"):
        fs.prepare_spmv_csr([1.0], idx, ptr, (2, 2))
    with pytest.raises(ValueError, match="indptr length must be n_rows\\+1=4, got 3"):
        fs.prepare_spmv_csr(data, idx, ptr, (3, 2))
    with pytest.raises(ValueError, match="transpose=True conflicts with op=non"):
        fs.prepare_spmv_csr(data, idx, ptr, (2, 2), transpose=True, op="non")
    with pytest.raises(ValueError, match="transpose conflicts with op"):
        fs.flagsparse_spmv_csr(data, idx, ptr, torch.ones(2), (2, 2), op="non", transpose=True)
    with pytest.raises(ValueError, match="required when prepared is not provided"):
        fs.flagsparse_spmv_csr(x=torch.ones(2))
    with pytest.raises(ValueError, match="shape must be a 2-tuple"):
        fs.flagsparse_spmm_csr(data, idx, ptr, torch.ones(2, 2), (2,))
    with pytest.raises(ValueError, match="data, indices, and indptr must be CUDA tensors"):
        fs.flagsparse_spmm_csr(data, idx, ptr, torch.ones(2, 2), (2, 2))
    with pytest.raises(ValueError, match="block_n must be positive"):
        fs.flagsparse_spmm_csr(data, idx, ptr, torch.ones(2, 2), (2, 2), block_n=0)


def test_fallback_policy_with_injected_launcher(monkeypatch):
    """The auto policy re-runs with int32 indices; strict re-raises; unsafe
    fallbacks raise the reference's message (runs on CPU: the launcher is
    replaced, nothing reaches the GPU)."""
    limit = spmv_mod._INDEX_LIMIT_INT32
    data = torch.ones(1)
    prep = spmv_mod.PreparedCsrSpmv(
        data=data,
        kernel_indices=torch.tensor([limit + 1], dtype=torch.int64),
        kernel_indptr=torch.tensor([0, 1], dtype=torch.int64),
        shape=(1, limit + 2), n_rows=1, n_cols=limit + 2, block_nnz=256, max_segments=1, max_row_nnz=1,
        opt_buckets=[], transpose=False, index_fallback_policy="auto",
    )

    def fail(_p, _x, use_opt=False, opt_buckets=None):
        raise RuntimeError("forced native int64 failure")

    monkeypatch.setattr(spmv_mod, "_run_spmv_prepared", fail)
    with pytest.raises(RuntimeError, match="int32 fallback is unsafe"):
        spmv_mod._run_spmv_prepared_with_fallback(prep, torch.empty(0))
    prep.index_fallback_policy = "strict"
    with pytest.raises(RuntimeError, match="forced native int64 failure"):
        spmv_mod._run_spmv_prepared_with_fallback(prep, torch.empty(0))

    # safe case: the injected launcher sees the int32 re-run
    seen = []

    def fail_int64(p, _x, use_opt=False, opt_buckets=None):
        seen.append(p.kernel_indices.dtype)
        if p.kernel_indices.dtype == torch.int64:
            raise RuntimeError("forced")
        return "ok"

    monkeypatch.setattr(spmv_mod, "_run_spmv_prepared", fail_int64)
    ok = spmv_mod.PreparedCsrSpmv(
        data=torch.ones(2), kernel_indices=torch.tensor([0, 1], dtype=torch.int64),
        kernel_indptr=torch.tensor([0, 1, 2], dtype=torch.int64), shape=(2, 2), n_rows=2, n_cols=2,
        block_nnz=256, max_segments=1, max_row_nnz=1,
    )
    assert spmv_mod._run_spmv_prepared_with_fallback(ok, torch.ones(2)) == "ok"
    assert seen == [torch.int64, torch.int32]


def test_algorithm_registry():
    assert fs.list_spmm_csr_algorithms() == tuple(fs.SPMM_CSR_ALGORITHMS)
    assert "csr_base" in fs.list_spmm_csr_algorithms(op="conj", dtype=torch.complex64)
    assert "spmm_csr_alg1" not in fs.list_spmm_csr_algorithms(dtype=torch.complex64)
    assert fs.resolve_spmm_csr_algorithm("auto", "non", torch.float32).name == "csr_base"
    assert fs.resolve_spmm_csr_algorithm("alg2", 1, torch.float64).name == "spmm_csr_alg2"
    with pytest.raises(ValueError, match="unsupported CSR SpMM algorithm"):
        fs.resolve_spmm_csr_algorithm("nope", "non", torch.float32)
    with pytest.raises(TypeError, match="does not support dtype"):
        fs.resolve_spmm_csr_algorithm("alg1", "non", torch.complex64)
    assert spmm_mod._normalize_dense_layout("F") == "col"
    with pytest.raises(ValueError, match="dense_layout must be one of"):
        spmm_mod._normalize_dense_layout("diag")


def test_error_metrics():
    ref = torch.tensor([1.0, -2.0, 4.0], dtype=torch.float64)
    cand = torch.tensor([1.0, -2.0, 4.5], dtype=torch.float64)
    m = spmm_mod._spmm_validation_metrics(cand, ref)
    assert m["max_relative_error"] == pytest.approx(0.125)
    assert m["relative_threshold"] == 1e-12 and m["matches_threshold"] is False


def test_coo_validation_before_launch_on_cpu_tensors():
    """spmv_coo.py:390-422, 726-790 and spmm_coo.py:335-368, 651-668: checks
    that fire before any device work, with the reference's messages."""
    from flagsparse_amd import spmv_coo as coo_mod

    d = torch.ones(3)
    i = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(TypeError, match="data, row, col must all be torch.Tensor"):
        fs.prepare_spmv_coo([1.0], i, i, (2, 2))
    with pytest.raises(ValueError, match="data, row, col must be 1D"):
        fs.prepare_spmv_coo(d.view(3, 1), i, i, (2, 2))
    with pytest.raises(ValueError, match="data, row, col must be CUDA tensors"):
        fs.prepare_spmv_coo(d, i, i, (2, 2))
    with pytest.raises(ValueError, match="data, row, col, x, shape required when prepared is None"):
        fs.flagsparse_spmv_coo(d, i, i, None, (2, 2))
    with pytest.raises(ValueError, match="transpose conflicts with op"):
        fs.flagsparse_spmv_coo(d, i, i, d, (2, 2), op="non", transpose=True)
    with pytest.raises(ValueError, match="transpose=True conflicts with op=non"):
        fs.prepare_spmv_coo(d, i, i, (2, 2), transpose=True, op="non")
    with pytest.raises(ValueError, match="index_fallback_policy must be 'auto' or 'strict'"):
        fs.prepare_spmv_coo(d, i, i, (2, 2), index_fallback_policy="maybe")
    with pytest.raises(ValueError, match="op must be one of: 0=non, 1=trans, 2=conj"):
        fs.flagsparse_spmv_coo(d, i, i, d, (2, 2), op="hermitian")
    assert coo_mod._normalize_spmv_coo_op(None, transpose=True) == 1
    assert coo_mod._normalize_spmv_coo_op(2) == 2 and coo_mod._spmv_coo_op_to_name("TRANS") == "trans"

    B = torch.ones(2, 4)
    with pytest.raises(ValueError, match="shape must be a 2-tuple"):
        fs.flagsparse_spmm_coo(d, i, i, B, (2, 2, 2))
    with pytest.raises(ValueError, match="data, row, and col must be 1D tensors"):
        fs.flagsparse_spmm_coo(d.view(3, 1), i, i, B, (2, 2))
    with pytest.raises(ValueError, match="B must be a 2D dense tensor"):
        fs.flagsparse_spmm_coo(d, i, i, B.view(-1), (2, 2))
    with pytest.raises(ValueError, match="shape dimensions must be non-negative"):
        fs.flagsparse_spmm_coo(d, i, i, B, (-1, 2))
    with pytest.raises(ValueError, match="same length"):
        fs.flagsparse_spmm_coo(d[:2], i, i, B, (2, 2))
    with pytest.raises(ValueError, match=r"B.shape\[0\] must be n_cols=3, got 2"):
        fs.flagsparse_spmm_coo(d, i, i, B, (2, 3))
    with pytest.raises(ValueError, match="data, row, col, and B must be CUDA tensors"):
        fs.flagsparse_spmm_coo(d, i, i, B, (2, 2))
    with pytest.raises(ValueError, match="block_n must be positive when provided"):
        fs.flagsparse_spmm_coo(d, i, i, B, (2, 2), block_n=0)
    with pytest.raises(TypeError, match="unexpected keyword argument 'op'"):
        fs.flagsparse_spmm_coo(d, i, i, B, (2, 2), op="trans")


def test_coo_int32_fallback_with_injected_launcher(monkeypatch):
    """spmv_coo.py:701-723 with an injected failing launch (CPU tensors, no
    device work): auto retries on int32 indices, strict re-raises, and an
    unsafe narrowing raises the reference's RuntimeError."""
    from flagsparse_amd import spmv_coo as coo_mod

    srt = coo_mod._SortedCoo(torch.ones(3), torch.tensor([0, 0, 1]), torch.tensor([0, 1, 1]),
                             torch.tensor([0, 2, 3]), torch.tensor([0, 2, 3]), (2, 2))
    launch = coo_mod._PreparedCooLaunch(srt, srt.data, srt.row, srt.col, (2, 2), seg_starts=srt.seg_starts)
    calls = []

    def fake(lau, x, block_size, num_warps, block_inner):
        calls.append(lau.row.dtype)
        if lau.row.dtype == torch.int64:
            raise RuntimeError("forced int64 launch failure")
        return torch.zeros(lau.n_rows)

    monkeypatch.setattr(coo_mod, "_hip_spmv_coo_kernel", fake)
    y = coo_mod._run_spmv_coo_prepared_with_fallback(launch, torch.ones(2), 256, 4, 128)
    assert calls == [torch.int64, torch.int32] and y.shape == (2,)
    strict = coo_mod._PreparedCooLaunch(srt, srt.data, srt.row, srt.col, (2, 2), seg_starts=srt.seg_starts,
                                        index_fallback_policy="strict")
    with pytest.raises(RuntimeError, match="forced int64 launch failure"):
        coo_mod._run_spmv_coo_prepared_with_fallback(strict, torch.ones(2), 256, 4, 128)
    big = torch.tensor([0, 2**31, 1])
    unsafe = coo_mod._PreparedCooLaunch(srt, srt.data, big, srt.col, (2**31 + 1, 2), seg_starts=srt.seg_starts)
    with pytest.raises(RuntimeError, match="native int64 COO SpMV failed and int32 fallback is unsafe: row index range"):
        coo_mod._run_spmv_coo_prepared_with_fallback(unsafe, torch.ones(2), 256, 4, 128)


def test_alpha_spmm_alg1_surface_and_validation_on_cpu():
    """alpha_spmm_alg1.py:39-150, 866-889, 1037-1182: TLE routes report
    unavailable; argument checks fire before any device work."""
    assert fs.is_alpha_spmm_alg1_tle_available() is False
    assert fs.is_alpha_spmm_alg1_tle_opt_available() is False and fs.is_alpha_spmm_alg1_tle_opt2_available() is False
    assert "FlagTree" in fs.alpha_spmm_alg1_tle_unavailable_reason()
    d = torch.ones(2)
    i = torch.zeros(2, dtype=torch.int32)
    p = torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(TypeError, match="prepared must be a PreparedAlphaSpmmAlg1 instance"):
        fs.flagsparse_alpha_spmm_alg1(B=torch.ones(2, 2), prepared=object())
    with pytest.raises(ValueError, match="data, indices, indptr, and shape are required"):
        fs.flagsparse_alpha_spmm_alg1(d, i, None, torch.ones(2, 2), (1, 2))
    with pytest.raises(ValueError, match="must be CUDA tensors|CUDA"):
        fs.prepare_alpha_spmm_alg1(d, i, p, (1, 2))


def test_sell_offsets_from_bits_matches_brute_force():
    """The SELL offset set comes back from the device as 2048 32-bit words,
    bit d + 32768 for offset d; decoding must return exactly the offsets set,
    sorted, including both ends of the range and bits in every byte of a
    word."""
    import numpy as np

    from flagsparse_amd.spmv_csr import _offsets_from_bits

    gen = np.random.default_rng(7)
    for offsets in ([], [0], [-32767, 32767], [-32768], sorted(gen.choice(np.arange(-32768, 32768), 300,
                                                                         replace=False).tolist())):
        words = np.zeros(2048, dtype=np.uint32)
        for d in offsets:
            b = d + 32768
            words[b >> 5] |= np.uint32(1) << np.uint32(b & 31)
        assert _offsets_from_bits(words.view(np.int32)) == sorted(offsets)
