"""CSR SpMM operators: the reference's public API on gfx950 HIP kernels.

Public surface and behaviour follow src/flagsparse/sparse_operations/
spmm_csr.py of the reference:
  flagsparse_spmm_csr                 spmm_csr.py:3292-3448
  op normalisation                    spmm_csr.py:22-45
  validation                          spmm_csr.py:239-297, 3312-3364
  transpose for op=trans/conj         spmm_csr.py:300-349 (every call)
  launch-config checks                spmm_csr.py:384-419
  error metrics / thresholds          spmm_csr.py:48-131
  route API (prepare_spmm_csr_route, flagsparse_spmm_csr_run,
  SPMM_CSR_ALGORITHMS, ...)           spmm_csr.py:512-788, 1973-2174
Error types and messages are the reference's.  Device work is one call
each into libflagsparse_hip; there is no CPU path.
"""

import ctypes
import os
import time
from dataclasses import dataclass

import torch

from . import _lib
from ._common import (
    SUPPORTED_INDEX_DTYPES,
    SUPPORTED_VALUE_DTYPES,
    _compute_dtype,
    _is_complex_dtype,
    _tolerance_for_dtype,
)
from ._csr import CsrPlan, analyze_csr, transpose_csr
from .spmv_csr import _PendingCheck, _build_sell, _check_structure, _sell_codes_possible, _spmv_sell_locality

SUPPORTED_SPMM_VALUE_DTYPES = SUPPORTED_VALUE_DTYPES

SPMM_OP_NON = 0
SPMM_OP_TRANS = 1
SPMM_OP_CONJ_TRANS = 2
SPMM_OP_NAMES = {SPMM_OP_NON: "non", SPMM_OP_TRANS: "trans", SPMM_OP_CONJ_TRANS: "conj"}
_SPMM_OP_NAME_TO_CODE = {name: code for code, name in SPMM_OP_NAMES.items()}
_OP_ERROR = "op must be one of: 0=non, 1=trans, 2=conj"


def _normalize_spmm_op(op=None, transpose=False):
    if op is None:
        return SPMM_OP_TRANS if bool(transpose) else SPMM_OP_NON
    if isinstance(op, str):
        code = _SPMM_OP_NAME_TO_CODE.get(op.strip().lower())
        if code is None:
            raise ValueError(_OP_ERROR)
        return code
    try:
        code = int(op)
    except (TypeError, ValueError) as exc:
        raise ValueError(_OP_ERROR) from exc
    if code not in SPMM_OP_NAMES:
        raise ValueError(_OP_ERROR)
    return code


def _spmm_op_to_name(op):
    return SPMM_OP_NAMES[_normalize_spmm_op(op)]


def _spmm_op_transposes(op):
    return _normalize_spmm_op(op) in (SPMM_OP_TRANS, SPMM_OP_CONJ_TRANS)


# -- accuracy helpers (spmm_csr.py:48-131) ----------------------------------
def _spmm_relative_threshold(value_dtype):
    if value_dtype == torch.float16:
        return 5e-3
    if value_dtype == torch.bfloat16:
        return 1e-2
    if value_dtype in (torch.float32, torch.complex64):
        return 1e-6
    if value_dtype in (torch.float64, torch.complex128):
        return 1e-12
    return 1e-6


def _spmm_error_metrics(candidate, reference):
    """Normwise errors: max|d| / max|ref| and sum|d| / sum|ref| (complex: on |.|)."""
    if candidate.shape != reference.shape:
        raise ValueError(
            f"candidate and reference must have the same shape, got {candidate.shape} vs {reference.shape}"
        )
    if candidate.numel() == 0:
        return {
            "max_abs_error": 0.0,
            "max_relative_error": 0.0,
            "sum_relative_error": 0.0,
            "reference_max_magnitude": 0.0,
            "reference_sum_magnitude": 0.0,
        }
    if _is_complex_dtype(reference.dtype):
        ref_mag = torch.abs(reference)
        diff = torch.abs(torch.abs(candidate) - ref_mag)
    else:
        ref_mag = torch.abs(reference)
        diff = torch.abs(candidate - reference)
    max_abs = float(torch.max(diff).item())
    ref_max = float(torch.max(ref_mag).item())
    sum_abs = float(torch.sum(diff).item())
    ref_sum = float(torch.sum(ref_mag).item())
    max_rel = (0.0 if max_abs == 0.0 else float("inf")) if ref_max == 0.0 else max_abs / ref_max
    sum_rel = (0.0 if sum_abs == 0.0 else float("inf")) if ref_sum == 0.0 else sum_abs / ref_sum
    return {
        "max_abs_error": max_abs,
        "max_relative_error": max_rel,
        "sum_relative_error": sum_rel,
        "reference_max_magnitude": ref_max,
        "reference_sum_magnitude": ref_sum,
    }


def _spmm_validation_metrics(candidate, reference):
    metrics = _spmm_error_metrics(candidate, reference)
    threshold = _spmm_relative_threshold(reference.dtype)
    atol, rtol = _tolerance_for_dtype(reference.dtype)
    metrics.update(
        {
            "relative_threshold": threshold,
            "matches_threshold": metrics["max_relative_error"] <= threshold,
            "strict_allclose_match": torch.allclose(candidate, reference, atol=atol, rtol=rtol),
        }
    )
    return metrics


_SPMM_STRUCT_MESSAGES = {
    "start": "indptr[0] must be 0",
    "last": None,  # filled per call (needs nnz)
    "monotone": "indptr must be nondecreasing",
}


def _prepare_spmm_csr_matrix(data, indices, indptr, shape, analyze=False, defer=False):
    """Validation of spmm_csr.py:239-297 (same order, types and messages).

    The HIP kernels take int32 and int64 column indices / row pointers
    natively, so the matrix is kept in its own index dtypes (the reference
    narrows indices to int32 and widens indptr to int64 for Triton).
    The last element returned is the row-length plan (analyze=True), or,
    with defer=True and a transpose that stays in bounds on any structure
    (fs_csr_transpose_bounded), a _PendingCheck whose finish() raises the
    structure errors later; otherwise None.
    """
    if len(shape) != 2:
        raise ValueError("shape must be a 2-tuple: (n_rows, n_cols)")
    if data.ndim != 1 or indices.ndim != 1 or indptr.ndim != 1:
        raise ValueError("data, indices, and indptr must be 1D tensors")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if n_rows < 0 or n_cols < 0:
        raise ValueError("shape dimensions must be non-negative")
    if indptr.numel() != n_rows + 1:
        raise ValueError(f"indptr length must be n_rows+1={n_rows + 1}, got {indptr.numel()}")
    if data.numel() != indices.numel():
        raise ValueError("data and indices must have the same length (nnz)")
    if not all(t.is_cuda for t in (data, indices, indptr)):
        raise ValueError("data, indices, and indptr must be CUDA tensors")
    if not all(t.device == data.device for t in (indices, indptr)):
        raise ValueError("data, indices, and indptr must be on the same CUDA device")
    if data.dtype not in SUPPORTED_SPMM_VALUE_DTYPES:
        raise TypeError("data dtype must be one of: float16, bfloat16, float32, float64, complex64, complex128")
    if indices.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("indices dtype must be torch.int32 or torch.int64")
    if indptr.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("indptr dtype must be torch.int32 or torch.int64")
    nnz = data.numel()
    messages = dict(_SPMM_STRUCT_MESSAGES)
    messages["last"] = lambda got: f"indptr[-1] must equal nnz={nnz}, got {got}"
    data = data.contiguous()
    indices = indices.contiguous()
    indptr = indptr.contiguous()
    if defer and nnz > 0 and _lib.lib().fs_csr_transpose_bounded(
            _lib.value_code(_compute_dtype(data.dtype)), n_rows, n_cols, nnz):
        return data, indices, indptr, n_rows, n_cols, _PendingCheck(data, indices, indptr, n_cols, messages, lazy=True)
    if analyze:
        # the row statistics ride on the structure check's round trip
        _, csr = _check_structure(data, indices, indptr, n_cols, messages, analyze=True)
        return data, indices, indptr, n_rows, n_cols, csr
    _check_structure(data, indices, indptr, n_cols, messages)
    return data, indices, indptr, n_rows, n_cols, None


def _spmm_transposed_deferred(data, indices, indptr, B, shape, op_code, pending):
    """op(A) @ B for A^T / A^H queued behind a pending structure check; the
    check is finished (and raises) before C is returned."""
    data, indices, indptr, shape = _materialize_spmm_csr_op(data, indices, indptr, shape, op_code,
                                                            compact=_compact_ok(data, B), check=pending)
    n_rows, n_cols = int(shape[0]), int(shape[1])
    plan = None
    if n_rows > 0:
        plan = _SpmmPlan(data, indices, indptr, n_rows, n_cols,
                         csr=CsrPlan.from_sizes(data, indices, indptr, n_rows, n_cols))
    C = _hip_spmm(data, indices, indptr, B, n_rows, plan, data.dtype)
    pending.finish()
    return C


def _compact_ok(data, B):
    """Whether this call's SpMM takes int32 indices as they are: all but
    complex64 launches with B rows of at least 512 bytes, which would widen
    them again (_SpmmPlan.launch_indices)."""
    return not (data.dtype == torch.complex64 and int(B.shape[1]) * 8 >= 512)


def _materialize_spmm_csr_op(data, indices, indptr, shape, op_code, compact=False, check=None):
    """A (non), A^T (trans) or A^H (conj) as CSR (spmm_csr.py:341-349);
    compact=True for a transpose that only this call's SpMM reads (int32
    indices and row pointer wherever they fit); check: a pending structure
    check that the transpose takes over (transpose_csr)."""
    if op_code == SPMM_OP_NON:
        if check is not None:
            check.queue()
        return data, indices, indptr, shape
    return transpose_csr(data, indices, indptr, shape, conj=(op_code == SPMM_OP_CONJ_TRANS), compact=compact,
                         check=check)


def _check_segment_override(max_row_nnz, block_nnz, max_segments):
    """Keep the reference's explicit max_segments contract (spmm_csr.py:400-408).

    The reference's Triton kernel walks ceil(max_row/block_nnz) segments; the
    HIP kernel has no segment limit, but an explicit override that the
    reference would reject is rejected the same way.
    """
    if max_segments is None:
        return
    block = 32 if block_nnz is None else int(block_nnz)
    required = (max_row_nnz + block - 1) // block if max_row_nnz > 0 else 0
    if required > int(max_segments):
        raise ValueError(
            "row nnz requires more CSR segments than the explicit max_segments override allows: "
            f"required {required}, provided {int(max_segments)}"
        )


# Skewed columns (a few columns hold much of the matrix, as in R-MAT / power-law
# graphs): for B rows of at least 512 bytes fs_spmm_csr then runs the merge-path
# kernel with at most _SPMM_SKEW_WG_CAP workgroups per CU, which keeps more hot
# B rows in L2.
_SPMM_SKEW_MIN_NNZ = 1 << 20
_SPMM_SKEW_SHARE = 0.2   # share of nnz in the top 1% of columns (uniform columns: ~1%)
_SPMM_SKEW_WG_CAP = 4
_SPMM_SKEW_MAX_COLS = 1 << 27  # wider: no per-column count array (1 GB of int64), no cap


_SPMM_SKEW_SAMPLE = 1 << 22  # entries sampled (evenly strided) for the column counts


def _column_skew(indices, n_cols):
    """Share of the sampled entries that fall in the 1% most frequent columns
    (one sync)."""
    step = max(1, indices.numel() // _SPMM_SKEW_SAMPLE)
    sample = indices[::step]
    counts = torch.bincount(sample, minlength=n_cols)
    top = torch.topk(counts, max(1, n_cols // 100), sorted=False).values
    return float(top.sum().item()) / float(max(1, sample.numel()))


class _SpmmPlan:
    """Analysis + merge-path partitions + workspace sizing for one SpMM matrix.

    The sub-tile size of the SpMM kernel depends on the dense width (it sets
    the lanes per B row), so partitions are built per tile size and cached."""

    __slots__ = ("csr", "indptr", "_skew_checked", "_wide", "kept", "_sell", "_sell_checked")

    def __init__(self, data, indices, indptr, n_rows, n_cols, kept=False, csr=None):
        # csr: a CsrPlan of this matrix from a round trip the caller already
        # made (the structure check's), or one built from its sizes alone
        # (CsrPlan.from_sizes) when no launch decision needs row statistics
        self.csr = csr if csr is not None else analyze_csr(data, indices, indptr, n_rows, n_cols)
        self.indptr = indptr
        self._skew_checked = False
        self._wide = None
        self.kept = bool(kept)  # a prepared matrix: worth a SELL-64 copy
        self._sell = None
        self._sell_checked = False

    def sell_copy(self, data, indices):
        """The SELL-64 copy of a kept matrix whose rows are short and whose
        neighbouring rows use neighbouring columns (stencils, bands), built on
        the first launch with the SpMV's criteria (_spmv_sell_locality), else
        None.  FLAGSPARSE_SPMM_SELL=0 / 1 switches it off / forces it."""
        if not self.kept or self._sell_checked:
            return self._sell
        self._sell_checked = True
        mode = os.environ.get("FLAGSPARSE_SPMM_SELL")
        if mode == "0":
            return None
        p = self.csr.plan
        locality = 1.0 if mode == "1" else _spmv_sell_locality(
            p, indices, self.indptr, False, _sell_codes_possible(data.element_size()))
        if locality is not None:
            try:
                self._sell = _build_sell(data, indices, self.indptr, int(p.n_rows), int(p.n_cols), int(p.nnz),
                                         locality, force=mode == "1")
            except torch.OutOfMemoryError:
                self._sell = None
                torch.cuda.empty_cache()
        return self._sell

    def tiling(self, value_dtype, n_dense):
        """(tile_items, n_tiles, partition) of the kernel fs_spmm_csr runs for
        this value type and dense width."""
        tile_items = int(_lib.lib().fs_spmm_tile_items(_lib.value_code(_compute_dtype(value_dtype)), int(n_dense)))
        return tile_items, self.csr.n_tiles(tile_items), self.csr.partition(self.indptr, tile_items)

    def launch_indices(self, indices, value_dtype, n_dense=None):
        """(column indices, plan struct) a launch passes to fs_spmm_csr.

        complex64 with int32 column indices and B rows of at least 512 bytes
        (the merge-path kernel's launches) runs the int64-index kernel on a
        widened copy of the indices (built once per plan): the int32
        instantiation of that kernel serialises its B-row gathers behind
        waits for outstanding loads (R-MAT 2^20, N = 64 / 128: 1.69 / 2.95
        ms against 1.28 / 2.68 ms with int64 indices).  The lane-group
        kernel (narrower B) runs as fast on int32 indices (N = 32: 0.73 /
        0.74 ms), so those launches skip the widening pass (0.1 ms on 32 M
        entries, which a per-call plan would pay every call).
        FLAGSPARSE_SPMM_WIDEN_C64=0 never widens (A/B)."""
        narrow_b = n_dense is not None and n_dense * 8 < 512
        if (value_dtype != torch.complex64 or indices.dtype != torch.int32 or narrow_b
                or os.environ.get("FLAGSPARSE_SPMM_WIDEN_C64", "1") == "0"):
            return indices, self.csr.plan
        if self._wide is None:
            wide_plan = _lib.FsCsrPlan()
            ctypes.memmove(ctypes.byref(wide_plan), ctypes.byref(self.csr.plan), ctypes.sizeof(wide_plan))
            wide_plan.idx_t = _lib.index_code(torch.int64)
            self._wide = (indices.to(torch.int64), wide_plan)
        wide_indices, wide_plan = self._wide
        wide_plan.spmm_wg_cap = self.csr.plan.spmm_wg_cap  # may be set after the copy
        return wide_indices, wide_plan

    def set_residency(self, indices, n_cols, n_dense, value_dtype):
        """Sets plan.spmm_wg_cap once, when a launch has B rows of at least
        512 bytes: for those, fs_spmm_csr picks its kernel by column skew (the
        merge-path kernel, under this residency cap, on skewed columns).
        Narrower launches never read it, so they skip the column count."""
        if self._skew_checked or n_dense * torch.empty(0, dtype=value_dtype).element_size() < 512:
            return
        self._skew_checked = True
        if (
            indices.numel() >= _SPMM_SKEW_MIN_NNZ
            and n_cols <= _SPMM_SKEW_MAX_COLS
            and _column_skew(indices, n_cols) >= _SPMM_SKEW_SHARE
        ):
            self.csr.plan.spmm_wg_cap = _SPMM_SKEW_WG_CAP


def _hip_spmm(data, indices, indptr, B, n_rows, plan, out_dtype, C=None):
    """C = A @ B for a dense B of any non-negative strides (row-major,
    column-major or strided views); returns C.

    C is written in place when it is given with the compute dtype, else a
    row-major C is allocated.  Strides go to the kernel as they are: no copy
    of B or C is made for column-major layouts."""
    device = data.device
    n_dense = int(B.shape[1])
    cdt = _compute_dtype(data.dtype)
    data_c = data if data.dtype == cdt else data.to(cdt)
    B_c = B if B.dtype == cdt else B.to(cdt)
    if any(st < 0 for st in B_c.stride()):
        B_c = B_c.contiguous()
    if C is None or C.dtype != cdt:
        C_k = torch.empty((n_rows, n_dense), dtype=cdt, device=device)
    else:
        C_k = C
    if n_rows == 0 or n_dense == 0:
        return C_k if cdt == out_dtype else C_k.to(out_dtype)
    sell = plan.sell_copy(data_c, indices) if data.numel() > 0 else None
    if sell is not None and sell.spmm_fits(B_c, C_k):
        sell.spmm(B_c, C_k)
    elif data.numel() == 0:
        C_k.zero_()
    else:
        plan.set_residency(indices, int(plan.csr.plan.n_cols), n_dense, cdt)
        launch_indices, launch_plan = plan.launch_indices(indices, cdt, n_dense)
        tile_items, n_tiles, part = plan.tiling(cdt, n_dense)
        lib = _lib.lib()
        ws = _lib.workspace(lib.fs_spmm_workspace_bytes(_lib.value_code(cdt), n_tiles, n_dense), device)
        _lib.check(
            lib.fs_spmm_csr_strided(
                launch_plan,
                _lib.ptr(data_c),
                _lib.ptr(launch_indices),
                _lib.ptr(indptr),
                _lib.ptr(B_c),
                int(B_c.stride(0)),
                int(B_c.stride(1)),
                _lib.ptr(C_k),
                int(C_k.stride(0)),
                int(C_k.stride(1)),
                n_dense,
                _lib.ptr(part),
                tile_items,
                n_tiles,
                _lib.ptr(ws),
                ws.numel(),
                _lib.stream_handle(device),
            ),
            "fs_spmm_csr",
        )
    if cdt != out_dtype:
        return C_k.to(out_dtype)
    return C_k


def flagsparse_spmm_csr(
    data,
    indices,
    indptr,
    B,
    shape,
    block_n=None,
    block_nnz=None,
    max_segments=None,
    out=None,
    return_time=False,
    transpose=None,
    op=None,
    return_meta=False,
):
    """CSR SpMM C = op(A) @ B on the HIP kernels.

    op: 0/'non' for A @ B, 1/'trans' for A.T @ B, 2/'conj' for A.conj().T @ B.
    Returns C, (C, ms), (C, meta) or (C, ms, meta) like spmm_csr.py:3292-3448;
    meta = {symbolic_ms, compute_ms, op_total_ms, op}.
    """
    op_explicit = op is not None
    op_code = _normalize_spmm_op(op, transpose=False if transpose is None else bool(transpose))
    if op_explicit and transpose is not None and bool(transpose) != _spmm_op_transposes(op_code):
        raise ValueError("transpose conflicts with op")
    if block_n is not None and block_n <= 0:
        raise ValueError("block_n must be positive when provided")
    if block_nnz is not None and block_nnz <= 0:
        raise ValueError("block_nnz must be positive when provided")
    if max_segments is not None and max_segments <= 0:
        raise ValueError("max_segments must be positive when provided")

    do_timing = bool(return_time or return_meta)
    # A^T / A^H into a fresh C: the structure check's answer is read after
    # the transpose and the SpMM are queued behind it (one synchronisation at
    # the end instead of a round trip in between); the reference's error, if
    # any, is raised before C is returned, and before any argument error
    # that the reference raises after its check.
    transposes = _spmm_op_transposes(op_code)
    defer = transposes and out is None and not do_timing and max_segments is None
    data, indices, indptr, n_rows, n_cols, csr0 = _prepare_spmm_csr_matrix(
        data, indices, indptr, shape, analyze=not transposes, defer=defer)
    pending = csr0 if isinstance(csr0, _PendingCheck) else None
    if pending is not None:
        csr0 = None
    try:
        if B.ndim != 2:
            raise ValueError("B must be a 2D dense tensor")
        eff_rows, eff_cols = (n_cols, n_rows) if transposes else (n_rows, n_cols)
        if B.shape[0] != eff_cols:
            raise ValueError(f"B.shape[0] must be n_cols={eff_cols}, got {B.shape[0]}")
        if not B.is_cuda:
            raise ValueError("B must be a CUDA tensor")
        if B.device != data.device:
            raise ValueError("B must be on the same CUDA device as the sparse matrix")
        if B.dtype != data.dtype:
            raise TypeError("B dtype must match data dtype")
        B = B.contiguous()
        n_dense = int(B.shape[1])
        if out is not None:
            if not out.is_cuda:
                raise ValueError("out must be a CUDA tensor")
            if out.device != data.device:
                raise ValueError("out must be on the same CUDA device as the inputs")
            if out.shape != (eff_rows, n_dense) or out.dtype != data.dtype:
                raise ValueError("out shape/dtype must match result")
        if pending is not None:
            return _spmm_transposed_deferred(data, indices, indptr, B, shape, op_code, pending)
    except Exception:
        if pending is not None:
            pending.finish()  # the structure error comes first
        raise

    symbolic_ms = compute_ms = op_total_ms = None
    if do_timing:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    if _spmm_op_transposes(op_code):
        data, indices, indptr, shape = _materialize_spmm_csr_op(data, indices, indptr, shape, op_code,
                                                                compact=_compact_ok(data, B))
        n_rows, n_cols = int(shape[0]), int(shape[1])
    if do_timing:
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        symbolic_ms = (t1 - t0) * 1000.0 if _spmm_op_transposes(op_code) else 0.0

    plan = None
    if n_rows > 0:
        if csr0 is None and max_segments is None:
            # A^T / A^H: no launch decision needs its row statistics (only an
            # explicit max_segments does), so no analysis round trip
            csr0 = CsrPlan.from_sizes(data, indices, indptr, n_rows, n_cols)
        plan = _SpmmPlan(data, indices, indptr, n_rows, n_cols, csr=csr0)
        _check_segment_override(plan.csr.max_row_nnz if max_segments is not None else 0, block_nnz, max_segments)
    if do_timing:
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    C = _hip_spmm(data, indices, indptr, B, n_rows, plan, data.dtype)
    if do_timing:
        torch.cuda.synchronize()
        compute_ms = (time.perf_counter() - t1) * 1000.0
        op_total_ms = symbolic_ms + compute_ms
    if out is not None:
        out.copy_(C)
        C = out
    if return_meta:
        meta = {
            "symbolic_ms": symbolic_ms,
            "compute_ms": compute_ms,
            "op_total_ms": op_total_ms,
            "op": _spmm_op_to_name(op_code),
        }
        if return_time:
            return C, op_total_ms, meta
        return C, meta
    if return_time:
        return C, op_total_ms
    return C


# ---------------------------------------------------------------------------
# Route API (spmm_csr.py:512-788, 1973-2174)
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class SpmmCsrAlgorithm:
    """Registered CSR SpMM route for the AlphaSparse-style run API."""

    name: str
    display_name: str
    supported_ops: tuple
    supported_dtypes: tuple
    run: object


class SpmmCsrAlgorithmUnavailable(RuntimeError):
    """Raised when a registered SpMM CSR route is unavailable in this runtime."""


class PreparedCsrSpmmRoute:
    """Matrix-level CSR SpMM route preparation shared by route algorithms."""

    __slots__ = (
        "data",
        "kernel_indices",
        "kernel_indptr",
        "shape",
        "n_rows",
        "n_cols",
        "row_lengths",
        "max_row_nnz",
        "nnz",
        "avg_nnz_per_row",
        "op",
        "alg",
        "_plan",
    )

    def __init__(self, data, kernel_indices, kernel_indptr, shape, n_rows, n_cols, row_lengths, max_row_nnz, op, alg):
        self.data = data
        self.kernel_indices = kernel_indices
        self.kernel_indptr = kernel_indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = int(n_rows)
        self.n_cols = int(n_cols)
        self.row_lengths = row_lengths
        self.max_row_nnz = int(max_row_nnz)
        self.nnz = int(data.numel())
        self.avg_nnz_per_row = float(self.nnz) / float(max(1, self.n_rows))
        self.op = str(op)
        self.alg = str(alg)
        self._plan = None

    def hip_plan(self):
        if self._plan is None and self.n_rows > 0:
            self._plan = _SpmmPlan(self.data, self.kernel_indices, self.kernel_indptr, self.n_rows, self.n_cols,
                                   kept=True)
        return self._plan


def _normalize_spmm_csr_alg(alg):
    token = "auto" if alg is None else str(alg).strip().lower()
    if token in ("base", "csr", "csr_base"):
        return "csr_base"
    if token in ("alg1", "csr_alg1", "spmm_csr_alg1"):
        return "spmm_csr_alg1"
    if token in ("alg2", "csr_alg2", "spmm_csr_alg2"):
        return "spmm_csr_alg2"
    return token


def _normalize_dense_layout(layout):
    token = "row" if layout is None else str(layout).strip().lower()
    if token in ("auto", "default", "row", "row_major", "row-major", "c", "c_order"):
        return "row"
    if token in ("col", "column", "col_major", "column_major", "col-major", "column-major", "f", "fortran"):
        return "col"
    raise ValueError("dense_layout must be one of: auto, row, col")


def _is_col_major_2d(tensor):
    return (
        torch.is_tensor(tensor)
        and tensor.ndim == 2
        and tensor.stride(0) == 1
        and tensor.stride(1) >= max(1, int(tensor.shape[0]))
    )


def _dense_layout_name(tensor):
    if not torch.is_tensor(tensor) or tensor.ndim != 2:
        return "unknown"
    if tensor.is_contiguous():
        return "row"
    if _is_col_major_2d(tensor):
        return "col"
    return "strided"


def _empty_dense_layout(shape, dtype, device, layout):
    rows, cols = int(shape[0]), int(shape[1])
    if _normalize_dense_layout(layout) == "col":
        return torch.empty_strided((rows, cols), (1, max(1, rows)), dtype=dtype, device=device)
    return torch.empty((rows, cols), dtype=dtype, device=device)


def _materialize_dense_layout(tensor, layout):
    if tensor.ndim != 2:
        raise ValueError("dense layout materialization expects a 2D tensor")
    if _normalize_dense_layout(layout) == "row":
        return tensor.contiguous()
    if _is_col_major_2d(tensor):
        return tensor
    out = _empty_dense_layout(tensor.shape, tensor.dtype, tensor.device, "col")
    out.copy_(tensor)
    return out


def _validate_spmm_route_runtime_inputs(prepared, B):
    if not isinstance(prepared, PreparedCsrSpmmRoute):
        raise TypeError("prepared must be a PreparedCsrSpmmRoute instance")
    if B is None:
        raise ValueError("B is required")
    if B.ndim != 2:
        raise ValueError("B must be a 2D dense tensor")
    if not B.is_cuda:
        raise ValueError("B must be a CUDA tensor")
    if B.device != prepared.data.device:
        raise ValueError("B must be on the same CUDA device as sparse matrix data")
    if B.dtype != prepared.data.dtype:
        raise TypeError("B dtype must match sparse matrix dtype")
    if B.shape[0] != prepared.n_cols:
        raise ValueError(f"B.shape[0] must be n_cols={prepared.n_cols}, got {B.shape[0]}")
    return B


def _route_from_materialized(prepared, data, indices, indptr, shape, op_name):
    n_rows = int(shape[0])
    row_lengths = indptr[1:] - indptr[:-1] if n_rows > 0 else indptr.new_empty((0,))
    route = PreparedCsrSpmmRoute(
        data=data.contiguous(),
        kernel_indices=indices.contiguous(),
        kernel_indptr=indptr.contiguous(),
        shape=shape,
        n_rows=n_rows,
        n_cols=int(shape[1]),
        row_lengths=row_lengths,
        max_row_nnz=0,
        op=op_name,
        alg=prepared.alg,
    )
    plan = route.hip_plan()
    route.max_row_nnz = plan.csr.max_row_nnz if plan is not None else 0
    return route


def _materialize_spmm_csr_route_op(prepared, op_name, *, timing=False):
    if op_name == "non":
        return prepared, (0.0 if timing else None)
    start = end = None
    if timing:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
    data, indices, indptr, shape = _materialize_spmm_csr_op(
        prepared.data, prepared.kernel_indices, prepared.kernel_indptr, prepared.shape, _normalize_spmm_op(op_name)
    )
    runtime = _route_from_materialized(prepared, data, indices, indptr, shape, op_name)
    if end is not None:
        end.record()
        torch.cuda.synchronize()
        return runtime, start.elapsed_time(end)
    return runtime, None


def _run_hip_route(prepared, B, *, route_name, display_name, timing=False, diagnostics=False, dense_layout="row"):
    """Shared runner: every registered route executes the merge-path kernel."""
    B = _validate_spmm_route_runtime_inputs(prepared, B)
    dense_layout = _normalize_dense_layout(dense_layout)
    if dense_layout == "col" and _is_complex_dtype(prepared.data.dtype):
        raise SpmmCsrAlgorithmUnavailable("csr_base col-major layout does not support complex dtypes yet")
    B = _materialize_dense_layout(B, dense_layout)
    n_dense = int(B.shape[1])
    compute_ms = None
    if timing:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
    plan = prepared.hip_plan()
    # Column-major B / C go to the kernel with their strides (spmm_csr.py:134-176
    # takes stride_bk / stride_bn / stride_cm / stride_cn the same way).
    C = _empty_dense_layout((prepared.n_rows, n_dense), prepared.data.dtype, prepared.data.device, dense_layout)
    C = _hip_spmm(
        prepared.data, prepared.kernel_indices, prepared.kernel_indptr, B, prepared.n_rows, plan,
        prepared.data.dtype, C=C,
    )
    if timing:
        end.record()
        torch.cuda.synchronize()
        compute_ms = start.elapsed_time(end)
    meta = {
        "alg": route_name,
        "display_name": display_name,
        "op": prepared.op,
        "process_cpu_ms": 0.0,
        "process_gpu_ms": 0.0 if timing else None,
        "compute_ms": compute_ms,
        "dense_layout": dense_layout,
        "b_stride": tuple(int(v) for v in B.stride()),
        "c_stride": tuple(int(v) for v in C.stride()),
        "output_layout": _dense_layout_name(C),
    }
    if diagnostics:
        tiling = plan.tiling(prepared.data.dtype, n_dense)[:2] if plan is not None else (0, 0)
        meta["diagnostics"] = {
            "launch_config_scope": "matrix",
            "launch_config_count": 1,
            "bucket_count": 0,
            "long_row_count": 0,
            "launch_version": "hip_group_v1",
            "kernel": "spmm_group",
            "tile_items": tiling[0],
            "n_tiles": tiling[1],
            "max_row_nnz": prepared.max_row_nnz,
            "dense_layout": dense_layout,
            "b_stride": meta["b_stride"],
            "c_stride": meta["c_stride"],
            "output_layout": meta["output_layout"],
        }
    return C, meta


def _run_spmm_csr_base_route(prepared, B, *, timing=False, diagnostics=False, dense_layout="row"):
    return _run_hip_route(prepared, B, route_name="csr_base", display_name="Base", timing=timing,
                          diagnostics=diagnostics, dense_layout=dense_layout)


def _run_spmm_csr_alg1_route(prepared, B, *, timing=False, diagnostics=False):
    return _run_hip_route(prepared, B, route_name="spmm_csr_alg1", display_name="Alg1", timing=timing,
                          diagnostics=diagnostics)


def _run_spmm_csr_alg2_route(prepared, B, *, timing=False, diagnostics=False):
    return _run_hip_route(prepared, B, route_name="spmm_csr_alg2", display_name="Alg2", timing=timing,
                          diagnostics=diagnostics)


def _run_alpha_tle_unavailable(prepared, B, *, timing=False, diagnostics=False):
    # The reference's TLE routes need FlagTree's triton.experimental.tle
    # (alpha_spmm_alg1.py:13-31) and raise this when it is absent.
    raise SpmmCsrAlgorithmUnavailable("FlagTree TLE routes are not available on the HIP backend")


SPMM_CSR_ALGORITHMS = {
    "csr_base": SpmmCsrAlgorithm(
        name="csr_base",
        display_name="Base",
        supported_ops=tuple(SPMM_OP_NAMES.values()),
        supported_dtypes=SUPPORTED_SPMM_VALUE_DTYPES,
        run=_run_spmm_csr_base_route,
    ),
    "alpha_alg1_tle_opt": SpmmCsrAlgorithm(
        name="alpha_alg1_tle_opt",
        display_name="TLEOpt",
        supported_ops=tuple(SPMM_OP_NAMES.values()),
        supported_dtypes=(torch.float32, torch.float64),
        run=_run_alpha_tle_unavailable,
    ),
    "alpha_alg1_tle_opt2": SpmmCsrAlgorithm(
        name="alpha_alg1_tle_opt2",
        display_name="TLEOpt2",
        supported_ops=tuple(SPMM_OP_NAMES.values()),
        supported_dtypes=(torch.float32, torch.float64),
        run=_run_alpha_tle_unavailable,
    ),
    "spmm_csr_alg1": SpmmCsrAlgorithm(
        name="spmm_csr_alg1",
        display_name="Alg1",
        supported_ops=tuple(SPMM_OP_NAMES.values()),
        supported_dtypes=(torch.float32, torch.float64),
        run=_run_spmm_csr_alg1_route,
    ),
    "spmm_csr_alg2": SpmmCsrAlgorithm(
        name="spmm_csr_alg2",
        display_name="Alg2",
        supported_ops=tuple(SPMM_OP_NAMES.values()),
        supported_dtypes=(torch.float32, torch.float64),
        run=_run_spmm_csr_alg2_route,
    ),
}


def resolve_spmm_csr_algorithm(alg, op, dtype):
    token = _normalize_spmm_csr_alg(alg)
    if token == "auto":
        token = "csr_base"
    if token not in SPMM_CSR_ALGORITHMS:
        supported = ", ".join(sorted(SPMM_CSR_ALGORITHMS))
        raise ValueError(f"unsupported CSR SpMM algorithm {alg!r}; supported: auto, {supported}")
    algorithm = SPMM_CSR_ALGORITHMS[token]
    op_name = _spmm_op_to_name(op)
    if op_name not in algorithm.supported_ops:
        raise ValueError(f"algorithm {token!r} does not support op {op_name!r}")
    if dtype not in algorithm.supported_dtypes:
        raise TypeError(f"algorithm {token!r} does not support dtype {dtype}")
    return algorithm


def list_spmm_csr_algorithms(op=None, dtype=None):
    op_name = None if op is None else _spmm_op_to_name(op)
    names = []
    for name, algorithm in SPMM_CSR_ALGORITHMS.items():
        if op_name is not None and op_name not in algorithm.supported_ops:
            continue
        if dtype is not None and dtype not in algorithm.supported_dtypes:
            continue
        names.append(name)
    return tuple(names)


def prepare_spmm_csr_route(data, indices, indptr, shape, *, op="non", alg="auto"):
    """Prepare matrix-level CSR SpMM metadata for the route-based run API."""
    op_code = _normalize_spmm_op(op)
    op_name = _spmm_op_to_name(op_code)
    data, indices, indptr, n_rows, n_cols, csr0 = _prepare_spmm_csr_matrix(data, indices, indptr, shape,
                                                                            analyze=True)
    resolved = _normalize_spmm_csr_alg(alg)
    if resolved != "auto":
        resolve_spmm_csr_algorithm(resolved, op_name, data.dtype)
    row_lengths = indptr[1:] - indptr[:-1] if n_rows > 0 else indptr.new_empty((0,))
    route = PreparedCsrSpmmRoute(
        data=data,
        kernel_indices=indices,
        kernel_indptr=indptr,
        shape=shape,
        n_rows=n_rows,
        n_cols=n_cols,
        row_lengths=row_lengths,
        max_row_nnz=0,
        op=op_name,
        alg=resolved,
    )
    if n_rows > 0:  # the row statistics came with the structure check's round trip
        route._plan = _SpmmPlan(data, indices, indptr, n_rows, n_cols, kept=True, csr=csr0)
    plan = route.hip_plan()
    route.max_row_nnz = plan.csr.max_row_nnz if plan is not None else 0
    return route


def flagsparse_spmm_csr_run(
    prepared,
    B,
    *,
    alg=None,
    op=None,
    dense_layout="auto",
    return_time=False,
    return_meta=False,
    timing=False,
    diagnostics=False,
):
    """Run a registered CSR SpMM route (spmm_csr.py:2070-2174).

    gpu_ms is an event pair around the route (transpose included for
    trans/conj); operator_ms = process_cpu_ms + gpu_ms.
    """
    if not isinstance(prepared, PreparedCsrSpmmRoute):
        raise TypeError("prepared must be a PreparedCsrSpmmRoute instance")
    op_name = prepared.op if op is None else _spmm_op_to_name(op)
    alg_name = prepared.alg if alg is None else _normalize_spmm_csr_alg(alg)
    algorithm = resolve_spmm_csr_algorithm(alg_name, op_name, prepared.data.dtype)
    dense_layout = _normalize_dense_layout(dense_layout)
    if dense_layout == "col" and algorithm.name != "csr_base":
        raise SpmmCsrAlgorithmUnavailable("col-major layout is currently supported only by csr_base")
    if B is None or not torch.is_tensor(B):
        raise TypeError("B must be a torch.Tensor")
    if B.ndim != 2:
        raise ValueError("B must be a 2D dense tensor")
    if not B.is_cuda:
        raise ValueError("B must be a CUDA tensor")
    if B.device != prepared.data.device:
        raise ValueError("B must be on the same CUDA device as sparse matrix data")
    if B.dtype != prepared.data.dtype:
        raise TypeError("B dtype must match sparse matrix dtype")

    timed = bool(return_time or return_meta)
    start = end = None
    if timed:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
    runtime, op_gpu_ms = _materialize_spmm_csr_route_op(prepared, op_name, timing=bool(timing))
    if algorithm.name == "csr_base":
        C, route_meta = algorithm.run(runtime, B, timing=bool(timing), diagnostics=bool(diagnostics),
                                      dense_layout=dense_layout)
    else:
        C, route_meta = algorithm.run(runtime, B, timing=bool(timing), diagnostics=bool(diagnostics))
    gpu_ms = None
    if end is not None:
        end.record()
        torch.cuda.synchronize()
        gpu_ms = start.elapsed_time(end)
    process_cpu_ms = float(route_meta.get("process_cpu_ms", 0.0) or 0.0)
    process_gpu_ms = (float(op_gpu_ms or 0.0) + float(route_meta.get("process_gpu_ms") or 0.0)) if timing else None
    operator_ms = (process_cpu_ms + float(gpu_ms)) if gpu_ms is not None else None
    meta = None
    if return_meta:
        meta = {
            "alg": algorithm.name,
            "display_name": algorithm.display_name,
            "op": op_name,
            "operator_ms": operator_ms,
            "gpu_ms": gpu_ms,
            "process_cpu_ms": process_cpu_ms,
            "dense_layout": route_meta.get("dense_layout", dense_layout),
            "b_stride": route_meta.get("b_stride"),
            "c_stride": route_meta.get("c_stride"),
            "output_layout": route_meta.get("output_layout"),
        }
        if timing:
            meta["process_gpu_ms"] = process_gpu_ms
            meta["compute_ms"] = route_meta.get("compute_ms")
        if diagnostics and "diagnostics" in route_meta:
            meta["diagnostics"] = route_meta["diagnostics"]
    if return_time and return_meta:
        return C, operator_ms, meta
    if return_time:
        return C, operator_ms
    if return_meta:
        return C, meta
    return C
