"""Prepared ("opt") CSR SpMM entry points on the HIP merge-path kernel.

Mirrors the reference's secondary SpMM surface:
  PreparedCsrSpmmOpt, prepare_spmm_csr_opt(_alg1)(_preprocess),
  flagsparse_spmm_csr_opt(_alg1)(_preprocess)        spmm_csr.py:2177-2251,
                                                      2586-2630, 3451-3607
  PreparedCsrSpmmOptAlg2, prepare_spmm_csr_opt_alg2(_preprocess),
  flagsparse_spmm_csr_opt_alg2(_preprocess)           spmm_csr_opt_alg2.py:20-58,
                                                      732-780, 906-1013
Signatures, the float32/float64-only restriction, validation order and
messages follow the reference.  The reference buckets rows by length and
splits long rows on every call; here the prepared object caches one
merge-path plan (analysis + partition) and every call is one kernel launch
plus the deterministic fix-up of rows that cross tiles.
"""

import time

import torch

from ._common import _INDEX_LIMIT_INT32
from .spmm_csr import _SpmmPlan, _hip_spmm, _prepare_spmm_csr_matrix

SUPPORTED_SPMM_OPT_DTYPES = (torch.float32, torch.float64)
SUPPORTED_SPMM_OPT_ALG2_DTYPES = (torch.float32, torch.float64)

# Row-length bins of the plan histogram (bin b holds lengths in [2^(b-1), 2^b)).
_LONG_ROW_BIN = 12  # rows with >= 2048 nnz, the reference's long-row threshold (spmm_csr.py:2246)


class _PreparedBase:
    def _hip_plan(self):
        if self._plan is None and self.n_rows > 0:
            self._plan = _SpmmPlan(self.data, self.kernel_indices, self.kernel_indptr, self.n_rows, self.n_cols,
                                   kept=True)
        return self._plan


class PreparedCsrSpmmOpt(_PreparedBase):
    """Cached CSR metadata for repeated SpMM-opt calls on the same sparse matrix."""

    __slots__ = (
        "data",
        "kernel_indices",
        "kernel_indptr",
        "shape",
        "n_rows",
        "n_cols",
        "row_lengths",
        "max_row_nnz",
        "row_buckets",
        "supports_opt",
        "long_part_rows",
        "long_part_starts",
        "long_part_ends",
        "long_row_ids",
        "long_row_part_ptr",
        "long_row_fallback_only",
        "_plan",
    )

    def __init__(self, data, kernel_indices, kernel_indptr, shape, n_rows, n_cols, row_lengths, max_row_nnz,
                 row_buckets=None, long_part_rows=None, long_part_starts=None, long_part_ends=None,
                 long_row_ids=None, long_row_part_ptr=None, long_row_fallback_only=False):
        self.data = data
        self.kernel_indices = kernel_indices
        self.kernel_indptr = kernel_indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = int(n_rows)
        self.n_cols = int(n_cols)
        self.row_lengths = row_lengths
        self.max_row_nnz = int(max_row_nnz)
        self.row_buckets = [] if row_buckets is None else row_buckets
        self.supports_opt = data.dtype in SUPPORTED_SPMM_OPT_DTYPES
        dev = data.device
        row_index_dtype = torch.int32 if self.n_rows <= _INDEX_LIMIT_INT32 else torch.int64
        empty_rows = torch.empty((0,), dtype=row_index_dtype, device=dev)
        self.long_part_rows = empty_rows if long_part_rows is None else long_part_rows
        self.long_part_starts = (torch.empty((0,), dtype=torch.int64, device=dev)
                                 if long_part_starts is None else long_part_starts)
        self.long_part_ends = (torch.empty((0,), dtype=torch.int64, device=dev)
                               if long_part_ends is None else long_part_ends)
        self.long_row_ids = empty_rows if long_row_ids is None else long_row_ids
        self.long_row_part_ptr = (torch.zeros(1, dtype=torch.int64, device=dev)
                                  if long_row_part_ptr is None else long_row_part_ptr)
        self.long_row_fallback_only = bool(long_row_fallback_only)
        self._plan = None


class PreparedCsrSpmmOptAlg2(_PreparedBase):
    """Cached CSR metadata for repeated alg2 CSR SpMM calls on the same sparse matrix."""

    __slots__ = (
        "data",
        "kernel_indices",
        "kernel_indptr",
        "shape",
        "n_rows",
        "n_cols",
        "row_lengths",
        "max_row_nnz",
        "opt_buckets",
        "supports_opt",
        "_plan",
    )

    def __init__(self, data, kernel_indices, kernel_indptr, shape, n_rows, n_cols, row_lengths, max_row_nnz,
                 opt_buckets=None):
        self.data = data
        self.kernel_indices = kernel_indices
        self.kernel_indptr = kernel_indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = int(n_rows)
        self.n_cols = int(n_cols)
        self.row_lengths = row_lengths
        self.max_row_nnz = int(max_row_nnz)
        self.opt_buckets = [] if opt_buckets is None else opt_buckets
        self.supports_opt = data.dtype in SUPPORTED_SPMM_OPT_ALG2_DTYPES
        self._plan = None


def _prepared_fields(data, indices, indptr, shape):
    data, indices, indptr, n_rows, n_cols, _ = _prepare_spmm_csr_matrix(data, indices, indptr, shape)
    row_lengths = indptr[1:] - indptr[:-1] if n_rows > 0 else indptr.new_empty((0,))
    return data, indices, indptr, n_rows, n_cols, row_lengths


def prepare_spmm_csr_opt_alg1(data, indices, indptr, shape):
    data, indices, indptr, n_rows, n_cols, row_lengths = _prepared_fields(data, indices, indptr, shape)
    prepared = PreparedCsrSpmmOpt(data, indices, indptr, shape, n_rows, n_cols, row_lengths, 0)
    plan = prepared._hip_plan()
    prepared.max_row_nnz = plan.csr.max_row_nnz if plan is not None else 0
    return prepared


def prepare_spmm_csr_opt(data, indices, indptr, shape):
    return prepare_spmm_csr_opt_alg1(data, indices, indptr, shape)


def prepare_spmm_csr_opt_alg1_preprocess(data, indices, indptr, shape):
    return prepare_spmm_csr_opt_alg1(data, indices, indptr, shape)


def prepare_spmm_csr_opt_alg2(data, indices, indptr, shape):
    data, indices, indptr, n_rows, n_cols, row_lengths = _prepared_fields(data, indices, indptr, shape)
    prepared = PreparedCsrSpmmOptAlg2(data, indices, indptr, shape, n_rows, n_cols, row_lengths, 0)
    plan = prepared._hip_plan()
    prepared.max_row_nnz = plan.csr.max_row_nnz if plan is not None else 0
    return prepared


def prepare_spmm_csr_opt_alg2_preprocess(data, indices, indptr, shape):
    return prepare_spmm_csr_opt_alg2(data, indices, indptr, shape)


def _resolve_prepared(prepared, cls, prepare_fn, data, indices, indptr, shape):
    if prepared is not None and not isinstance(prepared, cls):
        raise TypeError(f"prepared must be a {cls.__name__} instance")
    if prepared is None:
        if any(arg is None for arg in (data, indices, indptr, shape)):
            raise ValueError("data, indices, indptr, and shape are required when prepared is not provided")
        return prepare_fn(data, indices, indptr, shape)
    if shape is not None:
        resolved = (int(shape[0]), int(shape[1]))
        if resolved != prepared.shape:
            raise ValueError(f"shape {resolved} does not match prepared.shape {prepared.shape}")
    return prepared


def _check_out(prepared, B, out):
    if out is not None:
        if not out.is_cuda:
            raise ValueError("out must be a CUDA tensor")
        if out.device != prepared.data.device:
            raise ValueError("out must be on the same CUDA device as sparse matrix data")
        if out.shape != (prepared.n_rows, int(B.shape[1])) or out.dtype != prepared.data.dtype:
            raise ValueError("out shape/dtype must match result")


def _run(prepared, B, out, do_timing):
    """Plan lookup (the 'symbolic' phase) + one SpMM; returns C, symbolic_ms, compute_ms."""
    symbolic_ms = compute_ms = None
    if do_timing:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    plan = prepared._hip_plan()
    if do_timing:
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        symbolic_ms = (t1 - t0) * 1000.0
    C = _hip_spmm(prepared.data, prepared.kernel_indices, prepared.kernel_indptr, B.contiguous(), prepared.n_rows,
                  plan, prepared.data.dtype)
    if do_timing:
        torch.cuda.synchronize()
        compute_ms = (time.perf_counter() - t1) * 1000.0
    if out is not None:
        out.copy_(C)
        C = out
    return C, plan, symbolic_ms, compute_ms


def _long_row_count(plan):
    if plan is None:
        return 0
    return int(sum(plan.csr.row_length_histogram[_LONG_ROW_BIN:]))


def _spmm_opt_alg1_impl(data, indices, indptr, B, shape, prepared, out, return_time, return_meta, api_name):
    prepared = _resolve_prepared(prepared, PreparedCsrSpmmOpt, prepare_spmm_csr_opt_alg1, data, indices, indptr,
                                 shape)
    if B is None:
        raise ValueError("B is required")
    if not prepared.supports_opt:
        raise TypeError(f"{api_name} only supports float32 and float64")
    if not B.is_cuda:
        raise ValueError("B must be a CUDA tensor")
    if B.device != prepared.data.device:
        raise ValueError("B must be on the same CUDA device as sparse matrix data")
    if B.dtype != prepared.data.dtype:
        raise TypeError("B dtype must match sparse matrix dtype")
    if B.ndim != 2:
        raise ValueError("B must be a 2D dense tensor")
    if B.shape[0] != prepared.n_cols:
        raise ValueError(f"B.shape[0] must be n_cols={prepared.n_cols}, got {B.shape[0]}")
    _check_out(prepared, B, out)
    do_timing = bool(return_time or return_meta)
    C, plan, symbolic_ms, compute_ms = _run(prepared, B, out, do_timing)
    op_total_ms = (symbolic_ms + compute_ms) if do_timing else None
    if return_meta:
        meta = {
            "symbolic_ms": symbolic_ms,
            "compute_ms": compute_ms,
            "op_total_ms": op_total_ms,
            "long_part_count": plan.tiling(prepared.data.dtype, B.shape[1])[1] if plan is not None else 0,
            "long_row_count": _long_row_count(plan),
            "bucket_count": 1 if plan is not None else 0,
        }
        if return_time:
            return C, op_total_ms, meta
        return C, meta
    if return_time:
        return C, op_total_ms
    return C


def flagsparse_spmm_csr_opt_alg1(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None, out=None,
                                 return_time=False, return_meta=False):
    """CSR SpMM-opt alg1 (float32 / float64) on the merge-path HIP kernel."""
    return _spmm_opt_alg1_impl(data, indices, indptr, B, shape, prepared, out, return_time, return_meta,
                               "flagsparse_spmm_csr_opt_alg1")


def flagsparse_spmm_csr_opt_alg1_preprocess(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None,
                                            out=None, return_time=False, return_meta=False):
    """Compatibility alias for CSR SpMM-opt alg1 with runtime preprocessing."""
    return _spmm_opt_alg1_impl(data, indices, indptr, B, shape, prepared, out, return_time, return_meta,
                               "flagsparse_spmm_csr_opt_alg1_preprocess")


def flagsparse_spmm_csr_opt(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None, out=None,
                            return_time=False, return_meta=False):
    """Compatibility alias for CSR SpMM-opt alg1."""
    return flagsparse_spmm_csr_opt_alg1(data=data, indices=indices, indptr=indptr, B=B, shape=shape,
                                        prepared=prepared, out=out, return_time=return_time,
                                        return_meta=return_meta)


def _validate_alg2(prepared, B, out):
    """spmm_csr_opt_alg2.py:759-780."""
    if not prepared.supports_opt:
        raise TypeError("flagsparse_spmm_csr_opt_alg2 only supports float32 and float64")
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
    _check_out(prepared, B, out)


def flagsparse_spmm_csr_opt_alg2(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None, out=None,
                                 return_time=False, return_meta=False):
    """CSR SpMM opt-alg2 (float32 / float64) on the merge-path HIP kernel."""
    prepared = _resolve_prepared(prepared, PreparedCsrSpmmOptAlg2, prepare_spmm_csr_opt_alg2, data, indices, indptr,
                                 shape)
    _validate_alg2(prepared, B, out)
    do_timing = bool(return_time or return_meta)
    C, plan, symbolic_ms, compute_ms = _run(prepared, B, out, do_timing)
    op_total_ms = (symbolic_ms + compute_ms) if do_timing else None
    if return_meta:
        meta = {
            "kernel": "spmm_group",
            "n_tiles": plan.tiling(prepared.data.dtype, B.shape[1])[1] if plan is not None else 0,
            "symbolic_ms": symbolic_ms,
            "compute_ms": compute_ms,
            "op_total_ms": op_total_ms,
        }
    if return_time and return_meta:
        return C, op_total_ms, meta
    if return_time:
        return C, op_total_ms
    if return_meta:
        return C, meta
    return C


def flagsparse_spmm_csr_opt_alg2_preprocess(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None,
                                            out=None, return_time=False, return_meta=False):
    """Compatibility alias for CSR SpMM opt-alg2 with runtime preprocessing."""
    return flagsparse_spmm_csr_opt_alg2(data=data, indices=indices, indptr=indptr, B=B, shape=shape,
                                        prepared=prepared, out=out, return_time=return_time,
                                        return_meta=return_meta)
