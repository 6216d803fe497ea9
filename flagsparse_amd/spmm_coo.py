"""COO SpMM C = A @ B on the HIP kernels (reference: sparse_operations/spmm_coo.py).

The reference coalesces duplicate (row, col) entries, lex-sorts them and
runs a row-run Triton kernel (complex dtypes through an atomic kernel),
spmm_coo.py:101-142, 417-595.  Here one device radix sort
(``fs_coo_to_csr``, stable on row * n_cols + col) turns the COO into the
CSR the SpMM kernels walk; duplicates stay separate entries of the same
row, which is the same product up to rounding (the sum distributes), and
the merge-path SpMM kernel accumulates them in a fixed order (no atomics,
bit-reproducible).

Signature, argument checks and messages follow
``flagsparse_spmm_coo`` / ``_prepare_spmm_coo_inputs`` / ``_run_spmm_coo_route``
(spmm_coo.py:335-395, 597-724).  Compute precision: float16 / bfloat16 in
float32, float32 in float64, complex64 in complex128 components, as the
reference's compute-dtype rule (spmm_coo.py:11-18).
"""

import time

import torch

from ._common import _INDEX_LIMIT_INT32, SUPPORTED_INDEX_DTYPES
from .coo import coo_to_csr_for_spmv
from .spmm_csr import SUPPORTED_SPMM_VALUE_DTYPES, flagsparse_spmm_csr


def _prepare_spmm_coo_inputs(data, row, col, B, shape):
    """spmm_coo.py:335-394 (checks in the same order, same messages)."""
    if len(shape) != 2:
        raise ValueError("shape must be a 2-tuple: (n_rows, n_cols)")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1:
        raise ValueError("data, row, and col must be 1D tensors")
    if B.ndim != 2:
        raise ValueError("B must be a 2D dense tensor")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if n_rows < 0 or n_cols < 0:
        raise ValueError("shape dimensions must be non-negative")
    if data.numel() != row.numel() or data.numel() != col.numel():
        raise ValueError("data, row, and col must have the same length (nnz)")
    if B.shape[0] != n_cols:
        raise ValueError(f"B.shape[0] must be n_cols={n_cols}, got {B.shape[0]}")
    if not all(t.is_cuda for t in (data, row, col, B)):
        raise ValueError("data, row, col, and B must be CUDA tensors")
    if not all(t.device == data.device for t in (row, col, B)):
        raise ValueError("data, row, col, and B must be on the same CUDA device")
    if data.dtype not in SUPPORTED_SPMM_VALUE_DTYPES:
        raise TypeError("data dtype must be one of: float16, bfloat16, float32, float64, complex64, complex128")
    if B.dtype != data.dtype:
        raise TypeError("B dtype must match data dtype")
    if row.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("row dtype must be torch.int32 or torch.int64")
    if col.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("col dtype must be torch.int32 or torch.int64")
    nnz = data.numel()
    if nnz > _INDEX_LIMIT_INT32:
        # same limit and message as the reference's COO kernel contract
        raise ValueError("nnz exceeds the int32 range supported by the Triton COO kernel")
    if nnz > 0:
        lo_hi = torch.stack(
            [row.min().to(torch.int64), row.max().to(torch.int64), col.min().to(torch.int64), col.max().to(torch.int64)]
        ).cpu().tolist()
        min_row, max_row, min_col, max_col = (int(v) for v in lo_hi)
        if min_row < 0 or max_row >= n_rows:
            raise IndexError("row indices out of range for n_rows")
        if min_col < 0 or max_col >= n_cols:
            raise IndexError("col indices out of range for n_cols")
        if max_row > _INDEX_LIMIT_INT32:
            raise ValueError("row indices exceed the int32 range supported by the Triton kernel")
        if max_col > _INDEX_LIMIT_INT32:
            raise ValueError("column indices exceed the int32 range supported by the Triton kernel")
    return data.contiguous(), row.contiguous(), col.contiguous(), B.contiguous(), n_rows, n_cols, int(B.shape[1])


def _check_out(out, device, n_rows, n_dense, dtype):
    """spmm_coo.py:619-625."""
    if not out.is_cuda:
        raise ValueError("out must be a CUDA tensor")
    if out.device != device:
        raise ValueError("out must be on the same CUDA device as the inputs")
    if out.shape != (n_rows, n_dense) or out.dtype != dtype:
        raise ValueError("out shape/dtype must match result")


def flagsparse_spmm_coo(data, row, col, B, shape, block_n=None, block_nnz=256, out=None, return_time=False):
    """COO SpMM: C = A @ B (spmm_coo.py:696-723).  No op argument, like the
    reference.  Returns C, or (C, ms) with return_time."""
    if block_n is not None and block_n <= 0:
        raise ValueError("block_n must be positive when provided")
    if block_nnz is not None and block_nnz <= 0:
        raise ValueError("block_nnz must be positive when provided")
    data, row, col, B, n_rows, n_cols, n_dense = _prepare_spmm_coo_inputs(data, row, col, B, shape)
    if out is not None:
        _check_out(out, data.device, n_rows, n_dense, data.dtype)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    idx_dtype = torch.promote_types(row.dtype, col.dtype)
    # float16 / bfloat16 are sorted and multiplied as float32 (their compute
    # dtype), and the result is cast back to the input dtype
    half = data.dtype in (torch.float16, torch.bfloat16)
    data_k = data.to(torch.float32) if half else data
    B_k = B.to(torch.float32) if half else B
    d, c32, indptr = coo_to_csr_for_spmv(data_k, row.to(idx_dtype), col.to(idx_dtype), (n_rows, n_cols))
    C = flagsparse_spmm_csr(d, c32, indptr, B_k, (n_rows, n_cols), block_nnz=block_nnz)
    if half:
        C = C.to(data.dtype)
    torch.cuda.synchronize()
    elapsed_ms = (time.perf_counter() - t0) * 1000.0
    if out is not None:
        out.copy_(C)
        C = out
    if return_time:
        return C, elapsed_ms
    return C


__all__ = ["flagsparse_spmm_coo"]
