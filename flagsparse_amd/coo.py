"""COO -> CSR conversion and COO SpMV through CSR, on the HIP path.

Mirrors the reference's COO convenience layer in spmv_csr.py:
  coo_to_csr_for_spmv          spmv_csr.py:926-950
  prepare_spmv_coo_tocsr       spmv_csr.py:953-981
  flagsparse_spmv_coo_tocsr    spmv_csr.py:984-1057
The conversion is one call into libflagsparse_hip (fs_coo_to_csr): a stable
device radix sort on the key row * n_cols + col, column indices returned as
int32 and the row pointer as int64, like the reference.  For input without
duplicate (row, col) pairs the result is identical to the reference's; with
duplicates the stable sort keeps their input order (the reference's
non-stable argsort leaves it unspecified).
"""

import torch

from . import _lib
from .spmv_csr import (
    SUPPORTED_SPMV_VALUE_DTYPES,
    _spmv_dtype_error_message,
    flagsparse_spmv_csr,
    prepare_spmv_csr,
)


def coo_to_csr_for_spmv(data, row, col, shape, assume_sorted=False):
    """Convert COO to the CSR triple (data, int32 col indices, int64 indptr)."""
    n_rows, n_cols = int(shape[0]), int(shape[1])
    device = data.device
    nnz = row.numel()
    indptr = torch.empty(n_rows + 1, dtype=torch.int64, device=device)
    if nnz == 0:
        indptr.zero_()
        return data, col.to(torch.int32), indptr
    idx_dtype = torch.int64 if (row.dtype == torch.int64 or col.dtype == torch.int64) else torch.int32
    row_k = row.to(idx_dtype).contiguous()
    col_k = col.to(idx_dtype).contiguous()
    data_k = data.contiguous()
    out_data = torch.empty_like(data_k)
    out_cols = torch.empty(nnz, dtype=torch.int32, device=device)
    lib = _lib.lib()
    ws = _lib.workspace(lib.fs_coo_to_csr_workspace_bytes(n_rows, n_cols, nnz), device)
    _lib.check(
        lib.fs_coo_to_csr(
            _lib.value_code(data_k.dtype),
            _lib.index_code(idx_dtype),
            n_rows,
            n_cols,
            nnz,
            _lib.ptr(data_k),
            _lib.ptr(row_k),
            _lib.ptr(col_k),
            1 if assume_sorted else 0,
            _lib.ptr(out_data),
            _lib.ptr(out_cols),
            _lib.ptr(indptr),
            _lib.ptr(ws),
            ws.numel(),
            _lib.stream_handle(device),
        ),
        "fs_coo_to_csr",
    )
    return out_data, out_cols, indptr


def prepare_spmv_coo_tocsr(data, row, col, shape, block_nnz=256, max_segments=None, assume_sorted=False):
    """One-time COO -> CSR + analysis; use with flagsparse_spmv_coo_tocsr(..., prepared=p)."""
    if not all(torch.is_tensor(t) for t in (data, row, col)):
        raise TypeError("data, row, col must all be torch.Tensor")
    if not all(t.is_cuda for t in (data, row, col)):
        raise ValueError("data, row, col must all be CUDA tensors")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1:
        raise ValueError("data, row, col must all be 1D tensors")
    if data.dtype not in SUPPORTED_SPMV_VALUE_DTYPES:
        raise TypeError(_spmv_dtype_error_message())
    if row.numel() != col.numel() or data.numel() != row.numel():
        raise ValueError("data, row, col must have the same length")
    data_s, indices, indptr = coo_to_csr_for_spmv(data, row, col, shape, assume_sorted=assume_sorted)
    return prepare_spmv_csr(data_s, indices, indptr, shape, block_nnz=block_nnz, max_segments=max_segments)


def flagsparse_spmv_coo_tocsr(data=None, row=None, col=None, x=None, shape=None, block_nnz=256, max_segments=None,
                              out=None, return_time=False, use_opt=True, prepared=None, assume_sorted=False):
    """COO SpMV via CSR conversion: y = A @ x (spmv_csr.py:984-1057)."""
    if prepared is not None:
        if x is None:
            raise TypeError("x is required")
        if shape is None:
            shape = prepared.shape
        sh = (int(shape[0]), int(shape[1]))
        if sh != prepared.shape:
            raise ValueError(f"shape {sh} does not match prepared.shape {prepared.shape}")
        return flagsparse_spmv_csr(x=x, shape=shape, block_nnz=block_nnz, max_segments=max_segments, out=out,
                                   return_time=return_time, use_opt=use_opt, prepared=prepared)
    if not all(torch.is_tensor(t) for t in (data, row, col, x)):
        raise TypeError("data, row, col, x must all be torch.Tensor")
    if not all(t.is_cuda for t in (data, row, col, x)):
        raise ValueError("data, row, col, x must all be CUDA tensors")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1 or x.ndim != 1:
        raise ValueError("data, row, col, x must all be 1D tensors")
    if data.dtype not in SUPPORTED_SPMV_VALUE_DTYPES:
        raise TypeError(_spmv_dtype_error_message())
    if x.dtype != data.dtype:
        raise TypeError("x dtype must match data dtype")
    data_s, indices, indptr = coo_to_csr_for_spmv(data, row, col, shape, assume_sorted=assume_sorted)
    return flagsparse_spmv_csr(data_s, indices, indptr, x, shape, block_nnz=block_nnz, max_segments=max_segments,
                               out=out, return_time=return_time, use_opt=use_opt)
