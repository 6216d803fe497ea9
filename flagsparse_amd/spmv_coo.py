"""COO SpMV on the HIP kernels (reference: sparse_operations/spmv_coo.py).

The reference keeps a lex-sorted COO (row, col) plus row-run offsets
("seg_starts") and runs one Triton program per row run, or an atomic grid
over the nnz when ``sort_by_row=False`` (spmv_coo.py:1-9, 192-355).  Here
prepare sorts the entries on the device (the stable radix sort behind
``fs_coo_to_csr``) and keeps, next to the reference's fields, the row
pointer of the sorted entries, so a launch is one call of the CSR SpMV
kernels: nnz-balanced, short rows and power-law rows alike, no atomics and
bit-reproducible run to run.  ``sort_by_row=False`` keeps the caller's
order in the prepared fields (as the reference does) and still computes
through the sorted copy.

Public surface, argument meaning and error messages follow the reference:
  prepare_spmv_coo / PreparedCoo         spmv_coo.py:77-135, 425-474
  flagsparse_spmv_coo                    spmv_coo.py:726-810
  validation                             spmv_coo.py:390-422, 557-572
  int64 -> int32 launch fallback         spmv_coo.py:647-723
Numerics: float32 is accumulated in float64 and rounded once, complex64 in
complex128 (the reference accumulates both in single precision,
spmv_coo.py:192-355; the results agree within its tolerances).
"""

import time

import torch

from ._common import _INDEX_LIMIT_INT32, SUPPORTED_INDEX_DTYPES
from .coo import coo_to_csr_for_spmv
from .spmv_csr import _hip_spmv_csr_impl_prepared, _prepare_spmv

SUPPORTED_SPMV_COO_VALUE_DTYPES = (
    torch.float32,
    torch.float64,
    torch.complex64,
    torch.complex128,
)

SPMV_COO_OP_NON = 0
SPMV_COO_OP_TRANS = 1
SPMV_COO_OP_CONJ_TRANS = 2
SPMV_COO_OP_NAMES = {
    SPMV_COO_OP_NON: "non",
    SPMV_COO_OP_TRANS: "trans",
    SPMV_COO_OP_CONJ_TRANS: "conj",
}
_SPMV_COO_OP_NAME_TO_CODE = {name: code for code, name in SPMV_COO_OP_NAMES.items()}


def _spmv_coo_dtype_error_message():
    return "COO SpMV supports float32, float64, complex64, and complex128"


def _normalize_spmv_coo_op(op=None, transpose=False):
    """spmv_coo.py:41-55."""
    if op is None:
        return SPMV_COO_OP_TRANS if bool(transpose) else SPMV_COO_OP_NON
    if isinstance(op, str):
        token = op.strip().lower()
        if token not in _SPMV_COO_OP_NAME_TO_CODE:
            raise ValueError("op must be one of: 0=non, 1=trans, 2=conj")
        return _SPMV_COO_OP_NAME_TO_CODE[token]
    try:
        op_code = int(op)
    except (TypeError, ValueError) as exc:
        raise ValueError("op must be one of: 0=non, 1=trans, 2=conj") from exc
    if op_code not in SPMV_COO_OP_NAMES:
        raise ValueError("op must be one of: 0=non, 1=trans, 2=conj")
    return op_code


def _spmv_coo_op_to_name(op):
    return SPMV_COO_OP_NAMES[_normalize_spmv_coo_op(op)]


def _spmv_coo_op_transposes(op):
    return _normalize_spmv_coo_op(op) in (SPMV_COO_OP_TRANS, SPMV_COO_OP_CONJ_TRANS)


def _normalize_spmv_coo_index_fallback_policy(index_fallback_policy):
    policy = str(index_fallback_policy).lower()
    if policy not in ("auto", "strict"):
        raise ValueError("index_fallback_policy must be 'auto' or 'strict'")
    return policy


class _SortedCoo:
    """One orientation of the matrix, sorted by (row, col): the reference's
    (data, row, col, seg_starts) plus the row pointer the kernels walk."""

    __slots__ = ("data", "row", "col", "seg_starts", "indptr", "shape", "one_shot", "_csr", "_conj_csr")

    def __init__(self, data, row, col, seg_starts, indptr, shape):
        self.data = data
        self.row = row
        self.col = col
        self.seg_starts = seg_starts
        self.indptr = indptr
        self.shape = shape
        self.one_shot = False  # True for a single unprepared call: no column-panel copy
        self._csr = None
        self._conj_csr = None

    def csr(self, conj=False):
        """Prepared CSR SpMV over the sorted entries (built once per orientation)."""
        if conj:
            if self._conj_csr is None:
                data = self.data.conj().resolve_conj().contiguous()
                self._conj_csr = self._prepare(data)
            return self._conj_csr
        if self._csr is None:
            self._csr = self._prepare(self.data)
        return self._csr

    def _prepare(self, data):
        return _prepare_spmv(data, self.col, self.indptr, self.shape, 256, None, False, None, "auto",
                             one_shot=self.one_shot)


def _seg_starts_from_indptr(indptr, nnz, index_dtype):
    """Row-run boundaries of the sorted entries (spmv_coo.py:372-387): the start
    of every non-empty row, then nnz; None for an empty matrix."""
    if nnz == 0:
        return None
    if nnz > _INDEX_LIMIT_INT32:
        index_dtype = torch.int64
    starts = indptr[:-1][indptr[1:] > indptr[:-1]]
    tail = torch.tensor([nnz], dtype=torch.int64, device=indptr.device)
    return torch.cat([starts, tail]).to(index_dtype)


def _sort_coo(data, row, col, shape, index_dtype):
    """Sorted orientation: device radix sort on row * n_cols + col."""
    n_rows = int(shape[0])
    data_s, cols32, indptr = coo_to_csr_for_spmv(data, row, col, shape)
    nnz = data_s.numel()
    counts = indptr[1:] - indptr[:-1]
    row_s = torch.repeat_interleave(torch.arange(n_rows, dtype=index_dtype, device=data.device), counts)
    col_s = cols32.to(index_dtype)
    seg = _seg_starts_from_indptr(indptr, nnz, index_dtype)
    return _SortedCoo(data_s, row_s, col_s, seg, indptr, (int(shape[0]), int(shape[1])))


def _prepare_coo_tensors(data, row, col, shape):
    """Checks of spmv_coo.py:390-422, in the same order and with the same messages."""
    if not all(torch.is_tensor(t) for t in (data, row, col)):
        raise TypeError("data, row, col must all be torch.Tensor")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1:
        raise ValueError("data, row, col must be 1D")
    if not all(t.is_cuda for t in (data, row, col)):
        raise ValueError("data, row, col must be CUDA tensors")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if data.numel() != row.numel() or data.numel() != col.numel():
        raise ValueError("data, row, col must have the same length")
    if data.dtype not in SUPPORTED_SPMV_COO_VALUE_DTYPES:
        raise TypeError(_spmv_coo_dtype_error_message())
    if row.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("row dtype must be torch.int32 or torch.int64")
    if col.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("col dtype must be torch.int32 or torch.int64")
    if data.numel() > 0:
        lo_hi = torch.stack(
            [row.min().to(torch.int64), row.max().to(torch.int64), col.min().to(torch.int64), col.max().to(torch.int64)]
        ).cpu().tolist()
        if lo_hi[0] < 0 or lo_hi[1] >= n_rows:
            raise IndexError("row indices out of range")
        if lo_hi[2] < 0 or lo_hi[3] >= n_cols:
            raise IndexError("col indices out of range")
    if n_rows > _INDEX_LIMIT_INT32 or n_cols > _INDEX_LIMIT_INT32:
        # the sort emits int32 column indices (as coo_to_csr_for_spmv does)
        raise ValueError("COO SpMV here supports n_rows and n_cols up to 2**31 - 1")
    return torch.promote_types(row.dtype, col.dtype)


class PreparedCoo:
    """Prepared COO structure that serves non / trans / conj (spmv_coo.py:77-135).

    data_non / row_non / col_non / seg_starts_non: the entries sorted by
    (row, col) when sort_by_row, else the caller's order with no seg_starts;
    the *_trans fields are the same for A^T.
    """

    __slots__ = (
        "data_non",
        "row_non",
        "col_non",
        "seg_starts_non",
        "data_trans",
        "row_trans",
        "col_trans",
        "seg_starts_trans",
        "shape",
        "n_rows",
        "n_cols",
        "nnz",
        "sort_by_row",
        "op",
        "transpose",
        "index_fallback_policy",
        "index_fallback_applied",
        "index_fallback_reason",
        "_sorted_non",
        "_sorted_trans",
    )

    def __init__(self, sorted_non, sorted_trans, shape, raw=None, sort_by_row=True, transpose=False, op=None,
                 index_fallback_policy="auto"):
        self._sorted_non = sorted_non
        self._sorted_trans = sorted_trans
        if sort_by_row:
            self.data_non, self.row_non, self.col_non = sorted_non.data, sorted_non.row, sorted_non.col
            self.seg_starts_non = sorted_non.seg_starts
            self.data_trans, self.row_trans, self.col_trans = sorted_trans.data, sorted_trans.row, sorted_trans.col
            self.seg_starts_trans = sorted_trans.seg_starts
        else:
            data, row, col = raw
            self.data_non, self.row_non, self.col_non = data, row, col
            self.seg_starts_non = None
            self.data_trans, self.row_trans, self.col_trans = data, col, row
            self.seg_starts_trans = None
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows, self.n_cols = self.shape
        self.nnz = int(self.data_non.numel())
        self.sort_by_row = bool(sort_by_row)
        self.op = _normalize_spmv_coo_op(op, transpose=transpose)
        self.transpose = _spmv_coo_op_transposes(self.op)
        self.index_fallback_policy = str(index_fallback_policy).lower()
        self.index_fallback_applied = False
        self.index_fallback_reason = None


class _PreparedCooLaunch:
    """Launch view of one op on a prepared structure (spmv_coo.py:138-189)."""

    __slots__ = (
        "data",
        "row",
        "col",
        "shape",
        "n_rows",
        "n_cols",
        "nnz",
        "seg_starts",
        "n_segs",
        "use_seg_kernel",
        "op",
        "transpose",
        "index_fallback_policy",
        "index_fallback_applied",
        "index_fallback_reason",
        "sorted",
        "conj",
    )

    def __init__(self, sorted_coo, data, row, col, shape, seg_starts=None, op=SPMV_COO_OP_NON, conj=False,
                 index_fallback_policy="auto", index_fallback_applied=False, index_fallback_reason=None):
        self.sorted = sorted_coo
        self.conj = bool(conj)
        self.data = data
        self.row = row
        self.col = col
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows, self.n_cols = self.shape
        self.nnz = int(data.numel())
        self.seg_starts = seg_starts
        self.n_segs = 0 if seg_starts is None else int(seg_starts.numel()) - 1
        self.use_seg_kernel = self.n_segs > 0
        self.op = _normalize_spmv_coo_op(op)
        self.transpose = _spmv_coo_op_transposes(self.op)
        self.index_fallback_policy = str(index_fallback_policy).lower()
        self.index_fallback_applied = bool(index_fallback_applied)
        self.index_fallback_reason = index_fallback_reason


def prepare_spmv_coo(data, row, col, shape, sort_by_row=True, transpose=False, op=None, index_fallback_policy="auto"):
    """Sort both orientations once and cache them (spmv_coo.py:425-474)."""
    index_fallback_policy = _normalize_spmv_coo_index_fallback_policy(index_fallback_policy)
    op_code = _normalize_spmv_coo_op(op, transpose=transpose)
    if op is not None and bool(transpose) and op_code == SPMV_COO_OP_NON:
        raise ValueError("transpose=True conflicts with op=non")
    shape = (int(shape[0]), int(shape[1]))
    index_dtype = _prepare_coo_tensors(data, row, col, shape)
    data_c = data.contiguous()
    row_c = row.to(index_dtype).contiguous()
    col_c = col.to(index_dtype).contiguous()
    sorted_non = _sort_coo(data_c, row_c, col_c, shape, index_dtype)
    sorted_trans = _sort_coo(data_c, col_c, row_c, (shape[1], shape[0]), index_dtype)
    return PreparedCoo(sorted_non, sorted_trans, shape, raw=(data_c, row_c, col_c), sort_by_row=sort_by_row,
                       transpose=transpose, op=op_code, index_fallback_policy=index_fallback_policy)


def _resolve_spmv_coo_launch(prepared, op):
    """spmv_coo.py:525-554: op=conj conjugates the transposed data at launch."""
    op_code = _normalize_spmv_coo_op(op)
    common = dict(
        op=op_code,
        index_fallback_policy=prepared.index_fallback_policy,
        index_fallback_applied=prepared.index_fallback_applied,
        index_fallback_reason=prepared.index_fallback_reason,
    )
    if op_code == SPMV_COO_OP_NON:
        return _PreparedCooLaunch(prepared._sorted_non, prepared.data_non, prepared.row_non, prepared.col_non,
                                  prepared.shape, seg_starts=prepared.seg_starts_non, **common)
    conj = op_code == SPMV_COO_OP_CONJ_TRANS and prepared.data_trans.dtype.is_complex
    return _PreparedCooLaunch(prepared._sorted_trans, prepared.data_trans, prepared.row_trans, prepared.col_trans,
                              (prepared.n_cols, prepared.n_rows), seg_starts=prepared.seg_starts_trans, conj=conj,
                              **common)


def _validate_x_coo(x, launch):
    """spmv_coo.py:557-572."""
    if x is None or not torch.is_tensor(x):
        raise TypeError("x must be a torch.Tensor")
    if x.ndim != 1:
        raise ValueError("x must be a 1D tensor")
    if not x.is_cuda:
        raise ValueError("x must be a CUDA tensor")
    if x.dtype != launch.data.dtype:
        raise TypeError("x dtype must match sparse matrix dtype")
    if x.numel() != launch.n_cols:
        raise ValueError(f"x length must be n_cols={launch.n_cols}, got {x.numel()}")
    if x.device != launch.data.device:
        raise ValueError("x must be on the same device as sparse matrix data")
    return x.contiguous()


def _hip_spmv_coo_kernel(launch, x, block_size, num_warps, block_inner):
    """One launch (replaces _triton_spmv_coo_kernel, spmv_coo.py:575-644): the
    CSR SpMV kernels over the sorted entries of the launch's orientation."""
    if launch.n_rows == 0:
        return torch.zeros(0, dtype=launch.data.dtype, device=launch.data.device)
    return _hip_spmv_csr_impl_prepared(launch.sorted.csr(conj=launch.conj), x)


def _spmv_coo_uses_int64_indices(launch):
    return (
        launch.row.dtype == torch.int64
        or launch.col.dtype == torch.int64
        or (launch.seg_starts is not None and launch.seg_starts.dtype == torch.int64)
    )


def _spmv_coo_int32_fallback_blocker(launch):
    """spmv_coo.py:658-674."""
    for name, tensor in (("row", launch.row), ("col", launch.col)):
        if tensor.numel() > 0:
            lo_hi = torch.stack([tensor.min(), tensor.max()]).cpu().tolist()
            min_index, max_index = int(lo_hi[0]), int(lo_hi[1])
            if min_index < 0 or max_index > _INDEX_LIMIT_INT32:
                return f"{name} index range [{min_index}, {max_index}] cannot fit int32 for shape={launch.shape}"
    if launch.seg_starts is not None and launch.seg_starts.numel() > 0:
        max_offset = int(launch.seg_starts[-1].item())
        if max_offset > _INDEX_LIMIT_INT32:
            return f"COO nnz offset {max_offset} cannot fit int32 for shape={launch.shape}"
    if launch.n_rows > _INDEX_LIMIT_INT32 or launch.n_cols > _INDEX_LIMIT_INT32:
        return f"shape {launch.shape} cannot fit int32 row/col metadata"
    return None


def _spmv_coo_prepared_with_int32_indices(launch, reason):
    """spmv_coo.py:677-698: the same launch with int32 row / col / seg_starts."""
    blocker = _spmv_coo_int32_fallback_blocker(launch)
    if blocker is not None:
        raise RuntimeError(f"native int64 COO SpMV failed and int32 fallback is unsafe: {blocker}")
    seg = None if launch.seg_starts is None else launch.seg_starts.to(torch.int32).contiguous()
    srt = launch.sorted
    sorted32 = _SortedCoo(srt.data, srt.row.to(torch.int32), srt.col.to(torch.int32),
                          None if srt.seg_starts is None else srt.seg_starts.to(torch.int32), srt.indptr.to(torch.int32),
                          srt.shape)
    return _PreparedCooLaunch(sorted32, launch.data, launch.row.to(torch.int32).contiguous(),
                              launch.col.to(torch.int32).contiguous(), launch.shape, seg_starts=seg, op=launch.op,
                              conj=launch.conj, index_fallback_policy=launch.index_fallback_policy,
                              index_fallback_applied=True, index_fallback_reason=str(reason))


def _run_spmv_coo_prepared_with_fallback(launch, x, block_size, num_warps, block_inner):
    """spmv_coo.py:701-723."""
    try:
        return _hip_spmv_coo_kernel(launch, x, block_size, num_warps, block_inner)
    except Exception as exc:
        if launch.index_fallback_policy != "auto" or not _spmv_coo_uses_int64_indices(launch):
            raise
        fallback = _spmv_coo_prepared_with_int32_indices(launch, exc)
        return _hip_spmv_coo_kernel(fallback, x, block_size, num_warps, block_inner)


def flagsparse_spmv_coo(
    data=None,
    row=None,
    col=None,
    x=None,
    shape=None,
    out=None,
    return_time=False,
    prepared=None,
    sort_by_row=True,
    block_size=256,
    num_warps=4,
    block_inner=128,
    transpose=None,
    op=None,
    index_fallback_policy="auto",
):
    """COO SpMV y = op(A) @ x (spmv_coo.py:726-810).

    block_size / num_warps / block_inner keep the reference's validation;
    the HIP kernels size their own tiles.  Returns y or (y, ms).
    """
    transpose_flag = False if transpose is None else bool(transpose)
    op_explicit = op is not None
    op_code = _normalize_spmv_coo_op(op, transpose=transpose_flag)
    if op_explicit and transpose is not None and bool(transpose) != _spmv_coo_op_transposes(op_code):
        raise ValueError("transpose conflicts with op")
    if prepared is None:
        if any(a is None for a in (data, row, col, x, shape)):
            raise ValueError("data, row, col, x, shape required when prepared is None")
        prepared = prepare_spmv_coo(data, row, col, shape, sort_by_row=sort_by_row, transpose=transpose_flag, op=op,
                                    index_fallback_policy=index_fallback_policy)
        for srt in (prepared._sorted_non, prepared._sorted_trans):
            if srt is not None:
                srt.one_shot = True
    else:
        if x is None:
            raise TypeError("x is required when prepared is set")
        if shape is None:
            shape = prepared.shape
        sh = (int(shape[0]), int(shape[1]))
        if sh != prepared.shape:
            raise ValueError(f"shape {sh} does not match prepared.shape {prepared.shape}")
        if not op_explicit and transpose is None:
            op_code = prepared.op
        elif not op_explicit and transpose is not None:
            op_code = _normalize_spmv_coo_op(None, transpose=transpose_flag)
    launch = _resolve_spmv_coo_launch(prepared, op_code)
    x = _validate_x_coo(x, launch)
    if num_warps not in (1, 2, 4, 8, 16, 32):
        raise ValueError("num_warps must be a power of 2 in [1, 32]")
    if block_inner <= 0 or (block_inner & (block_inner - 1)) != 0:
        raise ValueError("block_inner must be a positive power of 2")
    t0 = None
    if return_time:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    y = _run_spmv_coo_prepared_with_fallback(launch, x, block_size=block_size, num_warps=num_warps,
                                             block_inner=block_inner)
    elapsed_ms = None
    if return_time:
        torch.cuda.synchronize()
        elapsed_ms = (time.perf_counter() - t0) * 1000.0
    if out is not None:
        if out.shape != y.shape or out.dtype != y.dtype:
            raise ValueError("out shape/dtype must match result")
        out.copy_(y)
        y = out
    if return_time:
        return y, elapsed_ms
    return y


__all__ = ["PreparedCoo", "prepare_spmv_coo", "flagsparse_spmv_coo", "SUPPORTED_SPMV_COO_VALUE_DTYPES"]
