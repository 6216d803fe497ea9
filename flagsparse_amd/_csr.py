"""Device-side CSR helpers shared by SpMV and SpMM: analysis, merge-path
partition and the transpose, each one call into libflagsparse_hip.

These replace the reference's torch-op implementations:
  - transpose: _transpose_csr_for_spmv (spmv_csr.py:477-515) and
    _transpose_csr_for_spmm (spmm_csr.py:300-338);
  - row statistics / launch sizing: prepare_spmv_csr (spmv_csr.py:623-647),
    _resolve_spmm_base_triton_launch (spmm_csr.py:451-509).
"""

import torch

from . import _lib
from ._common import _INDEX_LIMIT_INT32, _compute_dtype, _is_complex_dtype


class CsrPlan:
    """Analysis result for one CSR matrix plus the device partition(s)."""

    __slots__ = ("plan", "device", "_parts", "carry")

    def __init__(self, plan, device):
        self.plan = plan
        self.device = device
        self._parts = {}
        self.carry = None

    @property
    def kernel_name(self):
        return _lib.KERNEL_NAMES.get(self.plan.kernel, "unknown")

    @property
    def max_row_nnz(self):
        return int(self.plan.max_row)

    @property
    def row_length_histogram(self):
        return [int(v) for v in self.plan.hist]

    @classmethod
    def from_sizes(cls, data, indices, indptr, n_rows, n_cols):
        """A plan from the matrix's sizes and types alone, with no device
        work: enough for launches that read no row statistics (the SpMM
        kernels); its statistics (max_row_nnz, histogram) are unset."""
        p = _lib.FsCsrPlan()
        p.n_rows, p.n_cols, p.nnz = int(n_rows), int(n_cols), int(data.numel())
        p.val_t = _lib.value_code(_compute_dtype(data.dtype))
        p.idx_t = _lib.index_code(indices.dtype)
        p.ptr_t = _lib.index_code(indptr.dtype)
        p.kernel = _lib.FS_KERNEL_MERGE
        p.max_row = -1
        return cls(p, indptr.device)

    def n_tiles(self, tile_items):
        p = self.plan
        total = int(p.n_rows) + int(p.nnz)
        return (total + tile_items - 1) // tile_items

    def partition(self, indptr, tile_items):
        """Merge-path tile starts for `tile_items` items per tile (cached)."""
        part = self._parts.get(tile_items)
        if part is None:
            n_tiles = self.n_tiles(tile_items)
            part = torch.empty(n_tiles + 1, dtype=torch.int64, device=self.device)
            _lib.check(
                _lib.lib().fs_csr_partition(
                    self.plan, _lib.ptr(indptr), _lib.ptr(part), tile_items, n_tiles,
                    _lib.stream_handle(self.device),
                ),
                "fs_csr_partition",
            )
            self._parts[tile_items] = part
        return part


def analyze_csr(data, indices, indptr, n_rows, n_cols, force_kernel=-1):
    """Row-length histogram on the device, kernel choice on the host."""
    device = indptr.device
    lib = _lib.lib()
    plan = _lib.FsCsrPlan()
    stats = _lib.workspace(lib.fs_csr_stats_bytes(), device)
    _lib.check(
        lib.fs_csr_analyze(
            _lib.ptr(indptr),
            _lib.index_code(indptr.dtype),
            _lib.index_code(indices.dtype),
            _lib.value_code(_compute_dtype(data.dtype)),
            int(n_rows),
            int(n_cols),
            int(data.numel()),
            int(force_kernel),
            _lib.ptr(stats),
            plan,
            _lib.stream_handle(device),
        ),
        "fs_csr_analyze",
    )
    return CsrPlan(plan, device)


def transpose_out_dtypes(indices_dtype, indptr_dtype, n_rows, nnz):
    """Output index dtype rules of the reference (spmv_csr.py:482-483, 508-509)."""
    out_index_dtype = indices_dtype if n_rows <= _INDEX_LIMIT_INT32 else torch.int64
    out_indptr_dtype = indptr_dtype if nnz <= _INDEX_LIMIT_INT32 else torch.int64
    return out_index_dtype, out_indptr_dtype


def transpose_csr(data, indices, indptr, shape, conj=False, compact=False, check=None):
    """CSR of A^T (A^H when conj and complex): stable by column, on device.

    Returns (t_data, t_indices, t_indptr, (n_cols, n_rows)).  The index
    dtypes follow the reference's rules; compact=True (for a transpose that
    stays inside an operator call) takes int32 wherever the values fit, which
    the kernels then read at half the bytes.  check: a pending structure
    check of this matrix (spmv_csr._PendingCheck) that the transpose runs in
    its own passes where it can (fs_csr_transpose_checked), else queues first.
    """
    n_rows, n_cols = int(shape[0]), int(shape[1])
    nnz = data.numel()
    device = data.device
    if data.dtype in (torch.float16, torch.bfloat16):
        # the permutation is exact through float32 (16-bit values round-trip)
        td, ti, tp, tsh = transpose_csr(data.to(torch.float32), indices, indptr, shape, conj=False, compact=compact,
                                        check=check)
        return td.to(data.dtype), ti, tp, tsh
    out_index_dtype, out_indptr_dtype = transpose_out_dtypes(indices.dtype, indptr.dtype, n_rows, nnz)
    if compact:
        out_index_dtype = torch.int32 if n_rows <= _INDEX_LIMIT_INT32 else torch.int64
        out_indptr_dtype = torch.int32 if nnz <= _INDEX_LIMIT_INT32 else torch.int64
    t_indptr = torch.empty(n_cols + 1, dtype=out_indptr_dtype, device=device)
    lib = _lib.lib()
    fused = None
    if check is not None:
        if nnz > 0 and n_rows > 0 and n_cols > 0 and lib.fs_csr_transpose_bounded(
                _lib.value_code(data.dtype), n_rows, n_cols, nnz):
            fused = check.fuse()
        else:
            check.queue()
    if nnz == 0:
        t_indptr.zero_()
        return (
            data,
            torch.empty(0, dtype=out_index_dtype, device=device),
            t_indptr,
            (n_cols, n_rows),
        )
    t_data = torch.empty_like(data)
    t_indices = torch.empty(nnz, dtype=out_index_dtype, device=device)
    ws = _lib.workspace(lib.fs_csr_transpose_workspace_bytes(n_rows, n_cols, nnz), device)
    do_conj = 1 if (conj and _is_complex_dtype(data.dtype)) else 0
    if fused is not None:
        _lib.check(
            lib.fs_csr_transpose_checked(
                _lib.value_code(data.dtype), _lib.index_code(indices.dtype), _lib.index_code(indptr.dtype),
                _lib.index_code(out_index_dtype), _lib.index_code(out_indptr_dtype), n_rows, n_cols, nnz,
                _lib.ptr(data), _lib.ptr(indices), _lib.ptr(indptr), do_conj, _lib.ptr(t_data), _lib.ptr(t_indices),
                _lib.ptr(t_indptr), _lib.ptr(ws), ws.numel(), fused[0], fused[1], _lib.stream_handle(device),
            ),
            "fs_csr_transpose_checked",
        )
        return t_data, t_indices, t_indptr, (n_cols, n_rows)
    _lib.check(
        lib.fs_csr_transpose(
            _lib.value_code(data.dtype),
            _lib.index_code(indices.dtype),
            _lib.index_code(indptr.dtype),
            _lib.index_code(out_index_dtype),
            _lib.index_code(out_indptr_dtype),
            n_rows,
            n_cols,
            nnz,
            _lib.ptr(data),
            _lib.ptr(indices),
            _lib.ptr(indptr),
            do_conj,
            _lib.ptr(t_data),
            _lib.ptr(t_indices),
            _lib.ptr(t_indptr),
            _lib.ptr(ws),
            ws.numel(),
            _lib.stream_handle(device),
        ),
        "fs_csr_transpose",
    )
    return t_data, t_indices, t_indptr, (n_cols, n_rows)
