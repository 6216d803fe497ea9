"""CSR SpMV operators: the reference's public API on gfx950 HIP kernels.

Public surface and behaviour follow src/flagsparse/sparse_operations/
spmv_csr.py of the reference:
  flagsparse_spmv_csr            spmv_csr.py:813-913
  prepare_spmv_csr               spmv_csr.py:591-664
  PreparedCsrSpmv                spmv_csr.py:55-130
  op normalisation               spmv_csr.py:29-52
  validation                     spmv_csr.py:518-588
  int64 -> int32 index fallback  spmv_csr.py:464-468, 726-810
  COO -> CSR convenience         spmv_csr.py:916-1057
Error types and messages are the reference's, so its contract tests apply
unchanged.  The device work (transpose, analysis, SpMV) is one call each
into libflagsparse_hip; there is no CPU path.
"""

import ctypes
import os
import threading
import time

import numpy as np
import torch

from . import _lib
from ._common import (
    _INDEX_LIMIT_INT32,
    HIP_VALUE_DTYPES,
    SUPPORTED_INDEX_DTYPES,
    _compute_dtype,
)
from ._csr import CsrPlan, analyze_csr, transpose_csr

SUPPORTED_SPMV_VALUE_DTYPES = (
    torch.float16,
    torch.bfloat16,
    torch.float32,
    torch.float64,
    torch.complex64,
    torch.complex128,
)

SPMV_OP_NON = 0
SPMV_OP_TRANS = 1
SPMV_OP_CONJ_TRANS = 2
SPMV_OP_NAMES = {
    SPMV_OP_NON: "non",
    SPMV_OP_TRANS: "trans",
    SPMV_OP_CONJ_TRANS: "conj",
}
_SPMV_OP_NAME_TO_CODE = {name: code for code, name in SPMV_OP_NAMES.items()}
_OP_ERROR = "op must be one of: 0=non, 1=trans, 2=conj"


def _normalize_spmv_op(op=None, transpose=False):
    """None -> trans if transpose else non; 'non'|'trans'|'conj' or 0|1|2."""
    if op is None:
        return SPMV_OP_TRANS if bool(transpose) else SPMV_OP_NON
    if isinstance(op, str):
        code = _SPMV_OP_NAME_TO_CODE.get(op.strip().lower())
        if code is None:
            raise ValueError(_OP_ERROR)
        return code
    try:
        code = int(op)
    except (TypeError, ValueError) as exc:
        raise ValueError(_OP_ERROR) from exc
    if code not in SPMV_OP_NAMES:
        raise ValueError(_OP_ERROR)
    return code


def _spmv_op_to_name(op):
    return SPMV_OP_NAMES[_normalize_spmv_op(op)]


def _spmv_op_transposes(op):
    return _normalize_spmv_op(op) in (SPMV_OP_TRANS, SPMV_OP_CONJ_TRANS)


class PreparedCsrSpmv:
    """Cached CSR metadata for repeated SpMV calls on the same sparse matrix.

    Holds the (possibly transposed) matrix, the row-length analysis and the
    merge-path partition / carry workspace the HIP kernel needs.
    """

    __slots__ = (
        "data",
        "kernel_indices",
        "kernel_indptr",
        "shape",
        "n_rows",
        "n_cols",
        "block_nnz",
        "max_segments",
        "opt_max_segments",
        "_row_lengths",
        "max_row_nnz",
        "opt_buckets",
        "supports_opt",
        "transpose",
        "op",
        "index_fallback_policy",
        "index_fallback_applied",
        "index_fallback_reason",
        "_compute_data",
        "_plan",
        "_part",
        "_carry",
        "_panels",
        "_sell",
        "_opt",
        "_one_shot",
    )

    def __init__(
        self,
        data,
        kernel_indices,
        kernel_indptr,
        shape,
        n_rows,
        n_cols,
        block_nnz,
        max_segments,
        max_row_nnz,
        opt_buckets=None,
        opt_max_segments=None,
        row_lengths=None,
        transpose=False,
        op=None,
        index_fallback_policy="auto",
        index_fallback_applied=False,
        index_fallback_reason=None,
    ):
        self.data = data
        self.kernel_indices = kernel_indices
        self.kernel_indptr = kernel_indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = n_rows
        self.n_cols = n_cols
        self.block_nnz = block_nnz
        self.max_segments = max_segments
        self.opt_max_segments = opt_max_segments
        self._row_lengths = row_lengths  # computed on first access when None
        self.max_row_nnz = max_row_nnz
        self.opt_buckets = [] if opt_buckets is None else opt_buckets
        self.supports_opt = (
            data.dtype in (torch.float32, torch.float64) and kernel_indices.dtype == torch.int32
        )
        self.op = _normalize_spmv_op(op, transpose=transpose)
        self.transpose = _spmv_op_transposes(self.op)
        self.index_fallback_policy = str(index_fallback_policy).lower()
        self.index_fallback_applied = bool(index_fallback_applied)
        self.index_fallback_reason = index_fallback_reason
        self._compute_data = None
        self._plan = None
        self._part = None
        self._carry = None
        self._panels = None
        self._sell = None
        self._opt = None  # row-length buckets of the use_opt path (built on first use)
        self._one_shot = False  # built for a single call: no column-panel copy

    @property
    def row_lengths(self):
        """indptr[1:] - indptr[:-1] (spmv_csr.py:111-113), computed on first access."""
        if self._row_lengths is None:
            self._row_lengths = self.kernel_indptr[1:] - self.kernel_indptr[:-1]
        return self._row_lengths

    @row_lengths.setter
    def row_lengths(self, value):
        self._row_lengths = value

    # -- HIP plan (built lazily on first run, then cached) ------------------
    def hip_plan(self, analysed=None):
        """The analysis plan (built on first use, or taken from `analysed`,
        a CsrPlan of this same matrix) plus the copies and partitions the
        chosen kernel needs."""
        if self._plan is None:
            data = self.compute_data()
            self._plan = analysed if analysed is not None else analyze_csr(
                data, self.kernel_indices, self.kernel_indptr, self.n_rows, self.n_cols
            )
            p = self._plan.plan
            # The SELL and panel copies are optional: when device memory cannot
            # hold one next to the caller's matrix, the CSR kernels run instead.
            locality = _spmv_sell_locality(p, self.kernel_indices, self.kernel_indptr, self._one_shot,
                                            _sell_codes_possible(data.element_size()))
            if locality is not None:
                try:
                    self._sell = _build_sell(data, self.kernel_indices, self.kernel_indptr, self.n_rows,
                                             self.n_cols, int(p.nnz), locality)
                except torch.OutOfMemoryError:
                    self._sell = None
                    torch.cuda.empty_cache()
            if self._sell is not None:
                return self._plan  # the copy needs no partition or carry
            if p.kernel == _lib.FS_KERNEL_MERGE:
                n_panels = _spmv_panel_count(p, data.dtype, self._one_shot)
                if n_panels > 1:
                    try:
                        self._panels = PanelledCsr(
                            data, self.kernel_indices, self.kernel_indptr, self.n_rows, self.n_cols, n_panels
                        )
                    except torch.OutOfMemoryError:
                        self._panels = None
                        torch.cuda.empty_cache()
                if self._panels is None:
                    self._part = self._plan.partition(self.kernel_indptr, int(p.tile_items))
                    self._carry = _lib.workspace(p.carry_bytes, data.device)
            elif p.kernel == _lib.FS_KERNEL_NNZBLOCK:
                self._part = torch.empty(int(p.n_tiles) + 1, dtype=torch.int64, device=data.device)
                _lib.check(
                    _lib.lib().fs_spmv_partition(
                        p, _lib.ptr(self.kernel_indptr), _lib.ptr(self._part), _lib.stream_handle(data.device)
                    ),
                    "fs_spmv_partition",
                )
                self._carry = _lib.workspace(p.carry_bytes, data.device)
        return self._plan

    def compute_data(self):
        """Values in the dtype the kernel runs in (f16/bf16 -> f32, cached)."""
        cdt = _compute_dtype(self.data.dtype)
        if cdt == self.data.dtype:
            return self.data
        if self._compute_data is None or self._compute_data.dtype != cdt:
            self._compute_data = self.data.to(cdt)
        return self._compute_data

    @property
    def kernel_name(self):
        plan = self.hip_plan()
        if self._sell is not None:
            return "sell"
        return "panel" if self._panels is not None else plan.kernel_name


# Column panels pay off once x is larger than an XCD's 4 MiB L2: the random
# gather rate measured on MI355X drops from ~150-190 to ~70 gathers/ns when
# x (16.8 MB) no longer fits.  A panel slice of up to ~4.5 MiB measured best
# (4 panels on a 16.8 MB x: 0.61 ms against 0.67 ms with 8 and 1.01 ms with
# none) since every panel adds n_rows row ends and partials.
_PANEL_X_BYTES = 6 << 20
_PANEL_SLICE_BYTES = 9 << 19


def _spmv_panel_count(plan, dtype, one_shot=False):
    """Column panels for a merge-path matrix (0 = none).  FLAGSPARSE_SPMV_PANELS=N
    forces N (0/1 off); otherwise the fewest of 2, 4, 8 whose x slice is at most
    ~4.5 MiB, for x above 6 MiB and rows averaging at least 2 entries per panel.

    A one-shot call (no prepared object kept) gets none: building the panel
    copy costs several launches of the unpanelled kernel (C3: 2.7 ms to save
    0.4 ms)."""
    env = os.environ.get("FLAGSPARSE_SPMV_PANELS")
    if env is not None:
        return max(0, int(env))
    if one_shot:
        return 0
    n_rows, n_cols, nnz = int(plan.n_rows), int(plan.n_cols), int(plan.nnz)
    x_bytes = n_cols * torch.empty(0, dtype=dtype).element_size()
    if n_rows == 0 or x_bytes <= _PANEL_X_BYTES:
        return 0
    n_panels = 2
    while n_panels < 8 and x_bytes > _PANEL_SLICE_BYTES * n_panels:
        n_panels *= 2
    return n_panels if nnz >= 2 * n_panels * n_rows else 0


class PanelledCsr:
    """A in n_panels column panels, stacked into one CSR with n_panels*n_rows
    rows, plus its merge plan, partition and SpMV workspace (built once)."""

    __slots__ = ("n_panels", "panel_nnz", "data", "indices", "indptr", "plan", "part", "ws")

    def __init__(self, data, indices, indptr, n_rows, n_cols, n_panels):
        device = data.device
        nnz = data.numel()
        lib = _lib.lib()
        self.n_panels = int(n_panels)
        self.data = torch.empty_like(data)
        self.indices = torch.empty_like(indices)
        self.indptr = torch.empty(self.n_panels * n_rows + 1, dtype=indptr.dtype, device=device)
        ws = _lib.workspace(lib.fs_csr_panelize_workspace_bytes(n_rows, n_cols, nnz, self.n_panels), device)
        self.panel_nnz = (ctypes.c_int64 * (self.n_panels + 1))()
        _lib.check(
            lib.fs_csr_panelize(
                _lib.value_code(data.dtype), _lib.index_code(indices.dtype), _lib.index_code(indptr.dtype),
                n_rows, n_cols, nnz, self.n_panels, _lib.ptr(data), _lib.ptr(indices), _lib.ptr(indptr),
                _lib.ptr(self.data), _lib.ptr(self.indices), _lib.ptr(self.indptr), self.panel_nnz,
                _lib.ptr(ws), ws.numel(), _lib.stream_handle(device),
            ),
            "fs_csr_panelize",
        )
        del ws
        # The stacked copy is this build's own format: store it with int32
        # column indices / row pointer whenever they fit, so int64 inputs
        # stream 4 bytes less per entry (the caller's tensors keep their type).
        if self.indices.dtype == torch.int64 and n_cols - 1 <= _INDEX_LIMIT_INT32:
            self.indices = self.indices.to(torch.int32)
        if self.indptr.dtype == torch.int64 and nnz <= _INDEX_LIMIT_INT32:
            self.indptr = self.indptr.to(torch.int32)
        self.plan = analyze_csr(
            self.data, self.indices, self.indptr, self.n_panels * n_rows, n_cols, force_kernel=_lib.FS_KERNEL_MERGE
        )
        self.part = self.plan.partition(self.indptr, int(self.plan.plan.tile_items))
        self.ws = _lib.workspace(lib.fs_spmv_panels_workspace_bytes(self.plan.plan, self.n_panels), device)

    def spmv(self, x, y):
        device = self.data.device
        _lib.check(
            _lib.lib().fs_spmv_csr_panels(
                self.plan.plan, self.n_panels, self.panel_nnz, _lib.ptr(self.data), _lib.ptr(self.indices),
                _lib.ptr(self.indptr),
                _lib.ptr(x), _lib.ptr(y), _lib.ptr(self.part), _lib.ptr(self.ws), self.ws.numel(),
                _lib.stream_handle(device),
            ),
            "fs_spmv_csr_panels",
        )


# Sliced ELL (SELL-64) pays off when a slice's rows have nearly the same
# length (padding lanes idle for the whole slot loop) and neighbouring rows
# have neighbouring columns, so that a slot's 64-lane x gather is coalesced.
# Measured on MI355X against the row-block stream kernel, with int32 / int16
# column storage: 27-point stencil 128^3 f64 0.145 -> 0.123 ms, f32 0.129 ->
# 0.086 ms; but with 28% padding (a stencil with 30% of entries dropped,
# int16 offsets) 0.112 -> 0.129 ms, and with uniformly random columns (no
# locality) 0.198 -> 0.203 ms.  One-byte offset codes move the bounds (below).
_SELL_MIN_SLICES = 2048      # 131,072 rows: enough waves to fill 256 CUs
_SELL_MAX_PADDING = 1.03     # stored slots / nnz
# With one-byte offset codes the padding slots (never loaded) cost little:
# the 128^3 f64 stencil with 5 / 10 / 30% of its entries dropped (stored
# slots 1.10 / 1.16 / 1.30 x nnz) runs 0.0928 / 0.0950 / 0.0899 ms on the
# copy against 0.1417 / 0.1364 / 0.1119 ms on the row-block stream kernel.
# and on random in-band columns (2^21 rows, f64), offsets +-32 / 64 / 96 /
# 127 with 40 / 20 / 14 / 10% of the band kept, stored slots 1.38 / 1.45 /
# 1.46 / 1.48 x nnz: 0.116 / 0.118 / 0.125 / 0.121 ms on the copy against
# 0.164 / 0.163 / 0.168 / 0.164 ms; +-64 with 10% kept (1.70 x nnz): 0.074
# against 0.083 ms.
_SELL_MAX_PADDING_CODES = 1.75
_SELL_MIN_LOCALITY = 0.5     # share of sampled (row, k) whose column is row r-1's + 1
# With offset codes the copy wins at lower locality: the 128^3 stencil with
# 30% of its entries dropped samples 0.245 (10%: 0.50, 20%: 0.34) and runs
# 0.0899 ms on the copy against 0.1119 ms on the row-block stream kernel;
# uniformly random and power-law columns sample 0.
_SELL_MIN_LOCALITY_CODES = 0.2
# With few offsets (codes) the copy wins at any sampled locality, bounded by
# padding instead: 2^21 rows, f64, random in-band columns, offsets +-16 / 24
# / 32 / 64 with 80 / 55 / 40 / 20% of the band kept (sampled locality 0.34 /
# 0.16 / 0.10 / 0.04): 0.100 / 0.110 / 0.112 / 0.118 ms on the copy against
# 0.162 / 0.164 / 0.161 / 0.163 ms on the row-block stream kernel; the 128^3
# stencil with 45 / 60% of its entries dropped (locality 0.16 / 0.12):
# 0.0804 / 0.0673 against 0.0938 / 0.0713 ms (with 75% dropped the copy
# holds 1.91 x nnz slots and loses, 0.0524 against 0.0490 ms).  So a sample
# whose offsets c - r take at most _SELL_CODES values counts as local.
_SELL_SAMPLE_OFFSETS = 32
_SELL_SAMPLE_SLICES = 256
_SELL_SAMPLE_K = 8


def _sell_forced():
    return os.environ.get("FLAGSPARSE_SPMV_SELL") == "1"


def _sell_locality(indices, indptr, n_rows):
    """(locality, narrow) from a sample of 256 slices (one device->host sync).

    locality: share of sampled entries (row r, k-th entry, k < 8) whose
    column is exactly one more than row r-1's k-th column, over rows r-1, r
    of the same slice.  narrow: the sampled offsets c - r (first 32 entries
    of each sampled row) take at most _SELL_CODES distinct values, so the
    copy can likely store one-byte codes and a slot's gathers fall in a few
    windows of x whatever the column order (bands, stencils with gaps)."""
    device = indices.device
    n_slices = n_rows // 64
    step = max(1, n_slices // _SELL_SAMPLE_SLICES)
    sl = torch.arange(0, n_slices, step, device=device)[:_SELL_SAMPLE_SLICES]
    r = (sl[:, None] * 64 + torch.arange(1, 64, device=device)[None, :]).reshape(-1)
    p0 = indptr[r - 1].to(torch.int64)
    p1 = indptr[r].to(torch.int64)
    p2 = indptr[r + 1].to(torch.int64)
    k = torch.arange(_SELL_SAMPLE_K, device=device)[None, :]
    valid = k < torch.minimum(p1 - p0, p2 - p1)[:, None]
    last = max(0, indices.numel() - 1)
    prev = indices[(p0[:, None] + k).clamp(max=last)].to(torch.int64)
    cur = indices[(p1[:, None] + k).clamp(max=last)].to(torch.int64)
    hits = ((cur - prev == 1) & valid).sum()
    total = valid.sum().clamp(min=1)
    kk = torch.arange(_SELL_SAMPLE_OFFSETS, device=device)[None, :]
    in_row = kk < (p2 - p1)[:, None]
    off = indices[(p1[:, None] + kk).clamp(max=last)].to(torch.int64) - r[:, None]
    off = off[in_row]
    if off.numel() == 0:
        stats = torch.stack([hits.double() / total.double(), torch.zeros((), dtype=torch.float64, device=device),
                             torch.zeros((), dtype=torch.float64, device=device)])
    else:
        stats = torch.stack([hits.double() / total.double(), off.abs().max().double(),
                             torch.tensor(float(torch.unique(off).numel()), dtype=torch.float64, device=device)])
    locality, max_off, distinct = stats.cpu().tolist()
    return locality, distinct <= _SELL_CODES and max_off <= 32767


def _sell_codes_possible(value_bytes):
    """Whether a SELL copy could store one-byte offset codes (values of at
    most 8 bytes, codes and offsets not switched off)."""
    return (value_bytes <= 8 and os.environ.get("FLAGSPARSE_SELL_CODES") != "0"
            and os.environ.get("FLAGSPARSE_SELL_DELTA") != "0")


def _spmv_sell_locality(plan, indices, indptr, one_shot, codes_possible=True):
    """The sampled column locality when a prepared matrix may get a SELL-64
    copy, else None.  FLAGSPARSE_SPMV_SELL=0/1 forces it off / on (1.0);
    otherwise only for a kept prepared matrix (the copy costs more than one
    launch) whose rows are short (not the merge-path kernel), with at least
    _SELL_MIN_SLICES slices and a locality of at least
    _SELL_MIN_LOCALITY_CODES, or few sampled offsets (then at least that
    value is returned).  _build_sell applies the bound that fits the column
    storage, and the padding bound after the slot count."""
    env = os.environ.get("FLAGSPARSE_SPMV_SELL")
    n_rows = int(plan.n_rows)
    if env is not None:
        return 1.0 if env == "1" and n_rows > 0 else None
    if one_shot or plan.kernel == _lib.FS_KERNEL_MERGE or n_rows < 64 * _SELL_MIN_SLICES:
        return None
    locality, narrow = _sell_locality(indices, indptr, n_rows)
    # below the plain bound only offset codes can win: skip the offset pass
    # (one launch and a sync) when the values rule codes out
    if codes_possible and narrow:
        return max(locality, _SELL_MIN_LOCALITY_CODES)
    return locality if locality >= (_SELL_MIN_LOCALITY_CODES if codes_possible else _SELL_MIN_LOCALITY) else None


def _sell_slice_ptr(indptr, n_rows, group):
    """Start of every 64-row slice in the SELL-64 copy (int64, n_slices + 1):
    the prefix sum of 64 x the slice's slot count (its longest row, rounded
    up to a multiple of the layout's group size).  Also returns 64 x the sum of the
    unrounded counts, which the padding bound is judged on (one sync)."""
    device = indptr.device
    n_slices = -(-n_rows // 64)
    slots = torch.empty(n_slices, dtype=torch.int64, device=device)
    _lib.check(
        _lib.lib().fs_sell_slots(
            _lib.index_code(indptr.dtype), n_rows, _lib.ptr(indptr), _lib.ptr(slots), _lib.stream_handle(device)
        ),
        "fs_sell_slots",
    )
    unrounded = int(slots.sum().item()) * 64
    if group > 1:
        slots = (slots + group - 1) // group * group
    slice_ptr = torch.zeros(n_slices + 1, dtype=torch.int64, device=device)
    torch.cumsum(slots * 64, 0, out=slice_ptr[1:])
    return slice_ptr, unrounded


_SELL_I32, _SELL_I64, _SELL_D16, _SELL_C8 = 0, 1, 2, 3  # enum fs_sell_index
_SELL_SLOT, _SELL_PAIR = 0, 1  # enum fs_sell_layout
_SELL_GROUP = {_SELL_SLOT: 1, _SELL_PAIR: 2}  # slots stored side by side
_SELL_CODES = 256  # uint8 codes: at most this many distinct offsets


def _sell_offsets(indices, indptr, n_rows, want_bits):
    """max |c - r| over the entries and, with want_bits, the sorted distinct
    offsets c - r when every |c - r| <= 32767 (one device->host sync)."""
    if indices.numel() == 0:
        return 0, ([] if want_bits else None)
    device = indices.device
    out = torch.zeros(1 + (2048 // 2 if want_bits else 0), dtype=torch.int64, device=device)
    bits = out[1:].view(torch.int32) if want_bits else None
    _lib.check(
        _lib.lib().fs_sell_max_offset(
            _lib.index_code(indices.dtype), _lib.index_code(indptr.dtype), n_rows, _lib.ptr(indices),
            _lib.ptr(indptr), _lib.ptr(out), _lib.ptr(bits) if want_bits else None, _lib.stream_handle(device),
        ),
        "fs_sell_max_offset",
    )
    host = out.cpu()
    max_off = int(host[0])
    if not want_bits or max_off > 32767:
        return max_off, None
    return max_off, _offsets_from_bits(host[1:].view(torch.int32).numpy())


def _offsets_from_bits(words):
    """Sorted offsets d whose bit d + 32768 is set in 2048 32-bit words
    (bit b of word w is offset 32 * w + b - 32768)."""
    words = np.ascontiguousarray(words).view(np.uint32)
    bits = np.unpackbits(words.astype("<u4").view(np.uint8), bitorder="little")
    return (np.nonzero(bits)[0].astype(np.int64) - 32768).tolist()


def _sell_column_code(indices, indptr, n_rows, n_cols, value_bytes):
    """Column storage of the SELL copy, and the offsets the codes stand for:
    uint8 codes when every |c - r| <= 32767 and at most 256 distinct offsets
    occur, for values of at most 8 bytes (off with FLAGSPARSE_SELL_CODES=0),
    else int16 offsets c - r when every |c - r| <= 32767 (off with
    FLAGSPARSE_SELL_DELTA=0), else int32 when n_cols - 1 fits, else int64.

    Codes measured on the 27-point 128^3 stencil (ms, int16 -> codes): f32
    0.0772 -> 0.0650, f64 0.1071 -> 0.0924, complex64 0.1387 -> 0.1194, but
    complex128 0.1714 -> 0.1943 (the table lookup before each gather costs
    more than the byte saved on a 17-byte entry)."""
    if os.environ.get("FLAGSPARSE_SELL_DELTA") != "0":
        want_bits = value_bytes <= 8 and os.environ.get("FLAGSPARSE_SELL_CODES") != "0"
        max_off, offsets = _sell_offsets(indices, indptr, n_rows, want_bits)
        if max_off <= 32767:
            if offsets is not None and len(offsets) <= _SELL_CODES:
                return _SELL_C8, offsets
            return _SELL_D16, None
    return (_SELL_I32 if n_cols - 1 <= _INDEX_LIMIT_INT32 else _SELL_I64), None


def _build_sell(data, indices, indptr, n_rows, n_cols, nnz, locality=1.0, force=False):
    """The SELL-64 copy, or None, unless forced, when the sampled locality is
    below _SELL_MIN_LOCALITY (_SELL_MIN_LOCALITY_CODES with offset codes) or
    its stored slots would exceed _SELL_MAX_PADDING x nnz
    (_SELL_MAX_PADDING_CODES x nnz with offset codes; rows too uneven)."""
    col_code, offsets = _sell_column_code(indices, indptr, n_rows, n_cols, data.element_size())
    codes = col_code == _SELL_C8
    force = force or _sell_forced()
    if locality < (_SELL_MIN_LOCALITY_CODES if codes else _SELL_MIN_LOCALITY) and not force:
        return None
    # pairs pay with 2-byte offsets (f64 stencil 0.114 -> 0.107 ms, f32 0.086 -> 0.076);
    # with 4-byte columns they do not (f64 0.123 both, f32 0.086 -> 0.093)
    pair = col_code in (_SELL_D16, _SELL_C8) and not data.dtype.is_complex
    layout = _SELL_PAIR if pair else _SELL_SLOT
    slice_ptr, stored = _sell_slice_ptr(indptr, n_rows, _SELL_GROUP[layout])
    bound = _SELL_MAX_PADDING_CODES if codes else _SELL_MAX_PADDING
    if stored > bound * max(1, nnz) and not force:
        return None
    return SellCsr(data, indices, indptr, slice_ptr, col_code, layout, offsets)


class SellCsr:
    """A as SELL-64: slices of 64 consecutive rows, built once per prepared
    matrix (fs_sell_slots, fs_csr_to_sell).  Columns are stored as chosen by
    _sell_column_code; with offset codes or int16 offsets, real values use
    the pair layout (a row's consecutive slots side by side, loaded two at a
    time), otherwise the slot layout.  With codes, `table` holds the 256
    offsets the codes stand for.  The CSR row pointer of the prepared matrix supplies the
    row lengths."""

    __slots__ = ("vals", "cols", "col_code", "layout", "slice_ptr", "indptr", "n_rows", "padded", "table", "n_codes",
                 "offsets_host")

    def __init__(self, data, indices, indptr, slice_ptr, col_code, layout, offsets=None):
        device = data.device
        lib = _lib.lib()
        stream = _lib.stream_handle(device)
        n_rows = indptr.numel() - 1
        self.slice_ptr = slice_ptr
        self.layout = layout
        self.padded = int(slice_ptr[-1])
        self.indptr = indptr
        self.n_rows = n_rows
        self.vals = torch.zeros(self.padded, dtype=data.dtype, device=device)
        self.col_code = col_code
        col_dtype = {_SELL_C8: torch.uint8, _SELL_D16: torch.int16, _SELL_I32: torch.int32,
                     _SELL_I64: torch.int64}[col_code]
        self.cols = torch.zeros(self.padded, dtype=col_dtype, device=device)
        self.table = None
        self.n_codes = 0
        self.offsets_host = None
        lut = None
        if col_code == _SELL_C8:
            self.n_codes = len(offsets)
            # code k stands for offsets[k]; the lookup maps offset d (at d + 32768) to its code
            table = np.zeros(_SELL_CODES, dtype=np.int32)
            table[: len(offsets)] = offsets
            lut_host = np.zeros(65536, dtype=np.uint8)
            lut_host[np.asarray(offsets, dtype=np.int64) + 32768] = np.arange(len(offsets), dtype=np.uint8)
            self.table = torch.from_numpy(table).to(device)
            self.offsets_host = np.ascontiguousarray(np.asarray(offsets, dtype=np.int32))
            lut = torch.from_numpy(lut_host).to(device)
        _lib.check(
            lib.fs_csr_to_sell(
                _lib.value_code(data.dtype), _lib.index_code(indices.dtype), _lib.index_code(indptr.dtype),
                self.col_code, layout, n_rows, _lib.ptr(data), _lib.ptr(indices), _lib.ptr(indptr),
                _lib.ptr(self.slice_ptr), _lib.ptr(lut) if lut is not None else None, _lib.ptr(self.vals),
                _lib.ptr(self.cols), stream,
            ),
            "fs_csr_to_sell",
        )
        del lut  # stream-ordered: the caching allocator reuses it only after the fill

    def spmm_fits(self, B, C):
        """Whether fs_spmm_sell takes these B / C: row-major, rows of whole
        16-byte slices, 16-byte aligned, the copy's value type."""
        epl = 16 // self.vals.element_size()
        n = B.shape[1]
        return (B.dtype == self.vals.dtype and C.dtype == self.vals.dtype and B.stride(1) == 1 and C.stride(1) == 1
                and n % epl == 0 and B.stride(0) % epl == 0 and C.stride(0) % epl == 0
                and B.data_ptr() % 16 == 0 and C.data_ptr() % 16 == 0 and B.stride(0) >= n and C.stride(0) >= n)

    def spmm_call(self, B, C):
        """(entry point, name, arguments) of C = A B on this copy:
        fs_spmm_sell, or with FLAGSPARSE_SPMM_SELL_STAGE=1 and offset codes
        whose bands fit, the B-through-LDS kernel (fs_spmm_sell_staged; the
        same bits, measured slower on the 27-point stencil: 1.37 against
        0.59 ms at N = 32 f32, so it is not the default)."""
        lib = _lib.lib()
        stream = _lib.stream_handle(self.vals.device)
        if (self.col_code == _SELL_C8 and os.environ.get("FLAGSPARSE_SPMM_SELL_STAGE", "0") == "1"
                and lib.fs_spmm_sell_staged_fits(_lib.value_code(self.vals.dtype), self.offsets_host.ctypes.data,
                                                 self.n_codes, int(B.shape[1]))):
            return lib.fs_spmm_sell_staged, "fs_spmm_sell_staged", (
                _lib.value_code(self.vals.dtype), _lib.index_code(self.indptr.dtype), self.layout, self.n_rows,
                int(B.shape[0]), _lib.ptr(self.vals), _lib.ptr(self.cols), _lib.ptr(self.table),
                self.offsets_host.ctypes.data, self.n_codes, _lib.ptr(self.slice_ptr), _lib.ptr(self.indptr),
                _lib.ptr(B), int(B.stride(0)), _lib.ptr(C), int(C.stride(0)), int(B.shape[1]), stream)
        return lib.fs_spmm_sell, "fs_spmm_sell", (
            _lib.value_code(self.vals.dtype), self.col_code, _lib.index_code(self.indptr.dtype), self.layout,
            self.n_rows, _lib.ptr(self.vals), _lib.ptr(self.cols),
            _lib.ptr(self.table) if self.table is not None else None, _lib.ptr(self.slice_ptr),
            _lib.ptr(self.indptr), _lib.ptr(B), int(B.stride(0)), _lib.ptr(C), int(C.stride(0)), int(B.shape[1]),
            stream)

    def spmm(self, B, C):
        fn, name, args = self.spmm_call(B, C)
        _lib.check(fn(*args), name)

    def spmv(self, x, y):
        _lib.check(
            _lib.lib().fs_spmv_sell(
                _lib.value_code(self.vals.dtype), self.col_code, _lib.index_code(self.indptr.dtype), self.layout,
                self.n_rows, _lib.ptr(self.vals), _lib.ptr(self.cols),
                _lib.ptr(self.table) if self.table is not None else None, _lib.ptr(self.slice_ptr),
                _lib.ptr(self.indptr), _lib.ptr(x), _lib.ptr(y), _lib.stream_handle(self.vals.device),
            ),
            "fs_spmv_sell",
        )


def _normalize_spmv_index_fallback_policy(index_fallback_policy):
    policy = str(index_fallback_policy).lower()
    if policy not in ("auto", "strict"):
        raise ValueError("index_fallback_policy must be 'auto' or 'strict'")
    return policy


def _spmv_dtype_error_message():
    return "data dtype must be one of: " + ", ".join(
        str(dtype).replace("torch.", "") for dtype in SUPPORTED_SPMV_VALUE_DTYPES
    )


def _transpose_csr_for_spmv(data, indices, indptr, shape):
    """CSR of A^T, stable by column (reference: spmv_csr.py:477-515)."""
    return transpose_csr(data, indices, indptr, shape, conj=False)


def _check_structure(data, indices, indptr, n_cols, messages, analyze=False):
    """indptr / index checks in one native pass with one device->host sync
    (fs_csr_check).

    The reference checks indptr[0], indptr[-1], monotonicity and the column
    range with separate .item() syncs (spmv_csr.py:546-558); the checks and
    the order in which their errors are raised are kept.  Returns the column
    range (lo, hi), or None when nnz == 0.  With analyze=True the row-length
    analysis runs in the same round trip (fs_csr_check_analyze) and the
    result is (range, CsrPlan).
    """
    nnz = data.numel()
    if indptr.numel() == 0:
        return (None, None) if analyze else None
    lib = _lib.lib()
    vals = (ctypes.c_int64 * 5)()
    plan = None
    if analyze:
        ws = _lib.workspace(lib.fs_csr_check_analyze_bytes(), indptr.device)
        raw = _lib.FsCsrPlan()
        _lib.check(
            lib.fs_csr_check_analyze(
                _lib.ptr(indptr),
                _lib.index_code(indptr.dtype),
                _lib.ptr(indices) if nnz > 0 else None,
                _lib.index_code(indices.dtype),
                _lib.value_code(_compute_dtype(data.dtype)),
                indptr.numel() - 1,
                int(n_cols),
                nnz,
                -1,
                _lib.ptr(ws),
                vals,
                raw,
                _lib.stream_handle(indptr.device),
            ),
            "fs_csr_check_analyze",
        )
        plan = CsrPlan(raw, indptr.device)
    else:
        check = _lib.workspace(lib.fs_csr_check_bytes(), indptr.device)
        _lib.check(
            lib.fs_csr_check(
                _lib.ptr(indptr),
                _lib.index_code(indptr.dtype),
                _lib.ptr(indices) if nnz > 0 else None,
                _lib.index_code(indices.dtype),
                indptr.numel() - 1,
                nnz,
                _lib.ptr(check),
                vals,
                _lib.stream_handle(indptr.device),
            ),
            "fs_csr_check",
        )
    col_range = _raise_structure(vals, nnz, n_cols, messages)
    return (col_range, plan) if analyze else col_range


def _raise_structure(vals, nnz, n_cols, messages):
    """The reference's structure errors, in its order, from the five check
    values; the column range (lo, hi), or None when nnz == 0."""
    if vals[0] != 0:
        raise ValueError(messages["start"])
    if vals[1] != nnz:
        raise ValueError(messages["last"](vals[1]))
    if vals[2] != 0:
        raise ValueError(messages["monotone"])
    if nnz > 0:
        if vals[3] < 0 or vals[4] >= n_cols:
            raise IndexError("indices out of range for n_cols")
        return (vals[3], vals[4])
    return None


_check_local = threading.local()


class _PendingCheck:
    """A structure check whose answer is read later.  Queued at once
    (fs_csr_check_enqueue), or, with lazy=True, handed to the transpose that
    runs next (fuse(): fs_csr_transpose_checked tests the structure in its
    own passes), or queued by finish() if neither happened.  finish()
    synchronises the stream and raises the reference's error, if any."""

    __slots__ = ("words", "nnz", "n_cols", "messages", "stream", "_ws", "_indices", "_indptr", "_queued")

    def __init__(self, data, indices, indptr, n_cols, messages, lazy=False):
        words = getattr(_check_local, "words", None)
        if words is None:
            words = torch.zeros(5, dtype=torch.int64, pin_memory=True)
            _check_local.words = words
        self.words = words
        self.nnz = data.numel()
        self.n_cols = int(n_cols)
        self.messages = messages
        self.stream = torch.cuda.current_stream(indptr.device)
        self._ws = _lib.workspace(_lib.lib().fs_csr_check_bytes(), indptr.device)
        self._indices, self._indptr = indices, indptr
        self._queued = False
        if not lazy:
            self.queue()

    def queue(self):
        """Queue the standalone check pass (once)."""
        if self._queued:
            return
        lib = _lib.lib()
        indptr, indices = self._indptr, self._indices
        _lib.check(
            lib.fs_csr_check_enqueue(
                _lib.ptr(indptr), _lib.index_code(indptr.dtype), _lib.ptr(indices) if self.nnz > 0 else None,
                _lib.index_code(indices.dtype), indptr.numel() - 1, self.nnz, _lib.ptr(self._ws),
                self.words.data_ptr(), _lib.stream_handle(indptr.device),
            ),
            "fs_csr_check_enqueue",
        )
        self._queued = True

    def fuse(self):
        """(check_dev, host_words) for fs_csr_transpose_checked, which then
        stands for the check pass; None when the check is already queued."""
        if self._queued:
            return None
        self._queued = True
        return _lib.ptr(self._ws), self.words.data_ptr()

    def finish(self):
        self.queue()
        self.stream.synchronize()
        vals = (ctypes.c_int64 * 5)()
        _lib.check(_lib.lib().fs_csr_check_decode(self.words.data_ptr(), self.nnz, vals), "fs_csr_check_decode")
        return _raise_structure(vals, self.nnz, self.n_cols, self.messages)


_SPMV_STRUCT_MESSAGES = {
    "start": "indptr must start at zero",
    "last": lambda got: "indptr[-1] must equal nnz",
    "monotone": "indptr must be non-decreasing",
}


def _prepare_spmv_csr_matrix(data, indices, indptr, shape, index_fallback_policy="auto", analyze=False):
    """Validation of spmv_csr.py:518-572 (same order, types and messages).
    With analyze=True the row-length analysis shares the check's device
    round trip and its plan is returned last."""
    data, indices, indptr, n_rows, n_cols = _validate_spmv_host(data, indices, indptr, shape, index_fallback_policy)
    if analyze:
        _, plan = _check_structure(data, indices, indptr, n_cols, _SPMV_STRUCT_MESSAGES, analyze=True)
        return data, indices, indptr, n_rows, n_cols, None, plan
    _check_structure(data, indices, indptr, n_cols, _SPMV_STRUCT_MESSAGES)
    return data, indices, indptr, n_rows, n_cols, None


def _validate_spmv_host(data, indices, indptr, shape, index_fallback_policy="auto"):
    """The checks of spmv_csr.py:518-545 that need no device read, in order."""
    _normalize_spmv_index_fallback_policy(index_fallback_policy)
    if not all(torch.is_tensor(t) for t in (data, indices, indptr)):
        raise TypeError("data, indices, indptr must all be torch.Tensor")
    if data.ndim != 1 or indices.ndim != 1 or indptr.ndim != 1:
        raise ValueError("data, indices, indptr must be 1D tensors")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if indptr.numel() != n_rows + 1:
        raise ValueError(f"indptr length must be n_rows+1={n_rows + 1}, got {indptr.numel()}")
    if data.numel() != indices.numel():
        raise ValueError("data and indices must have the same length (nnz)")
    if not all(t.is_cuda for t in (data, indices, indptr)):
        raise ValueError("data, indices, indptr must be CUDA tensors")
    if not all(t.device == data.device for t in (indices, indptr)):
        raise ValueError("data, indices, indptr must be on the same CUDA device")
    if data.dtype not in SUPPORTED_SPMV_VALUE_DTYPES:
        raise TypeError(_spmv_dtype_error_message())
    if indices.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("indices dtype must be torch.int32 or torch.int64")
    if indptr.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("indptr dtype must be torch.int32 or torch.int64")

    return data.contiguous(), indices.contiguous(), indptr.contiguous(), n_rows, n_cols


def _validate_spmv_x(x, prepared):
    """spmv_csr.py:575-588."""
    return _validate_spmv_x_for(x, prepared.data.dtype, prepared.n_cols, prepared.data.device)


def _validate_spmv_x_for(x, dtype, n_cols, device):
    if x is None or not torch.is_tensor(x):
        raise TypeError("x must be a torch.Tensor")
    if x.ndim != 1:
        raise ValueError("x must be a 1D tensor")
    if not x.is_cuda:
        raise ValueError("x must be a CUDA tensor")
    if x.dtype != dtype:
        raise TypeError("x dtype must match sparse matrix dtype")
    if x.numel() != n_cols:
        raise ValueError(f"x length must be n_cols={n_cols}, got {x.numel()}")
    if x.device != device:
        raise ValueError("x must be on the same device as sparse matrix data")
    return x.contiguous()


def prepare_spmv_csr(
    data,
    indices,
    indptr,
    shape,
    block_nnz=256,
    max_segments=None,
    transpose=False,
    op=None,
    index_fallback_policy="auto",
):
    """Validate, transpose for op=trans/conj, analyse and cache (spmv_csr.py:591-664).

    block_nnz / max_segments keep the reference's meaning for callers that
    read them back; the HIP kernels do not iterate fixed segments, so they
    do not limit which rows can be processed.
    """
    return _prepare_spmv(data, indices, indptr, shape, block_nnz, max_segments, transpose, op, index_fallback_policy)


def _prepare_spmv(
    data, indices, indptr, shape, block_nnz, max_segments, transpose, op, index_fallback_policy, one_shot=False
):
    index_fallback_policy = _normalize_spmv_index_fallback_policy(index_fallback_policy)
    op_code = _normalize_spmv_op(op, transpose=transpose)
    if op is not None and bool(transpose) and op_code == SPMV_OP_NON:
        raise ValueError("transpose=True conflicts with op=non")
    transposes = _spmv_op_transposes(op_code)
    if transposes:
        data, indices, indptr, *_ = _prepare_spmv_csr_matrix(
            data, indices, indptr, shape, index_fallback_policy=index_fallback_policy
        )
        data, indices, indptr, shape = transpose_csr(
            data, indices, indptr, shape, conj=(op_code == SPMV_OP_CONJ_TRANS)
        )
    data, indices, indptr, n_rows, n_cols, row_lengths, plan0 = _prepare_spmv_csr_matrix(
        data, indices, indptr, shape, index_fallback_policy=index_fallback_policy, analyze=True
    )
    prepared = PreparedCsrSpmv(
        data=data,
        kernel_indices=indices,
        kernel_indptr=indptr,
        shape=shape,
        n_rows=n_rows,
        n_cols=n_cols,
        block_nnz=block_nnz,
        max_segments=1,
        opt_max_segments=max_segments,
        row_lengths=row_lengths,
        max_row_nnz=0,
        opt_buckets=None,
        transpose=transposes,
        op=op_code,
        index_fallback_policy=index_fallback_policy,
    )
    prepared._one_shot = bool(one_shot)
    if n_rows > 0:
        plan = prepared.hip_plan(analysed=plan0)
        max_row = plan.max_row_nnz
    else:
        max_row = 0
    prepared.max_row_nnz = max_row
    # Segment sizing as the reference reports it (spmv_csr.py:637-647).
    block_nnz_use = block_nnz
    if max_segments is None:
        segs = max((max_row + block_nnz_use - 1) // block_nnz_use, 1)
        while segs > 2048 and block_nnz_use < 65536:
            block_nnz_use *= 2
            segs = max((max_row + block_nnz_use - 1) // block_nnz_use, 1)
    else:
        segs = max_segments
    prepared.block_nnz = block_nnz_use
    prepared.max_segments = segs
    return prepared


def _hip_spmv_csr_impl_prepared(prepared, x):
    """One SpMV launch (replaces _triton_spmv_csr_impl_prepared, spmv_csr.py:679-723)."""
    device = prepared.data.device
    dtype = prepared.data.dtype
    y = torch.empty(prepared.n_rows, dtype=dtype, device=device)
    if prepared.n_rows == 0:
        return y
    data = prepared.compute_data()
    cdt = data.dtype
    x_in = x if x.dtype == cdt else x.to(cdt)
    y_out = y if cdt == dtype else torch.empty(prepared.n_rows, dtype=cdt, device=device)
    plan = prepared.hip_plan()
    copy = prepared._sell if prepared._sell is not None else prepared._panels
    if copy is not None:
        copy.spmv(x_in, y_out)
        if y_out is not y:
            y.copy_(y_out)
        return y
    carry = prepared._carry
    _lib.check(
        _lib.lib().fs_spmv_csr(
            plan.plan,
            _lib.ptr(data),
            _lib.ptr(prepared.kernel_indices),
            _lib.ptr(prepared.kernel_indptr),
            _lib.ptr(x_in),
            _lib.ptr(y_out),
            _lib.ptr(prepared._part),
            _lib.ptr(carry),
            0 if carry is None else carry.numel(),
            _lib.stream_handle(device),
        ),
        "fs_spmv_csr",
    )
    if y_out is not y:
        y.copy_(y_out)
    return y


def _spmv_uses_int64_indices(prepared):
    return prepared.kernel_indices.dtype == torch.int64 or prepared.kernel_indptr.dtype == torch.int64


def _spmv_int32_fallback_blocker(prepared):
    """Reason the int32 re-run would be unsafe, or None (spmv_csr.py:733-754)."""
    if prepared.kernel_indices.dtype == torch.int64 and prepared.kernel_indices.numel() > 0:
        lo_hi = torch.stack([prepared.kernel_indices.min(), prepared.kernel_indices.max()]).cpu().tolist()
        min_index, max_index = int(lo_hi[0]), int(lo_hi[1])
        if min_index < 0 or max_index > _INDEX_LIMIT_INT32:
            return f"column index range [{min_index}, {max_index}] cannot fit int32 for shape={prepared.shape}"
    if prepared.kernel_indptr.dtype == torch.int64 and prepared.kernel_indptr.numel() > 0:
        max_offset = int(prepared.kernel_indptr[-1].item())
        if max_offset > _INDEX_LIMIT_INT32:
            return f"CSR nnz offset {max_offset} cannot fit int32 for shape={prepared.shape}"
    if prepared.n_rows > _INDEX_LIMIT_INT32:
        return f"row count {prepared.n_rows} cannot fit int32 row metadata"
    return None


def _spmv_prepared_with_int32_indices(prepared, reason):
    blocker = _spmv_int32_fallback_blocker(prepared)
    if blocker is not None:
        raise RuntimeError(f"native int64 CSR SpMV failed and int32 fallback is unsafe: {blocker}")
    kernel_indices = prepared.kernel_indices.to(torch.int32)
    kernel_indptr = prepared.kernel_indptr.to(torch.int32)
    out = PreparedCsrSpmv(
        data=prepared.data,
        kernel_indices=kernel_indices,
        kernel_indptr=kernel_indptr,
        shape=prepared.shape,
        n_rows=prepared.n_rows,
        n_cols=prepared.n_cols,
        block_nnz=prepared.block_nnz,
        max_segments=prepared.max_segments,
        opt_max_segments=prepared.opt_max_segments,
        row_lengths=kernel_indptr[1:] - kernel_indptr[:-1],
        max_row_nnz=prepared.max_row_nnz,
        opt_buckets=None,
        transpose=prepared.transpose,
        op=prepared.op,
        index_fallback_policy=prepared.index_fallback_policy,
        index_fallback_applied=True,
        index_fallback_reason=str(reason),
    )
    return out


class _SpmvOptBuckets:
    """Row ids of the use_opt path partitioned into the reference's row-length
    tiers (spmv_csr.py:136-161, 353-410), on the device, with the tier sizes
    on the host."""

    __slots__ = ("ws", "counts")

    def __init__(self, prepared):
        lib = _lib.lib()
        device = prepared.data.device
        n_rows = int(prepared.n_rows)
        self.ws = _lib.workspace(lib.fs_spmv_opt_workspace_bytes(n_rows), device)
        self.counts = (ctypes.c_int64 * int(lib.fs_spmv_opt_max_buckets()))()
        _lib.check(
            lib.fs_spmv_opt_buckets(
                _lib.ptr(prepared.kernel_indptr),
                _lib.index_code(prepared.kernel_indptr.dtype),
                _lib.value_code(prepared.data.dtype),
                n_rows,
                _lib.ptr(self.ws),
                self.ws.numel(),
                self.counts,
                _lib.stream_handle(device),
            ),
            "fs_spmv_opt_buckets",
        )

    @property
    def bucket_count(self):
        """Non-empty buckets, as len(opt_buckets) in the reference."""
        return sum(1 for c in self.counts if c > 0)


def _spmv_opt_buckets(prepared):
    """The use_opt buckets of a prepared matrix: built once and kept, except
    for a one-shot call (the reference rebuilds them every call,
    spmv_csr.py:870-880)."""
    if prepared._opt is not None:
        return prepared._opt
    opt = _SpmvOptBuckets(prepared)
    if not prepared._one_shot:
        prepared._opt = opt
    return opt


def _hip_spmv_opt(prepared, x, opt):
    """y = A x with native-precision accumulation over the row-length buckets
    (_triton_spmv_csr_impl_opt_prepared, spmv_csr.py:412-461)."""
    device = prepared.data.device
    y = torch.empty(prepared.n_rows, dtype=prepared.data.dtype, device=device)
    if prepared.n_rows == 0:
        return y
    _lib.check(
        _lib.lib().fs_spmv_csr_opt(
            _lib.value_code(prepared.data.dtype),
            _lib.index_code(prepared.kernel_indices.dtype),
            _lib.index_code(prepared.kernel_indptr.dtype),
            int(prepared.n_rows),
            _lib.ptr(prepared.data),
            _lib.ptr(prepared.kernel_indices),
            _lib.ptr(prepared.kernel_indptr),
            _lib.ptr(x),
            _lib.ptr(y),
            _lib.ptr(opt.ws),
            opt.ws.numel(),
            opt.counts,
            _lib.stream_handle(device),
        ),
        "fs_spmv_csr_opt",
    )
    return y


def _run_spmv_prepared(prepared, x, use_opt=False, opt_buckets=None):
    """use_opt (float32 / float64 with int32 indices, as supports_opt) runs
    the native-precision bucketed kernels; otherwise the analysed kernel."""
    if use_opt and prepared.supports_opt:
        return _hip_spmv_opt(prepared, x, opt_buckets if opt_buckets is not None else _spmv_opt_buckets(prepared))
    return _hip_spmv_csr_impl_prepared(prepared, x)


def _run_spmv_prepared_with_fallback(prepared, x, use_opt=False, opt_buckets=None):
    try:
        return _run_spmv_prepared(prepared, x, use_opt=use_opt, opt_buckets=opt_buckets)
    except Exception as exc:
        if prepared.index_fallback_policy != "auto" or not _spmv_uses_int64_indices(prepared):
            raise
        fallback = _spmv_prepared_with_int32_indices(prepared, exc)
        return _run_spmv_prepared(fallback, x, use_opt=use_opt)


def flagsparse_spmv_csr(
    data=None,
    indices=None,
    indptr=None,
    x=None,
    shape=None,
    block_nnz=256,
    max_segments=None,
    out=None,
    return_time=False,
    return_meta=False,
    use_opt=False,
    prepared=None,
    transpose=None,
    op=None,
    index_fallback_policy="auto",
):
    """CSR SpMV y = op(A) @ x on the HIP kernels.

    op: 0/'non' for A @ x, 1/'trans' for A.T @ x, 2/'conj' for A.conj().T @ x.
    prepared: cached metadata from prepare_spmv_csr for steady-state runs.
    Returns y, (y, ms), (y, meta) or (y, ms, meta) like spmv_csr.py:813-913.
    """
    op_explicit = op is not None
    op_code = _normalize_spmv_op(op, transpose=False if transpose is None else bool(transpose))
    if op_explicit and transpose is not None and bool(transpose) != _spmv_op_transposes(op_code):
        raise ValueError("transpose conflicts with op")
    if prepared is None:
        if any(arg is None for arg in (data, indices, indptr, shape)):
            raise ValueError("data, indices, indptr, and shape are required when prepared is not provided")
        if op_code == SPMV_OP_NON and not use_opt:
            fast = _spmv_oneshot(data, indices, indptr, x, shape, index_fallback_policy, bool(return_time or return_meta))
            if fast is not None:
                return _finish_spmv(fast[0], out, return_time, return_meta, 0.0, fast[1], 0, "oneshot")
        if op_code != SPMV_OP_NON and not use_opt and not (return_time or return_meta):
            fast = _spmv_transposed_oneshot(data, indices, indptr, x, shape, op_code, index_fallback_policy)
            if fast is not None:
                return _finish_spmv(fast, out, False, False, 0.0, None, 0, "oneshot")
        prepared = _prepare_spmv(
            data,
            indices,
            indptr,
            shape,
            block_nnz,
            max_segments,
            False,
            op_code,
            index_fallback_policy,
            one_shot=True,
        )
    else:
        if op_explicit and op_code != prepared.op:
            raise ValueError(
                f"op={_spmv_op_to_name(op_code)} does not match prepared.op={_spmv_op_to_name(prepared.op)}"
            )
        if not op_explicit and transpose is not None and bool(transpose) != prepared.transpose:
            raise ValueError(
                f"transpose={bool(transpose)} does not match prepared.transpose={prepared.transpose}"
            )
    x = _validate_spmv_x(x, prepared)
    do_timing = bool(return_time or return_meta)
    symbolic_ms = compute_ms = op_total_ms = None
    opt = None
    if do_timing:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    if use_opt and prepared.supports_opt:
        opt = _spmv_opt_buckets(prepared)
    if do_timing:
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        symbolic_ms = (t1 - t0) * 1000.0 if opt is not None else 0.0
    y = _run_spmv_prepared_with_fallback(prepared, x, use_opt=use_opt, opt_buckets=opt)
    if do_timing:
        torch.cuda.synchronize()
        compute_ms = (time.perf_counter() - t1) * 1000.0
        op_total_ms = symbolic_ms + compute_ms
    kernel = ("opt" if opt is not None else prepared.kernel_name) if prepared.n_rows > 0 else None
    return _finish_spmv(y, out, return_time, return_meta, symbolic_ms, compute_ms,
                        opt.bucket_count if opt is not None else 0, kernel)


def _finish_spmv(y, out, return_time, return_meta, symbolic_ms, compute_ms, bucket_count, kernel):
    """`out` handling and the return forms of spmv_csr.py:892-913."""
    op_total_ms = None if compute_ms is None else (symbolic_ms or 0.0) + compute_ms
    if out is not None:
        if not out.is_cuda:
            raise ValueError("out must be a CUDA tensor")
        if out.device != y.device:
            raise ValueError("out must be on the same CUDA device as the result")
        if out.shape != y.shape or out.dtype != y.dtype:
            raise ValueError("out shape/dtype must match result")
        out.copy_(y)
        y = out
    if return_meta:
        meta = {
            "symbolic_ms": symbolic_ms,
            "compute_ms": compute_ms,
            "op_total_ms": op_total_ms,
            "bucket_count": bucket_count,
            "kernel": kernel,
        }
        if return_time:
            return y, op_total_ms, meta
        return y, meta
    if return_time:
        return y, op_total_ms
    return y


_oneshot_local = threading.local()


def _oneshot_flags():
    """This thread's 4 pinned int32 flags for the one-shot kernel (the kernel
    writes them in host memory; calls on one thread never overlap, each
    synchronises its stream before it returns)."""
    f = getattr(_oneshot_local, "flags", None)
    if f is None:
        f = torch.zeros(4, dtype=torch.int32, pin_memory=True)
        _oneshot_local.flags = f
    return f


def _oneshot_launch(data, indices, indptr, x, y, n_rows, n_cols, flags):
    """One fs_spmv_csr_oneshot call; its status (nonzero: the general path runs)."""
    return _lib.lib().fs_spmv_csr_oneshot(
        _lib.value_code(data.dtype), _lib.index_code(indices.dtype), _lib.index_code(indptr.dtype), n_rows, n_cols,
        data.numel(), _lib.ptr(data), _lib.ptr(indices), _lib.ptr(indptr), _lib.ptr(x), _lib.ptr(y),
        flags.data_ptr(), _lib.stream_handle(data.device))


def _spmv_transposed_oneshot(data, indices, indptr, x, shape, op_code, index_fallback_policy):
    """The unprepared y = A^T x / A^H x with one synchronisation: the
    structure check (fs_csr_check_enqueue), the transpose (which stays in
    bounds on any input, fs_csr_transpose_bounded) and the one-launch SpMV
    on A^T are queued back to back; the reference's structure error, if any,
    is raised before y is returned (spmv_csr.py:546-558, then the transpose
    of :477-515 and :615-618).  None when the general path must run: an
    invalid x, empty shapes, float16 / bfloat16 / complex128, a forced
    kernel or a failed launch."""
    if os.environ.get("FLAGSPARSE_SPMV_ONESHOT", "1") == "0" or os.environ.get("FLAGSPARSE_SPMV_KERNEL"):
        return None
    data, indices, indptr, n_rows, n_cols = _validate_spmv_host(data, indices, indptr, shape, index_fallback_policy)
    nnz = data.numel()
    if data.dtype not in HIP_VALUE_DTYPES or n_rows == 0 or n_cols == 0 or nnz == 0:
        return None
    try:
        x = _validate_spmv_x_for(x, data.dtype, n_rows, data.device)
    except (TypeError, ValueError):
        return None
    if not _lib.lib().fs_csr_transpose_bounded(_lib.value_code(data.dtype), n_rows, n_cols, nnz):
        return None
    pending = _PendingCheck(data, indices, indptr, n_cols, _SPMV_STRUCT_MESSAGES, lazy=True)
    td, ti, tp, tsh = transpose_csr(data, indices, indptr, (n_rows, n_cols), conj=(op_code == SPMV_OP_CONJ_TRANS),
                                    compact=True, check=pending)
    y = torch.empty(n_cols, dtype=data.dtype, device=data.device)
    flag_t = _oneshot_flags()
    rc = _oneshot_launch(td, ti, tp, x, y, n_cols, n_rows, flag_t)
    pending.finish()  # raises the reference's error for a malformed A
    if rc != 0:
        return None
    if any(flag_t.tolist()):
        raise RuntimeError("fs_spmv_csr_oneshot: the transpose of a valid matrix failed its structure check")
    return y


def _spmv_oneshot(data, indices, indptr, x, shape, index_fallback_policy, timed):
    """The unprepared y = A x in one launch (fs_spmv_csr_oneshot): the
    kernel checks the structure while it computes, and the reference's
    errors are raised here, in its order (spmv_csr.py:546-558), before y
    is returned or `out` is written.  Returns (y, compute_ms) or None when
    the general path must run: an invalid x (its error comes after the
    structure checks), empty shapes, float16 / bfloat16, a forced kernel,
    or a failed launch (the general path holds the int64 -> int32 fallback)."""
    if os.environ.get("FLAGSPARSE_SPMV_ONESHOT", "1") == "0" or os.environ.get("FLAGSPARSE_SPMV_KERNEL"):
        return None
    data, indices, indptr, n_rows, n_cols = _validate_spmv_host(data, indices, indptr, shape, index_fallback_policy)
    nnz = data.numel()
    if data.dtype not in HIP_VALUE_DTYPES or n_rows == 0 or n_cols == 0 or nnz == 0:
        return None
    try:
        x = _validate_spmv_x_for(x, data.dtype, n_cols, data.device)
    except (TypeError, ValueError):
        return None
    y = torch.empty(n_rows, dtype=data.dtype, device=data.device)
    flag_t = _oneshot_flags()
    if timed:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    rc = _oneshot_launch(data, indices, indptr, x, y, n_rows, n_cols, flag_t)
    if rc != 0:
        return None
    compute_ms = (time.perf_counter() - t0) * 1000.0 if timed else None
    flags = flag_t.tolist()
    if flags[0]:
        raise ValueError(_SPMV_STRUCT_MESSAGES["start"])
    if flags[1]:
        raise ValueError(_SPMV_STRUCT_MESSAGES["last"](None))
    if flags[2]:
        raise ValueError(_SPMV_STRUCT_MESSAGES["monotone"])
    if flags[3]:
        raise IndexError("indices out of range for n_cols")
    return y, compute_ms
