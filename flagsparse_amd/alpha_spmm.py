"""The AlphaSparse CSR ALG1 SpMM entry points on the HIP merge-path kernel.

Reference: sparse_operations/alpha_spmm_alg1.py.  There, ALG1 is a Triton
port of AlphaSparse's row-block CSR SpMM (one block of rows x one block of
dense columns per program), float32 / float64 only, plus three FlagTree
"TLE-Struct" variants that need ``triton.experimental.tle``
(alpha_spmm_alg1.py:13-31).  Here:

  prepare_alpha_spmm_alg1 (+ the _tle / _tle_opt / _tle_opt2 prepares)
  PreparedAlphaSpmmAlg1                 alpha_spmm_alg1.py:39-115
  flagsparse_alpha_spmm_alg1            alpha_spmm_alg1.py:1037-1071
      -> one launch of the merge-path SpMM kernel (C = A @ B, row-major
         B / C), accumulating float32 in float64 (the reference's ALG1
         accumulates float32 in float32), deterministic;
  flagsparse_alpha_spmm_alg1_tle / _tle_opt / _tle_opt2
      -> the same checks, then the RuntimeError the reference raises when
         the TLE runtime is missing (alpha_spmm_alg1.py:908-913): TLE is a
         Triton extension and this build has no Triton;
  is_alpha_spmm_alg1_tle*_available / alpha_spmm_alg1_tle*_unavailable_reason
      -> False and the reason.

The reference's build_alpha_spmm_alg1_tle_opt*_meta helpers return Triton
launch settings for the TLE kernels and are not provided.

The meta dict of flagsparse_alpha_spmm_alg1(return_meta=True) keeps the
reference's keys (alpha_spmm_alg1.py:153-178, 319-322) and fills them with
this build's launch: wavefronts of 64 lanes, four per 256-thread workgroup,
merge-path tiles of 512 items, and the column tiling the kernel uses.
"""

import torch

from ._common import _compute_dtype
from .spmm_csr import _SpmmPlan, _hip_spmm, _prepare_spmm_csr_matrix

SUPPORTED_ALPHA_SPMM_ALG1_DTYPES = (torch.float32, torch.float64)

_TLE_REASON = (
    "TLE-Struct is a FlagTree Triton extension; this build runs hand-written HIP kernels and has no Triton runtime"
)
_WAVE = 64
_WAVES_PER_GROUP = 4


class PreparedAlphaSpmmAlg1:
    """Cached CSR metadata for repeated alpha_spmm_alg1 calls (alpha_spmm_alg1.py:39-71)."""

    __slots__ = (
        "data",
        "kernel_indices",
        "kernel_indptr",
        "shape",
        "n_rows",
        "n_cols",
        "row_lengths",
        "max_row_nnz",
        "_plan",
    )

    def __init__(self, data, kernel_indices, kernel_indptr, shape, n_rows, n_cols, row_lengths, max_row_nnz):
        self.data = data
        self.kernel_indices = kernel_indices
        self.kernel_indptr = kernel_indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = int(n_rows)
        self.n_cols = int(n_cols)
        self.row_lengths = row_lengths
        self.max_row_nnz = int(max_row_nnz)
        self._plan = None

    def _hip_plan(self):
        if self._plan is None and self.n_rows > 0:
            self._plan = _SpmmPlan(self.data, self.kernel_indices, self.kernel_indptr, self.n_rows, self.n_cols)
        return self._plan


def _prepare_alpha_spmm_alg1_common(data, indices, indptr, shape):
    """alpha_spmm_alg1.py:74-95: the CSR checks of the SpMM path, then float32 / float64 only."""
    data, indices, indptr, n_rows, n_cols, _ = _prepare_spmm_csr_matrix(data, indices, indptr, shape)
    if data.dtype not in SUPPORTED_ALPHA_SPMM_ALG1_DTYPES:
        raise TypeError("alpha_spmm_alg1 TLE routes only support float32 and float64")
    row_lengths = indptr[1:] - indptr[:-1] if n_rows > 0 else indptr.new_empty((0,))
    max_row_nnz = int(row_lengths.max().item()) if n_rows > 0 else 0
    return PreparedAlphaSpmmAlg1(data, indices, indptr, shape, n_rows, n_cols, row_lengths, max_row_nnz)


def prepare_alpha_spmm_alg1(data, indices, indptr, shape):
    """Prepare CSR metadata for the ALG1 route."""
    return _prepare_alpha_spmm_alg1_common(data, indices, indptr, shape)


def prepare_alpha_spmm_alg1_tle(data, indices, indptr, shape):
    return _prepare_alpha_spmm_alg1_common(data, indices, indptr, shape)


def prepare_alpha_spmm_alg1_tle_opt(data, indices, indptr, shape):
    return _prepare_alpha_spmm_alg1_common(data, indices, indptr, shape)


def prepare_alpha_spmm_alg1_tle_opt2(data, indices, indptr, shape):
    return _prepare_alpha_spmm_alg1_common(data, indices, indptr, shape)


def _validate_runtime_inputs(prepared, B, out):
    """alpha_spmm_alg1.py:130-150 (same order and messages)."""
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
    if out is not None:
        if not out.is_cuda:
            raise ValueError("out must be a CUDA tensor")
        if out.device != prepared.data.device:
            raise ValueError("out must be on the same CUDA device as sparse matrix data")
        if out.shape != (prepared.n_rows, int(B.shape[1])) or out.dtype != prepared.data.dtype:
            raise ValueError("out shape/dtype must match result")
    return B.contiguous()


def _resolve(prepared, data, indices, indptr, shape, prepare_fn):
    """alpha_spmm_alg1.py:1047-1057."""
    if prepared is not None and not isinstance(prepared, PreparedAlphaSpmmAlg1):
        raise TypeError("prepared must be a PreparedAlphaSpmmAlg1 instance")
    raw_inputs_provided = any(arg is not None for arg in (data, indices, indptr, shape))
    if prepared is not None and raw_inputs_provided:
        raise ValueError("Pass either raw CSR inputs or prepared, not both")
    if prepared is None:
        if any(arg is None for arg in (data, indices, indptr, shape)):
            raise ValueError("data, indices, indptr, and shape are required when prepared is not provided")
        prepared = prepare_fn(data, indices, indptr, shape)
    return prepared


def _launch_meta(prepared, B, plan, route):
    """The reference's meta keys, filled with this build's launch."""
    n_dense = int(B.shape[1])
    props = torch.cuda.get_device_properties(prepared.data.device)
    # lanes per B row and columns per lane, as fs_spmm_csr chooses them
    epl = 16 // torch.empty(0, dtype=_compute_dtype(prepared.data.dtype)).element_size()
    lanes = 8
    while lanes < _WAVE and lanes * epl < n_dense:
        lanes *= 2
    vec = epl
    block_cols = lanes * epl
    tile_items, n_tiles = plan.tiling(prepared.data.dtype, n_dense)[:2] if plan is not None else (0, 0)
    waves = -(-n_tiles // (_WAVE // lanes))
    return {
        "device_name": str(getattr(props, "name", "hip")),
        "sm_count": int(getattr(props, "multi_processor_count", 0) or 0),
        "block_size": _WAVE * _WAVES_PER_GROUP,
        "block_rows": tile_items * (_WAVE // lanes),  # merge items (row ends + nnz) per wave
        "block_cols": block_cols,
        "grid_m": -(-waves // _WAVES_PER_GROUP),
        "grid_n": -(-n_dense // block_cols) if n_dense > 0 else 0,
        "warp_size": _WAVE,
        "factor": vec,
        "num_warps": _WAVES_PER_GROUP,
        "num_stages": 2,  # B-row gather batches in flight per wave (double buffered)
        "order_row_path": True,
        "alpha": 1,
        "beta": 0,
        "max_row_nnz": int(prepared.max_row_nnz),
        "route": route,
    }


def flagsparse_alpha_spmm_alg1(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None, out=None,
                               return_meta=False):
    """C = A @ B through the ALG1 entry point (alpha_spmm_alg1.py:1037-1071).  Returns C or (C, meta)."""
    prepared = _resolve(prepared, data, indices, indptr, shape, prepare_alpha_spmm_alg1)
    B = _validate_runtime_inputs(prepared, B, out)
    plan = prepared._hip_plan()
    C = _hip_spmm(prepared.data, prepared.kernel_indices, prepared.kernel_indptr, B, prepared.n_rows, plan,
                  prepared.data.dtype)
    if out is not None:
        out.copy_(C)
        C = out
    if return_meta:
        return C, _launch_meta(prepared, B, plan, "alpha_spmm_alg1")
    return C


def is_alpha_spmm_alg1_tle_available():
    return False


def alpha_spmm_alg1_tle_unavailable_reason():
    return _TLE_REASON


def is_alpha_spmm_alg1_tle_opt_available():
    return is_alpha_spmm_alg1_tle_available()


def alpha_spmm_alg1_tle_opt_unavailable_reason():
    return alpha_spmm_alg1_tle_unavailable_reason()


def is_alpha_spmm_alg1_tle_opt2_available():
    return is_alpha_spmm_alg1_tle_available()


def alpha_spmm_alg1_tle_opt2_unavailable_reason():
    return alpha_spmm_alg1_tle_unavailable_reason()


def _tle_route(name, prepare_fn, data, indices, indptr, B, shape, prepared, out):
    prepared = _resolve(prepared, data, indices, indptr, shape, prepare_fn)
    _validate_runtime_inputs(prepared, B, out)
    raise RuntimeError(f"{name} requires FlagTree/TLE-Struct runtime support ({alpha_spmm_alg1_tle_unavailable_reason()})")


def flagsparse_alpha_spmm_alg1_tle(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None, out=None,
                                   return_meta=False):
    """alpha_spmm_alg1.py:1074-1108: unavailable without the TLE runtime."""
    _tle_route("flagsparse_alpha_spmm_alg1_tle", prepare_alpha_spmm_alg1_tle, data, indices, indptr, B, shape,
               prepared, out)


def flagsparse_alpha_spmm_alg1_tle_opt(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None,
                                       out=None, return_meta=False, meta=None):
    """alpha_spmm_alg1.py:1111-1145: unavailable without the TLE runtime."""
    _tle_route("flagsparse_alpha_spmm_alg1_tle_opt", prepare_alpha_spmm_alg1_tle_opt, data, indices, indptr, B,
               shape, prepared, out)


def flagsparse_alpha_spmm_alg1_tle_opt2(data=None, indices=None, indptr=None, B=None, shape=None, prepared=None,
                                        out=None, return_meta=False, meta=None):
    """alpha_spmm_alg1.py:1148-1182: unavailable without the TLE runtime."""
    _tle_route("flagsparse_alpha_spmm_alg1_tle_opt2", prepare_alpha_spmm_alg1_tle_opt2, data, indices, indptr, B,
               shape, prepared, out)


__all__ = [
    "PreparedAlphaSpmmAlg1",
    "prepare_alpha_spmm_alg1",
    "prepare_alpha_spmm_alg1_tle",
    "prepare_alpha_spmm_alg1_tle_opt",
    "prepare_alpha_spmm_alg1_tle_opt2",
    "flagsparse_alpha_spmm_alg1",
    "flagsparse_alpha_spmm_alg1_tle",
    "flagsparse_alpha_spmm_alg1_tle_opt",
    "flagsparse_alpha_spmm_alg1_tle_opt2",
    "is_alpha_spmm_alg1_tle_available",
    "is_alpha_spmm_alg1_tle_opt_available",
    "is_alpha_spmm_alg1_tle_opt2_available",
    "alpha_spmm_alg1_tle_unavailable_reason",
    "alpha_spmm_alg1_tle_opt_unavailable_reason",
    "alpha_spmm_alg1_tle_opt2_unavailable_reason",
]
