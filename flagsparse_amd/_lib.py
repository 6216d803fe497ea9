"""ctypes binding of libflagsparse_hip.so (C ABI in include/flagsparse_hip.h).

torch is imported before the library is opened so that its bundled HIP
runtime (same soname, libamdhip64.so.7) is the one our library binds to;
torch streams and our launches then live in one runtime.

There is no CPU fallback: every compute entry point raises if the library
is missing or a call fails.
"""

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libflagsparse_hip.so")

FS_F32, FS_F64, FS_C64, FS_C128 = 0, 1, 2, 3
FS_I32, FS_I64 = 0, 1
FS_KERNEL_VECTOR, FS_KERNEL_MERGE, FS_KERNEL_STREAM, FS_KERNEL_NNZBLOCK = 0, 1, 2, 3
FS_HIST_BINS = 24
FS_OK, FS_E_INVALID, FS_E_WORKSPACE, FS_E_HIP = 0, -1, -2, -3

VALUE_TYPE_CODES = {
    torch.float32: FS_F32,
    torch.float64: FS_F64,
    torch.complex64: FS_C64,
    torch.complex128: FS_C128,
}
INDEX_TYPE_CODES = {torch.int32: FS_I32, torch.int64: FS_I64}
KERNEL_NAMES = {
    FS_KERNEL_VECTOR: "vector",
    FS_KERNEL_MERGE: "merge",
    FS_KERNEL_STREAM: "stream",
    FS_KERNEL_NNZBLOCK: "nnzblock",
}

# Every symbol the header declares (checked by the CPU test suite).
EXPORTED_SYMBOLS = (
    "fs_last_error",
    "fs_last_kernel",
    "fs_version",
    "fs_csr_check_bytes",
    "fs_csr_check",
    "fs_csr_check_enqueue",
    "fs_csr_transpose_bounded",
    "fs_csr_transpose_checked",
    "fs_csr_check_decode",
    "fs_csr_check_analyze_bytes",
    "fs_csr_check_analyze",
    "fs_csr_stats_bytes",
    "fs_csr_analyze",
    "fs_csr_partition",
    "fs_spmv_partition",
    "fs_spmv_csr",
    "fs_spmv_noalloc_scratch_bytes",
    "fs_spmv_csr_noalloc",
    "fs_spmv_csr_oneshot",
    "fs_spmv_opt_max_buckets",
    "fs_spmv_opt_workspace_bytes",
    "fs_spmv_opt_buckets",
    "fs_spmv_csr_opt",
    "fs_spmm_workspace_bytes",
    "fs_spmm_tile_items",
    "fs_spmm_csr",
    "fs_spmm_csr_strided",
    "fs_csr_transpose_workspace_bytes",
    "fs_csr_transpose",
    "fs_coo_to_csr_workspace_bytes",
    "fs_coo_to_csr",
    "fs_csr_panelize_workspace_bytes",
    "fs_csr_panelize",
    "fs_spmv_panels_workspace_bytes",
    "fs_spmv_csr_panels",
    "fs_sell_slots",
    "fs_sell_max_offset",
    "fs_csr_to_sell",
    "fs_spmv_sell",
    "fs_spmm_sell",
    "fs_spmm_sell_staged_fits",
    "fs_spmm_sell_staged",
)


class FsCsrPlan(ctypes.Structure):
    """Mirror of struct fs_csr_plan."""

    _fields_ = [
        ("n_rows", ctypes.c_int64),
        ("n_cols", ctypes.c_int64),
        ("nnz", ctypes.c_int64),
        ("val_t", ctypes.c_int32),
        ("idx_t", ctypes.c_int32),
        ("ptr_t", ctypes.c_int32),
        ("kernel", ctypes.c_int32),
        ("vec_width", ctypes.c_int32),
        ("tile_items", ctypes.c_int32),
        ("rows_per_block", ctypes.c_int32),
        ("spmm_wg_cap", ctypes.c_int32),
        ("n_tiles", ctypes.c_int64),
        ("max_row", ctypes.c_int64),
        ("min_row", ctypes.c_int64),
        ("hist", ctypes.c_int64 * FS_HIST_BINS),
        ("part_bytes", ctypes.c_size_t),
        ("carry_bytes", ctypes.c_size_t),
    ]


class HipLibraryError(RuntimeError):
    """A call into libflagsparse_hip failed (message from fs_last_error)."""


_lib = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_sz = ctypes.c_size_t


def _declare(lib):
    lib.fs_last_error.restype = ctypes.c_char_p
    lib.fs_last_error.argtypes = []
    lib.fs_version.restype = ctypes.c_char_p
    lib.fs_version.argtypes = []
    lib.fs_csr_check_bytes.restype = _sz
    lib.fs_csr_check_bytes.argtypes = []
    lib.fs_csr_check.restype = _i32
    lib.fs_csr_check.argtypes = [_vp, _i32, _vp, _i32, _i64, _i64, _vp, ctypes.POINTER(_i64), _vp]
    lib.fs_spmm_sell_staged_fits.restype = _i32
    lib.fs_spmm_sell_staged_fits.argtypes = [_i32, _vp, _i32, _i64]
    lib.fs_spmm_sell_staged.restype = _i32
    lib.fs_spmm_sell_staged.argtypes = [_i32, _i32, _i32, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i64,
                                        _vp, _i64, _i64, _vp]
    lib.fs_csr_transpose_bounded.restype = _i32
    lib.fs_csr_transpose_bounded.argtypes = [_i32, _i64, _i64, _i64]
    lib.fs_csr_check_enqueue.restype = _i32
    lib.fs_csr_check_enqueue.argtypes = [_vp, _i32, _vp, _i32, _i64, _i64, _vp, _vp, _vp]
    lib.fs_csr_check_decode.restype = _i32
    lib.fs_csr_check_decode.argtypes = [_vp, _i64, ctypes.POINTER(_i64)]
    lib.fs_csr_check_analyze_bytes.restype = _sz
    lib.fs_csr_check_analyze_bytes.argtypes = []
    lib.fs_csr_check_analyze.restype = _i32
    lib.fs_csr_check_analyze.argtypes = [_vp, _i32, _vp, _i32, _i32, _i64, _i64, _i64, _i32, _vp, ctypes.POINTER(_i64),
                                         ctypes.POINTER(FsCsrPlan), _vp]
    lib.fs_csr_stats_bytes.restype = _sz
    lib.fs_csr_stats_bytes.argtypes = []
    lib.fs_csr_analyze.restype = _i32
    lib.fs_csr_analyze.argtypes = [_vp, _i32, _i32, _i32, _i64, _i64, _i64, _i32, _vp,
                                   ctypes.POINTER(FsCsrPlan), _vp]
    lib.fs_csr_partition.restype = _i32
    lib.fs_csr_partition.argtypes = [ctypes.POINTER(FsCsrPlan), _vp, _vp, _i32, _i64, _vp]
    lib.fs_spmv_partition.restype = _i32
    lib.fs_spmv_partition.argtypes = [ctypes.POINTER(FsCsrPlan), _vp, _vp, _vp]
    lib.fs_spmv_csr.restype = _i32
    lib.fs_spmv_csr.argtypes = [ctypes.POINTER(FsCsrPlan), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]
    lib.fs_spmv_noalloc_scratch_bytes.restype = _sz
    lib.fs_spmv_noalloc_scratch_bytes.argtypes = []
    lib.fs_spmv_csr_noalloc.restype = _i32
    lib.fs_spmv_csr_noalloc.argtypes = [ctypes.POINTER(FsCsrPlan), _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.fs_spmv_opt_max_buckets.restype = _i32
    lib.fs_spmv_opt_max_buckets.argtypes = []
    lib.fs_spmv_opt_workspace_bytes.restype = _sz
    lib.fs_spmv_opt_workspace_bytes.argtypes = [_i64]
    lib.fs_spmv_opt_buckets.restype = _i32
    lib.fs_spmv_opt_buckets.argtypes = [_vp, _i32, _i32, _i64, _vp, _sz, ctypes.POINTER(_i64), _vp]
    lib.fs_spmv_csr_opt.restype = _i32
    lib.fs_spmv_csr_opt.argtypes = [_i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                    ctypes.POINTER(_i64), _vp]
    lib.fs_spmm_workspace_bytes.restype = _sz
    lib.fs_spmm_workspace_bytes.argtypes = [_i32, _i64, _i64]
    lib.fs_spmm_tile_items.restype = _i32
    lib.fs_spmm_tile_items.argtypes = [_i32, _i64]
    lib.fs_spmm_csr.restype = _i32
    lib.fs_spmm_csr.argtypes = [ctypes.POINTER(FsCsrPlan), _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64,
                                _vp, _i32, _i64, _vp, _sz, _vp]
    lib.fs_spmm_csr_strided.restype = _i32
    lib.fs_spmm_csr_strided.argtypes = [ctypes.POINTER(FsCsrPlan), _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64,
                                        _i64, _vp, _i32, _i64, _vp, _sz, _vp]
    lib.fs_csr_transpose_workspace_bytes.restype = _sz
    lib.fs_csr_transpose_workspace_bytes.argtypes = [_i64, _i64, _i64]
    lib.fs_csr_transpose.restype = _i32
    lib.fs_csr_transpose.argtypes = [_i32, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i32,
                                     _vp, _vp, _vp, _vp, _sz, _vp]
    lib.fs_csr_transpose_checked.restype = _i32
    lib.fs_csr_transpose_checked.argtypes = [_i32, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i32,
                                             _vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp]
    lib.fs_coo_to_csr_workspace_bytes.restype = _sz
    lib.fs_coo_to_csr_workspace_bytes.argtypes = [_i64, _i64, _i64]
    lib.fs_coo_to_csr.restype = _i32
    lib.fs_coo_to_csr.argtypes = [_i32, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _sz, _vp]
    lib.fs_csr_panelize_workspace_bytes.restype = _sz
    lib.fs_csr_panelize_workspace_bytes.argtypes = [_i64, _i64, _i64, _i32]
    lib.fs_csr_panelize.restype = _i32
    lib.fs_csr_panelize.argtypes = [_i32, _i32, _i32, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                    ctypes.POINTER(_i64), _vp, _sz, _vp]
    lib.fs_spmv_panels_workspace_bytes.restype = _sz
    lib.fs_spmv_panels_workspace_bytes.argtypes = [ctypes.POINTER(FsCsrPlan), _i32]
    lib.fs_spmv_csr_panels.restype = _i32
    lib.fs_spmv_csr_panels.argtypes = [ctypes.POINTER(FsCsrPlan), _i32, ctypes.POINTER(_i64), _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _sz, _vp]
    lib.fs_sell_slots.restype = _i32
    lib.fs_sell_slots.argtypes = [_i32, _i64, _vp, _vp, _vp]
    lib.fs_sell_max_offset.restype = _i32
    lib.fs_sell_max_offset.argtypes = [_i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp]
    lib.fs_csr_to_sell.restype = _i32
    lib.fs_csr_to_sell.argtypes = [_i32, _i32, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.fs_spmv_sell.restype = _i32
    lib.fs_spmv_sell.argtypes = [_i32, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.fs_spmv_csr_oneshot.restype = _i32
    lib.fs_spmv_csr_oneshot.argtypes = [_i32, _i32, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.fs_spmm_sell.restype = _i32
    lib.fs_spmm_sell.argtypes = [_i32, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64,
                                 _vp]
    lib.fs_last_kernel.restype = ctypes.c_char_p
    lib.fs_last_kernel.argtypes = []


def load_library(path=None):
    """Open the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise HipLibraryError(
            f"libflagsparse_hip.so not found at {p}; build it with "
            "`python -m flagsparse_amd.csrc.build` (there is no CPU fallback)"
        )
    lib = ctypes.CDLL(p, mode=ctypes.RTLD_LOCAL)
    _declare(lib)
    if path is None:
        _lib = lib
    return lib


def lib():
    return load_library()


DIAG_LIB_PATH = os.path.join(_HERE, "libflagsparse_diag.so")
_diag = None


def diag_lib():
    """The measurement-only library (libflagsparse_diag.so, declared in
    flagsparse_amd/csrc/flagsparse_diag.h): bench.py's gather-floor
    diagnostic.  Not part of the operator path or its C ABI."""
    global _diag
    if _diag is None:
        if not os.path.exists(DIAG_LIB_PATH):
            raise HipLibraryError(f"libflagsparse_diag.so not found at {DIAG_LIB_PATH}; build with "
                                  "`python -m flagsparse_amd.csrc.build`")
        d = ctypes.CDLL(DIAG_LIB_PATH, mode=ctypes.RTLD_LOCAL)
        d.fs_last_error.restype = ctypes.c_char_p
        d.fs_last_error.argtypes = []
        d.fs_diag_gather_rows.restype = ctypes.c_int32
        d.fs_diag_gather_rows.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        _diag = d
    return _diag


def last_kernel():
    """Name of the main kernel the calling thread's latest SpMV / SpMM launch
    ran, as the C side recorded it at the launch (fs_last_kernel)."""
    return lib().fs_last_kernel().decode()


def check(rc, what):
    if rc != 0:
        msg = lib().fs_last_error().decode("utf-8", "replace")
        raise HipLibraryError(f"{what} failed (status {rc}): {msg}")


def ptr(t):
    """Raw device pointer of a tensor as an int (None for empty tensors); the
    c_void_p argtypes take it as is."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


# torch's raw current-stream handle without building a Stream object (the
# public torch.cuda.current_stream path costs ~4 us per call).
_raw_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device):
    """hipStream_t of torch's current stream on `device` (an int for ctypes)."""
    if _raw_current_stream is None:
        return torch.cuda.current_stream(device).cuda_stream
    if isinstance(device, torch.device):
        index = device.index
    elif isinstance(device, int):
        index = device
    elif device is None:
        index = None
    else:
        index = torch.device(device).index
    if index is None:
        index = torch.cuda.current_device()
    return _raw_current_stream(index)


def value_code(dtype):
    try:
        return VALUE_TYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported value dtype for the HIP kernels: {dtype}") from None


def index_code(dtype):
    try:
        return INDEX_TYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported index dtype for the HIP kernels: {dtype}") from None


def workspace(nbytes, device):
    """Caller-owned scratch (the C ABI never allocates)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
