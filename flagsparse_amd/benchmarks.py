"""The reference's exported benchmark helpers for this path.

benchmark_spmv_case          (sparse_operations/benchmarks.py:343-505)
benchmark_spmm_case          (sparse_operations/spmm_csr.py:3744-4045)
benchmark_spmm_opt_case      (sparse_operations/spmm_csr.py:3619-3741)
benchmark_spmm_opt_alg2_case (sparse_operations/spmm_csr_opt_alg2.py:1024-1149)

Same signatures, same random-matrix recipe (sorted random rows, uniform
random columns with repeats, normal values; _common.py:169-203) and the
same result-dict keys, so the reference's perf scripts (tests/test_spmv.py,
tests/test_spmm.py) read them unchanged.  The keys keep the reference's
"triton_*" names; the timed operator is this package's HIP path.

The comparison legs:
  - the torch leg runs: torch.sparse.mm on a device CSR tensor (COO when
    CSR is refused), in a wider dtype for the reference values as the
    reference does (f32 -> f64, c64 -> c128, f16 / bf16 -> f32); if torch's
    sparse kernels are unavailable on this ROCm build, the reference values
    come from a dense-row expansion computed with torch ops (index_add_),
    and the reason is reported;
  - the cuSPARSE / CuPy leg reports itself unavailable (there is no CuPy on
    ROCm), with the reason in backend_status, and its fields None.
"""

import time

import torch

from ._common import _component_dtype_for_complex, _is_complex_dtype, _tolerance_for_dtype
from .spmm_csr import (
    _normalize_spmm_op,
    _spmm_op_to_name,
    _spmm_op_transposes,
    _spmm_relative_threshold,
    _spmm_validation_metrics,
    flagsparse_spmm_csr,
)
from .spmm_opt import (
    flagsparse_spmm_csr_opt,
    flagsparse_spmm_csr_opt_alg2,
    prepare_spmm_csr_opt,
    prepare_spmm_csr_opt_alg2,
)
from .spmv_csr import (
    SPMV_OP_NON,
    _normalize_spmv_op,
    _spmv_op_to_name,
    _spmv_op_transposes,
    flagsparse_spmv_csr,
    prepare_spmv_csr,
)

CUSPARSE_UNAVAILABLE = "CuPy/cuSPARSE is not available (ROCm build: no CUDA sparse backend)"


def _random_dense(size, value_dtype, device):
    """Normal values (complex: normal real and imaginary parts), as
    _build_random_dense (_common.py:169-176)."""
    if value_dtype in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        return torch.randn(size, dtype=value_dtype, device=device)
    if _is_complex_dtype(value_dtype):
        comp = _component_dtype_for_complex(value_dtype)
        return torch.complex(torch.randn(size, dtype=comp, device=device), torch.randn(size, dtype=comp, device=device))
    raise TypeError(f"Unsupported value dtype: {value_dtype}")


def _random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype, device):
    """nnz entries on sorted uniform-random rows, uniform-random columns
    (repeats allowed, unsorted within a row), int64 row pointer: the
    recipe of _build_random_csr (_common.py:186-203)."""
    if nnz <= 0 or n_rows <= 0 or n_cols <= 0:
        return (
            torch.empty(0, dtype=value_dtype, device=device),
            torch.empty(0, dtype=index_dtype, device=device),
            torch.zeros(n_rows + 1, dtype=torch.int64, device=device),
        )
    rows = torch.sort(torch.randint(0, n_rows, (nnz,), device=device))[0]
    indptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=device)
    indptr[1:] = torch.cumsum(torch.bincount(rows, minlength=n_rows), dim=0)
    indices = torch.randint(0, n_cols, (nnz,), dtype=index_dtype, device=device)
    return _random_dense(nnz, value_dtype, device), indices, indptr


def _time_device_op(op, warmup, iters):
    """(last output, wall ms per call) over `iters` calls after `warmup`,
    synchronised on both sides (the reference's _benchmark_cuda_op,
    _common.py:316-335)."""
    warmup, iters = max(0, int(warmup)), max(1, int(iters))
    out = None
    for _ in range(warmup):
        out = op()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        out = op()
    torch.cuda.synchronize()
    return out, (time.perf_counter() - t0) * 1000.0 / iters


def _wide_dtype(value_dtype):
    if value_dtype in (torch.float16, torch.bfloat16):
        return torch.float32
    if value_dtype == torch.float32:
        return torch.float64
    if value_dtype == torch.complex64:
        return torch.complex128
    return value_dtype


def _expanded_reference(data, indices, indptr, shape, dense, transposed, conj, wide):
    """op(A) @ dense in `wide` by expanding A's entries with torch ops
    (gather + index_add_): the fallback torch leg."""
    n_rows, n_cols = shape
    rows = torch.repeat_interleave(torch.arange(n_rows, device=data.device, dtype=torch.int64),
                                   indptr[1:].to(torch.int64) - indptr[:-1].to(torch.int64))
    cols = indices.to(torch.int64)
    vals = data.to(wide)
    if conj and vals.is_complex():
        vals = vals.conj()
    d = dense.to(wide)
    vec = d.ndim == 1
    if vec:
        d = d.unsqueeze(1)
    src, dst, n_out = (rows, cols, n_cols) if transposed else (cols, rows, n_rows)
    out = torch.zeros((n_out, d.shape[1]), dtype=wide, device=data.device)
    step = max(1, (1 << 24) // max(1, d.shape[1]))
    for s in range(0, vals.numel(), step):
        e = slice(s, s + step)
        out.index_add_(0, dst[e], vals[e].unsqueeze(1) * d[src[e]])
    return out.squeeze(1) if vec else out


def _torch_sparse(data, indices, indptr, shape, layout):
    idx64 = indices.to(torch.int64)
    ptr64 = indptr.to(torch.int64)
    if layout == "CSR":
        return torch.sparse_csr_tensor(ptr64, idx64, data, size=shape, device=data.device)
    rows = torch.repeat_interleave(torch.arange(shape[0], device=data.device, dtype=torch.int64), ptr64[1:] - ptr64[:-1])
    return torch.sparse_coo_tensor(torch.stack([rows, idx64]), data, shape, device=data.device).coalesce()


def _apply_op(A, dense2d, op_code_trans, conj):
    if not op_code_trans:
        return torch.sparse.mm(A, dense2d)
    At = A.conj().transpose(0, 1) if conj else A.transpose(0, 1)
    return torch.sparse.mm(At, dense2d)


def _torch_leg(data, indices, indptr, shape, dense, transposed, conj, value_dtype, warmup, iters, time_it=True):
    """(reference values in value_dtype, torch ms or None, sparse format,
    reason or None)."""
    wide = _wide_dtype(value_dtype)
    dense2d = dense.unsqueeze(1) if dense.ndim == 1 else dense
    reasons = []
    for layout in ("CSR", "COO"):
        try:
            A_ref = _torch_sparse(data.to(wide), indices, indptr, shape, layout)
            ref = _apply_op(A_ref, dense2d.to(wide), transposed, conj).to_dense()
            ref = (ref.squeeze(1) if dense.ndim == 1 else ref).to(value_dtype)
            ms = None
            if time_it:
                A = _torch_sparse(data, indices, indptr, shape, layout)
                _, ms = _time_device_op(lambda: _apply_op(A, dense2d, transposed, conj), warmup, iters)
            return ref, ms, layout, ("; ".join(reasons) or None)
        except Exception as exc:  # torch's sparse kernels refused this case
            reasons.append(f"{layout}: {exc}")
    ref = _expanded_reference(data, indices, indptr, shape, dense, transposed, conj, wide).to(value_dtype)
    return ref, None, "expanded", "; ".join(reasons)


def benchmark_spmv_case(
    n_rows=4096,
    n_cols=4096,
    nnz=65536,
    value_dtype=torch.float32,
    index_dtype=torch.int32,
    warmup=20,
    iters=200,
    block_nnz=256,
    max_segments=None,
    run_cusparse=True,
    transpose=False,
    op=None,
    index_fallback_policy="auto",
):
    """Time the prepared CSR SpMV against torch's sparse path and check it
    (benchmarks.py:343-505)."""
    device = torch.device("cuda")
    data, indices, indptr = _random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype, device)
    op_code = _normalize_spmv_op(op, transpose=transpose)
    if op is not None and bool(transpose) and op_code == SPMV_OP_NON:
        raise ValueError("transpose=True conflicts with op=non")
    transpose = _spmv_op_transposes(op_code)
    op_name = _spmv_op_to_name(op_code)
    x = _random_dense(n_rows if transpose else n_cols, value_dtype, device)
    y_size = n_cols if transpose else n_rows
    shape = (n_rows, n_cols)
    prepared = prepare_spmv_csr(data, indices, indptr, shape, block_nnz=block_nnz, max_segments=max_segments,
                                op=op_code, index_fallback_policy=index_fallback_policy)
    y, ms = _time_device_op(lambda: flagsparse_spmv_csr(x=x, prepared=prepared, return_time=False), warmup, iters)
    expected, _, _, _ = _torch_leg(data, indices, indptr, shape, x, transpose, op_name == "conj", value_dtype,
                                   warmup, iters, time_it=False)
    atol, rtol = _tolerance_for_dtype(value_dtype)
    match = torch.allclose(y, expected, atol=atol, rtol=rtol)
    max_err = float(torch.max(torch.abs(y - expected)).item()) if y_size > 0 else 0.0
    reason = CUSPARSE_UNAVAILABLE if run_cusparse else None
    if run_cusparse and value_dtype in (torch.float16, torch.bfloat16):
        reason = "float16/bfloat16 not supported by CuPy sparse; skipped"
    return {
        "parameters": {
            "n_rows": n_rows,
            "n_cols": n_cols,
            "nnz": nnz,
            "value_dtype": str(value_dtype),
            "index_dtype": str(index_dtype),
            "op": op_name,
            "transpose": transpose,
            "index_fallback_policy": str(index_fallback_policy).lower(),
            "warmup": warmup,
            "iters": iters,
        },
        "performance": {"triton_ms": ms, "cusparse_ms": None, "triton_speedup_vs_cusparse": None},
        "verification": {
            "triton_match_reference": match,
            "triton_max_error": max_err,
            "cusparse_match_reference": None,
            "cusparse_max_error": None,
        },
        "backend_status": {"cusparse_unavailable_reason": reason},
        "samples": {"triton": y, "reference": expected},
    }


def benchmark_spmm_case(
    n_rows=4096,
    n_cols=4096,
    nnz=65536,
    n_dense_cols=32,
    value_dtype=torch.float32,
    index_dtype=torch.int32,
    warmup=20,
    iters=200,
    block_n=None,
    block_nnz=None,
    max_segments=None,
    run_cusparse=True,
    op="non",
):
    """Time the public CSR SpMM (op applied per call, as the reference does)
    against torch.sparse.mm and check it (spmm_csr.py:3744-4045)."""
    op_code = _normalize_spmm_op(op)
    op_name = _spmm_op_to_name(op_code)
    transposed = _spmm_op_transposes(op_code)
    device = torch.device("cuda")
    data, indices, indptr = _random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype, device)
    B = _random_dense((n_rows if transposed else n_cols, n_dense_cols), value_dtype, device)
    shape = (n_rows, n_cols)
    kwargs = dict(data=data, indices=indices, indptr=indptr, B=B, shape=shape, block_n=block_n, block_nnz=block_nnz,
                  max_segments=max_segments, return_time=False, op=op_name)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    flagsparse_spmm_csr(**kwargs)
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1000.0
    C, ms = _time_device_op(lambda: flagsparse_spmm_csr(**kwargs), warmup, iters)
    expected, pt_ms, pt_format, pt_reason = _torch_leg(data, indices, indptr, shape, B, transposed,
                                                       op_name == "conj", value_dtype, warmup, iters)
    metrics = _spmm_validation_metrics(C, expected)
    threshold = _spmm_relative_threshold(value_dtype)
    if not run_cusparse:
        cu_reason = None
    elif value_dtype in (torch.float16, torch.bfloat16):
        cu_reason = "float16/bfloat16 not supported by CuPy sparse; skipped"
    else:
        cu_reason = CUSPARSE_UNAVAILABLE
    return {
        "parameters": {
            "format": "csr",
            "n_rows": n_rows,
            "n_cols": n_cols,
            "nnz": nnz,
            "n_dense_cols": n_dense_cols,
            "value_dtype": str(value_dtype),
            "index_dtype": str(index_dtype),
            "op": op_name,
            "warmup": warmup,
            "iters": iters,
            # Triton launch settings of the reference; the HIP kernels take
            # none of them (they are validated, then ignored)
            "block_n": block_n,
            "block_nnz": block_nnz,
            "max_segments": max_segments,
            "required_segments": None,
            "alg1_warp_size": None,
            "alg1_factor": None,
            "base_num_warps": None,
            "base_num_stages": None,
            "auto_max_segments": max_segments is None,
            "run_cusparse": run_cusparse,
        },
        "performance": {
            "pytorch_ms": pt_ms,
            "triton_ms": ms,
            "triton_first_call_ms": first_ms,
            "cusparse_ms": None,
            "triton_speedup_vs_pytorch": (pt_ms / ms if (pt_ms is not None and ms > 0) else None),
            "triton_speedup_vs_cusparse": None,
        },
        "verification": {
            "triton_match_reference": metrics["strict_allclose_match"],
            "triton_match_pytorch": metrics["strict_allclose_match"],
            "triton_max_error": metrics["max_abs_error"],
            "triton_max_abs_error": metrics["max_abs_error"],
            "triton_max_relative_error": metrics["max_relative_error"],
            "triton_sum_relative_error": metrics["sum_relative_error"],
            "triton_relative_threshold": metrics["relative_threshold"],
            "triton_strict_allclose_match": metrics["strict_allclose_match"],
            "pytorch_match_reference": True,
            "pytorch_max_error": 0.0,
            "pytorch_max_abs_error": 0.0,
            "pytorch_max_relative_error": 0.0,
            "pytorch_sum_relative_error": 0.0,
            "pytorch_relative_threshold": threshold,
            "cusparse_match_reference": None,
            "cusparse_match_pytorch": None,
            "cusparse_max_error": None,
            "cusparse_max_abs_error": None,
            "cusparse_max_relative_error": None,
            "cusparse_sum_relative_error": None,
            "cusparse_relative_threshold": threshold,
            "cusparse_strict_allclose_match": None,
        },
        "backend_status": {
            "pytorch_unavailable_reason": pt_reason,
            "pytorch_sparse_format": pt_format,
            "cusparse_unavailable_reason": cu_reason,
            "flagsparse_internal_route": "csr-hip-lane-group",
        },
        "samples": {"triton": C, "pytorch": expected, "cusparse": None},
    }


def _opt_reference_error(candidate, reference, value_dtype):
    """max |c - r| / (atol + rtol |r|) with the COO-reference tolerances
    (spmm_csr.py:3610-3616, spmm_csr_opt_alg2.py:1015-1021)."""
    if value_dtype in (torch.float32, torch.complex64):
        atol, rtol = 1e-4, 1e-2
    else:
        atol, rtol = 1e-12, 1e-10
    if candidate.numel() == 0:
        return 0.0
    return float(torch.max(torch.abs(candidate - reference) / (atol + rtol * torch.abs(reference))).item())


def benchmark_spmm_opt_case(
    n_rows=4096,
    n_cols=4096,
    nnz=65536,
    n_dense_cols=32,
    value_dtype=torch.float32,
    index_dtype=torch.int32,
    warmup=20,
    iters=200,
    run_cusparse=True,
):
    """Base vs opt SpMM against the same high-precision torch reference
    (spmm_csr.py:3619-3741)."""
    if value_dtype not in (torch.float32, torch.float64):
        raise TypeError("benchmark_spmm_opt_case only supports float32 and float64")
    device = torch.device("cuda")
    data, indices, indptr = _random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype, device)
    B = _random_dense((n_cols, n_dense_cols), value_dtype, device)
    shape = (n_rows, n_cols)
    prepared = prepare_spmm_csr_opt(data, indices, indptr, shape)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    flagsparse_spmm_csr(data, indices, indptr, B, shape)
    torch.cuda.synchronize()
    base_first = (time.perf_counter() - t0) * 1000.0
    base, base_ms = _time_device_op(lambda: flagsparse_spmm_csr(data, indices, indptr, B, shape), warmup, iters)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    flagsparse_spmm_csr_opt(B=B, prepared=prepared)
    torch.cuda.synchronize()
    opt_first = (time.perf_counter() - t0) * 1000.0
    opt, opt_ms = _time_device_op(lambda: flagsparse_spmm_csr_opt(B=B, prepared=prepared), warmup, iters)
    ref, pt_ms, _, _ = _torch_leg(data, indices, indptr, shape, B, False, False, value_dtype, warmup, iters)
    err_base = _opt_reference_error(base, ref, value_dtype)
    err_opt = _opt_reference_error(opt, ref, value_dtype)
    return {
        "parameters": {
            "n_rows": n_rows,
            "n_cols": n_cols,
            "nnz": nnz,
            "n_dense_cols": n_dense_cols,
            "value_dtype": str(value_dtype),
            "index_dtype": str(index_dtype),
        },
        "performance": {
            "base_ms": base_ms,
            "base_first_call_ms": base_first,
            "opt_ms": opt_ms,
            "opt_first_call_ms": opt_first,
            "pt_ms": pt_ms,
            "cu_ms": None,
            "opt_vs_base": (base_ms / opt_ms if opt_ms and opt_ms > 0 else None),
            "opt_vs_pt": (pt_ms / opt_ms if pt_ms is not None and opt_ms > 0 else None),
            "opt_vs_cu": None,
        },
        "verification": {
            "err_base": err_base,
            "err_opt": err_opt,
            "base_ok": err_base <= 1.0,
            "opt_ok": err_opt <= 1.0,
            "status": "PASS" if err_opt <= 1.0 else "FAIL",
        },
        "backend_status": {
            "long_row_fallback_used": bool(prepared.long_row_fallback_only),
            "flagsparse_internal_route": "csr-hip-merge-path",
        },
        "samples": {"base": base, "opt": opt, "reference": ref},
    }


def benchmark_spmm_opt_alg2_case(
    n_rows=4096,
    n_cols=4096,
    nnz=65536,
    n_dense_cols=32,
    value_dtype=torch.float32,
    index_dtype=torch.int32,
    warmup=20,
    iters=200,
    run_cusparse=True,
):
    """Base, opt and opt-alg2 SpMM against the torch reference
    (spmm_csr_opt_alg2.py:1024-1149)."""
    if value_dtype not in (torch.float32, torch.float64):
        raise TypeError("benchmark_spmm_opt_alg2_case only supports float32 and float64")
    device = torch.device("cuda")
    data, indices, indptr = _random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype, device)
    B = _random_dense((n_cols, n_dense_cols), value_dtype, device)
    shape = (n_rows, n_cols)
    prepared_opt = prepare_spmm_csr_opt(data, indices, indptr, shape)
    prepared_alg2 = prepare_spmm_csr_opt_alg2(data, indices, indptr, shape)
    base, base_ms = _time_device_op(lambda: flagsparse_spmm_csr(data, indices, indptr, B, shape), warmup, iters)
    opt, opt_ms = _time_device_op(lambda: flagsparse_spmm_csr_opt(B=B, prepared=prepared_opt), warmup, iters)
    alg2, alg2_ms = _time_device_op(lambda: flagsparse_spmm_csr_opt_alg2(B=B, prepared=prepared_alg2), warmup, iters)
    ref, pt_ms, _, _ = _torch_leg(data, indices, indptr, shape, B, False, False, value_dtype, warmup, iters)
    return {
        "parameters": {
            "n_rows": n_rows,
            "n_cols": n_cols,
            "nnz": nnz,
            "n_dense_cols": n_dense_cols,
            "value_dtype": str(value_dtype),
            "index_dtype": str(index_dtype),
        },
        "performance": {
            "base_ms": base_ms,
            "opt_ms": opt_ms,
            "opt_alg2_ms": alg2_ms,
            "torch_ms": pt_ms,
            "cusparse_ms": None,
        },
        "verification": {
            "base_vs_torch_err": _opt_reference_error(base, ref, value_dtype),
            "opt_vs_torch_err": _opt_reference_error(opt, ref, value_dtype),
            "opt_alg2_vs_torch_err": _opt_reference_error(alg2, ref, value_dtype),
            "base_vs_cusparse_err": None,
            "opt_vs_cusparse_err": None,
            "opt_alg2_vs_cusparse_err": None,
        },
        "backend_status": {"cusparse_unavailable_reason": CUSPARSE_UNAVAILABLE if run_cusparse else None},
        "samples": {
            "base_triton": base,
            "opt_triton": opt,
            "opt_alg2_triton": alg2,
            "torch_ref": ref,
            "cusparse_ref": None,
        },
    }
