"""Benchmark of the CSR SpMV / SpMM hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--no-cpu]

A step is one pass of the hot path over one synthetic input: one SpMV
y = A x (or one SpMM C = A B) through the public operator API with the
matrix prepared once (analysis / transpose outside the timed region, as
the reference's prepare_* APIs do).  Inputs are generated on the GPU from
a fixed seed and resident in HBM before timing starts.  Before the W
warm-up steps the step runs back to back, untimed, for 0.2 s so that the
timed steps do not see the GPU's clock ramp from idle.

By default every BASELINE configuration is run (C1-C5, int32 / int64,
op = non / trans / conj), each with its own K timed steps, and ONE JSON
line is printed: the headline fields are those of config 2 (27-point
stencil SpMV, 128^3 grid, fp64 / int32), and `configs` holds one entry per
configuration with the same fields.  --config NAME runs one configuration.
Each entry reports effective algorithmic HBM GB/s (bytes = values + col
indices + row pointer + x (or B) once + y (or C) once) and its fraction of
the 8 TB/s HBM3E peak, GFLOP/s, the dominant kernel's roofline entry timed
with HIP events on the launch stream, the reference CPU path (scipy CSR
product, 1 thread; torch.sparse.mm on all threads) on a bounded sample of
the same matrix, and the accuracy of the GPU output on that sample against
the fp64 oracle.
"""

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SAMPLE_MIN_FRAC = 0.01  # cpu_baseline / accuracy sample: at least 1% of nnz
SETTLE_S = 0.2  # untimed back-to-back steps before the warm-up (clock ramp)
METRIC = "effective HBM GB/s (% of peak) + GFLOP/s for CSR SpMV/SpMM, 1 MI355X"

CONFIGS = {
    "c2_spmv_stencil128_f64_i32": dict(op_kind="spmv", gen="stencil", dtype="f64", index="i32", op="non"),
    "c1_spmv_uniform4096_f32_i32": dict(op_kind="spmv", gen="uniform4096", dtype="f32", index="i32", op="non"),
    "c3_spmv_powerlaw4M_f32_i32": dict(op_kind="spmv", gen="powerlaw", dtype="f32", index="i32", op="non"),
    "c3_spmv_powerlaw4M_f32_i64": dict(op_kind="spmv", gen="powerlaw", dtype="f32", index="i64", op="non"),
    "c4_spmm_uniform1M_f32_i32_n64_non": dict(op_kind="spmm", gen="uniform1M", dtype="f32", index="i32", op="non", n=64),
    "c4_spmm_uniform1M_f32_i32_n64_trans": dict(op_kind="spmm", gen="uniform1M", dtype="f32", index="i32", op="trans",
                                                n=64),
    "c5_spmm_rmat21_f32_i64_n256_non": dict(op_kind="spmm", gen="rmat", dtype="f32", index="i64", op="non", n=256),
    "c5_spmm_rmat21_c64_i64_n32_conj": dict(op_kind="spmm", gen="rmat", dtype="c64", index="i64", op="conj", n=32),
    # not a BASELINE config: the stencil's SpMM on the prepared route (block vectors
    # in iterative solvers), where neighbouring rows share B rows
    "x_spmm_stencil128_f32_i32_n32": dict(op_kind="spmm", gen="stencil", dtype="f32", index="i32", op="non", n=32),
}
DEFAULT_CONFIG = "c2_spmv_stencil128_f64_i32"
CONFIG_ORDER = [DEFAULT_CONFIG] + [c for c in CONFIGS if c != DEFAULT_CONFIG]

PROFILES_DIR = os.path.join(ROOT, "profiles")


def profile_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` on `workload`, from the committed
    rocprofv3 summary profiles/<kernel>_<...>.md whose header reads
    "# <kernel> — <workload>" and whose table ends in a "| total | ... MB"
    row (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration).

    Returns (bytes or None, note).  A summary of the workload for another
    kernel is stale (the kernel changed since it was measured): its figure
    is not reported, the note says which kernel it covered."""
    stale = None
    try:
        names = sorted(os.listdir(PROFILES_DIR))
    except OSError:
        return None, "no profiles/ directory"
    for fn in names:
        if not fn.endswith(".md"):
            continue
        with open(os.path.join(PROFILES_DIR, fn)) as f:
            text = f.read()
        m = re.match(r"# (\S+) \u2014 (\S+)", text)
        if not m or m.group(2) != workload:
            continue
        t = re.search(r"^\| total \|[^\n]*?([0-9][0-9,]*\.?[0-9]*) MB", text, re.M)
        if t is None:
            continue
        if m.group(1) != kernel:
            stale = f"profiles/{fn} measured {m.group(1)}, not {kernel}: traffic not reported"
            continue
        return float(t.group(1).replace(",", "")) * 1e6, f"profiles/{fn}"
    return None, stale or f"no FETCH_SIZE/WRITE_SIZE summary for {kernel} on {workload} under profiles/"


def _dtypes(torch):
    return (
        {"f32": torch.float32, "f64": torch.float64, "c64": torch.complex64, "c128": torch.complex128},
        {"i32": torch.int32, "i64": torch.int64},
    )


def generate(cfg, device):
    import torch

    from flagsparse_amd import synthetic as S

    vt, it = _dtypes(torch)
    dtype, idx = vt[cfg["dtype"]], it[cfg["index"]]
    g = cfg["gen"]
    if g == "stencil":
        return S.stencil27(128, dtype, idx, device, seed=2)
    if g == "uniform4096":
        return S.uniform_rows(4096, 4096, 16, dtype, idx, device, seed=1)
    if g == "powerlaw":
        return S.powerlaw(4194304, dtype, idx, device, seed=3)
    if g == "uniform1M":
        return S.uniform_rows(1 << 20, 1 << 20, 32, dtype, idx, device, seed=5)
    if g == "rmat":
        return S.rmat(21, dtype=dtype, index_dtype=idx, device=device, seed=7)
    raise ValueError(g)


def elem_bytes(t):
    return t.element_size()


def time_loop(fn, steps, stream):
    """Average ms per call with HIP events recorded on `stream`."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def cpu_baseline(cfg, data, indices, indptr, shape, rhs, full_bytes, full_nnz, gpu_out):
    """Reference CPU path (scipy CSR product, 1 thread) on a bounded sample.

    Returns (baseline, accuracy): accuracy is max|out - y64| / max|y64| of
    the GPU output `gpu_out` on the sampled rows against the fp64 oracle
    (the reference's normwise metric, spmm_csr.py:95-103)."""
    import numpy as np
    import torch

    from oracle import cpu_baseline as CB

    d = data.cpu().numpy()
    i = indices.cpu().numpy()
    p = indptr.cpu().numpy().astype(np.int64)
    R = rhs.cpu().numpy()
    op = cfg["op"]
    if cfg["op_kind"] == "spmm" and op != "non":
        # A^T / A^H once (not timed), then rows of it: same sample policy as op=non.
        import scipy.sparse as sp

        A = sp.csr_matrix((d, i, p), shape=shape)
        A = (A.conj() if op == "conj" else A).T.tocsr()
        d, i, p, shape = A.data, A.indices, A.indptr.astype(np.int64), A.shape
        op = "non"
    budget = 1e8 if cfg["op_kind"] == "spmv" else 5e7 / max(1, R.shape[1] if R.ndim == 2 else 1)
    target = max(budget, SAMPLE_MIN_FRAC * float(p[-1]))
    rows_sel, ds, is_, ps = strided_row_sample(d, i, p, target)
    nnz_s = int(ps[-1])
    n_s = int(rows_sel.size)
    secs, reps = CB.time_scipy(ds, is_, ps, (n_s, shape[1]), R, op=op, min_seconds=2.0)
    frac = nnz_s / max(1, full_nnz)
    value = full_bytes * frac / secs / 1e9
    info = CB.host_info()
    # the other CPU path the reference compares against: torch.sparse.mm on a
    # CPU CSR tensor, all torch threads, same sample (1 s budget)
    t_secs, t_reps, t_threads = CB.time_torch_cpu(ds, is_, ps, (n_s, shape[1]), R, min_seconds=1.0)
    stride = int(rows_sel[1] - rows_sel[0]) if n_s > 1 else 1
    sample = f"every {stride}-th row of the same matrix ({n_s} rows, {nnz_s} of {full_nnz} nnz = {100.0 * frac:.2f}%)"
    torch_leg = {
        "value": round(full_bytes * frac / t_secs / 1e9, 3),
        "unit": "GB/s",
        "cores": int(t_threads),
        "sample": f"torch.sparse.mm(CPU CSR, dense) on the same rows, median of {t_reps} runs ({t_secs * 1e3:.2f} ms each)",
    }
    return {
        "value": round(value, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (
            f"scipy.sparse csr_matrix @ {'x' if R.ndim == 1 else 'B'} (the reference's CPU path), native dtype, "
            f"{sample}, median of {reps} runs ({secs * 1e3:.2f} ms each); value = full algorithmic bytes x "
            f"sampled nnz fraction / time; host {info['model']}, {info['affinity']} cores visible"
        ),
        "torch_sparse_mm": torch_leg,
    }, _accuracy(ds, is_, ps, (n_s, shape[1]), R, gpu_out[torch.from_numpy(rows_sel).to(gpu_out.device)])


def strided_row_sample(d, i, p, target_nnz):
    """Rows 0, k, 2k, ... of a CSR matrix, k the largest stride whose sample
    holds at least `target_nnz` entries (all rows when the matrix has fewer):
    the sample spreads over the whole row range instead of a leading prefix
    (which on a graph is its hub rows).  Returns (row ids, data, indices,
    indptr) of the sampled sub-matrix, same columns."""
    import numpy as np

    n_rows = p.size - 1
    total = float(p[-1])
    if total <= target_nnz or n_rows <= 1:
        rows = np.arange(n_rows, dtype=np.int64)
    else:
        lens = np.diff(p)
        k = max(1, int(total // max(1.0, target_nnz)))
        while k > 1 and float(lens[::k].sum()) < target_nnz:
            k = max(1, k * 3 // 4) if k > 4 else k - 1
        rows = np.arange(0, n_rows, k, dtype=np.int64)
    lens = (p[rows + 1] - p[rows]).astype(np.int64)
    ps = np.zeros(rows.size + 1, dtype=np.int64)
    np.cumsum(lens, out=ps[1:])
    take = np.repeat(p[rows] - ps[:-1], lens) + np.arange(int(ps[-1]), dtype=np.int64)
    return rows, d[take], i[take], ps


def _accuracy(d, i, p, shape, R, out_rows):
    """Normwise relative error of the GPU rows against the fp64 oracle."""
    from oracle import csr_oracle as O

    wide = O.spmv_csr_wide if R.ndim == 1 else O.spmm_csr_wide
    ref = wide(d, i, p, R, shape, op="non")
    import numpy as np
    import torch

    from flagsparse_amd._common import _tolerance_for_dtype

    out = out_rows.cpu().numpy()
    err = O.relative_error(out, ref)
    tol = 1e-12 if d.dtype in ("float64", "complex128") else 1e-5
    atol, rtol = _tolerance_for_dtype(torch.from_numpy(np.empty(0, dtype=d.dtype)).dtype)
    return {
        "max_rel_err": float(f"{err:.3e}"),
        "tolerance": tol,
        "pass": bool(err <= tol),
        # the reference suite's elementwise check, reported as information
        "allclose": bool(np.allclose(out, ref.astype(out.dtype), rtol=rtol, atol=atol)),
        "allclose_rtol_atol": [rtol, atol],
        "rows": int(shape[0]),
        "reference": "fp64 oracle (oracle/csr_oracle.py) on the cpu_baseline row sample",
    }


def run_config(name, args):
    """One configuration: its bench entry (the fields of the JSON line)."""
    import torch

    import flagsparse_amd as fs
    from flagsparse_amd import _lib
    from flagsparse_amd import synthetic as S

    cfg = CONFIGS[name]
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    stream = torch.cuda.current_stream(device)
    t0 = time.perf_counter()
    data, indices, indptr, shape = generate(cfg, device)
    torch.cuda.synchronize()
    gen_s = time.perf_counter() - t0
    nnz = data.numel()
    vb, ib, pb = elem_bytes(data), elem_bytes(indices), elem_bytes(indptr)
    complex_values = data.dtype.is_complex
    op = cfg["op"]
    extra = {}

    if cfg["op_kind"] == "spmv":
        t1 = time.perf_counter()
        prep = fs.prepare_spmv_csr(data, indices, indptr, shape, op=op)
        torch.cuda.synchronize()
        analysis_ms = (time.perf_counter() - t1) * 1e3
        # the same prepare again: library, allocator and code objects warm
        t1 = time.perf_counter()
        fs.prepare_spmv_csr(data, indices, indptr, shape, op=op)
        torch.cuda.synchronize()
        extra["analysis_warm_ms"] = round((time.perf_counter() - t1) * 1e3, 3)
        x = S.vector(prep.n_cols, data.dtype, device, seed=11)
        rhs = x
        step = lambda: fs.flagsparse_spmv_csr(x=x, prepared=prep)  # noqa: E731
        plan = prep.hip_plan()
        y = torch.empty(prep.n_rows, dtype=data.dtype, device=device)
        carry = prep._carry
        lib = _lib.lib()
        args_abi = (
            plan.plan, _lib.ptr(prep.data), _lib.ptr(prep.kernel_indices), _lib.ptr(prep.kernel_indptr),
            _lib.ptr(x), _lib.ptr(y), _lib.ptr(prep._part), _lib.ptr(carry), 0 if carry is None else carry.numel(),
            _lib.stream_handle(device),
        )
        kernel_call = lambda: lib.fs_spmv_csr(*args_abi)  # noqa: E731
        sell = prep._sell
        if sell is not None:
            # SELL-64 copy of a short-row matrix with column locality (the stencil)
            args_abi = (
                _lib.value_code(sell.vals.dtype), sell.col_code, _lib.index_code(sell.indptr.dtype), sell.layout,
                sell.n_rows, _lib.ptr(sell.vals), _lib.ptr(sell.cols),
                _lib.ptr(sell.table) if sell.table is not None else None, _lib.ptr(sell.slice_ptr),
                _lib.ptr(sell.indptr), _lib.ptr(x), _lib.ptr(y), _lib.stream_handle(device),
            )
            kernel_call = lambda: lib.fs_spmv_sell(*args_abi)  # noqa: E731
            extra["sell_stored_slots"] = sell.padded
            extra["sell_layout"] = "pair" if sell.layout == 1 else "slot"
            extra["sell_column_storage"] = {0: "int32", 1: "int64", 2: "int16 offset from the row",
                                            3: "uint8 code of the offset from the row"}[sell.col_code]
            if sell.table is not None:
                extra["sell_distinct_offsets"] = sell.n_codes
        pan = prep._panels
        if pan is not None:
            # column panels: the timed call is the whole panel sequence
            # (block table, panel merge, fixup, panel reduction)
            args_abi = (
                pan.plan.plan, pan.n_panels, pan.panel_nnz, _lib.ptr(pan.data), _lib.ptr(pan.indices), _lib.ptr(pan.indptr),
                _lib.ptr(x), _lib.ptr(y), _lib.ptr(pan.part), _lib.ptr(pan.ws), pan.ws.numel(),
                _lib.stream_handle(device),
            )
            kernel_call = lambda: lib.fs_spmv_csr_panels(*args_abi)  # noqa: E731
            extra["n_panels"] = pan.n_panels
        bytes_alg = S.bytes_spmv(nnz, prep.n_rows, prep.n_cols, vb, ib, pb)
        flops = S.flops_spmv(nnz, complex_values)
        extra.update(kernel_variant=prep.kernel_name, max_row_nnz=plan.max_row_nnz, analysis_ms=round(analysis_ms, 3))
        if cfg["gen"] == "stencil":
            extra["one_shot"] = _one_shot_spmv(fs, _lib, data, indices, indptr, shape, x, bytes_alg_for=(
                S.bytes_spmv(nnz, prep.n_rows, prep.n_cols, vb, ib, pb)), steps=args.steps, stream=stream, device=device)
        m, k, n_dense = prep.n_rows, prep.n_cols, 1
    else:
        n_dense = cfg["n"]
        t1 = time.perf_counter()
        if op != "non":
            from flagsparse_amd import _csr

            d_op, i_op, p_op, sh_op = _csr.transpose_csr(data, indices, indptr, shape, conj=(op == "conj"))
        else:
            d_op, i_op, p_op, sh_op = data, indices, indptr, shape
        route = fs.prepare_spmm_csr_route(d_op, i_op, p_op, sh_op, op="non")
        torch.cuda.synchronize()
        analysis_ms = (time.perf_counter() - t1) * 1e3
        m, k = sh_op
        B = S.dense(k, n_dense, data.dtype, device, seed=13, dist="normal" if cfg["gen"] == "rmat" else "uniform")
        rhs = B
        step = lambda: fs.flagsparse_spmm_csr_run(route, B)  # noqa: E731
        plan = route.hip_plan()
        plan.set_residency(route.kernel_indices, k, n_dense, route.data.dtype)  # as the public call does
        C = torch.empty((m, n_dense), dtype=data.dtype, device=device)
        lib = _lib.lib()
        tile_items, n_tiles, part = plan.tiling(data.dtype, n_dense)
        ws = _lib.workspace(lib.fs_spmm_workspace_bytes(_lib.value_code(data.dtype), n_tiles, n_dense), device)
        launch_indices, launch_plan = plan.launch_indices(route.kernel_indices, route.data.dtype, n_dense)
        args_abi = (
            launch_plan, _lib.ptr(route.data), _lib.ptr(launch_indices), _lib.ptr(route.kernel_indptr),
            _lib.ptr(B), n_dense, _lib.ptr(C), n_dense, n_dense, _lib.ptr(part), tile_items, n_tiles,
            _lib.ptr(ws), ws.numel(), _lib.stream_handle(device),
        )
        kernel_call = lambda: lib.fs_spmm_csr(*args_abi)  # noqa: E731
        step()  # the first launch builds the route's copies (the SELL-64 copy of a stencil)
        sell = plan._sell
        if sell is not None and sell.spmm_fits(B, C):
            sell_fn, sell_name, sell_args = sell.spmm_call(B, C)
            kernel_call = lambda: sell_fn(*sell_args)  # noqa: E731
            extra["sell_entry_point"] = sell_name
            extra["sell_column_storage"] = {0: "int32", 1: "int64", 2: "int16 offset from the row",
                                            3: "uint8 code of the offset from the row"}[sell.col_code]
        bytes_alg = S.bytes_spmm(nnz, m, k, n_dense, vb, ib, pb)
        flops = S.flops_spmm(nnz, n_dense, complex_values)
        extra.update(max_row_nnz=plan.csr.max_row_nnz, analysis_ms=round(analysis_ms, 3), n_dense=n_dense)
        if op != "non":
            # Public call including the per-call transpose (reference semantics).
            full = lambda: fs.flagsparse_spmm_csr(data, indices, indptr, B, shape, op=op)  # noqa: E731
            settle(full)
            extra["ms_with_transpose"] = round(time_loop(full, max(5, args.steps // 4), stream), 4)
            # the transpose alone (fs_csr_transpose), as the public call runs it
            tr = lambda: _csr.transpose_csr(data, indices, indptr, shape, conj=(op == "conj"))  # noqa: E731
            settle(tr)
            extra["transpose_ms"] = round(time_loop(tr, max(5, args.steps // 4), stream), 4)

    # Untimed clock settle (at least SETTLE_S of back-to-back steps: a step
    # is ~0.15 ms, so a handful of warm-up steps ends before the GPU leaves
    # its idle clocks), then the W warm-up steps, then exactly K timed steps.
    torch.cuda.synchronize()
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < SETTLE_S:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    ms_per_step = time_loop(step, args.steps, stream)
    rc = kernel_call()
    if rc != 0:
        raise RuntimeError(lib.fs_last_error().decode())
    kernel_name = _lib.last_kernel()  # the main kernel that launch ran
    kernel_ms = time_loop(kernel_call, args.steps, stream)

    if args.traffic_bytes is not None:
        traffic, traffic_note = args.traffic_bytes, "--traffic-bytes"
    else:
        traffic, traffic_note = profile_traffic(name, kernel_name)
    value = bytes_alg / (ms_per_step * 1e-3) / 1e9
    achieved = bytes_alg / (kernel_ms * 1e-3) / 1e9
    dtype_name = {"f32": "f32 (fp64 accumulate)", "f64": "f64", "c64": "c64 (fp64 accumulate)"}[cfg["dtype"]]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_name,
        "data": "synthetic (seeded on-device generator, flagsparse_amd/synthetic.py)",
        "config": {
            "workload": name,
            "op": op,
            "n_rows": int(m),
            "n_cols": int(k),
            "nnz": int(nnz),
            "n_dense": int(n_dense),
            "index_dtype": cfg["index"],
            "value_dtype": cfg["dtype"],
            "algorithmic_bytes": int(bytes_alg),
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "gflops": round(flops / (ms_per_step * 1e-3) / 1e9, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name,
            "kernel_ms": round(kernel_ms, 5),
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
        },
        "extra": dict(extra, generate_s=round(gen_s, 2)),
    }
    if not args.no_cpu:
        out = step()
        torch.cuda.synchronize()
        line["cpu_baseline"], line["accuracy"] = cpu_baseline(cfg, data, indices, indptr, shape, rhs, bytes_alg, nnz,
                                                              out)
    return line


def settle(fn):
    """Untimed calls of fn for at least SETTLE_S (the GPU clock ramp)."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()


def _one_shot_spmv(fs, _lib, data, indices, indptr, shape, x, bytes_alg_for, steps, stream, device):
    """What an unprepared flagsparse_spmv_csr(data, indices, indptr, x, shape)
    costs per call, wall clock: the structure checks, the launch of the
    one-launch kernel that validates while it computes, and the round trip
    that reports its flags (every call synchronises)."""
    import time

    import torch

    call = lambda: fs.flagsparse_spmv_csr(data, indices, indptr, x, shape)  # noqa: E731
    settle(call)  # the same untimed clock settle as the other legs
    kernel = _lib.last_kernel()
    n = max(20, steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        call()
    torch.cuda.synchronize()
    ms_call = (time.perf_counter() - t0) * 1e3 / n
    return {
        "ms_per_call": round(ms_call, 5),
        "kernel": kernel,
        "achieved_per_call": round(bytes_alg_for / (ms_call * 1e-3) / 1e9, 2),
        "frac_per_call": round(bytes_alg_for / (ms_call * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }


def copy_calibration(args):
    """A plain device copy of known size (for scaling FETCH_SIZE / WRITE_SIZE)."""
    import torch

    n = 1 << 28  # 1 GiB of fp32
    a = torch.ones(n, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(max(1, args.steps)):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_each_way": n * 4, "launches": max(1, args.steps)}))


def _diag_check(rc):
    if rc != 0:
        from flagsparse_amd import _lib

        raise RuntimeError("fs_diag_gather_rows: " + _lib.diag_lib().fs_last_error().decode())


def _gather_floor_spmv(name, cfg, args, lib, device, stream):
    """SpMV: the x gathers alone, in the order the prepared kernel reads them
    (panel by panel for a column-panelled matrix, one launch per panel, so a
    launch's footprint is one x slice as in the panel kernel), and in plain
    CSR order in one launch."""
    import torch

    import flagsparse_amd as fs
    from flagsparse_amd import _lib
    from flagsparse_amd import synthetic as S

    data, indices, indptr, shape = generate(cfg, device)
    prep = fs.prepare_spmv_csr(data, indices, indptr, shape)
    x = S.vector(shape[1], data.dtype, device, seed=11)
    esz = x.element_size()
    chk = torch.zeros(1, dtype=torch.int32, device=device)
    sh = _lib.stream_handle(device)

    def launcher(idx_t, base_ptr, isz, lo, hi):
        return lambda: lib.fs_diag_gather_rows(idx_t, _lib.ptr(x), shape[1], esz, base_ptr + lo * isz, hi - lo,
                                               _lib.ptr(chk), sh)

    calls = []
    pan = prep._panels
    if pan is not None:
        pn = [int(pan.panel_nnz[q]) for q in range(pan.n_panels + 1)]
        isz = pan.indices.element_size()
        calls = [launcher(_lib.index_code(pan.indices.dtype), pan.indices.data_ptr(), isz, pn[q], pn[q + 1])
                 for q in range(pan.n_panels) if pn[q + 1] > pn[q]]
    plain = launcher(_lib.index_code(indices.dtype), indices.data_ptr(), indices.element_size(), 0, indices.numel())

    def seq():
        for c in calls:
            _diag_check(c())

    _diag_check(plain())
    for _ in range(max(1, args.warmup)):
        seq()
        plain()
    ms_panels = time_loop(seq, args.steps, stream) if calls else None
    ms_plain = time_loop(plain, args.steps, stream)
    spmv = run_config(name, argparse.Namespace(**{**vars(args), "no_cpu": True}))
    floor = ms_panels if ms_panels is not None else ms_plain
    print(json.dumps({
        "workload": name, "gather_floor_ms": round(floor, 5),
        "gather_floor_order": "panel by panel" if ms_panels is not None else "CSR order",
        "gather_csr_order_ms": round(ms_plain, 5), "entries_gathered": int(indices.numel()), "entry_bytes": esz,
        "gathers_per_ns": round(indices.numel() / floor / 1e6, 1),
        "spmv_kernel": spmv["roofline"]["kernel"], "spmv_kernel_ms": spmv["roofline"]["kernel_ms"],
        "spmv_over_floor": round(spmv["roofline"]["kernel_ms"] / floor, 3),
    }), flush=True)
    del data, indices, indptr, prep, x
    torch.cuda.empty_cache()


def gather_floor(args):
    """The gathers alone (fs_diag_gather_rows): for the SpMM configs the same
    B rows in the same order as the SpMM kernel reads them, for the
    power-law SpMV configs the x entries; nothing else in flight.  One JSON
    line per config: the gather time next to the kernel time from
    run_config."""
    import torch

    from flagsparse_amd import _lib
    from flagsparse_amd import synthetic as S

    device = torch.device("cuda:0")
    stream = torch.cuda.current_stream(device)
    lib = _lib.diag_lib()
    names = [args.config] if args.config else [n for n in CONFIG_ORDER if CONFIGS[n]["gen"] in ("powerlaw",)
                                                 or CONFIGS[n]["op_kind"] == "spmm"]
    for name in names:
        cfg = CONFIGS[name]
        if cfg["op_kind"] == "spmv":
            _gather_floor_spmv(name, cfg, args, lib, device, stream)
            continue
        data, indices, indptr, shape = generate(cfg, device)
        if cfg["op"] != "non":
            from flagsparse_amd import _csr

            data, indices, indptr, shape = _csr.transpose_csr(data, indices, indptr, shape, conj=cfg["op"] == "conj")
        n_dense = cfg["n"]
        B = S.dense(shape[1], n_dense, data.dtype, device, seed=13)
        row_bytes = n_dense * data.element_size()
        chk = torch.zeros(1, dtype=torch.int32, device=device)
        call = lambda: lib.fs_diag_gather_rows(  # noqa: E731
            _lib.index_code(indices.dtype), _lib.ptr(B), shape[1], row_bytes, _lib.ptr(indices), indices.numel(),
            _lib.ptr(chk), _lib.stream_handle(device))
        _diag_check(call())
        for _ in range(max(1, args.warmup)):
            call()
        ms = time_loop(call, args.steps, stream)
        gathered = indices.numel() * row_bytes
        spmm = run_config(name, argparse.Namespace(**{**vars(args), "no_cpu": True}))
        print(json.dumps({
            "workload": name, "gather_floor_ms": round(ms, 5), "rows_gathered": int(indices.numel()),
            "row_bytes": row_bytes, "gathered_GBps": round(gathered / ms / 1e6, 1),
            "spmm_kernel": spmm["roofline"]["kernel"], "spmm_kernel_ms": spmm["roofline"]["kernel_ms"],
            "spmm_over_floor": round(spmm["roofline"]["kernel_ms"] / ms, 3),
        }), flush=True)
        del data, indices, indptr, B
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="run one configuration (default: all of them, headline = " + DEFAULT_CONFIG + ")")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--traffic-bytes", type=float, default=None,
                    help="HBM bytes per launch measured with rocprofv3 FETCH_SIZE+WRITE_SIZE (scaled)")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--gather-floor", action="store_true",
                    help="time the SpMM / power-law SpMV configs' gathers alone (fs_diag_gather_rows) beside the kernel")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            json.dumps({"error": "this build runs on one GPU only: sharding the path over several GPUs "
                                 "is not implemented", "n_gpus": args.gpus}),
            flush=True,
        )
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "multi-process runs are not supported"}), flush=True)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args)
        return
    if args.gather_floor:
        gather_floor(args)
        return
    if args.config:
        print(json.dumps(run_config(args.config, args)), flush=True)
        return
    import gc

    import torch

    entries = []
    for name in CONFIG_ORDER:
        print(f"bench: {name}", file=sys.stderr, flush=True)
        entries.append(run_config(name, args))
        # the full entry on its own line; the last line carries the summary
        print(json.dumps({"bench_config_detail": entries[-1]}), flush=True)
        gc.collect()
        torch.cuda.empty_cache()
    line = {k: v for k, v in entries[0].items() if k not in ("extra",)}
    line["configs"] = [compact_entry(e) for e in entries]
    print(json.dumps(line, separators=(",", ":")), flush=True)


def compact_entry(e):
    """The figures of one config that the summary line keeps (a few hundred
    bytes each, so the last line of a full run stays near 4 KB)."""
    r = e["roofline"]
    out = {
        "workload": e["config"]["workload"],
        "value": e["value"],
        "ms_per_step": e["ms_per_step"],
        "kernel": r["kernel"],
        "kernel_ms": r["kernel_ms"],
        "frac": r["frac"],
        "traffic": r["traffic"],
    }
    x = e.get("extra", {})
    if "ms_with_transpose" in x:
        out["ms_with_transpose"] = x["ms_with_transpose"]
        out["transpose_ms"] = x.get("transpose_ms")
    if "one_shot" in x:
        out["one_shot_ms"] = x["one_shot"]["ms_per_call"]
    if "cpu_baseline" in e:
        out["cpu_GBps"] = e["cpu_baseline"]["value"]
        out["cpu_torch_GBps"] = e["cpu_baseline"]["torch_sparse_mm"]["value"]
    if "accuracy" in e:
        out["max_rel_err"] = e["accuracy"]["max_rel_err"]
        out["acc_pass"] = e["accuracy"]["pass"]
    return out


if __name__ == "__main__":
    main()
