"""CPU baseline timing (the reference's CPU path: scipy / torch CSR matmul).

TEST / BENCHMARK INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg calls
this to time the CPU path on the GPU box's host cores, on the same seeded
matrix the GPU run used.  scipy's CSR matvec / matmat is single-threaded;
torch.sparse.mm on a CPU CSR tensor uses torch.get_num_threads() threads.
"""

import os
import time

import numpy as np


def _median_time(fn, min_seconds, max_reps=50):
    fn()  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < min_seconds and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def host_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"cpu_count": os.cpu_count(), "affinity": affinity, "model": model}


def time_scipy(data, indices, indptr, shape, rhs, op="non", min_seconds=10.0):
    """Median seconds of one scipy CSR product (op applied to A), 1 thread."""
    import scipy.sparse as sp

    A = sp.csr_matrix((data, indices, indptr), shape=shape)
    if op == "trans":
        A = A.T.tocsr()
    elif op == "conj":
        A = A.conj().T.tocsr()
    secs, reps = _median_time(lambda: A @ rhs, min_seconds)
    return secs, reps


def time_torch_cpu(data, indices, indptr, shape, rhs, min_seconds=5.0):
    """Median seconds of torch.sparse.mm on a CPU CSR tensor (all threads)."""
    import torch

    A = torch.sparse_csr_tensor(
        torch.from_numpy(np.asarray(indptr).astype(np.int64)),
        torch.from_numpy(np.asarray(indices).astype(np.int64)),
        torch.from_numpy(np.asarray(data)),
        size=shape,
    )
    X = torch.from_numpy(np.asarray(rhs))
    if X.ndim == 1:
        X = X.reshape(-1, 1)
    secs, reps = _median_time(lambda: torch.sparse.mm(A, X), min_seconds)
    return secs, reps, torch.get_num_threads()
