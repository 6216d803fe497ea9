"""Shared test helpers: tensor <-> numpy, tolerances, random inputs."""

import numpy as np
import torch

# Normwise bound max|y - y64| / max|y64| against the fp64-accumulated
# oracle, per value dtype (the reference's metric, spmm_csr.py:95-103).
# fp32 / complex64 results are the fp64 sum rounded once, so they sit
# within a few ulp of the oracle; the stated contract is 1e-5 / 1e-12.
REL_TOL = {
    torch.float32: 1e-5,
    torch.complex64: 1e-5,
    torch.float64: 1e-12,
    torch.complex128: 1e-12,
    torch.float16: 2e-3,
    torch.bfloat16: 1e-2,
}

# Elementwise tolerance of the reference's accuracy suite
# (tests/pytest/accuracy_utils.py:17-30), used as rtol = atol.
ELEM_TOL = {
    torch.float32: 1.3e-6,
    torch.complex64: 1.3e-6,
    torch.float64: 1e-7,
    torch.complex128: 1e-7,
}

VALUE_DTYPES = [torch.float32, torch.float64, torch.complex64, torch.complex128]
VALUE_IDS = ["float32", "float64", "complex64", "complex128"]
INDEX_DTYPES = [torch.int32, torch.int64]
INDEX_IDS = ["int32", "int64"]
OPS = ["non", "trans", "conj"]


def np_(t):
    return t.detach().cpu().numpy()


def rel_err(candidate, reference):
    c = np.asarray(candidate)
    r = np.asarray(reference)
    wide = np.complex128 if (np.iscomplexobj(c) or np.iscomplexobj(r)) else np.float64
    c = c.astype(wide)
    r = r.astype(wide)
    if r.size == 0:
        return 0.0
    num = float(np.max(np.abs(c - r)))
    den = float(np.max(np.abs(r)))
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


def csr_to_np(data, indices, indptr):
    return np_(data), np_(indices), np_(indptr)
