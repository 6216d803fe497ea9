"""MatrixMarket files through the HIP path: the committed hand-written .mtx
files (general / symmetric / skew-symmetric / pattern) loaded with
load_mtx_to_csr, then SpMV (base and use_opt) and SpMM for every op,
checked against the oracle and against the hand-worked dense matrices."""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd.mtx import load_mtx_to_csr
from oracle import csr_oracle as O
from tests._helpers import OPS, np_, rel_err
from tests.test_mtx import GOLDEN_MTX, golden_mtx_path

pytestmark = pytest.mark.gpu


def _dense_op(name, op):
    a = np.array(GOLDEN_MTX[name], dtype=np.float64)
    return a if op == "non" else a.T


@pytest.mark.parametrize("name", sorted(GOLDEN_MTX))
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["float32", "float64"])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
@pytest.mark.parametrize("op", OPS)
def test_mtx_spmv_spmm(device, name, dtype, index_dtype, op):
    d, i, p, sh = load_mtx_to_csr(golden_mtx_path(name), dtype=dtype, device=device, index_dtype=index_dtype)
    assert d.is_cuda and d.dtype == dtype and i.dtype == index_dtype
    a = _dense_op(name, op)
    g = torch.Generator(device="cpu").manual_seed(len(name))
    x = torch.rand(a.shape[1], generator=g, dtype=torch.float64).to(dtype).to(device)
    tol = 1e-6 if dtype == torch.float32 else 1e-14
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(d, i, p, x, sh, op=op, use_opt=use_opt)
        ref = O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh, op=op)
        assert rel_err(np_(y), ref) <= tol
        assert rel_err(np_(y), a @ np_(x).astype(np.float64)) <= tol
    B = torch.rand(a.shape[1], 5, generator=g, dtype=torch.float64).to(dtype).to(device)
    C = fs.flagsparse_spmm_csr(d, i, p, B, sh, op=op)
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh, op=op)
    assert rel_err(np_(C), ref) <= tol
    assert rel_err(np_(C), a @ np_(B).astype(np.float64)) <= tol
