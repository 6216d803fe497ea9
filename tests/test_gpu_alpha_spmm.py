"""GPU: the AlphaSparse ALG1 SpMM entry points (alpha_spmm_alg1.py:39-182,
1037-1182) on the HIP merge-path kernel, against the CPU oracle."""

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import REL_TOL, np_, rel_err

pytestmark = pytest.mark.gpu

META_KEYS = {"device_name", "sm_count", "block_size", "block_rows", "block_cols", "grid_m", "grid_n", "warp_size",
             "factor", "num_warps", "num_stages", "order_row_path", "alpha", "beta", "max_row_nnz", "route"}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["float32", "float64"])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
@pytest.mark.parametrize("n_dense", [1, 8, 33, 64, 128, 300])
def test_alpha_spmm_alg1_matches_oracle(device, dtype, index_dtype, n_dense):
    d, i, p, sh = S.random_csr(700, 450, 0.02, dtype, index_dtype, device, seed=n_dense, empty_row_every=7,
                               long_rows=((5, 440),))
    B = S.dense(sh[1], n_dense, dtype, device, seed=3)
    C = fs.flagsparse_alpha_spmm_alg1(d, i, p, B, sh)
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)
    assert C.dtype == dtype and tuple(C.shape) == ref.shape
    assert rel_err(np_(C), ref) <= REL_TOL[dtype]


def test_alpha_spmm_alg1_prepared_meta_out_and_tle(device):
    d, i, p, sh = S.powerlaw(1 << 12, torch.float32, torch.int32, device, seed=5)
    prep = fs.prepare_alpha_spmm_alg1(d, i, p, sh)
    assert isinstance(prep, fs.PreparedAlphaSpmmAlg1)
    assert prep.max_row_nnz == int((p[1:] - p[:-1]).max())
    B = S.dense(sh[1], 96, torch.float32, device, seed=6)
    C, meta = fs.flagsparse_alpha_spmm_alg1(B=B, prepared=prep, return_meta=True)
    assert META_KEYS <= set(meta) and meta["route"] == "alpha_spmm_alg1"
    assert meta["alpha"] == 1 and meta["beta"] == 0 and meta["max_row_nnz"] == prep.max_row_nnz
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh)
    assert rel_err(np_(C), ref) <= REL_TOL[torch.float32]
    out = torch.empty_like(C)
    C2 = fs.flagsparse_alpha_spmm_alg1(B=B, prepared=prep, out=out)
    assert C2.data_ptr() == out.data_ptr() and torch.equal(C2, C)  # bit-identical repeat
    with pytest.raises(ValueError, match="Pass either raw CSR inputs or prepared, not both"):
        fs.flagsparse_alpha_spmm_alg1(d, i, p, B, sh, prepared=prep)
    with pytest.raises(ValueError, match=r"B.shape\[0\] must be n_cols"):
        fs.flagsparse_alpha_spmm_alg1(B=B[:-1], prepared=prep)
    with pytest.raises(ValueError, match="out shape/dtype must match result"):
        fs.flagsparse_alpha_spmm_alg1(B=B, prepared=prep, out=torch.empty(3, 3, device=device))
    with pytest.raises(TypeError, match="alpha_spmm_alg1 TLE routes only support float32 and float64"):
        fs.prepare_alpha_spmm_alg1(d.to(torch.complex64), i, p, sh)
    for fn in (fs.flagsparse_alpha_spmm_alg1_tle, fs.flagsparse_alpha_spmm_alg1_tle_opt,
               fs.flagsparse_alpha_spmm_alg1_tle_opt2):
        with pytest.raises(RuntimeError, match="requires FlagTree/TLE-Struct runtime support"):
            fn(B=B, prepared=prep)
        with pytest.raises(ValueError, match="B must be a 2D dense tensor"):  # checks run first
            fn(B=B[0], prepared=prep)


def test_alpha_spmm_alg1_empty(device):
    d = torch.empty(0, device=device)
    i = torch.empty(0, dtype=torch.int32, device=device)
    p = torch.zeros(6, dtype=torch.int32, device=device)
    C = fs.flagsparse_alpha_spmm_alg1(d, i, p, torch.ones(4, 3, device=device), (5, 4))
    assert C.shape == (5, 3) and int((C != 0).sum()) == 0
