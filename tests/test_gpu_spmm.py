"""GPU parity of CSR SpMM (HIP kernels vs the CPU oracle and dense references).

Mirrors tests/pytest/test_spmm_csr_accuracy.py:85-247 and the API contract
checks of tests/test_spmm.py:766-898 of the reference (op x dtype x index
dtype, transpose timing meta, validation errors, out= path, empty matrix,
N = 0, non-contiguous B, a long row), plus dense widths that exercise every
vector width and column-tile edge, the route API and full-size properties.
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _lib
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import ELEM_TOL, INDEX_DTYPES, INDEX_IDS, OPS, REL_TOL, VALUE_DTYPES, VALUE_IDS, np_, rel_err

pytestmark = pytest.mark.gpu


def _check(data, indices, indptr, shape, B, op, **kw):
    C = fs.flagsparse_spmm_csr(data, indices, indptr, B, shape, op=op, **kw)
    ref = O.spmm_csr_wide(np_(data), np_(indices), np_(indptr), np_(B), shape, op=op)
    assert C.dtype == data.dtype and tuple(C.shape) == ref.shape
    err = rel_err(np_(C), ref)
    assert err <= REL_TOL[data.dtype], f"rel err {err:.3e}"
    return C


_LAYOUT_ENV = ("FLAGSPARSE_SPMM_KERNEL", "FLAGSPARSE_SPMM_LPR", "FLAGSPARSE_SPMM_WAVE_ITEMS", "FLAGSPARSE_SPMM_G",
               "FLAGSPARSE_SPMM_VEC", "FLAGSPARSE_SPMM_XCD", "FLAGSPARSE_SPMM_WG_CAP")


@pytest.fixture(params=["auto", "LPR8", "LPR16", "LPR64", "LPR16-WI256", "merge", "merge-VEC2-G2"])
def lane_layout(request, monkeypatch):
    """SpMM kernel and lane layout under test.  Lane-group kernel: lanes per
    B row (LPR) and items per wave (WI, 256 gives sub-tiles of 32..256 items,
    so rows cross sub-tiles often).  Merge-path kernel: lane groups per wave
    (G) and columns per lane (VEC)."""
    for k in _LAYOUT_ENV:
        monkeypatch.delenv(k, raising=False)
    for part in request.param.split("-"):
        if part == "merge":
            monkeypatch.setenv("FLAGSPARSE_SPMM_KERNEL", "merge")
        elif part.startswith("LPR"):
            monkeypatch.setenv("FLAGSPARSE_SPMM_LPR", part[3:])
        elif part.startswith("WI"):
            monkeypatch.setenv("FLAGSPARSE_SPMM_WAVE_ITEMS", part[2:])
        elif part.startswith("G"):
            monkeypatch.setenv("FLAGSPARSE_SPMM_G", part[1:])
        elif part.startswith("VEC"):
            monkeypatch.setenv("FLAGSPARSE_SPMM_VEC", part[3:])
    return request.param


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("n_dense", [1, 4, 33, 64, 96, 130, 256, 300])
def test_spmm_matches_oracle(lane_layout, device, dtype, index_dtype, op, n_dense):
    m, k = 611, 333
    d, i, p, sh = S.random_csr(m, k, 0.03, dtype, index_dtype, device, seed=n_dense, empty_row_every=9,
                               long_rows=((300, 330),))
    B = S.dense(m if op != "non" else k, n_dense, dtype, device, seed=5)
    _check(d, i, p, sh, B, op)


@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("lpr", ["16", "32"])
def test_spmm_group_row_pointer_view_at_odd_word(device, monkeypatch, index_dtype, lpr):
    """The lane-group kernel reads row pointers by aligned 8-byte words: an
    int32 row-pointer view that starts 4 bytes into its storage (entries in
    the upper half of their words) gives the same result as a fresh copy,
    with rows that cross sub-tiles (256 items per wave)."""
    for k in _LAYOUT_ENV:
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("FLAGSPARSE_SPMM_KERNEL", "group")
    monkeypatch.setenv("FLAGSPARSE_SPMM_LPR", lpr)
    monkeypatch.setenv("FLAGSPARSE_SPMM_WAVE_ITEMS", "256")
    d, i, p, sh = S.random_csr(1003, 517, 0.04, torch.float32, index_dtype, device, seed=11, empty_row_every=7,
                               long_rows=((500, 510),))
    store = torch.zeros(p.numel() + 1, dtype=p.dtype, device=device)
    store[1:] = p
    view = store[1:]
    if p.dtype == torch.int32:
        assert view.data_ptr() % 8 == 4
    B = S.dense(517, 24, torch.float32, device, seed=2)
    C = _check(d, i, view, sh, B, "non")
    assert _lib.last_kernel() == "spmm_group_kernel"
    assert torch.equal(C, fs.flagsparse_spmm_csr(d, i, p.clone(), B, sh))


@pytest.mark.parametrize("M,N,K", [(8, 4, 16), (64, 16, 96)])
@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("op", OPS)
def test_spmm_matches_dense_reference(device, M, N, K, dtype, index_dtype, op):
    """The reference's test_spmm_csr_op_matches_dense_reference with its tolerance."""
    g = torch.Generator(device=device)
    g.manual_seed(M * 31 + N * 7 + K)
    p = min(0.25, max(0.06, 32.0 / max(M * K, 1)))
    mask = torch.rand(M, K, device=device, generator=g) < p
    if int(mask.sum().item()) == 0:
        mask[0, 0] = True
    dense = S.dense(M, K, dtype, device, seed=3, dist="normal") * 0.125 * mask.to(dtype)
    rows, cols = torch.nonzero(mask, as_tuple=True)
    data = dense[rows, cols].contiguous()
    indptr = torch.zeros(M + 1, dtype=torch.int64, device=device)
    indptr[1:] = torch.cumsum(torch.bincount(rows, minlength=M), 0)
    indices = cols.to(index_dtype)
    indptr = indptr.to(index_dtype)
    eff = M if op != "non" else K
    B = S.dense(eff, N, dtype, device, seed=4, dist="normal") * 0.125
    wide = torch.complex128 if dtype.is_complex else torch.float64
    mat = {"non": dense, "trans": dense.t(), "conj": dense.conj().t()}[op]
    ref = (mat.to(wide) @ B.to(wide)).to(dtype)
    out = fs.flagsparse_spmm_csr(data, indices, indptr, B, (M, K), op=op)
    tol = ELEM_TOL[dtype]
    assert torch.allclose(out, ref, rtol=tol, atol=tol)


def test_spmm_long_rows_and_empty_rows(lane_layout, device):
    # rows far longer than a tile (split across tiles, fixed up in order)
    d, i, p, sh = S.random_csr(40, 20000, 0.0, torch.float32, torch.int32, device, seed=1,
                               long_rows=((3, 12000), (4, 7000), (30, 19999)))
    for n_dense in (1, 64, 256):
        B = S.dense(20000, n_dense, torch.float32, device, seed=2)
        _check(d, i, p, sh, B, "non")
    Bt = S.dense(40, 64, torch.float32, device, seed=2)
    _check(d, i, p, sh, Bt, "trans")


def test_spmm_deterministic(device):
    d, i, p, sh = S.powerlaw(1 << 15, torch.float32, torch.int32, device, seed=2)
    B = S.dense(sh[1], 64, torch.float32, device, seed=3)
    C1 = fs.flagsparse_spmm_csr(d, i, p, B, sh)
    C2 = fs.flagsparse_spmm_csr(d, i, p, B, sh)
    assert torch.equal(C1, C2)


@pytest.mark.parametrize("lanes", [{"FLAGSPARSE_SPMM_LPR": "16"}, {"FLAGSPARSE_SPMM_LPR": "64"},
                                   {"FLAGSPARSE_SPMM_KERNEL": "merge", "FLAGSPARSE_SPMM_VEC": "2"},
                                   {"FLAGSPARSE_SPMM_KERNEL": "merge", "FLAGSPARSE_SPMM_G": "2"}],
                         ids=["LPR16", "LPR64", "merge-VEC2", "merge-G2"])
def test_spmm_xcd_column_tiles_bit_identical(device, monkeypatch, lanes):
    """The XCD-affine mapping of column tiles (1-D grid, tile = id % tiles)
    changes only which XCD runs a tile: results are bit-identical to the
    2-D grid, for 2, 4 and 8 column tiles and for other counts."""
    for k in _LAYOUT_ENV:
        monkeypatch.delenv(k, raising=False)
    for k, v in lanes.items():
        monkeypatch.setenv(k, v)
    d, i, p, sh = S.powerlaw(1 << 13, torch.float32, torch.int64, device, seed=4)
    for n_dense in (64, 128, 200, 256, 512, 1024):
        B = S.dense(sh[1], n_dense, torch.float32, device, seed=n_dense)
        monkeypatch.setenv("FLAGSPARSE_SPMM_XCD", "1")
        C_xcd = fs.flagsparse_spmm_csr(d, i, p, B, sh)
        monkeypatch.setenv("FLAGSPARSE_SPMM_XCD", "0")
        C_2d = fs.flagsparse_spmm_csr(d, i, p, B, sh)
        assert torch.equal(C_xcd, C_2d), n_dense
    monkeypatch.delenv("FLAGSPARSE_SPMM_XCD")
    _check(d, i, p, sh, S.dense(sh[1], 256, torch.float32, device, seed=9), "non")


def test_spmm_api_contract(device):
    """Negative / positive API checks of tests/test_spmm.py:766-898."""
    data = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float32, device=device)
    indices = torch.tensor([0, 1, 1], dtype=torch.int32, device=device)
    indptr = torch.tensor([0, 2, 3], dtype=torch.int64, device=device)
    B = torch.randn((2, 4), dtype=torch.float32, device=device)
    f = fs.flagsparse_spmm_csr
    cases = [
        (lambda: f(data, indices, indptr, B, (2,)), ValueError),
        (lambda: f(data, indices, indptr, B[0], (2, 2)), ValueError),
        (lambda: f(data, indices, indptr, B.to(torch.float64), (2, 2)), TypeError),
        (lambda: f(data, indices, indptr, torch.randn((3, 4), device=device), (2, 2)), ValueError),
        (lambda: f(data, indices, indptr[:-1], B, (2, 2)), ValueError),
        (lambda: f(data, indices, torch.tensor([1, 2, 3], dtype=torch.int64, device=device), B, (2, 2)), ValueError),
        (lambda: f(data, indices, torch.tensor([0, 2, 2], dtype=torch.int64, device=device), B, (2, 2)), ValueError),
        (lambda: f(data, indices, torch.tensor([0, 3, 2], dtype=torch.int64, device=device), B, (2, 2)), ValueError),
        (lambda: f(data, torch.tensor([0, 3, 1], dtype=torch.int32, device=device), indptr, B, (2, 2)), IndexError),
        (lambda: f(data, indices, indptr, B, (2, 2), block_n=0), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), block_nnz=0), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), max_segments=0), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), out=torch.empty((3, 4), device=device)), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), out=torch.empty((2, 4))), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), op="bad"), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), op="non", transpose=True), ValueError),
        (lambda: f(data, indices, indptr, torch.randn((3, 4), device=device), (2, 2), op="trans"), ValueError),
        (lambda: f(data, indices, indptr, torch.randn((2, 4), device=device), (2, 2), op="trans",
                   out=torch.empty((2, 3), device=device)), ValueError),
    ]
    for fn, exc in cases:
        with pytest.raises(exc):
            fn()
    # segment-overflow override on a 1536-nnz row
    ld, li, lp, lsh = S.random_csr(4, 2048, 0.0, torch.float32, torch.int32, device, seed=1, long_rows=((1, 1536),))
    with pytest.raises(ValueError, match="max_segments override"):
        f(ld, li, lp, S.dense(2048, 8, torch.float32, device), lsh, block_nnz=128, max_segments=4)
    # positive paths
    out = torch.empty((2, 4), dtype=torch.float32, device=device)
    res = f(data, indices, indptr, B, (2, 2), out=out)
    assert res.data_ptr() == out.data_ptr()
    _check(data, indices, indptr, (2, 2), B, "non")
    _check(data, indices, indptr, (2, 2), torch.randn((2, 4), device=device), "trans")
    empty = f(torch.empty(0, device=device), torch.empty(0, dtype=torch.int32, device=device),
              torch.zeros(3, dtype=torch.int64, device=device), B, (2, 2))
    assert empty.shape == (2, 4) and torch.count_nonzero(empty).item() == 0
    assert f(data, indices, indptr, torch.empty((2, 0), device=device), (2, 2)).shape == (2, 0)
    nc = torch.randn((4, 2), device=device).t()
    assert not nc.is_contiguous()
    _check(data, indices, indptr, (2, 2), nc, "non")
    _check(ld, li, lp, lsh, S.dense(2048, 8, torch.float32, device), "non")


@pytest.mark.parametrize("op", ["trans", "conj"])
def test_spmm_transposed_structure_errors(device, op):
    """A^T / A^H queue the transpose and the SpMM behind the structure check
    and read its answer at the end: the reference's error and message still
    come first (also before a B error the reference raises after its check),
    and the next call is unaffected."""
    dt = torch.complex64 if op == "conj" else torch.float32
    data = torch.tensor([1.0, 2.0, 3.0], dtype=dt, device=device)
    good_i = torch.tensor([0, 1, 1], dtype=torch.int32, device=device)
    good_p = torch.tensor([0, 2, 3], dtype=torch.int64, device=device)
    B = torch.randn((2, 4), dtype=torch.float32, device=device).to(dt)
    bad_B = torch.randn((5, 4), dtype=torch.float32, device=device).to(dt)
    f = fs.flagsparse_spmm_csr
    cases = [
        (good_i, torch.tensor([1, 2, 3], dtype=torch.int64, device=device), ValueError, "must be 0"),
        (good_i, torch.tensor([0, 2, 2], dtype=torch.int64, device=device), ValueError, "nnz=3"),
        (good_i, torch.tensor([0, 4, 3], dtype=torch.int64, device=device), ValueError, "nondecreasing"),
        (torch.tensor([0, 3, 1], dtype=torch.int32, device=device), good_p, IndexError, "out of range"),
        (torch.tensor([0, -1, 1], dtype=torch.int32, device=device), good_p, IndexError, "out of range"),
    ]
    for idx, ptr, exc, msg in cases:
        for rhs in (B, bad_B):
            with pytest.raises(exc, match=msg):
                f(data, idx, ptr, rhs, (2, 2), op=op)
        got = f(data, good_i, good_p, B, (2, 2), op=op)
        _check(data, good_i, good_p, (2, 2), B, op)
        assert got.shape == (2, 4)
    # a valid structure with a wrong B still gets the B error
    with pytest.raises(ValueError, match="B.shape"):
        f(data, good_i, good_p, bad_B, (2, 2), op=op)


@pytest.mark.parametrize("op", ["trans", "conj"])
def test_spmm_transposed_deferred_matches_synchronous(device, op):
    """The queued-behind-the-check path (fresh C) and the synchronous one
    (out= given) give the same bits."""
    dt = torch.complex64 if op == "conj" else torch.float32
    d, i, p, sh = S.powerlaw(1 << 15, dt, torch.int32, device, seed=21)
    B = S.dense(sh[0], 16, dt, device, seed=3)
    a = fs.flagsparse_spmm_csr(d, i, p, B, sh, op=op)
    out = torch.empty_like(a)
    b = fs.flagsparse_spmm_csr(d, i, p, B, sh, op=op, out=out)
    assert torch.equal(a, b)


def test_spmm_op_validation_messages(device):
    d, i, p, sh = S.random_csr(8, 12, 0.3, torch.float32, torch.int32, device, seed=1)
    B_non = torch.randn(12, 4, device=device)
    B_trans = torch.randn(8, 4, device=device)
    with pytest.raises(ValueError, match="op must be one of"):
        fs.flagsparse_spmm_csr(d, i, p, B_non, sh, op="bad")
    with pytest.raises(ValueError, match="transpose conflicts with op"):
        fs.flagsparse_spmm_csr(d, i, p, B_non, sh, op="non", transpose=True)
    with pytest.raises(ValueError, match="transpose conflicts with op"):
        fs.flagsparse_spmm_csr(d, i, p, B_trans, sh, op="trans", transpose=False)
    with pytest.raises(ValueError, match="B.shape\\[0\\] must be n_cols=8"):
        fs.flagsparse_spmm_csr(d, i, p, B_non, sh, op="trans")
    with pytest.raises(ValueError, match="out shape/dtype must match result"):
        fs.flagsparse_spmm_csr(d, i, p, B_trans, sh, op="trans", out=torch.empty((8, 4), device=device))


def test_spmm_meta(device):
    d, i, p, sh = S.random_csr(8, 12, 0.3, torch.float32, torch.int64, device, seed=1)
    B = torch.randn(8, 4, device=device)
    out, ms, meta = fs.flagsparse_spmm_csr(d, i, p, B, sh, op="trans", return_time=True, return_meta=True)
    assert out.shape == (12, 4) and meta["op"] == "trans"
    assert meta["symbolic_ms"] >= 0.0 and meta["compute_ms"] >= 0.0
    assert ms == pytest.approx(meta["op_total_ms"])
    assert meta["op_total_ms"] == pytest.approx(meta["symbolic_ms"] + meta["compute_ms"])
    out, meta = fs.flagsparse_spmm_csr(d, i, p, torch.randn(12, 4, device=device), sh, op="non", return_meta=True)
    assert meta["symbolic_ms"] == 0.0


@pytest.mark.parametrize("alg", ["auto", "csr_base", "alg1", "alg2"])
@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("layout", ["row", "col"])
def test_spmm_route_api(device, alg, op, layout):
    d, i, p, sh = S.random_csr(97, 65, 0.1, torch.float64, torch.int32, device, seed=3)
    prep = fs.prepare_spmm_csr_route(d, i, p, sh, op=op, alg=alg)
    B = S.dense(97 if op != "non" else 65, 40, torch.float64, device, seed=1)
    if layout == "col" and alg not in ("auto", "csr_base"):
        # the reference raises for col-major on any route but csr_base (spmm_csr.py:2095-2098)
        with pytest.raises(fs.SpmmCsrAlgorithmUnavailable, match="only by csr_base"):
            fs.flagsparse_spmm_csr_run(prep, B, dense_layout=layout)
        return
    C, ms, meta = fs.flagsparse_spmm_csr_run(prep, B, dense_layout=layout, return_time=True, return_meta=True,
                                             timing=True, diagnostics=True)
    ref = O.spmm_csr_wide(np_(d), np_(i), np_(p), np_(B), sh, op=op)
    assert rel_err(np_(C), ref) <= 1e-12
    assert meta["output_layout"] == layout and meta["op"] == op
    assert ms == pytest.approx(meta["operator_ms"])


def test_spmm_route_unavailable(device):
    d, i, p, sh = S.random_csr(9, 9, 0.3, torch.float32, torch.int32, device, seed=3)
    prep = fs.prepare_spmm_csr_route(d, i, p, sh)
    with pytest.raises(fs.SpmmCsrAlgorithmUnavailable):
        fs.flagsparse_spmm_csr_run(prep, torch.randn(9, 4, device=device), alg="alpha_alg1_tle_opt")


def _host(a):
    return a if isinstance(a, np.ndarray) else np_(a)


def _sampled_rows(data, indices, indptr, B, C, rows, tol):
    """Oracle on a subset of rows; only the B rows they touch leave the GPU.
    The CSR arrays may be device tensors or host numpy arrays."""
    p = _host(indptr).astype(np.int64)
    d, c = _host(data), _host(indices).astype(np.int64)
    sub_p, sub_d, sub_c = [0], [], []
    for r in rows:
        sub_d.append(d[p[r]:p[r + 1]])
        sub_c.append(c[p[r]:p[r + 1]])
        sub_p.append(sub_p[-1] + p[r + 1] - p[r])
    cols = np.concatenate(sub_c)
    uniq, remap = np.unique(cols, return_inverse=True)
    B_sub = np_(B[torch.from_numpy(uniq).to(B.device)])
    ref = O.spmm_csr_wide(np.concatenate(sub_d), remap, np.array(sub_p), B_sub, (len(rows), len(uniq)))
    err = rel_err(np_(C[torch.tensor(rows, device=C.device)]), ref)
    assert err <= tol, f"sampled-row rel err {err:.3e}"


@pytest.mark.parametrize("config", ["uniform1M_n64", "uniform1M_n64_trans", "rmat21_n256", "rmat21_c64_n32_conj"])
def test_spmm_full_size_configs(device, config):
    """BASELINE SpMM configs at full size: sampled-row oracle + determinism."""
    if config.startswith("uniform"):
        d, i, p, sh = S.uniform_rows(1 << 20, 1 << 20, 32, torch.float32, torch.int32, device, seed=5)
        n_dense, op = 64, ("trans" if config.endswith("trans") else "non")
        B = S.dense(sh[1], n_dense, torch.float32, device, seed=6)
    else:
        cplx = "c64" in config
        dt = torch.complex64 if cplx else torch.float32
        d, i, p, sh = S.rmat(21, dtype=dt, index_dtype=torch.int64, device=device, seed=7)
        n_dense, op = (32, "conj") if cplx else (256, "non")
        B = S.dense(sh[1], n_dense, dt, device, seed=8, dist="normal")
    C = fs.flagsparse_spmm_csr(d, i, p, B, sh, op=op)
    assert torch.equal(C, fs.flagsparse_spmm_csr(d, i, p, B, sh, op=op))
    if op != "non":
        # A^T / A^H from the CPU oracle's stable transpose, not the product's
        d, i, p, sh = O.transpose_csr(np_(d), np_(i), np_(p), sh, conj=(op == "conj"))
        lengths = np.diff(p.astype(np.int64))
        longest = int(np.argmax(lengths))
    else:
        lengths = (p[1:] - p[:-1]).to(torch.int64)
        longest = int(torch.argmax(lengths).item())
    gen = np.random.default_rng(1)
    rows = sorted(set(gen.integers(0, sh[0], 1500).tolist()) | {0, sh[0] - 1, longest})
    _sampled_rows(d, i, p, B, C, rows, REL_TOL[C.dtype])


def test_spmm_skewed_columns_cap_residency_bit_identical(device, monkeypatch):
    """An R-MAT matrix (skewed columns) gets a residency cap for the
    two-columns-per-lane kernel; uniform columns do not.  The cap changes
    only how many workgroups share a CU, so results are bit-identical."""
    for k in ("FLAGSPARSE_SPMM_WG_CAP", "FLAGSPARSE_SPMM_VEC", "FLAGSPARSE_SPMM_G", "FLAGSPARSE_SPMM_XCD"):
        monkeypatch.delenv(k, raising=False)
    d, i, p, sh = S.rmat(17, dtype=torch.float32, index_dtype=torch.int64, device=device, seed=3)
    route = fs.prepare_spmm_csr_route(d, i, p, sh)
    fs.flagsparse_spmm_csr_run(route, S.dense(sh[1], 64, torch.float32, device, seed=4))
    assert route.hip_plan().csr.plan.spmm_wg_cap == 0  # N = 64: one column per lane, not measured
    B = S.dense(sh[1], 256, torch.float32, device, seed=5, dist="normal")
    C_cap = fs.flagsparse_spmm_csr_run(route, B)
    assert route.hip_plan().csr.plan.spmm_wg_cap == 4
    monkeypatch.setenv("FLAGSPARSE_SPMM_WG_CAP", "0")
    C_free = fs.flagsparse_spmm_csr_run(route, B)
    assert torch.equal(C_cap, C_free)
    _check(d, i, p, sh, S.dense(sh[1], 64, torch.float32, device, seed=6), "non")
    d, i, p, sh = S.uniform_rows(1 << 16, 1 << 16, 32, torch.float32, torch.int32, device, seed=7)
    route = fs.prepare_spmm_csr_route(d, i, p, sh)
    fs.flagsparse_spmm_csr_run(route, S.dense(sh[1], 256, torch.float32, device, seed=8))
    assert route.hip_plan().csr.plan.spmm_wg_cap == 0


@pytest.mark.parametrize("n_dense", [32, 64, 128])
def test_spmm_complex64_int32_indices_run_widened(device, monkeypatch, n_dense):
    """complex64 with int32 column indices and B rows of at least 512 bytes
    launches the int64-index kernel on a widened copy of the indices (narrower
    B runs the int32 indices as they are); the result is bit-identical to the
    int64 input's and matches the oracle."""
    for k in ("FLAGSPARSE_SPMM_WG_CAP", "FLAGSPARSE_SPMM_VEC", "FLAGSPARSE_SPMM_G", "FLAGSPARSE_SPMM_XCD"):
        monkeypatch.delenv(k, raising=False)
    d, i64, p, sh = S.rmat(14, dtype=torch.complex64, index_dtype=torch.int64, device=device, seed=9)
    B = S.dense(sh[1], n_dense, torch.complex64, device, seed=10, dist="normal")
    r32 = fs.prepare_spmm_csr_route(d, i64.to(torch.int32), p, sh)
    C32 = fs.flagsparse_spmm_csr_run(r32, B)
    if n_dense * 8 >= 512:
        wide_indices, wide_plan = r32.hip_plan()._wide
        assert wide_indices.dtype == torch.int64 and wide_plan.idx_t == 1
    else:
        assert r32.hip_plan()._wide is None
    C64 = fs.flagsparse_spmm_csr_run(fs.prepare_spmm_csr_route(d, i64, p, sh), B)
    assert torch.equal(C32, C64)
    _check(d, i64.to(torch.int32), p, sh, B, "non")


@pytest.mark.parametrize("layout", ["group", "merge"])
def test_spmm_hub_rows_spanning_hundreds_of_tiles(device, monkeypatch, layout):
    """Rows of 150,000 and 120,000 entries cross hundreds of sub-tiles (256
    items per wave for the lane-group kernel): the fix-up finds where each
    starts by a binary search over the partition and adds its fragments in
    order."""
    for k in _LAYOUT_ENV:
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("FLAGSPARSE_SPMM_KERNEL", layout)
    if layout == "group":
        monkeypatch.setenv("FLAGSPARSE_SPMM_WAVE_ITEMS", "256")
    d, i, p, sh = S.random_csr(400, 200_000, 0.0005, torch.float32, torch.int32, device, seed=9,
                               empty_row_every=11, long_rows=((7, 150_000), (200, 120_000)))
    B = S.dense(200_000, 40, torch.float32, device, seed=4)
    _check(d, i, p, sh, B, "non")
    assert _lib.last_kernel() == ("spmm_group_kernel" if layout == "group" else "spmm_merge_kernel")
