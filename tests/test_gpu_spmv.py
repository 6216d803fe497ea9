"""GPU parity of CSR SpMV (HIP kernels vs the CPU oracle and dense references).

Mirrors the reference's accuracy suite (tests/pytest/test_spmv_csr_accuracy.py:
98-233): every value dtype x index dtype x op, prepared-plan contracts and
the int64 -> int32 fallback policy; plus both kernel variants, edge cases
(empty rows / matrix, a 50,000-nnz row) and full-size properties.
"""

import os

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _lib
from flagsparse_amd import spmv_csr as spmv_mod
from flagsparse_amd import synthetic as S
from oracle import csr_oracle as O
from tests._helpers import (
    ELEM_TOL,
    INDEX_DTYPES,
    INDEX_IDS,
    OPS,
    REL_TOL,
    VALUE_DTYPES,
    VALUE_IDS,
    np_,
    rel_err,
)

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["auto", "vector", "merge", "merge-tile", "stream", "stream-vgpr-stage", "stream-entry-order", "nnzblock", "sell", "panel2",
                        "panel3", "panel4", "panel4-tile", "panel8", "panel16"])
def kernel_choice(request, monkeypatch):
    """Kernel variant under test; panelN = merge path over N column panels;
    stream-vgpr-stage = K3t staging its block through registers instead of
    direct global-to-LDS loads;
    merge-tile = the merge path with one tile per wave instead of the
    persistent pipelined walk;
    panelN-tile = the same with one tile per wave instead of the persistent
    pipelined panel kernel (which runs when N divides 8);
    sell = the SELL-64 copy, forced for every matrix; stream = row blocks
    with the slot-order gather (K3t) where rows fit, stream-entry-order =
    the entry-order row-block kernel (K3)."""
    monkeypatch.delenv("FLAGSPARSE_SPMV_PANELS", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SPMV_SELL", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SPMV_STREAM_T", raising=False)
    monkeypatch.delenv("FLAGSPARSE_PANEL_PIPE", raising=False)
    monkeypatch.delenv("FLAGSPARSE_MERGE_PIPE", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SPMV_STREAM_T_DL", raising=False)
    if request.param == "stream-vgpr-stage":
        monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", "stream")
        monkeypatch.setenv("FLAGSPARSE_SPMV_STREAM_T_DL", "0")
        return request.param
    if request.param == "merge-tile":
        monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", "merge")
        monkeypatch.setenv("FLAGSPARSE_MERGE_PIPE", "0")
        return request.param
    if request.param == "stream-entry-order":
        monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", "stream")
        monkeypatch.setenv("FLAGSPARSE_SPMV_STREAM_T", "0")
        return request.param
    if request.param == "sell":
        monkeypatch.delenv("FLAGSPARSE_SPMV_KERNEL", raising=False)
        monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
    elif request.param.startswith("panel"):
        monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", "merge")
        monkeypatch.setenv("FLAGSPARSE_SPMV_PANELS", request.param[len("panel"):].split("-")[0])
        if request.param.endswith("-tile"):
            monkeypatch.setenv("FLAGSPARSE_PANEL_PIPE", "0")
    elif request.param != "auto":
        monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", request.param)
    else:
        monkeypatch.delenv("FLAGSPARSE_SPMV_KERNEL", raising=False)
    return request.param


def _check_spmv(data, indices, indptr, shape, x, op, kernel=None):
    y = fs.flagsparse_spmv_csr(data, indices, indptr, x, shape, op=op)
    if kernel is not None and (kernel.startswith("panel") or kernel == "sell") and shape[0] > 0:
        prep = fs.prepare_spmv_csr(data, indices, indptr, shape, op=op)
        assert prep.kernel_name == ("sell" if kernel == "sell" else "panel")
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), shape, op=op)
    assert y.dtype == data.dtype
    assert tuple(y.shape) == (ref.shape[0],)
    err = rel_err(np_(y), ref)
    assert err <= REL_TOL[data.dtype], f"rel err {err:.3e} (kernel={kernel})"
    return y, ref


SHAPES = [(1, 32), (160, 1024), (128, 256), (777, 3001), (4099, 517)]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}" for m, n in SHAPES])
@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("op", OPS)
def test_spmv_matches_oracle(kernel_choice, device, shape, dtype, index_dtype, op):
    m, n = shape
    long_rows = ((m // 2, min(n - 1, 2900)),) if m > 100 else ()
    data, indices, indptr, sh = S.random_csr(m, n, 0.05, dtype, index_dtype, device, seed=m + n,
                                             empty_row_every=7 if m > 7 else 0, long_rows=long_rows)
    x = S.vector(m if op != "non" else n, dtype, device, seed=3)
    _check_spmv(data, indices, indptr, sh, x, op, kernel_choice)


def _reference_style_csr(M, N, dtype, index_dtype, device):
    # Dense-masked random matrix as in test_spmv_csr_accuracy.py:53-69.
    g = torch.Generator(device=device)
    g.manual_seed(M * 1000 + N)
    p = min(0.25, max(0.06, 32.0 / max(M * N, 1)))
    mask = torch.rand(M, N, device=device, generator=g) < p
    if int(mask.sum().item()) == 0:
        mask[0, 0] = True
    vals = S.dense(M, N, dtype, device, seed=M + 7 * N, dist="normal")
    dense = torch.where(mask, vals, torch.zeros((), dtype=dtype, device=device))
    rows, cols = torch.nonzero(mask, as_tuple=True)
    data = dense[rows, cols].contiguous()
    indptr = torch.zeros(M + 1, dtype=torch.int64, device=device)
    indptr[1:] = torch.cumsum(torch.bincount(rows, minlength=M), 0)
    return data, cols.to(index_dtype).contiguous(), indptr.to(index_dtype), dense


@pytest.mark.parametrize("M,N", [(1, 32), (160, 1024), (128, 256)])
@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("op", OPS)
def test_spmv_matches_dense_reference(device, M, N, dtype, index_dtype, op):
    """The reference's own accuracy test, with its tolerance (allclose vs dense)."""
    data, indices, indptr, dense = _reference_style_csr(M, N, dtype, index_dtype, device)
    x = S.vector(M if op != "non" else N, dtype, device, seed=11)
    wide = torch.complex128 if dtype.is_complex else torch.float64
    mat = {"non": dense, "trans": dense.t(), "conj": dense.conj().t()}[op]
    ref = (mat.to(wide) @ x.to(wide)).to(dtype)
    out = fs.flagsparse_spmv_csr(data, indices, indptr, x, shape=(M, N), op=op, index_fallback_policy="auto")
    tol = ELEM_TOL[dtype]
    assert torch.allclose(out.to(wide), ref.to(wide), rtol=tol, atol=tol)


def test_spmv_golden_fixtures(device):
    """Committed fixtures (tests/golden/spmv_*.npz) reproduce exactly."""
    import glob

    files = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "spmv_*.npz")))
    assert files, "golden fixtures missing"
    for f in files:
        z = np.load(f, allow_pickle=False)
        d = torch.from_numpy(z["data"]).to(device)
        i = torch.from_numpy(z["indices"]).to(device)
        p = torch.from_numpy(z["indptr"]).to(device)
        x = torch.from_numpy(z["x"]).to(device)
        shape = tuple(int(v) for v in z["shape"])
        op = str(z["op"])
        y = fs.flagsparse_spmv_csr(d, i, p, x, shape, op=op)
        err = rel_err(np_(y), z["y_wide"])
        assert err <= REL_TOL[d.dtype], f"{os.path.basename(f)}: rel err {err:.3e}"


@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
def test_spmv_edge_cases(kernel_choice, device, dtype):
    # empty matrix (nnz = 0): zeros
    indptr = torch.zeros(6, dtype=torch.int32, device=device)
    data = torch.empty(0, dtype=dtype, device=device)
    idx = torch.empty(0, dtype=torch.int32, device=device)
    x = S.vector(4, dtype, device)
    y = fs.flagsparse_spmv_csr(data, idx, indptr, x, (5, 4))
    assert torch.count_nonzero(y).item() == 0 and y.shape == (5,)
    # zero rows
    y = fs.flagsparse_spmv_csr(data, idx, torch.zeros(1, dtype=torch.int32, device=device), x, (0, 4))
    assert y.shape == (0,)
    # one 50,000-nnz row between empty rows, and a single-row matrix
    for m, n, rows in [(9, 60000, ((4, 50000),)), (1, 70000, ((0, 50000),))]:
        d, i, p, sh = S.random_csr(m, n, 0.0, dtype, torch.int32, device, seed=5, long_rows=rows)
        for op in ("non", "trans"):
            xx = S.vector(m if op == "trans" else n, dtype, device, seed=9)
            _check_spmv(d, i, p, sh, xx, op, kernel_choice)


def test_spmv_prepared_reuse_and_out(device):
    d, i, p, sh = S.random_csr(300, 200, 0.05, torch.float32, torch.int32, device, seed=1)
    prep = fs.prepare_spmv_csr(d, i, p, sh)
    x = S.vector(200, torch.float32, device, seed=2)
    out = torch.empty(300, dtype=torch.float32, device=device)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep, out=out)
    assert y.data_ptr() == out.data_ptr()
    y2, ms, meta = fs.flagsparse_spmv_csr(x=x, prepared=prep, return_time=True, return_meta=True)
    assert torch.equal(y, y2)
    assert ms == pytest.approx(meta["op_total_ms"])
    assert meta["symbolic_ms"] == 0.0
    # deterministic: bit-identical across runs
    assert torch.equal(y2, fs.flagsparse_spmv_csr(x=x, prepared=prep))


def test_spmv_prepared_transpose_mismatch_rejected(device):
    d, i, p, sh = S.random_csr(8, 10, 0.3, torch.float32, torch.int32, device, seed=1)
    prepared = fs.prepare_spmv_csr(d, i, p, sh, transpose=True)
    x = torch.randn(8, dtype=torch.float32, device=device)
    with pytest.raises(ValueError, match="does not match prepared.transpose"):
        fs.flagsparse_spmv_csr(x=x, prepared=prepared, transpose=False)


def test_spmv_prepared_op_mismatch_rejected(device):
    d, i, p, sh = S.random_csr(8, 10, 0.3, torch.complex64, torch.int32, device, seed=1)
    prepared = fs.prepare_spmv_csr(d, i, p, sh, op="conj")
    x = S.vector(8, torch.complex64, device)
    with pytest.raises(ValueError, match="does not match prepared.op"):
        fs.flagsparse_spmv_csr(x=x, prepared=prepared, op="trans")


def test_spmv_int64_auto_fallback_to_int32(device, monkeypatch):
    monkeypatch.setenv("FLAGSPARSE_SPMV_ONESHOT", "0")  # the general path's launcher fails
    d, i, p, sh = S.random_csr(12, 9, 0.4, torch.float32, torch.int64, device, seed=2)
    x = S.vector(9, torch.float32, device)
    ref = O.spmv_csr_wide(np_(d), np_(i), np_(p), np_(x), sh)
    state = {"forced": False}
    original = spmv_mod._hip_spmv_csr_impl_prepared

    def fail_int64_once(prepared, x_in):
        if prepared.kernel_indices.dtype == torch.int64 and not state["forced"]:
            state["forced"] = True
            raise RuntimeError("forced int64 launch failure")
        return original(prepared, x_in)

    monkeypatch.setattr(spmv_mod, "_hip_spmv_csr_impl_prepared", fail_int64_once)
    out = fs.flagsparse_spmv_csr(d, i, p, x, sh, index_fallback_policy="auto")
    assert state["forced"]
    assert rel_err(np_(out), ref) <= REL_TOL[torch.float32]


def test_spmv_int64_strict_no_fallback(device, monkeypatch):
    monkeypatch.setenv("FLAGSPARSE_SPMV_ONESHOT", "0")
    d, i, p, sh = S.random_csr(12, 9, 0.4, torch.float32, torch.int64, device, seed=2)
    x = S.vector(9, torch.float32, device)

    def fail_int64(prepared, x_in):
        raise RuntimeError("forced int64 launch failure")

    monkeypatch.setattr(spmv_mod, "_hip_spmv_csr_impl_prepared", fail_int64)
    with pytest.raises(RuntimeError, match="forced int64 launch failure"):
        fs.flagsparse_spmv_csr(d, i, p, x, sh, index_fallback_policy="strict")


def _sampled_rows_check(data, indices, indptr, shape, x, y, rows, tol):
    """Oracle on a subset of rows (cheap at full size)."""
    p = np_(indptr).astype(np.int64)
    d = np_(data)
    c = np_(indices)
    xs = np_(x)
    ys = np_(y)
    sub_p = [0]
    sub_d, sub_c = [], []
    for r in rows:
        sub_d.append(d[p[r]:p[r + 1]])
        sub_c.append(c[p[r]:p[r + 1]])
        sub_p.append(sub_p[-1] + p[r + 1] - p[r])
    ref = O.spmv_csr_wide(np.concatenate(sub_d), np.concatenate(sub_c), np.array(sub_p), xs, (len(rows), shape[1]))
    err = rel_err(ys[np.asarray(rows)], ref)
    assert err <= tol, f"sampled-row rel err {err:.3e}"


@pytest.mark.parametrize("use_opt", [False, True], ids=["base", "opt"])
def test_spmv_c1_config_full_oracle(device, use_opt):
    """BASELINE config 1 at its exact shape (4096 x 4096, f32 / int32, exactly
    16 distinct sorted columns per row): every row against the oracle,
    through the prepared and the unprepared call."""
    data, indices, indptr, sh = S.uniform_rows(4096, 4096, 16, torch.float32, torch.int32, device, seed=1)
    assert data.numel() == 4096 * 16 and indices.dtype == torch.int32 and indptr.dtype == torch.int32
    p = np_(indptr)
    c = np_(indices)
    assert np.array_equal(np.diff(p), np.full(4096, 16))
    rows_c = c.reshape(4096, 16)
    assert np.all(np.diff(rows_c, axis=1) > 0) and c.min() >= 0 and c.max() < 4096
    x = S.vector(4096, torch.float32, device, seed=11)
    ref = O.spmv_csr_wide(np_(data), c, p, np_(x), sh)
    y = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh, use_opt=use_opt)
    assert rel_err(np_(y), ref) <= REL_TOL[torch.float32]
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    y2 = fs.flagsparse_spmv_csr(x=x, prepared=prep, use_opt=use_opt)
    assert torch.equal(y, y2)
    assert np.allclose(np_(y2), ref, rtol=ELEM_TOL[torch.float32], atol=ELEM_TOL[torch.float32])


@pytest.mark.parametrize("config", ["stencil128_f64_i32", "powerlaw_f32_i32", "powerlaw_f32_i64"])
def test_spmv_full_size_configs(device, config):
    """BASELINE configs at full size: sampled-row oracle, linearity, determinism."""
    if config.startswith("stencil"):
        data, indices, indptr, sh = S.stencil27(128, torch.float64, torch.int32, device, seed=2)
        assert data.numel() == 382**3
    else:
        idt = torch.int32 if config.endswith("i32") else torch.int64
        data, indices, indptr, sh = S.powerlaw(4194304, torch.float32, idt, device, seed=3)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    x1 = S.vector(sh[1], data.dtype, device, seed=21)
    x2 = S.vector(sh[1], data.dtype, device, seed=22)
    y1 = fs.flagsparse_spmv_csr(x=x1, prepared=prep)
    y2 = fs.flagsparse_spmv_csr(x=x2, prepared=prep)
    y12 = fs.flagsparse_spmv_csr(x=x1 + x2, prepared=prep)
    lin = rel_err(np_(y12).astype(np.float64), np_(y1).astype(np.float64) + np_(y2).astype(np.float64))
    assert lin <= (1e-6 if data.dtype == torch.float32 else 1e-12)
    assert torch.equal(y1, fs.flagsparse_spmv_csr(x=x1, prepared=prep))
    lengths = (indptr[1:] - indptr[:-1]).to(torch.int64)
    longest = int(torch.argmax(lengths).item())
    gen = np.random.default_rng(0)
    rows = sorted(set(gen.integers(0, sh[0], 4000).tolist()) | {0, sh[0] - 1, longest})
    _sampled_rows_check(data, indices, indptr, sh, x1, y1, rows, REL_TOL[data.dtype])


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
def test_spmv_panels_match_unpanelled(device, monkeypatch, index_dtype):
    """Power-law matrix at the BASELINE size: the column-panel path (chosen by
    default there) agrees with the single-pass merge path and the oracle on
    sampled rows, and is deterministic.  int64 input is stacked with int32
    indices (the stacked copy is internal; the caller's tensors keep int64)."""
    monkeypatch.delenv("FLAGSPARSE_SPMV_KERNEL", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SPMV_PANELS", raising=False)
    data, indices, indptr, sh = S.powerlaw(4194304, torch.float32, index_dtype, device, seed=3)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep.kernel_name == "panel"
    assert prep._panels.indices.dtype == torch.int32 and prep._panels.indptr.dtype == torch.int32
    assert prep.kernel_indices.dtype == index_dtype
    x = S.vector(sh[1], data.dtype, device, seed=23)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x, prepared=prep))
    monkeypatch.setenv("FLAGSPARSE_SPMV_PANELS", "0")
    prep0 = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep0.kernel_name == "merge"
    y0 = fs.flagsparse_spmv_csr(x=x, prepared=prep0)
    # both are f64 sums rounded once to f32: at most one ulp apart
    diff = (y.double() - y0.double()).abs()
    assert bool((diff <= y0.double().abs() * 2.0**-23 + 1e-30).all())
    # a one-shot call (no prepared object) skips the panel copy and runs the
    # one-launch kernel: again an f64 sum rounded once
    monkeypatch.delenv("FLAGSPARSE_SPMV_PANELS")
    y1, meta = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh, return_meta=True)
    assert meta["kernel"] == "oneshot"
    diff = (y1.double() - y0.double()).abs()
    assert bool((diff <= y0.double().abs() * 2.0**-23 + 1e-30).all())
    gen = np.random.default_rng(1)
    rows = sorted(set(gen.integers(0, sh[0], 3000).tolist()) | {0, sh[0] - 1})
    _sampled_rows_check(data, indices, indptr, sh, x, y, rows, REL_TOL[data.dtype])


@pytest.mark.parametrize("n_panels", [1, 2, 4, 8, 13, 64])
def test_csr_panelize_layout(device, n_panels):
    """fs_csr_panelize writes, for row r and panel p, exactly the entries of r
    whose column lies in panel p, in CSR order (checked against numpy)."""
    from flagsparse_amd.spmv_csr import PanelledCsr

    m, n = 1500, 7001
    data, indices, indptr, sh = S.random_csr(m, n, 0.01, torch.float64, torch.int32, device, seed=4,
                                             empty_row_every=5, long_rows=((3, 6000),))
    pc = PanelledCsr(data, indices, indptr, m, n, n_panels)
    width = -(-n // n_panels)
    d, c, p = np_(data), np_(indices).astype(np.int64), np_(indptr).astype(np.int64)
    exp_d, exp_c, exp_p = [], [], [0]
    for panel in range(n_panels):
        for r in range(m):
            seg = slice(p[r], p[r + 1])
            keep = (c[seg] // width) == panel
            exp_d.append(d[seg][keep])
            exp_c.append(c[seg][keep])
            exp_p.append(exp_p[-1] + int(keep.sum()))
    assert np.array_equal(np_(pc.indptr).astype(np.int64), np.array(exp_p))
    assert np.array_equal(np_(pc.indices).astype(np.int64), np.concatenate(exp_c))
    assert np.array_equal(np_(pc.data), np.concatenate(exp_d))
    assert pc.indptr.dtype == indptr.dtype and pc.indices.dtype == indices.dtype


def _dropped(data, indices, indptr, shape, frac, seed):
    """The matrix with a random share `frac` of its entries removed."""
    g = torch.Generator(device=data.device)
    g.manual_seed(seed)
    keep = torch.rand(data.numel(), generator=g, device=data.device) >= frac
    rows = torch.repeat_interleave(torch.arange(shape[0], device=data.device), indptr[1:] - indptr[:-1])
    counts = torch.bincount(rows[keep], minlength=shape[0])
    p = torch.zeros(shape[0] + 1, dtype=indptr.dtype, device=data.device)
    p[1:] = torch.cumsum(counts, 0)
    return data[keep].contiguous(), indices[keep].contiguous(), p, shape


# column storage of the SELL copy -> (FLAGSPARSE_SELL_DELTA, FLAGSPARSE_SELL_CODES)
_SELL_STORAGE_ENV = {"codes": ("1", "1"), "int16": ("1", "0"), "int32": ("0", "1")}


def _sell_cols_dtype(storage, dtype):
    """dtype of the SELL copy's columns for a stencil-like matrix: codes are
    for values of at most 8 bytes (complex128 keeps int16 offsets)."""
    if storage == "codes" and dtype.itemsize > 8:
        return torch.int16
    return {"codes": torch.uint8, "int16": torch.int16, "int32": torch.int32}[storage]


@pytest.mark.parametrize("storage", ["codes", "int16", "int32"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64, torch.complex128],
                         ids=["f32", "f64", "c64", "c128"])
def test_spmv_sell_chosen_for_stencils(device, monkeypatch, dtype, storage):
    """A prepared 27-point stencil (64^3, 262,144 rows) gets the SELL-64 copy
    by itself and matches the oracle on sampled rows and the row-block stream
    kernel to within rounding; one-shot calls keep the CSR kernels."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_SPMV_PANELS"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("FLAGSPARSE_SELL_DELTA", _SELL_STORAGE_ENV[storage][0])
    monkeypatch.setenv("FLAGSPARSE_SELL_CODES", _SELL_STORAGE_ENV[storage][1])
    data, indices, indptr, sh = S.stencil27(64, torch.float64, torch.int32, device, seed=5)
    if dtype == torch.complex64:
        imag = S.vector(data.numel(), torch.float64, device, seed=6)
        data = torch.complex(data, imag).to(torch.complex64)
    else:
        data = data.to(dtype)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep.kernel_name == "sell"
    # 27 entries per interior row: 28 stored slots with pairs (real values with
    # offset codes or int16 offsets), 27 with slots
    pair = storage != "int32" and not dtype.is_complex
    assert prep._sell.layout == (1 if pair else 0)
    assert prep._sell.padded <= (1.07 if pair else 1.03) * data.numel()
    assert prep._sell.cols.dtype == _sell_cols_dtype(storage, dtype)
    if prep._sell.cols.dtype == torch.uint8:
        assert prep._sell.n_codes == 27
    x = S.vector(sh[1], dtype, device, seed=7)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x, prepared=prep))  # deterministic
    _, meta = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh, return_meta=True)
    assert meta["kernel"] != "sell"
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "0")
    prep0 = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep0.kernel_name != "sell"
    y0 = fs.flagsparse_spmv_csr(x=x, prepared=prep0)
    # the same per-row sums in two orders, each rounded once from the wide type
    tol = REL_TOL[dtype]
    assert rel_err(np_(y), np_(y0)) <= tol
    gen = np.random.default_rng(2)
    rows = sorted(set(gen.integers(0, sh[0], 3000).tolist()) | {0, sh[0] - 1})
    _sampled_rows_check(data, indices, indptr, sh, x, y, rows, tol)


def test_spmv_sell_not_chosen_without_locality_or_with_padding(device, monkeypatch):
    """Uniformly random columns (no locality) keep the CSR kernels.  Uneven
    rows: a stencil with 10% or 30% of its entries dropped (stored slots
    ~1.16 / ~1.30 x nnz, sampled locality ~0.50 / ~0.25) gets the copy with
    offset codes (padding bound 1.75, few offsets) but not with int16
    offsets (bounds 1.03 and 0.5); with 60% dropped (~1.6 x nnz slots) it
    still gets the copy with codes, with 75% dropped (~1.9 x) none."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_SPMV_PANELS", "FLAGSPARSE_SELL_DELTA",
              "FLAGSPARSE_SELL_CODES"):
        monkeypatch.delenv(k, raising=False)
    d, i, p, sh = S.uniform_rows(1 << 18, 1 << 18, 16, torch.float32, torch.int32, device, seed=8)
    assert fs.prepare_spmv_csr(d, i, p, sh).kernel_name != "sell"
    stencil = S.stencil27(64, torch.float64, torch.int32, device, seed=5)
    for frac in (0.1, 0.3):
        d, i, p, sh = _dropped(*stencil, frac, 9)
        prep = fs.prepare_spmv_csr(d, i, p, sh)
        assert prep.kernel_name == "sell" and prep._sell.cols.dtype == torch.uint8, frac
        x = S.vector(sh[1], torch.float64, device, seed=10)
        y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
        gen = np.random.default_rng(3)
        rows = sorted(set(gen.integers(0, sh[0], 2000).tolist()) | {0, sh[0] - 1})
        _sampled_rows_check(d, i, p, sh, x, y, rows, REL_TOL[torch.float64])
        monkeypatch.setenv("FLAGSPARSE_SELL_CODES", "0")
        assert fs.prepare_spmv_csr(d, i, p, sh).kernel_name != "sell", frac
        monkeypatch.delenv("FLAGSPARSE_SELL_CODES")
    d, i, p, sh = _dropped(*stencil, 0.6, 9)
    assert fs.prepare_spmv_csr(d, i, p, sh).kernel_name == "sell"
    d, i, p, sh = _dropped(*stencil, 0.75, 9)
    assert fs.prepare_spmv_csr(d, i, p, sh).kernel_name != "sell"


def _band(n, half, keep, dtype, device, seed):
    """Random in-band columns: each of the 2 * half + 1 diagonals kept with
    probability `keep` per row."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    offs = torch.arange(-half, half + 1, device=device)
    r = torch.arange(n, device=device).unsqueeze(1)
    c = r + offs.unsqueeze(0)
    m = (c >= 0) & (c < n) & (torch.rand(c.shape, device=device, generator=g) < keep)
    indptr = torch.zeros(n + 1, dtype=torch.int64, device=device)
    indptr[1:] = torch.cumsum(m.sum(1), 0)
    cols = c[m].to(torch.int32)
    data = torch.rand(cols.numel(), dtype=dtype, device=device, generator=g) - 0.5
    return data, cols, indptr.to(torch.int32), (n, n)


@pytest.mark.parametrize("half,keep", [(16, 0.8), (64, 0.2)])
def test_spmv_sell_chosen_for_narrow_bands(device, monkeypatch, half, keep):
    """Random in-band columns have little row-to-row locality (sampled 0.34 /
    0.04) but few offsets: the copy with offset codes is chosen (stored slots
    up to ~1.45 x nnz), and matches the oracle."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_SPMV_PANELS", "FLAGSPARSE_SELL_DELTA",
              "FLAGSPARSE_SELL_CODES"):
        monkeypatch.delenv(k, raising=False)
    d, i, p, sh = _band(1 << 18, half, keep, torch.float64, device, seed=half)
    prep = fs.prepare_spmv_csr(d, i, p, sh)
    assert prep.kernel_name == "sell" and prep._sell.cols.dtype == torch.uint8
    x = S.vector(sh[1], torch.float64, device, seed=4)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    gen = np.random.default_rng(5)
    rows = sorted(set(gen.integers(0, sh[0], 2000).tolist()) | {0, 1, sh[0] - 1})
    _sampled_rows_check(d, i, p, sh, x, y, rows, REL_TOL[torch.float64])
    # complex128 keeps int16 offsets, whose bound needs locality: not chosen
    dc = torch.complex(d, d)
    assert fs.prepare_spmv_csr(dc, i, p, sh).kernel_name != "sell"


@pytest.mark.parametrize("storage", ["int16", "int32"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["f32", "f64"])
def test_spmv_sell_padding_never_multiplied(device, monkeypatch, dtype, storage):
    """Rows of one slice with different lengths (1..7 entries, so odd lengths
    leave half-used pairs too).  Every row references only columns n..2n-1;
    x is infinite on columns 0..n-1, which is where a padding entry points
    (column 0, or offset 0 = the row's own index).  A padding entry that was
    gathered and multiplied would turn its row into nan; no row may."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
    monkeypatch.setenv("FLAGSPARSE_SELL_DELTA", _SELL_STORAGE_ENV[storage][0])
    monkeypatch.setenv("FLAGSPARSE_SELL_CODES", _SELL_STORAGE_ENV[storage][1])
    n = 256
    lengths = torch.tensor([(r % 7) + 1 for r in range(n)], dtype=torch.int64, device=device)
    indptr = torch.zeros(n + 1, dtype=torch.int32, device=device)
    indptr[1:] = torch.cumsum(lengths, 0)
    cols = []
    for r in range(n):
        start = n + (r * 13) % (n - 8)
        cols.extend(range(start, start + int(lengths[r])))
    indices = torch.tensor(cols, dtype=torch.int32, device=device)
    data = torch.ones(indices.numel(), dtype=dtype, device=device)
    x = torch.ones(2 * n, dtype=dtype, device=device)
    x[:n] = float("inf")
    prep = fs.prepare_spmv_csr(data, indices, indptr, (n, 2 * n))
    assert prep.kernel_name == "sell" and prep._sell.padded > data.numel()
    assert prep._sell.cols.dtype == _sell_cols_dtype(storage, dtype)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    assert torch.equal(y, lengths.to(dtype))


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["int32", "int64"])
def test_spmv_sell_wide_offsets_keep_absolute_columns(device, monkeypatch, index_dtype):
    """Forced SELL on a matrix with an entry 70,000 columns from its row: the
    int16 offset would overflow, so the copy stores absolute int32 columns
    and still matches the oracle."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
    monkeypatch.delenv("FLAGSPARSE_SELL_DELTA", raising=False)
    n_rows, n_cols = 1000, 80000
    data, indices, indptr, sh = S.random_csr(n_rows, n_cols, 8.0 / n_cols, torch.float64, index_dtype, device,
                                             seed=12)
    # make row 0's last entry column 70,000 (row 0 is non-empty with high probability; force it)
    assert int(indptr[1]) > 0
    indices = indices.clone()
    indices[int(indptr[1]) - 1] = 70000
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep.kernel_name == "sell" and prep._sell.cols.dtype == torch.int32
    x = S.vector(n_cols, torch.float64, device, seed=13)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), sh)
    assert rel_err(np_(y), ref) <= REL_TOL[torch.float64]


@pytest.mark.parametrize("copy", ["sell", "panel"])
def test_spmv_copy_out_of_memory_falls_back_to_csr(device, monkeypatch, copy):
    """When the optional SELL / panel copy cannot be allocated, prepare keeps
    the CSR kernels and the result is still correct."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_SPMV_PANELS"):
        monkeypatch.delenv(k, raising=False)

    def no_memory(*args, **kwargs):
        raise torch.OutOfMemoryError("injected")

    if copy == "sell":
        monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
        monkeypatch.setattr(spmv_mod.SellCsr, "__init__", no_memory)
        data, indices, indptr, sh = S.stencil27(16, torch.float64, torch.int32, device, seed=3)
    else:
        monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", "merge")
        monkeypatch.setenv("FLAGSPARSE_SPMV_PANELS", "4")
        monkeypatch.setattr(spmv_mod.PanelledCsr, "__init__", no_memory)
        data, indices, indptr, sh = S.random_csr(500, 700, 0.02, torch.float64, torch.int32, device, seed=3)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep.kernel_name not in ("sell", "panel")
    x = S.vector(sh[1], torch.float64, device, seed=4)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), sh)
    assert rel_err(np_(y), ref) <= REL_TOL[torch.float64]


def _grid_stencil(dims, offsets, dtype, device):
    """CSR of a grid stencil (row-major grid, neighbours truncated at the
    boundary), columns sorted within each row."""
    n = 1
    for d in dims:
        n *= d
    idx = torch.arange(n, device=device)
    coords, rem = [], idx
    for d in reversed(dims):
        coords.append(rem % d)
        rem = rem // d
    coords = coords[::-1]
    rows, cols = [], []
    for off in offsets:
        ok = torch.ones(n, dtype=torch.bool, device=device)
        nb = torch.zeros(n, dtype=torch.int64, device=device)
        stride = 1
        for ax in reversed(range(len(dims))):
            c = coords[ax] + off[ax]
            ok &= (c >= 0) & (c < dims[ax])
            nb += c.clamp(0, dims[ax] - 1) * stride
            stride *= dims[ax]
        rows.append(idx[ok])
        cols.append(nb[ok])
    r, c = torch.cat(rows), torch.cat(cols)
    order = torch.argsort(r * n + c)
    r, c = r[order], c[order]
    indptr = torch.zeros(n + 1, dtype=torch.int32, device=device)
    indptr[1:] = torch.cumsum(torch.bincount(r, minlength=n), 0)
    data = S.vector(c.numel(), torch.float64, device, seed=21).to(dtype)
    return data, c.to(torch.int32), indptr, (n, n)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["f32", "f64"])
@pytest.mark.parametrize(
    "grid",
    [((64, 64, 64), [(0, 0, 0), (1, 0, 0), (-1, 0, 0), (0, 1, 0), (0, -1, 0), (0, 0, 1), (0, 0, -1)]),
     ((512, 512), [(0, 0), (1, 0), (-1, 0), (0, 1), (0, -1)])],
    ids=["3d-7pt", "2d-5pt"],
)
def test_spmv_sell_other_stencils(device, monkeypatch, grid, dtype):
    """7-point 3D and 5-point 2D stencils (262,144 rows) also get the SELL copy
    (offset codes, pair layout) and match the oracle on sampled rows."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_SPMV_PANELS", "FLAGSPARSE_SELL_DELTA",
              "FLAGSPARSE_SELL_CODES"):
        monkeypatch.delenv(k, raising=False)
    dims, offsets = grid
    data, indices, indptr, sh = _grid_stencil(dims, offsets, dtype, device)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep.kernel_name == "sell" and prep._sell.layout == 1 and prep._sell.cols.dtype == torch.uint8
    assert prep._sell.n_codes == len(offsets)
    x = S.vector(sh[1], dtype, device, seed=22)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    gen = np.random.default_rng(5)
    rows = sorted(set(gen.integers(0, sh[0], 3000).tolist()) | {0, 1, sh[0] - 2, sh[0] - 1})
    _sampled_rows_check(data, indices, indptr, sh, x, y, rows, REL_TOL[dtype])


@pytest.mark.parametrize("op", ["non", "trans"])
@pytest.mark.parametrize("offset", [0, 1], ids=["aligned", "offset"])
@pytest.mark.parametrize("ptr_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("idx_dtype", INDEX_DTYPES, ids=INDEX_IDS)
def test_spmv_structure_errors(device, ptr_dtype, idx_dtype, offset, op):
    """The reference's structure checks (spmv_csr.py:546-558), their messages
    and order, with each fault placed deep in arrays larger than one
    workgroup's share so that the one-pass device check must find it.
    offset=1 passes indices that start one element into their storage (not
    16-byte aligned), which takes the scalar-load path of the check.
    op="trans" takes the path that queues the transpose and the SpMV behind
    the check (every column also holds three ones, so y is the same)."""
    n = 300_000
    per = 3
    indptr = torch.arange(0, (n + 1) * per, per, dtype=torch.int64)
    cols = (torch.arange(n * per, dtype=torch.int64) * 7) % n
    data = torch.ones(n * per, dtype=torch.float32, device=device)
    x = torch.ones(n, dtype=torch.float32, device=device)

    def call(p, c, shape=(n, n)):
        c_dev = torch.cat([c[:offset], c]).to(idx_dtype).to(device)[offset:]
        return fs.flagsparse_spmv_csr(data, c_dev, p.to(ptr_dtype).to(device), x, shape, op=op)

    y = call(indptr, cols)  # valid: every row sums three ones
    assert torch.equal(y, torch.full((n,), 3.0, device=device))

    bad = indptr.clone()
    bad += 1
    with pytest.raises(ValueError, match="indptr must start at zero"):
        call(bad, cols)
    bad = indptr.clone()
    bad[-1] -= 1
    with pytest.raises(ValueError, match="indptr\\[-1\\] must equal nnz"):
        call(bad, cols)
    bad = indptr.clone()
    bad[n - 7] = bad[n - 6] + 1  # one decreasing step near the end
    with pytest.raises(ValueError, match="non-decreasing"):
        call(bad, cols)
    # a wrong start is reported before a decreasing step
    bad[0] = 5
    with pytest.raises(ValueError, match="start at zero"):
        call(bad, cols)
    for pos, v in ((n * per - 2, n), (n * per // 2 + 11, -1), (0, -(2 ** 31) if idx_dtype == torch.int32 else -(2 ** 40))):
        c = cols.clone()
        c[pos] = v
        with pytest.raises(IndexError, match="indices out of range for n_cols"):
            call(indptr, c)
    # a column index equal to n_cols - 1 at the very end is in range
    c = cols.clone()
    c[-1] = n - 1
    call(indptr, c)
    # empty matrices pass the check
    empty = fs.flagsparse_spmv_csr(
        data[:0], cols[:0].to(idx_dtype).to(device), torch.zeros(5, dtype=ptr_dtype, device=device),
        x[:3], (4, 3))
    assert torch.equal(empty, torch.zeros(4, device=device))
    with pytest.raises(ValueError, match="must equal nnz"):
        fs.flagsparse_spmv_csr(
            data[:0], cols[:0].to(idx_dtype).to(device), torch.tensor([0, 0, 1], dtype=ptr_dtype, device=device),
            x[:3], (2, 3))


@pytest.mark.parametrize("idx_dtype", INDEX_DTYPES, ids=INDEX_IDS)
@pytest.mark.parametrize("n_panels", [1, 2, 3, 5, 8, 17, 64])
@pytest.mark.parametrize("shape", [(1, 7), (300, 1000), (20_000, 333_333), (70_000, 64)],
                         ids=["1row", "small", "wide", "narrow"])
def test_panelize_matches_stable_partition(device, idx_dtype, n_panels, shape):
    """The stacked column-panel CSR equals a stable sort of the entries by
    (panel, row) computed on the host, exactly: values, columns, row
    pointer and panel offsets.  Rows are ragged and include empty rows and a
    row spanning several sub-tiles."""
    n_rows, n_cols = shape
    g = torch.Generator().manual_seed(n_rows * 131 + n_panels)
    lengths = torch.randint(0, 9, (n_rows,), generator=g)
    lengths[torch.randint(0, n_rows, (max(1, n_rows // 50),), generator=g)] = 0
    lengths[n_rows // 2] = 5000
    indptr = torch.zeros(n_rows + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(lengths, 0)
    nnz = int(indptr[-1])
    cols = torch.randint(0, n_cols, (nnz,), generator=g)
    vals = torch.randn(nnz, generator=g, dtype=torch.float64)
    pc = spmv_mod.PanelledCsr(vals.to(device), cols.to(idx_dtype).to(device), indptr.to(device), n_rows, n_cols,
                              n_panels)
    width = -(-n_cols // n_panels)
    rows = torch.repeat_interleave(torch.arange(n_rows), lengths)
    key = (cols // width) * n_rows + rows
    order = torch.sort(key, stable=True)[1]
    assert torch.equal(pc.data.cpu(), vals[order])
    assert torch.equal(pc.indices.cpu().to(torch.int64), cols[order])
    want_ptr = torch.zeros(n_panels * n_rows + 1, dtype=torch.int64)
    want_ptr[1:] = torch.cumsum(torch.bincount(key, minlength=n_panels * n_rows), 0)
    assert torch.equal(pc.indptr.cpu().to(torch.int64), want_ptr)
    assert list(pc.panel_nnz) == [int(want_ptr[q * n_rows]) for q in range(n_panels + 1)]


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64], ids=["i32", "i64"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["f32", "f64", "c64"])
@pytest.mark.parametrize("n_offsets", [1, 255, 256, 257])
def test_spmv_sell_offset_codes_limit(device, monkeypatch, dtype, n_offsets, index_dtype):
    """Rows whose entries sit at offsets drawn from a set of K distinct offsets
    in [-1000, 1000]: with K <= 256 the SELL copy stores uint8 codes, with
    K = 257 int16 offsets.  The code path gathers the same x entries and sums
    in the same order as the int16 path, so the results are bit-identical;
    both match the oracle."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
    monkeypatch.delenv("FLAGSPARSE_SELL_DELTA", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SELL_CODES", raising=False)
    n = 20_000
    gen = np.random.default_rng(n_offsets)
    offsets = np.sort(gen.choice(np.arange(-1000, 1001), n_offsets, replace=False))
    per = min(4, n_offsets)
    rows, cols = [], []
    for r in range(n):
        picks = sorted({int(offsets[(per * r + j) % n_offsets]) for j in range(per)})
        for d in picks:
            if 0 <= r + d < n:
                rows.append(r)
                cols.append(r + d)
    rows = np.asarray(rows)
    indptr = torch.zeros(n + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(torch.bincount(torch.from_numpy(rows), minlength=n), 0)
    indices = torch.tensor(cols, dtype=index_dtype, device=device)
    indptr = indptr.to(index_dtype).to(device)
    data = S.vector(indices.numel(), dtype, device, seed=31)
    x = S.vector(n, dtype, device, seed=32)
    prep = fs.prepare_spmv_csr(data, indices, indptr, (n, n))
    assert prep.kernel_name == "sell" and prep._sell.layout == (0 if dtype.is_complex else 1)
    if n_offsets <= 256:
        assert prep._sell.cols.dtype == torch.uint8 and prep._sell.n_codes == n_offsets
    else:
        assert prep._sell.cols.dtype == torch.int16
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    monkeypatch.setenv("FLAGSPARSE_SELL_CODES", "0")
    prep16 = fs.prepare_spmv_csr(data, indices, indptr, (n, n))
    assert prep16._sell.cols.dtype == torch.int16
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x, prepared=prep16))
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), (n, n))
    assert rel_err(np_(y), ref) <= REL_TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["f32", "f64"])
def test_spmv_sell_codes_padding_never_multiplied(device, monkeypatch, dtype):
    """With offset codes a padding entry holds code 0, the smallest offset.
    Row 0 alone has offset 0 (column 0); every row has 1..7 entries at
    offsets 1000..1006, so rows of one slice differ in length and leave
    padding, including half-used pairs.  x is infinite on columns 1..n-1,
    where the padding of rows 1..n-1 points (offset 0 = the row's own
    index), and no real entry reads there.  A padding entry that was gathered
    and multiplied would turn its row into nan; no row may."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "1")
    monkeypatch.delenv("FLAGSPARSE_SELL_DELTA", raising=False)
    monkeypatch.delenv("FLAGSPARSE_SELL_CODES", raising=False)
    n = 256
    n_cols = n + 1007
    cols, lengths = [], []
    for r in range(n):
        row = ([0] if r == 0 else []) + [r + 1000 + j for j in range((r % 7) + 1)]
        cols.extend(row)
        lengths.append(len(row))
    lengths = torch.tensor(lengths, dtype=torch.int64, device=device)
    indptr = torch.zeros(n + 1, dtype=torch.int32, device=device)
    indptr[1:] = torch.cumsum(lengths, 0)
    indices = torch.tensor(cols, dtype=torch.int32, device=device)
    data = torch.ones(indices.numel(), dtype=dtype, device=device)
    x = torch.ones(n_cols, dtype=dtype, device=device)
    x[1:n] = float("inf")
    prep = fs.prepare_spmv_csr(data, indices, indptr, (n, n_cols))
    assert prep.kernel_name == "sell" and prep._sell.padded > data.numel()
    assert prep._sell.cols.dtype == torch.uint8 and prep._sell.n_codes == 8
    assert int(prep._sell.table[0]) == 0
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    assert torch.equal(y, lengths.to(dtype))


@pytest.mark.parametrize("n_panels", [2, 4, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["f32", "f64", "c64"])
def test_panel_pipelined_walk_matches_one_tile_per_wave(device, monkeypatch, n_panels, dtype):
    """The persistent pipelined panel kernel, held to one workgroup per CU so
    every wave walks many tiles (prefetch, register rotation, the repeated
    last tile), gives the same bits as one tile per wave (the per-tile
    arithmetic is the same) and matches the oracle on sampled rows."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_PANEL_PIPE"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("FLAGSPARSE_SPMV_PANELS", str(n_panels))
    data, indices, indptr, sh = S.powerlaw(300000, dtype, torch.int32, device, seed=11, clip=20000)
    x = S.vector(sh[1], dtype, device, seed=5)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    assert prep.kernel_name == "panel"
    monkeypatch.setenv("FLAGSPARSE_PANEL_WG_CAP", "1")
    y_pipe = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    assert _lib.last_kernel() == "spmv_panel_pipe_kernel"
    assert torch.equal(y_pipe, fs.flagsparse_spmv_csr(x=x, prepared=prep))
    monkeypatch.delenv("FLAGSPARSE_PANEL_WG_CAP")
    assert torch.equal(y_pipe, fs.flagsparse_spmv_csr(x=x, prepared=prep))
    monkeypatch.setenv("FLAGSPARSE_PANEL_PIPE", "0")
    y_tile = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    assert _lib.last_kernel() == "spmv_panel_merge_kernel"
    assert torch.equal(y_pipe, y_tile)
    gen = np.random.default_rng(2)
    rows = sorted(set(gen.integers(0, sh[0], 2000).tolist()) | {0, sh[0] - 1})
    _sampled_rows_check(data, indices, indptr, sh, x, y_pipe, rows, REL_TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64], ids=["f32", "f64", "c64"])
def test_stream_t_misaligned_arrays_match(device, monkeypatch, dtype):
    """Value / index arrays that are not 16-byte aligned (views one element
    into a buffer) take K3t's register-staged path; aligned copies take the
    direct-to-LDS path; both give the same bits."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_SPMV_STREAM_T_DL"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "0")
    monkeypatch.setenv("FLAGSPARSE_SPMV_ONESHOT", "0")  # the unprepared call runs K3t itself
    data, indices, indptr, sh = S.stencil27(24, dtype, torch.int32, device, seed=9)
    x = S.vector(sh[1], dtype, device, seed=4)
    y = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh, return_meta=True)
    y, meta = y
    assert meta["kernel"] == "stream"
    dbuf = torch.empty(data.numel() + 1, dtype=dtype, device=device)
    ibuf = torch.empty(indices.numel() + 1, dtype=indices.dtype, device=device)
    dbuf[1:] = data
    ibuf[1:] = indices
    d_view, i_view = dbuf[1:], ibuf[1:]
    assert d_view.data_ptr() % 16 != 0 and i_view.data_ptr() % 16 != 0
    y_mis = fs.flagsparse_spmv_csr(d_view, i_view, indptr, x, sh)
    assert torch.equal(y, y_mis)
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), sh)
    assert rel_err(np_(y), ref) <= REL_TOL[dtype]


@pytest.mark.parametrize("per_row", [33, 48, 64])
@pytest.mark.parametrize("dtype", VALUE_DTYPES, ids=VALUE_IDS)
@pytest.mark.parametrize("index_dtype", INDEX_DTYPES, ids=INDEX_IDS)
def test_stream_t_eight_lanes_per_row(device, monkeypatch, per_row, dtype, index_dtype):
    """Rows of 33-64 entries (too long for four lanes per row in a 64-row
    block): K3t with eight lanes per row and 32-row blocks, against the oracle,
    and against the entry-order row-block kernel K3 within rounding."""
    for k in ("FLAGSPARSE_SPMV_SELL", "FLAGSPARSE_SPMV_KERNEL", "FLAGSPARSE_SPMV_STREAM_T_WIDE",
              "FLAGSPARSE_SPMV_STREAM_T"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "0")
    data, indices, indptr, sh = S.uniform_rows(3001, 2500, per_row, dtype, index_dtype, device, seed=per_row)
    x = S.vector(sh[1], dtype, device, seed=6)
    prep = fs.prepare_spmv_csr(data, indices, indptr, sh)
    y = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    if per_row * 32 <= (1024 if dtype.is_complex else 2048):
        assert _lib.last_kernel() == "spmv_stream_t_kernel"
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), sh)
    assert rel_err(np_(y), ref) <= REL_TOL[dtype]
    monkeypatch.setenv("FLAGSPARSE_SPMV_STREAM_T_WIDE", "0")
    y3 = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    assert rel_err(np_(y3), ref) <= REL_TOL[dtype]


@pytest.mark.parametrize("forced,expect", [
    ("vector", "spmv_vector_kernel"), ("merge", "spmv_merge_pipe_kernel"), ("stream", "spmv_stream_t_kernel"),
    ("nnzblock", "spmv_nnzblock_kernel"),
])
def test_last_kernel_names_the_launched_kernel(device, monkeypatch, forced, expect):
    """fs_last_kernel reports the kernel the launch itself chose (recorded
    at the launch in C, so the name cannot drift from the dispatch)."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", forced)
    monkeypatch.setenv("FLAGSPARSE_SPMV_SELL", "0")
    data, indices, indptr, sh = S.uniform_rows(2000, 2000, 8, torch.float32, torch.int32, device, seed=3)
    x = S.vector(sh[1], torch.float32, device, seed=4)
    fs.flagsparse_spmv_csr(data, indices, indptr, x, sh)
    assert _lib.last_kernel() == expect
    monkeypatch.delenv("FLAGSPARSE_SPMV_KERNEL")
    monkeypatch.delenv("FLAGSPARSE_SPMV_SELL")
    d2, i2, p2, sh2 = S.stencil27(64, torch.float64, torch.int32, device, seed=7)
    prep = fs.prepare_spmv_csr(d2, i2, p2, sh2)
    fs.flagsparse_spmv_csr(x=S.vector(sh2[1], torch.float64, device, seed=8), prepared=prep)
    assert _lib.last_kernel() == "spmv_sell_group_kernel"


@pytest.mark.parametrize("op", ["trans", "conj"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.complex64, torch.complex128],
                         ids=["float32", "float64", "complex64", "complex128"])
def test_spmv_transposed_one_sync_matches_prepared(device, dtype, op):
    """The unprepared A^T x / A^H x (check, transpose and one-launch SpMV
    queued back to back) against the prepared route on the same matrix,
    within the dtype's tolerance, and its meta kernel name."""
    d, i, p, sh = S.powerlaw(1 << 15, dtype, torch.int32, device, seed=31)
    x = S.vector(sh[0], dtype, device, seed=2)
    y = fs.flagsparse_spmv_csr(d, i, p, x, sh, op=op)
    prep = fs.prepare_spmv_csr(d, i, p, sh, op=op)
    ref = fs.flagsparse_spmv_csr(x=x, prepared=prep)
    tol = REL_TOL[dtype]
    err = ((y - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
    assert err <= tol, err
    # a wrong x length still raises the reference's error, after the checks
    with pytest.raises(ValueError, match="x length"):
        fs.flagsparse_spmv_csr(d, i, p, S.vector(sh[1] + 1, dtype, device, seed=2), sh, op=op)


@pytest.mark.parametrize("kernel", ["merge", "nnzblock"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.complex64], ids=["f32", "c64"])
def test_spmv_hub_rows_spanning_hundreds_of_tiles(device, monkeypatch, kernel, dtype):
    """Rows of 150,000 and 120,000 entries cross hundreds of tiles: the
    fix-up finds where each starts (a binary search over the partition) and
    adds its fragments in tile order."""
    monkeypatch.setenv("FLAGSPARSE_SPMV_KERNEL", kernel)
    data, indices, indptr, sh = S.random_csr(400, 200_000, 0.0005, dtype, torch.int32, device, seed=9,
                                             empty_row_every=11, long_rows=((7, 150_000), (200, 120_000)))
    x = S.vector(sh[1], dtype, device, seed=3)
    y = fs.flagsparse_spmv_csr(data, indices, indptr, x, sh)
    ref = O.spmv_csr_wide(np_(data), np_(indices), np_(indptr), np_(x), sh)
    assert rel_err(np_(y), ref) <= REL_TOL[dtype]
