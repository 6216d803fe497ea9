"""Pins the CPU oracle (oracle/csr_oracle.py) — runs on CPU only.

The reference ships no golden vectors for this path (its .mtx files are
absent and its accuracy tests are randomized against torch dense results),
so every oracle function is pinned here against things that do not share
its code: dense brute force, scipy's independent CSR->CSC conversion and
CSR matvec, closed forms, a hand-computed example, and invariants chosen so
a dropped term, wrong sign / conjugation, or transposed operand fails.
"""

import glob
import os

import numpy as np
import pytest
import scipy.sparse as sp

from oracle import csr_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _rand_csr(rng, m, n, density, dtype, index_dtype=np.int32, long_row=None):
    A = sp.random(m, n, density=density, format="csr", random_state=rng, dtype=np.float64)
    if long_row is not None:
        A = A.tolil()
        r, ln = long_row
        A[r, :ln] = rng.uniform(-1, 1, ln)
        A = A.tocsr()
    A.sort_indices()
    data = A.data.astype(np.float64)
    if np.dtype(dtype).kind == "c":
        data = data + 1j * rng.uniform(-1, 1, data.shape[0])
    return data.astype(dtype), A.indices.astype(index_dtype), A.indptr.astype(index_dtype), (m, n)


def test_hand_computed_example():
    # A = [[1, 0, 2],
    #      [0, 0, 0],
    #      [3, 4, 0]]    x = [1, 10, 100]
    data = np.array([1.0, 2.0, 3.0, 4.0])
    indices = np.array([0, 2, 0, 1], dtype=np.int32)
    indptr = np.array([0, 2, 2, 4], dtype=np.int32)
    x = np.array([1.0, 10.0, 100.0])
    assert np.array_equal(O.spmv_csr(data, indices, indptr, x, (3, 3)), [201.0, 0.0, 43.0])
    # A^T x = [1*1 + 3*100, 4*100, 2*1]
    assert np.array_equal(O.spmv_csr(data, indices, indptr, x, (3, 3), op="trans"), [301.0, 400.0, 2.0])
    td, ti, tp, tsh = O.transpose_csr(data, indices, indptr, (3, 3))
    assert tsh == (3, 3)
    assert np.array_equal(tp, [0, 2, 3, 4]) and np.array_equal(ti, [0, 2, 2, 0]) and np.array_equal(td, [1, 3, 4, 2])
    B = np.array([[1.0, 2.0], [10.0, 20.0], [100.0, 200.0]])
    assert np.array_equal(O.spmm_csr(data, indices, indptr, B, (3, 3)), [[201, 402], [0, 0], [43, 86]])


def test_complex_conj_hand_example():
    # A = [[1+2j, 3j]], conj(A)^T x for x = [2]  ->  [(1-2j)*2, (-3j)*2]
    data = np.array([1 + 2j, 3j], dtype=np.complex128)
    indices = np.array([0, 1], dtype=np.int64)
    indptr = np.array([0, 2], dtype=np.int64)
    x = np.array([2 + 0j])
    assert np.array_equal(O.spmv_csr(data, indices, indptr, x, (1, 2), op="conj"), [2 - 4j, -6j])
    assert np.array_equal(O.spmv_csr(data, indices, indptr, x, (1, 2), op="trans"), [2 + 4j, 6j])


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.complex64, np.complex128])
@pytest.mark.parametrize("op", ["non", "trans", "conj"])
def test_spmv_spmm_vs_dense_brute_force(dtype, op):
    rng = np.random.default_rng(1)
    data, idx, ptr, sh = _rand_csr(rng, 37, 23, 0.2, dtype, long_row=(5, 20))
    dense = O.to_dense(data, idx, ptr, sh)
    mat = {"non": dense, "trans": dense.T, "conj": dense.conj().T}[op]
    x = rng.uniform(-1, 1, mat.shape[1]).astype(np.float64)
    B = rng.uniform(-1, 1, (mat.shape[1], 5))
    if np.dtype(dtype).kind == "c":
        x = x + 1j * rng.uniform(-1, 1, x.shape)
        B = B + 1j * rng.uniform(-1, 1, B.shape)
    x = x.astype(dtype)
    B = B.astype(dtype)
    y = O.spmv_csr_wide(data, idx, ptr, x, sh, op=op)
    y_ref = mat @ x.astype(mat.dtype)
    assert np.max(np.abs(y - y_ref)) <= 1e-13 * max(1.0, np.max(np.abs(y_ref)))
    C = O.spmm_csr_wide(data, idx, ptr, B, sh, op=op)
    C_ref = mat @ B.astype(mat.dtype)
    assert np.max(np.abs(C - C_ref)) <= 1e-13 * max(1.0, np.max(np.abs(C_ref)))
    # the narrow result is the wide one rounded once
    assert np.array_equal(O.spmv_csr(data, idx, ptr, x, sh, op=op), y.astype(dtype))


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_transpose_vs_scipy_tocsc(index_dtype):
    rng = np.random.default_rng(2)
    data, idx, ptr, sh = _rand_csr(rng, 300, 211, 0.05, np.float64, index_dtype)
    td, ti, tp, tsh = O.transpose_csr(data, idx, ptr, sh)
    csc = sp.csr_matrix((data, idx, ptr), shape=sh).tocsc()
    assert tsh == (211, 300)
    assert np.array_equal(tp, csc.indptr) and np.array_equal(ti, csc.indices) and np.array_equal(td, csc.data)
    assert ti.dtype == np.dtype(index_dtype) and tp.dtype == np.dtype(index_dtype)


def test_transpose_stable_with_duplicates_and_unsorted_columns():
    # rows hold repeated / unsorted columns: a stable sort keeps CSR order
    data = np.arange(1.0, 8.0)
    idx = np.array([3, 1, 3, 0, 1, 1, 3], dtype=np.int32)
    ptr = np.array([0, 4, 4, 7], dtype=np.int32)
    td, ti, tp, _ = O.transpose_csr(data, idx, ptr, (3, 4))
    assert np.array_equal(tp, [0, 1, 4, 4, 7])
    # col 0: (row0, 4.0); col 1: (row0, 2.0), (row2, 5.0), (row2, 6.0); col 3: (row0, 1.0), (row0, 3.0), (row2, 7.0)
    assert np.array_equal(ti, [0, 0, 2, 2, 0, 0, 2])
    assert np.array_equal(td, [4.0, 2.0, 5.0, 6.0, 1.0, 3.0, 7.0])


def test_transpose_double_is_identity_and_dtype_rules():
    rng = np.random.default_rng(3)
    data, idx, ptr, sh = _rand_csr(rng, 64, 99, 0.1, np.complex64)
    t = O.transpose_csr(data, idx, ptr, sh, conj=True)
    back = O.transpose_csr(*t, conj=True)
    assert back[3] == sh
    assert np.array_equal(back[2], ptr) and np.array_equal(back[1], idx) and np.array_equal(back[0], data)
    # output index dtype widens only past int32 (spmv_csr.py:508-509)
    assert O.transpose_out_dtypes(np.int32, np.int32, 2**31 - 1, 5) == (np.dtype(np.int32), np.dtype(np.int32))
    assert O.transpose_out_dtypes(np.int32, np.int32, 2**31, 2**31) == (np.dtype(np.int64), np.dtype(np.int64))


def test_closed_forms():
    n = 50
    eye = sp.identity(n, format="csr")
    x = np.linspace(-1, 1, n)
    assert np.array_equal(O.spmv_csr(eye.data, eye.indices, eye.indptr, x, (n, n)), x)
    diag = sp.diags(np.arange(1.0, n + 1), format="csr")
    assert np.array_equal(O.spmv_csr(diag.data, diag.indices, diag.indptr, x, (n, n), op="trans"), x * np.arange(1, n + 1))
    # 27-point stencil of ones on a k^3 grid: y = A 1 = neighbour counts
    k = 5
    one = np.ones(k)
    T = sp.diags([1.0, 1.0, 1.0], [-1, 0, 1], shape=(k, k)).tocsr()
    T.eliminate_zeros()
    counts1 = T.toarray() @ one
    A = sp.kron(sp.kron(T, T), T).tocsr()
    A.eliminate_zeros()
    A.sort_indices()
    y = O.spmv_csr(A.data.astype(np.float64), A.indices, A.indptr, np.ones(k**3), A.shape)
    assert np.array_equal(y, np.kron(np.kron(counts1, counts1), counts1))
    assert A.nnz == (3 * k - 2) ** 3


def test_empty_cases():
    d = np.empty(0, dtype=np.float32)
    i = np.empty(0, dtype=np.int32)
    p = np.zeros(4, dtype=np.int32)
    assert np.array_equal(O.spmv_csr(d, i, p, np.ones(5, np.float32), (3, 5)), np.zeros(3, np.float32))
    assert O.spmm_csr(d, i, p, np.ones((5, 0), np.float32), (3, 5)).shape == (3, 0)
    td, ti, tp, tsh = O.transpose_csr(d, i, p, (3, 5))
    assert tsh == (5, 3) and np.array_equal(tp, np.zeros(6)) and ti.size == 0


def test_linearity():
    rng = np.random.default_rng(4)
    data, idx, ptr, sh = _rand_csr(rng, 80, 70, 0.1, np.float64)
    x1, x2 = rng.uniform(-1, 1, 70), rng.uniform(-1, 1, 70)
    y = O.spmv_csr(data, idx, ptr, 2 * x1 - 3 * x2, sh)
    y2 = 2 * O.spmv_csr(data, idx, ptr, x1, sh) - 3 * O.spmv_csr(data, idx, ptr, x2, sh)
    assert np.max(np.abs(y - y2)) < 1e-13


def test_op_normalisation_table():
    assert O.normalize_op(None) == 0 and O.normalize_op(None, transpose=True) == 1
    assert [O.normalize_op(v) for v in ("non", " TRANS ", "conj", 0, 1, 2)] == [0, 1, 2, 0, 1, 2]
    assert O.normalize_op("Conj") == 2
    with pytest.raises(ValueError):
        O.normalize_op("bad")
    with pytest.raises(ValueError):
        O.normalize_op(3)


def test_golden_fixtures_reproduce():
    files = sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))
    assert len(files) >= 8
    for f in files:
        z = np.load(f, allow_pickle=False)
        shape = tuple(int(v) for v in z["shape"])
        op = str(z["op"])
        if "y_wide" in z:
            y = O.spmv_csr_wide(z["data"], z["indices"], z["indptr"], z["x"], shape, op=op)
            assert np.array_equal(y, z["y_wide"]), f
        if "C_wide" in z:
            C = O.spmm_csr_wide(z["data"], z["indices"], z["indptr"], z["B"], shape, op=op)
            assert np.array_equal(C, z["C_wide"]), f
        if "t_indptr" in z:
            td, ti, tp, _ = O.transpose_csr(z["data"], z["indices"], z["indptr"], shape, conj=(op == "conj"))
            assert np.array_equal(tp, z["t_indptr"]) and np.array_equal(ti, z["t_indices"])
            assert np.array_equal(td, z["t_data"])


def test_coo_to_csr_vs_scipy_and_stability():
    rng = np.random.default_rng(5)
    n_rows, n_cols, nnz = 50, 40, 300
    flat = rng.choice(n_rows * n_cols, nnz, replace=False)
    row, col = flat // n_cols, flat % n_cols
    data = rng.uniform(-1, 1, nnz)
    d, c, p = O.coo_to_csr(data, row, col, (n_rows, n_cols))
    ref = sp.coo_matrix((data, (row, col)), shape=(n_rows, n_cols)).tocsr()
    ref.sort_indices()
    assert c.dtype == np.int32 and p.dtype == np.int64
    assert np.array_equal(p, ref.indptr) and np.array_equal(c, ref.indices) and np.array_equal(d, ref.data)
    # duplicates keep input order; already-sorted input is unchanged
    row = np.array([1, 0, 1, 1]); col = np.array([2, 3, 2, 0]); data = np.array([10.0, 20.0, 30.0, 40.0])
    d, c, p = O.coo_to_csr(data, row, col, (2, 4))
    assert np.array_equal(d, [20.0, 40.0, 10.0, 30.0]) and np.array_equal(c, [3, 0, 2, 2]) and np.array_equal(p, [0, 1, 4])
    d2, c2, p2 = O.coo_to_csr(d, np.array([0, 1, 1, 1]), c, (2, 4))
    assert np.array_equal(d2, d) and np.array_equal(c2, c)


def _dense_from_coo(data, row, col, shape):
    D = np.zeros(shape, dtype=np.result_type(data.dtype, np.float64))
    np.add.at(D, (row, col), data)  # duplicates summed
    return D


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.complex64, np.complex128])
@pytest.mark.parametrize("op", ["non", "trans", "conj"])
def test_spmv_coo_vs_dense_with_duplicates(dtype, op):
    rng = np.random.default_rng(11)
    m, n, nnz = 23, 17, 150  # dense enough that duplicates occur
    row = rng.integers(0, m, nnz)
    col = rng.integers(0, n, nnz)
    data = rng.uniform(-1, 1, nnz)
    if np.dtype(dtype).kind == "c":
        data = data + 1j * rng.uniform(-1, 1, nnz)
    data = data.astype(dtype)
    D = _dense_from_coo(data, row, col, (m, n))
    A = {"non": D, "trans": D.T, "conj": D.conj().T}[op]
    x = rng.uniform(-1, 1, A.shape[1]).astype(dtype)
    y = O.spmv_coo(data, row, col, x, (m, n), op=op)
    assert y.shape == (A.shape[0],)
    assert O.relative_error(y, A @ x.astype(A.dtype)) < 1e-12
    if np.dtype(dtype).kind == "c" and op != "non":
        # trans and conj differ on complex data: a dropped conjugation fails here
        other = O.spmv_coo(data, row, col, x, (m, n), op="trans" if op == "conj" else "conj")
        assert O.relative_error(other, y) > 1e-3


def test_spmv_coo_hand_example():
    # A = [[1, 0, 2], [0, 0, 0]] with the (0, 2) entry given as 0.5 + 1.5 (a duplicate)
    data = np.array([0.5, 1.0, 1.5]); row = np.array([0, 0, 0]); col = np.array([2, 0, 2])
    x = np.array([10.0, 20.0, 30.0])
    assert np.array_equal(O.spmv_coo(data, row, col, x, (2, 3)), [70.0, 0.0])
    assert np.array_equal(O.spmv_coo(data, row, col, np.array([3.0, 5.0]), (2, 3), op="trans"), [3.0, 0.0, 6.0])


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.complex64, np.complex128])
def test_spmm_coo_vs_dense_with_duplicates(dtype):
    rng = np.random.default_rng(12)
    m, k, n, nnz = 19, 13, 7, 120
    row = rng.integers(0, m, nnz)
    col = rng.integers(0, k, nnz)
    data = rng.uniform(-1, 1, nnz)
    B = rng.uniform(-1, 1, (k, n))
    if np.dtype(dtype).kind == "c":
        data = data + 1j * rng.uniform(-1, 1, nnz)
        B = B + 1j * rng.uniform(-1, 1, (k, n))
    data, B = data.astype(dtype), B.astype(dtype)
    D = _dense_from_coo(data, row, col, (m, k))
    C = O.spmm_coo(data, row, col, B, (m, k))
    assert C.shape == (m, n)
    assert O.relative_error(C, D @ B.astype(D.dtype)) < 1e-12
    # homogeneity in B (scaling by 2 is exact in binary floating point)
    assert O.relative_error(O.spmm_coo(data, row, col, 2 * B, (m, k)), 2 * C) < 1e-15
