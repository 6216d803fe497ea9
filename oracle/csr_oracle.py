"""CPU oracle for FlagSparse's CSR SpMV / SpMM path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker / CPU baseline; the product
path (flagsparse_amd) never calls it.

It restates the reference algorithm in numpy:

  op codes                 spmv_csr.py:18-52, spmm_csr.py:11-45
  transpose (op=trans)     spmv_csr.py:477-515, spmm_csr.py:300-338:
                           row ids by repeat, STABLE argsort by column,
                           gather, bincount + cumsum; index dtype rules
                           spmv_csr.py:482-483, 508-509
  conj before transpose    spmv_csr.py:615-618, spmm_csr.py:341-349
  SpMV numerics            spmv_csr.py:124-130, 679-723: float32 is computed
                           in float64 and rounded once; float64 / complex
                           in their own precision (complex64 here in
                           complex128, the more accurate of the two)
  SpMM numerics            spmm_csr.py:2684-2789 (same dtype policy)
  empty cases              spmm_csr.py:2706-2710 (zeros)
  COO -> CSR               spmv_csr.py:926-950 (key row * n_cols + col)
  COO SpMV / SpMM          spmv_coo.py:425-644, spmm_coo.py:101-142, 696-723
                           (duplicates summed; trans / conj swap row and col)

Pinning (tests/test_oracle.py): every function is checked against dense
brute force on small inputs, scipy's independent CSR->CSC conversion and
CSR matvec, closed forms (identity, diagonal, all-ones stencil row sums),
double-transpose idempotence, linearity and a hand-computed example, and
against the committed fixtures in tests/golden/.
"""

import numpy as np

INDEX_LIMIT_INT32 = 2**31 - 1

OP_NON, OP_TRANS, OP_CONJ = 0, 1, 2
_OP_NAMES = {"non": OP_NON, "trans": OP_TRANS, "conj": OP_CONJ}


def normalize_op(op=None, transpose=False):
    """spmv_csr.py:29-43: None -> trans if transpose else non."""
    if op is None:
        return OP_TRANS if transpose else OP_NON
    if isinstance(op, str):
        key = op.strip().lower()
        if key not in _OP_NAMES:
            raise ValueError("op must be one of: 0=non, 1=trans, 2=conj")
        return _OP_NAMES[key]
    code = int(op)
    if code not in (OP_NON, OP_TRANS, OP_CONJ):
        raise ValueError("op must be one of: 0=non, 1=trans, 2=conj")
    return code


def accumulate_dtype(dtype):
    dtype = np.dtype(dtype)
    if dtype.kind == "c":
        return np.complex128
    return np.float64


def transpose_out_dtypes(index_dtype, indptr_dtype, n_rows, nnz):
    """spmv_csr.py:482-483, 508-509."""
    out_index = np.dtype(index_dtype) if n_rows <= INDEX_LIMIT_INT32 else np.dtype(np.int64)
    out_indptr = np.dtype(indptr_dtype) if nnz <= INDEX_LIMIT_INT32 else np.dtype(np.int64)
    return out_index, out_indptr


def transpose_csr(data, indices, indptr, shape, conj=False):
    """CSR of A^T (A^H if conj and complex), stable by column.

    Follows spmv_csr.py:477-515: row ids are repeated per row, entries are
    ordered by a stable argsort of the column index, the new row pointer
    is bincount + cumsum over the columns.
    """
    n_rows, n_cols = int(shape[0]), int(shape[1])
    data = np.asarray(data)
    indices = np.asarray(indices)
    indptr = np.asarray(indptr)
    nnz = data.shape[0]
    out_index, out_indptr = transpose_out_dtypes(indices.dtype, indptr.dtype, n_rows, nnz)
    if conj and np.iscomplexobj(data):
        data = np.conj(data)
    if nnz == 0:
        return data.copy(), np.empty(0, dtype=out_index), np.zeros(n_cols + 1, dtype=out_indptr), (n_cols, n_rows)
    counts = np.diff(indptr.astype(np.int64))
    row_ids = np.repeat(np.arange(n_rows, dtype=np.int64), counts)
    cols = indices.astype(np.int64)
    order = np.argsort(cols, kind="stable")
    t_data = data[order]
    t_indices = row_ids[order].astype(out_index)
    t_indptr = np.zeros(n_cols + 1, dtype=np.int64)
    t_indptr[1:] = np.cumsum(np.bincount(cols, minlength=n_cols))
    return t_data, t_indices, t_indptr.astype(out_indptr), (n_cols, n_rows)


def materialize_op(data, indices, indptr, shape, op):
    code = normalize_op(op)
    if code == OP_NON:
        return np.asarray(data), np.asarray(indices), np.asarray(indptr), (int(shape[0]), int(shape[1]))
    return transpose_csr(data, indices, indptr, shape, conj=(code == OP_CONJ))


def _row_dot_products(data, indices, indptr, X, n_rows):
    """Sum_j A[i, j] * X[j, ...] per row, accumulated in the wide dtype.

    Vectorised segment sums (np.add.reduceat in CSR order); empty rows
    give zero.
    """
    indptr = np.asarray(indptr).astype(np.int64)
    acc = accumulate_dtype(data.dtype)
    d = np.asarray(data).astype(acc)
    Xw = np.asarray(X).astype(acc)
    prod = d.reshape((-1,) + (1,) * (Xw.ndim - 1)) * Xw[np.asarray(indices).astype(np.int64)]
    out = np.zeros((n_rows,) + Xw.shape[1:], dtype=acc)
    if prod.shape[0] == 0 or n_rows == 0:
        return out
    lengths = np.diff(indptr)
    nonempty = lengths > 0
    starts = indptr[:-1][nonempty]
    sums = np.add.reduceat(prod, starts, axis=0)
    out[nonempty] = sums
    return out


def spmv_csr(data, indices, indptr, x, shape, op=None):
    """y = op(A) @ x in the reference's precision policy, cast to data's dtype."""
    data = np.asarray(data)
    d, i, p, sh = materialize_op(data, indices, indptr, shape, op)
    y = _row_dot_products(d, i, p, np.asarray(x), sh[0])
    return y.astype(data.dtype)


def spmv_csr_wide(data, indices, indptr, x, shape, op=None):
    """Like spmv_csr but returns the wide (float64 / complex128) result."""
    d, i, p, sh = materialize_op(np.asarray(data), indices, indptr, shape, op)
    return _row_dot_products(d, i, p, np.asarray(x), sh[0])


def spmm_csr(data, indices, indptr, B, shape, op=None):
    """C = op(A) @ B, cast to data's dtype (zeros for empty cases)."""
    data = np.asarray(data)
    B = np.asarray(B)
    d, i, p, sh = materialize_op(data, indices, indptr, shape, op)
    if sh[0] == 0 or B.shape[1] == 0:
        return np.zeros((sh[0], B.shape[1]), dtype=data.dtype)
    C = _row_dot_products(d, i, p, B, sh[0])
    return C.astype(data.dtype)


def spmm_csr_wide(data, indices, indptr, B, shape, op=None):
    d, i, p, sh = materialize_op(np.asarray(data), indices, indptr, shape, op)
    if sh[0] == 0 or np.asarray(B).shape[1] == 0:
        return np.zeros((sh[0], np.asarray(B).shape[1]), dtype=accumulate_dtype(np.asarray(data).dtype))
    return _row_dot_products(d, i, p, np.asarray(B), sh[0])


def to_dense(data, indices, indptr, shape):
    """Dense matrix (duplicates summed) for brute-force checks."""
    n_rows, n_cols = int(shape[0]), int(shape[1])
    data = np.asarray(data)
    dense = np.zeros((n_rows, n_cols), dtype=accumulate_dtype(data.dtype))
    indptr = np.asarray(indptr).astype(np.int64)
    for r in range(n_rows):
        for k in range(indptr[r], indptr[r + 1]):
            dense[r, int(indices[k])] += data[k]
    return dense


def relative_error(candidate, reference):
    """max|c - r| / max|r| (the reference's normwise metric, spmm_csr.py:95-103).

    Complex inputs use the element magnitude of the difference (stricter
    than the reference, which compares magnitudes)."""
    c = np.asarray(candidate).astype(np.complex128 if np.iscomplexobj(candidate) else np.float64)
    r = np.asarray(reference).astype(c.dtype)
    if r.size == 0:
        return 0.0
    num = np.max(np.abs(c - r))
    den = np.max(np.abs(r))
    if den == 0:
        return 0.0 if num == 0 else float("inf")
    return float(num / den)


def coo_to_csr(data, row, col, shape):
    """COO -> (data, int32 cols, int64 indptr), spmv_csr.py:926-950.

    Entries ordered by the key row * n_cols + col.  The reference sorts with
    a non-stable argsort (duplicate order unspecified); this restatement uses
    a stable sort, which is the order the HIP path produces."""
    n_rows, n_cols = int(shape[0]), int(shape[1])
    data = np.asarray(data)
    row = np.asarray(row).astype(np.int64)
    col = np.asarray(col).astype(np.int64)
    indptr = np.zeros(n_rows + 1, dtype=np.int64)
    if row.size == 0:
        return data.copy(), col.astype(np.int32), indptr
    key = row * max(1, n_cols) + col
    order = np.argsort(key, kind="stable")
    indptr[1:] = np.cumsum(np.bincount(row[order], minlength=n_rows))
    return data[order], col[order].astype(np.int32), indptr


def spmv_coo(data, row, col, x, shape, op=None):
    """COO SpMV y = op(A) x in the wide accumulator type (spmv_coo.py:425-644).

    A is the COO with duplicate (row, col) entries summed; op=trans / conj
    work on (col, row) with the data conjugated for conj (spmv_coo.py:525-554).
    Restated as: sort to CSR (coo_to_csr), then spmv_csr_wide."""
    code = normalize_op(op)
    n_rows, n_cols = int(shape[0]), int(shape[1])
    data = np.asarray(data)
    if code != 0:
        if code == 2 and np.iscomplexobj(data):
            data = np.conj(data)
        row, col, n_rows, n_cols = col, row, n_cols, n_rows
    d, c, p = coo_to_csr(data, row, col, (n_rows, n_cols))
    return spmv_csr_wide(d, c, p, x, (n_rows, n_cols))


def spmm_coo(data, row, col, B, shape):
    """COO SpMM C = A B in the wide accumulator type (spmm_coo.py:101-142,
    696-723: duplicates coalesced by summation, then the row-run product)."""
    d, c, p = coo_to_csr(data, row, col, shape)
    return spmm_csr_wide(d, c, p, B, shape)


def load_mtx_reference(file_path):
    """Literal restatement of the reference's loader (tests/test_spmv.py:103-176):
    per-row dicts accumulated in file order, sorted columns.  Returns float64
    data, int64 indices / indptr and the shape."""
    with open(file_path, "r", encoding="utf-8") as f:
        lines = f.readlines()
    field, symmetry = "real", "general"
    data_lines, header = [], None
    for line in lines:
        s = line.strip()
        if s.startswith("%%MatrixMarket"):
            tok = s.split()
            if len(tok) >= 5:
                field, symmetry = tok[3].lower(), tok[4].lower()
            continue
        if s.startswith("%"):
            continue
        if not header and s:
            p = s.split()
            header = (int(p[0]), int(p[1]), int(p[2]) if len(p) > 2 else 0)
            continue
        if s:
            data_lines.append(s)
    n_rows, n_cols, nnz = header
    if nnz == 0:
        return np.empty(0), np.empty(0, dtype=np.int64), np.zeros(n_rows + 1, dtype=np.int64), (n_rows, n_cols)
    pattern = field == "pattern"
    sym = symmetry in ("symmetric", "hermitian")
    skew = symmetry == "skew-symmetric"
    rows = [dict() for _ in range(n_rows)]
    for line in data_lines[:nnz]:
        p = line.split()
        r, c = int(p[0]) - 1, int(p[1]) - 1
        v = 1.0 if pattern else float(p[2])
        if 0 <= r < n_rows and 0 <= c < n_cols:
            rows[r][c] = rows[r].get(c, 0.0) + v
            if r != c:
                if sym and 0 <= c < n_rows and 0 <= r < n_cols:
                    rows[c][r] = rows[c].get(r, 0.0) + v
                elif skew and 0 <= c < n_rows and 0 <= r < n_cols:
                    rows[c][r] = rows[c].get(r, 0.0) - v
    cols, vals, indptr = [], [], [0]
    for row in rows:
        for c in sorted(row):
            cols.append(c)
            vals.append(row[c])
        indptr.append(len(cols))
    return np.array(vals, dtype=np.float64), np.array(cols, dtype=np.int64), np.array(indptr, dtype=np.int64), (n_rows, n_cols)
