"""MatrixMarket (.mtx) ingestion into CSR for SpMV / SpMM runs.

Follows the reference's loader, load_mtx_to_csr_torch
(tests/test_spmv.py:103-176):
  - `pattern` entries have value 1.0;
  - `symmetric` and `hermitian` mirror each off-diagonal entry (the
    reference mirrors hermitian entries without conjugating them);
  - `skew-symmetric` mirrors with the sign flipped;
  - duplicate (row, col) entries are summed in file order;
  - columns are sorted within each row.
Parsing is host-side (numpy); the CSR arrays are then moved to `device`.
Only the first three fields of a line are read, so complex files load
their real parts, as in the reference.
"""

import numpy as np
import torch


def _read(file_path):
    field, symmetry = "real", "general"
    header = None
    body = []
    with open(file_path, "r", encoding="utf-8") as f:
        for line in f:
            s = line.strip()
            if s.startswith("%%MatrixMarket"):
                tok = s.split()
                if len(tok) >= 5:
                    field, symmetry = tok[3].lower(), tok[4].lower()
                continue
            if s.startswith("%") or not s:
                continue
            if header is None:
                parts = s.split()
                header = (int(parts[0]), int(parts[1]), int(parts[2]) if len(parts) > 2 else 0)
                continue
            body.append(s)
    if header is None:
        raise ValueError(f"Cannot parse .mtx header: {file_path}")
    return field, symmetry, header, body


def mtx_to_coo(file_path):
    """Expanded COO (row, col, value float64) in the reference's insertion order."""
    field, symmetry, (n_rows, n_cols, nnz), body = _read(file_path)
    body = body[:nnz]
    if nnz == 0 or not body:
        empty = np.empty(0, dtype=np.int64)
        return empty, empty, np.empty(0, dtype=np.float64), (n_rows, n_cols)
    toks = [b.split() for b in body]
    r = np.array([int(t[0]) - 1 for t in toks], dtype=np.int64)
    c = np.array([int(t[1]) - 1 for t in toks], dtype=np.int64)
    if field == "pattern":
        v = np.ones(len(toks), dtype=np.float64)
    else:
        v = np.array([float(t[2]) for t in toks], dtype=np.float64)
    ok = (r >= 0) & (r < n_rows) & (c >= 0) & (c < n_cols)
    r, c, v = r[ok], c[ok], v[ok]
    mirror_sign = 0.0
    if symmetry in ("symmetric", "hermitian"):
        mirror_sign = 1.0
    elif symmetry == "skew-symmetric":
        mirror_sign = -1.0
    if mirror_sign != 0.0:
        m = (r != c) & (c < n_rows) & (r < n_cols)
        # interleave each entry with its mirror so duplicates sum in the
        # order the reference's dict accumulation sees them
        rows = np.stack([r, np.where(m, c, -1)], 1).reshape(-1)
        cols = np.stack([c, np.where(m, r, -1)], 1).reshape(-1)
        vals = np.stack([v, mirror_sign * v], 1).reshape(-1)
        keep = rows >= 0
        r, c, v = rows[keep], cols[keep], vals[keep]
    return r, c, v, (n_rows, n_cols)


def load_mtx_to_csr(file_path, dtype=torch.float32, device=None, index_dtype=torch.int64):
    """(data, indices, indptr, shape) with duplicates summed and sorted columns."""
    if device is None:
        device = torch.device("cuda" if torch.cuda.is_available() else "cpu")
    r, c, v, (n_rows, n_cols) = mtx_to_coo(file_path)
    indptr = np.zeros(n_rows + 1, dtype=np.int64)
    if r.size == 0:
        return (torch.empty(0, dtype=dtype, device=device), torch.empty(0, dtype=index_dtype, device=device),
                torch.from_numpy(indptr).to(index_dtype).to(device), (n_rows, n_cols))
    key = r * max(1, n_cols) + c
    order = np.argsort(key, kind="stable")
    key_s, v_s = key[order], v[order]
    starts = np.flatnonzero(np.r_[True, key_s[1:] != key_s[:-1]])
    sums = np.empty(starts.size, dtype=np.float64)
    bounds = np.r_[starts, key_s.size]
    for i in range(starts.size):  # sequential, file-order sums (0.0 + v1 + v2 + ...)
        acc = 0.0
        for val in v_s[bounds[i]:bounds[i + 1]]:
            acc = acc + float(val)
        sums[i] = acc
    uk = key_s[starts]
    rows, cols = uk // max(1, n_cols), uk % max(1, n_cols)
    indptr[1:] = np.cumsum(np.bincount(rows, minlength=n_rows))
    data = torch.tensor(sums, dtype=torch.float64).to(dtype)
    return (data.to(device), torch.from_numpy(cols).to(index_dtype).to(device),
            torch.from_numpy(indptr).to(index_dtype).to(device), (n_rows, n_cols))
