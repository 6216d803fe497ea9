"""Writes the golden fixtures in this directory (run from the repo root:
`python tests/golden/make_golden.py`).

Inputs come from a fixed numpy PCG64 seed; expected outputs come from the
CPU oracle after it has been checked, case by case, against dense brute
force (SpMV / SpMM) and scipy's CSR->CSC conversion (transpose).  The
fixtures are data only: CSR arrays, x / B, and the expected results.
"""

import os
import sys

import numpy as np
import scipy.sparse as sp

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import csr_oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def make_matrix(rng, m, n, density, dtype, index_dtype, long_row=None, empty_every=0):
    A = sp.random(m, n, density=density, format="lil", random_state=rng, dtype=np.float64)
    if long_row is not None:
        r, ln = long_row
        A[r, :] = 0
        cols = np.sort(rng.choice(n, ln, replace=False))
        A[r, cols] = rng.uniform(-1, 1, ln)
    if empty_every:
        for r in range(0, m, empty_every):
            A[r, :] = 0
    A = A.tocsr()
    A.sort_indices()
    data = A.data
    if np.dtype(dtype).kind == "c":
        data = data + 1j * rng.uniform(-1, 1, data.shape[0])
    return data.astype(dtype), A.indices.astype(index_dtype), A.indptr.astype(index_dtype), (m, n)


def vec(rng, shape, dtype):
    v = rng.uniform(-1, 1, shape)
    if np.dtype(dtype).kind == "c":
        v = v + 1j * rng.uniform(-1, 1, shape)
    return v.astype(dtype)


def check_against_brute_force(data, idx, ptr, sh, op, y_or_C, rhs):
    dense = O.to_dense(data, idx, ptr, sh)
    mat = {"non": dense, "trans": dense.T, "conj": dense.conj().T}[op]
    ref = mat @ rhs.astype(mat.dtype)
    err = np.max(np.abs(y_or_C - ref)) if ref.size else 0.0
    assert err <= 1e-12 * max(1.0, float(np.max(np.abs(ref))) if ref.size else 1.0), err


def main():
    rng = np.random.default_rng(np.random.PCG64(20260101))
    dtypes = {"f32": np.float32, "f64": np.float64, "c64": np.complex64, "c128": np.complex128}
    count = 0
    for tname, dt in dtypes.items():
        for iname, it in (("i32", np.int32), ("i64", np.int64)):
            for op in ("non", "trans", "conj"):
                long_row = (5, 1500) if (tname == "f64" and iname == "i32") else (5, 120)
                data, idx, ptr, sh = make_matrix(rng, 48, 1600 if long_row[1] > 1000 else 200, 0.02, dt, it,
                                                 long_row=long_row, empty_every=11)
                n_in = sh[0] if op != "non" else sh[1]
                x = vec(rng, n_in, dt)
                y = O.spmv_csr_wide(data, idx, ptr, x, sh, op=op)
                check_against_brute_force(data, idx, ptr, sh, op, y, x)
                extra = {}
                if op != "non":
                    td, ti, tp, _ = O.transpose_csr(data, idx, ptr, sh, conj=(op == "conj"))
                    csc = sp.csr_matrix((data, idx, ptr), shape=sh).tocsc()
                    assert np.array_equal(tp, csc.indptr) and np.array_equal(ti, csc.indices)
                    assert np.array_equal(td, np.conj(csc.data) if op == "conj" else csc.data)
                    extra = {"t_data": td, "t_indices": ti, "t_indptr": tp}
                np.savez_compressed(os.path.join(OUT, f"spmv_{tname}_{iname}_{op}.npz"), data=data, indices=idx,
                                    indptr=ptr, x=x, shape=np.array(sh), op=np.array(op), y_wide=y, **extra)
                count += 1
    for tname, dt in dtypes.items():
        for op, n_dense in (("non", 5), ("trans", 64), ("conj", 33)):
            data, idx, ptr, sh = make_matrix(rng, 40, 60, 0.08, dt, np.int32, long_row=(3, 50), empty_every=7)
            B = vec(rng, (sh[0] if op != "non" else sh[1], n_dense), dt)
            C = O.spmm_csr_wide(data, idx, ptr, B, sh, op=op)
            check_against_brute_force(data, idx, ptr, sh, op, C, B)
            np.savez_compressed(os.path.join(OUT, f"spmm_{tname}_{op}.npz"), data=data, indices=idx, indptr=ptr,
                                B=B, shape=np.array(sh), op=np.array(op), C_wide=C)
            count += 1
    print(f"wrote {count} fixtures to {OUT}")


if __name__ == "__main__":
    main()
