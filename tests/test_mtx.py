"""MatrixMarket ingestion matches a literal restatement of the reference's
loader (tests/test_spmv.py:103-176), bit for bit (CPU only)."""

import numpy as np
import pytest
import torch

from flagsparse_amd.mtx import load_mtx_to_csr
from oracle import csr_oracle as O


def _write(path, field, symmetry, shape, entries, comments=("% test",)):
    with open(path, "w") as f:
        f.write(f"%%MatrixMarket matrix coordinate {field} {symmetry}\n")
        for c in comments:
            f.write(c + "\n")
        f.write(f"{shape[0]} {shape[1]} {len(entries)}\n")
        for e in entries:
            f.write(" ".join(str(t) for t in e) + "\n")


CASES = {
    "general": ("real", "general", (5, 4), [(1, 1, 1.5), (3, 2, -2.0), (1, 1, 0.25), (5, 4, 3.0), (2, 4, 1e-3)]),
    "symmetric": ("real", "symmetric", (4, 4), [(1, 1, 2.0), (3, 1, -1.0), (4, 2, 0.5), (3, 1, 0.125)]),
    "skew": ("real", "skew-symmetric", (4, 4), [(2, 1, 1.0), (4, 3, -2.5), (4, 1, 7.0)]),
    "pattern": ("pattern", "general", (3, 6), [(1, 6), (3, 2), (1, 6), (2, 2)]),
    "pattern_sym": ("pattern", "symmetric", (4, 4), [(2, 1), (3, 3), (4, 1)]),
    "hermitian_as_sym": ("real", "hermitian", (3, 3), [(2, 1, 1.0), (3, 3, 4.0)]),
    "empty": ("real", "general", (3, 3), []),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_mtx_matches_reference_loader(tmp_path, name):
    field, sym, shape, entries = CASES[name]
    path = tmp_path / f"{name}.mtx"
    _write(path, field, sym, shape, entries)
    d, i, p, sh = load_mtx_to_csr(str(path), dtype=torch.float64, device="cpu")
    rd, ri, rp, rsh = O.load_mtx_reference(str(path))
    assert sh == rsh
    assert np.array_equal(p.numpy(), rp) and np.array_equal(i.numpy(), ri) and np.array_equal(d.numpy(), rd)


def test_mtx_random_large_with_duplicates(tmp_path):
    rng = np.random.default_rng(0)
    n = 300
    entries = [(int(a) + 1, int(b) + 1, float(v)) for a, b, v in
               zip(rng.integers(0, n, 3000), rng.integers(0, n, 3000), rng.uniform(-1, 1, 3000))]
    for sym in ("general", "symmetric", "skew-symmetric"):
        path = tmp_path / f"r_{sym}.mtx"
        _write(path, "real", sym, (n, n), entries)
        d, i, p, sh = load_mtx_to_csr(str(path), dtype=torch.float64, device="cpu")
        rd, ri, rp, rsh = O.load_mtx_reference(str(path))
        assert np.array_equal(p.numpy(), rp) and np.array_equal(i.numpy(), ri) and np.array_equal(d.numpy(), rd)


# Committed, hand-written files (tests/golden/mtx) and their matrices worked
# out by hand from the reference loader's rules (tests/test_spmv.py:103-176):
# duplicates summed, symmetric / skew-symmetric mirrored, pattern values 1.
GOLDEN_MTX = {
    "general": [[1.75, 0, 0, 0], [-0.5, 0, 0, 1e-3], [0, -2, 0, 0], [0, 0, 0, 0], [2, 0, 0, 3]],
    "symmetric": [[2, 0, -0.875, 0], [0, 0, 0, 0.5], [-0.875, 0, 0, 0], [0, 0.5, 0, -3]],
    "skew": [[0, -1, 0, -7], [1, 0, 0, 0], [0, 0, 0, 2.5], [7, 0, -2.5, 0]],
    "pattern": [[0, 0, 0, 0, 0, 2], [0, 1, 0, 0, 0, 0], [0, 1, 0, 0, 0, 0]],
    "pattern_symmetric": [[0, 1, 0, 1], [1, 0, 0, 0], [0, 0, 1, 0], [1, 0, 0, 0]],
}


def golden_mtx_path(name):
    import os

    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mtx", f"{name}.mtx")


@pytest.mark.parametrize("name", sorted(GOLDEN_MTX))
def test_mtx_golden_files_known_answers(name):
    d, i, p, sh = load_mtx_to_csr(golden_mtx_path(name), dtype=torch.float64, device="cpu")
    dense = O.to_dense(d.numpy(), i.numpy(), p.numpy(), sh)
    assert np.array_equal(dense, np.array(GOLDEN_MTX[name], dtype=np.float64))
    rd, ri, rp, rsh = O.load_mtx_reference(golden_mtx_path(name))
    assert sh == rsh and np.array_equal(p.numpy(), rp) and np.array_equal(i.numpy(), ri)
    assert np.array_equal(d.numpy(), rd)
