"""CPU checks of bench.py's accuracy report (no GPU: tensors stay on the host)."""

import numpy as np
import pytest
import torch

import bench


def _small():
    # [[2, 0, 1], [0, 0, 0], [0, 3, 4]] in CSR
    d = np.array([2.0, 1.0, 3.0, 4.0], dtype=np.float32)
    i = np.array([0, 2, 1, 2], dtype=np.int32)
    p = np.array([0, 2, 2, 4], dtype=np.int64)
    return d, i, p, (3, 3)


def test_accuracy_exact_output_passes():
    d, i, p, sh = _small()
    x = np.array([1.0, 2.0, 3.0], dtype=np.float32)
    out = torch.tensor([5.0, 0.0, 18.0])
    acc = bench._accuracy(d, i, p, sh, x, out)
    assert acc["max_rel_err"] == 0.0 and acc["pass"] and acc["tolerance"] == 1e-5 and acc["rows"] == 3
    assert acc["allclose"] and acc["allclose_rtol_atol"] == [1e-5, 1e-6]


def test_accuracy_detects_a_wrong_row():
    d, i, p, sh = _small()
    x = np.array([1.0, 2.0, 3.0], dtype=np.float32)
    out = torch.tensor([5.0, 0.0, 18.5])  # |0.5| / max|y| = 0.5 / 18
    acc = bench._accuracy(d, i, p, sh, x, out)
    assert acc["max_rel_err"] == pytest.approx(0.5 / 18, rel=1e-3) and not acc["pass"]
    assert not acc["allclose"]


def test_accuracy_spmm_and_f64_tolerance():
    d, i, p, sh = _small()
    d = d.astype(np.float64)
    B = np.arange(6, dtype=np.float64).reshape(3, 2)  # rows [0,1], [2,3], [4,5]
    out = torch.tensor([[4.0, 7.0], [0.0, 0.0], [22.0, 29.0]], dtype=torch.float64)
    acc = bench._accuracy(d, i, p, sh, B, out)
    assert acc["max_rel_err"] == 0.0 and acc["tolerance"] == 1e-12


def test_strided_row_sample_spreads_over_all_rows():
    # 100 rows of lengths 0..99 (row r holds r entries with columns 0..r-1)
    lens = np.arange(100)
    p = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    i = np.concatenate([np.arange(n) for n in lens]).astype(np.int32)
    d = np.arange(p[-1], dtype=np.float64)
    rows, ds, is_, ps = bench.strided_row_sample(d, i, p, target_nnz=500)
    k = int(rows[1] - rows[0])
    assert k > 1 and np.array_equal(rows, np.arange(0, 100, k))
    assert ps[-1] >= 500 and rows[-1] >= 100 - k
    for j, r in enumerate(rows):  # each sampled row is the original row, same entries
        assert np.array_equal(ds[ps[j]:ps[j + 1]], d[p[r]:p[r + 1]])
        assert np.array_equal(is_[ps[j]:ps[j + 1]], i[p[r]:p[r + 1]])


def test_strided_row_sample_small_matrix_is_whole():
    d, i, p, sh = _small()
    rows, ds, is_, ps = bench.strided_row_sample(d, i, p, target_nnz=1e6)
    assert np.array_equal(rows, [0, 1, 2]) and np.array_equal(ps, p) and np.array_equal(ds, d)


def test_profile_traffic_reads_summary_and_flags_stale_kernel(tmp_path, monkeypatch):
    (tmp_path / "k_a.md").write_text("# kern_a — work1\n\n| total | | | 1,234.5 MB (12 % of algorithmic) |\n")
    monkeypatch.setattr(bench, "PROFILES_DIR", str(tmp_path))
    b, note = bench.profile_traffic("work1", "kern_a")
    assert b == 1234.5e6 and note.endswith("k_a.md")
    b, note = bench.profile_traffic("work1", "kern_b")
    assert b is None and "kern_a" in note
    b, note = bench.profile_traffic("work2", "kern_a")
    assert b is None
