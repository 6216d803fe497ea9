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
