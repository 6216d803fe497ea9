"""The gather-floor diagnostic (fs_diag_gather_rows): it must really load
every row it is given, so its checksum is the XOR of all gathered words."""

import numpy as np
import pytest
import torch

from flagsparse_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("row_bytes", [4, 8, 16, 64, 256, 1024])
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64], ids=["i32", "i64"])
def test_gather_rows_checksum(device, row_bytes, idx_dtype):
    g = torch.Generator(device="cpu").manual_seed(row_bytes)
    n_rows = 5000
    words = row_bytes // 4
    B = torch.randint(0, 2**31 - 1, (n_rows, words), generator=g, dtype=torch.int32)
    group = 64 // (row_bytes // 16) if row_bytes >= 16 else 64
    n_idx = 8 * group * 37  # whole batches: no index is repeated past the end
    idx = torch.randint(0, n_rows, (n_idx,), generator=g, dtype=torch.int64)
    expect = np.bitwise_xor.reduce(B[idx].numpy().view(np.uint32).reshape(-1))
    Bd, idxd = B.to(device), idx.to(idx_dtype).to(device)
    chk = torch.zeros(1, dtype=torch.int32, device=device)
    rc = _lib.diag_lib().fs_diag_gather_rows(_lib.index_code(idx_dtype), _lib.ptr(Bd), n_rows, row_bytes,
                                             _lib.ptr(idxd), n_idx, _lib.ptr(chk), _lib.stream_handle(device))
    assert rc == 0, _lib.diag_lib().fs_last_error()
    torch.cuda.synchronize()
    assert int(chk.cpu().numpy().view(np.uint32)[0]) == int(expect)


def test_gather_rows_rejects_bad_row_bytes(device):
    B = torch.zeros(4, 8, dtype=torch.int32, device=device)
    idx = torch.zeros(4, dtype=torch.int32, device=device)
    chk = torch.zeros(1, dtype=torch.int32, device=device)
    rc = _lib.diag_lib().fs_diag_gather_rows(_lib.index_code(torch.int32), _lib.ptr(B), 4, 12, _lib.ptr(idx), 4,
                                        _lib.ptr(chk), _lib.stream_handle(device))
    assert rc != 0
    assert b"row_bytes" in _lib.diag_lib().fs_last_error()


def test_gather_rows_clamps_stray_indices(device):
    """Indices outside [0, n_b_rows) read the nearest row of B, never past it."""
    B = torch.arange(8 * 4, dtype=torch.int32).reshape(8, 4)
    idx = torch.tensor([-5, 3, 8, 1 << 30] * 16 * 8, dtype=torch.int64)  # whole batches of 64 rows
    clamped = idx.clamp(0, 7)
    expect = np.bitwise_xor.reduce(B[clamped].numpy().view(np.uint32).reshape(-1))
    Bd, idxd = B.to(device), idx.to(device)
    chk = torch.zeros(1, dtype=torch.int32, device=device)
    rc = _lib.diag_lib().fs_diag_gather_rows(_lib.index_code(torch.int64), _lib.ptr(Bd), 8, 16, _lib.ptr(idxd),
                                             idx.numel(), _lib.ptr(chk), _lib.stream_handle(device))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(chk.cpu().numpy().view(np.uint32)[0]) == int(expect)
