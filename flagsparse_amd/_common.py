"""Dtype sets, limits and tolerances shared by the CSR operators.

Mirrors sparse_operations/_common.py:21-31 (value / index dtype sets,
_INDEX_LIMIT_INT32), _common.py:61-62 (_is_complex_dtype) and
_common.py:96-105 (_tolerance_for_dtype) of the reference.
"""

import torch

_SUPPORTED_VALUE_DTYPES = [
    torch.float16,
    torch.bfloat16,
    torch.float32,
    torch.float64,
    torch.complex64,
    torch.complex128,
]
SUPPORTED_VALUE_DTYPES = tuple(_SUPPORTED_VALUE_DTYPES)
SUPPORTED_INDEX_DTYPES = (torch.int32, torch.int64)
_INDEX_LIMIT_INT32 = 2**31 - 1

# Value dtypes the HIP kernels compute natively.  float16 / bfloat16 are
# accepted by validation (same messages as the reference) and computed in
# float32 (the reference's f16/bf16 base path also computes in float32,
# spmv_csr.py:124-127, spmm_csr.py:2716-2719).
HIP_VALUE_DTYPES = (torch.float32, torch.float64, torch.complex64, torch.complex128)


def _is_complex_dtype(value_dtype):
    return value_dtype in (torch.complex64, torch.complex128)


def _component_dtype_for_complex(value_dtype):
    if value_dtype == torch.complex64:
        return torch.float32
    if value_dtype == torch.complex128:
        return torch.float64
    raise TypeError(f"Unsupported complex dtype: {value_dtype}")


def _tolerance_for_dtype(value_dtype):
    """(atol, rtol) used by the reference's allclose checks."""
    if value_dtype == torch.float16:
        return 2e-3, 2e-3
    if value_dtype == torch.bfloat16:
        return 1e-1, 1e-1
    if value_dtype in (torch.float32, torch.complex64):
        return 1e-6, 1e-5
    if value_dtype in (torch.float64, torch.complex128):
        return 1e-10, 1e-8
    return 1e-6, 1e-5


def _compute_dtype(value_dtype):
    """dtype the HIP kernel is invoked with for a given input dtype."""
    if value_dtype in (torch.float16, torch.bfloat16):
        return torch.float32
    return value_dtype
