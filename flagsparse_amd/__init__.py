"""flagsparse_amd — FlagSparse's CSR SpMV / SpMM path on MI355X (gfx950).

Drop-in for the reference's CSR SpMV/SpMM operators
(src/flagsparse/__init__.py:124-254, sparse_operations/__init__.py): same
function names, signatures, return shapes and error messages; the device
work runs in hand-written HIP kernels (libflagsparse_hip.so, C ABI in
include/flagsparse_hip.h).

    import flagsparse_amd as flagsparse
    y = flagsparse.flagsparse_spmv_csr(data, indices, indptr, x, shape)
"""

from ._common import (
    SUPPORTED_INDEX_DTYPES,
    SUPPORTED_VALUE_DTYPES,
    _INDEX_LIMIT_INT32,
    _tolerance_for_dtype,
)
from .benchmarks import (
    benchmark_spmm_case,
    benchmark_spmm_opt_alg2_case,
    benchmark_spmm_opt_case,
    benchmark_spmv_case,
)
from .coo import coo_to_csr_for_spmv, flagsparse_spmv_coo_tocsr, prepare_spmv_coo_tocsr
from .spmm_opt import (
    PreparedCsrSpmmOpt,
    PreparedCsrSpmmOptAlg2,
    flagsparse_spmm_csr_opt,
    flagsparse_spmm_csr_opt_alg1,
    flagsparse_spmm_csr_opt_alg1_preprocess,
    flagsparse_spmm_csr_opt_alg2,
    flagsparse_spmm_csr_opt_alg2_preprocess,
    prepare_spmm_csr_opt,
    prepare_spmm_csr_opt_alg1,
    prepare_spmm_csr_opt_alg1_preprocess,
    prepare_spmm_csr_opt_alg2,
    prepare_spmm_csr_opt_alg2_preprocess,
)
from .spmm_csr import (
    SPMM_CSR_ALGORITHMS,
    PreparedCsrSpmmRoute,
    SpmmCsrAlgorithm,
    SpmmCsrAlgorithmUnavailable,
    flagsparse_spmm_csr,
    flagsparse_spmm_csr_run,
    list_spmm_csr_algorithms,
    prepare_spmm_csr_route,
    resolve_spmm_csr_algorithm,
)
from .spmv_csr import PreparedCsrSpmv, flagsparse_spmv_csr, prepare_spmv_csr
from .spmv_coo import PreparedCoo, flagsparse_spmv_coo, prepare_spmv_coo
from .spmm_coo import flagsparse_spmm_coo
from .alpha_spmm import (
    PreparedAlphaSpmmAlg1,
    alpha_spmm_alg1_tle_opt2_unavailable_reason,
    alpha_spmm_alg1_tle_opt_unavailable_reason,
    alpha_spmm_alg1_tle_unavailable_reason,
    flagsparse_alpha_spmm_alg1,
    flagsparse_alpha_spmm_alg1_tle,
    flagsparse_alpha_spmm_alg1_tle_opt,
    flagsparse_alpha_spmm_alg1_tle_opt2,
    is_alpha_spmm_alg1_tle_available,
    is_alpha_spmm_alg1_tle_opt2_available,
    is_alpha_spmm_alg1_tle_opt_available,
    prepare_alpha_spmm_alg1,
    prepare_alpha_spmm_alg1_tle,
    prepare_alpha_spmm_alg1_tle_opt,
    prepare_alpha_spmm_alg1_tle_opt2,
)

__all__ = [
    "benchmark_spmv_case",
    "benchmark_spmm_case",
    "benchmark_spmm_opt_case",
    "benchmark_spmm_opt_alg2_case",
    "SUPPORTED_VALUE_DTYPES",
    "SUPPORTED_INDEX_DTYPES",
    "flagsparse_spmv_csr",
    "prepare_spmv_csr",
    "PreparedCsrSpmv",
    "flagsparse_spmm_csr",
    "flagsparse_spmm_csr_run",
    "prepare_spmm_csr_route",
    "list_spmm_csr_algorithms",
    "resolve_spmm_csr_algorithm",
    "SPMM_CSR_ALGORITHMS",
    "SpmmCsrAlgorithm",
    "SpmmCsrAlgorithmUnavailable",
    "PreparedCsrSpmmRoute",
    "PreparedCsrSpmmOpt",
    "PreparedCsrSpmmOptAlg2",
    "prepare_spmm_csr_opt",
    "prepare_spmm_csr_opt_alg1",
    "prepare_spmm_csr_opt_alg1_preprocess",
    "prepare_spmm_csr_opt_alg2",
    "prepare_spmm_csr_opt_alg2_preprocess",
    "flagsparse_spmm_csr_opt",
    "flagsparse_spmm_csr_opt_alg1",
    "flagsparse_spmm_csr_opt_alg1_preprocess",
    "flagsparse_spmm_csr_opt_alg2",
    "flagsparse_spmm_csr_opt_alg2_preprocess",
    "coo_to_csr_for_spmv",
    "prepare_spmv_coo_tocsr",
    "flagsparse_spmv_coo_tocsr",
    "PreparedCoo",
    "prepare_spmv_coo",
    "flagsparse_spmv_coo",
    "flagsparse_spmm_coo",
    "PreparedAlphaSpmmAlg1",
    "prepare_alpha_spmm_alg1",
    "prepare_alpha_spmm_alg1_tle",
    "prepare_alpha_spmm_alg1_tle_opt",
    "prepare_alpha_spmm_alg1_tle_opt2",
    "flagsparse_alpha_spmm_alg1",
    "flagsparse_alpha_spmm_alg1_tle",
    "flagsparse_alpha_spmm_alg1_tle_opt",
    "flagsparse_alpha_spmm_alg1_tle_opt2",
    "is_alpha_spmm_alg1_tle_available",
    "is_alpha_spmm_alg1_tle_opt_available",
    "is_alpha_spmm_alg1_tle_opt2_available",
    "alpha_spmm_alg1_tle_unavailable_reason",
    "alpha_spmm_alg1_tle_opt_unavailable_reason",
    "alpha_spmm_alg1_tle_opt2_unavailable_reason",
]
