/*
 * flagsparse_diag.h — C ABI of libflagsparse_diag.so, a measurement-only
 * library built beside libflagsparse_hip.so.  It is not part of the
 * operator path or its drop-in C ABI (include/flagsparse_hip.h) and has no
 * counterpart in the reference; bench.py --gather-floor and its GPU test
 * are its only callers.
 */
#ifndef FLAGSPARSE_DIAG_H
#define FLAGSPARSE_DIAG_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread in this library ("" if none). */
const char* fs_last_error(void);

/*
 * fs_diag_gather_rows gathers the rows idx[0..n_idx) of a row-major B of
 * n_b_rows rows of row_bytes bytes (a power of two in [4, 1024]; B aligned to
 * min(row_bytes, 16) bytes; rows of 4 or 8 bytes are SpMV x entries) with
 * nothing else in flight, and XORs the loaded words into *checksum (one
 * uint32 of device memory).  Index values outside [0, n_b_rows) are clamped
 * into it, so no index can address past B.  It measures the gather floor an
 * SpMM (SpMV) with the same column order cannot beat.  Does not synchronise
 * `stream`.
 */
int fs_diag_gather_rows(int idx_t, const void* B, int64_t n_b_rows, int64_t row_bytes,
                        const void* idx, int64_t n_idx, void* checksum, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLAGSPARSE_DIAG_H */
