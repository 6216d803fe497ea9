/*
 * flagsparse_hip.h — C ABI of the MI355X (gfx950) CSR SpMV / SpMM library.
 *
 * The library replaces the device half of FlagSparse's CSR SpMV/SpMM path.
 * In the reference that half is a set of Triton kernels launched from
 * Python (src/flagsparse/sparse_operations/spmv_csr.py,
 * spmm_csr.py); here it is hand-written HIP for gfx950 behind plain C
 * functions.  The Python host layer (flagsparse_amd/) keeps the reference's
 * public signatures and calls only these entry points.
 *
 * Conventions shared by every entry point:
 *   - all array arguments are raw device pointers; sizes are int64_t;
 *   - value / index types are passed as the enums below;
 *   - every launch goes to the caller's hipStream_t and returns without
 *     synchronising, except fs_csr_check, fs_csr_analyze and
 *     fs_csr_panelize, which read small results back to the host
 *     (documented below);
 *   - nothing is allocated: scratch memory comes from a caller workspace
 *     whose size the matching *_workspace_bytes / plan fields report;
 *   - the return value is 0 on success, a negative FS_E* code otherwise;
 *     fs_last_error() returns a human-readable message for the calling
 *     thread's last failure.
 *   - op=trans/conj are expressed by transposing first (fs_csr_transpose),
 *     exactly as the reference materialises A^T / A^H before its kernel.
 */
#ifndef FLAGSPARSE_HIP_H
#define FLAGSPARSE_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Value types: the reference's SUPPORTED_VALUE_DTYPES minus f16/bf16
 * (sparse_operations/_common.py:21-28). */
enum fs_value_type { FS_F32 = 0, FS_F64 = 1, FS_C64 = 2, FS_C128 = 3 };
/* Index types: SUPPORTED_INDEX_DTYPES (_common.py:29). */
enum fs_index_type { FS_I32 = 0, FS_I64 = 1 };
/* Column storage of a SELL-64 copy: absolute int32 / int64, the int16
 * offset c - r from the entry's row (banded matrices, |c - r| <= 32767), or
 * a uint8 code of that offset into a table of at most 256 offsets (matrices
 * with few distinct offsets, such as stencils). */
enum fs_sell_index { FS_SELL_I32 = 0, FS_SELL_I64 = 1, FS_SELL_D16 = 2, FS_SELL_C8 = 3 };
/* Entry order inside a SELL-64 slice: one slot of 64 rows after another, or
 * pairs of a row's consecutive slots side by side (real values only). */
enum fs_sell_layout { FS_SELL_SLOT = 0, FS_SELL_PAIR = 1 };

enum fs_status {
  FS_OK = 0,
  FS_E_INVALID = -1,   /* bad argument (type code, size, null pointer) */
  FS_E_WORKSPACE = -2, /* caller workspace too small */
  FS_E_HIP = -3        /* a HIP runtime call failed */
};

/* Kernel variants chosen by fs_csr_analyze. */
enum fs_kernel { FS_KERNEL_VECTOR = 0, FS_KERNEL_MERGE = 1, FS_KERNEL_STREAM = 2, FS_KERNEL_NNZBLOCK = 3 };

#define FS_HIST_BINS 24 /* bin b counts rows with length in [2^(b-1), 2^b); bin 0 = empty rows */

/* Analysis result for one CSR matrix (plain data, host memory). */
typedef struct fs_csr_plan {
  int64_t n_rows, n_cols, nnz;
  int32_t val_t, idx_t, ptr_t;
  int32_t kernel;        /* FS_KERNEL_* chosen for SpMV */
  int32_t vec_width;     /* lanes per row (FS_KERNEL_VECTOR, FS_KERNEL_NNZBLOCK) */
  int32_t tile_items;    /* merge-path items (rows + nnz) per tile; entries
                            per block for FS_KERNEL_NNZBLOCK */
  int32_t rows_per_block; /* rows per workgroup for FS_KERNEL_STREAM */
  int32_t spmm_wg_cap;   /* fs_spmm_csr: workgroups per CU for the two-columns-
                            per-lane kernel (0 = as many as resources allow).
                            fs_csr_analyze writes 0; the caller may set it. */
  int64_t n_tiles;       /* merge-path tiles / entry blocks */
  int64_t max_row, min_row;
  int64_t hist[FS_HIST_BINS];
  size_t part_bytes;     /* device bytes for the SpMV partition */
  size_t carry_bytes;    /* device bytes for the SpMV carries */
} fs_csr_plan;

/* Last error message of the calling thread ("" if none). */
const char* fs_last_error(void);

/*
 * Name of the main kernel (e.g. "spmv_sell_group_kernel") that the calling
 * thread's latest successful SpMV / SpMM launch ran ("" before any).  For
 * reports and profiles.  No counterpart in the reference, whose Triton
 * kernels are named by the Python function that launches them.
 */
const char* fs_last_kernel(void);

/* Library version string. */
const char* fs_version(void);

/*
 * Row-length statistics of a device CSR row pointer, and the SpMV kernel
 * choice made from them.  Replaces the reference's host-side preparation
 * (spmv_csr.py:591-664: max_row_nnz, block_nnz / max_segments sizing;
 * opt buckets spmv_csr.py:353-410).  Runs one histogram kernel into
 * `stats_dev` (>= fs_csr_stats_bytes() bytes of device memory), then
 * synchronises `stream` and decides on the host.  force_kernel < 0 lets the
 * analysis choose; 0/1/2/3 forces FS_KERNEL_VECTOR / FS_KERNEL_MERGE /
 * FS_KERNEL_STREAM / FS_KERNEL_NNZBLOCK (STREAM falls back to MERGE when
 * rows are too long; NNZBLOCK to STREAM when nnz == 0).
 */
size_t fs_csr_stats_bytes(void);
int fs_csr_analyze(const void* indptr, int ptr_t, int idx_t, int val_t,
                   int64_t n_rows, int64_t n_cols, int64_t nnz,
                   int force_kernel, void* stats_dev, fs_csr_plan* plan,
                   hipStream_t stream);

/*
 * Structure check of a CSR matrix, replacing the reference's separate
 * indptr / column-range checks (spmv_csr.py:546-558; the same checks guard
 * spmm_csr.py's prepare).  One pass over indptr and indices into `check_dev`
 * (>= fs_csr_check_bytes() bytes of device memory), then synchronises
 * `stream` and writes five values to host `out`: indptr[0], indptr[n_rows],
 * the number of rows r with indptr[r+1] < indptr[r], the smallest and the
 * largest column index (0 and -1 when nnz == 0).  The caller raises the
 * reference's errors from them, in the reference's order.
 */
size_t fs_csr_check_bytes(void);
int fs_csr_check(const void* indptr, int ptr_t, const void* indices, int idx_t,
                 int64_t n_rows, int64_t nnz, void* check_dev, int64_t* out,
                 hipStream_t stream);

/*
 * fs_csr_check without the round trip, for a caller that launches more work
 * before it needs the answer: launches the check pass into `check_dev` and
 * an asynchronous copy of its five result words (40 bytes) into
 * `host_words`, which must be pinned host memory; returns without
 * synchronising.  After the caller has synchronised `stream`,
 * fs_csr_check_decode turns the words into fs_csr_check's five values.
 * Used by flagsparse_spmm_csr with op="trans" / "conj" (the reference checks,
 * spmm_csr.py:239-297, then transposes, :300-349): the transpose and the
 * SpMM run behind the check, and the reference's error is raised before C is
 * returned.
 */
int fs_csr_check_enqueue(const void* indptr, int ptr_t, const void* indices, int idx_t,
                         int64_t n_rows, int64_t nnz, void* check_dev, void* host_words,
                         hipStream_t stream);
int fs_csr_check_decode(const void* host_words, int64_t nnz, int64_t* out);

/*
 * fs_csr_check and fs_csr_analyze in one device round trip: both passes are
 * launched, then one read-back fills `out` (as fs_csr_check) and `plan` (as
 * fs_csr_analyze) and synchronises `stream`.  `ws` holds
 * fs_csr_check_analyze_bytes() bytes of device memory.  The plan is only
 * meaningful when `out` shows a valid structure.  Used by the reference's
 * prepare path (spmv_csr.py:546-558 checks, then 623-647 sizing), which
 * every unprepared flagsparse_spmv_csr call runs.
 */
size_t fs_csr_check_analyze_bytes(void);
int fs_csr_check_analyze(const void* indptr, int ptr_t, const void* indices, int idx_t,
                         int val_t, int64_t n_rows, int64_t n_cols, int64_t nnz,
                         int force_kernel, void* ws, int64_t* out, fs_csr_plan* plan,
                         hipStream_t stream);

/*
 * Merge-path partition: for each tile t, the row coordinate where the
 * tile's merge path starts.  Writes plan->n_tiles+1 int64 into part_dev
 * (plan->part_bytes bytes).
 */
int fs_csr_partition(const fs_csr_plan* plan, const void* indptr,
                     void* part_dev, int tile_items, int64_t n_tiles,
                     hipStream_t stream);

/*
 * The partition fs_spmv_csr needs for the plan's kernel: the merge-path
 * partition (FS_KERNEL_MERGE) or, for FS_KERNEL_NNZBLOCK, the first owned
 * row of every entry block (block b owns the rows whose end pointer lies in
 * (b*C, (b+1)*C], C = plan->tile_items).  Writes plan->part_bytes bytes;
 * nothing for the other kernels.
 */
int fs_spmv_partition(const fs_csr_plan* plan, const void* indptr,
                      void* part_dev, hipStream_t stream);

/*
 * y = A x for a CSR A (n_rows x n_cols).  Replaces
 * _triton_spmv_csr_impl_prepared (spmv_csr.py:679-723) and the opt path
 * (spmv_csr.py:412-461).  fp32 accumulates in fp64 and rounds once, like the
 * reference's fp32 base path (spmv_csr.py:124-130, 685-705); complex64
 * accumulates in fp64 components.  For FS_KERNEL_MERGE, part_dev is the
 * fs_csr_partition output and carry_dev holds plan->carry_bytes.
 */
int fs_spmv_csr(const fs_csr_plan* plan, const void* vals, const void* cols,
                const void* indptr, const void* x, void* y,
                const void* part_dev, void* carry_dev, size_t carry_bytes,
                hipStream_t stream);

/*
 * The unprepared public SpMV call in one launch and one round trip.
 * Replaces the structure checks of _prepare_spmv_csr_matrix
 * (spmv_csr.py:546-558: indptr[0] == 0, indptr[-1] == nnz, a non-decreasing
 * indptr, columns in [0, n_cols)) and the launch of
 * _triton_spmv_csr_impl_prepared (spmv_csr.py:679-723) as the reference's
 * flagsparse_spmv_csr runs them without `prepared` (spmv_csr.py:813-913).
 * The kernel checks the structure while it computes y = A x; malformed
 * input is never read out of bounds (row pointers are clamped, stray
 * columns read column 0) and its y is garbage.  flags is 4 int32 of pinned,
 * device-accessible host memory (hipHostMalloc, or a torch tensor with
 * pin_memory=True): the call zeroes it, the kernel writes it directly, and
 * on return (the call synchronises `stream`) flags[0..3] are nonzero for a
 * bad start, a bad end, a decrease and a column out of range, the
 * reference's order of checks.  Needs n_rows, n_cols and nnz > 0.
 */
int fs_spmv_csr_oneshot(int val_t, int idx_t, int ptr_t, int64_t n_rows, int64_t n_cols,
                        int64_t nnz, const void* vals, const void* cols, const void* indptr,
                        const void* x, void* y, int32_t* flags, hipStream_t stream);

/*
 * fs_spmv_csr without a caller workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * carry fragments of the merge-path / entry-block kernels live in a static
 * device array of fs_spmv_noalloc_scratch_bytes() bytes (16 MiB) per GPU,
 * held until the process ends; matrices whose plan needs more
 * (plan->carry_bytes) are rejected with FS_E_WORKSPACE.  The entry point
 * calls no allocator.  All calls on one GPU share the array; calls from
 * several streams or host threads are ordered on the GPU (each call waits
 * for the previous call's kernels when that call used another stream, by an
 * event created at the first call on the device).  Under stream capture the
 * ordering is skipped: replays of captured calls that run at the same time
 * on one GPU race on the array.
 */
size_t fs_spmv_noalloc_scratch_bytes(void);
int fs_spmv_csr_noalloc(const fs_csr_plan* plan, const void* vals, const void* cols,
                        const void* indptr, const void* x, void* y,
                        const void* part_dev, hipStream_t stream);

/*
 * The use_opt SpMV path: native-precision accumulation (float32 in float32,
 * float64 in float64) over row-length buckets.  Replaces the reference's
 * _build_spmv_opt_buckets with its bucket tiers (spmv_csr.py:136-161,
 * 353-410; float32 <= 64 / <= 512 / <= 4096 / longer, float64 <= 64 /
 * <= 256 / <= 2048 / <= 8192 / longer, empty rows in the first bucket) and
 * _triton_spmv_csr_impl_opt_prepared with its four kernels
 * (spmv_csr.py:233-351, 412-461).  float32 / float64 values, int32 column
 * indices, int32 / int64 row pointer, as the reference's supports_opt.
 *
 * fs_spmv_opt_buckets partitions the row ids into the buckets, in `ws`
 * (fs_spmv_opt_workspace_bytes(n_rows) bytes of device memory), writes the
 * fs_spmv_opt_max_buckets() bucket sizes to host `counts_out` and
 * synchronises `stream`.  fs_spmv_csr_opt runs y = A x from that workspace
 * and those counts (one launch per non-empty bucket; no synchronisation).
 */
int fs_spmv_opt_max_buckets(void);
size_t fs_spmv_opt_workspace_bytes(int64_t n_rows);
int fs_spmv_opt_buckets(const void* indptr, int ptr_t, int val_t, int64_t n_rows,
                        void* ws, size_t ws_bytes, int64_t* counts_out,
                        hipStream_t stream);
int fs_spmv_csr_opt(int val_t, int idx_t, int ptr_t, int64_t n_rows,
                    const void* vals, const void* cols, const void* indptr,
                    const void* x, void* y, const void* ws, size_t ws_bytes,
                    const int64_t* counts, hipStream_t stream);

/*
 * C = A B, A CSR (n_rows x n_cols), B dense n_cols x n_dense with row stride
 * ldb (elements), C dense n_rows x n_dense with row stride ldc.  Replaces
 * _triton_spmm_csr_impl + _spmm_csr_real_kernel / _spmm_csr_complex_kernel
 * (spmm_csr.py:2684-2789, 134-237).  fp32 accumulates in fp64 (the
 * reference upcasts data and B to fp64, spmm_csr.py:2720-2759).  The
 * matrix is walked along a merge path of tile_items items per sub-tile:
 * tile_items = fs_spmm_tile_items(val_t, n_dense) (it depends on the dense
 * width), partition from fs_csr_partition with the same tile size.  Rows
 * that cross sub-tiles are finished by a fix-up pass using `ws`
 * (fs_spmm_workspace_bytes bytes).
 */
size_t fs_spmm_workspace_bytes(int val_t, int64_t n_tiles, int64_t n_dense);
int fs_spmm_tile_items(int val_t, int64_t n_dense);
int fs_spmm_csr(const fs_csr_plan* plan, const void* vals, const void* cols,
                const void* indptr, const void* B, int64_t ldb, void* C,
                int64_t ldc, int64_t n_dense, const void* part_dev,
                int tile_items, int64_t n_tiles, void* ws, size_t ws_bytes,
                hipStream_t stream);

/*
 * fs_spmm_csr with any element strides: B(k, n) = B[k * sbk + n * sbn],
 * C(m, n) = C[m * scm + n * scn].  The reference's SpMM kernel takes the
 * same four strides (spmm_csr.py:134-176: stride_bk, stride_bn, stride_cm,
 * stride_cn), which is how its csr_base route serves column-major B / C
 * (spmm_csr.py:585-639, 2090-2098).  Row-major operands with 16-byte
 * aligned rows take vector loads / stores; other layouts element accesses.
 * C's strides must not make two (row, column) pairs share an element.
 */
int fs_spmm_csr_strided(const fs_csr_plan* plan, const void* vals, const void* cols,
                        const void* indptr, const void* B, int64_t sbk, int64_t sbn,
                        void* C, int64_t scm, int64_t scn, int64_t n_dense,
                        const void* part_dev, int tile_items, int64_t n_tiles,
                        void* ws, size_t ws_bytes, hipStream_t stream);

/*
 * Transpose (CSR -> CSR of A^T, conjugating values when conj != 0).
 * Replaces _transpose_csr_for_spmv / _transpose_csr_for_spmm
 * (spmv_csr.py:477-515, spmm_csr.py:300-349) and the conj step
 * (spmv_csr.py:615-618, spmm_csr.py:341-349).  The result is identical to a
 * stable sort of the entries by column: within each output row the entries
 * keep ascending source-row order.  Built by an LSD radix sort on the column
 * index (per-tile digit counts, scan, stable scatter; no global atomics in
 * the partition); for 4- and 8-byte values with positions below 2^32 the
 * column pointer comes from integer atomic minima of each column's first
 * position and a suffix minimum (order-independent, so deterministic).
 * Output types: out_idx_t / out_ptr_t (the reference's rules: indices keep
 * their type unless n_rows > 2^31-1, indptr keeps its type unless
 * nnz > 2^31-1).
 */
size_t fs_csr_transpose_workspace_bytes(int64_t n_rows, int64_t n_cols,
                                        int64_t nnz);
/*
 * 1 when fs_csr_transpose of a matrix of this value type and these sizes
 * reads and writes only inside its arguments whatever the structure holds
 * (a row pointer or column indices that the structure check would reject
 * give a meaningless transpose, no out-of-bounds access), 0 otherwise.  The
 * caller may then queue the transpose before it has the check's answer.
 * No counterpart in the reference (its checks synchronise before the
 * transpose, spmm_csr.py:239-297).
 */
int fs_csr_transpose_bounded(int val_t, int64_t n_rows, int64_t n_cols, int64_t nnz);
/*
 * fs_csr_transpose with fs_csr_check_enqueue fused into its passes: the
 * reference's structure check (spmv_csr.py:546-558, spmm_csr.py:239-297)
 * followed by its transpose (spmv_csr.py:477-515, spmm_csr.py:300-349), in
 * one queue of kernels that reads the row pointer and the columns once for
 * both.  The five check words go to `check_dev` (fs_csr_check_bytes) and,
 * by an asynchronous copy, to the pinned `host_words`; after the caller has
 * synchronised `stream`, fs_csr_check_decode gives fs_csr_check's values,
 * except that a valid matrix reports its column range as [0, 0] (outside
 * [0, n_cols) the range holds the offending extremes).  Only where
 * fs_csr_transpose_bounded holds, with nnz > 0 (else FS_E_INVALID).
 */
int fs_csr_transpose_checked(int val_t, int idx_t, int ptr_t, int out_idx_t, int out_ptr_t,
                             int64_t n_rows, int64_t n_cols, int64_t nnz, const void* vals,
                             const void* cols, const void* indptr, int conj, void* t_vals,
                             void* t_cols, void* t_indptr, void* ws, size_t ws_bytes,
                             void* check_dev, void* host_words, hipStream_t stream);
int fs_csr_transpose(int val_t, int idx_t, int ptr_t, int out_idx_t,
                     int out_ptr_t, int64_t n_rows, int64_t n_cols,
                     int64_t nnz, const void* vals, const void* cols,
                     const void* indptr, int conj, void* t_vals,
                     void* t_cols, void* t_indptr, void* ws, size_t ws_bytes,
                     hipStream_t stream);

/*
 * COO -> CSR.  Replaces coo_to_csr_for_spmv (spmv_csr.py:926-950): entries
 * are ordered by the lexicographic key row * n_cols + col (a stable sort, so
 * already-sorted input keeps its order and duplicates keep input order; the
 * reference's non-stable argsort leaves duplicate order unspecified), the
 * column indices are written as int32 and the row pointer as int64, as the
 * reference does.  rows / cols share idx_t.  assume_sorted != 0 skips the
 * sort (the caller guarantees lexicographic order).
 */
size_t fs_coo_to_csr_workspace_bytes(int64_t n_rows, int64_t n_cols,
                                     int64_t nnz);
int fs_coo_to_csr(int val_t, int idx_t, int64_t n_rows, int64_t n_cols,
                  int64_t nnz, const void* vals, const void* rows,
                  const void* cols, int assume_sorted, void* out_vals,
                  void* out_cols, void* out_indptr, void* ws, size_t ws_bytes,
                  hipStream_t stream);

/*
 * Column panels for SpMV on matrices whose x does not fit one XCD's L2.
 * No counterpart call in the reference: it is part of what prepare_spmv_csr
 * (spmv_csr.py:591-676) may precompute once per matrix, and
 * fs_spmv_csr_panels then replaces _triton_spmv_csr_impl_prepared
 * (spmv_csr.py:679-723) for such a prepared matrix, with the same result
 * up to the order of the floating-point additions.
 *
 * fs_csr_panelize splits A (n_rows x n_cols) into n_panels (<= 64) column
 * panels of width ceil(n_cols / n_panels) and writes them as one stacked CSR
 * with n_panels * n_rows rows: row p * n_rows + r holds the entries of row r
 * whose column lies in panel p, in their CSR order; column indices are
 * unchanged.  p_vals / p_cols hold nnz entries, p_indptr n_panels * n_rows + 1.
 * panel_nnz (host, n_panels + 1) receives the entry offset of each panel; the
 * call synchronises `stream` to return it.
 *
 * fs_spmv_csr_panels computes y = A x from the stacked matrix: `plan` is
 * fs_csr_analyze of the stacked CSR (merge tiles), part_dev its partition
 * (fs_csr_partition with plan->tile_items), panel_nnz the host offsets from
 * fs_csr_panelize.  Each panel's tiles go to one XCD (workgroup b runs on
 * XCD b % 8); per-row panel partials stay in the accumulator type and are
 * summed in panel order (deterministic; float32 is still rounded once from
 * float64).  Does not synchronise.
 */
size_t fs_csr_panelize_workspace_bytes(int64_t n_rows, int64_t n_cols,
                                       int64_t nnz, int n_panels);
int fs_csr_panelize(int val_t, int idx_t, int ptr_t, int64_t n_rows,
                    int64_t n_cols, int64_t nnz, int n_panels,
                    const void* vals, const void* cols, const void* indptr,
                    void* p_vals, void* p_cols, void* p_indptr,
                    int64_t* panel_nnz, void* ws, size_t ws_bytes,
                    hipStream_t stream);
size_t fs_spmv_panels_workspace_bytes(const fs_csr_plan* plan, int n_panels);
int fs_spmv_csr_panels(const fs_csr_plan* plan, int n_panels,
                       const int64_t* panel_nnz, const void* vals,
                       const void* cols, const void* indptr, const void* x,
                       void* y, const void* part_dev, void* ws,
                       size_t ws_bytes, hipStream_t stream);

/* ---- Sliced-ELL copy (SELL-64) of a prepared CSR matrix ------------------
 * No counterpart call in the reference: like the column panels it is a
 * per-matrix copy that prepare_spmv_csr (spmv_csr.py:591-676) may build,
 * and fs_spmv_sell then replaces _triton_spmv_csr_impl_prepared
 * (spmv_csr.py:679-723) for that prepared matrix, with the same result up
 * to the order of the floating-point additions (each row is summed in its
 * CSR order).
 *
 * Layout: rows are cut into slices of 64 consecutive rows; slice s holds
 * S_s slots of 64 entries each.  FS_SELL_SLOT: S_s = slots[s] (the slice's
 * longest row), and entry k of row r sits at slice_ptr[r / 64] + 64 * k +
 * r % 64.  FS_SELL_PAIR: S_s = slots[s] rounded up to even, and entry k of
 * row r sits at slice_ptr[r / 64] + 128 * (k / 2) + 2 * (r % 64) + k % 2.
 * slice_ptr (device, int64, n_slices + 1 with n_slices = ceil(n_rows / 64))
 * is the exclusive prefix sum of 64 * S_s.  Padding entries are never
 * gathered or multiplied by fs_spmv_sell.
 *
 * fs_sell_slots writes slots[s] (device, int64, n_slices).
 * fs_sell_max_offset raises *max_dev (device, caller-initialised to 0) to
 * the largest |c - r| over the entries (c = column, r = row).  When
 * offset_bits_dev is not null (2048 uint32 words of device memory,
 * caller-zeroed) it also sets bit d + 32768 for every offset d = c - r with
 * |d| <= 32767.
 * fs_csr_to_sell writes the values and the columns into buffers of
 * slice_ptr[n_slices] entries, as sell_idx_t: FS_SELL_I32 / FS_SELL_I64
 * (absolute, wide enough for n_cols - 1), FS_SELL_D16 (int16 c - r; the
 * caller has checked fs_sell_max_offset <= 32767) or FS_SELL_C8 (uint8
 * code_lut[c - r + 32768]; code_lut is 65536 bytes of device memory that map
 * every offset present to its index in the code table).
 * code_lut is ignored for the other column storages.
 * fs_spmv_sell computes y = A x from the copy; row lengths come from the
 * CSR indptr (ptr_t).  With FS_SELL_C8, code_table holds 256 int32 offsets
 * (device memory; entry k is the offset of code k); otherwise it is ignored.
 * Rows may hold up to 2^31 - 1 entries.
 * None of the four synchronises `stream`.
 */
int fs_sell_slots(int ptr_t, int64_t n_rows, const void* indptr,
                  int64_t* slots_dev, hipStream_t stream);
int fs_sell_max_offset(int idx_t, int ptr_t, int64_t n_rows, const void* cols,
                       const void* indptr, unsigned long long* max_dev,
                       unsigned* offset_bits_dev, hipStream_t stream);
int fs_csr_to_sell(int val_t, int idx_t, int ptr_t, int sell_idx_t,
                   int layout, int64_t n_rows, const void* vals, const void* cols,
                   const void* indptr, const int64_t* slice_ptr,
                   const void* code_lut, void* sell_vals, void* sell_cols,
                   hipStream_t stream);
/*
 * C = A B on the SELL-64 copy of a prepared matrix (fs_csr_to_sell) with a
 * row-major B (n_cols x n_dense, leading dimension ldb) and C (n_rows x
 * n_dense, ldc): n_dense, ldb and ldc multiples of 16 / sizeof(value), B and
 * C 16-byte aligned.  Each row sums its entries in CSR order in the
 * accumulator type, in one sequence.  Replaces, for banded and
 * stencil matrices, the reference's SpMM kernels on its prepared route
 * (spmm_csr.py:134-237 launched from spmm_csr.py:2040-2174).
 */
int fs_spmm_sell(int val_t, int sell_idx_t, int ptr_t, int layout, int64_t n_rows,
                 const void* sell_vals, const void* sell_cols,
                 const int32_t* code_table, const int64_t* slice_ptr,
                 const void* indptr, const void* B, int64_t ldb, void* C, int64_t ldc,
                 int64_t n_dense, hipStream_t stream);
/*
 * fs_spmm_sell for a copy with offset codes (FS_SELL_C8), B staged through
 * LDS: per (slice, column tile) a workgroup copies the B-row tiles its
 * codes' windows cover (`offsets_host`: the n_codes offsets the codes stand
 * for, host memory; `code_table`: the same 256-entry table on the device)
 * with coalesced 16-byte loads, then sums every row from LDS in the same
 * order as fs_spmm_sell (the same bits).  `n_b_rows` is B's row count.
 * fs_spmm_sell_staged_fits says whether the offsets' bands (merged windows
 * of 64 rows) fit: at most 32 bands within 64 KB of LDS.  The row-block SpMM
 * that streams dense-B tiles through LDS, for banded and stencil matrices on
 * the reference's prepared route (spmm_csr.py:134-237, 2040-2174).
 */
int fs_spmm_sell_staged_fits(int val_t, const int32_t* offsets_host, int n_codes, int64_t n_dense);
int fs_spmm_sell_staged(int val_t, int ptr_t, int layout, int64_t n_rows, int64_t n_b_rows,
                        const void* sell_vals, const void* sell_codes, const int32_t* code_table,
                        const int32_t* offsets_host, int n_codes, const int64_t* slice_ptr,
                        const void* indptr, const void* B, int64_t ldb, void* C, int64_t ldc,
                        int64_t n_dense, hipStream_t stream);
int fs_spmv_sell(int val_t, int sell_idx_t, int ptr_t, int layout, int64_t n_rows,
                 const void* sell_vals, const void* sell_cols,
                 const int32_t* code_table, const int64_t* slice_ptr,
                 const void* indptr, const void* x, void* y, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLAGSPARSE_HIP_H */
