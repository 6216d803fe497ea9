// spmm_group.hip — CSR SpMM (C = A B) for gfx950: the lane-group kernel
// and the C-ABI entry points.
//
// Replaces the reference's base SpMM (spmm_csr.py:2684-2789 with
// _spmm_csr_real_kernel / _spmm_csr_complex_kernel, spmm_csr.py:134-237,
// whose B / C strides, spmm_csr.py:134-176, this kernel takes too) and the
// bucketed opt kernels (spmm_csr.py:2792-3109, spmm_csr_opt_alg2.py:438-729).
#include "fs_common.hpp"

#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>

namespace fs {

constexpr int kMergeTileItems = 512;  // tile of the merge-path kernel in spmm.hip

int spmm_merge_dispatch(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                        const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense, const int64_t* part,
                        int64_t n_tiles, void* ws, hipStream_t stream);

template <class T>
__device__ inline T readlane_any(const T& v, int lane) {
  constexpr int W = (int)(sizeof(T) / 4);
  int w[W];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = __builtin_amdgcn_readlane(w[k], lane);
  T out;
  __builtin_memcpy(&out, w, sizeof(T));
  return out;
}

// ---------------------------------------------------------------------------
// Lane-group SpMM (the default kernel).
//
// A wave is split into G = 64 / LPR groups of LPR lanes.  Each lane owns EPL
// consecutive columns of B / C (EPL * sizeof(V) = 16 bytes, so a B-row slice
// is one 16-byte load per lane: 64 lanes gather G rows per instruction).
// Every group walks its own merge-path sub-tile of S items (rows + nnz), so
// one load instruction gathers G different B rows and no FMA is predicated
// per group.  The sub-tile's row ends are staged in LDS (2-byte offsets from
// the sub-tile's first nnz); column / value chunks of LPR entries sit one per
// lane and reach the group's lanes by ds_bpermute (readlane when G == 1).
// Gathers are double buffered (U steps per batch).  Rows that cross
// sub-tiles leave head / tail fragments, summed in sub-tile order by
// spmm_group_fixup_kernel: deterministic, no floating-point atomics.
//
// B(k, n) is B[k * sbk + n * sbn] and C(m, n) is C[m * scm + n * scn]: the
// row-major fast path (sbn == scn == 1, 16-byte aligned) uses vector loads
// and stores, any other layout (column-major B / C) element accesses.
// ---------------------------------------------------------------------------
template <class V>
constexpr int group_epl() {
  return (int)(16 / sizeof(V));
}

template <class T>
__device__ inline T bcast_lane(const T& v, int src_lane) {
  constexpr int W = (int)(sizeof(T) / 4);
  int w[W];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = __builtin_amdgcn_ds_bpermute(src_lane << 2, w[k]);
  T out;
  __builtin_memcpy(&out, w, sizeof(T));
  return out;
}

// VEC: 16-byte vector loads / stores of row-major slices; otherwise element
// accesses at any strides.  Measured alternatives, not kept: 16-byte buffer
// loads with 32-bit offsets (C4 1.264 / 1.275 ms, R-MAT complex64 N = 32
// 1.447 / 1.400 ms), two gathers per batch instead of four (more waves per
// SIMD; C4 1.33 ms against 1.26), a residency bound through
// amdgpu_waves_per_eu (spills registers).
template <class V, int LPR, int U, bool VEC, class I, class T = VT<V>>
__global__ __launch_bounds__(256) void spmm_group_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const void* __restrict__ rowptr_raw, int ptr64,
    const V* __restrict__ B, int64_t sbk, int64_t sbn, V* __restrict__ C, int64_t scm, int64_t scn,
    int64_t n_dense, const int64_t* __restrict__ part, int sub_items,
    typename T::acc* __restrict__ head, typename T::acc* __restrict__ tail, int64_t n_rows,
    int64_t nnz, int64_t n_sub, int xcd_cols, int row_ranges) {
  using A = typename T::acc;
  constexpr int G = 64 / LPR;
  constexpr int EPL = group_epl<V>();
  using L4 = __attribute__((ext_vector_type(4))) unsigned int;
  extern __shared__ uint16_t lds_re[];
  const int lane = threadIdx.x & 63;
  const int g = lane / LPR;
  const int gl = lane % LPR;
  const int64_t ctile = xcd_cols > 0 ? (int64_t)(blockIdx.x % (unsigned)xcd_cols) : (int64_t)blockIdx.y;
  // row_ranges (2-D grid only): each XCD walks one contiguous range of tile
  // blocks, so the rows in flight on an XCD at any moment are adjacent
  const int64_t tblk = xcd_cols > 0 ? (int64_t)(blockIdx.x / (unsigned)xcd_cols)
                                    : (row_ranges ? xcd_range_block(blockIdx.x, gridDim.x) : (int64_t)blockIdx.x);
  const int64_t wid = tblk * 4 + (threadIdx.x >> 6);
  if (wid * G >= n_sub) return;  // wave-uniform; no barriers below
  const int64_t st = wid * G + g;
  const bool live = st < n_sub;
  const int64_t col0 = ctile * (int64_t)(LPR * EPL) + (int64_t)gl * EPL;
  const int64_t vrem = n_dense - col0;
  const int valid = vrem <= 0 ? 0 : (vrem >= EPL ? EPL : (int)vrem);
  // Loads are unconditional (so the compiler can count the ones in flight):
  // lanes past the last column read column 0's slice and discard it, steps
  // past a group's last nnz read B row 0.
  const int64_t col0_ld = valid > 0 ? col0 : 0;

  // sub-tile coordinates (merge path).  The prologue's loads are
  // unconditional, and each waits only on what its address needs: the
  // partition entries, then at once the row pointers and the first entry
  // chunks (a load in a branch is waited for at the branch's end).
  const int64_t st_ld = live ? st : n_sub - 1;
  const int64_t p0 = part[st_ld], p1 = part[st_ld + 1];
  int64_t r0 = 0, r1 = 0, n0 = 0;
  int nz = 0, R = 0;
  if (live) {
    r0 = p0;
    r1 = p1;
    const int64_t d0 = st * (int64_t)sub_items;
    const int64_t total = n_rows + nnz;
    const int64_t dend = d0 + sub_items < total ? d0 + sub_items : total;
    n0 = d0 - r0;
    nz = (int)(dend - r1 - n0);
    R = (int)(r1 - r0);
  }
  // Row pointer entries, int32 or int64, by one 8-byte load either way: an
  // int32 entry is read from the aligned 8-byte word that holds it (which
  // never crosses a page).
  auto rp = [&](int64_t i) -> int64_t {
    const unsigned char* a = static_cast<const unsigned char*>(rowptr_raw) + (i << (ptr64 ? 3 : 2));
    const uintptr_t mis = (uintptr_t)a & 7;
    const uint64_t w = *reinterpret_cast<const uint64_t*>(a - mis);
    return ptr64 ? (int64_t)w : (int64_t)(int32_t)(uint32_t)(mis ? w >> 32 : w);
  };

  const I* colp = cols + n0;
  const V* valp = vals + n0;
  // Entry chunks: LPR entries per group, one per lane; chunk c + 1 is loaded
  // while chunk c is walked.  Every global load below is unconditional, so
  // the compiler counts the ones in flight exactly and waits for a gather
  // only when its row is consumed: past a group's nnz, chunk entries re-read
  // entry 0 of the matrix (it exists whenever the kernel runs) and the steps
  // that use them are skipped.
  auto load_chunk = [&](int ch, I& cc, V& vv) {
    const int q = ch * LPR + gl;
    const bool in = q < nz;
    cc = *(in ? colp + q : cols);
    vv = *(in ? valp + q : vals);
  };
  I colC, colN;
  V valC, valN;
  load_chunk(0, colC, valC);
  load_chunk(1, colN, valN);

  const int64_t row_start = rp(r0);
  // row ends of the sub-tile -> LDS, as offsets from n0 (<= nz <= sub_items),
  // four loads in flight per lane; the first four go out with the loads
  // above (an index clamped to R - 1 reads a real entry, r0 itself when R
  // is 0)
  uint16_t* re_tab = lds_re + (size_t)((threadIdx.x >> 6) * G + g) * (size_t)sub_items;
  auto row_ends = [&](int k0) {
    int64_t e[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = k0 + u * LPR + gl;
      e[u] = rp(r0 + 1 + (k < R ? k : R - 1));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = k0 + u * LPR + gl;
      if (k < R) re_tab[k] = (uint16_t)(e[u] - n0);
    }
  };
  row_ends(0);
  for (int k0 = 4 * LPR; k0 < R; k0 += 4 * LPR) row_ends(k0);
  const bool head_partial = R > 0 && row_start < n0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int maxnz = nz;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) maxnz = max(maxnz, __shfl_xor(maxnz, off));
  maxnz = __builtin_amdgcn_readfirstlane(maxnz);

  const V* Bl = B + col0_ld * sbn;
  const uint32_t row_bytes = (uint32_t)(sbk * (int64_t)sizeof(V));
  int row = 0;
  int re = R > 0 ? (int)re_tab[0] : 0x7fffffff;

  A acc[EPL];
#pragma unroll
  for (int k = 0; k < EPL; ++k) acc[k] = T::zero();
  auto emit = [&]() {
    if (valid > 0) {
      if (row == 0 && head_partial) {
        A* h = head + st * n_dense + col0;
#pragma unroll
        for (int k = 0; k < EPL; ++k)
          if (k < valid) h[k] = acc[k];
      } else {
        V* c = C + (r0 + row) * scm + col0 * scn;
        if constexpr (VEC) {
          V o[EPL];
#pragma unroll
          for (int k = 0; k < EPL; ++k) o[k] = T::out(acc[k]);
          L4 q;
          __builtin_memcpy(&q, o, 16);
          *reinterpret_cast<L4*>(c) = q;
        } else {
#pragma unroll
          for (int k = 0; k < EPL; ++k)
            if (k < valid) c[k * scn] = T::out(acc[k]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < EPL; ++k) acc[k] = T::zero();
  };
  auto next_row = [&]() {
    ++row;
    re = row < R ? (int)re_tab[row] : 0x7fffffff;
  };

  // Gathers of batch b (U steps) of a chunk held in (cc, vv).
  auto issue = [&](int b, const I& cch, const V& vch, V (&bb)[U][EPL], V (&aa)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int li = b * U + u;
      I cc;
      if constexpr (G == 1) {
        cc = readlane_any(cch, li);
        aa[u] = readlane_any(vch, li);
      } else {
        cc = bcast_lane(cch, g * LPR + li);
        aa[u] = bcast_lane(vch, g * LPR + li);
      }
      if constexpr (VEC) {
        // one 32 x 32 + 64-bit multiply-add per gather (the host takes this
        // path only when columns and the row stride in bytes fit 32 bits)
        const char* pb = reinterpret_cast<const char*>(Bl) + (uint64_t)(uint32_t)cc * (uint64_t)row_bytes;
        L4 q = *reinterpret_cast<const L4*>(pb);
        __builtin_memcpy(bb[u], &q, 16);
      } else {
        const V* p = Bl + (int64_t)cc * sbk;
#pragma unroll
        for (int k = 0; k < EPL; ++k) bb[u][k] = p[(k < valid ? k : 0) * sbn];
      }
    }
  };
  auto consume = [&](int s0, V (&bb)[U][EPL], V (&aa)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u;
      if (s < nz) {
        while (re <= s) {  // rows that end before nnz s (empty rows included)
          emit();
          next_row();
        }
#pragma unroll
        for (int k = 0; k < EPL; ++k) acc[k] = T::fma(aa[u], bb[u][k], acc[k]);
      }
    }
  };

  constexpr int NB = LPR / U;  // batches per chunk (even)
  static_assert(NB % 2 == 0, "an even number of batches per chunk");
  const int n_chunks = (maxnz + LPR - 1) / LPR;
  V bA[U][EPL], bB[U][EPL];
  V aA[U], aB[U];
  issue(0, colC, valC, bA, aA);
  for (int c = 0; c < n_chunks; ++c) {
#pragma unroll
    for (int b = 0; b < NB; b += 2) {
      issue(b + 1, colC, valC, bB, aB);
      consume(c * LPR + b * U, bA, aA);
      if (b + 2 < NB) issue(b + 2, colC, valC, bA, aA);
      else issue(0, colN, valN, bA, aA);  // first batch of the next chunk (unused after the last)
      consume(c * LPR + (b + 1) * U, bB, aB);
    }
    colC = colN;
    valC = valN;
    load_chunk(c + 2, colN, valN);
  }
  while (row < R) {  // rows ending at the sub-tile's last nnz, and trailing empty rows
    emit();
    next_row();
  }
  if (live && r1 < n_rows && valid > 0) {
    A* tl = tail + st * n_dense + col0;
#pragma unroll
    for (int k = 0; k < EPL; ++k)
      if (k < valid) tl[k] = acc[k];
  }
}

// C = 0 for a matrix without entries (any strides).
template <class V>
__global__ __launch_bounds__(256) void spmm_zero_kernel(V* __restrict__ C, int64_t scm, int64_t scn, int64_t n_rows,
                                                        int64_t n_dense) {
  const int64_t total = n_rows * n_dense;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / n_dense, c = i - r * n_dense;
    C[r * scm + c * scn] = V{};
  }
}

// Rows that cross sub-tiles: C[row] = tail[f] + ... + tail[t-1] + head[t].
template <class V, class T = VT<V>>
__global__ __launch_bounds__(256) void spmm_group_fixup_kernel(
    const void* __restrict__ rowptr_raw, int ptr64, const int64_t* __restrict__ part, int sub_items,
    const typename T::acc* __restrict__ head, const typename T::acc* __restrict__ tail,
    V* __restrict__ C, int64_t scm, int64_t scn, int64_t n_dense, int64_t n_sub) {
  using A = typename T::acc;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_sub) return;
  const int64_t r0 = part[t];
  if (part[t + 1] == r0) return;
  const int64_t n0 = t * (int64_t)sub_items - r0;
  const int64_t start = ptr64 ? static_cast<const int64_t*>(rowptr_raw)[r0]
                              : (int64_t) static_cast<const int32_t*>(rowptr_raw)[r0];
  if (start >= n0) return;
  const int64_t f = fixup_start_tile(part, t, r0);
  for (int64_t col = (int64_t)blockIdx.y * 64 + (threadIdx.x & 63); col < n_dense;
       col += (int64_t)gridDim.y * 64) {
    A sum = tail[f * n_dense + col];
    sum = sum_fragments(tail + col, n_dense, f + 1, t, sum);  // in sub-tile order
    sum = add(sum, head[t * n_dense + col]);
    C[r0 * scm + col * scn] = T::out(sum);
  }
}

// Lanes per group for a dense width: twice the lanes whose 16-byte slices
// cover n_dense, at least 16 and at most 64 (wider B runs several column
// tiles of 64 lanes).  The idle upper half of a group re-reads its first
// slice, which shares the row's cache lines; fewer groups per wave walk
// fewer sub-tiles side by side.  Measured on MI355X (kernel ms, lanes per
// group 16 / 32): 1M x 1M with 32 uniform columns per row, f32, N = 64:
// 1.32 / 1.26; R-MAT 2^21 complex64 N = 32: 1.55 / 1.39.
// FLAGSPARSE_SPMM_LPR forces a width (8, 16, 32 or 64).
inline int group_lpr(int val_t, int64_t n_dense) {
  const int esz[] = {4, 8, 8, 16};
  const int epl = 16 / esz[val_t];
  int need = 1;
  while (need < 64 && (int64_t)need * epl < n_dense) need <<= 1;
  int lpr = std::min(64, std::max(16, 2 * need));
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_LPR")) {
    const int v = std::atoi(e);
    if (v == 8 || v == 16 || v == 32 || v == 64) lpr = v;
  }
  return lpr;
}

// Items per sub-tile: a wave covers kGroupWaveItems items whatever its
// group count (FLAGSPARSE_SPMM_WAVE_ITEMS overrides, 256..16384).
constexpr int kGroupWaveItems = 2048;
inline int group_sub_items(int val_t, int64_t n_dense) {
  int wave_items = kGroupWaveItems;
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_WAVE_ITEMS")) {
    const int v = std::atoi(e);
    if (v >= 256 && v <= 16384) wave_items = v;
  }
  return wave_items * group_lpr(val_t, n_dense) / 64;
}

// Kernel choice.  The lane-group kernel is the default.  For B rows of at
// least 512 bytes on matrices with skewed columns (the caller sets
// plan->spmm_wg_cap when a few columns hold much of the matrix) the
// merge-path kernel wins: two columns per lane in XCD-affine column tiles
// under a residency cap keep more hot B rows in L2.  Kernel ms, merge /
// lane-group, R-MAT 2^20: f32 N = 128 1.27 / 1.37, N = 256 2.50 / 3.14;
// complex64 N = 64 1.26 / 1.38, N = 128 2.66 / 3.15; on uniform columns
// the lane-group kernel ties or wins (complex64 N = 128: 6.63 / 5.85).
// Both kernels use 512-item tiles for such rows, so the partition does not
// depend on the choice; the merge kernel reads row-major B / C only.
// FLAGSPARSE_SPMM_KERNEL=merge|group forces one.
inline int forced_kernel() {  // 0 none, 1 merge, 2 group
  const char* e = std::getenv("FLAGSPARSE_SPMM_KERNEL");
  if (!e) return 0;
  if (std::string(e) == "merge") return 1;
  if (std::string(e) == "group") return 2;
  return 0;
}
inline bool wide_rows(int val_t, int64_t n_dense) {
  const int esz[] = {4, 8, 8, 16};
  return n_dense * esz[val_t] >= 512;
}
inline int spmm_tile_items_for(int val_t, int64_t n_dense) {
  const int f = forced_kernel();
  if (f == 1 || (f == 0 && wide_rows(val_t, n_dense))) return kMergeTileItems;
  return group_sub_items(val_t, n_dense);
}

template <class V, int LPR, class T>
int launch_spmm_group(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                      const void* B, int64_t sbk, int64_t sbn, void* C, int64_t scm, int64_t scn,
                      int64_t n_dense, const int64_t* part, int sub_items, int64_t n_sub, void* ws,
                      hipStream_t stream) {
  using A = typename T::acc;
  constexpr int G = 64 / LPR;
  constexpr int EPL = group_epl<V>();
  A* head = static_cast<A*>(ws);
  A* tail = head + n_sub * n_dense;
  const int64_t col_tiles = ceil_div(n_dense, (int64_t)LPR * EPL);
  const int64_t waves = ceil_div(n_sub, G);
  const int64_t blocks = ceil_div(waves, 4);
  if (blocks > 0x7fffffffLL || col_tiles > 65535) return fail(FS_E_INVALID, "fs_spmm_csr: grid too large");
  int xcd_cols = (col_tiles == 2 || col_tiles == 4 || col_tiles == 8) ? (int)col_tiles : 0;
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_XCD")) xcd_cols = std::atoi(e) != 0 ? (int)col_tiles : 0;
  if (xcd_cols > 0 && blocks * col_tiles > 0x7fffffffLL) xcd_cols = 0;
  int row_ranges = 0;
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_ROW_RANGES")) row_ranges = std::atoi(e) != 0;
  dim3 grid = xcd_cols > 0 ? dim3((unsigned)(blocks * col_tiles)) : dim3((unsigned)blocks, (unsigned)col_tiles);
  size_t lds = (size_t)4 * G * (size_t)sub_items * sizeof(uint16_t);
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_WG_CAP")) lds = std::max(lds, lds_pad_for_cap(std::atoi(e), 0));
  // vector path: every lane's B / C slice is EPL unit-stride elements, 16-byte aligned
  // (and 32-bit gather offsets: column indices and B's row stride in bytes fit 32 bits)
  const bool vec = sbn == 1 && scn == 1 && (n_dense % EPL) == 0 && (sbk % EPL) == 0 && (scm % EPL) == 0 &&
                   ((uintptr_t)B % 16) == 0 && ((uintptr_t)C % 16) == 0 && plan->n_cols <= (int64_t(1) << 32) &&
                   sbk * (int64_t)sizeof(V) < (int64_t(1) << 32);
  const int ptr64 = plan->ptr_t == FS_I64 ? 1 : 0;
  auto go = [&](auto icode) {
    using I = std::conditional_t<decltype(icode)::value, int64_t, int32_t>;
    auto launch = [&](auto vcode) {
      hipLaunchKernelGGL((spmm_group_kernel<V, LPR, 4, decltype(vcode)::value, I, T>), grid, dim3(256), lds, stream,
                         static_cast<const V*>(vals), static_cast<const I*>(cols), indptr, ptr64,
                         static_cast<const V*>(B), sbk, sbn, static_cast<V*>(C), scm, scn, n_dense, part, sub_items,
                         head, tail, plan->n_rows, plan->nnz, n_sub, xcd_cols, row_ranges);
    };
    if (vec) launch(std::true_type{});
    else launch(std::false_type{});
  };
  if (plan->idx_t == FS_I64) go(std::true_type{});
  else go(std::false_type{});
  FS_CHECK_MAIN_LAUNCH("spmm_group_kernel");
  const int64_t fix_blocks = ceil_div(n_sub, 4);
  const int64_t fix_cols = ceil_div(n_dense, 64) < 64 ? ceil_div(n_dense, 64) : 64;
  hipLaunchKernelGGL((spmm_group_fixup_kernel<V, T>), dim3((unsigned)fix_blocks, (unsigned)fix_cols), dim3(256), 0,
                     stream, indptr, plan->ptr_t == FS_I64 ? 1 : 0, part, sub_items, head, tail,
                     static_cast<V*>(C), scm, scn, n_dense, n_sub);
  FS_CHECK_LAUNCH("spmm_group_fixup_kernel");
  return FS_OK;
}

template <class V, class T>
int launch_spmm_group_lpr_t(int lpr, const fs_csr_plan* plan, const void* vals, const void* cols,
                            const void* indptr, const void* B, int64_t sbk, int64_t sbn, void* C, int64_t scm,
                            int64_t scn, int64_t n_dense, const int64_t* part, int sub_items, int64_t n_sub,
                            void* ws, hipStream_t s) {
  switch (lpr) {
    case 8: return launch_spmm_group<V, 8, T>(plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, sub_items, n_sub, ws, s);
    case 16: return launch_spmm_group<V, 16, T>(plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, sub_items, n_sub, ws, s);
    case 32: return launch_spmm_group<V, 32, T>(plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, sub_items, n_sub, ws, s);
    case 64: return launch_spmm_group<V, 64, T>(plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, sub_items, n_sub, ws, s);
  }
  return fail(FS_E_INVALID, "fs_spmm_csr: unsupported lane-group width");
}

// native = 1: float32 / complex64 accumulate in their own precision (VN);
// otherwise, and always for float64 / complex128, in VT's.
template <class V>
int launch_spmm_group_lpr(int lpr, int native, const fs_csr_plan* plan, const void* vals, const void* cols,
                          const void* indptr, const void* B, int64_t sbk, int64_t sbn, void* C, int64_t scm,
                          int64_t scn, int64_t n_dense, const int64_t* part, int sub_items, int64_t n_sub,
                          void* ws, hipStream_t s) {
  if constexpr (std::is_same_v<V, float> || std::is_same_v<V, c32>) {
    if (native)
      return launch_spmm_group_lpr_t<V, VN<V>>(lpr, plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense,
                                               part, sub_items, n_sub, ws, s);
  }
  return launch_spmm_group_lpr_t<V, VT<V>>(lpr, plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part,
                                           sub_items, n_sub, ws, s);
}

}  // namespace fs

using namespace fs;

extern "C" int fs_spmm_tile_items(int val_t, int64_t n_dense) {
  if (val_t < FS_F32 || val_t > FS_C128) return kMergeTileItems;
  return spmm_tile_items_for(val_t, n_dense);
}

extern "C" size_t fs_spmm_workspace_bytes(int val_t, int64_t n_tiles, int64_t n_dense) {
  const size_t acc = (val_t == FS_C64 || val_t == FS_C128) ? sizeof(c64) : sizeof(double);
  return (size_t)n_tiles * (size_t)n_dense * 2 * acc;
}

extern "C" int fs_spmm_csr_strided(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                                   const void* B, int64_t sbk, int64_t sbn, void* C, int64_t scm, int64_t scn,
                                   int64_t n_dense, const void* part_dev, int tile_items, int64_t n_tiles, void* ws,
                                   size_t ws_bytes, hipStream_t stream) {
  if (!plan) return fail(FS_E_INVALID, "fs_spmm_csr: plan is null");
  if (!valid_types(plan->val_t, plan->idx_t, plan->ptr_t)) return fail(FS_E_INVALID, "fs_spmm_csr: bad type code");
  if (n_dense < 0 || sbk < 0 || sbn < 0 || scm < 0 || scn < 0) return fail(FS_E_INVALID, "fs_spmm_csr: negative size");
  if (plan->n_rows == 0 || n_dense == 0) return FS_OK;
  const int forced = forced_kernel();
  const bool merge = forced == 1 || (forced == 0 && wide_rows(plan->val_t, n_dense) && plan->spmm_wg_cap > 0);
  const bool group = !merge || sbn != 1 || scn != 1;
  const int want_items = fs_spmm_tile_items(plan->val_t, n_dense);
  if (tile_items != want_items) return fail(FS_E_INVALID, "fs_spmm_csr: tile_items must come from fs_spmm_tile_items");
  if (n_tiles != ceil_div(plan->n_rows + plan->nnz, tile_items))
    return fail(FS_E_INVALID, "fs_spmm_csr: n_tiles does not match the matrix");
  // C must not overlap itself: distinct (row, column) pairs map to distinct elements.
  const bool c_rowmajor = scn == 1 && scm >= n_dense;
  const bool c_colmajor = scm == 1 && scn >= plan->n_rows;
  if (!(c_rowmajor || c_colmajor) && !(n_dense == 1 && scm >= 1) && !(plan->n_rows == 1 && scn >= 1))
    return fail(FS_E_INVALID, "fs_spmm_csr: C strides overlap (leading dimension smaller than the other extent)");
  if (!indptr || !C || !part_dev || (plan->nnz > 0 && (!vals || !cols || !B)))
    return fail(FS_E_INVALID, "fs_spmm_csr: null pointer");
  if (ws_bytes < fs_spmm_workspace_bytes(plan->val_t, n_tiles, n_dense) || (!ws && n_tiles > 0))
    return fail(FS_E_WORKSPACE, "fs_spmm_csr: workspace too small");
  const int64_t* part = static_cast<const int64_t*>(part_dev);
  if (plan->nnz == 0) {
    const int64_t blocks = std::min<int64_t>(ceil_div(plan->n_rows * n_dense, 256), 65536);
    switch (plan->val_t) {
      case FS_F32: hipLaunchKernelGGL(spmm_zero_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<float*>(C), scm, scn, plan->n_rows, n_dense); break;
      case FS_F64: hipLaunchKernelGGL(spmm_zero_kernel<double>, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<double*>(C), scm, scn, plan->n_rows, n_dense); break;
      case FS_C64: hipLaunchKernelGGL(spmm_zero_kernel<c32>, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<c32*>(C), scm, scn, plan->n_rows, n_dense); break;
      default: hipLaunchKernelGGL(spmm_zero_kernel<c64>, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<c64*>(C), scm, scn, plan->n_rows, n_dense); break;
    }
    FS_CHECK_LAUNCH("spmm_zero_kernel");
    return FS_OK;
  }
  if (group) {
    const int lpr = group_lpr(plan->val_t, n_dense);
    int native = 0;
    if (const char* e = std::getenv("FLAGSPARSE_SPMM_ACC")) native = std::string(e) == "native";
    switch (plan->val_t) {
      case FS_F32: return launch_spmm_group_lpr<float>(lpr, native, plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, tile_items, n_tiles, ws, stream);
      case FS_F64: return launch_spmm_group_lpr<double>(lpr, native, plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, tile_items, n_tiles, ws, stream);
      case FS_C64: return launch_spmm_group_lpr<c32>(lpr, native, plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, tile_items, n_tiles, ws, stream);
      default: return launch_spmm_group_lpr<c64>(lpr, native, plan, vals, cols, indptr, B, sbk, sbn, C, scm, scn, n_dense, part, tile_items, n_tiles, ws, stream);
    }
  }
  // Merge-path kernel (FLAGSPARSE_SPMM_KERNEL=merge): row-major B / C only.
  if (sbn != 1 || scn != 1) return fail(FS_E_INVALID, "fs_spmm_csr: the merge kernel takes row-major B and C only");
  if (scm < n_dense || (plan->n_cols > 0 && sbk < n_dense))
    return fail(FS_E_INVALID, "fs_spmm_csr: leading dimension smaller than n_dense");
  return spmm_merge_dispatch(plan, vals, cols, indptr, B, sbk, C, scm, n_dense, part, n_tiles, ws, stream);
}

extern "C" int fs_spmm_csr(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                           const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense,
                           const void* part_dev, int tile_items, int64_t n_tiles, void* ws, size_t ws_bytes,
                           hipStream_t stream) {
  if (plan && plan->n_rows > 0 && n_dense > 0 && (ldc < n_dense || (plan->n_cols > 0 && ldb < n_dense)))
    return fail(FS_E_INVALID, "fs_spmm_csr: leading dimension smaller than n_dense");
  return fs_spmm_csr_strided(plan, vals, cols, indptr, B, ldb, 1, C, ldc, 1, n_dense, part_dev, tile_items, n_tiles,
                             ws, ws_bytes, stream);
}
