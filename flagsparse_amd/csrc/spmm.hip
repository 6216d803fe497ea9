// spmm.hip — merge-path CSR SpMM (C = A B, dense B/C row-major) for gfx950,
// the FLAGSPARSE_SPMM_KERNEL=merge variant (the default kernel and the C-ABI
// entry points are in spmm_group.hip).
//
// Replaces the reference's base SpMM (spmm_csr.py:2684-2789 with
// _spmm_csr_real_kernel / _spmm_csr_complex_kernel, spmm_csr.py:134-237)
// and the long-row split + deterministic reduce of the opt path
// (spmm_csr.py:2968-3109).
//
// Each wave owns one merge-path tile of kSpmmTile items (row ends + nnz)
// and one column tile of 64*VEC columns.  The walk through the tile is
// wave-uniform: the sparse value / column of each nnz is a scalar, and each
// lane gathers VEC consecutive elements of the B row it names.  Gathers are
// issued kBatch at a time so several B rows are in flight per wave.  Row
// sums stay in registers (fp64 for fp32/complex64 inputs, as the reference
// upcasts fp32 data and B to fp64, spmm_csr.py:2720-2759).  A row that
// starts in an earlier tile writes its in-tile part to `head`, the last
// open row of a tile writes to `tail`, and spmm_fixup_kernel adds them in
// tile order: deterministic, no floating-point atomics.
#include "fs_common.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace fs {

constexpr int kSpmmTile = 512;  // merge items per tile (rows + nnz)
constexpr int kBatch = 8;       // B rows gathered per batch

template <class V, int VEC>
struct Frag {
  typename VT<V>::acc a[VEC];
};

template <class V, int VEC>
__device__ inline void load_row(const V* __restrict__ p, int valid, V (&out)[VEC]) {
  // valid: number of in-range elements for this lane (0..VEC)
  if (valid == VEC) {
    if constexpr (sizeof(V) * VEC == 16) {
      using L = __attribute__((ext_vector_type(4))) unsigned int;
      L q = *reinterpret_cast<const L*>(p);
      __builtin_memcpy(out, &q, 16);
    } else if constexpr (sizeof(V) * VEC == 8) {
      using L = __attribute__((ext_vector_type(2))) unsigned int;
      L q = *reinterpret_cast<const L*>(p);
      __builtin_memcpy(out, &q, 8);
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k) out[k] = p[k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      if (k < valid) out[k] = p[k];
  }
}

// Broadcast lane `lane` of a per-lane value to the whole wave (the index is
// wave-uniform, so this is one v_readlane per dword into scalar registers).
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

// Gathers per batch (double buffered, so 2x this many B rows per wave are
// in flight).
template <class V, int VEC>
constexpr int spmm_batch() {
  return 4;  // measured best on MI355X for N = 32 .. 256 (8 within 3%)
}

// One wave per merge-path tile.  The tile's nnz (<= kSpmmTile) are staged 64
// at a time in lane registers (coalesced loads, next chunk prefetched) and
// broadcast with readlane; row ends are staged the same way.  B-row gathers
// are double buffered: batch k+1 is issued before batch k is accumulated,
// so a wave keeps up to 2*U*G gathers in flight.
//
// G = 2 splits the wave into two 32-lane halves for narrow B (at most
// 32*VEC columns per column tile): each step takes a pair of nnz, the lower
// half gathers the B row of the even one and the upper half that of the odd
// one, so every gather instruction uses all 64 lanes.  The walk stays
// wave-uniform: a row end between the two nnz of a pair is handled between
// the two predicated accumulations, and a row's sum is the sum of the two
// halves' accumulators (one cross-half permute per row).
// Minimum waves per SIMD asked of the register allocator.  4-byte values
// and column indices, one column per lane, one lane group and 4 gathers per
// batch fit in 64 VGPRs without spilling, i.e. 8 waves instead of 7
// (1M x 1M, 32 per row, N = 64: 1.439 -> 1.342 ms).  Elsewhere the
// allocator keeps its choice: 64 VGPRs would spill there (int64 indices,
// two lane groups, 8 gathers per batch), and wider lanes lose more to L2
// thrashing than they gain (R-MAT N = 256 at 6 / 8 waves: 5.65 -> 5.89 /
// 8.06 ms; complex64 N = 32: 2.04 -> 3.33 / 6.15 ms).
template <class V, int VEC, int U, int G, class I>
constexpr int spmm_min_waves() {
  return (sizeof(V) == 4 && sizeof(I) == 4 && VEC == 1 && U == 4 && G == 1) ? 8 : 1;
}

template <class V, int VEC, int U, int G, class I, class P>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(spmm_min_waves<V, VEC, U, G, I>()))) void spmm_merge_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ B, int64_t ldb, V* __restrict__ C, int64_t ldc, int64_t n_dense,
    const int64_t* __restrict__ part, typename VT<V>::acc* __restrict__ head,
    typename VT<V>::acc* __restrict__ tail, int64_t n_rows, int64_t nnz, int64_t n_tiles, int xcd_cols) {
  static_assert(G == 1 || G == 2, "one or two lane groups per wave");
  using T = VT<V>;
  using A = typename T::acc;
  constexpr int LG = 64 / G;  // lanes per group
  const int lane = threadIdx.x & 63;
  const int grp = G == 1 ? 0 : lane / LG;
  const int gl = lane % LG;
  // Column tile and tile block.  With xcd_cols > 0 the grid is 1-D and
  // column tile = workgroup id % xcd_cols: workgroups go to the 8 XCDs
  // round-robin, so (for xcd_cols a power of two up to 8) each XCD always
  // works on the same slice of B's columns and its L2 keeps the hot rows of
  // that slice.
  const int64_t ctile = xcd_cols > 0 ? (int64_t)(blockIdx.x % (unsigned)xcd_cols) : (int64_t)blockIdx.y;
  const int64_t tblk = xcd_cols > 0 ? (int64_t)(blockIdx.x / (unsigned)xcd_cols) : (int64_t)blockIdx.x;
  const int64_t t = tblk * 4 + (threadIdx.x >> 6);
  if (t >= n_tiles) return;  // wave-uniform, no barriers below
  const int64_t col0 = ctile * LG * VEC + (int64_t)gl * VEC;
  const int64_t vrem = n_dense - col0;
  const int valid = vrem <= 0 ? 0 : (vrem >= VEC ? VEC : (int)vrem);

  const int64_t r0 = part[t];
  const int64_t r1 = part[t + 1];
  const int64_t d0 = t * kSpmmTile;
  const int64_t total = n_rows + nnz;
  const int64_t dend = d0 + kSpmmTile < total ? d0 + kSpmmTile : total;
  const int64_t n0 = d0 - r0;
  const int nz = (int)(dend - r1 - n0);  // nnz in the tile
  const int R = (int)(r1 - r0);          // row ends in the tile
  const bool head_partial = R > 0 && (int64_t)rowptr[r0] < n0;

  // nnz chunks (current + prefetched next)
  I colC, colN;
  V valC, valN;
  auto load_chunk = [&](int ch, I& cc, V& vv) {
    const int q = ch * 64 + lane;
    cc = 0;
    vv = V{};
    if (q < nz) {
      cc = cols[n0 + q];
      vv = vals[n0 + q];
    }
  };
  load_chunk(0, colC, valC);
  load_chunk(1, colN, valN);
  int chunk = 0;
  // row-end chunks, as offsets from n0
  int reC, reN;
  auto load_re = [&](int base, int& dst) {
    const int k = base + lane;
    dst = k < R ? (int)((int64_t)rowptr[r0 + 1 + k] - n0) : 0x7fffffff;
  };
  load_re(0, reC);
  load_re(64, reN);
  int rbase = 0;
  int row = 0;  // tile-local
  int re = R > 0 ? readlane_any(reC, 0) : 0x7fffffff;
  auto next_row = [&]() {
    ++row;
    if (row - rbase == 64) {
      reC = reN;
      rbase += 64;
      load_re(rbase + 64, reN);
    }
    re = row < R ? readlane_any(reC, row - rbase) : 0x7fffffff;
  };

  A acc[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) acc[k] = T::zero();
  // row total in the lanes of group 0
  auto combine = [&](int k) -> A {
    if constexpr (G == 1) {
      return acc[k];
    } else {
      return add(acc[k], shfl(acc[k], lane ^ 32));
    }
  };
  auto emit = [&]() {
    A s[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) s[k] = combine(k);
    if (valid > 0 && grp == 0) {
      if (row == 0 && head_partial) {
        A* h = head + t * n_dense + col0;
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          if (k < valid) h[k] = s[k];
      } else {
        V* c = C + (r0 + row) * ldc + col0;
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          if (k < valid) c[k] = T::out(s[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = T::zero();
  };

  // Batch kb covers steps [kb*U, kb*U + U); step s covers nnz [s*G, s*G + G).
  auto issue = [&](int kb, V (&bb)[U][VEC], V (&aa)[U]) {
    const int ch = (kb * U * G) >> 6;
    if (ch != chunk) {
      colC = colN;
      valC = valN;
      chunk = ch;
      load_chunk(ch + 1, colN, valN);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = kb * U + u;
      if (s * G < nz) {
        const int li = (s * G) & 63;  // G divides 64: a step never straddles a chunk
        I cc = readlane_any(colC, li);
        V av = readlane_any(valC, li);
        if constexpr (G == 2) {
          const I c1 = readlane_any(colC, li + 1);
          const V a1 = readlane_any(valC, li + 1);
          if (grp) {
            cc = c1;
            av = a1;
          }
        }
        aa[u] = av;
        if (s * G + grp < nz) load_row<V, VEC>(B + (int64_t)cc * ldb + col0, valid, bb[u]);
      }
    }
  };
  auto consume = [&](int kb, V (&bb)[U][VEC], V (&aa)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = kb * U + u;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int q = s * G + g;
        if (q >= nz) break;
        while (re <= q) {  // rows that end before nnz q (empty rows included)
          emit();
          next_row();
        }
        if (grp == g) {
#pragma unroll
          for (int k = 0; k < VEC; ++k) acc[k] = T::fma(aa[u], bb[u][k], acc[k]);
        }
      }
    }
  };

  const int steps = (nz + G - 1) / G;
  const int nb = (steps + U - 1) / U;
  V bA[U][VEC], bB[U][VEC];
  V aA[U], aB[U];
  if (nb > 0) issue(0, bA, aA);
  for (int kb = 0; kb < nb; kb += 2) {
    if (kb + 1 < nb) issue(kb + 1, bB, aB);
    consume(kb, bA, aA);
    if (kb + 1 < nb) {
      if (kb + 2 < nb) issue(kb + 2, bA, aA);
      consume(kb + 1, bB, aB);
    }
  }
  while (row < R) {  // rows ending at the tile's last nnz, and trailing empty rows
    emit();
    next_row();
  }
  if (r1 < n_rows) {
    A s[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) s[k] = combine(k);
    if (valid > 0 && grp == 0) {
      A* tl = tail + t * n_dense + col0;
#pragma unroll
      for (int k = 0; k < VEC; ++k)
        if (k < valid) tl[k] = s[k];
    }
  }
}

// Rows that cross tiles: C[row] = tail[f] + ... + tail[t-1] + head[t].
template <class V>
__global__ __launch_bounds__(256) void spmm_fixup_kernel(
    const void* __restrict__ rowptr_raw, int ptr64, const int64_t* __restrict__ part,
    const typename VT<V>::acc* __restrict__ head, const typename VT<V>::acc* __restrict__ tail,
    V* __restrict__ C, int64_t ldc, int64_t n_dense, int64_t n_tiles) {
  using T = VT<V>;
  using A = typename T::acc;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tiles) return;
  const int64_t r0 = part[t];
  if (part[t + 1] == r0) return;
  const int64_t n0 = t * kSpmmTile - r0;
  const int64_t start = ptr64 ? static_cast<const int64_t*>(rowptr_raw)[r0]
                              : (int64_t) static_cast<const int32_t*>(rowptr_raw)[r0];
  if (start >= n0) return;
  const int64_t f = fixup_start_tile(part, t, r0);
  for (int64_t col = (int64_t)blockIdx.y * 64 + (threadIdx.x & 63); col < n_dense;
       col += (int64_t)gridDim.y * 64) {
    A sum = tail[f * n_dense + col];
    sum = sum_fragments(tail + col, n_dense, f + 1, t, sum);  // in sub-tile order
    sum = add(sum, head[t * n_dense + col]);
    C[r0 * ldc + col] = T::out(sum);
  }
}

int spmm_vec_for(int val_t, int64_t n_dense) {
  const int max_vec = (val_t == FS_C128) ? 1 : 2;
  int vec = 1;
  while (vec < max_vec && n_dense > 64 * vec) vec <<= 1;
  return vec;
}

template <class V, int VEC, int G>
int launch_spmm_vec(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                    const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense,
                    const int64_t* part, int64_t n_tiles, void* ws, hipStream_t stream) {
  using A = typename VT<V>::acc;
  A* head = static_cast<A*>(ws);
  A* tail = head + n_tiles * n_dense;
  const int64_t col_tiles = ceil_div(n_dense, (int64_t)(64 / G) * VEC);
  const int64_t blocks = ceil_div(n_tiles, 4);
  if (blocks > 0x7fffffffLL || col_tiles > 65535) return fail(FS_E_INVALID, "fs_spmm_csr: grid too large");
  // XCD-affine column tiles when B has 2, 4 or 8 of them (C5, N = 256: 5.69
  // against 5.88 ms; neutral elsewhere).  FLAGSPARSE_SPMM_XCD=0/1 forces it.
  int xcd_cols = (col_tiles == 2 || col_tiles == 4 || col_tiles == 8) ? (int)col_tiles : 0;
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_XCD")) xcd_cols = std::atoi(e) != 0 ? (int)col_tiles : 0;
  if (xcd_cols > 0 && blocks * col_tiles > 0x7fffffffLL) xcd_cols = 0;
  dim3 g = xcd_cols > 0 ? dim3((unsigned)(blocks * col_tiles)) : dim3((unsigned)blocks, (unsigned)col_tiles);
  // Residency cap for the two-columns-per-lane kernel: dynamic LDS of
  // (LDS per CU) / cap bytes per workgroup leaves room for `cap` workgroups
  // per CU.  On matrices with skewed columns (R-MAT) fewer concurrent waves
  // keep more hot B rows in L2: 4 per CU instead of 5, N = 256: 5.69 ->
  // 5.43 ms, N = 128: 2.86 -> 2.73 ms.  On uniform columns it costs 7-13%, so
  // the caller sets plan->spmm_wg_cap only for skewed matrices.
  // FLAGSPARSE_SPMM_WG_CAP=N sets the cap for every lane width (A/B runs).
  size_t lds_pad = 0;  // the kernel has no static LDS
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_WG_CAP")) lds_pad = lds_pad_for_cap(std::atoi(e), 0);
  else if (VEC == 2) lds_pad = lds_pad_for_cap(plan->spmm_wg_cap, 0);
  int u = spmm_batch<V, VEC>();
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_U")) u = std::atoi(e);
  auto go = [&](auto icode, auto pcode) {
    using I = std::conditional_t<decltype(icode)::value, int64_t, int32_t>;
    using P = std::conditional_t<decltype(pcode)::value, int64_t, int32_t>;
    auto launch = [&](auto uc) {
      hipLaunchKernelGGL((spmm_merge_kernel<V, VEC, decltype(uc)::value, G, I, P>), g, dim3(256), lds_pad, stream,
                         static_cast<const V*>(vals), static_cast<const I*>(cols), static_cast<const P*>(indptr),
                         static_cast<const V*>(B), ldb, static_cast<V*>(C), ldc, n_dense, part, head, tail,
                         plan->n_rows, plan->nnz, n_tiles, xcd_cols);
    };
    if (u <= 4) launch(std::integral_constant<int, 4>{});
    else launch(std::integral_constant<int, 8>{});
  };
  using T1 = std::true_type;
  using F1 = std::false_type;
  const bool i64 = plan->idx_t == FS_I64, p64 = plan->ptr_t == FS_I64;
  if (i64 && p64) go(T1{}, T1{});
  else if (i64) go(T1{}, F1{});
  else if (p64) go(F1{}, T1{});
  else go(F1{}, F1{});
  FS_CHECK_MAIN_LAUNCH("spmm_merge_kernel");
  const int64_t fix_cols = ceil_div(n_dense, 64) < 64 ? ceil_div(n_dense, 64) : 64;
  hipLaunchKernelGGL((spmm_fixup_kernel<V>), dim3((unsigned)blocks, (unsigned)fix_cols), dim3(256), 0, stream,
                     indptr, plan->ptr_t == FS_I64 ? 1 : 0, part, head, tail, static_cast<V*>(C), ldc, n_dense,
                     n_tiles);
  FS_CHECK_LAUNCH("spmm_fixup_kernel");
  return FS_OK;
}

template <class V, int VEC>
int launch_spmm_g(const fs_csr_plan* plan, int groups, const void* vals, const void* cols, const void* indptr,
                  const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense, const int64_t* part,
                  int64_t n_tiles, void* ws, hipStream_t s) {
  if (groups == 2)
    return launch_spmm_vec<V, VEC, 2>(plan, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
  return launch_spmm_vec<V, VEC, 1>(plan, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
}

template <class V>
int launch_spmm(const fs_csr_plan* plan, int vec, int groups, const void* vals, const void* cols,
                const void* indptr, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense,
                const int64_t* part, int64_t n_tiles, void* ws, hipStream_t s) {
  switch (vec) {
    case 1: return launch_spmm_g<V, 1>(plan, groups, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
    case 2:
      if constexpr (sizeof(V) <= 8)
        return launch_spmm_g<V, 2>(plan, groups, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
      break;
    case 4:
      if constexpr (sizeof(V) == 4)
        return launch_spmm_g<V, 4>(plan, groups, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
      break;
  }
  return fail(FS_E_INVALID, "fs_spmm_csr: unsupported vector width");
}


// Merge-path kernel entry (FLAGSPARSE_SPMM_KERNEL=merge): row-major B / C.
int spmm_merge_dispatch(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                        const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense, const int64_t* part,
                        int64_t n_tiles, void* ws, hipStream_t stream) {
  const size_t vsz[] = {4, 8, 8, 16};
  const size_t esz = vsz[plan->val_t];
  int vec = spmm_vec_for(plan->val_t, n_dense);
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_VEC")) {
    const int v = std::atoi(e);
    if ((v == 1 || v == 2 || v == 4) && (size_t)v * esz <= 16) vec = v;
  }
  // Vector loads need every lane's B/C slice aligned to the vector width.
  while (vec > 1 && ((ldb % vec) || (ldc % vec) || ((uintptr_t)B % (esz * vec)) || ((uintptr_t)C % (esz * vec))))
    vec >>= 1;
  // Narrow B: two 32-lane groups per wave, each gathering its own B row.
  int groups = n_dense <= 32 * vec ? 2 : 1;
  if (const char* e = std::getenv("FLAGSPARSE_SPMM_G")) {
    const int gv = std::atoi(e);
    if (gv == 1 || gv == 2) groups = gv;
  }
  switch (plan->val_t) {
    case FS_F32: return launch_spmm<float>(plan, vec, groups, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
    case FS_F64: return launch_spmm<double>(plan, vec, groups, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
    case FS_C64: return launch_spmm<c32>(plan, vec, groups, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
    default: return launch_spmm<c64>(plan, vec, groups, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
  }
}

}  // namespace fs
