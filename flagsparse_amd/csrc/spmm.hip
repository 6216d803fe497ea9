// spmm.hip — CSR SpMM (C = A B, dense B/C row-major) for gfx950.
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

template <class V, int VEC>
__global__ __launch_bounds__(256) void spmm_merge_kernel(
    const V* __restrict__ vals, const void* __restrict__ cols_raw, int idx64,
    const void* __restrict__ rowptr_raw, int ptr64, const V* __restrict__ B, int64_t ldb,
    V* __restrict__ C, int64_t ldc, int64_t n_dense, const int64_t* __restrict__ part,
    typename VT<V>::acc* __restrict__ head, typename VT<V>::acc* __restrict__ tail,
    int64_t n_rows, int64_t nnz, int64_t n_tiles) {
  using T = VT<V>;
  using A = typename T::acc;
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tiles) return;  // wave-uniform, no barriers below
  const int64_t col0 = (int64_t)blockIdx.y * 64 * VEC + (int64_t)lane * VEC;
  int64_t vrem = n_dense - col0;
  const int valid = vrem <= 0 ? 0 : (vrem >= VEC ? VEC : (int)vrem);

  const int32_t* rp32 = static_cast<const int32_t*>(rowptr_raw);
  const int64_t* rp64 = static_cast<const int64_t*>(rowptr_raw);
  const int32_t* ci32 = static_cast<const int32_t*>(cols_raw);
  const int64_t* ci64 = static_cast<const int64_t*>(cols_raw);
  auto rowptr = [&](int64_t r) -> int64_t { return ptr64 ? rp64[r] : (int64_t)rp32[r]; };
  auto colidx = [&](int64_t j) -> int64_t { return idx64 ? ci64[j] : (int64_t)ci32[j]; };

  const int64_t r0 = part[t];
  const int64_t r1 = part[t + 1];
  const int64_t d0 = t * kSpmmTile;
  const int64_t total = n_rows + nnz;
  const int64_t dend = d0 + kSpmmTile < total ? d0 + kSpmmTile : total;
  const int64_t n0 = d0 - r0;
  const int64_t n1 = dend - r1;
  const bool head_partial = r1 > r0 && rowptr(r0) < n0;

  A acc[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) acc[k] = T::zero();

  int64_t row = r0;
  int64_t re = row < r1 ? rowptr(row + 1) : n1;  // end of the current row inside the tile

  auto emit = [&](int64_t r) {
    if (valid > 0) {
      if (r == r0 && head_partial) {
        A* h = head + t * n_dense + col0;
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          if (k < valid) h[k] = acc[k];
      } else {
        V* c = C + r * ldc + col0;
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          if (k < valid) c[k] = T::out(acc[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = T::zero();
  };

  for (int64_t jb = n0; jb < n1; jb += kBatch) {
    V a[kBatch];
    int64_t c[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t j = jb + u;
      a[u] = V{};
      c[u] = 0;
      if (j < n1) {
        a[u] = vals[j];
        c[u] = colidx(j);
      }
    }
    V b[kBatch][VEC];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (jb + u < n1) load_row<V, VEC>(B + c[u] * ldb + col0, valid, b[u]);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t j = jb + u;
      if (j >= n1) break;
      while (row < r1 && re <= j) {  // rows ending before nnz j (incl. empty rows)
        emit(row);
        ++row;
        re = row < r1 ? rowptr(row + 1) : n1;
      }
#pragma unroll
      for (int k = 0; k < VEC; ++k) acc[k] = T::fma(a[u], b[u][k], acc[k]);
    }
  }
  while (row < r1) {  // rows ending at the tile's last nnz, and trailing empty rows
    emit(row);
    ++row;
  }
  if (r1 < n_rows && valid > 0) {
    A* tl = tail + t * n_dense + col0;
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      if (k < valid) tl[k] = acc[k];
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
  int64_t f = t - 1;
  while (f > 0 && part[f] == r0) --f;
  for (int64_t col = (int64_t)blockIdx.y * 64 + (threadIdx.x & 63); col < n_dense;
       col += (int64_t)gridDim.y * 64) {
    A sum = tail[f * n_dense + col];
    for (int64_t k = f + 1; k < t; ++k) sum = add(sum, tail[k * n_dense + col]);
    sum = add(sum, head[t * n_dense + col]);
    C[r0 * ldc + col] = T::out(sum);
  }
}

int spmm_vec_for(int val_t, int64_t n_dense) {
  const int max_vec = (val_t == FS_F32) ? 4 : (val_t == FS_C128 ? 1 : 2);
  int vec = 1;
  while (vec < max_vec && n_dense > 64 * vec) vec <<= 1;
  return vec;
}

template <class V, int VEC>
int launch_spmm_vec(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                    const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense,
                    const int64_t* part, int64_t n_tiles, void* ws, hipStream_t stream) {
  using A = typename VT<V>::acc;
  A* head = static_cast<A*>(ws);
  A* tail = head + n_tiles * n_dense;
  const int64_t col_tiles = ceil_div(n_dense, 64 * VEC);
  const int64_t blocks = ceil_div(n_tiles, 4);
  if (blocks > 0x7fffffffLL || col_tiles > 65535) return fail(FS_E_INVALID, "fs_spmm_csr: grid too large");
  hipLaunchKernelGGL((spmm_merge_kernel<V, VEC>), dim3((unsigned)blocks, (unsigned)col_tiles), dim3(256), 0,
                     stream, static_cast<const V*>(vals), cols, plan->idx_t == FS_I64 ? 1 : 0, indptr,
                     plan->ptr_t == FS_I64 ? 1 : 0, static_cast<const V*>(B), ldb, static_cast<V*>(C), ldc,
                     n_dense, part, head, tail, plan->n_rows, plan->nnz, n_tiles);
  FS_CHECK_LAUNCH("spmm_merge_kernel");
  const int64_t fix_cols = ceil_div(n_dense, 64) < 64 ? ceil_div(n_dense, 64) : 64;
  hipLaunchKernelGGL((spmm_fixup_kernel<V>), dim3((unsigned)blocks, (unsigned)fix_cols), dim3(256), 0, stream,
                     indptr, plan->ptr_t == FS_I64 ? 1 : 0, part, head, tail, static_cast<V*>(C), ldc, n_dense,
                     n_tiles);
  FS_CHECK_LAUNCH("spmm_fixup_kernel");
  return FS_OK;
}

template <class V>
int launch_spmm(const fs_csr_plan* plan, int vec, const void* vals, const void* cols, const void* indptr,
                const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense, const int64_t* part,
                int64_t n_tiles, void* ws, hipStream_t s) {
  switch (vec) {
    case 1: return launch_spmm_vec<V, 1>(plan, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
    case 2:
      if constexpr (sizeof(V) <= 8)
        return launch_spmm_vec<V, 2>(plan, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
      break;
    case 4:
      if constexpr (sizeof(V) == 4)
        return launch_spmm_vec<V, 4>(plan, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, s);
      break;
  }
  return fail(FS_E_INVALID, "fs_spmm_csr: unsupported vector width");
}

}  // namespace fs

using namespace fs;

extern "C" int fs_spmm_tile_items(int val_t, int64_t n_dense) {
  (void)val_t;
  (void)n_dense;
  return kSpmmTile;
}

extern "C" size_t fs_spmm_workspace_bytes(int val_t, int64_t n_tiles, int64_t n_dense) {
  const size_t acc = (val_t == FS_C64 || val_t == FS_C128) ? sizeof(c64) : sizeof(double);
  return (size_t)n_tiles * (size_t)n_dense * 2 * acc;
}

extern "C" int fs_spmm_csr(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                           const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense,
                           const void* part_dev, int tile_items, int64_t n_tiles, void* ws, size_t ws_bytes,
                           hipStream_t stream) {
  if (!plan) return fail(FS_E_INVALID, "fs_spmm_csr: plan is null");
  if (!valid_types(plan->val_t, plan->idx_t, plan->ptr_t)) return fail(FS_E_INVALID, "fs_spmm_csr: bad type code");
  if (n_dense < 0 || ldb < 0 || ldc < 0) return fail(FS_E_INVALID, "fs_spmm_csr: negative size");
  if (plan->n_rows == 0 || n_dense == 0) return FS_OK;
  if (tile_items != kSpmmTile) return fail(FS_E_INVALID, "fs_spmm_csr: tile_items must come from fs_spmm_tile_items");
  if (n_tiles != ceil_div(plan->n_rows + plan->nnz, kSpmmTile))
    return fail(FS_E_INVALID, "fs_spmm_csr: n_tiles does not match the matrix");
  if (ldc < n_dense || (plan->n_cols > 0 && ldb < n_dense))
    return fail(FS_E_INVALID, "fs_spmm_csr: leading dimension smaller than n_dense");
  if (!indptr || !C || !part_dev || (plan->nnz > 0 && (!vals || !cols || !B)))
    return fail(FS_E_INVALID, "fs_spmm_csr: null pointer");
  if (ws_bytes < fs_spmm_workspace_bytes(plan->val_t, n_tiles, n_dense) || (!ws && n_tiles > 0))
    return fail(FS_E_WORKSPACE, "fs_spmm_csr: workspace too small");
  int vec = spmm_vec_for(plan->val_t, n_dense);
  // Vector loads need every lane's B/C slice aligned to the vector width.
  const size_t vsz[] = {4, 8, 8, 16};
  const size_t esz = vsz[plan->val_t];
  while (vec > 1 && ((ldb % vec) || (ldc % vec) || ((uintptr_t)B % (esz * vec)) || ((uintptr_t)C % (esz * vec))))
    vec >>= 1;
  const int64_t* part = static_cast<const int64_t*>(part_dev);
  switch (plan->val_t) {
    case FS_F32: return launch_spmm<float>(plan, vec, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
    case FS_F64: return launch_spmm<double>(plan, vec, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
    case FS_C64: return launch_spmm<c32>(plan, vec, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
    default: return launch_spmm<c64>(plan, vec, vals, cols, indptr, B, ldb, C, ldc, n_dense, part, n_tiles, ws, stream);
  }
}
