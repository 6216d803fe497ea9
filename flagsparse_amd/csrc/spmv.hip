// spmv.hip — CSR SpMV for gfx950: analysis, merge-path partition, and the
// two SpMV kernel families.
//
// Reference behaviour being replaced (NCIC-AlphaSparse/FlagSparse):
//   _spmv_csr_real_kernel / _spmv_csr_complex_kernel   spmv_csr.py:166-227
//   opt CSR-Vector buckets                             spmv_csr.py:233-461
//   prepare_spmv_csr block/segment sizing              spmv_csr.py:591-664
// The reference walks every row for ceil(max_row/BLOCK) segments; here the
// work is either one short vector per row (regular matrices) or an
// nnz+row balanced merge path (any matrix), so a 50,000-nnz row costs the
// same per item as a 10-nnz row.
#include "fs_common.hpp"

#include <algorithm>
#include <type_traits>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace fs {

// ---------------------------------------------------------------------------
// Row-length statistics (input to the host-side kernel choice).
// stats layout (uint64): [0..FS_HIST_BINS) histogram, [FS_HIST_BINS] max,
// [FS_HIST_BINS+1] min.
// ---------------------------------------------------------------------------
constexpr int kStatsWords = FS_HIST_BINS + 2;

__global__ void stats_init_kernel(unsigned long long* stats) {
  int k = threadIdx.x;
  if (k < kStatsWords) stats[k] = (k == FS_HIST_BINS + 1) ? ~0ull : 0ull;
}

// Row-length statistics of the rows this thread's wave visits: LDS
// histogram by bit length, max / min length, and (COUNT_BAD) the rows whose
// pointer decreases.
template <class P, bool COUNT_BAD>
__device__ inline void stats_rows(const P* __restrict__ rowptr, int64_t n_rows, unsigned int* s_hist,
                                  unsigned long long& vmax, unsigned long long& vmin, unsigned long long& bad) {
  static_assert(FS_HIST_BINS <= 32, "bins are grouped with 5 ballots");
  // Whole waves run every iteration (the bound is wave-uniform), so the
  // ballots below see every active lane.
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t first = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~63);
  // kStatsUnroll rows per lane per step, all loads issued before any is used:
  // with a few hundred workgroups, one dependent pair of loads per step left
  // the kernel latency-bound (88 us for 4 M rows).
  constexpr int kStatsUnroll = 8;
  for (int64_t r0 = first; r0 < n_rows; r0 += kStatsUnroll * stride) {
    int64_t lens[kStatsUnroll];
    bool valids[kStatsUnroll];
#pragma unroll
    for (int u = 0; u < kStatsUnroll; ++u) {
      const int64_t r = r0 + u * stride + (threadIdx.x & 63);
      valids[u] = r < n_rows;
      lens[u] = valids[u] ? (int64_t)rowptr[r + 1] - (int64_t)rowptr[r] : 0;
    }
#pragma unroll
    for (int u = 0; u < kStatsUnroll; ++u) {
      const bool valid = valids[u];
      if constexpr (COUNT_BAD) bad += (valid && lens[u] < 0) ? 1ull : 0ull;
      const unsigned long long len = (unsigned long long)lens[u];
      int bin = len == 0 ? 0 : (64 - __clzll(len));
      bin = bin < FS_HIST_BINS ? bin : FS_HIST_BINS - 1;
      // lanes with the same bin: one of them adds the group's count
      unsigned long long peers = __ballot(valid);
      if (peers == 0) continue;  // wave-uniform
#pragma unroll
      for (int b = 0; b < 5; ++b) {
        const bool bit = (bin >> b) & 1;
        const unsigned long long m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
      const int below = __builtin_amdgcn_mbcnt_hi((unsigned)(peers >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)peers, 0u));
      if (valid && below == 0) atomicAdd(&s_hist[bin], (unsigned)__popcll(peers));
      if (valid) {
        vmax = len > vmax ? len : vmax;
        vmin = len < vmin ? len : vmin;
      }
    }
  }
}

// Max / min over the workgroup first (wave butterflies, then 4 partials in
// LDS), so each workgroup issues one global atomic per statistic: a global
// atomic per thread on one address serialises in L2.  Integer max / min /
// count are order independent, so the result is deterministic.  All
// threads call it (it has a barrier); s_hist must be complete.
__device__ inline void stats_flush(unsigned long long vmax, unsigned long long vmin, const unsigned int* s_hist,
                                   unsigned long long* stats) {
  __shared__ unsigned long long s_max[4], s_min[4];
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long omax = __shfl_xor(vmax, off);
    const unsigned long long omin = __shfl_xor(vmin, off);
    vmax = omax > vmax ? omax : vmax;
    vmin = omin < vmin ? omin : vmin;
  }
  if ((threadIdx.x & 63) == 0) {
    s_max[threadIdx.x >> 6] = vmax;
    s_min[threadIdx.x >> 6] = vmin;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long bmax = s_max[0], bmin = s_min[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
      bmax = s_max[w] > bmax ? s_max[w] : bmax;
      bmin = s_min[w] < bmin ? s_min[w] : bmin;
    }
    atomicMax(&stats[FS_HIST_BINS], bmax);
    atomicMin(&stats[FS_HIST_BINS + 1], bmin);
  }
  if (threadIdx.x < FS_HIST_BINS && s_hist[threadIdx.x])
    atomicAdd(&stats[threadIdx.x], (unsigned long long)s_hist[threadIdx.x]);
}

template <class P>
__global__ __launch_bounds__(256) void stats_kernel(const P* __restrict__ rowptr,
                                                    int64_t n_rows,
                                                    unsigned long long* stats) {
  __shared__ unsigned int s_hist[FS_HIST_BINS];
  if (threadIdx.x < FS_HIST_BINS) s_hist[threadIdx.x] = 0;
  __syncthreads();
  unsigned long long vmax = 0, vmin = ~0ull, bad = 0;
  stats_rows<P, false>(rowptr, n_rows, s_hist, vmax, vmin, bad);
  __syncthreads();
  stats_flush(vmax, vmin, s_hist, stats);
}

// ---------------------------------------------------------------------------
// Structure check: indptr[0], indptr[n_rows], whether any row pointer
// decreases, and the column range, in one pass over indptr and indices.
// check layout (uint64): [0] indptr[0], [1] indptr[n_rows], [2] rows whose
// pointer decreases, [3] min column, [4] max column; the columns are stored
// with the sign bit flipped so that the unsigned atomics order signed values.
// ---------------------------------------------------------------------------

template <class P>
__global__ void check_init_kernel(const P* __restrict__ rowptr, int64_t n_rows, unsigned long long* check) {
  const int k = threadIdx.x;
  if (k == 0) check[0] = (unsigned long long)(int64_t)rowptr[0];
  if (k == 1) check[1] = (unsigned long long)(int64_t)rowptr[n_rows];
  if (k == 2) check[2] = 0ull;
  if (k == 3) check[3] = ~0ull;
  if (k == 4) check[4] = 0ull;
}

template <class I>
__device__ inline void check_range(I c, unsigned long long& lo, unsigned long long& hi) {
  const unsigned long long v = (unsigned long long)(int64_t)c ^ kSignFlip;
  lo = v < lo ? v : lo;
  hi = v > hi ? v : hi;
}

// VEC: the indices are 16-byte aligned and read as 16-byte vectors, eight
// per lane in flight (128 bytes; 4-byte loads left the pass at 3.3 TB/s).
// Min / max column over this thread's share of the indices.
template <class I, bool VEC>
__device__ inline void check_cols(const I* __restrict__ cols, int64_t nnz, unsigned long long& lo,
                                  unsigned long long& hi) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t done = 0;  // leading entries covered by the vector loop
  if constexpr (VEC) {
    constexpr int W = 16 / sizeof(I);
    typedef I vec_t __attribute__((ext_vector_type(W)));
    const vec_t* cv = reinterpret_cast<const vec_t*>(cols);
    const int64_t nv = nnz / W;
    int64_t k = tid;
    for (; k + 7 * stride < nv; k += 8 * stride) {
      vec_t c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = __builtin_nontemporal_load(cv + k + u * stride);
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int w = 0; w < W; ++w) check_range<I>(c[u][w], lo, hi);
    }
    for (; k < nv; k += stride) {
      const vec_t c = __builtin_nontemporal_load(cv + k);
#pragma unroll
      for (int w = 0; w < W; ++w) check_range<I>(c[w], lo, hi);
    }
    done = nv * W;
  }
  for (int64_t k = done + tid; k < nnz; k += stride) check_range<I>(__builtin_nontemporal_load(cols + k), lo, hi);
}

// Workgroup reduction of (bad rows, min, max column), then one global atomic
// each.  All threads call it (it has a barrier).
__device__ inline void check_flush(unsigned long long bad, unsigned long long lo, unsigned long long hi, int64_t nnz,
                                   unsigned long long* check) {
  for (int off = 32; off > 0; off >>= 1) {
    bad += __shfl_xor(bad, off);
    const unsigned long long olo = __shfl_xor(lo, off), ohi = __shfl_xor(hi, off);
    lo = olo < lo ? olo : lo;
    hi = ohi > hi ? ohi : hi;
  }
  __shared__ unsigned long long s_bad[4], s_lo[4], s_hi[4];
  if ((threadIdx.x & 63) == 0) {
    s_bad[threadIdx.x >> 6] = bad;
    s_lo[threadIdx.x >> 6] = lo;
    s_hi[threadIdx.x >> 6] = hi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
      bad += s_bad[w];
      lo = s_lo[w] < lo ? s_lo[w] : lo;
      hi = s_hi[w] > hi ? s_hi[w] : hi;
    }
    if (bad) atomicAdd(&check[2], bad);
    if (nnz > 0) {
      atomicMin(&check[3], lo);
      atomicMax(&check[4], hi);
    }
  }
}

// VEC: the indices are 16-byte aligned and read as 16-byte vectors, eight
// per lane in flight (128 bytes; 4-byte loads left the pass at 3.3 TB/s).
template <class P, class I, bool VEC>
__global__ __launch_bounds__(256) void check_kernel(const P* __restrict__ rowptr, int64_t n_rows,
                                                    const I* __restrict__ cols, int64_t nnz,
                                                    unsigned long long* check) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long bad = 0;
  for (int64_t r = tid; r < n_rows; r += stride)
    bad += __builtin_nontemporal_load(rowptr + r + 1) < __builtin_nontemporal_load(rowptr + r) ? 1ull : 0ull;
  unsigned long long lo = ~0ull, hi = 0;
  check_cols<I, VEC>(cols, nnz, lo, hi);
  check_flush(bad, lo, hi, nnz, check);
}

// Structure check and row-length statistics in one pass (the row pointer is
// read once, for both): check words as check_kernel, statistics as
// stats_kernel.
template <class P, class I, bool VEC>
__global__ __launch_bounds__(256) void check_stats_kernel(const P* __restrict__ rowptr, int64_t n_rows,
                                                          const I* __restrict__ cols, int64_t nnz,
                                                          unsigned long long* check, unsigned long long* stats) {
  __shared__ unsigned int s_hist[FS_HIST_BINS];
  if (threadIdx.x < FS_HIST_BINS) s_hist[threadIdx.x] = 0;
  __syncthreads();
  unsigned long long vmax = 0, vmin = ~0ull, bad = 0;
  stats_rows<P, true>(rowptr, n_rows, s_hist, vmax, vmin, bad);
  unsigned long long lo = ~0ull, hi = 0;
  check_cols<I, VEC>(cols, nnz, lo, hi);
  check_flush(bad, lo, hi, nnz, check);  // its barrier also completes s_hist
  if (n_rows > 0) stats_flush(vmax, vmin, s_hist, stats);
}

// ---------------------------------------------------------------------------
// Merge-path partition.  The merge path interleaves the row-end offsets
// (rowptr[1..n_rows]) with the nnz indices 0..nnz-1; a row end is consumed
// before nnz j when rowptr[i+1] <= j.  Tile t starts at diagonal t*T; part[t]
// is the number of row ends consumed before that diagonal.
// ---------------------------------------------------------------------------
template <class P>
__global__ __launch_bounds__(256) void partition_kernel(const P* __restrict__ rowptr,
                                                        int64_t n_rows, int64_t nnz,
                                                        int64_t tile_items, int64_t n_tiles,
                                                        int64_t* __restrict__ part) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t > n_tiles) return;
  int64_t diag = t * tile_items;
  int64_t total = n_rows + nnz;
  diag = diag < total ? diag : total;
  int64_t lo = diag - nnz > 0 ? diag - nnz : 0;
  int64_t hi = diag < n_rows ? diag : n_rows;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if ((int64_t)rowptr[mid + 1] <= diag - mid - 1)
      lo = mid + 1;
    else
      hi = mid;
  }
  part[t] = lo;
}

// ---------------------------------------------------------------------------
// K1: vector-per-row.  VW lanes share a row; each lane walks the row with
// stride VW and issues kUnroll loads before using any of them, so a wave
// keeps (64/VW rows) x kUnroll value/index loads and x gathers in flight.
// Products accumulate in the accumulator type and are combined with a DPP /
// ds_swizzle butterfly.
// ---------------------------------------------------------------------------
constexpr int kUnroll = 4;
constexpr int kXcds = 8;  // MI355X: workgroup w is dispatched to XCD w % 8

// Logical workgroup index.  With remap, the grid (padded to a multiple of 8)
// is split into 8 contiguous ranges and XCD k walks range k in order, so the
// rows an XCD works on at any moment are adjacent and their x slice stays
// in that XCD's L2.  Returns -1 for padding workgroups.
__device__ inline int64_t logical_block(int remap, int64_t n_blocks) {
  if (!remap) return blockIdx.x;
  const int64_t per = (n_blocks + kXcds - 1) / kXcds;
  const int64_t b = (int64_t)(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  return b < n_blocks ? b : -1;
}

template <int VW, class V, class I, class P>
__global__ __launch_bounds__(256) void spmv_vector_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, V* __restrict__ y, int64_t n_rows, int64_t n_blocks, int remap) {
  using T = VT<V>;
  using A = typename T::acc;
  const int64_t blk = logical_block(remap, n_blocks);
  if (blk < 0) return;
  const int64_t gid = blk * blockDim.x + threadIdx.x;
  const int64_t row = gid / VW;
  const int sub = threadIdx.x & (VW - 1);
  if (row >= n_rows) return;  // whole VW-group leaves together
  const int64_t s = (int64_t)rowptr[row];
  const int64_t e = (int64_t)rowptr[row + 1];
  A acc = T::zero();
  for (int64_t j = s + sub; j < e; j += kUnroll * VW) {
    V v[kUnroll];
    I c[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t jj = j + (int64_t)u * VW;
      c[u] = 0;
      if (jj < e) {
        v[u] = vals[jj];
        c[u] = cols[jj];
      }
    }
    V xv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (j + (int64_t)u * VW < e) xv[u] = x[c[u]];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (j + (int64_t)u * VW < e) acc = T::fma(v[u], xv[u], acc);
  }
  if constexpr (VW <= 32) {
    acc = group_sum<VW>(acc);
  } else {
    acc = group_sum<32>(acc);
    acc = add(acc, shfl(acc, (threadIdx.x & 63) ^ 32));
  }
  if (sub == 0) y[row] = T::out(acc);
}

// ---------------------------------------------------------------------------
// K3: row-block streaming SpMV for matrices whose rows are all short.
//
// A workgroup owns R = 256/TPR consecutive rows, whose nnz form one
// contiguous range of at most stream_items(A) entries.  The 256 threads
// stream that range with unit stride (every load instruction covers
// consecutive addresses), gather x, and stage the products in LDS; then
// TPR threads per row add the row's products and combine them with a DPP
// butterfly.  The plan picks R so that R * max_row fits the LDS stage.
// ---------------------------------------------------------------------------
template <class A>
constexpr int stream_items() {
  return 16384 / (int)sizeof(A);
}

// One workgroup per row block.
template <int TPR, class V, class I, class P>
__global__ __launch_bounds__(256) void spmv_stream_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, V* __restrict__ y, int64_t n_rows, int64_t n_blocks, int remap) {
  using T = VT<V>;
  using A = typename T::acc;
  constexpr int R = 256 / TPR;
  constexpr int kItems = stream_items<A>();
  constexpr int K = kItems / 256;
  __shared__ A s_prod[kItems];
  __shared__ int64_t s_ptr[R + 1];
  const int t = threadIdx.x;
  const int64_t blk = logical_block(remap, n_blocks);
  if (blk < 0) return;  // whole workgroup
  const int64_t rb0 = blk * R;
  const int rows = n_rows - rb0 < R ? (int)(n_rows - rb0) : R;
  for (int k = t; k <= rows; k += 256) s_ptr[k] = (int64_t)rowptr[rb0 + k];  // rows + 1 pointers
  const int64_t S = (int64_t)rowptr[rb0];
  const int cnt = (int)((int64_t)rowptr[rb0 + rows] - S);
  V v[K];
  I c[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int q = t + 256 * k;
    c[k] = 0;
    if (q < cnt) {
      v[k] = vals[S + q];
      c[k] = cols[S + q];
    }
  }
  V xv[K];
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (t + 256 * k < cnt) xv[k] = x[c[k]];
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (t + 256 * k < cnt) s_prod[t + 256 * k] = T::mul(v[k], xv[k]);
  __syncthreads();
  const int r = t / TPR;
  const int sub = t % TPR;
  A acc = T::zero();
  if (r < rows) {
    const int a = (int)(s_ptr[r] - S);
    const int b = (int)(s_ptr[r + 1] - S);
    for (int q = a + sub; q < b; q += TPR) acc = add(acc, s_prod[q]);
  }
  if constexpr (TPR > 1) acc = group_sum<TPR>(acc);
  if (sub == 0 && r < rows) store_stream(y + rb0 + r, T::out(acc));  // measured 2% faster than a plain store
}

// ---------------------------------------------------------------------------
// K3t: row-block SpMV with a slot-order x gather, for blocks of 64 short rows.
//
// The load phase is K3's: the 256 threads stream the block's entries with
// unit stride, but stage (column, value) pairs in LDS instead of products.
// Then wave w takes rows 16w..16w+15 and lane l works on row 16w + (l & 15)
// with sub-lane s = l >> 4, walking the row's entries s, s+4, s+8, ...  So
// for each gather instruction the 16 lanes of one sub-lane hold the same
// entry slot of 16 consecutive rows: on a stencil (or any matrix whose
// neighbouring rows have neighbouring columns) those are 16 consecutive x
// entries, where K3's entry-order gather spreads a wave over ~2 rows' worth
// of scattered offsets.  Each row's four partial sums combine over lanes
// l, l^16, l^32 in a fixed order: deterministic.
// ---------------------------------------------------------------------------
// LDS layout of K3t for a stage of `stage` entries: values, then column
// indices (16-byte aligned), then the 65 row offsets.  With direct-to-LDS
// staging (DL) each array starts at the 16-byte boundary at or below the
// block's first entry and ends at one at or above its last, so it holds up
// to two 16-byte chunks more.
struct StreamTLayout {
  size_t col_off, off_off, total;
};
__host__ __device__ inline StreamTLayout stream_t_layout(int stage, size_t vsz, size_t isz, bool dl) {
  const size_t nv = (size_t)stage + (dl ? 2 * (16 / vsz) : 0);
  const size_t ni = (size_t)stage + (dl ? 2 * (16 / isz) : 0);
  StreamTLayout L;
  L.col_off = (nv * vsz + 15) & ~(size_t)15;
  L.off_off = (L.col_off + ni * isz + 15) & ~(size_t)15;
  L.total = L.off_off + 65 * sizeof(int);
  return L;
}

// Copy 16-byte chunks [0, n) of g into LDS (chunk c to dst + 16 c) with
// direct global-to-LDS loads: wave w of NW takes chunks (k NW + w) 64 + lane.
// The data never passes through VGPRs and no LDS store is issued.
template <int NW, int KC>
__device__ inline void lds_copy16(const unsigned char* g, unsigned char* dst, int n) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c0 = (k * NW + w) * 64;  // wave-uniform
    if (c0 >= n) break;
    if (c0 + lane < n)
      __builtin_amdgcn_global_load_lds((const void*)(g + (size_t)(c0 + lane) * 16),
                                       (__attribute__((address_space(3))) void*)(dst + (size_t)c0 * 16), 16, 0, 0);
  }
}

// One lane's walk over its slots of a staged row [a, b): entries sub,
// sub + SUBS, ... into four partial sums, four slots per step.  A step past
// the row's end reads its last entry again (an index clamped to b - 1), so
// every LDS read and gather is issued unconditionally and all four gathers
// are in flight together; the sums of such slots are computed and dropped,
// so each partial sum adds exactly the row's own slots, in order.  `guard`
// maps each column before its gather.
template <int SUBS, class T, class V, class I, class A, class G>
__device__ inline void slot_walk(const I* sc, const V* sv, const V* __restrict__ x, int a, int b, int sub, A& acc0,
                                 A& acc1, A& acc2, A& acc3, G guard) {
  const int e = b - 1;
  for (int q = a + sub; q < b; q += 4 * SUBS) {
    const int q1 = q + SUBS < e ? q + SUBS : e, q2 = q + 2 * SUBS < e ? q + 2 * SUBS : e,
              q3 = q + 3 * SUBS < e ? q + 3 * SUBS : e;
    const I c0 = guard(sc[q]), c1 = guard(sc[q1]), c2 = guard(sc[q2]), c3 = guard(sc[q3]);
    const V x0 = x[c0], x1 = x[c1], x2 = x[c2], x3 = x[c3];
    const V v0 = sv[q], v1 = sv[q1], v2 = sv[q2], v3 = sv[q3];
    acc0 = T::fma(v0, x0, acc0);
    const A n1 = T::fma(v1, x1, acc1), n2 = T::fma(v2, x2, acc2), n3 = T::fma(v3, x3, acc3);
    if (q + SUBS < b) acc1 = n1;
    if (q + 2 * SUBS < b) acc2 = n2;
    if (q + 3 * SUBS < b) acc3 = n3;
  }
}

// SUBS lanes per row (4, 8, 16, 32 or 64): a 256-thread workgroup owns
// 256 / SUBS rows, so rows of up to stream_items / (256 / SUBS) entries fit
// the stage (f64: 32 entries at 4 lanes per row, 512 at 64).
template <int SUBS, class V, class I, class P, bool DL>
__global__ __launch_bounds__(256) void spmv_stream_t_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, V* __restrict__ y, int64_t n_rows, int64_t n_blocks, int remap, int stage) {
  using T = VT<V>;
  using A = typename T::acc;
  constexpr int NT = 256;           // threads
  constexpr int RPW = 64 / SUBS;    // rows per wave
  constexpr int R = 4 * RPW;        // rows per workgroup
  constexpr int K = stream_items<A>() / NT;
  extern __shared__ __align__(16) unsigned char t_lds[];
  const StreamTLayout L = stream_t_layout(stage, sizeof(V), sizeof(I), DL);
  V* s_val = reinterpret_cast<V*>(t_lds);
  I* s_col = reinterpret_cast<I*>(t_lds + L.col_off);
  int* s_off = reinterpret_cast<int*>(t_lds + L.off_off);
  const int t = threadIdx.x;
  const int64_t blk = logical_block(remap, n_blocks);
  if (blk < 0) return;  // whole workgroup
  const int64_t rb0 = blk * R;
  const int rows = n_rows - rb0 < R ? (int)(n_rows - rb0) : R;
  const int64_t S = (int64_t)rowptr[rb0];
  for (int k = t; k <= rows; k += NT) s_off[k] = (int)((int64_t)rowptr[rb0 + k] - S);  // rows + 1 offsets
  const int cnt = (int)((int64_t)rowptr[rb0 + rows] - S);
  // entry q of the block (0 <= q < cnt) sits at s_val[q + ov], s_col[q + oi]
  int ov = 0, oi = 0;
  if constexpr (DL) {
    // Each array is copied from the 16-byte boundary at or below entry S to
    // the one at or above S + cnt: a 16-byte aligned load never crosses a
    // page, so reading the rest of a granule that holds a valid entry is safe.
    constexpr int EV = 16 / (int)sizeof(V);
    constexpr int EI = 16 / (int)sizeof(I);
    const int64_t Sv = S & ~(int64_t)(EV - 1);
    const int64_t Si = S & ~(int64_t)(EI - 1);
    ov = (int)(S - Sv);
    oi = (int)(S - Si);
    constexpr int KV = (stream_items<A>() + 2 * EV + NT * EV - 1) / (NT * EV);
    constexpr int KI = (stream_items<A>() + 2 * EI + NT * EI - 1) / (NT * EI);
    lds_copy16<NT / 64, KV>(reinterpret_cast<const unsigned char*>(vals + Sv), reinterpret_cast<unsigned char*>(s_val),
                         (ov + cnt + EV - 1) / EV);
    lds_copy16<NT / 64, KI>(reinterpret_cast<const unsigned char*>(cols + Si), reinterpret_cast<unsigned char*>(s_col),
                         (oi + cnt + EI - 1) / EI);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's LDS copies have landed
  } else {
    V v[K];
    I c[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int q = t + NT * k;
      if (q < cnt) {
        v[k] = load_stream(vals + S + q);  // A is read once: non-temporal
        c[k] = __builtin_nontemporal_load(cols + S + q);
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int q = t + NT * k;
      if (q < cnt) {
        s_col[q] = c[k];
        s_val[q] = v[k];
      }
    }
  }
  __syncthreads();
  const int lane = t & 63;
  const int r = (t >> 6) * RPW + lane % RPW;
  const int sub = lane / RPW;
  A acc0 = T::zero(), acc1 = T::zero(), acc2 = T::zero(), acc3 = T::zero();
  if (r < rows) {
    const int a = s_off[r], b = s_off[r + 1];
    const I* sc = s_col + oi;
    const V* sv = s_val + ov;
    slot_walk<SUBS, T>(sc, sv, x, a, b, sub, acc0, acc1, acc2, acc3, [](I c) { return c; });
  }
  A acc = add(add(acc0, acc1), add(acc2, acc3));
#pragma unroll
  for (int off = RPW; off < 64; off <<= 1) acc = add(acc, shfl(acc, lane ^ off));  // fixed order
  if (sub == 0 && r < rows) store_stream(y + rb0 + r, T::out(acc));
}

// ---------------------------------------------------------------------------
// One-shot SpMV: the unprepared public call's kernel.  The reference
// validates the CSR structure with separate device reads before its launch
// (spmv_csr.py:546-558) and picks its launch from the row lengths
// (spmv_csr.py:623-647); here one kernel does both jobs while it computes:
//   - every workgroup reads its 65 row pointers (it needs them anyway) and
//     flags a start other than 0 (first block), an end other than nnz (last
//     block) and any decrease; every gathered column outside [0, n_cols)
//     is flagged and read as the last column, so no access leaves the
//     arrays;
//   - row pointers are clamped into [0, nnz] before use, so a malformed
//     matrix is computed on garbage but never read out of bounds; the host
//     raises the reference's error for any flag and discards y;
//   - the block's rows go through K3t's LDS stage with 4 lanes per row when
//     their entries fit it, else as two 32-row halves with 8 lanes per row,
//     else row by row with the whole workgroup per row (long rows).
// flags[0..3]: start, end, decrease, column (set to 1; zeroed by the host).
// ---------------------------------------------------------------------------
// Column range check of the one-shot kernel: column c is in [0, n_cols)
// iff (U)c <= last (for int32 columns `last` is capped at INT32_MAX, so a
// negative column, at or above 2^31 as unsigned, is out of range for any
// n_cols).
template <class I>
struct ColGuard;
template <>
struct ColGuard<int32_t> {
  using U = uint32_t;
  __device__ static U last(uint64_t n_cols) { return n_cols - 1 > 0x7fffffffull ? 0x7fffffffu : (U)(n_cols - 1); }
};
template <>
struct ColGuard<int64_t> {
  using U = uint64_t;
  __device__ static U last(uint64_t n_cols) { return n_cols - 1; }
};

// The DL stage copy (global -> LDS, asynchronous) of `cnt` entries from S;
// returns the value / index offsets of S inside the staged 16-byte rows.
template <class V, class I, class A>
__device__ inline void oneshot_stage_dl(const V* __restrict__ vals, const I* __restrict__ cols, int64_t S, int cnt,
                                        unsigned char* t_lds, int C, int& ov, int& oi) {
  constexpr int NT = 256;
  constexpr int CMAX = stream_items<A>();
  constexpr int EV = 16 / (int)sizeof(V);
  constexpr int EI = 16 / (int)sizeof(I);
  const StreamTLayout L = stream_t_layout(C, sizeof(V), sizeof(I), true);
  const int64_t Sv = S & ~(int64_t)(EV - 1);
  const int64_t Si = S & ~(int64_t)(EI - 1);
  ov = (int)(S - Sv);
  oi = (int)(S - Si);
  constexpr int KV = (CMAX + 2 * EV + NT * EV - 1) / (NT * EV);
  constexpr int KI = (CMAX + 2 * EI + NT * EI - 1) / (NT * EI);
  lds_copy16<NT / 64, KV>(reinterpret_cast<const unsigned char*>(vals + Sv), t_lds, (ov + cnt + EV - 1) / EV);
  lds_copy16<NT / 64, KI>(reinterpret_cast<const unsigned char*>(cols + Si), t_lds + L.col_off,
                          (oi + cnt + EI - 1) / EI);
}

// PRESTAGED (with DL): the caller issued oneshot_stage_dl already (offsets
// ov0 / oi0), before its row-pointer phase, so the copy's latency overlaps it.
template <int SUBS, class V, class I, bool DL, bool PRESTAGED = false>
__device__ inline void oneshot_rows(const V* __restrict__ vals, const I* __restrict__ cols,
                                    const V* __restrict__ x, V* __restrict__ y, int64_t row0, int rows,
                                    int64_t S, int cnt, const int* s_off, unsigned char* t_lds, int C,
                                    uint64_t n_cols, bool& bad, int ov0 = 0, int oi0 = 0) {
  using T = VT<V>;
  using A = typename T::acc;
  constexpr int NT = 256;
  constexpr int RPW = 64 / SUBS;
  constexpr int CMAX = stream_items<A>();
  constexpr int K = CMAX / NT;
  const StreamTLayout L = stream_t_layout(C, sizeof(V), sizeof(I), DL);
  V* s_val = reinterpret_cast<V*>(t_lds);
  I* s_col = reinterpret_cast<I*>(t_lds + L.col_off);
  const int t = threadIdx.x;
  int ov = ov0, oi = oi0;
  if constexpr (DL) {
    if constexpr (!PRESTAGED) oneshot_stage_dl<V, I, A>(vals, cols, S, cnt, t_lds, C, ov, oi);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's LDS copies have landed
  } else {
    V v[K];
    I c[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int q = t + NT * k;
      if (q < cnt) {
        v[k] = load_stream(vals + S + q);
        c[k] = __builtin_nontemporal_load(cols + S + q);
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int q = t + NT * k;
      if (q < cnt) {
        s_col[q] = c[k];
        s_val[q] = v[k];
      }
    }
  }
  __syncthreads();
  const int lane = t & 63;
  const int r = (t >> 6) * RPW + lane % RPW;
  const int sub = lane / RPW;
  A acc0 = T::zero(), acc1 = T::zero(), acc2 = T::zero(), acc3 = T::zero();
  // Columns as unsigned: a negative one is above `last`, like one past the
  // end.  Each is clamped to `last` for its gather and folded into a running
  // maximum that is tested once, after the walk.
  using U = typename ColGuard<I>::U;
  const U last = ColGuard<I>::last(n_cols);
  U cmax = 0;
  auto guard = [&](I c) -> I {
    const U u = (U)c;
    cmax = u > cmax ? u : cmax;
    return (I)(u < last ? u : last);
  };
  if (r < rows) {
    const int a = s_off[r], b = s_off[r + 1];
    const I* sc = s_col + oi;
    const V* sv = s_val + ov;
    slot_walk<SUBS, T>(sc, sv, x, a, b, sub, acc0, acc1, acc2, acc3, guard);
  }
  A acc = add(add(acc0, acc1), add(acc2, acc3));
#pragma unroll
  for (int off = RPW; off < 64; off <<= 1) acc = add(acc, shfl(acc, lane ^ off));  // fixed order
  if (sub == 0 && r < rows) store_stream(y + row0 + r, T::out(acc));
  if (cmax > last) bad = true;
  __syncthreads();  // the stage is reused by the caller
}

__device__ inline int64_t readlane_i64(int64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <class V, class I, class P, bool DL>
__global__ __launch_bounds__(256) void spmv_oneshot_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, V* __restrict__ y, int64_t n_rows, int64_t n_cols, int64_t nnz, int64_t n_blocks,
    int remap, int stage, int32_t* __restrict__ flags) {
  using T = VT<V>;
  using A = typename T::acc;
  constexpr int R = 64;
  const int C = stage;  // LDS stage in entries (at most stream_items)
  extern __shared__ __align__(16) unsigned char t_lds[];
  const StreamTLayout L = stream_t_layout(C, sizeof(V), sizeof(I), DL);
  // flags live in pinned host memory: system-scope stores reach it directly
  auto raise = [&](int k) { __hip_atomic_store(flags + k, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); };
  int* s_off = reinterpret_cast<int*>(t_lds + L.off_off);
  __shared__ A s_red[4];
  const int t = threadIdx.x;
  const int64_t blk = logical_block(remap, n_blocks);
  if (blk < 0) return;  // whole workgroup
  const int64_t rb0 = blk * R;
  const int rows = n_rows - rb0 < R ? (int)(n_rows - rb0) : R;
  // Row pointers: each of threads 0..rows loads its own and (below rows) the
  // next one into registers first.  The block's entry range [S, E] comes
  // from its first and last (uniform loads), clamped within [0, nnz], so
  // only the arrays' own entries are read.  With DL and a range that fits
  // the stage, the stage copy is issued next, before anything waits on the
  // row-pointer loads, so its latency overlaps theirs and the checks.
  // The loads are unconditional (threads past the block read its last row
  // pointer) and converted only after all are issued: a load in a divergent
  // branch, or one whose address waits on another, puts one memory latency
  // after another before the stage copy can start.  Lane 63's raw_q is the
  // block's last row pointer in every wave (rows <= 64).
  const P raw_p = rowptr[rb0 + (t <= rows ? t : rows)];
  const P raw_q = rowptr[rb0 + (t < rows ? t + 1 : rows)];
  const P raw_lo = rowptr[rb0];
  const int64_t my_p = (int64_t)raw_p, my_q = (int64_t)raw_q;
  const int64_t p_lo = (int64_t)raw_lo, p_hi = readlane_i64(my_q, 63);
  const int64_t S = p_lo < 0 ? 0 : (p_lo > nnz ? nnz : p_lo);
  const int64_t E = p_hi < S ? S : (p_hi > nnz ? nnz : p_hi);
  const int cnt = (int)(E - S);
  int ov = 0, oi = 0;
  if constexpr (DL) {
    if (cnt <= C) oneshot_stage_dl<V, I, A>(vals, cols, S, cnt, t_lds, C, ov, oi);
  }
  if (t < rows && my_q < my_p) raise(2);
  if (t == 0 && blk == 0 && p_lo != 0) raise(0);
  if (t == 0 && rb0 + rows == n_rows && p_hi != nnz) raise(1);
  if (t <= rows) {
    const int64_t v = my_p < S ? S : (my_p > E ? E : my_p);
    s_off[t] = (int)(v - S);
  }
  __syncthreads();
  const uint64_t nc = (uint64_t)n_cols;
  bool bad = false;
  if (cnt <= C) {
    oneshot_rows<4, V, I, DL, DL>(vals, cols, x, y, rb0, rows, S, cnt, s_off, t_lds, C, nc, bad, ov, oi);
  } else {
    const int half = rows < 32 ? rows : 32;
    const int c0 = s_off[half] - s_off[0], c1 = s_off[rows] - s_off[half];
    if (c0 >= 0 && c0 <= C && c1 >= 0 && c1 <= C) {
      // two 32-row halves, 8 lanes per row (offsets rebased on each half)
      for (int h = 0; h < 2; ++h) {
        const int lo = h * half, nr = h == 0 ? half : rows - half;
        if (nr <= 0) break;
        const int base = s_off[lo];
        __syncthreads();
        int* s_half = s_off + R + 1;  // 33 rebased offsets past the block's own
        if (t <= nr) s_half[t] = s_off[lo + t] - base;
        __syncthreads();
        oneshot_rows<8, V, I, DL>(vals, cols, x, y, rb0 + lo, nr, S + base, h == 0 ? c0 : c1, s_half, t_lds, C,
                                  nc, bad);
      }
    } else {
      // long rows: the whole workgroup per row, straight from global memory
      const int lane = t & 63;
      for (int r = 0; r < rows; ++r) {
        const int a = s_off[r], b = s_off[r + 1];
        A acc = T::zero();
        for (int q = a + t; q < b; q += 256) {
          const auto u = (typename ColGuard<I>::U)cols[S + q];
          const auto last = ColGuard<I>::last(nc);
          if (u > last) bad = true;
          acc = T::fma(vals[S + q], x[u < last ? u : last], acc);
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) acc = add(acc, shfl(acc, lane ^ off));  // fixed order
        if (lane == 0) s_red[t >> 6] = acc;
        __syncthreads();
        if (t == 0) y[rb0 + r] = T::out(add(add(s_red[0], s_red[1]), add(s_red[2], s_red[3])));
        __syncthreads();
      }
    }
  }
  if (bad) raise(3);
}

// ---------------------------------------------------------------------------
// K3b: entry-aligned streaming SpMV.  Block b owns the entry range
// [b*C, (b+1)*C) (C = the LDS stage), so its value / index loads depend on
// nothing and go out at once; the rows it owns (those whose last entry, or
// position when empty, falls in the range) come from a precomputed table
// part[b] and their row pointers load in parallel with the data.  Owned
// rows are summed from the LDS stage by TPR threads each, in passes of
// 256/TPR rows.  A row that begins in an earlier block stores its in-block
// part to head[b]; the entries after the last owned row go to tail[b]
// (they belong to row part[b+1]); nnz_fixup_kernel adds these in block
// order, so the result is deterministic.
// ---------------------------------------------------------------------------
template <int TPR, class V, class I, class P>
__global__ __launch_bounds__(256) void spmv_nnzblock_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, V* __restrict__ y, const int64_t* __restrict__ part,
    typename VT<V>::acc* __restrict__ head, typename VT<V>::acc* __restrict__ tail, int64_t n_rows, int64_t nnz) {
  using T = VT<V>;
  using A = typename T::acc;
  constexpr int C = stream_items<A>();
  constexpr int K = C / 256;
  constexpr int RP = 256 / TPR;  // rows per pass
  __shared__ A s_prod[C];
  __shared__ int64_t s_ptr[RP + 1];
  __shared__ A s_red[4];
  const int t = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int64_t e0 = blk * C;
  const int cnt = nnz - e0 < C ? (int)(nnz - e0) : C;
  V v[K];
  I c[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int q = t + 256 * k;
    c[k] = 0;
    if (q < cnt) {
      v[k] = vals[e0 + q];
      c[k] = cols[e0 + q];
    }
  }
  const int64_t ra = part[blk];
  const int64_t rb = part[blk + 1];
  // first pass's row pointers go out with the data
  // rows + 1 pointers per pass: thread t < rows loads row t's start,
  // thread 0 also the pass's end pointer (rows can equal 256)
  int rows = rb - ra < RP ? (int)(rb - ra) : RP;
  int64_t my_ptr = t < rows ? (int64_t)rowptr[ra + t] : 0;
  int64_t end_ptr = t == 0 ? (int64_t)rowptr[ra + rows] : 0;
  V xv[K];
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (t + 256 * k < cnt) xv[k] = x[c[k]];
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (t + 256 * k < cnt) s_prod[t + 256 * k] = T::mul(v[k], xv[k]);
  const int r = t / TPR;
  const int sub = t % TPR;
  for (int64_t base = ra;;) {
    if (t < rows) s_ptr[t] = my_ptr;
    if (t == 0) s_ptr[rows] = end_ptr;
    __syncthreads();
    A acc = T::zero();
    int64_t start = 0;
    if (r < rows) {
      start = s_ptr[r];
      const int a = (int)((start > e0 ? start : e0) - e0);
      const int b = (int)(s_ptr[r + 1] - e0);
      for (int q = a + sub; q < b; q += TPR) acc = add(acc, s_prod[q]);
    }
    if constexpr (TPR > 1) acc = group_sum<TPR>(acc);
    if (sub == 0 && r < rows) {
      if (start < e0)
        head[blk] = acc;  // only the first owned row can begin before e0
      else
        y[base + r] = T::out(acc);
    }
    base += rows;
    if (base >= rb) break;
    rows = rb - base < RP ? (int)(rb - base) : RP;
    my_ptr = t < rows ? (int64_t)rowptr[base + t] : 0;
    end_ptr = t == 0 ? (int64_t)rowptr[base + rows] : 0;
    __syncthreads();  // s_ptr is rewritten
  }
  if (rb < n_rows) {
    // entries after the last owned row end belong to row rb
    const int64_t rs = (int64_t)rowptr[rb];
    const int ts = (int)((rs > e0 ? rs : e0) - e0);
    A acc = T::zero();
    for (int q = ts + t; q < cnt; q += 256) acc = add(acc, s_prod[q]);
    acc = wave_total(acc);
    if ((t & 63) == 0) s_red[t >> 6] = acc;
    __syncthreads();
    if (t == 0) tail[blk] = add(add(s_red[0], s_red[1]), add(s_red[2], s_red[3]));
  }
}

// Rows that begin in an earlier block: y[row] = tail[f] + ... + tail[b-1] +
// head[b], where blocks f..b-1 end inside `row` and block b owns its end.
template <class V, class P>
__global__ __launch_bounds__(256) void nnz_fixup_kernel(const P* __restrict__ rowptr, const int64_t* __restrict__ part,
                                                        const typename VT<V>::acc* __restrict__ head,
                                                        const typename VT<V>::acc* __restrict__ tail,
                                                        V* __restrict__ y, int64_t n_blocks, int64_t C) {
  using T = VT<V>;
  using A = typename T::acc;
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const int64_t ra = part[b];
  if (part[b + 1] == ra) return;                // owns no row
  if ((int64_t)rowptr[ra] >= b * C) return;     // first row begins inside
  const int64_t f = fixup_start_tile(part, b, ra);  // blocks f..b-1 have tails for row ra
  const A sum = sum_fragments(tail, 1, f + 1, b, tail[f]);
  y[ra] = T::out(add(sum, head[b]));
}

// part[b] = first row whose end pointer exceeds b*C (part[0] = 0,
// part[n_blocks] = n_rows): block b owns rows [part[b], part[b+1]).
template <class P>
__global__ __launch_bounds__(256) void nnz_partition_kernel(const P* __restrict__ rowptr, int64_t n_rows,
                                                            int64_t C, int64_t n_blocks, int64_t* __restrict__ part) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b > n_blocks) return;
  if (b == 0) {
    part[0] = 0;
    return;
  }
  if (b == n_blocks) {
    part[b] = n_rows;
    return;
  }
  const int64_t e = b * C;
  int64_t lo = 0, hi = n_rows;  // count of rows r with rowptr[r + 1] <= e
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)rowptr[mid + 1] <= e)
      lo = mid + 1;
    else
      hi = mid;
  }
  part[b] = lo;
}

// ---------------------------------------------------------------------------
// K2: merge-path SpMV, one wave per tile of 512 merge items (row ends +
// nnz; the partition balances their sum, so long and short rows cost the
// same per item).
//
// The tile's nnz are loaded with unit stride, x is gathered, and the
// products are staged in LDS.  Row ends become a 512-bit tile mask in LDS
// (one ds_or per row end).  Each lane then walks 8 consecutive items
// sequentially: its starting row comes from popcounts of the mask, rows
// that start and end inside the lane are stored directly, the first row it
// closes waits for the lane carry.  One segmented scan of the 64 lane
// tails per tile (DPP row shifts and row broadcasts) supplies the carries.
// Rows that start in an earlier tile write their in-tile part to head[t];
// the part of the last open row goes to tail[t]; merge_fixup_kernel adds
// them in tile order, so results are deterministic and no floating-point
// atomics are used.
// ---------------------------------------------------------------------------
constexpr int kSlabs = 8;
constexpr int kMergeTile = kSlabs * 64;
constexpr int kMergeWaves = 4;

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ inline int count_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((unsigned)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((unsigned)mask, 0u));
}

// DPP-shifted copy of a 32-bit value; lanes whose source is outside the
// enabled rows / row bounds receive 0.
template <int CTRL, int ROWMASK>
__device__ inline int dpp_shift(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWMASK, 0xF, false);
}

template <int CTRL, int ROWMASK>
__device__ inline double dpp_shift(double v) {
  int lo = dpp_shift<CTRL, ROWMASK>(__double2loint(v));
  int hi = dpp_shift<CTRL, ROWMASK>(__double2hiint(v));
  return __hiloint2double(hi, lo);
}

template <int CTRL, int ROWMASK>
__device__ inline c64 dpp_shift(c64 v) {
  return c64{dpp_shift<CTRL, ROWMASK>(v.re), dpp_shift<CTRL, ROWMASK>(v.im)};
}

// One step of the segmented scan: lanes that have not yet reached their
// segment head absorb the shifted partial and its head flag.
template <int CTRL, int ROWMASK, class A>
__device__ inline void seg_step(A& v, int& f) {
  A pv = dpp_shift<CTRL, ROWMASK>(v);
  int pf = dpp_shift<CTRL, ROWMASK>(f);
  if (!f) {
    v = add(v, pv);
    f = pf;
  }
}

// Segmented inclusive scan over the wave; f = 1 marks a segment head.
// row_shr 1,2,4,8 scan each 16-lane row; row_bcast15 / row_bcast31 carry
// across rows (the standard CDNA wave-scan sequence).
template <class A>
__device__ inline A seg_scan(A v, int f) {
  seg_step<0x111, 0xF>(v, f);  // row_shr:1
  seg_step<0x112, 0xF>(v, f);  // row_shr:2
  seg_step<0x114, 0xF>(v, f);  // row_shr:4
  seg_step<0x118, 0xF>(v, f);  // row_shr:8
  seg_step<0x142, 0xA>(v, f);  // row_bcast:15 -> rows 1,3
  seg_step<0x143, 0xC>(v, f);  // row_bcast:31 -> rows 2,3
  return v;
}

template <class A>
__device__ inline A readlane_acc(A v, int lane);
template <>
__device__ inline double readlane_acc<double>(double v, int lane) { return readlane_f64(v, lane); }
template <>
__device__ inline c64 readlane_acc<c64>(c64 v, int lane) {
  return c64{readlane_f64(v.re, lane), readlane_f64(v.im, lane)};
}

// Item layout of a tile: item d (0..511) is a row end if bit d of the
// tile mask is set, otherwise the next nnz.  Lane l walks items
// [8l, 8l+8) sequentially; the products it needs were staged in LDS by
// coalesced loads (index padded by j/8 so that lanes starting 8 products
// apart hit different banks).
__device__ inline int prod_slot(int j) { return j + (j >> 3); }

// Row results go to y as the value type, or (for column-panel partials)
// as the accumulator type, so that a later reduction rounds only once.
template <class V, class Y>
__device__ inline void store_row(Y* y, int64_t row, typename VT<V>::acc v) {
  if constexpr (std::is_same<Y, typename VT<V>::acc>::value)
    y[row] = v;
  else
    y[row] = VT<V>::out(v);
}

// Geometry of merge tile t: its first row r0 = part[t], its row ends
// r0 .. r1-1, its first nnz n0, R row ends and Nz nnz.
struct TileGeom {
  int64_t r0, r1, n0;
  int R, Nz;
};
__device__ inline TileGeom tile_geom(int64_t t, int64_t r0, int64_t r1, int64_t total) {
  const int64_t d0 = t * kMergeTile;
  const int64_t dend = d0 + kMergeTile < total ? d0 + kMergeTile : total;
  TileGeom g;
  g.r0 = r0;
  g.r1 = r1;
  g.n0 = d0 - r0;
  g.R = (int)(r1 - r0);
  g.Nz = (int)(dend - r1 - g.n0);
  return g;
}

// The tile's own loads: values and columns of its nnz (coalesced, read
// once: non-temporal, which keeps x in L2, power-law 0.608 -> 0.591 ms),
// and the row pointers of its row ends (lane-striped), plus rowptr[r0].
template <class V, class I, class P>
__device__ inline void tile_loads(const V* __restrict__ vals, const I* __restrict__ cols,
                                  const P* __restrict__ rowptr, const TileGeom& g, V (&av)[kMergeTile / 64],
                                  I (&cv)[kMergeTile / 64], P (&rp)[kMergeTile / 64], P& rp0) {
  constexpr int kIpt = kMergeTile / 64;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < kIpt; ++k) {
    const int j = k * 64 + lane;
    if (j < g.Nz) {  // lanes past the tile keep stale registers, never read
      av[k] = load_stream(vals + g.n0 + j);
      cv[k] = __builtin_nontemporal_load(cols + g.n0 + j);
    }
  }
#pragma unroll
  for (int i = 0; i < kIpt; ++i) {
    const int k = lane + 64 * i;
    if (k < g.R) rp[i] = rowptr[g.r0 + 1 + k];
  }
  rp0 = g.R > 0 ? rowptr[g.r0] : P(0);
}

// tile_loads without branches, for the pipelined loop: lanes past the
// tile's nnz re-read the matrix's last entry and lanes past its row ends the
// last row pointer (n_rows_total = rows of the CSR), so every load is issued
// and the compiler can count loads in flight exactly (a load skipped on
// some path makes it wait for all of them).  Needs nnz >= 1.
template <class V, class I, class P>
__device__ inline void tile_loads_all(const V* __restrict__ vals, const I* __restrict__ cols,
                                      const P* __restrict__ rowptr, const TileGeom& g, int64_t nnz,
                                      int64_t n_rows_total, V (&av)[kMergeTile / 64], I (&cv)[kMergeTile / 64],
                                      P (&rp)[kMergeTile / 64], P& rp0) {
  constexpr int kIpt = kMergeTile / 64;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < kIpt; ++k) {
    const int j = k * 64 + lane;
    const int64_t e = j < g.Nz ? g.n0 + j : nnz - 1;
    av[k] = load_stream(vals + e);
    cv[k] = __builtin_nontemporal_load(cols + e);
  }
#pragma unroll
  for (int i = 0; i < kIpt; ++i) {
    const int k = lane + 64 * i;
    rp[i] = rowptr[k < g.R ? g.r0 + 1 + k : n_rows_total];
  }
  rp0 = rowptr[g.r0];
}

// Everything after the x gathers of one tile: row-end mask, products in
// LDS, per-lane walk, carry scan, row stores and head / tail fragments.
template <class V, class P, class Y>
__device__ inline void tile_finish(Y* __restrict__ y, typename VT<V>::acc* __restrict__ head,
                                   typename VT<V>::acc* __restrict__ tail, int64_t n_rows, int64_t t,
                                   const TileGeom& g, const V (&av)[kMergeTile / 64], const V (&xv)[kMergeTile / 64],
                                   const P (&rp)[kMergeTile / 64], P rp0, unsigned* msk,
                                   typename VT<V>::acc* prod) {
  using T = VT<V>;
  using A = typename T::acc;
  constexpr int kIpt = kMergeTile / 64;  // items per lane
  const int lane = threadIdx.x & 63;
  const int64_t r0 = g.r0;
  const int R = g.R;
  const int Nz = g.Nz;
  const int items = R + Nz;
  // row-end mask (one ds_or per row end).
  if (lane < kMergeTile / 32) msk[lane] = 0u;
  wave_sync();
#pragma unroll
  for (int i = 0; i < kIpt; ++i) {
    const int k = lane + 64 * i;
    if (k < R) {
      const int q = (int)(k + (int64_t)rp[i] - g.n0);
      atomicOr(&msk[q >> 5], 1u << (q & 31));
    }
  }
  const bool head_partial = R > 0 && (int64_t)rp0 < g.n0;
#pragma unroll
  for (int k = 0; k < kIpt; ++k) {
    const int j = k * 64 + lane;
    if (j < Nz) prod[prod_slot(j)] = T::mul(av[k], xv[k]);
  }
  wave_sync();
  // sequential walk of this lane's 8 items.  Row ends before the lane:
  // popcounts of the 16 mask words, scanned over lanes 0..15 with DPP row
  // shifts (one 16-lane row), read back from lane d/32 by a permute.
  static_assert(kMergeTile / 32 == 16, "word scan covers one DPP row");
  const int d = kIpt * lane;                          // first item of the lane
  const unsigned word = msk[d >> 5];
  const int cnt = lane < 16 ? __popc(msk[lane]) : 0;
  int inc = cnt;
  inc += dpp_shift<0x111, 0xF>(inc);  // row_shr:1
  inc += dpp_shift<0x112, 0xF>(inc);  // row_shr:2
  inc += dpp_shift<0x114, 0xF>(inc);  // row_shr:4
  inc += dpp_shift<0x118, 0xF>(inc);  // row_shr:8
  const int word_pre = __shfl(inc - cnt, d >> 5);
  const unsigned pattern = (word >> (d & 31)) & 0xFFu;  // 8 items never straddle a word
  const int i_l = word_pre + __popc(word & ((1u << (d & 31)) - 1u));
  int j = d - i_l;                                     // tile-local nnz index
  int ends = 0;
  A acc = T::zero(), first = T::zero();
#pragma unroll
  for (int u = 0; u < kIpt; ++u) {
    if (d + u < items) {
      if ((pattern >> u) & 1u) {
        if (ends == 0) {
          first = acc;
        } else {
          store_row<V>(y, r0 + i_l + ends, acc);
        }
        ++ends;
        acc = T::zero();
      } else {
        acc = add(acc, prod[prod_slot(j)]);
        ++j;
      }
    }
  }

  // carry across lanes: inclusive segmented scan of lane tails (a lane
  // with a row end starts a new segment), shifted to exclusive.
  const A incl = seg_scan(acc, ends > 0 ? 1 : 0);
  A carry_in = shfl(incl, lane > 0 ? lane - 1 : 0);
  if (lane == 0) carry_in = T::zero();
  if (ends > 0) {
    const A v = add(carry_in, first);
    const int64_t row = r0 + i_l;
    if (row == r0 && head_partial)
      head[t] = v;
    else
      store_row<V>(y, row, v);
  }
  if (lane == 63 && g.r1 < n_rows) tail[t] = incl;
}

// One merge tile, processed by one wave (per-wave LDS slices passed in).
template <class V, class I, class P, class Y>
__device__ inline void merge_tile(const V* __restrict__ vals, const I* __restrict__ cols,
                                  const P* __restrict__ rowptr, const V* __restrict__ x, Y* __restrict__ y,
                                  const int64_t* __restrict__ part, typename VT<V>::acc* __restrict__ head,
                                  typename VT<V>::acc* __restrict__ tail, int64_t n_rows, int64_t nnz,
                                  int64_t t, unsigned* msk, typename VT<V>::acc* prod) {
  constexpr int kIpt = kMergeTile / 64;
  const int lane = threadIdx.x & 63;
  const TileGeom g = tile_geom(t, part[t], part[t + 1], n_rows + nnz);
  V av[kIpt];
  I cv[kIpt];
  P rp[kIpt];
  P rp0;
  tile_loads<V, I, P>(vals, cols, rowptr, g, av, cv, rp, rp0);
  V xv[kIpt];
#pragma unroll
  for (int k = 0; k < kIpt; ++k)
    if (k * 64 + lane < g.Nz) xv[k] = x[cv[k]];
  tile_finish<V, P, Y>(y, head, tail, n_rows, t, g, av, xv, rp, rp0, msk, prod);
}

// A wave's run of merge tiles t0, t0 + stride, ... (< t_end), software
// pipelined: the x gathers of tile i are issued first, then the loads of
// tile i+1 (values, columns, row pointers) and the partition entries of
// tile i+2, and only then does the wave wait for its gathers and finish
// tile i.  Loads complete in issue order, so the wait for the gathers does
// not wait for the prefetch: the HBM latency of the next tile's A overlaps
// the L2 latency of this tile's gathers, where one tile per wave pays both
// in turn.
template <class V, class I, class P, class Y>
__device__ inline void merge_tiles_pipelined(const V* __restrict__ vals, const I* __restrict__ cols,
                                             const P* __restrict__ rowptr, const V* __restrict__ x,
                                             Y* __restrict__ y, const int64_t* __restrict__ part,
                                             typename VT<V>::acc* __restrict__ head,
                                             typename VT<V>::acc* __restrict__ tail, int64_t n_rows, int64_t nnz,
                                             int64_t t0, int64_t stride, int64_t t_end, unsigned* msk,
                                             typename VT<V>::acc* prod) {
  constexpr int kIpt = kMergeTile / 64;
  const int lane = threadIdx.x & 63;
  const int64_t total = n_rows + nnz;
  if (t0 >= t_end) return;
  TileGeom g = tile_geom(t0, part[t0], part[t0 + 1], total);
  V av[kIpt];
  I cv[kIpt];
  P rp[kIpt];
  P rp0;
  tile_loads_all<V, I, P>(vals, cols, rowptr, g, nnz, n_rows, av, cv, rp, rp0);
  int64_t t = t0;
  int64_t tn = t0 + stride;
  // partition entries of the next tile (the current one again past the end,
  // so that the loop body always issues the same loads)
  int64_t pn0 = part[tn < t_end ? tn : t0], pn1 = part[(tn < t_end ? tn : t0) + 1];
  while (true) {
    V xv[kIpt];
#pragma unroll
    for (int k = 0; k < kIpt; ++k) xv[k] = x[cv[k]];  // every column is valid (lanes past the tile repeat one)
    const bool more = tn < t_end;
    const int64_t tl = more ? tn : t;  // tile whose loads are issued now
    const TileGeom gn = tile_geom(tl, pn0, pn1, total);
    V avn[kIpt];
    I cvn[kIpt];
    P rpn[kIpt];
    P rp0n;
    tile_loads_all<V, I, P>(vals, cols, rowptr, gn, nnz, n_rows, avn, cvn, rpn, rp0n);
    const int64_t tnn = tn + stride < t_end ? tn + stride : tl;
    const int64_t pnn0 = part[tnn], pnn1 = part[tnn + 1];
    tile_finish<V, P, Y>(y, head, tail, n_rows, t, g, av, xv, rp, rp0, msk, prod);
    if (!more) break;
    wave_sync();  // this tile's LDS reads are done before the next tile's writes
    g = gn;
#pragma unroll
    for (int k = 0; k < kIpt; ++k) {
      av[k] = avn[k];
      cv[k] = cvn[k];
      rp[k] = rpn[k];
    }
    rp0 = rp0n;
    t = tn;
    tn += stride;
    pn0 = pnn0;
    pn1 = pnn1;
  }
}

template <class V, class I, class P>
__global__ __launch_bounds__(256) void spmv_merge_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, V* __restrict__ y, const int64_t* __restrict__ part,
    typename VT<V>::acc* __restrict__ head, typename VT<V>::acc* __restrict__ tail,
    int64_t n_rows, int64_t nnz, int64_t n_tiles) {
  using A = typename VT<V>::acc;
  __shared__ unsigned s_mask[kMergeWaves][kMergeTile / 32];
  __shared__ A s_prod[kMergeWaves][kMergeTile + kMergeTile / 8];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int64_t t = (int64_t)blockIdx.x * kMergeWaves + w;
  if (t >= n_tiles) return;  // per-wave work only; no block barriers
  merge_tile<V, I, P, V>(vals, cols, rowptr, x, y, part, head, tail, n_rows, nnz, t, s_mask[w], s_prod[w]);
}

// K2, persistent and pipelined: a fixed grid whose waves each walk tiles
// w, w + W, ... (W = waves in the grid) with merge_tiles_pipelined.
template <class V, class I, class P>
__global__ __launch_bounds__(256) void spmv_merge_pipe_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, V* __restrict__ y, const int64_t* __restrict__ part,
    typename VT<V>::acc* __restrict__ head, typename VT<V>::acc* __restrict__ tail,
    int64_t n_rows, int64_t nnz, int64_t n_tiles) {
  using A = typename VT<V>::acc;
  __shared__ unsigned s_mask[kMergeWaves][kMergeTile / 32];
  __shared__ A s_prod[kMergeWaves][kMergeTile + kMergeTile / 8];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int64_t t0 = (int64_t)blockIdx.x * kMergeWaves + w;
  const int64_t stride = (int64_t)gridDim.x * kMergeWaves;
  merge_tiles_pipelined<V, I, P, V>(vals, cols, rowptr, x, y, part, head, tail, n_rows, nnz, t0, stride, n_tiles,
                                    s_mask[w], s_prod[w]);
}

// ---------------------------------------------------------------------------
// K2p: merge-path SpMV over a column-panelled matrix.  The stacked CSR holds
// panel p's entries (columns [p*width, (p+1)*width)) as rows p*n + r, so the
// x gathers of one panel touch one slice of x.  Workgroups are handed out to
// the 8 XCDs round-robin by workgroup id; workgroup b runs on XCD b % 8 and
// takes the tile blocks of panel (b % 8), so each XCD's L2 holds one x
// slice instead of all of x.  Panel results are accumulator-typed partials
// (panel-major); panel_reduce_kernel sums them per row in panel order.
// ---------------------------------------------------------------------------
constexpr int kMaxPanels = 64;
constexpr int kPanelWgPerCu = 6;
struct PanelTable {
  int64_t first[kMaxPanels + 1];  // first merge block of each panel; [n_panels] = number of blocks
};

template <class V, class I, class P>
__global__ __launch_bounds__(256) void spmv_panel_merge_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, typename VT<V>::acc* __restrict__ y, const int64_t* __restrict__ part,
    typename VT<V>::acc* __restrict__ head, typename VT<V>::acc* __restrict__ tail, const PanelTable tab,
    int n_panels, int64_t n_rows, int64_t nnz, int64_t n_tiles) {
  using A = typename VT<V>::acc;
  __shared__ unsigned s_mask[kMergeWaves][kMergeTile / 32];
  __shared__ A s_prod[kMergeWaves][kMergeTile + kMergeTile / 8];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  // With fewer panels than XCDs (n_panels dividing 8) panel p is shared by
  // XCDs p, p + n_panels, ...; each takes every G-th block of the panel.
  // Otherwise XCD x owns panels x, x + 8, ... and its workgroups (slot 0,
  // 1, ...) take their blocks in that order.  One block per workgroup.
  const int xcd = (int)(blockIdx.x % kXcds);
  int64_t slot = blockIdx.x / kXcds;
  int64_t b = -1;
  if (n_panels < kXcds && kXcds % n_panels == 0) {
    const int G = kXcds / n_panels;
    const int p = xcd % n_panels;
    b = tab.first[p] + slot * G + xcd / n_panels;
    if (b >= tab.first[p + 1]) return;
  } else {
    for (int p = xcd; p < n_panels; p += kXcds) {
      const int64_t nb = tab.first[p + 1] - tab.first[p];
      if (slot < nb) {
        b = tab.first[p] + slot;
        break;
      }
      slot -= nb;
    }
    if (b < 0) return;
  }
  const int64_t t = b * kMergeWaves + w;
  if (t >= n_tiles) return;
  merge_tile<V, I, P, A>(vals, cols, rowptr, x, y, part, head, tail, n_rows, nnz, t, s_mask[w], s_prod[w]);
}

// K2p, persistent and pipelined: for n_panels dividing 8 (panel p on XCDs
// p, p + n_panels, ...), a fixed grid of workgroups whose waves each walk
// a strided run of their panel's tiles with merge_tiles_pipelined.  Wave
// slot ws of the XCD's W waves takes tiles T0 + (ws + i W) G + s of panel p
// (G XCDs per panel, s = this XCD's index among them), so the waves of a
// panel sweep its tiles front to back together.
template <class V, class I, class P>
__global__ __launch_bounds__(256) void spmv_panel_pipe_kernel(
    const V* __restrict__ vals, const I* __restrict__ cols, const P* __restrict__ rowptr,
    const V* __restrict__ x, typename VT<V>::acc* __restrict__ y, const int64_t* __restrict__ part,
    typename VT<V>::acc* __restrict__ head, typename VT<V>::acc* __restrict__ tail, const PanelTable tab,
    int n_panels, int64_t n_rows, int64_t nnz, int64_t n_tiles) {
  using A = typename VT<V>::acc;
  __shared__ unsigned s_mask[kMergeWaves][kMergeTile / 32];
  __shared__ A s_prod[kMergeWaves][kMergeTile + kMergeTile / 8];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int xcd = (int)(blockIdx.x % kXcds);
  const int64_t slot = blockIdx.x / kXcds;
  const int64_t n_slots = gridDim.x / kXcds;
  const int G = kXcds / n_panels;
  const int p = xcd % n_panels;
  const int s = xcd / n_panels;
  const int64_t T0 = tab.first[p] * kMergeWaves;
  const int64_t T1 = tab.first[p + 1] * kMergeWaves < n_tiles ? tab.first[p + 1] * kMergeWaves : n_tiles;
  const int64_t ws = slot * kMergeWaves + w;
  const int64_t t0 = T0 + ws * G + s;
  const int64_t stride = n_slots * kMergeWaves * G;
  merge_tiles_pipelined<V, I, P, A>(vals, cols, rowptr, x, y, part, head, tail, n_rows, nnz, t0, stride, T1,
                                    s_mask[w], s_prod[w]);
}

// y[r] = sum over panels p (in order) of partial[p * n_rows + r], rounded once.
template <class V>
__global__ __launch_bounds__(256) void panel_reduce_kernel(const typename VT<V>::acc* __restrict__ partial,
                                                           V* __restrict__ y, int64_t n_rows, int n_panels) {
  using T = VT<V>;
  using A = typename T::acc;
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n_rows) return;
  A sum = partial[r];
  for (int p = 1; p < n_panels; ++p) sum = add(sum, partial[(int64_t)p * n_rows + r]);
  y[r] = T::out(sum);
}

// Rows that span tiles: y[row] = tail[f] + ... + tail[t-1] + head[t], where
// tiles f..t-1 all end inside `row` and tile t holds its row end.
template <class V, class P, class Y = V>
__global__ __launch_bounds__(256) void merge_fixup_kernel(
    const P* __restrict__ rowptr, const int64_t* __restrict__ part,
    const typename VT<V>::acc* __restrict__ head, const typename VT<V>::acc* __restrict__ tail,
    Y* __restrict__ y, int64_t n_tiles, int64_t tile_items) {
  using T = VT<V>;
  using A = typename T::acc;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tiles) return;
  const int64_t r0 = part[t];
  if (part[t + 1] == r0) return;  // tile holds no row end
  const int64_t n0 = t * tile_items - r0;
  if ((int64_t)rowptr[r0] >= n0) return;  // row r0 starts inside tile t
  const int64_t f = fixup_start_tile(part, t, r0);
  A sum = sum_fragments(tail, 1, f + 1, t, tail[f]);
  sum = add(sum, head[t]);
  store_row<V>(y, r0, sum);
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
// XCD-contiguous workgroup mapping (FLAGSPARSE_XCD_REMAP=0/1 for A/B).
// K3t (slot-order gather) in place of K3 for blocks of 64 rows; off with
// FLAGSPARSE_SPMV_STREAM_T=0 (A/B).
inline bool stream_t_enabled() {
  const char* e = std::getenv("FLAGSPARSE_SPMV_STREAM_T");
  return !(e && std::atoi(e) == 0);
}

// Persistent, software-pipelined K2 (spmv_merge_pipe_kernel): power-law 4M
// without panels 0.998 -> 0.974 ms (f32 / i32), 1.020 -> 1.010 (i64).
// FLAGSPARSE_MERGE_PIPE=0 runs one tile per wave (A/B).
inline bool merge_pipe_enabled() {
  const char* e = std::getenv("FLAGSPARSE_MERGE_PIPE");
  return !(e && std::atoi(e) == 0);
}

// Persistent, software-pipelined K2p (spmv_panel_pipe_kernel) when the
// panel count divides the XCD count; FLAGSPARSE_PANEL_PIPE=0 runs one tile
// per wave instead (A/B).
inline bool panel_pipe_enabled() {
  const char* e = std::getenv("FLAGSPARSE_PANEL_PIPE");
  return !(e && std::atoi(e) == 0);
}

// Direct global-to-LDS staging in K3t (kernel ms, staged through VGPRs ->
// direct): 27-point stencil f64 0.1364 -> 0.1249, f32 0.103 -> 0.086, f64 /
// int64 0.167 -> 0.156; 2M x 2M with 16 random columns per row f64 0.482 ->
// 0.496, f32 0.325 -> 0.338 (their x gathers bound them).
// FLAGSPARSE_SPMV_STREAM_T_DL=0 stages through VGPRs (A/B).
inline bool stream_t_dl_enabled() {
  const char* e = std::getenv("FLAGSPARSE_SPMV_STREAM_T_DL");
  return !(e && std::atoi(e) == 0);
}

// K3t with eight lanes per row (32-row workgroups) for rows too long for
// four lanes; FLAGSPARSE_SPMV_STREAM_T_WIDE=0 runs K3 there instead (A/B).
inline bool stream_t_wide_enabled() {
  const char* e = std::getenv("FLAGSPARSE_SPMV_STREAM_T_WIDE");
  return !(e && std::atoi(e) == 0);
}

inline int xcd_remap() {
  if (const char* e = std::getenv("FLAGSPARSE_XCD_REMAP")) return std::atoi(e) != 0;
  return 0;  // measured neutral (within 5%) on the stencil and uniform matrices
}

// Resident workgroups per CU of kernel `kern` at 256 threads and `lds`
// bytes of dynamic LDS, cached per (kernel, device, lds) so that the
// persistent launches do not query the runtime on every call.
template <class F>
inline int resident_per_cu(F kern, size_t lds) {
  struct Entry {
    const void* k;
    int dev;
    size_t lds;
    int n;
  };
  static thread_local Entry cache[16];
  static thread_local int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  const void* key = reinterpret_cast<const void*>(kern);
  for (int i = 0; i < used; ++i)
    if (cache[i].k == key && cache[i].dev == dev && cache[i].lds == lds) return cache[i].n;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, 256, lds) != hipSuccess || n <= 0) n = 1;
  Entry e{key, dev, lds, n};
  if (used < 16) cache[used++] = e;
  else cache[(dev < 0 ? 0 : dev) % 16] = e;
  return n;
}

// Compute units of the current device (cached per device id; relaxed
// atomics, so concurrent host threads at most query the device twice).
inline int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <class V, class I, class P>
int launch_spmv(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                const void* x, void* y, const void* part, void* carry, size_t carry_bytes,
                hipStream_t stream) {
  using A = typename VT<V>::acc;
  const int64_t n_rows = plan->n_rows;
  if (n_rows == 0) return FS_OK;
  const V* v = static_cast<const V*>(vals);
  const I* c = static_cast<const I*>(cols);
  const P* p = static_cast<const P*>(indptr);
  const V* xv = static_cast<const V*>(x);
  V* yv = static_cast<V*>(y);
  if (plan->kernel == FS_KERNEL_VECTOR) {
    const int vw = plan->vec_width;
    const int64_t blocks = ceil_div(n_rows * vw, 256);
    const int remap = xcd_remap();
    const int64_t grid = remap ? ceil_div(blocks, kXcds) * kXcds : blocks;
    if (grid > 0x7fffffffLL) return fail(FS_E_INVALID, "fs_spmv_csr: grid too large for vector kernel");
    dim3 g((unsigned)grid);
    switch (vw) {
      case 2: hipLaunchKernelGGL((spmv_vector_kernel<2, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      case 4: hipLaunchKernelGGL((spmv_vector_kernel<4, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      case 8: hipLaunchKernelGGL((spmv_vector_kernel<8, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      case 16: hipLaunchKernelGGL((spmv_vector_kernel<16, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      case 32: hipLaunchKernelGGL((spmv_vector_kernel<32, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      case 64: hipLaunchKernelGGL((spmv_vector_kernel<64, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      default: return fail(FS_E_INVALID, "fs_spmv_csr: vec_width must be a power of two in [2, 64]");
    }
    FS_CHECK_MAIN_LAUNCH("spmv_vector_kernel");
    return FS_OK;
  }
  if (plan->kernel == FS_KERNEL_STREAM) {
    using Acc = typename VT<V>::acc;
    const int rpb = plan->rows_per_block;
    if (rpb < 32 || rpb > 256 || (rpb & (rpb - 1)) || (int64_t)plan->max_row * rpb > stream_items<Acc>())
      return fail(FS_E_INVALID, "fs_spmv_csr: rows_per_block does not fit the stream kernel");
    // (the dispatch counts work-items in 32 bits: beyond 2^32 threads, K3's
    // larger row blocks run instead)
    // four lanes per row (64 rows per workgroup) when 64 rows fit the stage,
    // else eight (32 rows): the rows the stream plan admits (f64: up to 64
    // entries) all fit one or the other.
    const int subs = (int64_t)plan->max_row * 64 <= stream_items<Acc>() ? 4
                   : ((int64_t)plan->max_row * 32 <= stream_items<Acc>() && stream_t_wide_enabled()) ? 8 : 0;
    const int64_t rows_per_wg = subs ? 256 / subs : 1;
    if (stream_t_enabled() && subs && ceil_div(n_rows, rows_per_wg) * 256 < (int64_t(1) << 32)) {
      const int64_t blocks = ceil_div(n_rows, rows_per_wg);
      const int remap = xcd_remap();
      dim3 g((unsigned)(remap ? ceil_div(blocks, kXcds) * kXcds : blocks));
      const int stage = (int)std::max<int64_t>(rows_per_wg * plan->max_row, 1);
      // direct-to-LDS staging needs 16-byte aligned value / index arrays
      const bool dl = stream_t_dl_enabled() && ((uintptr_t)v % 16) == 0 && ((uintptr_t)c % 16) == 0;
      const size_t lds = stream_t_layout(stage, sizeof(V), sizeof(I), dl).total;
      // four lanes per row: 16 rows per gather instruction.  One or two lanes
      // per row (64 / 32 rows per instruction, 64- / 128-thread workgroups)
      // measured slower on the f64 stencil: 0.176 / 0.150 against 0.136 ms.
      auto launch = [&](auto sc, auto dc) {
        hipLaunchKernelGGL((spmv_stream_t_kernel<decltype(sc)::value, V, I, P, decltype(dc)::value>), g, dim3(256),
                           lds, stream, v, c, p, xv, yv, n_rows, blocks, remap, stage);
      };
      using S4 = std::integral_constant<int, 4>;
      using S8 = std::integral_constant<int, 8>;
      if (subs == 4) {
        if (dl) launch(S4{}, std::true_type{});
        else launch(S4{}, std::false_type{});
      } else {
        if (dl) launch(S8{}, std::true_type{});
        else launch(S8{}, std::false_type{});
      }
      FS_CHECK_MAIN_LAUNCH("spmv_stream_t_kernel");
      return FS_OK;
    }
    const int64_t blocks = ceil_div(n_rows, (int64_t)rpb);
    const int remap = xcd_remap();
    dim3 g((unsigned)(remap ? ceil_div(blocks, kXcds) * kXcds : blocks));
    switch (256 / rpb) {
      case 1: hipLaunchKernelGGL((spmv_stream_kernel<1, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      case 2: hipLaunchKernelGGL((spmv_stream_kernel<2, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      case 4: hipLaunchKernelGGL((spmv_stream_kernel<4, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
      default: hipLaunchKernelGGL((spmv_stream_kernel<8, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, n_rows, blocks, remap); break;
    }
    FS_CHECK_MAIN_LAUNCH("spmv_stream_kernel");
    return FS_OK;
  }
  if (plan->kernel == FS_KERNEL_NNZBLOCK) {
    constexpr int C = stream_items<A>();
    const int64_t n_blocks = plan->n_tiles;
    if (plan->tile_items != C || n_blocks != ceil_div(plan->nnz, C) || n_blocks == 0)
      return fail(FS_E_INVALID, "fs_spmv_csr: plan does not describe entry blocks");
    if (part == nullptr) return fail(FS_E_INVALID, "fs_spmv_csr: entry-block kernel needs the partition");
    if (carry == nullptr || carry_bytes < (size_t)n_blocks * 2 * sizeof(A))
      return fail(FS_E_WORKSPACE, "fs_spmv_csr: carry workspace too small");
    if (n_blocks > 0x7fffffffLL) return fail(FS_E_INVALID, "fs_spmv_csr: grid too large");
    A* head = static_cast<A*>(carry);
    A* tail = head + n_blocks;
    const int64_t* pt = static_cast<const int64_t*>(part);
    dim3 g((unsigned)n_blocks);
    switch (plan->vec_width) {
      case 1: hipLaunchKernelGGL((spmv_nnzblock_kernel<1, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, pt, head, tail, n_rows, plan->nnz); break;
      case 2: hipLaunchKernelGGL((spmv_nnzblock_kernel<2, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, pt, head, tail, n_rows, plan->nnz); break;
      case 4: hipLaunchKernelGGL((spmv_nnzblock_kernel<4, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, pt, head, tail, n_rows, plan->nnz); break;
      case 8: hipLaunchKernelGGL((spmv_nnzblock_kernel<8, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, pt, head, tail, n_rows, plan->nnz); break;
      case 16: hipLaunchKernelGGL((spmv_nnzblock_kernel<16, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, pt, head, tail, n_rows, plan->nnz); break;
      case 32: hipLaunchKernelGGL((spmv_nnzblock_kernel<32, V, I, P>), g, dim3(256), 0, stream, v, c, p, xv, yv, pt, head, tail, n_rows, plan->nnz); break;
      default: return fail(FS_E_INVALID, "fs_spmv_csr: entry-block threads per row must be a power of two in [1, 32]");
    }
    FS_CHECK_MAIN_LAUNCH("spmv_nnzblock_kernel");
    hipLaunchKernelGGL((nnz_fixup_kernel<V, P>), dim3((unsigned)ceil_div(n_blocks, 256)), dim3(256), 0, stream, p, pt,
                       head, tail, yv, n_blocks, (int64_t)C);
    FS_CHECK_LAUNCH("nnz_fixup_kernel");
    return FS_OK;
  }
  if (plan->kernel != FS_KERNEL_MERGE) return fail(FS_E_INVALID, "fs_spmv_csr: unknown kernel");
  if (plan->tile_items != kMergeTile)
    return fail(FS_E_INVALID, "fs_spmv_csr: plan tile_items does not match the merge kernel");
  const int64_t n_tiles = plan->n_tiles;
  if (part == nullptr) return fail(FS_E_INVALID, "fs_spmv_csr: merge kernel needs the partition");
  const size_t need = (size_t)n_tiles * 2 * sizeof(A);
  if (carry == nullptr || carry_bytes < need)
    return fail(FS_E_WORKSPACE, "fs_spmv_csr: carry workspace too small");
  A* head = static_cast<A*>(carry);
  A* tail = head + n_tiles;
  const int64_t blocks = ceil_div(n_tiles, kMergeWaves);
  if (plan->nnz > 0 && merge_pipe_enabled()) {
    const int per_cu = resident_per_cu(spmv_merge_pipe_kernel<V, I, P>, 0);
    const int64_t wgs = std::min<int64_t>(blocks, (int64_t)device_cus() * std::max(per_cu, 1));
    hipLaunchKernelGGL((spmv_merge_pipe_kernel<V, I, P>), dim3((unsigned)wgs), dim3(256), 0, stream, v, c, p, xv, yv,
                       static_cast<const int64_t*>(part), head, tail, n_rows, plan->nnz, n_tiles);
    FS_CHECK_MAIN_LAUNCH("spmv_merge_pipe_kernel");
  } else {
    hipLaunchKernelGGL((spmv_merge_kernel<V, I, P>), dim3((unsigned)blocks), dim3(256), 0, stream, v, c, p,
                       xv, yv, static_cast<const int64_t*>(part), head, tail, n_rows, plan->nnz, n_tiles);
    FS_CHECK_MAIN_LAUNCH("spmv_merge_kernel");
  }
  hipLaunchKernelGGL((merge_fixup_kernel<V, P>), dim3((unsigned)ceil_div(n_tiles, 256)), dim3(256), 0,
                     stream, p, static_cast<const int64_t*>(part), head, tail, yv, n_tiles,
                     (int64_t)kMergeTile);
  FS_CHECK_LAUNCH("merge_fixup_kernel");
  return FS_OK;
}

// Column-panel SpMV: workspace = head/tail carries and accumulator partials
// (one per stacked row).
struct PanelWs {
  size_t off_carry, off_partial, total;
};
inline size_t align256s(size_t v) { return (v + 255) & ~(size_t)255; }
inline PanelWs panel_ws(const fs_csr_plan* plan, int n_panels, size_t acc) {
  PanelWs L{};
  size_t o = 0;
  L.off_carry = o; o = align256s(o + (size_t)plan->n_tiles * 2 * acc);
  L.off_partial = o; o = align256s(o + (size_t)plan->n_rows * acc);
  L.total = o;
  return L;
}

template <class V, class I, class P>
int launch_spmv_panels(const fs_csr_plan* plan, int n_panels, const int64_t* panel_nnz, const void* vals,
                       const void* cols, const void* indptr, const void* x, void* y, const void* part, void* ws,
                       size_t ws_bytes, int64_t n_out, hipStream_t stream) {
  using A = typename VT<V>::acc;
  const PanelWs L = panel_ws(plan, n_panels, sizeof(A));
  if (ws == nullptr || ws_bytes < L.total) return fail(FS_E_WORKSPACE, "fs_spmv_csr_panels: workspace too small");
  char* w = static_cast<char*>(ws);
  A* head = reinterpret_cast<A*>(w + L.off_carry);
  A* tail = head + plan->n_tiles;
  A* partial = reinterpret_cast<A*>(w + L.off_partial);
  const P* p = static_cast<const P*>(indptr);
  const int64_t n_tiles = plan->n_tiles;
  const int64_t n_blocks = ceil_div(n_tiles, kMergeWaves);
  // Block table from the panel starts: panel q begins at merge item
  // q * n_out + panel_nnz[q]; a block shared by two panels goes to the later.
  PanelTable tab{};
  tab.first[0] = 0;
  for (int q = 1; q < n_panels; ++q) {
    const int64_t item = (int64_t)q * n_out + panel_nnz[q];
    tab.first[q] = std::min<int64_t>(item / ((int64_t)kMergeTile * kMergeWaves), n_blocks);
  }
  tab.first[n_panels] = n_blocks;
  int64_t per_xcd = 1;
  if (n_panels < kXcds && kXcds % n_panels == 0) {
    const int G = kXcds / n_panels;
    for (int q = 0; q < n_panels; ++q) per_xcd = std::max(per_xcd, ceil_div(tab.first[q + 1] - tab.first[q], G));
  } else {
    for (int xcd = 0; xcd < kXcds; ++xcd) {
      int64_t sum = 0;
      for (int q = xcd; q < n_panels; q += kXcds) sum += tab.first[q + 1] - tab.first[q];
      per_xcd = std::max(per_xcd, sum);
    }
  }
  if (per_xcd * kXcds > 0x7fffffffLL) return fail(FS_E_INVALID, "fs_spmv_csr_panels: grid too large");
  // At most 6 workgroups per CU instead of the 8 that LDS allows: fewer
  // concurrent tiles contend for the L2 request queues that the random x
  // gathers saturate (power-law 4M, 4 panels: 0.593 -> 0.577 ms; 5 per CU
  // the same, 4 per CU 0.615, 2 per CU 0.846).  FLAGSPARSE_PANEL_WG_CAP=N
  // overrides (0 = no cap).
  int cap = kPanelWgPerCu;
  if (const char* e = std::getenv("FLAGSPARSE_PANEL_WG_CAP")) cap = std::atoi(e);
  const size_t static_lds = sizeof(unsigned) * kMergeWaves * (kMergeTile / 32) +
                            sizeof(typename VT<V>::acc) * kMergeWaves * (kMergeTile + kMergeTile / 8);
  const size_t lds_pad = lds_pad_for_cap(cap, static_lds);
  if (kXcds % n_panels == 0 && plan->nnz > 0 && panel_pipe_enabled()) {
    // persistent: as many workgroups per CU as can be resident at once (at
    // most `cap`), on every CU of each XCD.  The kernel takes 120 VGPRs (4
    // waves per SIMD).  Power-law 4M, 4 panels: 0.581 -> 0.570 ms against
    // one tile per wave; forcing 5 / 6 waves per SIMD (spills) 0.597 /
    // 0.633; 2 / 3 / 4 workgroups per CU 0.571 / 0.582 / 0.571.  The x
    // gathers' L2 request rate bounds it, not the latency the pipeline hides.
    auto launch = [&](auto kern) -> int {
      int per_cu = resident_per_cu(kern, lds_pad);
      if (cap > 0) per_cu = std::min(per_cu, cap);
      const int64_t wgs = std::max<int64_t>(1, (int64_t)(device_cus() / kXcds) * std::max(per_cu, 1));
      hipLaunchKernelGGL(kern, dim3((unsigned)(std::min(wgs, per_xcd) * kXcds)), dim3(256), lds_pad, stream,
                         static_cast<const V*>(vals), static_cast<const I*>(cols), p, static_cast<const V*>(x), partial,
                         static_cast<const int64_t*>(part), head, tail, tab, n_panels, plan->n_rows, plan->nnz,
                         n_tiles);
      return FS_OK;
    };
    const int rc = launch(spmv_panel_pipe_kernel<V, I, P>);
    if (rc != FS_OK) return rc;
    FS_CHECK_MAIN_LAUNCH("spmv_panel_pipe_kernel");
  } else {
    hipLaunchKernelGGL((spmv_panel_merge_kernel<V, I, P>), dim3((unsigned)(per_xcd * kXcds)), dim3(256), lds_pad,
                       stream, static_cast<const V*>(vals), static_cast<const I*>(cols), p, static_cast<const V*>(x),
                       partial, static_cast<const int64_t*>(part), head, tail, tab, n_panels, plan->n_rows,
                       plan->nnz, n_tiles);
    FS_CHECK_MAIN_LAUNCH("spmv_panel_merge_kernel");
  }
  hipLaunchKernelGGL((merge_fixup_kernel<V, P, A>), dim3((unsigned)ceil_div(n_tiles, 256)), dim3(256), 0, stream, p,
                     static_cast<const int64_t*>(part), head, tail, partial, n_tiles, (int64_t)kMergeTile);
  FS_CHECK_LAUNCH("merge_fixup_kernel");
  hipLaunchKernelGGL((panel_reduce_kernel<V>), dim3((unsigned)ceil_div(n_out, 256)), dim3(256), 0, stream, partial,
                     static_cast<V*>(y), n_out, n_panels);
  FS_CHECK_LAUNCH("panel_reduce_kernel");
  return FS_OK;
}

template <class V, class I>
int dispatch_ptr(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                 const void* x, void* y, const void* part, void* carry, size_t cb, hipStream_t s) {
  if (plan->ptr_t == FS_I32) return launch_spmv<V, I, int32_t>(plan, vals, cols, indptr, x, y, part, carry, cb, s);
  return launch_spmv<V, I, int64_t>(plan, vals, cols, indptr, x, y, part, carry, cb, s);
}

template <class V>
int dispatch_idx(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                 const void* x, void* y, const void* part, void* carry, size_t cb, hipStream_t s) {
  if (plan->idx_t == FS_I32) return dispatch_ptr<V, int32_t>(plan, vals, cols, indptr, x, y, part, carry, cb, s);
  return dispatch_ptr<V, int64_t>(plan, vals, cols, indptr, x, y, part, carry, cb, s);
}

size_t acc_bytes(int val_t) {
  return (val_t == FS_C64 || val_t == FS_C128) ? sizeof(c64) : sizeof(double);
}


// Kernel choice from the row-length histogram.
void choose_spmv_kernel(fs_csr_plan* plan, int force_kernel) {
  const int64_t n_rows = plan->n_rows;
  const double mean = n_rows > 0 ? (double)plan->nnz / (double)n_rows : 0.0;
  const int items = (plan->val_t == FS_C64 || plan->val_t == FS_C128) ? stream_items<c64>() : stream_items<double>();
  // Rows per workgroup for the streaming kernel: as many as fit the LDS stage.
  int rpb = 256;
  while (rpb > 32 && (int64_t)rpb * plan->max_row > items) rpb >>= 1;
  const bool stream_fits = (int64_t)rpb * plan->max_row <= items;
  // Short rows only -> stream a row block through LDS; anything longer or
  // skewed -> the merge path, which balances rows + nnz exactly.
  int kernel = stream_fits ? FS_KERNEL_STREAM : FS_KERNEL_MERGE;
  const char* env = std::getenv("FLAGSPARSE_SPMV_KERNEL");
  if (env && std::strcmp(env, "vector") == 0) kernel = FS_KERNEL_VECTOR;
  if (env && std::strcmp(env, "merge") == 0) kernel = FS_KERNEL_MERGE;
  if (env && std::strcmp(env, "stream") == 0) kernel = FS_KERNEL_STREAM;
  if (env && std::strcmp(env, "nnzblock") == 0) kernel = FS_KERNEL_NNZBLOCK;
  if (force_kernel == FS_KERNEL_VECTOR || force_kernel == FS_KERNEL_MERGE || force_kernel == FS_KERNEL_STREAM ||
      force_kernel == FS_KERNEL_NNZBLOCK)
    kernel = force_kernel;
  if (kernel == FS_KERNEL_STREAM && !stream_fits) kernel = FS_KERNEL_MERGE;
  if (kernel == FS_KERNEL_NNZBLOCK && plan->nnz == 0) kernel = FS_KERNEL_STREAM;  // nothing to block
  plan->kernel = kernel;
  plan->rows_per_block = rpb;
  int vw = 2;
  while (vw < 64 && (double)vw * kUnroll < mean) vw <<= 1;
  const char* env_vw = std::getenv("FLAGSPARSE_SPMV_VW");
  if (env_vw) {
    const int v = std::atoi(env_vw);
    if (v >= 2 && v <= 64 && (v & (v - 1)) == 0) vw = v;
  }
  plan->vec_width = vw;
  plan->tile_items = kMergeTile;
  plan->n_tiles = ceil_div(n_rows + plan->nnz, kMergeTile);
  if (kernel == FS_KERNEL_NNZBLOCK) {
    // entries per block = the LDS stage; threads per row from the mean row
    // so that one pass of 256 / tpr rows covers a block's rows on average
    plan->tile_items = items;
    plan->n_tiles = ceil_div(plan->nnz, items);
    int tpr = 1;
    while (tpr < 32 && (double)(2 * tpr) * items <= 256.0 * mean) tpr <<= 1;
    plan->vec_width = tpr;
  }
  plan->part_bytes = (size_t)(plan->n_tiles + 1) * sizeof(int64_t);
  plan->carry_bytes = (size_t)plan->n_tiles * 2 * acc_bytes(plan->val_t);
}

template <class V, class I, class P>
int launch_spmv_oneshot(int64_t n_rows, int64_t n_cols, int64_t nnz, const void* vals, const void* cols,
                        const void* indptr, const void* x, void* y, int32_t* flags, hipStream_t stream) {
  using A = typename VT<V>::acc;
  const int64_t blocks = ceil_div(n_rows, (int64_t)64);
  const int remap = xcd_remap();
  const int64_t grid = remap ? ceil_div(blocks, kXcds) * kXcds : blocks;
  if (grid * 256 >= (int64_t(1) << 32)) return fail(FS_E_INVALID, "fs_spmv_csr_oneshot: grid too large");
  const V* v = static_cast<const V*>(vals);
  const I* c = static_cast<const I*>(cols);
  const bool dl = stream_t_dl_enabled() && ((uintptr_t)v % 16) == 0 && ((uintptr_t)c % 16) == 0;
  // The stage holds 64 rows of 1.1 x the average row (rounded up to 64
  // entries, at most the K3t stage): blocks of regular matrices fit it
  // without paying LDS for the longest possible block; a block that does
  // not fit takes the half-block or row-by-row path.
  const int64_t want = ceil_div((nnz * 64 * 11) / 10 + 63, n_rows);
  const int stage = (int)std::min<int64_t>(stream_items<A>(), std::max<int64_t>(64, ceil_div(want, 64) * 64));
  // plus 33 rebased offsets for the half-block path
  const size_t lds = stream_t_layout(stage, sizeof(V), sizeof(I), dl).total + 33 * sizeof(int);
  auto go = [&](auto dc) {
    hipLaunchKernelGGL((spmv_oneshot_kernel<V, I, P, decltype(dc)::value>), dim3((unsigned)grid), dim3(256), lds,
                       stream, v, c, static_cast<const P*>(indptr), static_cast<const V*>(x), static_cast<V*>(y),
                       n_rows, n_cols, nnz, blocks, remap, stage, flags);
  };
  if (dl) go(std::true_type{});
  else go(std::false_type{});
  FS_CHECK_MAIN_LAUNCH("spmv_oneshot_kernel");
  return FS_OK;
}

}  // namespace fs

using namespace fs;

extern "C" size_t fs_csr_stats_bytes(void) { return kStatsWords * sizeof(unsigned long long); }

static void init_plan(fs_csr_plan* plan, int ptr_t, int idx_t, int val_t, int64_t n_rows, int64_t n_cols,
                      int64_t nnz) {
  std::memset(plan, 0, sizeof(*plan));
  plan->n_rows = n_rows;
  plan->n_cols = n_cols;
  plan->nnz = nnz;
  plan->val_t = val_t;
  plan->idx_t = idx_t;
  plan->ptr_t = ptr_t;
}

// Row-length statistics into st[kStatsWords] (no synchronisation).
static int launch_stats(const void* indptr, int ptr_t, int64_t n_rows, unsigned long long* st, hipStream_t stream) {
  hipLaunchKernelGGL(stats_init_kernel, dim3(1), dim3(64), 0, stream, st);
  FS_CHECK_LAUNCH("stats_init_kernel");
  // Each workgroup ends with a handful of global atomics on shared addresses,
  // which serialise in L2, so the grid is bounded: at least 2048 rows per
  // workgroup (8 per lane), at most 1024 workgroups.  Measured on 4 M + 16.7 M
  // rows (a power-law matrix and its 4-panel stacked copy): 256 / 512 / 1024 /
  // 2048 / 4096 workgroups 173 / 113 / 104 / 135 / 177 us.
  int64_t blocks = std::min<int64_t>(ceil_div(n_rows, 2048), 1024);
  if (ptr_t == FS_I32)
    hipLaunchKernelGGL((stats_kernel<int32_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int32_t*>(indptr), n_rows, st);
  else
    hipLaunchKernelGGL((stats_kernel<int64_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int64_t*>(indptr), n_rows, st);
  FS_CHECK_LAUNCH("stats_kernel");
  return FS_OK;
}

static void finish_plan(fs_csr_plan* plan, const unsigned long long* host, int force_kernel) {
  if (plan->n_rows > 0) {
    for (int b = 0; b < FS_HIST_BINS; ++b) plan->hist[b] = (int64_t)host[b];
    plan->max_row = (int64_t)host[FS_HIST_BINS];
    plan->min_row = (int64_t)host[FS_HIST_BINS + 1];
  }
  choose_spmv_kernel(plan, force_kernel);
}

extern "C" int fs_csr_analyze(const void* indptr, int ptr_t, int idx_t, int val_t, int64_t n_rows,
                              int64_t n_cols, int64_t nnz, int force_kernel, void* stats_dev,
                              fs_csr_plan* plan, hipStream_t stream) {
  if (!plan) return fail(FS_E_INVALID, "fs_csr_analyze: plan is null");
  if (!valid_types(val_t, idx_t, ptr_t)) return fail(FS_E_INVALID, "fs_csr_analyze: bad type code");
  if (n_rows < 0 || n_cols < 0 || nnz < 0) return fail(FS_E_INVALID, "fs_csr_analyze: negative size");
  init_plan(plan, ptr_t, idx_t, val_t, n_rows, n_cols, nnz);
  unsigned long long host[kStatsWords] = {};
  if (n_rows > 0) {
    if (!indptr || !stats_dev) return fail(FS_E_INVALID, "fs_csr_analyze: null pointer");
    unsigned long long* st = static_cast<unsigned long long*>(stats_dev);
    const int rc = launch_stats(indptr, ptr_t, n_rows, st, stream);
    if (rc != FS_OK) return rc;
    FS_CHECK_HIP(hipMemcpyAsync(host, st, sizeof(host), hipMemcpyDeviceToHost, stream));
    FS_CHECK_HIP(hipStreamSynchronize(stream));
  }
  finish_plan(plan, host, force_kernel);
  return FS_OK;
}

extern "C" size_t fs_csr_check_bytes(void) { return 5 * sizeof(unsigned long long); }

// Structure-check kernels into ck[5] (no synchronisation).
static int launch_check(const void* indptr, int ptr_t, const void* indices, int idx_t, int64_t n_rows, int64_t nnz,
                        unsigned long long* ck, hipStream_t stream) {
  // enough workgroups to stream the indices at full rate (eight 16-byte
  // loads in flight per lane); each ends with three global atomics on shared
  // addresses, which serialise in L2.  27-point stencil (223 MB of columns),
  // kernel us at 2048 / 1024 / 512 / 256 workgroups: 67.4 / 55.3 / 46.8 /
  // 49.3.  FLAGSPARSE_CHECK_BLOCKS overrides (A/B).
  int64_t cap_blocks = 512;
  if (const char* e = std::getenv("FLAGSPARSE_CHECK_BLOCKS")) cap_blocks = std::max(1, std::atoi(e));
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(std::max(n_rows, nnz), 1024), cap_blocks));
#define FS_CHECK_CASE(P, I)                                                                                   \
  do {                                                                                                        \
    hipLaunchKernelGGL((check_init_kernel<P>), dim3(1), dim3(64), 0, stream, static_cast<const P*>(indptr),   \
                       n_rows, ck);                                                                           \
    FS_CHECK_LAUNCH("check_init_kernel");                                                                     \
    if (reinterpret_cast<uintptr_t>(indices) % 16 == 0)                                                       \
      hipLaunchKernelGGL((check_kernel<P, I, true>), dim3((unsigned)blocks), dim3(256), 0, stream,            \
                         static_cast<const P*>(indptr), n_rows, static_cast<const I*>(indices), nnz, ck);     \
    else                                                                                                      \
      hipLaunchKernelGGL((check_kernel<P, I, false>), dim3((unsigned)blocks), dim3(256), 0, stream,           \
                         static_cast<const P*>(indptr), n_rows, static_cast<const I*>(indices), nnz, ck);     \
    FS_CHECK_LAUNCH("check_kernel");                                                                          \
  } while (0)
  if (ptr_t == FS_I32 && idx_t == FS_I32) FS_CHECK_CASE(int32_t, int32_t);
  else if (ptr_t == FS_I32) FS_CHECK_CASE(int32_t, int64_t);
  else if (idx_t == FS_I32) FS_CHECK_CASE(int64_t, int32_t);
  else FS_CHECK_CASE(int64_t, int64_t);
#undef FS_CHECK_CASE
  return FS_OK;
}

// Structure check and statistics in one kernel (fs_csr_check_analyze).
static int launch_check_stats(const void* indptr, int ptr_t, const void* indices, int idx_t, int64_t n_rows,
                              int64_t nnz, unsigned long long* ck, unsigned long long* st, hipStream_t stream) {
  int64_t cap_blocks = 512;  // as launch_check
  if (const char* e = std::getenv("FLAGSPARSE_CHECK_BLOCKS")) cap_blocks = std::max(1, std::atoi(e));
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(std::max(n_rows, nnz), 1024), cap_blocks));
  hipLaunchKernelGGL(stats_init_kernel, dim3(1), dim3(64), 0, stream, st);
  FS_CHECK_LAUNCH("stats_init_kernel");
#define FS_CHECK_STATS_CASE(P, I)                                                                             \
  do {                                                                                                        \
    hipLaunchKernelGGL((check_init_kernel<P>), dim3(1), dim3(64), 0, stream, static_cast<const P*>(indptr),   \
                       n_rows, ck);                                                                           \
    FS_CHECK_LAUNCH("check_init_kernel");                                                                     \
    if (reinterpret_cast<uintptr_t>(indices) % 16 == 0)                                                       \
      hipLaunchKernelGGL((check_stats_kernel<P, I, true>), dim3((unsigned)blocks), dim3(256), 0, stream,      \
                         static_cast<const P*>(indptr), n_rows, static_cast<const I*>(indices), nnz, ck, st); \
    else                                                                                                      \
      hipLaunchKernelGGL((check_stats_kernel<P, I, false>), dim3((unsigned)blocks), dim3(256), 0, stream,     \
                         static_cast<const P*>(indptr), n_rows, static_cast<const I*>(indices), nnz, ck, st); \
    FS_CHECK_LAUNCH("check_stats_kernel");                                                                    \
  } while (0)
  if (ptr_t == FS_I32 && idx_t == FS_I32) FS_CHECK_STATS_CASE(int32_t, int32_t);
  else if (ptr_t == FS_I32) FS_CHECK_STATS_CASE(int32_t, int64_t);
  else if (idx_t == FS_I32) FS_CHECK_STATS_CASE(int64_t, int32_t);
  else FS_CHECK_STATS_CASE(int64_t, int64_t);
#undef FS_CHECK_STATS_CASE
  return FS_OK;
}

static void decode_check(const unsigned long long* host, int64_t nnz, int64_t* out) {
  out[0] = (int64_t)host[0];
  out[1] = (int64_t)host[1];
  out[2] = (int64_t)host[2];
  out[3] = nnz > 0 ? (int64_t)(host[3] ^ kSignFlip) : 0;
  out[4] = nnz > 0 ? (int64_t)(host[4] ^ kSignFlip) : -1;
}

static int check_args(const char* who, const void* indptr, int ptr_t, const void* indices, int idx_t, int64_t n_rows,
                      int64_t nnz, const void* ws, const int64_t* out) {
  if (!indptr || !ws || !out) return fail(FS_E_INVALID, std::string(who) + ": null pointer");
  if ((ptr_t != FS_I32 && ptr_t != FS_I64) || (idx_t != FS_I32 && idx_t != FS_I64))
    return fail(FS_E_INVALID, std::string(who) + ": bad index type code");
  if (n_rows < 0 || nnz < 0) return fail(FS_E_INVALID, std::string(who) + ": negative size");
  if (nnz > 0 && !indices) return fail(FS_E_INVALID, std::string(who) + ": indices is null");
  return FS_OK;
}

extern "C" int fs_csr_check(const void* indptr, int ptr_t, const void* indices, int idx_t, int64_t n_rows,
                            int64_t nnz, void* check_dev, int64_t* out, hipStream_t stream) {
  int rc = check_args("fs_csr_check", indptr, ptr_t, indices, idx_t, n_rows, nnz, check_dev, out);
  if (rc != FS_OK) return rc;
  unsigned long long* ck = static_cast<unsigned long long*>(check_dev);
  rc = launch_check(indptr, ptr_t, indices, idx_t, n_rows, nnz, ck, stream);
  if (rc != FS_OK) return rc;
  unsigned long long host[5];
  FS_CHECK_HIP(hipMemcpyAsync(host, ck, sizeof(host), hipMemcpyDeviceToHost, stream));
  FS_CHECK_HIP(hipStreamSynchronize(stream));
  decode_check(host, nnz, out);
  return FS_OK;
}

extern "C" int fs_csr_check_enqueue(const void* indptr, int ptr_t, const void* indices, int idx_t, int64_t n_rows,
                                    int64_t nnz, void* check_dev, void* host_words, hipStream_t stream) {
  if (!host_words) return fail(FS_E_INVALID, "fs_csr_check_enqueue: host_words is null");
  const int64_t dummy = 0;
  int rc = check_args("fs_csr_check_enqueue", indptr, ptr_t, indices, idx_t, n_rows, nnz, check_dev, &dummy);
  if (rc != FS_OK) return rc;
  unsigned long long* ck = static_cast<unsigned long long*>(check_dev);
  rc = launch_check(indptr, ptr_t, indices, idx_t, n_rows, nnz, ck, stream);
  if (rc != FS_OK) return rc;
  FS_CHECK_HIP(hipMemcpyAsync(host_words, ck, 5 * sizeof(unsigned long long), hipMemcpyDeviceToHost, stream));
  return FS_OK;
}

extern "C" int fs_csr_check_decode(const void* host_words, int64_t nnz, int64_t* out) {
  if (!host_words || !out) return fail(FS_E_INVALID, "fs_csr_check_decode: null pointer");
  decode_check(static_cast<const unsigned long long*>(host_words), nnz, out);
  return FS_OK;
}

extern "C" size_t fs_csr_check_analyze_bytes(void) { return (5 + kStatsWords) * sizeof(unsigned long long); }

extern "C" int fs_csr_check_analyze(const void* indptr, int ptr_t, const void* indices, int idx_t, int val_t,
                                    int64_t n_rows, int64_t n_cols, int64_t nnz, int force_kernel, void* ws,
                                    int64_t* out, fs_csr_plan* plan, hipStream_t stream) {
  int rc = check_args("fs_csr_check_analyze", indptr, ptr_t, indices, idx_t, n_rows, nnz, ws, out);
  if (rc != FS_OK) return rc;
  if (!plan) return fail(FS_E_INVALID, "fs_csr_check_analyze: plan is null");
  if (!valid_types(val_t, idx_t, ptr_t)) return fail(FS_E_INVALID, "fs_csr_check_analyze: bad type code");
  if (n_cols < 0) return fail(FS_E_INVALID, "fs_csr_check_analyze: negative size");
  init_plan(plan, ptr_t, idx_t, val_t, n_rows, n_cols, nnz);
  unsigned long long* ck = static_cast<unsigned long long*>(ws);
  unsigned long long* st = ck + 5;
  rc = launch_check_stats(indptr, ptr_t, indices, idx_t, n_rows, nnz, ck, st, stream);
  if (rc != FS_OK) return rc;
  unsigned long long host[5 + kStatsWords] = {};
  FS_CHECK_HIP(hipMemcpyAsync(host, ck, (n_rows > 0 ? 5 + kStatsWords : 5) * sizeof(unsigned long long),
                              hipMemcpyDeviceToHost, stream));
  FS_CHECK_HIP(hipStreamSynchronize(stream));
  decode_check(host, nnz, out);
  finish_plan(plan, host + 5, force_kernel);
  return FS_OK;
}

extern "C" int fs_csr_partition(const fs_csr_plan* plan, const void* indptr, void* part_dev,
                                int tile_items, int64_t n_tiles, hipStream_t stream) {
  if (!plan || !part_dev) return fail(FS_E_INVALID, "fs_csr_partition: null pointer");
  if (tile_items <= 0) return fail(FS_E_INVALID, "fs_csr_partition: tile_items must be positive");
  if (n_tiles != ceil_div(plan->n_rows + plan->nnz, tile_items))
    return fail(FS_E_INVALID, "fs_csr_partition: n_tiles does not match tile_items");
  if (plan->n_rows > 0 && !indptr) return fail(FS_E_INVALID, "fs_csr_partition: indptr is null");
  const int64_t blocks = ceil_div(n_tiles + 1, 256);
  if (plan->ptr_t == FS_I32)
    hipLaunchKernelGGL((partition_kernel<int32_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int32_t*>(indptr), plan->n_rows, plan->nnz, (int64_t)tile_items,
                       n_tiles, static_cast<int64_t*>(part_dev));
  else
    hipLaunchKernelGGL((partition_kernel<int64_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int64_t*>(indptr), plan->n_rows, plan->nnz, (int64_t)tile_items,
                       n_tiles, static_cast<int64_t*>(part_dev));
  FS_CHECK_LAUNCH("partition_kernel");
  return FS_OK;
}

extern "C" int fs_spmv_partition(const fs_csr_plan* plan, const void* indptr, void* part_dev, hipStream_t stream) {
  if (!plan || !part_dev) return fail(FS_E_INVALID, "fs_spmv_partition: null pointer");
  if (plan->kernel == FS_KERNEL_MERGE) return fs_csr_partition(plan, indptr, part_dev, plan->tile_items, plan->n_tiles, stream);
  if (plan->kernel != FS_KERNEL_NNZBLOCK) return FS_OK;  // no partition needed
  if (!indptr) return fail(FS_E_INVALID, "fs_spmv_partition: indptr is null");
  const int64_t n_blocks = plan->n_tiles;
  const unsigned blocks = (unsigned)ceil_div(n_blocks + 1, 256);
  if (plan->ptr_t == FS_I32)
    hipLaunchKernelGGL((nnz_partition_kernel<int32_t>), dim3(blocks), dim3(256), 0, stream,
                       static_cast<const int32_t*>(indptr), plan->n_rows, (int64_t)plan->tile_items, n_blocks,
                       static_cast<int64_t*>(part_dev));
  else
    hipLaunchKernelGGL((nnz_partition_kernel<int64_t>), dim3(blocks), dim3(256), 0, stream,
                       static_cast<const int64_t*>(indptr), plan->n_rows, (int64_t)plan->tile_items, n_blocks,
                       static_cast<int64_t*>(part_dev));
  FS_CHECK_LAUNCH("nnz_partition_kernel");
  return FS_OK;
}

extern "C" int fs_spmv_csr(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                           const void* x, void* y, const void* part_dev, void* carry_dev,
                           size_t carry_bytes, hipStream_t stream) {
  if (!plan) return fail(FS_E_INVALID, "fs_spmv_csr: plan is null");
  if (!valid_types(plan->val_t, plan->idx_t, plan->ptr_t)) return fail(FS_E_INVALID, "fs_spmv_csr: bad type code");
  if (plan->n_rows == 0) return FS_OK;
  if (!indptr || !y || (plan->nnz > 0 && (!vals || !cols || !x)))
    return fail(FS_E_INVALID, "fs_spmv_csr: null pointer");
  switch (plan->val_t) {
    case FS_F32: return dispatch_idx<float>(plan, vals, cols, indptr, x, y, part_dev, carry_dev, carry_bytes, stream);
    case FS_F64: return dispatch_idx<double>(plan, vals, cols, indptr, x, y, part_dev, carry_dev, carry_bytes, stream);
    case FS_C64: return dispatch_idx<c32>(plan, vals, cols, indptr, x, y, part_dev, carry_dev, carry_bytes, stream);
    default: return dispatch_idx<c64>(plan, vals, cols, indptr, x, y, part_dev, carry_dev, carry_bytes, stream);
  }
}

extern "C" int fs_spmv_csr_oneshot(int val_t, int idx_t, int ptr_t, int64_t n_rows, int64_t n_cols, int64_t nnz,
                                   const void* vals, const void* cols, const void* indptr, const void* x, void* y,
                                   int32_t* flags, hipStream_t stream) {
  if (!valid_types(val_t, idx_t, ptr_t)) return fail(FS_E_INVALID, "fs_spmv_csr_oneshot: bad type code");
  if (n_rows <= 0 || n_cols <= 0 || nnz <= 0)
    return fail(FS_E_INVALID, "fs_spmv_csr_oneshot: needs rows, columns and entries (use fs_spmv_csr)");
  if (!vals || !cols || !indptr || !x || !y || !flags) return fail(FS_E_INVALID, "fs_spmv_csr_oneshot: null pointer");
  // the kernel writes the flags through the pinned buffer's device mapping
  // (memory that is not pinned and mapped fails here, before any launch)
  void* dflags = nullptr;
  FS_CHECK_HIP(hipHostGetDevicePointer(&dflags, flags, 0));
  for (int k = 0; k < 4; ++k) flags[k] = 0;  // host memory: no copy either way
  int32_t* dev_flags = static_cast<int32_t*>(dflags);
  auto by_idx = [&](auto vtag) -> int {
    using V = decltype(vtag);
    if (idx_t == FS_I32) {
      if (ptr_t == FS_I32)
        return launch_spmv_oneshot<V, int32_t, int32_t>(n_rows, n_cols, nnz, vals, cols, indptr, x, y, dev_flags, stream);
      return launch_spmv_oneshot<V, int32_t, int64_t>(n_rows, n_cols, nnz, vals, cols, indptr, x, y, dev_flags, stream);
    }
    if (ptr_t == FS_I32)
      return launch_spmv_oneshot<V, int64_t, int32_t>(n_rows, n_cols, nnz, vals, cols, indptr, x, y, dev_flags, stream);
    return launch_spmv_oneshot<V, int64_t, int64_t>(n_rows, n_cols, nnz, vals, cols, indptr, x, y, dev_flags, stream);
  };
  int rc;
  switch (val_t) {
    case FS_F32: rc = by_idx(float{}); break;
    case FS_F64: rc = by_idx(double{}); break;
    case FS_C64: rc = by_idx(c32{}); break;
    default: rc = by_idx(c64{}); break;
  }
  if (rc != FS_OK) return rc;
  // the kernel's flags are in host memory once the stream has drained: the
  // caller raises before y is used
  FS_CHECK_HIP(hipStreamSynchronize(stream));
  return FS_OK;
}

// ---------------------------------------------------------------------------
// fs_spmv_csr_noalloc: fs_spmv_csr with its carry workspace (the merge-path
// and entry-block kernels' head / tail fragments of rows that cross tiles)
// in a file-scope device array instead of a caller buffer.  Each GPU holds
// its own copy of the array until the process ends; its address on a device
// comes from hipGetSymbolAddress on the first call there, with that device
// current, and is kept per device.  The kernels write every fragment the
// fix-up reads, so nothing needs clearing between calls.  Calls on one GPU
// from several streams or host threads are ordered on the GPU: each call
// that uses the array records an event on its stream, and a call on another
// stream waits for the previous call's event before its kernels run.  (Under
// stream capture the wait and the record are skipped, and a caller that
// replays captured calls on several streams at once must order them itself.)
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
struct ScratchSlot {
  void* ptr = nullptr;
  hipEvent_t done = nullptr;       // recorded after the latest call's kernels
  hipStream_t last = nullptr;      // the stream of that call
  bool used = false;
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxDevices];
}  // namespace

// Set-up on the first call on a device (with it current): the array's device
// address and the ordering event.  Called with g_scratch_mu held.
static int scratch_for_current_device(ScratchSlot** out) {
  int dev = 0;
  FS_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(FS_E_INVALID, "fs_spmv_csr_noalloc: device id out of range");
  ScratchSlot& s = g_scratch[dev];
  if (s.ptr == nullptr) {
    void* ptr = nullptr;
    FS_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (ptr == nullptr) return fail(FS_E_HIP, "fs_spmv_csr_noalloc: no device address for the scratch array");
    FS_CHECK_HIP(hipEventCreateWithFlags(&s.done, hipEventDisableTiming));
    s.ptr = ptr;
  }
  *out = &s;
  return FS_OK;
}

extern "C" size_t fs_spmv_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int fs_spmv_csr_noalloc(const fs_csr_plan* plan, const void* vals, const void* cols, const void* indptr,
                                   const void* x, void* y, const void* part_dev, hipStream_t stream) {
  if (!plan) return fail(FS_E_INVALID, "fs_spmv_csr_noalloc: plan is null");
  if (!valid_types(plan->val_t, plan->idx_t, plan->ptr_t))
    return fail(FS_E_INVALID, "fs_spmv_csr_noalloc: bad type code");
  if (plan->n_rows == 0) return FS_OK;
  const bool uses_carry = plan->kernel == FS_KERNEL_MERGE || plan->kernel == FS_KERNEL_NNZBLOCK;
  const size_t need = uses_carry ? (size_t)(plan->n_tiles > 0 ? plan->n_tiles : 0) * 2 * acc_bytes(plan->val_t) : 0;
  if (need > kNoAllocScratchBytes)
    return fail(FS_E_WORKSPACE, "fs_spmv_csr_noalloc: the matrix needs " + std::to_string(need) +
                                    " bytes of carry scratch, more than the " + std::to_string(kNoAllocScratchBytes) +
                                    " bytes this entry point holds; call fs_spmv_csr with a workspace");
  if (!uses_carry) return fs_spmv_csr(plan, vals, cols, indptr, x, y, part_dev, nullptr, 0, stream);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot* slot = nullptr;
  int rc = scratch_for_current_device(&slot);
  if (rc != FS_OK) return rc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  FS_CHECK_HIP(hipStreamIsCapturing(stream, &cap));
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order && slot->used && slot->last != stream) FS_CHECK_HIP(hipStreamWaitEvent(stream, slot->done, 0));
  rc = fs_spmv_csr(plan, vals, cols, indptr, x, y, part_dev, slot->ptr, kNoAllocScratchBytes, stream);
  if (rc != FS_OK) return rc;
  if (order) {
    FS_CHECK_HIP(hipEventRecord(slot->done, stream));
    slot->last = stream;
    slot->used = true;
  }
  return FS_OK;
}

extern "C" size_t fs_spmv_panels_workspace_bytes(const fs_csr_plan* plan, int n_panels) {
  if (!plan || n_panels <= 0) return 0;
  return panel_ws(plan, n_panels, acc_bytes(plan->val_t)).total;
}

extern "C" int fs_spmv_csr_panels(const fs_csr_plan* plan, int n_panels, const int64_t* panel_nnz,
                                  const void* vals, const void* cols, const void* indptr, const void* x, void* y,
                                  const void* part_dev, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!plan) return fail(FS_E_INVALID, "fs_spmv_csr_panels: plan is null");
  if (!valid_types(plan->val_t, plan->idx_t, plan->ptr_t))
    return fail(FS_E_INVALID, "fs_spmv_csr_panels: bad type code");
  if (n_panels <= 0 || n_panels > kMaxPanels || plan->n_rows % n_panels != 0)
    return fail(FS_E_INVALID, "fs_spmv_csr_panels: n_rows of the stacked matrix must be a multiple of n_panels (<= 64)");
  if (plan->tile_items != kMergeTile || plan->n_tiles != ceil_div(plan->n_rows + plan->nnz, kMergeTile))
    return fail(FS_E_INVALID, "fs_spmv_csr_panels: plan does not describe merge tiles");
  if (!panel_nnz) return fail(FS_E_INVALID, "fs_spmv_csr_panels: panel_nnz is null");
  if (panel_nnz[0] != 0 || panel_nnz[n_panels] != plan->nnz)
    return fail(FS_E_INVALID, "fs_spmv_csr_panels: panel_nnz must run from 0 to nnz");
  for (int q = 0; q < n_panels; ++q)
    if (panel_nnz[q + 1] < panel_nnz[q]) return fail(FS_E_INVALID, "fs_spmv_csr_panels: panel_nnz must not decrease");
  const int64_t n_out = plan->n_rows / n_panels;
  if (n_out == 0) return FS_OK;
  if (!indptr || !y || !part_dev || (plan->nnz > 0 && (!vals || !cols || !x)))
    return fail(FS_E_INVALID, "fs_spmv_csr_panels: null pointer");
  auto by_idx = [&](auto vtag) -> int {
    using V = decltype(vtag);
    if (plan->idx_t == FS_I32) {
      if (plan->ptr_t == FS_I32)
        return launch_spmv_panels<V, int32_t, int32_t>(plan, n_panels, panel_nnz, vals, cols, indptr, x, y, part_dev, ws, ws_bytes, n_out, stream);
      return launch_spmv_panels<V, int32_t, int64_t>(plan, n_panels, panel_nnz, vals, cols, indptr, x, y, part_dev, ws, ws_bytes, n_out, stream);
    }
    if (plan->ptr_t == FS_I32)
      return launch_spmv_panels<V, int64_t, int32_t>(plan, n_panels, panel_nnz, vals, cols, indptr, x, y, part_dev, ws, ws_bytes, n_out, stream);
    return launch_spmv_panels<V, int64_t, int64_t>(plan, n_panels, panel_nnz, vals, cols, indptr, x, y, part_dev, ws, ws_bytes, n_out, stream);
  };
  switch (plan->val_t) {
    case FS_F32: return by_idx(float{});
    case FS_F64: return by_idx(double{});
    case FS_C64: return by_idx(c32{});
    default: return by_idx(c64{});
  }
}
