// spmv_opt.hip — the native-precision, row-length-bucketed CSR SpMV behind
// flagsparse_spmv_csr(..., use_opt=True) for gfx950.
//
// Replaces the reference's opt path: the bucket tiers of
// _SPMV_OPT_BUCKET_CONFIGS / _SPMV_OPT_BUCKET_CONFIGS_FP64 and
// _build_spmv_opt_buckets (spmv_csr.py:136-161, 353-410), and the four
// Triton kernels _spmv_csr_batched_short_f32/f64 and
// _spmv_csr_vector_rows_f32/f64 launched per bucket by
// _triton_spmv_csr_impl_opt_prepared (spmv_csr.py:233-351, 412-461).  As
// there, float32 accumulates in float32 and float64 in float64, and the
// first bucket holds the empty rows, so every row is written once.
//
// Buckets are built on the device: one counting pass (per-workgroup LDS
// counts, one global atomic per bucket and workgroup), a one-thread scan,
// and a scatter whose per-wave ranks come from ballots (one global atomic
// per bucket and wave).  Row order inside a bucket is unspecified, as it
// only decides which wave computes a row; each row's sum has a fixed order,
// so y is bit-reproducible.  A bucket runs L lanes per row (a row's
// entries are strided over its lanes, each lane keeps four loads in
// flight) and a fixed butterfly reduction.
#include "fs_common.hpp"

#include <cstring>
#include <type_traits>

namespace fs {

constexpr int kOptMaxBuckets = 5;

// Upper row-length bound of each tier (-1 = unbounded) and lanes per row.
struct OptTiers {
  int n;
  int64_t upper[kOptMaxBuckets];
  int lanes[kOptMaxBuckets];
};

inline OptTiers opt_tiers(int val_t) {
  if (val_t == FS_F64) return OptTiers{5, {64, 256, 2048, 8192, -1}, {8, 32, 64, 256, 256}};
  return OptTiers{4, {64, 512, 4096, -1, -1}, {8, 64, 256, 256, 256}};
}

__device__ inline int opt_bucket_of(int64_t len, const int64_t* upper, int n) {
  int b = 0;
  while (b < n - 1 && len > upper[b]) ++b;
  return b;
}

template <class P>
__global__ __launch_bounds__(256) void opt_count_kernel(const P* __restrict__ indptr, int64_t n_rows,
                                                        OptTiers tiers, unsigned long long* __restrict__ counts) {
  __shared__ unsigned int c[kOptMaxBuckets];
  if (threadIdx.x < kOptMaxBuckets) c[threadIdx.x] = 0;
  __syncthreads();
  for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < n_rows; r += (int64_t)gridDim.x * 256) {
    const int64_t len = (int64_t)indptr[r + 1] - (int64_t)indptr[r];
    atomicAdd(&c[opt_bucket_of(len, tiers.upper, tiers.n)], 1u);
  }
  __syncthreads();
  if (threadIdx.x < (unsigned)tiers.n && c[threadIdx.x]) atomicAdd(&counts[threadIdx.x], (unsigned long long)c[threadIdx.x]);
}

__global__ void opt_offsets_kernel(const unsigned long long* __restrict__ counts,
                                   unsigned long long* __restrict__ cursor, int n) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    unsigned long long s = 0;
    for (int b = 0; b < n; ++b) {
      cursor[b] = s;
      s += counts[b];
    }
  }
}

__global__ void opt_zero_kernel(unsigned long long* __restrict__ p, int n) {
  if ((int)threadIdx.x < n) p[threadIdx.x] = 0;
}

template <class P, class R>
__global__ __launch_bounds__(256) void opt_scatter_kernel(const P* __restrict__ indptr, int64_t n_rows,
                                                          OptTiers tiers, unsigned long long* __restrict__ cursor,
                                                          R* __restrict__ rows) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * 256;
  // every wave runs the same trip count, so the ballots see full waves
  const int64_t trips = (n_rows + stride - 1) / stride;
  for (int64_t t = 0; t < trips; ++t) {
    const int64_t r = t * stride + (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool in = r < n_rows;
    const int b = in ? opt_bucket_of((int64_t)indptr[r + 1] - (int64_t)indptr[r], tiers.upper, tiers.n) : -1;
    for (int k = 0; k < tiers.n; ++k) {
      const unsigned long long m = __ballot(b == k);
      if (m == 0) continue;
      unsigned long long base = 0;
      const int leader = __ffsll((long long)m) - 1;
      if (lane == leader) base = atomicAdd(&cursor[k], (unsigned long long)__popcll(m));
      base = __shfl(base, leader);
      if (b == k) {
        const unsigned long long below = m & ((1ull << lane) - 1ull);
        rows[base + __popcll(below)] = (R)r;
      }
    }
  }
}

template <class T>
__device__ inline T xor_shfl(T v, int mask) {
  return __shfl_xor(v, mask);
}

// L (8, 32 or 64) lanes per row, 256 / L rows per workgroup per step; the
// workgroups stride over the bucket (the trip count depends only on the
// workgroup, so every lane of a group takes part in the reduction).
template <class V, class I, class P, class R, int L>
__global__ __launch_bounds__(256) void opt_rows_kernel(const V* __restrict__ vals, const I* __restrict__ cols,
                                                       const P* __restrict__ indptr, const V* __restrict__ x,
                                                       V* __restrict__ y, const R* __restrict__ rows,
                                                       int64_t n_bucket) {
  constexpr int RPB = 256 / L;
  const int gl = threadIdx.x % L;
  for (int64_t base = (int64_t)blockIdx.x * RPB; base < n_bucket; base += (int64_t)gridDim.x * RPB) {
    const int64_t slot = base + threadIdx.x / L;
    const bool in = slot < n_bucket;
    const int64_t row = in ? (int64_t)rows[slot] : 0;
    const int64_t start = in ? (int64_t)indptr[row] : 0;
    const int64_t end = in ? (int64_t)indptr[row + 1] : 0;
    V acc0 = V(0), acc1 = V(0), acc2 = V(0), acc3 = V(0);
    int64_t k = start + gl;
    for (; k + 3 * L < end; k += 4 * L) {
      const I c0 = cols[k], c1 = cols[k + L], c2 = cols[k + 2 * L], c3 = cols[k + 3 * L];
      const V a0 = vals[k], a1 = vals[k + L], a2 = vals[k + 2 * L], a3 = vals[k + 3 * L];
      acc0 = __builtin_fma(a0, x[c0], acc0);
      acc1 = __builtin_fma(a1, x[c1], acc1);
      acc2 = __builtin_fma(a2, x[c2], acc2);
      acc3 = __builtin_fma(a3, x[c3], acc3);
    }
    for (; k < end; k += L) acc0 = __builtin_fma(vals[k], x[cols[k]], acc0);
    V s = (acc0 + acc1) + (acc2 + acc3);
#pragma unroll
    for (int m = L / 2; m >= 1; m >>= 1) s += xor_shfl(s, m);
    if (in && gl == 0) y[row] = s;
  }
}

// One 256-thread workgroup per row (the long-row tiers).
template <class V, class I, class P, class R>
__global__ __launch_bounds__(256) void opt_block_kernel(const V* __restrict__ vals, const I* __restrict__ cols,
                                                        const P* __restrict__ indptr, const V* __restrict__ x,
                                                        V* __restrict__ y, const R* __restrict__ rows) {
  __shared__ V part[4];
  const int64_t row = (int64_t)rows[blockIdx.x];
  const int64_t start = (int64_t)indptr[row];
  const int64_t end = (int64_t)indptr[row + 1];
  constexpr int L = 256;
  V acc0 = V(0), acc1 = V(0), acc2 = V(0), acc3 = V(0);
  int64_t k = start + threadIdx.x;
  for (; k + 3 * L < end; k += 4 * L) {
    const I c0 = cols[k], c1 = cols[k + L], c2 = cols[k + 2 * L], c3 = cols[k + 3 * L];
    const V a0 = vals[k], a1 = vals[k + L], a2 = vals[k + 2 * L], a3 = vals[k + 3 * L];
    acc0 = __builtin_fma(a0, x[c0], acc0);
    acc1 = __builtin_fma(a1, x[c1], acc1);
    acc2 = __builtin_fma(a2, x[c2], acc2);
    acc3 = __builtin_fma(a3, x[c3], acc3);
  }
  for (; k < end; k += L) acc0 = __builtin_fma(vals[k], x[cols[k]], acc0);
  V s = (acc0 + acc1) + (acc2 + acc3);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += xor_shfl(s, m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) y[row] = (part[0] + part[1]) + (part[2] + part[3]);
}

inline bool rows32(int64_t n_rows) { return n_rows <= 0x7fffffffLL; }

template <class V, class I, class P, class R>
int launch_opt(const OptTiers& t, const void* vals, const void* cols, const void* indptr, const void* x, void* y,
               const R* rows, const int64_t* counts, hipStream_t s) {
  int64_t off = 0;
  for (int b = 0; b < t.n; ++b) {
    const int64_t n = counts[b];
    if (n == 0) continue;
    const R* rb = rows + off;
    off += n;
    const V* v = static_cast<const V*>(vals);
    const I* c = static_cast<const I*>(cols);
    const P* p = static_cast<const P*>(indptr);
    const V* xv = static_cast<const V*>(x);
    V* yv = static_cast<V*>(y);
    const int L = t.lanes[b];
    if (L == 256) {
      if (n >= (int64_t(1) << 24)) return fail(FS_E_INVALID, "fs_spmv_csr_opt: too many long rows for one grid");
      hipLaunchKernelGGL((opt_block_kernel<V, I, P, R>), dim3((unsigned)n), dim3(256), 0, s, v, c, p, xv, yv, rb);
    } else {
      // at most 2^20 workgroups (the dispatch counts work-items in 32 bits)
      const int64_t blocks = std::min<int64_t>(ceil_div(n * L, 256), int64_t(1) << 20);
      if (L == 8)
        hipLaunchKernelGGL((opt_rows_kernel<V, I, P, R, 8>), dim3((unsigned)blocks), dim3(256), 0, s, v, c, p, xv, yv, rb, n);
      else if (L == 32)
        hipLaunchKernelGGL((opt_rows_kernel<V, I, P, R, 32>), dim3((unsigned)blocks), dim3(256), 0, s, v, c, p, xv, yv, rb, n);
      else
        hipLaunchKernelGGL((opt_rows_kernel<V, I, P, R, 64>), dim3((unsigned)blocks), dim3(256), 0, s, v, c, p, xv, yv, rb, n);
    }
    FS_CHECK_LAUNCH("fs_spmv_csr_opt");
  }
  return FS_OK;
}

template <class V, class R>
int launch_opt_ip(int idx_t, int ptr_t, const OptTiers& t, const void* vals, const void* cols, const void* indptr,
                  const void* x, void* y, const R* rows, const int64_t* counts, hipStream_t s) {
  if (idx_t != FS_I32) return fail(FS_E_INVALID, "fs_spmv_csr_opt: column indices must be int32");
  if (ptr_t == FS_I64) return launch_opt<V, int32_t, int64_t, R>(t, vals, cols, indptr, x, y, rows, counts, s);
  return launch_opt<V, int32_t, int32_t, R>(t, vals, cols, indptr, x, y, rows, counts, s);
}

}  // namespace fs

using namespace fs;

extern "C" int fs_spmv_opt_max_buckets(void) { return kOptMaxBuckets; }

extern "C" size_t fs_spmv_opt_workspace_bytes(int64_t n_rows) {
  const size_t rb = rows32(n_rows) ? 4 : 8;
  return 256 + (size_t)(n_rows > 0 ? n_rows : 0) * rb;
}

extern "C" int fs_spmv_opt_buckets(const void* indptr, int ptr_t, int val_t, int64_t n_rows, void* ws, size_t ws_bytes,
                                   int64_t* counts_out, hipStream_t stream) {
  if (val_t != FS_F32 && val_t != FS_F64) return fail(FS_E_INVALID, "fs_spmv_opt_buckets: float32 / float64 only");
  if (ptr_t != FS_I32 && ptr_t != FS_I64) return fail(FS_E_INVALID, "fs_spmv_opt_buckets: bad index type");
  if (n_rows < 0 || !counts_out) return fail(FS_E_INVALID, "fs_spmv_opt_buckets: bad argument");
  for (int b = 0; b < kOptMaxBuckets; ++b) counts_out[b] = 0;
  if (n_rows == 0) return FS_OK;
  if (!indptr || !ws || ws_bytes < fs_spmv_opt_workspace_bytes(n_rows))
    return fail(FS_E_WORKSPACE, "fs_spmv_opt_buckets: workspace too small");
  const OptTiers t = opt_tiers(val_t);
  unsigned long long* counts = static_cast<unsigned long long*>(ws);
  unsigned long long* cursor = counts + kOptMaxBuckets;
  void* rows = static_cast<char*>(ws) + 256;
  const int64_t blocks = std::min<int64_t>(ceil_div(n_rows, 256), 4096);
  hipLaunchKernelGGL(opt_zero_kernel, dim3(1), dim3(64), 0, stream, counts, 2 * kOptMaxBuckets);
  FS_CHECK_LAUNCH("opt_zero_kernel");
  if (ptr_t == FS_I64)
    hipLaunchKernelGGL((opt_count_kernel<int64_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int64_t*>(indptr), n_rows, t, counts);
  else
    hipLaunchKernelGGL((opt_count_kernel<int32_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const int32_t*>(indptr), n_rows, t, counts);
  FS_CHECK_LAUNCH("opt_count_kernel");
  hipLaunchKernelGGL(opt_offsets_kernel, dim3(1), dim3(64), 0, stream, counts, cursor, t.n);
  FS_CHECK_LAUNCH("opt_offsets_kernel");
  auto scatter = [&](auto* rp) {
    using R = std::remove_pointer_t<decltype(rp)>;
    if (ptr_t == FS_I64)
      hipLaunchKernelGGL((opt_scatter_kernel<int64_t, R>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const int64_t*>(indptr), n_rows, t, cursor, rp);
    else
      hipLaunchKernelGGL((opt_scatter_kernel<int32_t, R>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const int32_t*>(indptr), n_rows, t, cursor, rp);
  };
  if (rows32(n_rows)) scatter(static_cast<int32_t*>(rows));
  else scatter(static_cast<int64_t*>(rows));
  FS_CHECK_LAUNCH("opt_scatter_kernel");
  unsigned long long h[kOptMaxBuckets];
  FS_CHECK_HIP(hipMemcpyAsync(h, counts, sizeof(h), hipMemcpyDeviceToHost, stream));
  FS_CHECK_HIP(hipStreamSynchronize(stream));
  for (int b = 0; b < kOptMaxBuckets; ++b) counts_out[b] = b < t.n ? (int64_t)h[b] : 0;
  return FS_OK;
}

extern "C" int fs_spmv_csr_opt(int val_t, int idx_t, int ptr_t, int64_t n_rows, const void* vals, const void* cols,
                               const void* indptr, const void* x, void* y, const void* ws, size_t ws_bytes,
                               const int64_t* counts, hipStream_t stream) {
  if (val_t != FS_F32 && val_t != FS_F64) return fail(FS_E_INVALID, "fs_spmv_csr_opt: float32 / float64 only");
  if ((ptr_t != FS_I32 && ptr_t != FS_I64) || !counts || n_rows < 0)
    return fail(FS_E_INVALID, "fs_spmv_csr_opt: bad argument");
  if (n_rows == 0) return FS_OK;
  if (!ws || ws_bytes < fs_spmv_opt_workspace_bytes(n_rows) || !indptr || !y || !x)
    return fail(FS_E_INVALID, "fs_spmv_csr_opt: null pointer or workspace too small");
  int64_t total = 0;
  for (int b = 0; b < kOptMaxBuckets; ++b) {
    if (counts[b] < 0) return fail(FS_E_INVALID, "fs_spmv_csr_opt: negative bucket count");
    total += counts[b];
  }
  if (total != n_rows) return fail(FS_E_INVALID, "fs_spmv_csr_opt: bucket counts do not add up to n_rows");
  const OptTiers t = opt_tiers(val_t);
  const void* rows = static_cast<const char*>(ws) + 256;
  if (val_t == FS_F32) {
    if (rows32(n_rows))
      return launch_opt_ip<float, int32_t>(idx_t, ptr_t, t, vals, cols, indptr, x, y, static_cast<const int32_t*>(rows), counts, stream);
    return launch_opt_ip<float, int64_t>(idx_t, ptr_t, t, vals, cols, indptr, x, y, static_cast<const int64_t*>(rows), counts, stream);
  }
  if (rows32(n_rows))
    return launch_opt_ip<double, int32_t>(idx_t, ptr_t, t, vals, cols, indptr, x, y, static_cast<const int32_t*>(rows), counts, stream);
  return launch_opt_ip<double, int64_t>(idx_t, ptr_t, t, vals, cols, indptr, x, y, static_cast<const int64_t*>(rows), counts, stream);
}
