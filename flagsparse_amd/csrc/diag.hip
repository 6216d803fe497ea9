// diag.hip — a diagnostic kernel, not part of the operator path: the rate at
// which the GPU returns rows of B (or entries of x) gathered in a given index
// order, with nothing else in flight.  It is the floor the SpMM (SpMV)
// kernels are measured against on matrices whose gathers miss the caches
// (bench.py --gather-floor).  Built into its own library,
// libflagsparse_diag.so (C ABI in flagsparse_diag.h), not the product one.
//
// A wave splits into 64 / LPR groups of LPR lanes; lane l of a group loads
// the l-th 16 bytes of its row, so one instruction gathers 64 / LPR rows.
// Each wave keeps kDiagU such instructions in flight and folds the loaded
// words into an XOR checksum (one word per run), so no load is dead code.
#include "fs_common.hpp"
#include "flagsparse_diag.h"

#include <type_traits>

namespace fs {

constexpr int kDiagU = 8;

// An index clamped into [0, n): a stray value reads a row of B, never past it.
template <class I>
__device__ inline int64_t clamp_row(I r, int64_t n) {
  const int64_t v = (int64_t)r;
  return v < 0 ? 0 : (v >= n ? n - 1 : v);
}

template <int LPR, class I>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint4* __restrict__ B, int64_t row_vecs,
                                                          int64_t n_b_rows, const I* __restrict__ idx, int64_t n_idx,
                                                          unsigned* __restrict__ out) {
  constexpr int G = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int grp = lane / LPR;
  const int gl = lane % LPR;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  unsigned acc = 0;
  for (int64_t s0 = wave * (G * kDiagU); s0 < n_idx; s0 += n_waves * (G * kDiagU)) {
    uint4 v[kDiagU];
#pragma unroll
    for (int u = 0; u < kDiagU; ++u) {
      int64_t e = s0 + (int64_t)u * G + grp;
      e = e < n_idx ? e : n_idx - 1;  // every load issued: a repeat past the end
      v[u] = B[clamp_row(idx[e], n_b_rows) * row_vecs + gl];
    }
#pragma unroll
    for (int u = 0; u < kDiagU; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (int off = 32; off > 0; off >>= 1) acc ^= (unsigned)__shfl_xor((int)acc, off);
  __shared__ unsigned s_acc[4];
  if (lane == 0) s_acc[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) atomicXor(out, s_acc[0] ^ s_acc[1] ^ s_acc[2] ^ s_acc[3]);
}

// Rows of 4 or 8 bytes (SpMV x entries): one row per lane, index loads
// coalesced, kDiagU gathers in flight per lane.
template <class W, class I>
__global__ __launch_bounds__(256) void gather_words_kernel(const W* __restrict__ x, int64_t n_b_rows,
                                                           const I* __restrict__ idx, int64_t n_idx, unsigned* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  unsigned acc = 0;
  for (int64_t s0 = wave * (64 * kDiagU); s0 < n_idx; s0 += n_waves * (64 * kDiagU)) {
    W v[kDiagU];
#pragma unroll
    for (int u = 0; u < kDiagU; ++u) {
      int64_t e = s0 + (int64_t)u * 64 + lane;
      e = e < n_idx ? e : n_idx - 1;
      v[u] = x[clamp_row(idx[e], n_b_rows)];
    }
#pragma unroll
    for (int u = 0; u < kDiagU; ++u) {
      if constexpr (sizeof(W) == 8)
        acc ^= (unsigned)v[u] ^ (unsigned)(v[u] >> 32);
      else
        acc ^= (unsigned)v[u];
    }
  }
  for (int off = 32; off > 0; off >>= 1) acc ^= (unsigned)__shfl_xor((int)acc, off);
  __shared__ unsigned s_acc[4];
  if (lane == 0) s_acc[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) atomicXor(out, s_acc[0] ^ s_acc[1] ^ s_acc[2] ^ s_acc[3]);
}

template <class I>
int launch_gather(const void* B, int64_t n_b_rows, int64_t row_bytes, const void* idx, int64_t n_idx, unsigned* out,
                  hipStream_t stream) {
  if (row_bytes < 16) {
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n_idx, 4 * 64 * kDiagU), 8192));
    if (row_bytes == 4)
      hipLaunchKernelGGL((gather_words_kernel<uint32_t, I>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const uint32_t*>(B), n_b_rows, static_cast<const I*>(idx), n_idx, out);
    else
      hipLaunchKernelGGL((gather_words_kernel<uint64_t, I>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const uint64_t*>(B), n_b_rows, static_cast<const I*>(idx), n_idx, out);
    FS_CHECK_LAUNCH("gather_words_kernel");
    return FS_OK;
  }
  const int lpr = (int)(row_bytes / 16);
  const int64_t rows_per_wave_step = (int64_t)(64 / lpr) * kDiagU;
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n_idx, 4 * rows_per_wave_step), 8192));
  const int64_t row_vecs = row_bytes / 16;
  const uint4* b = static_cast<const uint4*>(B);
  const I* ix = static_cast<const I*>(idx);
  switch (lpr) {
    case 1: hipLaunchKernelGGL((gather_rows_kernel<1, I>), dim3((unsigned)blocks), dim3(256), 0, stream, b, row_vecs, n_b_rows, ix, n_idx, out); break;
    case 2: hipLaunchKernelGGL((gather_rows_kernel<2, I>), dim3((unsigned)blocks), dim3(256), 0, stream, b, row_vecs, n_b_rows, ix, n_idx, out); break;
    case 4: hipLaunchKernelGGL((gather_rows_kernel<4, I>), dim3((unsigned)blocks), dim3(256), 0, stream, b, row_vecs, n_b_rows, ix, n_idx, out); break;
    case 8: hipLaunchKernelGGL((gather_rows_kernel<8, I>), dim3((unsigned)blocks), dim3(256), 0, stream, b, row_vecs, n_b_rows, ix, n_idx, out); break;
    case 16: hipLaunchKernelGGL((gather_rows_kernel<16, I>), dim3((unsigned)blocks), dim3(256), 0, stream, b, row_vecs, n_b_rows, ix, n_idx, out); break;
    case 32: hipLaunchKernelGGL((gather_rows_kernel<32, I>), dim3((unsigned)blocks), dim3(256), 0, stream, b, row_vecs, n_b_rows, ix, n_idx, out); break;
    default: hipLaunchKernelGGL((gather_rows_kernel<64, I>), dim3((unsigned)blocks), dim3(256), 0, stream, b, row_vecs, n_b_rows, ix, n_idx, out); break;
  }
  FS_CHECK_LAUNCH("gather_rows_kernel");
  return FS_OK;
}

}  // namespace fs

using namespace fs;

extern "C" int fs_diag_gather_rows(int idx_t, const void* B, int64_t n_b_rows, int64_t row_bytes, const void* idx,
                                   int64_t n_idx, void* checksum, hipStream_t stream) {
  if (idx_t != FS_I32 && idx_t != FS_I64) return fail(FS_E_INVALID, "fs_diag_gather_rows: bad index type code");
  if (row_bytes < 4 || row_bytes > 1024 || (row_bytes & (row_bytes - 1)))
    return fail(FS_E_INVALID, "fs_diag_gather_rows: row_bytes must be a power of two in [4, 1024]");
  if (n_idx < 0 || n_b_rows <= 0) return fail(FS_E_INVALID, "fs_diag_gather_rows: bad size");
  if (n_idx == 0) return FS_OK;
  if (!B || !idx || !checksum) return fail(FS_E_INVALID, "fs_diag_gather_rows: null pointer");
  if ((reinterpret_cast<uintptr_t>(B) % (row_bytes < 16 ? row_bytes : 16)) != 0)
    return fail(FS_E_INVALID, "fs_diag_gather_rows: B must be aligned to min(row_bytes, 16) bytes");
  unsigned* out = static_cast<unsigned*>(checksum);
  return idx_t == FS_I32 ? launch_gather<int32_t>(B, n_b_rows, row_bytes, idx, n_idx, out, stream)
                         : launch_gather<int64_t>(B, n_b_rows, row_bytes, idx, n_idx, out, stream);
}
