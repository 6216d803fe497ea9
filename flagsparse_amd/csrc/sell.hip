// sell.hip — sliced-ELL (SELL-64) copy of a CSR matrix and its SpMV, gfx950.
//
// A prepared matrix whose rows are short and of similar length (stencils,
// FEM meshes) is copied once into SELL-64: rows are cut into slices of 64
// consecutive rows, one slice per wave, and entry k of each row is stored
// next to entry k of the slice's other rows, so a wave's load of one slot
// is one coalesced 64-lane access.  In the pair layout (real values with
// 16-bit column offsets) a row's slots 2i and 2i+1 also sit side by side,
// so each lane loads two slots with one vector load.  Rows keep their CSR
// entry order, and each lane sums its own row sequentially in the
// accumulator type (f64 for f32 data): no cross-lane reduction, no LDS.
//
// What it buys over the row-block stream kernel: on matrices whose
// neighbouring rows have neighbouring columns (a stencil's slot j of rows
// r..r+63 gathers x[r + offset_j .. r + 63 + offset_j]) the x gather becomes
// as coalesced as the A stream, which takes most of the per-CU address work
// off the gather.  Slots past a row's length are padding: never gathered,
// never multiplied (an inf / nan in x cannot leak in through 0 * x).
//
// Reference path replaced: the per-row SpMV kernels behind
// _triton_spmv_csr_impl_prepared (spmv_csr.py:166-227, 679-723); the format
// is this build's own prepared copy, like the fp64 value copy the
// reference's prepare caches (spmv_csr.py:124-130).
#include "fs_common.hpp"

#include <algorithm>
#include <cstdlib>
#include <vector>
#include <type_traits>

namespace fs {

template <class T>
struct type_tag {
  using type = T;
};

constexpr int kSellRows = 64;  // rows per slice = wave width

// slots[s] = longest row of slice s.
template <class P>
__global__ __launch_bounds__(256) void sell_slots_kernel(const P* __restrict__ rowptr, int64_t n_rows,
                                                         int64_t n_slices, int64_t* __restrict__ slots) {
  const int lane = threadIdx.x & 63;
  const int64_t slice = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (slice >= n_slices) return;  // whole wave
  const int64_t r = slice * kSellRows + lane;
  int64_t len = r < n_rows ? (int64_t)rowptr[r + 1] - (int64_t)rowptr[r] : 0;
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t o = (int64_t)__shfl_xor((long long)len, off);
    len = o > len ? o : len;
  }
  if (lane == 0) slots[slice] = len;
}

// Entry k of row r goes to slice_ptr[r / 64] + (k / G) * 64 G + G (r % 64)
// + k % G with G slots side by side: 1 (slot layout) or 2 (pair layout).
//
// Build kernels: one wave per slice.  A slice's entries are contiguous in
// the CSR arrays, so the wave reads them with unit stride; each entry's row
// inside the slice comes from a binary search over the slice's 65 row
// pointers in LDS.  Writes stay inside the slice's region of the copy.
__device__ inline int sell_local_row(const int64_t* ptr, int64_t e) {
  int lo = 0, hi = kSellRows - 1;  // last local row whose start <= e
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ptr[mid] <= e)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// Loads the 65 row pointers of slice `slice` (rows past n_rows repeat the end).
template <class P>
__device__ inline void sell_load_ptr(const P* __restrict__ rowptr, int64_t n_rows, int64_t slice, int lane,
                                     int64_t* ptr) {
  const int64_t r = slice * kSellRows + lane;
  ptr[lane] = (int64_t)rowptr[r < n_rows ? r : n_rows];
  if (lane == 0) {
    const int64_t r_end = slice * kSellRows + kSellRows;
    ptr[kSellRows] = (int64_t)rowptr[r_end < n_rows ? r_end : n_rows];
  }
}

// With DELTA the column is stored as the 16-bit offset c - r from the row
// (the caller has checked |c - r| <= 32767 with fs_sell_max_offset).
// GROUP (1 or 2): consecutive slots of a row stored side by side.
// With SI = uint8_t the column is stored as the code lut[c - r + 32768] of
// its offset (the caller has built lut from fs_sell_max_offset's bitmap).
template <class V, class I, class P, class SI, bool DELTA, int GROUP>
__global__ __launch_bounds__(256) void sell_fill_kernel(const V* __restrict__ vals, const I* __restrict__ cols,
                                                        const P* __restrict__ rowptr, int64_t n_rows,
                                                        const int64_t* __restrict__ slice_ptr,
                                                        const uint8_t* __restrict__ lut,
                                                        V* __restrict__ sell_vals, SI* __restrict__ sell_cols) {
  __shared__ int64_t s_ptr[4][kSellRows + 1];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t n_slices = (n_rows + kSellRows - 1) / kSellRows;
  const int64_t slice = (int64_t)blockIdx.x * 4 + w;
  if (slice >= n_slices) return;  // whole wave; no block barrier below
  int64_t* ptr = s_ptr[w];
  sell_load_ptr(rowptr, n_rows, slice, lane, ptr);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int64_t base = slice_ptr[slice];
  const int64_t row0 = slice * kSellRows;
  // Entry-major: loads are coalesced, stores scattered over the slice's slots.
  // Measured against it on the 27-point 128^3 stencil (0.55 ms, plus 0.08 ms
  // for the caller's zero fill of the padding): lanes walking the output
  // slots with coalesced stores and scattered loads, 1.0 ms; the slice staged
  // in LDS (one wave per workgroup, 24 KB), then slot-order stores with the
  // padding written, 0.71 ms.
  for (int64_t e = ptr[0] + lane; e < ptr[kSellRows]; e += kSellRows) {
    const int lr = sell_local_row(ptr, e);
    const unsigned k = (unsigned)(e - ptr[lr]);  // rows hold < 2^31 entries
    const int64_t dst = base + (int64_t)(k / GROUP) * (GROUP * kSellRows) + GROUP * lr + (int)(k % GROUP);
    sell_vals[dst] = vals[e];
    const I c = cols[e];
    if constexpr (std::is_same<SI, uint8_t>::value)
      sell_cols[dst] = lut[(int64_t)c - (row0 + lr) + 32768];
    else
      sell_cols[dst] = DELTA ? (SI)((int64_t)c - (row0 + lr)) : (SI)c;
  }
}

// max over entries of |c - r|.  Waves stride over slices; the workgroup
// reduces in LDS and issues one integer atomic (order independent).  An
// atomic per slice on the one address serialised in L2: 390 us for 32 K
// slices.
constexpr int kSellMaxOffsetBlocks = 1024;

// With a bitmap (kSellOffsetWords words, bit d + 32768 for offset d) every
// offset with |d| <= 32767 also sets its bit: LDS bits per workgroup, then
// one global atomic OR per non-zero word.
constexpr int kSellOffsetWords = 65536 / 32;

template <class I, class P, bool BITS>
__global__ __launch_bounds__(256) void sell_max_offset_kernel(const I* __restrict__ cols, const P* __restrict__ rowptr,
                                                              int64_t n_rows, unsigned long long* __restrict__ out,
                                                              unsigned* __restrict__ bitmap) {
  __shared__ int64_t s_ptr[4][kSellRows + 1];
  __shared__ unsigned long long s_max[4];
  __shared__ unsigned s_bits[BITS ? kSellOffsetWords : 1];
  if constexpr (BITS) {
    for (int k = threadIdx.x; k < kSellOffsetWords; k += 256) s_bits[k] = 0u;
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t n_slices = (n_rows + kSellRows - 1) / kSellRows;
  int64_t* ptr = s_ptr[w];
  unsigned long long m = 0;
  for (int64_t slice = (int64_t)blockIdx.x * 4 + w; slice < n_slices; slice += (int64_t)gridDim.x * 4) {
    sell_load_ptr(rowptr, n_rows, slice, lane, ptr);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t row0 = slice * kSellRows;
    for (int64_t e = ptr[0] + lane; e < ptr[kSellRows]; e += kSellRows) {
      const int64_t d = (int64_t)cols[e] - (row0 + sell_local_row(ptr, e));
      const unsigned long long a = (unsigned long long)(d < 0 ? -d : d);
      m = a > m ? a : m;
      if constexpr (BITS) {
        if (a <= 32767) {
          const unsigned b = (unsigned)(d + 32768);
          atomicOr(&s_bits[b >> 5], 1u << (b & 31));
        }
      }
    }
    // the next slice overwrites ptr: every lane has finished reading it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(m, off);
    m = o > m ? o : m;
  }
  if (lane == 0) s_max[w] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k) m = s_max[k] > m ? s_max[k] : m;
    if (m > 0) atomicMax(out, m);
  }
  if constexpr (BITS) {
    for (int k = threadIdx.x; k < kSellOffsetWords; k += 256)
      if (s_bits[k]) atomicOr(&bitmap[k], s_bits[k]);
  }
}

// One wave per slice, lane = row.  Row lengths come from the CSR row
// pointer; the loop runs to the slice's slot count with every slot past a
// lane's own length masked off.  U slots are loaded before any is used.
// Slot layout: complex values, and columns stored as int32 / int64.
// Offset codes (I = uint8_t): code k stands for table[k], one of at most
// kSellCodes int32 offsets c - r, staged in LDS per workgroup.
constexpr int kSellCodes = 256;

template <class V, class I, class P, int U, bool DELTA>
__global__ __launch_bounds__(256) void spmv_sell_kernel(const V* __restrict__ sell_vals,
                                                        const I* __restrict__ sell_cols,
                                                        const int* __restrict__ table,
                                                        const int64_t* __restrict__ slice_ptr,
                                                        const P* __restrict__ rowptr, const V* __restrict__ x,
                                                        V* __restrict__ y, int64_t n_rows, int64_t n_slices) {
  using T = VT<V>;
  using A = typename T::acc;
  constexpr bool kCodes = std::is_same<I, uint8_t>::value;
  __shared__ int s_tab[kCodes ? kSellCodes : 1];
  if constexpr (kCodes) {
    s_tab[threadIdx.x] = table[threadIdx.x];  // blockDim.x == kSellCodes
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int64_t slice = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (slice >= n_slices) return;  // whole wave
  const int64_t r = slice * kSellRows + lane;
  const int len = r < n_rows ? (int)((int64_t)rowptr[r + 1] - (int64_t)rowptr[r]) : 0;
  const int64_t base = slice_ptr[slice];
  const int slots = (int)((slice_ptr[slice + 1] - base) / kSellRows);
  const V* pv = sell_vals + base + lane;
  const I* pc = sell_cols + base + lane;
  A acc = T::zero();
  for (int j = 0; j < slots; j += U) {
    V v[U];
    I c[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      c[u] = 0;
      if (j + u < len) {
        v[u] = load_stream(pv + (int64_t)(j + u) * kSellRows);
        c[u] = __builtin_nontemporal_load(pc + (int64_t)(j + u) * kSellRows);
      }
    }
    V xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j + u < len) {
        if constexpr (kCodes)
          xv[u] = x[r + s_tab[c[u]]];
        else
          xv[u] = DELTA ? x[r + (int64_t)c[u]] : x[c[u]];
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j + u < len) acc = T::fma(v[u], xv[u], acc);
  }
  if (r < n_rows) store_stream(y + r, T::out(acc));
}

// Pair layout (real values): each lane loads G = 2 consecutive slots of its
// row with one 2-element vector load of values and one of columns, which
// halves the load instructions and doubles the bytes per request (27-point
// stencil with int16 offsets, f64: 0.1140 -> 0.1075 ms; f32: 0.0858 ->
// 0.0756 ms).  Groups of 4 measured no better for f32 (0.0750 ms) and worse
// for f64 (0.132 ms).  UP groups are loaded before any is used.  The tail
// of a row's last group may be padding: it is loaded with its group but
// never gathered or multiplied.
// With I = uint8_t the columns are codes into `table`, as in the slot
// kernel: one byte per entry instead of two is 9% less traffic (27-point
// 128^3 f64: 0.1077 -> 0.0930 ms).
template <class V, class I, class P, int G, int UP, bool DELTA>
__global__ __launch_bounds__(256) void spmv_sell_group_kernel(const V* __restrict__ sell_vals,
                                                              const I* __restrict__ sell_cols,
                                                              const int* __restrict__ table,
                                                              const int64_t* __restrict__ slice_ptr,
                                                              const P* __restrict__ rowptr, const V* __restrict__ x,
                                                              V* __restrict__ y, int64_t n_rows, int64_t n_slices) {
  static_assert(!VT<V>::complex, "grouped layouts are for real values");
  using T = VT<V>;
  using A = typename T::acc;
  typedef V VG __attribute__((ext_vector_type(G)));
  typedef I IG __attribute__((ext_vector_type(G)));
  constexpr bool kCodes = std::is_same<I, uint8_t>::value;
  __shared__ int s_tab[kCodes ? kSellCodes : 1];
  if constexpr (kCodes) {
    s_tab[threadIdx.x] = table[threadIdx.x];  // blockDim.x == kSellCodes
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int64_t slice = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (slice >= n_slices) return;  // whole wave
  const int64_t r = slice * kSellRows + lane;
  const int len = r < n_rows ? (int)((int64_t)rowptr[r + 1] - (int64_t)rowptr[r]) : 0;
  const int64_t base = slice_ptr[slice];  // a multiple of 64 * G entries: groups are aligned
  const int groups = (int)((slice_ptr[slice + 1] - base) / (G * kSellRows));
  const VG* pv = reinterpret_cast<const VG*>(sell_vals + base) + lane;
  const IG* pc = reinterpret_cast<const IG*>(sell_cols + base) + lane;
  A acc = T::zero();
  for (int j = 0; j < groups; j += UP) {
    VG v[UP];
    IG c[UP];
#pragma unroll
    for (int u = 0; u < UP; ++u) {
      c[u] = IG(0);
      if (G * (j + u) < len) {
        v[u] = __builtin_nontemporal_load(pv + (int64_t)(j + u) * kSellRows);
        c[u] = __builtin_nontemporal_load(pc + (int64_t)(j + u) * kSellRows);
      }
    }
    V xs[UP][G];
#pragma unroll
    for (int u = 0; u < UP; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (G * (j + u) + g < len) {
          if constexpr (kCodes)
            xs[u][g] = x[r + s_tab[c[u][g]]];
          else
            xs[u][g] = DELTA ? x[r + (int64_t)c[u][g]] : x[c[u][g]];
        }
#pragma unroll
    for (int u = 0; u < UP; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (G * (j + u) + g < len) acc = T::fma(v[u][g], xs[u][g], acc);
  }
  if (r < n_rows) store_stream(y + r, T::out(acc));
}

template <class P>
int sell_slots_p(const void* indptr, int64_t n_rows, int64_t* slots, hipStream_t s) {
  const int64_t n_slices = ceil_div(n_rows, kSellRows);
  hipLaunchKernelGGL((sell_slots_kernel<P>), dim3((unsigned)ceil_div(n_slices, 4)), dim3(256), 0, s,
                     static_cast<const P*>(indptr), n_rows, n_slices, slots);
  FS_CHECK_LAUNCH("sell_slots_kernel");
  return FS_OK;
}

template <class V, class I, class P, int GROUP>
void sell_fill_launch(int sidx_t, int64_t n_rows, const void* vals, const void* cols, const void* indptr,
                      const int64_t* slice_ptr, const uint8_t* lut, void* sv, void* sc, hipStream_t s) {
  const dim3 g((unsigned)ceil_div(ceil_div(n_rows, kSellRows), 4));
  if (sidx_t == FS_SELL_C8)
    hipLaunchKernelGGL((sell_fill_kernel<V, I, P, uint8_t, true, GROUP>), g, dim3(256), 0, s,
                       static_cast<const V*>(vals), static_cast<const I*>(cols), static_cast<const P*>(indptr),
                       n_rows, slice_ptr, lut, static_cast<V*>(sv), static_cast<uint8_t*>(sc));
  else if (sidx_t == FS_SELL_D16)
    hipLaunchKernelGGL((sell_fill_kernel<V, I, P, int16_t, true, GROUP>), g, dim3(256), 0, s,
                       static_cast<const V*>(vals), static_cast<const I*>(cols), static_cast<const P*>(indptr),
                       n_rows, slice_ptr, lut, static_cast<V*>(sv), static_cast<int16_t*>(sc));
  else if (sidx_t == FS_SELL_I32)
    hipLaunchKernelGGL((sell_fill_kernel<V, I, P, int32_t, false, GROUP>), g, dim3(256), 0, s,
                       static_cast<const V*>(vals), static_cast<const I*>(cols), static_cast<const P*>(indptr),
                       n_rows, slice_ptr, lut, static_cast<V*>(sv), static_cast<int32_t*>(sc));
  else
    hipLaunchKernelGGL((sell_fill_kernel<V, I, P, int64_t, false, GROUP>), g, dim3(256), 0, s,
                       static_cast<const V*>(vals), static_cast<const I*>(cols), static_cast<const P*>(indptr),
                       n_rows, slice_ptr, lut, static_cast<V*>(sv), static_cast<int64_t*>(sc));
}

template <class V, class I, class P>
int sell_fill_t(int sidx_t, int layout, int64_t n_rows, const void* vals, const void* cols, const void* indptr,
                const int64_t* slice_ptr, const uint8_t* lut, void* sv, void* sc, hipStream_t s) {
  if (layout == FS_SELL_PAIR)  // slots side by side in pairs
    sell_fill_launch<V, I, P, 2>(sidx_t, n_rows, vals, cols, indptr, slice_ptr, lut, sv, sc, s);
  else
    sell_fill_launch<V, I, P, 1>(sidx_t, n_rows, vals, cols, indptr, slice_ptr, lut, sv, sc, s);
  FS_CHECK_LAUNCH("sell_fill_kernel");
  return FS_OK;
}

inline int env_int(const char* name, int dflt) {
  if (const char* e = std::getenv(name)) return std::atoi(e);
  return dflt;
}

template <class V, class I, class P, bool DELTA>
int spmv_sell_t(int layout, int64_t n_rows, const void* sv, const void* sc, const int* table,
                const int64_t* slice_ptr, const void* indptr, const void* x, void* y, hipStream_t s) {
  const int64_t n_slices = ceil_div(n_rows, kSellRows);
  const dim3 grid((unsigned)ceil_div(n_slices, 4));
  if constexpr (!VT<V>::complex) {
    if (layout == FS_SELL_PAIR) {
      // pairs in flight: 8 for 4-byte values (f32 stencil with int16 offsets: 0.0852 /
      // 0.0804 / 0.0756 ms with 2 / 4 / 8; with codes 0.0697 / 0.0675 / 0.0633); for 8-byte
      // values 4 with int16 offsets (f64: 0.1084 / 0.1074 / 0.1178) and 2 with codes
      // (0.0898 / 0.0921 / 0.1036; 1 pair: 0.1096).  16 pairs of f32 with codes: 0.0842.
      constexpr bool kCodes = std::is_same<I, uint8_t>::value;
      const int up = env_int("FLAGSPARSE_SELL_UP", sizeof(V) <= 4 ? 8 : (kCodes ? 2 : 4));
      auto go = [&](auto gc, auto uc) {
        hipLaunchKernelGGL((spmv_sell_group_kernel<V, I, P, decltype(gc)::value, decltype(uc)::value, DELTA>), grid,
                           dim3(256), 0, s, static_cast<const V*>(sv), static_cast<const I*>(sc), table,
                           slice_ptr, static_cast<const P*>(indptr), static_cast<const V*>(x),
                           static_cast<V*>(y), n_rows, n_slices);
      };
      auto by_up = [&](auto gc) {
        if (up <= 1) go(gc, std::integral_constant<int, 1>{});
        else if (up <= 2) go(gc, std::integral_constant<int, 2>{});
        else if (up <= 4) go(gc, std::integral_constant<int, 4>{});
        else go(gc, std::integral_constant<int, 8>{});
      };
      by_up(std::integral_constant<int, 2>{});
      FS_CHECK_MAIN_LAUNCH("spmv_sell_group_kernel");
      return FS_OK;
    }
  }
  if (layout != FS_SELL_SLOT) return fail(FS_E_INVALID, "fs_spmv_sell: the pair layout is for real values");
  // Slots in flight: 16 for 4-byte values, 4 for wider ones.
  const int u = env_int("FLAGSPARSE_SELL_U", sizeof(V) <= 4 ? 16 : 4);
  auto go = [&](auto uc) {
    hipLaunchKernelGGL((spmv_sell_kernel<V, I, P, decltype(uc)::value, DELTA>), grid, dim3(256), 0, s,
                       static_cast<const V*>(sv), static_cast<const I*>(sc), table, slice_ptr,
                       static_cast<const P*>(indptr), static_cast<const V*>(x), static_cast<V*>(y), n_rows,
                       n_slices);
  };
  if (u <= 4) go(std::integral_constant<int, 4>{});
  else if (u <= 8) go(std::integral_constant<int, 8>{});
  else go(std::integral_constant<int, 16>{});
  FS_CHECK_MAIN_LAUNCH("spmv_sell_kernel");
  return FS_OK;
}

// Type dispatch: F is a functor template taking <V, I, P>.
template <template <class, class, class> class F, class... Args>
int dispatch_vip(int val_t, int idx_t, int ptr_t, Args... args) {
  auto by_ptr = [&](auto vtag, auto itag) -> int {
    using V = typename decltype(vtag)::type;
    using I = typename decltype(itag)::type;
    if (ptr_t == FS_I32) return F<V, I, int32_t>()(args...);
    return F<V, I, int64_t>()(args...);
  };
  auto by_idx = [&](auto vtag) -> int {
    if (idx_t == FS_SELL_C8) return by_ptr(vtag, type_tag<uint8_t>{});
    if (idx_t == FS_SELL_D16) return by_ptr(vtag, type_tag<int16_t>{});
    if (idx_t == FS_I32) return by_ptr(vtag, type_tag<int32_t>{});
    return by_ptr(vtag, type_tag<int64_t>{});
  };
  switch (val_t) {
    case FS_F32: return by_idx(type_tag<float>{});
    case FS_F64: return by_idx(type_tag<double>{});
    case FS_C64: return by_idx(type_tag<c32>{});
    default: return by_idx(type_tag<c64>{});
  }
}

template <class V, class I, class P>
struct FillF {
  int operator()(int sidx_t, int layout, int64_t n_rows, const void* vals, const void* cols, const void* indptr,
                 const int64_t* slice_ptr, const uint8_t* lut, void* sv, void* sc, hipStream_t s) const {
    return sell_fill_t<V, I, P>(sidx_t, layout, n_rows, vals, cols, indptr, slice_ptr, lut, sv, sc, s);
  }
};

template <class V, class I, class P>
struct SpmvF {
  int operator()(int layout, int64_t n_rows, const void* sv, const void* sc, const int* table,
                 const int64_t* slice_ptr, const void* indptr, const void* x, void* y, hipStream_t s) const {
    return spmv_sell_t<V, I, P, std::is_same<I, int16_t>::value>(layout, n_rows, sv, sc, table, slice_ptr, indptr,
                                                                  x, y, s);
  }
};

// ---------------------------------------------------------------------------
// SELL-64 SpMM: C = A B for a prepared matrix with a SELL-64 copy (banded and
// stencil matrices) and a row-major B / C.  Replaces, for these matrices,
// the reference's per-row SpMM kernels (spmm_csr.py:134-237) on the
// prepared route (spmm_csr.py:2040-2174).
//
// One wave per (slice, column tile): LPR lanes cover a B-row slice of
// LPR x 16 bytes (one 16-byte load each), so one load instruction gathers
// 64 / LPR consecutive rows' B rows, and for a stencil's slot j those are
// B rows r + o_j .. r + o_j + 64 / LPR - 1: one contiguous run of
// 64 x 16 bytes, as coalesced as a dense row block.  A lane accumulates
// LPR rows (rows sub, sub + 64 / LPR, ...) of its column slice, each in CSR
// entry order and in the accumulator type, as the lane-group kernel sums a
// row that stays inside one of its sub-tiles.  Slots past a row's length are never
// loaded or multiplied.  U slots' gathers are issued before any is used.
// ---------------------------------------------------------------------------
// Lane `src`'s value of any 4-byte-multiple type, by ds_bpermute.
template <class X>
__device__ inline X bcast_lane_any(const X& v, int src) {
  constexpr int W = (int)(sizeof(X) / 4);
  int w[W];
  __builtin_memcpy(w, &v, sizeof(X));
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = __builtin_amdgcn_ds_bpermute(src << 2, w[k]);
  X out;
  __builtin_memcpy(&out, w, sizeof(X));
  return out;
}

template <class V, class SI, class P, int LPR, int G, bool DELTA, int U>
__global__ __launch_bounds__(256) void spmm_sell_kernel(const V* __restrict__ sell_vals,
                                                        const SI* __restrict__ sell_cols,
                                                        const int* __restrict__ table,
                                                        const int64_t* __restrict__ slice_ptr,
                                                        const P* __restrict__ rowptr, const V* __restrict__ B,
                                                        int64_t ldb, V* __restrict__ C, int64_t ldc,
                                                        int64_t n_dense, int64_t n_rows, int64_t n_slices,
                                                        int col_tiles, int64_t n_blocks, int remap) {
  using T = VT<V>;
  using A = typename T::acc;
  using L4 = __attribute__((ext_vector_type(4))) unsigned int;
  constexpr int EPL = (int)(16 / sizeof(V));
  constexpr int RW = 64 / LPR;  // rows per load instruction
  constexpr bool kCodes = std::is_same<SI, uint8_t>::value;
  __shared__ int s_tab[kCodes ? kSellCodes : 1];
  if constexpr (kCodes) {
    s_tab[threadIdx.x] = table[threadIdx.x];  // blockDim.x == kSellCodes
    __syncthreads();
  }
  int64_t blk = blockIdx.x;
  if (remap) {  // XCD k walks a contiguous range of slices (their B rows overlap)
    const int64_t per = (n_blocks + 7) / 8;
    blk = (int64_t)(blockIdx.x % 8) * per + blockIdx.x / 8;
    if (blk >= n_blocks) return;  // whole workgroup
  }
  const int lane = threadIdx.x & 63;
  const int64_t wid = blk * 4 + (threadIdx.x >> 6);
  const int64_t slice = wid / col_tiles;
  const int ctile = (int)(wid - slice * col_tiles);
  if (slice >= n_slices) return;  // whole wave
  const int sub = lane / LPR;
  const int gl = lane % LPR;
  const int64_t col = (int64_t)ctile * (LPR * EPL) + (int64_t)gl * EPL;
  const bool cvalid = col < n_dense;
  const int64_t col_ld = cvalid ? col : 0;
  const int64_t row0 = slice * kSellRows;
  // Row lengths by unconditional loads (row indices clamped to n_rows, so a
  // row past the matrix reads rowptr[n_rows] twice and gets length 0): all
  // of them in flight at once, where loads under a row test had been waited
  // for one by one.
  auto row_len = [&](int64_t r) -> int {
    const int64_t ra = r < n_rows ? r : n_rows, rb = r + 1 < n_rows ? r + 1 : n_rows;
    return (int)((int64_t)rowptr[rb] - (int64_t)rowptr[ra]);
  };
  int len[LPR];
#pragma unroll
  for (int k = 0; k < LPR; ++k) len[k] = row_len(row0 + sub + RW * k);
  const int64_t base = slice_ptr[slice];
  const int slots = (int)((slice_ptr[slice + 1] - base) / kSellRows);
  // lane = row for the slot's value and column (one coalesced load each);
  // the lanes that gather a row's B slice take them by ds_bpermute
  const int64_t my_r = row0 + lane;
  const int my_len = row_len(my_r);
  A acc[LPR][EPL];
#pragma unroll
  for (int k = 0; k < LPR; ++k)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[k][e] = T::zero();
  const char* Bc = reinterpret_cast<const char*>(B + col_ld);
  const int64_t row_bytes = ldb * (int64_t)sizeof(V);
  for (int j0 = 0; j0 < slots; j0 += U) {
    V a[U][LPR];
    L4 q[U][LPR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u;
      V my_a = V{};
      int64_t my_b = 0;  // B row of this lane's row at slot j
      if (j < my_len) {
        const int64_t idx = base + (int64_t)(j / G) * (G * kSellRows) + G * lane + (j % G);
        my_a = load_stream(sell_vals + idx);
        const SI c = __builtin_nontemporal_load(sell_cols + idx);
        if constexpr (kCodes)
          my_b = my_r + s_tab[c];
        else
          my_b = DELTA ? my_r + (int64_t)c : (int64_t)c;
      }
#pragma unroll
      for (int k = 0; k < LPR; ++k) {
        const int src = sub + RW * k;
        a[u][k] = bcast_lane_any(my_a, src);
        const int64_t brow = bcast_lane_any(my_b, src);
        if (j < len[k]) q[u][k] = *reinterpret_cast<const L4*>(Bc + brow * row_bytes);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int k = 0; k < LPR; ++k) {
        if (j0 + u < len[k]) {
          V b[EPL];
          __builtin_memcpy(b, &q[u][k], 16);
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[k][e] = T::fma(a[u][k], b[e], acc[k][e]);
        }
      }
    }
  }
  if (!cvalid) return;
#pragma unroll
  for (int k = 0; k < LPR; ++k) {
    const int64_t r = row0 + sub + RW * k;
    if (r < n_rows) {
      V o[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = T::out(acc[k][e]);
      L4 w;
      __builtin_memcpy(&w, o, 16);
      *reinterpret_cast<L4*>(C + r * ldc + col) = w;
    }
  }
}

template <class V, class I, class P, bool DELTA>
int spmm_sell_t(int layout, int64_t n_rows, const void* sv, const void* sc, const int* table,
                const int64_t* slice_ptr, const void* indptr, const void* B, int64_t ldb, void* C, int64_t ldc,
                int64_t n_dense, hipStream_t s) {
  constexpr int EPL = (int)(16 / sizeof(V));
  if (n_dense % EPL || ldb % EPL || ldc % EPL || ((uintptr_t)B % 16) || ((uintptr_t)C % 16))
    return fail(FS_E_INVALID, "fs_spmm_sell: B / C rows must be whole 16-byte slices (n_dense, ldb, ldc multiples of " +
                                  std::to_string(EPL) + ", 16-byte aligned)");
  if (layout == FS_SELL_PAIR && VT<V>::complex) return fail(FS_E_INVALID, "fs_spmm_sell: the pair layout is for real values");
  const int64_t n_slices = ceil_div(n_rows, kSellRows);
  const int64_t slices_lanes = n_dense / EPL;  // 16-byte slices per B row
  // lanes per row: 8 (a 128-byte tile of the row per lane group; wider B runs
  // several column tiles), fewer for narrower B
  int lpr = env_int("FLAGSPARSE_SPMM_SELL_LPR", 8);
  if (lpr != 1 && lpr != 2 && lpr != 4) lpr = 8;
  while (lpr > 1 && lpr / 2 >= slices_lanes) lpr /= 2;
  const int u = env_int("FLAGSPARSE_SPMM_SELL_U", 1);  // 27-point 128^3 f32 N = 32: 0.588 / 0.650 / 1.028 ms at 1 / 2 / 4
  const int col_tiles = (int)ceil_div(slices_lanes, lpr);
  const int64_t waves = n_slices * col_tiles;
  const int64_t blocks = ceil_div(waves, 4);
  int remap = env_int("FLAGSPARSE_SPMM_SELL_REMAP", 1);
  const int64_t grid = remap ? ceil_div(blocks, 8) * 8 : blocks;
  if (grid > 0x7fffffffLL) return fail(FS_E_INVALID, "fs_spmm_sell: grid too large");
  auto go = [&](auto lc, auto gc) {
    auto launch = [&](auto uc) {
      hipLaunchKernelGGL((spmm_sell_kernel<V, I, P, decltype(lc)::value, decltype(gc)::value, DELTA,
                                           decltype(uc)::value>),
                         dim3((unsigned)grid), dim3(256), 0, s, static_cast<const V*>(sv), static_cast<const I*>(sc),
                         table, slice_ptr, static_cast<const P*>(indptr), static_cast<const V*>(B), ldb,
                         static_cast<V*>(C), ldc, n_dense, n_rows, n_slices, col_tiles, blocks, remap);
    };
    if (u <= 1) launch(std::integral_constant<int, 1>{});
    else if (u >= 4) launch(std::integral_constant<int, 4>{});
    else launch(std::integral_constant<int, 2>{});
  };
  auto by_g = [&](auto lc) {
    if (layout == FS_SELL_PAIR) go(lc, std::integral_constant<int, 2>{});
    else go(lc, std::integral_constant<int, 1>{});
  };
  switch (lpr) {
    case 1: by_g(std::integral_constant<int, 1>{}); break;
    case 2: by_g(std::integral_constant<int, 2>{}); break;
    case 4: by_g(std::integral_constant<int, 4>{}); break;
    default: by_g(std::integral_constant<int, 8>{}); break;
  }
  FS_CHECK_MAIN_LAUNCH("spmm_sell_kernel");
  return FS_OK;
}

// ---------------------------------------------------------------------------
// SpMM on the SELL-64 copy with offset codes, B staged through LDS.
// A slice's 64 rows read B rows row + offset[code]: for every code a window
// of 64 consecutive B rows, and codes whose windows overlap or touch (a
// stencil's x-neighbours: offsets -1, 0, +1) share one band.  A workgroup
// per (slice, column tile) first copies its bands' B-row tiles into LDS with
// coalesced 16-byte loads (each B row of a band once), then every row walks
// its slots and reads its B slices from LDS: the B rows a 27-point stencil
// slice needs are 9 bands of 66 rows, read once instead of once per use.
// Slots are summed in the same order as spmm_sell_kernel (bit-identical).
// ---------------------------------------------------------------------------
constexpr int kSellMaxBands = 32;
struct SellBands {
  int n;                      // bands
  int lo[kSellMaxBands];      // smallest offset of the band's codes
  int hi[kSellMaxBands];      // largest offset
  int lds[kSellMaxBands];     // first LDS row of the band (hi - lo + 64 rows each)
  int rows;                   // LDS rows of all bands
};
constexpr int kSellStageSlots = 32;  // slots of values and codes staged at a time
constexpr int kSellStageU = 8;       // slots read from LDS together
constexpr int kSellStageBatch = 8;   // B loads in flight per thread while staging

template <class V, class P, int TL, int G>
__global__ __launch_bounds__(256) void spmm_sell_staged_kernel(
    const V* __restrict__ sell_vals, const uint8_t* __restrict__ codes, const int* __restrict__ table,
    const int64_t* __restrict__ slice_ptr, const P* __restrict__ rowptr, const V* __restrict__ B, int64_t ldb,
    int64_t n_b_rows, V* __restrict__ C, int64_t ldc, int64_t n_dense, int64_t n_rows, int col_tiles,
    SellBands bands) {
  using T = VT<V>;
  using A = typename T::acc;
  using L4 = __attribute__((ext_vector_type(4))) unsigned int;
  constexpr int EPL = (int)(16 / sizeof(V));
  constexpr int RW = 64 / TL;  // rows per wave instruction
  constexpr int KR = 16 / RW;  // a wave's 16 rows take KR instruction rows
  static_assert(TL == 4 || TL == 8, "4 or 8 lanes per row tile (a wave's 16 rows in whole instructions)");
  extern __shared__ L4 s_b[];  // the bands' B tiles, then a chunk of the slice's values and codes
  __shared__ int s_base[kSellCodes];
  const int t = threadIdx.x;
  // consecutive slices on one XCD: neighbouring slices' bands overlap in its L2
  const int64_t blk = xcd_range_block(blockIdx.x, gridDim.x);
  const int64_t slice = blk / col_tiles;
  const int ctile = (int)(blk - slice * col_tiles);
  const int64_t row0 = slice * kSellRows;
  const int64_t col0 = (int64_t)ctile * TL * EPL;
  {  // LDS row of code t's window for local row 0 (-1: the code is not in use)
    const int off = table[t];
    int base = -1;
    for (int b = 0; b < bands.n; ++b)
      if (off >= bands.lo[b] && off <= bands.hi[b]) base = bands.lds[b] + (off - bands.lo[b]);
    s_base[t] = base;
  }
  __syncthreads();
  // the bands' B tiles: LDS rows are the bands' rows back to back; each
  // thread issues kSellStageBatch loads before it stores any (one latency
  // per batch, not per band)
  {
    const int total = bands.rows * TL;
    for (int i0 = t; i0 < total; i0 += 256 * kSellStageBatch) {
      L4 v[kSellStageBatch];
      int at[kSellStageBatch];
#pragma unroll
      for (int u = 0; u < kSellStageBatch; ++u) {
        const int i = i0 + u * 256;
        at[u] = -1;
        v[u] = L4{0u, 0u, 0u, 0u};
        if (i < total) {
          const int q = i / TL, pc = i - q * TL;
          int b = 0;
          while (b + 1 < bands.n && bands.lds[b + 1] <= q) ++b;
          const int64_t g = row0 + bands.lo[b] + (q - bands.lds[b]);
          const int64_t c = col0 + (int64_t)pc * EPL;
          at[u] = i;
          if (g >= 0 && g < n_b_rows && c < n_dense) v[u] = *reinterpret_cast<const L4*>(B + g * ldb + c);
        }
      }
#pragma unroll
      for (int u = 0; u < kSellStageBatch; ++u)
        if (at[u] >= 0) s_b[at[u]] = v[u];
    }
  }
  V* s_v = reinterpret_cast<V*>(s_b + (size_t)bands.rows * TL);
  int16_t* s_o = reinterpret_cast<int16_t*>(s_v + kSellStageSlots * kSellRows);  // LDS row of the entry's window
  const int lane = t & 63;
  const int sub = lane / TL, gl = lane - sub * TL;
  const int64_t base = slice_ptr[slice];
  const int slots = (int)((slice_ptr[slice + 1] - base) / kSellRows);
  int lr[KR], len[KR];
#pragma unroll
  for (int k = 0; k < KR; ++k) {
    lr[k] = (t >> 6) * 16 + sub + RW * k;
    const int64_t r = row0 + lr[k];
    len[k] = r < n_rows ? (int)((int64_t)rowptr[r + 1] - (int64_t)rowptr[r]) : 0;
  }
  A acc[KR][EPL];
#pragma unroll
  for (int k = 0; k < KR; ++k)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[k][e] = T::zero();
  // the slice's values and codes pass through LDS kSellStageSlots slots at a
  // time (their storage is contiguous per slot range: chunks start on pair
  // boundaries)
  for (int j0 = 0; j0 < slots; j0 += kSellStageSlots) {
    const int nj = slots - j0 < kSellStageSlots ? slots - j0 : kSellStageSlots;
    const int64_t cbase = base + (int64_t)j0 * kSellRows;
    for (int i = t; i < nj * kSellRows; i += 256) {
      s_v[i] = load_stream(sell_vals + cbase + i);
      s_o[i] = (int16_t)s_base[__builtin_nontemporal_load(codes + cbase + i)];
    }
    __syncthreads();  // (the first time also the bands)
    // kSellStageU slots at a time: their LDS loads are independent
    for (int jj0 = 0; jj0 < nj; jj0 += kSellStageU) {
#pragma unroll
      for (int k = 0; k < KR; ++k) {
        V a[kSellStageU];
        int o[kSellStageU];
#pragma unroll
        for (int u = 0; u < kSellStageU; ++u) {
          const int jj = jj0 + u < nj ? jj0 + u : nj - 1;
          const int li = (jj / G) * (G * kSellRows) + G * lr[k] + (jj % G);
          a[u] = s_v[li];
          o[u] = s_o[li] < 0 ? 0 : s_o[li];  // (an unused code: a read inside the bands, discarded)
        }
        L4 q[kSellStageU];
#pragma unroll
        for (int u = 0; u < kSellStageU; ++u) q[u] = s_b[(o[u] + lr[k]) * TL + gl];
#pragma unroll
        for (int u = 0; u < kSellStageU; ++u) {
          if (jj0 + u < nj && j0 + jj0 + u < len[k]) {
            V bv[EPL];
            __builtin_memcpy(bv, &q[u], 16);
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[k][e] = T::fma(a[u], bv[e], acc[k][e]);
          }
        }
      }
    }
    __syncthreads();
  }
  const int64_t col = col0 + (int64_t)gl * EPL;
  if (col >= n_dense) return;
#pragma unroll
  for (int k = 0; k < KR; ++k) {
    const int64_t r = row0 + lr[k];
    if (r < n_rows) {
      V o[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = T::out(acc[k][e]);
      L4 w;
      __builtin_memcpy(&w, o, 16);
      *reinterpret_cast<L4*>(C + r * ldc + col) = w;
    }
  }
}

// Bands from the codes' offsets (host): sorted, merged while windows of 64
// rows overlap or touch.  Returns the LDS rows they take, or -1 when there
// are more than kSellMaxBands.
inline int sell_bands(const int* offsets, int n_codes, SellBands& bands) {
  std::vector<int> o(offsets, offsets + n_codes);
  std::sort(o.begin(), o.end());
  o.erase(std::unique(o.begin(), o.end()), o.end());
  bands.n = 0;
  int rows = 0;
  for (size_t i = 0; i < o.size();) {
    int lo = o[i], hi = o[i];
    ++i;
    while (i < o.size() && (int64_t)o[i] <= (int64_t)hi + kSellRows) hi = o[i++];
    if (bands.n == kSellMaxBands) return -1;
    bands.lo[bands.n] = lo;
    bands.hi[bands.n] = hi;
    bands.lds[bands.n] = rows;
    rows += hi - lo + kSellRows;
    ++bands.n;
  }
  bands.rows = rows;
  return rows;
}

// dynamic LDS per workgroup (at least 2 per CU); FLAGSPARSE_SPMM_SELL_STAGE_LDS_KB overrides
inline size_t sell_stage_lds_limit() {
  const int kb = env_int("FLAGSPARSE_SPMM_SELL_STAGE_LDS_KB", 64);
  return (size_t)(kb >= 16 && kb <= 80 ? kb : 64) * 1024;
}

// Dynamic LDS of the staged kernel for these offsets and B width, 0 when it
// does not apply (more than kSellMaxBands bands, or over sell_stage_lds_limit()).
inline size_t sell_staged_lds(int val_size, const int* offsets, int n_codes, int64_t n_dense, int* tl_out,
                              SellBands* bands_out) {
  SellBands bands{};
  const int rows = sell_bands(offsets, n_codes, bands);
  if (rows < 0) return 0;
  const int epl = 16 / val_size;
  const int64_t pieces = (n_dense + epl - 1) / epl;
  int tl = pieces <= 4 ? 4 : 8;
  if (const int e = env_int("FLAGSPARSE_SPMM_SELL_STAGE_TL", 0); e == 4 || e == 8) tl = e;
  const size_t chunk = (size_t)kSellStageSlots * kSellRows * ((size_t)val_size + 2);
  if (tl == 8 && (size_t)rows * tl * 16 + chunk > sell_stage_lds_limit()) tl = 4;
  const size_t lds = (size_t)rows * tl * 16 + chunk;
  if (lds > sell_stage_lds_limit()) return 0;
  if (tl_out) *tl_out = tl;
  if (bands_out) *bands_out = bands;
  return lds;
}

template <class V, class P>
int spmm_sell_staged_t(int layout, int64_t n_rows, int64_t n_b_rows, const void* sv, const uint8_t* codes,
                       const int* table, const int* offsets, int n_codes, const int64_t* slice_ptr,
                       const void* indptr, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t n_dense,
                       hipStream_t s) {
  constexpr int EPL = (int)(16 / sizeof(V));
  if (n_dense % EPL || ldb % EPL || ldc % EPL || ((uintptr_t)B % 16) || ((uintptr_t)C % 16))
    return fail(FS_E_INVALID, "fs_spmm_sell_staged: B / C rows must be whole 16-byte slices");
  if (layout == FS_SELL_PAIR && VT<V>::complex)
    return fail(FS_E_INVALID, "fs_spmm_sell_staged: the pair layout is for real values");
  SellBands bands{};
  int tl = 8;
  const size_t lds = sell_staged_lds((int)sizeof(V), offsets, n_codes, n_dense, &tl, &bands);
  if (lds == 0) return fail(FS_E_INVALID, "fs_spmm_sell_staged: the offsets' bands do not fit LDS");
  const int64_t pieces = n_dense / EPL;  // 16-byte slices per B row
  const int col_tiles = (int)ceil_div(pieces, tl);
  const int64_t n_slices = ceil_div(n_rows, kSellRows);
  const int64_t blocks = n_slices * col_tiles;
  if (blocks > 0x7fffffffLL) return fail(FS_E_INVALID, "fs_spmm_sell_staged: grid too large");
  auto go = [&](auto tc, auto gc) {
    hipLaunchKernelGGL((spmm_sell_staged_kernel<V, P, decltype(tc)::value, decltype(gc)::value>),
                       dim3((unsigned)blocks), dim3(256), lds, s, static_cast<const V*>(sv), codes, table, slice_ptr,
                       static_cast<const P*>(indptr), static_cast<const V*>(B), ldb, n_b_rows, static_cast<V*>(C),
                       ldc, n_dense, n_rows, col_tiles, bands);
  };
  auto by_g = [&](auto tc) {
    if (layout == FS_SELL_PAIR) go(tc, std::integral_constant<int, 2>{});
    else go(tc, std::integral_constant<int, 1>{});
  };
  if (tl == 4) by_g(std::integral_constant<int, 4>{});
  else by_g(std::integral_constant<int, 8>{});
  FS_CHECK_MAIN_LAUNCH("spmm_sell_staged_kernel");
  return FS_OK;
}

template <class V, class I, class P>
struct SpmmF {
  int operator()(int layout, int64_t n_rows, const void* sv, const void* sc, const int* table,
                 const int64_t* slice_ptr, const void* indptr, const void* B, int64_t ldb, void* C, int64_t ldc,
                 int64_t n_dense, hipStream_t s) const {
    return spmm_sell_t<V, I, P, std::is_same<I, int16_t>::value>(layout, n_rows, sv, sc, table, slice_ptr, indptr,
                                                                  B, ldb, C, ldc, n_dense, s);
  }
};

}  // namespace fs

using namespace fs;

extern "C" int fs_sell_slots(int ptr_t, int64_t n_rows, const void* indptr, int64_t* slots_dev, hipStream_t stream) {
  if (!(ptr_t == FS_I32 || ptr_t == FS_I64)) return fail(FS_E_INVALID, "fs_sell_slots: bad type code");
  if (n_rows < 0) return fail(FS_E_INVALID, "fs_sell_slots: negative size");
  if (n_rows == 0) return FS_OK;
  if (!indptr || !slots_dev) return fail(FS_E_INVALID, "fs_sell_slots: null pointer");
  if (ptr_t == FS_I32) return sell_slots_p<int32_t>(indptr, n_rows, slots_dev, stream);
  return sell_slots_p<int64_t>(indptr, n_rows, slots_dev, stream);
}

extern "C" int fs_sell_max_offset(int idx_t, int ptr_t, int64_t n_rows, const void* cols, const void* indptr,
                                  unsigned long long* max_dev, unsigned* offset_bits_dev, hipStream_t stream) {
  if (!valid_types(FS_F32, idx_t, ptr_t)) return fail(FS_E_INVALID, "fs_sell_max_offset: bad type code");
  if (n_rows < 0) return fail(FS_E_INVALID, "fs_sell_max_offset: negative size");
  if (n_rows == 0) return FS_OK;
  if (!cols || !indptr || !max_dev) return fail(FS_E_INVALID, "fs_sell_max_offset: null pointer");
  const dim3 g((unsigned)std::min<int64_t>(ceil_div(ceil_div(n_rows, kSellRows), 4), kSellMaxOffsetBlocks));
  auto go = [&](auto itag, auto ptag) {
    using I = typename decltype(itag)::type;
    using P = typename decltype(ptag)::type;
    if (offset_bits_dev)
      hipLaunchKernelGGL((sell_max_offset_kernel<I, P, true>), g, dim3(256), 0, stream, static_cast<const I*>(cols),
                         static_cast<const P*>(indptr), n_rows, max_dev, offset_bits_dev);
    else
      hipLaunchKernelGGL((sell_max_offset_kernel<I, P, false>), g, dim3(256), 0, stream, static_cast<const I*>(cols),
                         static_cast<const P*>(indptr), n_rows, max_dev, offset_bits_dev);
  };
  if (idx_t == FS_I32 && ptr_t == FS_I32) go(type_tag<int32_t>{}, type_tag<int32_t>{});
  else if (idx_t == FS_I32) go(type_tag<int32_t>{}, type_tag<int64_t>{});
  else if (ptr_t == FS_I32) go(type_tag<int64_t>{}, type_tag<int32_t>{});
  else go(type_tag<int64_t>{}, type_tag<int64_t>{});
  FS_CHECK_LAUNCH("sell_max_offset_kernel");
  return FS_OK;
}

extern "C" int fs_csr_to_sell(int val_t, int idx_t, int ptr_t, int sell_idx_t, int layout, int64_t n_rows,
                              const void* vals, const void* cols, const void* indptr, const int64_t* slice_ptr,
                              const void* code_lut, void* sell_vals, void* sell_cols, hipStream_t stream) {
  if (!valid_types(val_t, idx_t, ptr_t) || !(sell_idx_t == FS_SELL_I32 || sell_idx_t == FS_SELL_I64 ||
                                             sell_idx_t == FS_SELL_D16 || sell_idx_t == FS_SELL_C8))
    return fail(FS_E_INVALID, "fs_csr_to_sell: bad type code");
  if (sell_idx_t == FS_SELL_C8 && !code_lut) return fail(FS_E_INVALID, "fs_csr_to_sell: code_lut is null");
  if (!(layout == FS_SELL_SLOT || layout == FS_SELL_PAIR) ||
      (layout == FS_SELL_PAIR && (val_t == FS_C64 || val_t == FS_C128)))
    return fail(FS_E_INVALID, "fs_csr_to_sell: bad layout (the pair layout is for real values)");
  if (n_rows < 0) return fail(FS_E_INVALID, "fs_csr_to_sell: negative size");
  if (n_rows == 0) return FS_OK;
  if (!indptr || !slice_ptr) return fail(FS_E_INVALID, "fs_csr_to_sell: null pointer");
  return dispatch_vip<FillF>(val_t, idx_t, ptr_t, sell_idx_t, layout, n_rows, vals, cols, indptr, slice_ptr,
                             static_cast<const uint8_t*>(code_lut), sell_vals, sell_cols, stream);
}

extern "C" int fs_spmv_sell(int val_t, int sell_idx_t, int ptr_t, int layout, int64_t n_rows,
                            const void* sell_vals, const void* sell_cols, const int32_t* code_table,
                            const int64_t* slice_ptr, const void* indptr, const void* x, void* y,
                            hipStream_t stream) {
  if (!valid_types(val_t, (sell_idx_t == FS_SELL_D16 || sell_idx_t == FS_SELL_C8) ? FS_I32 : sell_idx_t, ptr_t))
    return fail(FS_E_INVALID, "fs_spmv_sell: bad type code");
  if (sell_idx_t == FS_SELL_C8 && !code_table) return fail(FS_E_INVALID, "fs_spmv_sell: code table is null");
  if (n_rows < 0) return fail(FS_E_INVALID, "fs_spmv_sell: negative size");
  if (n_rows == 0) return FS_OK;
  if (!indptr || !slice_ptr || !y) return fail(FS_E_INVALID, "fs_spmv_sell: null pointer");
  return dispatch_vip<SpmvF>(val_t, sell_idx_t, ptr_t, layout, n_rows, sell_vals, sell_cols, code_table, slice_ptr,
                             indptr, x, y, stream);
}

extern "C" int fs_spmm_sell(int val_t, int sell_idx_t, int ptr_t, int layout, int64_t n_rows,
                            const void* sell_vals, const void* sell_cols, const int32_t* code_table,
                            const int64_t* slice_ptr, const void* indptr, const void* B, int64_t ldb, void* C,
                            int64_t ldc, int64_t n_dense, hipStream_t stream) {
  if (!valid_types(val_t, (sell_idx_t == FS_SELL_D16 || sell_idx_t == FS_SELL_C8) ? FS_I32 : sell_idx_t, ptr_t))
    return fail(FS_E_INVALID, "fs_spmm_sell: bad type code");
  if (sell_idx_t == FS_SELL_C8 && !code_table) return fail(FS_E_INVALID, "fs_spmm_sell: code table is null");
  if (!(layout == FS_SELL_SLOT || layout == FS_SELL_PAIR)) return fail(FS_E_INVALID, "fs_spmm_sell: bad layout");
  if (n_rows < 0 || n_dense < 0) return fail(FS_E_INVALID, "fs_spmm_sell: negative size");
  if (n_rows == 0 || n_dense == 0) return FS_OK;
  if (ldc < n_dense || ldb < n_dense) return fail(FS_E_INVALID, "fs_spmm_sell: leading dimension smaller than n_dense");
  if (!indptr || !slice_ptr || !C || !B) return fail(FS_E_INVALID, "fs_spmm_sell: null pointer");
  return dispatch_vip<SpmmF>(val_t, sell_idx_t, ptr_t, layout, n_rows, sell_vals, sell_cols, code_table, slice_ptr,
                             indptr, B, ldb, C, ldc, n_dense, stream);
}

extern "C" int fs_spmm_sell_staged_fits(int val_t, const int32_t* offsets_host, int n_codes, int64_t n_dense) {
  if (val_t < FS_F32 || val_t > FS_C128 || !offsets_host || n_codes <= 0 || n_codes > kSellCodes || n_dense <= 0)
    return 0;
  const int esz[] = {4, 8, 8, 16};
  return sell_staged_lds(esz[val_t], offsets_host, n_codes, n_dense, nullptr, nullptr) > 0 ? 1 : 0;
}

extern "C" int fs_spmm_sell_staged(int val_t, int ptr_t, int layout, int64_t n_rows, int64_t n_b_rows,
                                   const void* sell_vals, const void* sell_codes, const int32_t* code_table,
                                   const int32_t* offsets_host, int n_codes, const int64_t* slice_ptr,
                                   const void* indptr, const void* B, int64_t ldb, void* C, int64_t ldc,
                                   int64_t n_dense, hipStream_t stream) {
  if (!valid_types(val_t, FS_I32, ptr_t)) return fail(FS_E_INVALID, "fs_spmm_sell_staged: bad type code");
  if (!(layout == FS_SELL_SLOT || layout == FS_SELL_PAIR)) return fail(FS_E_INVALID, "fs_spmm_sell_staged: bad layout");
  if (n_rows < 0 || n_b_rows < 0 || n_dense < 0 || n_codes < 0 || n_codes > kSellCodes)
    return fail(FS_E_INVALID, "fs_spmm_sell_staged: bad size");
  if (n_rows == 0 || n_dense == 0) return FS_OK;
  if (ldc < n_dense || ldb < n_dense) return fail(FS_E_INVALID, "fs_spmm_sell_staged: leading dimension smaller than n_dense");
  if (!sell_vals || !sell_codes || !code_table || !offsets_host || !slice_ptr || !indptr || !B || !C)
    return fail(FS_E_INVALID, "fs_spmm_sell_staged: null pointer");
  const uint8_t* codes = static_cast<const uint8_t*>(sell_codes);
  auto by_p = [&](auto vtag) {
    using V = typename decltype(vtag)::type;
    if (ptr_t == FS_I32)
      return spmm_sell_staged_t<V, int32_t>(layout, n_rows, n_b_rows, sell_vals, codes, code_table, offsets_host,
                                            n_codes, slice_ptr, indptr, B, ldb, C, ldc, n_dense, stream);
    return spmm_sell_staged_t<V, int64_t>(layout, n_rows, n_b_rows, sell_vals, codes, code_table, offsets_host,
                                          n_codes, slice_ptr, indptr, B, ldb, C, ldc, n_dense, stream);
  };
  switch (val_t) {
    case FS_F32: return by_p(type_tag<float>{});
    case FS_F64: return by_p(type_tag<double>{});
    case FS_C64: return by_p(type_tag<c32>{});
    default: return by_p(type_tag<c64>{});
  }
}
