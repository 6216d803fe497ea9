// fs_common.hpp — shared device/host helpers for the gfx950 CSR kernels.
//
// Value types and their accumulators.  The reference computes fp32 CSR
// products in fp64 and rounds once at the end (spmv_csr.py:124-130,
// spmm_csr.py:2720-2759); every kernel here does the same for fp32 and also
// accumulates complex64 in fp64 components.  fp64 / complex128 accumulate
// natively.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <stdint.h>

#include <algorithm>
#include <string>

#include "../../include/flagsparse_hip.h"

namespace fs {

constexpr int kWave = 64;  // CDNA wavefront width

struct alignas(8) c32 {
  float re, im;
};
struct alignas(16) c64 {
  double re, im;
};

// ---------------------------------------------------------------------------
// Value traits: load type V, accumulator A.
// ---------------------------------------------------------------------------
template <class V>
struct VT;

template <>
struct VT<float> {
  using acc = double;
  static constexpr bool complex = false;
  __device__ static acc zero() { return 0.0; }
  __device__ static acc mul(float a, float x) { return (double)a * (double)x; }
  __device__ static acc fma(float a, float x, acc s) {
    return __builtin_fma((double)a, (double)x, s);
  }
  __device__ static float out(acc s) { return (float)s; }
  __device__ static float conj(float v) { return v; }
};

template <>
struct VT<double> {
  using acc = double;
  static constexpr bool complex = false;
  __device__ static acc zero() { return 0.0; }
  __device__ static acc mul(double a, double x) { return a * x; }
  __device__ static acc fma(double a, double x, acc s) {
    return __builtin_fma(a, x, s);
  }
  __device__ static double out(acc s) { return s; }
  __device__ static double conj(double v) { return v; }
};

template <>
struct VT<c32> {
  using acc = c64;
  static constexpr bool complex = true;
  __device__ static acc zero() { return c64{0.0, 0.0}; }
  __device__ static acc mul(c32 a, c32 x) {
    double ar = a.re, ai = a.im, xr = x.re, xi = x.im;
    return c64{__builtin_fma(ar, xr, -ai * xi), __builtin_fma(ar, xi, ai * xr)};
  }
  __device__ static acc fma(c32 a, c32 x, acc s) {
    double ar = a.re, ai = a.im, xr = x.re, xi = x.im;
    s.re = __builtin_fma(ar, xr, s.re);
    s.re = __builtin_fma(-ai, xi, s.re);
    s.im = __builtin_fma(ar, xi, s.im);
    s.im = __builtin_fma(ai, xr, s.im);
    return s;
  }
  __device__ static c32 out(acc s) { return c32{(float)s.re, (float)s.im}; }
  __device__ static c32 conj(c32 v) { return c32{v.re, -v.im}; }
};

template <>
struct VT<c64> {
  using acc = c64;
  static constexpr bool complex = true;
  __device__ static acc zero() { return c64{0.0, 0.0}; }
  __device__ static acc mul(c64 a, c64 x) {
    return c64{__builtin_fma(a.re, x.re, -a.im * x.im),
               __builtin_fma(a.re, x.im, a.im * x.re)};
  }
  __device__ static acc fma(c64 a, c64 x, acc s) {
    s.re = __builtin_fma(a.re, x.re, s.re);
    s.re = __builtin_fma(-a.im, x.im, s.re);
    s.im = __builtin_fma(a.re, x.im, s.im);
    s.im = __builtin_fma(a.im, x.re, s.im);
    return s;
  }
  __device__ static c64 out(acc s) { return s; }
  __device__ static c64 conj(c64 v) { return c64{v.re, -v.im}; }
};

__device__ inline double add(double a, double b) { return a + b; }
__device__ inline c64 add(c64 a, c64 b) { return c64{a.re + b.re, a.im + b.im}; }
__device__ inline float add(float a, float b) { return a + b; }
__device__ inline c32 add(c32 a, c32 b) { return c32{a.re + b.re, a.im + b.im}; }

// Fix-up of a row that ends in tile t but starts before it: the tile where
// it starts is the last f < t whose first row precedes r0 (part is
// non-decreasing and part[t] == r0), or 0.  A binary search: a hub row
// spanning many tiles is found in log steps, not one dependent load per tile.
__device__ inline int64_t fixup_start_tile(const int64_t* __restrict__ part, int64_t t, int64_t r0) {
  int64_t lo = 0, hi = t - 1;
  if (part[hi] < r0) return hi;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (part[mid] < r0) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Sum of acc-typed fragments v[f..t) in order, 8 loads in flight at a time.
template <class A>
__device__ inline A sum_fragments(const A* __restrict__ v, int64_t stride, int64_t f, int64_t t, A sum) {
  int64_t k = f;
  for (; k + 8 <= t; k += 8) {
    A w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = v[(k + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) sum = add(sum, w[u]);
  }
  for (; k < t; ++k) sum = add(sum, v[k * stride]);
  return sum;
}

// Accumulation in the value type itself (float in float, complex64 in
// complex64), as the reference's opt / alg1 / alg2 SpMM kernels accumulate
// float32 data (spmm_csr.py:2792-3109, spmm_csr_opt_alg2.py:438-729); double
// and complex128 are the same as VT.
template <class V>
struct VN : VT<V> {};
template <>
struct VN<float> {
  using acc = float;
  static constexpr bool complex = false;
  __device__ static acc zero() { return 0.0f; }
  __device__ static acc fma(float a, float x, acc s) { return __builtin_fmaf(a, x, s); }
  __device__ static float out(acc s) { return s; }
};
template <>
struct VN<c32> {
  using acc = c32;
  static constexpr bool complex = true;
  __device__ static acc zero() { return c32{0.0f, 0.0f}; }
  __device__ static acc fma(c32 a, c32 x, acc s) {
    s.re = __builtin_fmaf(a.re, x.re, s.re);
    s.re = __builtin_fmaf(-a.im, x.im, s.re);
    s.im = __builtin_fmaf(a.re, x.im, s.im);
    s.im = __builtin_fmaf(a.im, x.re, s.im);
    return s;
  }
  __device__ static c32 out(acc s) { return s; }
};

// Streaming (non-temporal) load of one element.
__device__ inline float load_stream(const float* p) { return __builtin_nontemporal_load(p); }
__device__ inline double load_stream(const double* p) { return __builtin_nontemporal_load(p); }
__device__ inline c32 load_stream(const c32* p) {
  return c32{__builtin_nontemporal_load(&p->re), __builtin_nontemporal_load(&p->im)};
}
__device__ inline c64 load_stream(const c64* p) {
  return c64{__builtin_nontemporal_load(&p->re), __builtin_nontemporal_load(&p->im)};
}

// Streaming (non-temporal) store of one output element: results written
// once and not re-read by the kernel skip L2 allocation priority.
__device__ inline void store_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ inline void store_stream(double* p, double v) { __builtin_nontemporal_store(v, p); }
__device__ inline void store_stream(c32* p, c32 v) {
  __builtin_nontemporal_store(v.re, &p->re);
  __builtin_nontemporal_store(v.im, &p->im);
}
__device__ inline void store_stream(c64* p, c64 v) {
  __builtin_nontemporal_store(v.re, &p->re);
  __builtin_nontemporal_store(v.im, &p->im);
}

// ---------------------------------------------------------------------------
// Cross-lane moves.  DPP for distances inside a 16-lane row, ds_swizzle for
// the 16-lane xor inside each 32-lane half, readlane across halves.
// ---------------------------------------------------------------------------
// DPP control words (GCN3+ encoding).
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // reverse within 8 lanes
constexpr int kDppRowMirror = 0x140;     // reverse within 16 lanes
// ds_swizzle bit mode: and=0x1f, or=0, xor=0x10 -> lane ^ 16 within 32.
constexpr int kSwzXor16 = (0x10 << 10) | 0x1F;

template <int CTRL>
__device__ inline double dpp_f64(double v) {
  int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xF, 0xF, false);
  int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xF, 0xF, false);
  return __hiloint2double(hi, lo);
}

__device__ inline double swz_xor16_f64(double v) {
  int lo = __builtin_amdgcn_ds_swizzle(__double2loint(v), kSwzXor16);
  int hi = __builtin_amdgcn_ds_swizzle(__double2hiint(v), kSwzXor16);
  return __hiloint2double(hi, lo);
}

// Butterfly all-reduce over aligned groups of W lanes (W power of two, <=32).
// Each step's partner set is closed under the group, so every lane of a
// group ends with the group total.  Mirror permutations act as xor-4 /
// xor-8 because the values are already uniform within quads / octets.
template <int W>
__device__ inline double group_sum(double v) {
  if constexpr (W >= 2) v += dpp_f64<kDppQuadXor1>(v);
  if constexpr (W >= 4) v += dpp_f64<kDppQuadXor2>(v);
  if constexpr (W >= 8) v += dpp_f64<kDppRowHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_f64<kDppRowMirror>(v);
  if constexpr (W >= 32) v += swz_xor16_f64(v);
  return v;
}

template <int W>
__device__ inline c64 group_sum(c64 v) {
  return c64{group_sum<W>(v.re), group_sum<W>(v.im)};
}

__device__ inline double readlane_f64(double v, int lane) {
  int lo = __builtin_amdgcn_readlane(__double2loint(v), lane);
  int hi = __builtin_amdgcn_readlane(__double2hiint(v), lane);
  return __hiloint2double(hi, lo);
}

// Sum over the whole wave, returned uniformly (lanes 0 and 32 hold the two
// half totals after the 32-lane butterfly).
__device__ inline double wave_total(double v) {
  v = group_sum<32>(v);
  return readlane_f64(v, 0) + readlane_f64(v, 32);
}
__device__ inline c64 wave_total(c64 v) { return c64{wave_total(v.re), wave_total(v.im)}; }

// Generic shuffle (ds_bpermute) of 64-bit values, used for scans.
__device__ inline double shfl_f64(double v, int src_lane) {
  int lo = __builtin_amdgcn_ds_bpermute(src_lane << 2, __double2loint(v));
  int hi = __builtin_amdgcn_ds_bpermute(src_lane << 2, __double2hiint(v));
  return __hiloint2double(hi, lo);
}
__device__ inline c64 shfl(c64 v, int src) { return c64{shfl_f64(v.re, src), shfl_f64(v.im, src)}; }
__device__ inline double shfl(double v, int src) { return shfl_f64(v, src); }
__device__ inline int shfl(int v, int src) { return __builtin_amdgcn_ds_bpermute(src << 2, v); }

// ---------------------------------------------------------------------------
// Error reporting (thread-local message, see fs_last_error()).
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_hip(hipError_t e, const char* what);
// Records the main kernel of the calling thread's latest hot-path launch
// (see fs_last_kernel()).
void note_kernel(const char* name);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// LDS bytes per CU of the current device (cached per device id).
// (The caches below are relaxed atomics: concurrent host threads may each
// query the device once and store the same value.)
inline size_t lds_per_cu() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 163840;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess || v <= 0)
      v = 163840;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return (size_t)v;
}

// Dynamic LDS bytes that leave room for at most `wg_per_cu` workgroups per
// CU of a kernel using `static_lds` bytes of LDS per workgroup (0 when the
// cap is off or already implied).
inline size_t lds_pad_for_cap(int wg_per_cu, size_t static_lds) {
  if (wg_per_cu <= 0) return 0;
  const size_t share = lds_per_cu() / (size_t)wg_per_cu;
  return share > static_lds ? std::min<size_t>(share - static_lds, 65536 - static_lds) : 0;
}

// Structure-check words (fs_csr_check_bytes): [0] indptr[0], [1]
// indptr[n_rows], [2] rows whose pointer decreases, [3] / [4] the column
// minimum / maximum, stored with the sign bit flipped so that unsigned
// atomics order signed values.
constexpr unsigned long long kSignFlip = 1ull << 63;

// Type-code validation shared by every entry point.
bool valid_types(int val_t, int idx_t, int ptr_t);

}  // namespace fs

#define FS_CHECK_HIP(expr)                                  \
  do {                                                      \
    int _rc = ::fs::check_hip((expr), #expr);               \
    if (_rc != FS_OK) return _rc;                           \
  } while (0)

#define FS_CHECK_LAUNCH(name)                               \
  do {                                                      \
    int _rc = ::fs::check_hip(hipGetLastError(), name);     \
    if (_rc != FS_OK) return _rc;                           \
  } while (0)

// Workgroup b of a 1-D grid of n, renumbered so that each of the 8 XCDs (to
// which the hardware deals workgroups in turn) walks one contiguous range:
// a bijection on [0, n).
__device__ inline int64_t xcd_range_block(uint32_t b, uint32_t n) {
  constexpr uint32_t kX = 8;
  const uint32_t q = n / kX, r = n % kX, x = b % kX, i = b / kX;
  return x < r ? (int64_t)x * (q + 1) + i : (int64_t)r * (q + 1) + (int64_t)(x - r) * q + i;
}

// FS_CHECK_LAUNCH for the main kernel of an entry point: also records its
// name for fs_last_kernel().
#define FS_CHECK_MAIN_LAUNCH(name)                          \
  do {                                                      \
    int _rc = ::fs::check_hip(hipGetLastError(), name);     \
    if (_rc != FS_OK) return _rc;                           \
    ::fs::note_kernel(name);                                \
  } while (0)
