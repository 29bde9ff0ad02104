// Shared device helpers for the gfx950 paged-KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "lvamd_paged_kv.h"

namespace lvamd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From& v) {
  static_assert(sizeof(To) == sizeof(From), "bitcast size mismatch");
  return __builtin_bit_cast(To, v);
}

__device__ __forceinline__ uint4 zero_u4() { return make_uint4(0u, 0u, 0u, 0u); }

// 16-byte global load of a row chunk.  The pointer is cast to the global
// address space: callers select between pools and input tensors at run time,
// and a generic pointer would make LLVM emit a flat load (which also counts
// against the LDS wait counter).
template <typename T>
using gptr = __attribute__((address_space(1))) T*;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ uint4 load16(gptr<const T> p) {
  const u32x4 v = *(gptr<const u32x4>)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <typename T>
__device__ __forceinline__ uint4 load16(const T* p) {
  return load16((gptr<const T>)(p));
}
// Streaming (non-temporal, `nt`) 16-byte load, for K/V bytes that a launch
// reads once.  On MI355X a plain stream of such loads reads 2 GiB at
// 7.03-7.10 TB/s against 6.62-6.69 TB/s with ordinary loads (1024 one-wave
// workgroups, same process); the sc0/sc1 scope bits alone change nothing.
template <typename T>
__device__ __forceinline__ uint4 load16_stream(gptr<const T> p) {
  const u32x4 v = __builtin_nontemporal_load((gptr<const u32x4>)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <typename T>
__device__ __forceinline__ void store16(gptr<T> p, uint4 v) {
  *(gptr<u32x4>)(p) = u32x4{v.x, v.y, v.z, v.w};
}

// fp32 -> storage type with round-to-nearest-even (matches torch's .to()).
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }

template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }

// Split-K partial rows are stored in the pool's element type, normalised by
// the piece's own sum: a convex combination of V rows, so it stays within
// the range of V's type.  Four consecutive elements per call (8 bytes for
// 16-bit types, 16 for fp32).  Streaming (non-temporal) stores when NT: the
// prefill kernel's partials then leave the L2 during the kernel instead of in
// the write-back at its end (C5: 627 -> 595 us per step); the decode kernel's
// few partials are faster as ordinary stores.
template <bool NT, typename T, typename V>
__device__ __forceinline__ void store_partial_vec(V* p, V x) {
  if constexpr (NT) {
    __builtin_nontemporal_store(x, p);
  } else {
    *p = x;
  }
}
template <bool NT, typename T>
__device__ __forceinline__ void store_partial4(T* p, f32x4 v, float s) {
  if constexpr (sizeof(T) == 4) {
    store_partial_vec<NT, T>(reinterpret_cast<f32x4*>(p), f32x4{v[0] * s, v[1] * s, v[2] * s, v[3] * s});
  } else {
    typedef T t4 __attribute__((ext_vector_type(4)));
    store_partial_vec<NT, T>(reinterpret_cast<t4*>(p), t4{from_f32<T>(v[0] * s), from_f32<T>(v[1] * s),
                                                          from_f32<T>(v[2] * s), from_f32<T>(v[3] * s)});
  }
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// N consecutive partial elements (N = 1, 2 or 4): one load, converted to
// fp32 apart from it (partial_f32) so that a caller can issue all its loads
// before the first conversion waits.
template <typename T, int N> struct PartialVec { typedef T type __attribute__((ext_vector_type(N))); };
template <typename T> struct PartialVec<T, 1> { typedef T type; };

template <typename T, int N>
__device__ __forceinline__ float partial_f32(const typename PartialVec<T, N>::type& x, int k) {
  if constexpr (N == 1) {
    return to_f32(x);
  } else {
    return to_f32<T>(x[k]);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// Max / sum across the four 16-lane rows of a wave64 (xor 16 then xor 32),
// with permlane swaps in VALU (no LDS traffic).
__device__ __forceinline__ float row_max4(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row_sum4(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// MFMA building blocks per storage type.
template <typename T> struct Mma;

template <> struct Mma<__bf16> {
  // One 16-byte chunk = 8 elements = one 16x16x32 MFMA k-step.
  __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
  }
};
template <> struct Mma<_Float16> {
  __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
  }
};
template <> struct Mma<float> {
  // One 16-byte chunk = 4 elements = four 16x16x4 MFMA k-steps.
  __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
    return c;
  }
};

template <typename T, int D>
struct TileShape {
  static constexpr int E16 = 16 / (int)sizeof(T);             // elements per 16-byte chunk
  static constexpr int NCH = (D + 4 * E16 - 1) / (4 * E16);    // chunk steps per lane per row
  static constexpr int NT = D / 16;                            // 16-row tiles of O^T
  static constexpr int RSE = D + E16;                          // LDS row stride, +16 bytes
  static constexpr int CPR = D / E16;                          // 16-byte chunks per row
  static_assert(D % 16 == 0 && D <= 256, "head size must be a multiple of 16, at most 256");
};

inline int dtype_size(int dtype) {
  switch (dtype) {
    case LVAMD_F32: return 4;
    case LVAMD_F16: return 2;
    case LVAMD_BF16: return 2;
    default: return 0;
  }
}

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? LVAMD_OK : LVAMD_ERR_LAUNCH;
}

}  // namespace lvamd
