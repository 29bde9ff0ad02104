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

// 16-byte global load/store of a row chunk.
template <typename T>
__device__ __forceinline__ uint4 load16(const T* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// fp32 -> storage type with round-to-nearest-even (matches torch's .to()).
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }

template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }

// Wave64 butterfly across the four 16-lane rows (xor 16, xor 32).
__device__ __forceinline__ float wave_max_across_rows(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}
__device__ __forceinline__ float wave_sum_across_rows(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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

// O^T[16n + l%16][col] += sum_t V[t][16n + l%16] * P[col][t] over a 32-token tile held
// in LDS as natural rows (stride RSE elements), with P in the S^T accumulator
// layout: p[s][r] is token 16s + 4*(l/16) + r of this lane's column.
template <typename T, int RSE>
__device__ __forceinline__ f32x4 pv_tile(const T* vt, int n, int l16, int g, const float (&p)[2][4], f32x4 acc) {
  if constexpr (sizeof(T) == 2) {
    using V8 = typename std::conditional<std::is_same<T, __bf16>::value, bf16x8, f16x8>::type;
    V8 av, b;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        av[s * 4 + r] = vt[(16 * s + 4 * g + r) * RSE + 16 * n + l16];
        b[s * 4 + r] = from_f32<T>(p[s][r]);
      }
    if constexpr (std::is_same<T, __bf16>::value) {
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b, acc, 0, 0, 0);
    } else {
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, acc, 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float av = vt[(16 * s + 4 * g + r) * RSE + 16 * n + l16];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, p[s][r], acc, 0, 0, 0);
      }
    return acc;
  }
}

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
