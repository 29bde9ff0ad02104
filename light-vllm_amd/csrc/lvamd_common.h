// Shared device helpers for the gfx950 paged-KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
