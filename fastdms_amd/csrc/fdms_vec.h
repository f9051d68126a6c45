// Vectorised row copy with dtype conversion, shared by the pack / append /
// expiry kernels.  VEC elements are moved per call; the host picks VEC so
// that every source and destination address is VEC*sizeof aligned.
#pragma once

#include <type_traits>

#include "fdms_common.h"

namespace fdms {

template <typename T, int N>
struct alignas(sizeof(T) * N) Vec {
  T v[N];
};

// Element-wise dtype conversion of a vector; conversions into FP8 go four
// values at a time through f32x4_to_fp8x4.
template <typename TI, typename TO, int N>
__device__ __forceinline__ Vec<TO, N> convert_vec(const Vec<TI, N>& in) {
  Vec<TO, N> out;
  if constexpr (std::is_same<TO, fp8_t>::value && !std::is_same<TI, fp8_t>::value && N % 4 == 0) {
    uint32_t* o = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
      o[i] = f32x4_to_fp8x4(ld<TI>(&in.v[4 * i]), ld<TI>(&in.v[4 * i + 1]), ld<TI>(&in.v[4 * i + 2]),
                            ld<TI>(&in.v[4 * i + 3]));
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) Copy<TI, TO>::run(&out.v[i], &in.v[i]);
  }
  return out;
}

// As convert_vec with every value multiplied by `mul` (fp32, one rounding)
// before the store conversion: x * (1 / scale) for scaled FP8 KV.  mul == 1
// gives convert_vec's results exactly; a same-dtype move ignores mul (the
// host allows scales with FP8 arenas only).
template <typename TI, typename TO, int N>
__device__ __forceinline__ Vec<TO, N> convert_vec_scaled(const Vec<TI, N>& in, float mul) {
  if constexpr (std::is_same<TI, TO>::value) return convert_vec<TI, TO, N>(in);
  Vec<TO, N> out;
  if constexpr (std::is_same<TO, fp8_t>::value && !std::is_same<TI, fp8_t>::value && N % 4 == 0) {
    uint32_t* o = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
      o[i] = f32x4_to_fp8x4(ld<TI>(&in.v[4 * i]) * mul, ld<TI>(&in.v[4 * i + 1]) * mul,
                            ld<TI>(&in.v[4 * i + 2]) * mul, ld<TI>(&in.v[4 * i + 3]) * mul);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) st<TO>(&out.v[i], ld<TI>(&in.v[i]) * mul);
  }
  return out;
}

// 1 / scale[h] in fp32 (IEEE division), 1 without a scale table.
__device__ __forceinline__ float inv_scale(const float* scale, int h) {
  return scale ? 1.0f / scale[h] : 1.0f;
}

template <typename TI, typename TO, int N>
__device__ __forceinline__ void copy_vec(TO* __restrict__ dst, const TI* __restrict__ src) {
  *reinterpret_cast<Vec<TO, N>*>(dst) = convert_vec<TI, TO, N>(*reinterpret_cast<const Vec<TI, N>*>(src));
}

// Byte-level moves for same-dtype arenas (expiry): N bytes per call.
template <int N>
__device__ __forceinline__ void move_bytes(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src) {
  *reinterpret_cast<Vec<uint8_t, N>*>(dst) = *reinterpret_cast<const Vec<uint8_t, N>*>(src);
}

}  // namespace fdms

// Dispatch a runtime vector width (elements) to a compile-time constant.
#define FDMS_DISPATCH_VEC(vec, V, ...)              \
  switch (vec) {                                    \
    case 16: { constexpr int V = 16; __VA_ARGS__; break; } \
    case 8: { constexpr int V = 8; __VA_ARGS__; break; } \
    case 4: { constexpr int V = 4; __VA_ARGS__; break; } \
    case 2: { constexpr int V = 2; __VA_ARGS__; break; } \
    case 1: { constexpr int V = 1; __VA_ARGS__; break; } \
    default: return (int)hipErrorInvalidValue;      \
  }
