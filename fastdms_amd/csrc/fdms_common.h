// Shared device helpers for the fastdms_amd HIP library (gfx950, wave64).
//
// Storage dtypes are passed across the C-ABI as small integer codes so one
// entry point serves every K/V / q dtype the reference's kernels accept
// (its Triton kernels cast implicitly on load/store).  Conversions are done
// in integer arithmetic so their rounding is fixed by this file, not by a
// hardware mode: f32->bf16 and f32->fp8 round to nearest-even, fp8 saturates
// to +-448 (the behaviour of the reference's Triton store casts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdms {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2, kFP8 = 3 };

struct bf16_t { uint16_t bits; };
struct fp8_t { uint8_t bits; };
struct u4x2_t { uint8_t bits; };  // two INT4 codes: low nibble = even k, high nibble = odd k
typedef _Float16 f16_t;

constexpr int kWave = 64;

// ---------------------------------------------------------------- fp8 e4m3fn
__device__ __forceinline__ float fp8_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t em = b & 0x7Fu;
  float mag;
  if (em >= 8u) {
    mag = __uint_as_float((em << 20) + (120u << 23));
  } else {
    mag = (float)em * 0.001953125f;  // subnormal: m * 2^-9
  }
  uint32_t r = __float_as_uint(mag) | sign;
  if (em == 0x7Fu) r = 0x7FC00000u | sign;
  return __uint_as_float(r);
}

__device__ __forceinline__ uint32_t f32_to_fp8(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;   // NaN
  if (a >= 0x43E00000u) return sign | 0x7Eu;  // |x| >= 448 (and inf) saturate
  if (a >= 0x3C800000u) {                     // normal e4m3 range, |x| >= 2^-6
    uint32_t base = (((a >> 23) - 120u) << 3) | ((a >> 20) & 7u);
    const uint32_t rem = a & 0xFFFFFu;
    base += (rem > 0x80000u) || (rem == 0x80000u && (base & 1u));
    return sign | base;
  }
  const float f = __uint_as_float(a) * 512.0f;  // exact power-of-two scale
  return sign | (uint32_t)__builtin_rintf(f);  // 0..8, half-to-even
}

// f32_to_fp8 of four values packed into one dword (byte i = value i), on the
// gfx950 converter v_cvt_pk_fp8_f32.  The converter rounds to nearest even
// but turns out-of-range values into NaN, so inputs are clamped to +-448 first
// (saturation, as above); a NaN input is then re-encoded as sign | 0x7F.  Equal
// to f32_to_fp8 on every bf16 bit pattern and on random / tie / subnormal f32
// inputs (checked on the device against the scalar routine).
__device__ __forceinline__ uint32_t f32x4_to_fp8x4(float a, float b, float c, float d) {
  const float ca = __builtin_amdgcn_fmed3f(a, -448.0f, 448.0f);
  const float cb = __builtin_amdgcn_fmed3f(b, -448.0f, 448.0f);
  const float cc = __builtin_amdgcn_fmed3f(c, -448.0f, 448.0f);
  const float cd = __builtin_amdgcn_fmed3f(d, -448.0f, 448.0f);
  uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false);
  r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(cc, cd, (int)r, true);
  if (__builtin_expect((a != a) | (b != b) | (c != c) | (d != d), 0)) {
    r = f32_to_fp8(a) | (f32_to_fp8(b) << 8) | (f32_to_fp8(c) << 16) | (f32_to_fp8(d) << 24);
  }
  return r;
}

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x40u) & 0xFFFFu;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// ---------------------------------------------------------------- typed load/store
template <typename T> struct Conv;
template <> struct Conv<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <> struct Conv<f16_t> {
  static __device__ __forceinline__ float load(const f16_t* p) { return (float)*p; }
  static __device__ __forceinline__ void store(f16_t* p, float v) { *p = (f16_t)v; }
};
template <> struct Conv<bf16_t> {
  static __device__ __forceinline__ float load(const bf16_t* p) { return bf16_to_f32(p->bits); }
  static __device__ __forceinline__ void store(bf16_t* p, float v) { p->bits = (uint16_t)f32_to_bf16(v); }
};
template <> struct Conv<fp8_t> {
  static __device__ __forceinline__ float load(const fp8_t* p) { return fp8_to_f32(p->bits); }
  static __device__ __forceinline__ void store(fp8_t* p, float v) { p->bits = (uint8_t)f32_to_fp8(v); }
};

template <typename T> __device__ __forceinline__ float ld(const T* p) { return Conv<T>::load(p); }
template <typename T> __device__ __forceinline__ void st(T* p, float v) { Conv<T>::store(p, v); }

// Same-type copies keep the bits (a cast fp8->fp8 is the identity).
template <typename TI, typename TO> struct Copy {
  static __device__ __forceinline__ void run(TO* d, const TI* s) { st<TO>(d, ld<TI>(s)); }
};
template <typename T> struct Copy<T, T> {
  static __device__ __forceinline__ void run(T* d, const T* s) { *d = *s; }
};

// ---------------------------------------------------------------- wave helpers
// DPP move within 16-lane rows (CTRL e.g. 0x120 + n = row_ror:n).
template <int CTRL>
__device__ __forceinline__ float dpp_mov_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Max / sum over the four 16-lane rows (lanes l, l^16, l^32, l^48) with the
// gfx950 row-swap permutes: permlane16_swap(x, x) yields (even rows, odd rows)
// of x in every row pair and permlane32_swap(x, x) (low half, high half), so
// combining the two results reduces over xor 16 then xor 32 without an LDS
// round trip.  Every lane gets the same bits (the combines are commutative).
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Whole-wave max / sum: rotations by 8, 4, 2, 1 inside each row (DPP), then
// across rows.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov_f<0x128>(v));
  v = fmaxf(v, dpp_mov_f<0x124>(v));
  v = fmaxf(v, dpp_mov_f<0x122>(v));
  v = fmaxf(v, dpp_mov_f<0x121>(v));
  return rows_max(v);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov_f<0x128>(v);
  v += dpp_mov_f<0x124>(v);
  v += dpp_mov_f<0x122>(v);
  v += dpp_mov_f<0x121>(v);
  return rows_sum(v);
}

// Row amax with NaN propagation, in the bit domain: for a float with its sign
// cleared the unsigned order of the bits is the numeric order and every NaN
// lies above +inf, so an unsigned max of abs_bits(x) is max |x| -- NaN when
// any element is NaN, as torch's amax -- independent of the order of the
// combines.
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x122, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x121, 0xF, 0xF, true));
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((uint32_t)a[0], (uint32_t)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((uint32_t)b[0], (uint32_t)b[1]);
}

// Per-row FP8 activation scale from the row amax (linear.py:386-388, 514-523,
// 683-694): 448 / amax, 1 where amax > 0 fails (0 or NaN); torch_form rounds
// as the reference's tensor expression (reciprocal, then times 448).
__device__ __forceinline__ float fp8_row_scale(float amax, bool torch_form) {
  return amax > 0.0f ? (torch_form ? (1.0f / amax) * 448.0f : 448.0f / amax) : 1.0f;
}
// True when every x * scale of the row is finite with |x * scale| <= 448 (1 +
// 2^-22) (amax and scale finite): then the clamped hardware conversion below
// equals f32_to_fp8 on the row, and no element needs the NaN re-encode.
__device__ __forceinline__ bool fp8_row_finite(float amax, float scale) {
  return amax <= 3.40282347e38f && scale <= 3.40282347e38f;
}
// f32x4_to_fp8x4 without the NaN re-encode, for values known to be finite.
__device__ __forceinline__ uint32_t f32x4_to_fp8x4_finite(float a, float b, float c, float d) {
  const uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(a, -448.0f, 448.0f),
                                                               __builtin_amdgcn_fmed3f(b, -448.0f, 448.0f), 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(c, -448.0f, 448.0f),
                                                   __builtin_amdgcn_fmed3f(d, -448.0f, 448.0f), (int)r, true);
}
__device__ __forceinline__ uint32_t f32x4_to_fp8x4_sw(float a, float b, float c, float d) {
  return f32_to_fp8(a) | (f32_to_fp8(b) << 8) | (f32_to_fp8(c) << 16) | (f32_to_fp8(d) << 24);
}

// torch.argmax order: NaN beats every number (lowest NaN index wins), ties go
// to the lowest index.  True if (v, i) should replace the current best (bv, bi).
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// DMS threshold (dms.py:37-40): v > offset/scale (quotient pre-rounded to
// fp32 on the host) when scale > 0, else v*scale - offset > 0 with each step
// rounded to fp32.
__device__ __forceinline__ bool dms_decide(float v, float alpha_scale, float alpha_offset, float threshold,
                                           int positive_scale) {
#pragma clang fp contract(off)
  if (positive_scale) return v > threshold;
  const float prod = v * alpha_scale;
  return (prod - alpha_offset) > 0.0f;
}

// Rotate-half RoPE pair in fp32 with each product and sum rounded separately
// (rotary_embedding.py:12-14: y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin).
__device__ __forceinline__ void rope_f32(float x1, float x2, float c, float s, float* y1, float* y2) {
#pragma clang fp contract(off)
  const float a = x1 * c, b = x2 * s, cc = x2 * c, d = x1 * s;
  *y1 = a - b;
  *y2 = cc + d;
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Cross-workgroup handoff of split partials.  On gfx942 / gfx950 an
// agent-scope fence writes back and invalidates the whole L2 of the XCD
// (buffer_wbl2 sc1 / buffer_inv sc1), which costs microseconds per call; the
// split kernels instead keep the handoff coherent through the accesses
// themselves and order it with workgroup-scope fences, the protocol AMD's
// rocPRIM look-back scan uses on these chips:
//   producer: partials written with relaxed agent-scope atomic stores (sc1:
//     they bypass the non-coherent cache levels), then handoff_release()
//     (workgroup release fence + wait until every vector-memory operation of
//     the thread has completed), then the ticket, a relaxed agent-scope
//     atomic add performed at the device coherence point;
//   consumer (the workgroup that takes the last ticket): handoff_acquire()
//     (wait for the ticket + workgroup acquire fence, so no later load is
//     issued before it), then relaxed agent-scope atomic loads (sc1: served
//     from the coherence point, never a stale cache line).
// The stores have completed at the coherence point before the ticket is
// taken, and the loads are issued after the last ticket returned.
__device__ __forceinline__ void handoff_release() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));  // vmcnt(0)
}
__device__ __forceinline__ void handoff_acquire() {
  __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));  // vmcnt(0)
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}
__device__ __forceinline__ int ticket_add(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int popc64(uint64_t x) { return __popcll(x); }

// Sum over aligned segments of N lanes (N a power of two <= 64) of a wave;
// every lane of the wave must call it.
template <int N>
__device__ __forceinline__ float segment_sum(float v) {
#pragma unroll
  for (int o = N / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace fdms

#define FDMS_LAUNCH_CHECK()                         \
  do {                                              \
    hipError_t _e = hipGetLastError();              \
    if (_e != hipSuccess) return (int)_e;           \
  } while (0)

#define FDMS_EXPORT extern "C" __attribute__((visibility("default")))

// True when every non-null pointer is 16-byte aligned (host-side argument check
// for kernels that move rows as 16-byte vectors).
template <typename... P>
inline bool fdms_aligned16(const P*... p) {
  return ((((uintptr_t)p) % 16 == 0) && ...);
}

// Dispatch a runtime dtype code to a C++ storage type.
#define FDMS_DISPATCH_DTYPE(code, T, ...)                     \
  switch (code) {                                             \
    case fdms::kF32: { typedef float T; __VA_ARGS__; break; } \
    case fdms::kF16: { typedef fdms::f16_t T; __VA_ARGS__; break; } \
    case fdms::kBF16: { typedef fdms::bf16_t T; __VA_ARGS__; break; } \
    case fdms::kFP8: { typedef fdms::fp8_t T; __VA_ARGS__; break; } \
    default: return (int)hipErrorInvalidValue;                \
  }

#define FDMS_DISPATCH_FLOAT(code, T, ...)                     \
  switch (code) {                                             \
    case fdms::kF32: { typedef float T; __VA_ARGS__; break; } \
    case fdms::kF16: { typedef fdms::f16_t T; __VA_ARGS__; break; } \
    case fdms::kBF16: { typedef fdms::bf16_t T; __VA_ARGS__; break; } \
    default: return (int)hipErrorInvalidValue;                \
  }
