// Utility entry points: the plain copy kernel the roofline numbers are
// calibrated against (known bytes in, known bytes out), and element-wise
// dtype conversions that expose the library's rounding for exhaustive tests.
#include "fdms_vec.h"

using namespace fdms;

FDMS_EXPORT int fdms_abi_version() { return 4; }

__global__ __launch_bounds__(256) void copy16_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                     int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// Copies nbytes (multiple of 16, 16-byte aligned pointers).
FDMS_EXPORT int fdms_copy_bytes(const void* src, void* dst, int64_t nbytes, int num_blocks, void* stream) {
  if (!src || !dst || nbytes < 0 || (nbytes & 15) || num_blocks <= 0) return (int)hipErrorInvalidValue;
  if (((uintptr_t)src | (uintptr_t)dst) & 15) return (int)hipErrorInvalidValue;
  if (nbytes == 0) return 0;
  hipLaunchKernelGGL(copy16_kernel, dim3(num_blocks), dim3(256), 0, (hipStream_t)stream, (const uint4*)src,
                     (uint4*)dst, nbytes / 16);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Thread i converts elements [4i, 4i + 4) with the vector conversion the row
// kernels use (convert_vec: the FP8 encoder four values at a time), and the
// last n % 4 elements one by one, so a test over this entry point checks the
// kernels' own rounding.
template <typename TI, typename TO>
__global__ void convert_kernel(const TI* __restrict__ src, TO* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n4 = n / 4;
  if (i < n4) {
    *reinterpret_cast<Vec<TO, 4>*>(dst + 4 * i) =
        convert_vec<TI, TO, 4>(*reinterpret_cast<const Vec<TI, 4>*>(src + 4 * i));
  } else if (i < n4 + (n & 3)) {
    const int64_t j = 4 * n4 + (i - n4);
    Copy<TI, TO>::run(dst + j, src + j);
  }
}

// Element-wise dtype conversion with the library's rounding (RNE, fp8
// saturating).  src / dst aligned to four elements.
FDMS_EXPORT int fdms_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream) {
  if (!src || !dst || n < 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  const int64_t threads = n / 4 + (n & 3);
  const int64_t grid = (threads + 255) / 256;
  if (grid > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  FDMS_DISPATCH_DTYPE(src_dtype, TI,
    FDMS_DISPATCH_DTYPE(dst_dtype, TO,
      if (reinterpret_cast<uintptr_t>(src) % (4 * sizeof(TI)) || reinterpret_cast<uintptr_t>(dst) % (4 * sizeof(TO)))
        return (int)hipErrorInvalidValue;
      hipLaunchKernelGGL((convert_kernel<TI, TO>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                         (const TI*)src, (TO*)dst, n)));
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Decode FP8 e4m3fn bytes to fp32 with the hardware conversion the attention
// kernels use (v_cvt_pk_f32_fp8, bytes 0-1 / 2-3 of each dword), so a test can
// compare it with the format's definition on all 256 codes.
__global__ void fp8_decode_hw_kernel(const uint32_t* __restrict__ in, float* __restrict__ out, int64_t words) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const uint32_t w = in[i];
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[4 * i + 0] = lo[0];
  out[4 * i + 1] = lo[1];
  out[4 * i + 2] = hi[0];
  out[4 * i + 3] = hi[1];
}

FDMS_EXPORT int fdms_fp8_decode_hw(const void* in, float* out, int64_t n, void* stream) {
  if (n < 0 || n % 4) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  if (!in || !out || ((uintptr_t)in % 4)) return (int)hipErrorInvalidValue;
  const int64_t words = n / 4;
  hipLaunchKernelGGL(fp8_decode_hw_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)in, out, words);
  FDMS_LAUNCH_CHECK();
  return 0;
}
