// Utility entry points: the plain copy kernel the roofline numbers are
// calibrated against (known bytes in, known bytes out), and element-wise
// dtype conversions that expose the library's rounding for exhaustive tests.
#include "fdms_vec.h"

using namespace fdms;

FDMS_EXPORT int fdms_abi_version() { return 1; }

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

template <typename TI, typename TO>
__global__ void convert_kernel(const TI* __restrict__ src, TO* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) Copy<TI, TO>::run(dst + i, src + i);
}

// Element-wise dtype conversion with the library's rounding (RNE, fp8 saturating).
FDMS_EXPORT int fdms_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream) {
  if (!src || !dst || n < 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  const int64_t grid = (n + 255) / 256;
  if (grid > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  FDMS_DISPATCH_DTYPE(src_dtype, TI,
    FDMS_DISPATCH_DTYPE(dst_dtype, TO,
      hipLaunchKernelGGL((convert_kernel<TI, TO>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                         (const TI*)src, (TO*)dst, n)));
  FDMS_LAUNCH_CHECK();
  return 0;
}
