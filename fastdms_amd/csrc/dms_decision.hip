// DMS eviction decision extraction (reference: fastdms/engine/dms.py:12-42,
// 152-232).  One thread per (token, kv_head): read the borrowed decision
// channel q[t, h*G, D-1], threshold it, write the evict flag and zero the
// channel.  Reads and writes one element per (token, head): launch-bound.
#include "fdms_common.h"

using namespace fdms;

template <typename QT>
__global__ __launch_bounds__(256) void extract_dms_kernel(
    QT* __restrict__ q, int64_t qs_t, int64_t qs_h, int64_t qs_d, uint8_t* __restrict__ evict,
    int64_t es_t, int64_t es_h, int64_t total, int num_kv_heads, int group_size, int head_dim,
    float alpha_scale, float alpha_offset, float threshold, int positive_scale) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t t = i / num_kv_heads;
  const int h = (int)(i - t * num_kv_heads);
  QT* p = q + t * qs_t + (int64_t)h * group_size * qs_h + (int64_t)(head_dim - 1) * qs_d;
  const float v = ld<QT>(p);
  const bool e = dms_decide(v, alpha_scale, alpha_offset, threshold, positive_scale);
  evict[t * es_t + h * es_h] = e ? 1 : 0;
  st<QT>(p, 0.0f);
}

FDMS_EXPORT int fdms_extract_dms_decisions(void* q, int q_dtype, int64_t qs_t, int64_t qs_h, int64_t qs_d,
                                           uint8_t* evict, int64_t es_t, int64_t es_h, int64_t num_tokens,
                                           int num_kv_heads, int group_size, int head_dim, float alpha_scale,
                                           float alpha_offset, float threshold, int positive_scale,
                                           void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || group_size <= 0 || head_dim <= 0) return (int)hipErrorInvalidValue;
  const int64_t total = num_tokens * num_kv_heads;
  if (total == 0) return 0;
  if (!q || !evict) return (int)hipErrorInvalidValue;
  const int block = 256;
  const int64_t grid = (total + block - 1) / block;
  FDMS_DISPATCH_FLOAT(q_dtype, QT,
    hipLaunchKernelGGL(extract_dms_kernel<QT>, dim3((unsigned)grid), dim3(block), 0, (hipStream_t)stream,
                       (QT*)q, qs_t, qs_h, qs_d, evict, es_t, es_h, total, num_kv_heads, group_size, head_dim,
                       alpha_scale, alpha_offset, threshold, positive_scale));
  FDMS_LAUNCH_CHECK();
  return 0;
}
