// Decode-step DMS decision + RoPE + compact append (reference:
// fastdms/layers/compact_attention.py:67-209 fused kernel, 968-1113 wrappers,
// 212-246 unfused store).
//
// One block per (sequence, kv head); thread j owns the RoPE pair (j, j+D/2)
// of every query head of the GQA group and of the key.  RoPE is computed with
// explicitly rounded fp32 multiplies/adds (no contraction into FMA), so the
// stored values are a fixed function of the inputs.  The rotated key goes to
// the arena straight from fp32; v is stored from its own dtype.
#include "fdms_vec.h"

using namespace fdms;

template <typename QT, typename KT, typename CT>
__global__ void dms_rope_store_kernel(QT* __restrict__ q, KT* __restrict__ k, const KT* __restrict__ v,
                                      const float* __restrict__ cos_sin, CT* __restrict__ ck, CT* __restrict__ cv,
                                      const int32_t* __restrict__ slot_mapping, uint8_t* __restrict__ evict_out,
                                      const int64_t* __restrict__ positions, int64_t qs_b, int64_t qs_h,
                                      int64_t ks_b, int64_t ks_h, int64_t vs_b, int64_t vs_h, int64_t cs_p,
                                      int64_t cs_d, int64_t c_s, int64_t sm_b, int64_t sm_h, int64_t ev_b,
                                      int64_t ev_h, int num_kv_heads, int group_size, int head_dim,
                                      float alpha_scale, float alpha_offset, float threshold, int positive_scale,
                                      int store_q, int store_transient_k, const float* __restrict__ k_scale,
                                      const float* __restrict__ v_scale) {
  const int h = blockIdx.x % num_kv_heads;
  const int b = blockIdx.x / num_kv_heads;
  const int half = head_dim / 2;
  const int j = threadIdx.x;
  if (j >= half) return;
  const int64_t pos = positions[b];
  const float c = cos_sin[pos * cs_p + (int64_t)j * cs_d];
  const float s = cos_sin[pos * cs_p + (int64_t)(j + half) * cs_d];
  QT* qg = q + b * qs_b + (int64_t)h * group_size * qs_h;
  if (j == half - 1) {
    // The decision lane (g=0, d=D-1) is owned by this thread: read it before
    // any store to q.
    const float dv = ld<QT>(qg + (head_dim - 1));
    const bool e = dms_decide(dv, alpha_scale, alpha_offset, threshold, positive_scale);
    evict_out[b * ev_b + h * ev_h] = e ? 1 : 0;
  }
  if (store_q) {
    for (int g = 0; g < group_size; ++g) {
      QT* qh = qg + (int64_t)g * qs_h;
      const float x1 = ld<QT>(qh + j);
      float x2 = ld<QT>(qh + j + half);
      if (g == 0 && j == half - 1) x2 = 0.0f;
      float y1, y2;
      rope_f32(x1, x2, c, s, &y1, &y2);
      st<QT>(qh + j, y1);
      st<QT>(qh + j + half, y2);
    }
  }
  KT* kh = k + b * ks_b + h * ks_h;
  float y1, y2;
  rope_f32(ld<KT>(kh + j), ld<KT>(kh + j + half), c, s, &y1, &y2);
  if (store_transient_k) {
    st<KT>(kh + j, y1);
    st<KT>(kh + j + half, y2);
  }
  const int32_t slot = slot_mapping[b * sm_b + h * sm_h];
  if (slot >= 0) {
    // per-head FP8 scales: stored = x * (1 / scale) (none: x)
    CT* dk = ck + (int64_t)slot * c_s;
    CT* dv = cv + (int64_t)slot * c_s;
    const float km = inv_scale(k_scale, h);
    st<CT>(dk + j, y1 * km);
    st<CT>(dk + j + half, y2 * km);
    const KT* vh = v + b * vs_b + h * vs_h;
    if (v_scale) {
      const float vm = inv_scale(v_scale, h);
      st<CT>(dv + j, ld<KT>(vh + j) * vm);
      st<CT>(dv + j + half, ld<KT>(vh + j + half) * vm);
    } else {
      Copy<KT, CT>::run(dv + j, vh + j);
      Copy<KT, CT>::run(dv + j + half, vh + j + half);
    }
  }
}

FDMS_EXPORT int fdms_dms_rope_store_compact_decode(
    void* q, int q_dtype, int64_t qs_b, int64_t qs_h, void* k, const void* v, int kv_dtype, int64_t ks_b,
    int64_t ks_h, int64_t vs_b, int64_t vs_h, const float* cos_sin, int64_t cs_p, int64_t cs_d, void* compact_k,
    void* compact_v, int compact_dtype, int64_t c_s, const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h,
    uint8_t* evict_out, int64_t ev_b, int64_t ev_h, const int64_t* positions, int batch, int num_kv_heads,
    int group_size, int head_dim, float alpha_scale, float alpha_offset, float threshold, int positive_scale,
    int store_q, int store_transient_k, const float* k_scale, const float* v_scale, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || group_size <= 0 || head_dim <= 0 || head_dim % 2) return (int)hipErrorInvalidValue;
  if ((k_scale || v_scale) && compact_dtype != kFP8) return (int)hipErrorInvalidValue;
  if (head_dim > 512) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  if (!q || !k || !v || !cos_sin || !compact_k || !compact_v || !slot_mapping || !evict_out || !positions)
    return (int)hipErrorInvalidValue;
  const int threads = ((head_dim / 2 + 63) / 64) * 64;
  FDMS_DISPATCH_FLOAT(q_dtype, QT,
    FDMS_DISPATCH_FLOAT(kv_dtype, KT,
      FDMS_DISPATCH_DTYPE(compact_dtype, CT,
        hipLaunchKernelGGL((dms_rope_store_kernel<QT, KT, CT>), dim3(batch * num_kv_heads), dim3(threads), 0,
                           (hipStream_t)stream, (QT*)q, (KT*)k, (const KT*)v, cos_sin, (CT*)compact_k,
                           (CT*)compact_v, slot_mapping, evict_out, positions, qs_b, qs_h, ks_b, ks_h, vs_b, vs_h,
                           cs_p, cs_d, c_s, sm_b, sm_h, ev_b, ev_h, num_kv_heads, group_size, head_dim, alpha_scale,
                           alpha_offset, threshold, positive_scale, store_q, store_transient_k, k_scale,
                           v_scale))));
  FDMS_LAUNCH_CHECK();
  return 0;
}

// compact_attention.py:212-246: compact[slot] = key/value (cast on store).
template <typename KT, typename CT>
__global__ void store_compact_kernel(const KT* __restrict__ key, const KT* __restrict__ value, CT* __restrict__ ck,
                                     CT* __restrict__ cv, const int32_t* __restrict__ slot_mapping, int64_t ks_b,
                                     int64_t ks_h, int64_t vs_b, int64_t vs_h, int64_t c_s, int64_t sm_b,
                                     int64_t sm_h, int num_kv_heads, int head_dim, const float* __restrict__ k_scale,
                                     const float* __restrict__ v_scale) {
  const int h = blockIdx.x % num_kv_heads;
  const int b = blockIdx.x / num_kv_heads;
  const int32_t slot = slot_mapping[b * sm_b + h * sm_h];
  if (slot < 0) return;
  const float km = inv_scale(k_scale, h), vm = inv_scale(v_scale, h);
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    if (k_scale || v_scale) {  // per-head FP8 scales: stored = x * (1 / scale)
      st<CT>(ck + (int64_t)slot * c_s + d, ld<KT>(key + b * ks_b + h * ks_h + d) * km);
      st<CT>(cv + (int64_t)slot * c_s + d, ld<KT>(value + b * vs_b + h * vs_h + d) * vm);
    } else {
      Copy<KT, CT>::run(ck + (int64_t)slot * c_s + d, key + b * ks_b + h * ks_h + d);
      Copy<KT, CT>::run(cv + (int64_t)slot * c_s + d, value + b * vs_b + h * vs_h + d);
    }
  }
}

FDMS_EXPORT int fdms_store_compact_kvcache(const void* key, const void* value, int kv_dtype, int64_t ks_b,
                                           int64_t ks_h, int64_t vs_b, int64_t vs_h, void* compact_k,
                                           void* compact_v, int compact_dtype, int64_t c_s,
                                           const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, int batch,
                                           int num_kv_heads, int head_dim, const float* k_scale,
                                           const float* v_scale, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || head_dim <= 0) return (int)hipErrorInvalidValue;
  if ((k_scale || v_scale) && compact_dtype != kFP8) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  if (!key || !value || !compact_k || !compact_v || !slot_mapping) return (int)hipErrorInvalidValue;
  FDMS_DISPATCH_DTYPE(kv_dtype, KT,
    FDMS_DISPATCH_DTYPE(compact_dtype, CT,
      hipLaunchKernelGGL((store_compact_kernel<KT, CT>), dim3(batch * num_kv_heads), dim3(64), 0,
                         (hipStream_t)stream, (const KT*)key, (const KT*)value, (CT*)compact_k, (CT*)compact_v,
                         slot_mapping, ks_b, ks_h, vs_b, vs_h, c_s, sm_b, sm_h, num_kv_heads, head_dim, k_scale,
                         v_scale)));
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Prefill RoPE in place on a [tokens, heads, D] view (rotary_embedding.py:75-86:
// x <- cast(rotate(x.float(), cos[pos], sin[pos]))).  One block per token,
// thread per (head, pair).
template <typename T>
__global__ void rope_inplace_kernel(T* __restrict__ x, int64_t xs_t, int64_t xs_h, const float* __restrict__ cos_sin,
                                    int64_t cs_p, int64_t cs_d, const int64_t* __restrict__ positions, int num_heads,
                                    int head_dim) {
  const int64_t t = blockIdx.x;
  const int half = head_dim / 2;
  const int64_t pos = positions[t];
  for (int i = threadIdx.x; i < num_heads * half; i += blockDim.x) {
    const int h = i / half, j = i - h * half;
    T* xh = x + t * xs_t + (int64_t)h * xs_h;
    const float c = cos_sin[pos * cs_p + (int64_t)j * cs_d];
    const float s = cos_sin[pos * cs_p + (int64_t)(j + half) * cs_d];
    float y1, y2;
    rope_f32(ld<T>(xh + j), ld<T>(xh + j + half), c, s, &y1, &y2);
    st<T>(xh + j, y1);
    st<T>(xh + j + half, y2);
  }
}

FDMS_EXPORT int fdms_rope_inplace(void* x, int dtype, int64_t xs_t, int64_t xs_h, int64_t num_tokens, int num_heads,
                                  int head_dim, const float* cos_sin, int64_t cs_p, int64_t cs_d,
                                  const int64_t* positions, void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 2) return (int)hipErrorInvalidValue;
  if (num_tokens == 0) return 0;
  if (!x || !cos_sin || !positions || num_tokens > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  FDMS_DISPATCH_FLOAT(dtype, T,
    hipLaunchKernelGGL((rope_inplace_kernel<T>), dim3((unsigned)num_tokens), dim3(256), 0, (hipStream_t)stream,
                       (T*)x, xs_t, xs_h, cos_sin, cs_p, cs_d, positions, num_heads, head_dim));
  FDMS_LAUNCH_CHECK();
  return 0;
}
