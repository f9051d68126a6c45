// Decode-step metadata (reference: fastdms/engine/compact_kv.py:1727-1770
// prepare_decode_metadata, 426-484 + 1562-1725 record_appended_dms_decisions).
//
// prepare: slot[l,b,h] = base + live; live += 1 (the append slot of this step,
//          reserved before the forward).
// record:  positions[l,row_b,h,live-1] = pos[b]; evict[...] = evict_all[l,b,h]
//          (the appended token's DMS decision, after the forward).
// One thread per (layer, seq, head); one launch for all layers.  Launch-bound.
#include "fdms_common.h"

__global__ void prepare_decode_kernel(const int32_t* __restrict__ base, int64_t b_l, int64_t b_b, int64_t b_h,
                                      int32_t* __restrict__ live, int64_t l_l, int64_t l_b, int64_t l_h,
                                      int32_t* __restrict__ slot, int64_t s_l, int64_t s_b, int64_t s_h, int num_seqs,
                                      int num_kv_heads, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int h = i % num_kv_heads;
  const int b = (i / num_kv_heads) % num_seqs;
  const int l = i / (num_kv_heads * num_seqs);
  int32_t* lp = live + l * l_l + b * l_b + h * l_h;
  const int32_t old = *lp;
  slot[l * s_l + b * s_b + h * s_h] = base[l * b_l + b * b_b + h * b_h] + old;
  *lp = old + 1;
}

FDMS_EXPORT int fdms_prepare_decode_metadata(const int32_t* base, int64_t b_l, int64_t b_b, int64_t b_h,
                                             int32_t* live, int64_t l_l, int64_t l_b, int64_t l_h,
                                             int32_t* slot_out, int64_t s_l, int64_t s_b, int64_t s_h,
                                             int num_layers, int num_seqs, int num_kv_heads, void* stream) {
  if (num_layers <= 0 || num_seqs < 0 || num_kv_heads <= 0) return (int)hipErrorInvalidValue;
  const int total = num_layers * num_seqs * num_kv_heads;
  if (total == 0) return 0;
  if (!base || !live || !slot_out) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(prepare_decode_kernel, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream, base, b_l,
                     b_b, b_h, live, l_l, l_b, l_h, slot_out, s_l, s_b, s_h, num_seqs, num_kv_heads, total);
  FDMS_LAUNCH_CHECK();
  return 0;
}

__global__ void record_decisions_kernel(int32_t* __restrict__ positions, int64_t p_l, int64_t p_s, int64_t p_h,
                                        int64_t p_c, uint8_t* __restrict__ evict, int64_t e_l, int64_t e_s,
                                        int64_t e_h, int64_t e_c, const int32_t* __restrict__ live, int64_t l_l,
                                        int64_t l_s, int64_t l_h, const uint8_t* __restrict__ evict_all, int64_t a_l,
                                        int64_t a_b, int64_t a_h, const void* __restrict__ cur_positions,
                                        int pos_is_64, const int32_t* __restrict__ meta_rows, int row_start,
                                        int num_seqs, int num_kv_heads, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int h = i % num_kv_heads;
  const int b = (i / num_kv_heads) % num_seqs;
  const int l = i / (num_kv_heads * num_seqs);
  const int64_t row = meta_rows ? meta_rows[b] : (int64_t)row_start + b;
  const int64_t idx = (int64_t)live[l * l_l + row * l_s + h * l_h] - 1;
  const int32_t p = pos_is_64 ? (int32_t)((const int64_t*)cur_positions)[b] : ((const int32_t*)cur_positions)[b];
  positions[l * p_l + row * p_s + h * p_h + idx * p_c] = p;
  evict[l * e_l + row * e_s + h * e_h + idx * e_c] = evict_all[l * a_l + b * a_b + h * a_h];
}

FDMS_EXPORT int fdms_record_dms_decisions(int32_t* positions, int64_t p_l, int64_t p_s, int64_t p_h, int64_t p_c,
                                          uint8_t* evict, int64_t e_l, int64_t e_s, int64_t e_h, int64_t e_c,
                                          const int32_t* live, int64_t l_l, int64_t l_s, int64_t l_h,
                                          const uint8_t* evict_all, int64_t a_l, int64_t a_b, int64_t a_h,
                                          const void* cur_positions, int pos_is_64, const int32_t* meta_rows,
                                          int row_start, int num_layers, int num_seqs, int num_kv_heads,
                                          void* stream) {
  if (num_layers <= 0 || num_seqs < 0 || num_kv_heads <= 0) return (int)hipErrorInvalidValue;
  const int total = num_layers * num_seqs * num_kv_heads;
  if (total == 0) return 0;
  if (!positions || !evict || !live || !evict_all || !cur_positions) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(record_decisions_kernel, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     positions, p_l, p_s, p_h, p_c, evict, e_l, e_s, e_h, e_c, live, l_l, l_s, l_h, evict_all, a_l,
                     a_b, a_h, cur_positions, pos_is_64, meta_rows, row_start, num_seqs, num_kv_heads, total);
  FDMS_LAUNCH_CHECK();
  return 0;
}
