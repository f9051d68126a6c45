/*
 * fastdms_amd C-ABI — MI355X (gfx950) HIP kernels for FastDMS's compact-DMS
 * inference hot path.
 *
 * Conventions (all entry points):
 *   - return 0 on success, a hipError_t code otherwise (hipErrorInvalidValue = 1
 *     for rejected arguments; nothing is launched then);
 *   - tensors are raw device pointers; strides are in ELEMENTS of the pointed
 *     type unless the name ends in _bytes; the innermost (head_dim / slot)
 *     dimension is contiguous;
 *   - dtype codes: 0 = float32, 1 = float16, 2 = bfloat16, 3 = float8_e4m3fn
 *     (OCP; stores round to nearest-even and saturate to +-448);
 *   - bool tensors are uint8_t (0/1);
 *   - `stream` is a hipStream_t; kernels are enqueued on it and never
 *     synchronise, allocate or call hipMemset, so every call is capturable in a
 *     HIP graph;
 *   - k_scale / v_scale (where taken): optional per-kv-head FP8 scale tables
 *     [num_kv_heads] fp32 of the layer (NULL = none, the reference's bare
 *     cast).  Stores write e4m3(x * fp32(1 / scale)); the matrix-core
 *     attention kernel dequantises in registers (K scale folded into the score
 *     scale, V scale on the output).  No reference counterpart: the reference
 *     casts K/V to FP8 without a scale (compact_kv.py:243-252,
 *     compact_attention.py:387, 399).  Only FP8 arenas take scales.
 *
 * Reference citations are path:line in shisa-ai/FastDMS.
 */
#ifndef FASTDMS_AMD_H
#define FASTDMS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header (2: per-kv-head FP8 scale tables on the pack,
 * append and attention entry points; 3: the paged compact-KV entry points, the
 * FP8 GEMM, and the producer-side activation amax / FP8 split partials on
 * fdms_linear_small_m and the RMSNorm entry points; 4: the QK-norm weights on
 * the fused decode attention entry points). */
int fdms_abi_version(void);

/* Plain 16-byte-vector copy used to calibrate HBM byte counters and the copy
 * roofline (no reference counterpart: measurement support). */
int fdms_copy_bytes(const void* src, void* dst, int64_t nbytes, int num_blocks, void* stream);

/* Element-wise dtype conversion with the library's store rounding (no
 * reference counterpart: exposes the cast the reference's Triton stores apply,
 * compact_kv.py:243-252, for exhaustive tests).  Runs the row kernels' vector
 * conversion (FP8 encoded four values at a time); src and dst must be aligned
 * to four elements. */
int fdms_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream);

/* Decode n (multiple of 4) FP8 e4m3fn bytes to fp32 with the hardware
 * conversion the attention kernels use (no reference counterpart: lets a test
 * check that instruction against the format on all 256 codes). */
int fdms_fp8_decode_hw(const void* in, float* out, int64_t n, void* stream);

/* A1 — DMS decision extraction.  Replaces _extract_dms_eviction_decisions_kernel
 * and the CUDA branch of extract_dms_eviction_decisions (fastdms/engine/dms.py:12-42,
 * 196-220).  evict[t,h] = q[t, h*G, D-1] > threshold (positive_scale, threshold =
 * fp32(alpha_offset/alpha_scale)) or q*alpha_scale - alpha_offset > 0; then
 * q[t, h*G, D-1] = 0. */
int fdms_extract_dms_decisions(void* q, int q_dtype, int64_t qs_t, int64_t qs_h, int64_t qs_d, uint8_t* evict,
                               int64_t es_t, int64_t es_h, int64_t num_tokens, int num_kv_heads, int group_size,
                               int head_dim, float alpha_scale, float alpha_offset, float threshold,
                               int positive_scale, void* stream);

/* A4 — prefill pack counts + exclusive chunk scan.  Replaces
 * _streaming_pack_count_kernel + _streaming_pack_fused_rank_prepare
 * (fastdms/engine/compact_kv.py:140-165, 265-296).  One call covers a ragged
 * batch: cu_seqlens [num_seqs+1] (device) or, when NULL, one sequence of
 * single_len tokens.  Outputs live[b,h] and block_offsets[b,h,chunk] (256-token
 * chunks).  When positions != NULL the (seq, head) metadata rows are first reset
 * to (-1, 0) over meta_cap slots (compact_kv.py:1031-1032); meta_rows maps a
 * batch index to its metadata row (NULL = identity). */
int fdms_streaming_pack_prepare(const uint8_t* evict, int64_t es_t, int64_t es_h, const int32_t* cu_seqlens,
                                int single_len, int num_seqs, int window, int num_kv_heads, int max_chunks,
                                int32_t* live_out, int64_t lo_b, int64_t lo_h, int32_t* block_offsets, int64_t of_b,
                                int64_t of_h, int64_t of_c, int32_t* positions, uint8_t* evict_meta,
                                const int32_t* meta_rows, int64_t tp_b, int64_t tp_h, int64_t em_b, int64_t em_h,
                                int meta_cap, void* stream);

/* A5 — fused rank scatter of kept K/V rows into compact spans.  Replaces
 * _streaming_pack_rank_scatter_kernel / _streaming_pack_rank_scatter_triton
 * (compact_kv.py:168-262, 299-361).  compact[base[b,h] + rank] = cast(k/v[t,h]),
 * positions[row_b,h,rank] = t, evict_meta[row_b,h,rank] = evict[t,h].  Ragged
 * batch via cu_seqlens as above (k/v indexed at cu[b]+t, or single_start+t). */
int fdms_streaming_pack_rank_scatter(const void* k, const void* v, int kv_dtype, int64_t ks_t, int64_t ks_h,
                                     int64_t vs_t, int64_t vs_h, const uint8_t* evict, int64_t es_t, int64_t es_h,
                                     const int32_t* cu_seqlens, int single_start, int single_len, int num_seqs,
                                     const int32_t* block_offsets, int64_t bo_b, int64_t bo_h, int64_t bo_c,
                                     const int32_t* base, int64_t bs_b, int64_t bs_h, void* compact_k,
                                     void* compact_v, int compact_dtype, int64_t cs_s, int32_t* positions,
                                     uint8_t* evict_meta, const int32_t* meta_rows, int64_t tp_b, int64_t tp_h,
                                     int64_t tp_s, int64_t em_b, int64_t em_h, int64_t em_s, int window,
                                     int num_kv_heads, int head_dim, int max_chunks, int vec, const float* k_scale,
                                     const float* v_scale, void* stream);

/* A6 — scatter with precomputed keep/rank.  Replaces _streaming_pack_scatter_kernel
 * / _streaming_pack_scatter_triton (compact_kv.py:38-137, 364-423). */
int fdms_streaming_pack_scatter(const void* k, const void* v, int kv_dtype, int64_t ks_t, int64_t ks_h,
                                int64_t vs_t, int64_t vs_h, const uint8_t* keep, int64_t kp_t, int64_t kp_h,
                                const int32_t* rank, int64_t rk_t, int64_t rk_h, const uint8_t* seq_evict,
                                int64_t es_t, int64_t es_h, const int32_t* base, int64_t bs_h, void* compact_k,
                                void* compact_v, int compact_dtype, int64_t cs_s, int32_t* positions, int64_t tp_h,
                                int64_t tp_s, uint8_t* evict_meta, int64_t em_h, int64_t em_s, int start,
                                int seq_len, int num_kv_heads, int head_dim, int vec, const float* k_scale,
                                const float* v_scale, void* stream);

/* A9 — fused decode DMS decision + RoPE + compact append.  Replaces
 * _dms_rope_store_compact_decode_kernel / fused_dms_rope_store_compact_decode
 * (fastdms/layers/compact_attention.py:67-209, 1010-1113).  cos_sin is the fp32
 * [max_pos, 1, D] cat(cos, sin) cache; positions are int64. */
int fdms_dms_rope_store_compact_decode(void* q, int q_dtype, int64_t qs_b, int64_t qs_h, void* k, const void* v,
                                       int kv_dtype, int64_t ks_b, int64_t ks_h, int64_t vs_b, int64_t vs_h,
                                       const float* cos_sin, int64_t cs_p, int64_t cs_d, void* compact_k,
                                       void* compact_v, int compact_dtype, int64_t c_s, const int32_t* slot_mapping,
                                       int64_t sm_b, int64_t sm_h, uint8_t* evict_out, int64_t ev_b, int64_t ev_h,
                                       const int64_t* positions, int batch, int num_kv_heads, int group_size,
                                       int head_dim, float alpha_scale, float alpha_offset, float threshold,
                                       int positive_scale, int store_q, int store_transient_k, const float* k_scale,
                                       const float* v_scale, void* stream);

/* B8 — prefill RoPE in place on a [tokens, heads, D] view.  Replaces
 * RotaryEmbedding.forward / apply_rotary_emb (fastdms/layers/rotary_embedding.py:7-15,
 * 75-86): x = cast(x1*cos - x2*sin, x2*cos + x1*sin) computed in fp32. */
int fdms_rope_inplace(void* x, int dtype, int64_t xs_t, int64_t xs_h, int64_t num_tokens, int num_heads,
                      int head_dim, const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
                      void* stream);

/* A10 — unfused append store.  Replaces _store_compact_kvcache_kernel /
 * store_compact_kvcache (compact_attention.py:212-246, 968-1007). */
int fdms_store_compact_kvcache(const void* key, const void* value, int kv_dtype, int64_t ks_b, int64_t ks_h,
                               int64_t vs_b, int64_t vs_h, void* compact_k, void* compact_v, int compact_dtype,
                               int64_t c_s, const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, int batch,
                               int num_kv_heads, int head_dim, const float* k_scale, const float* v_scale,
                               void* stream);

/* B2/B3/B5 — split-K GQA decode attention over compact spans with the split
 * merge fused into the same launch.  Replaces compact_decode_attention and its
 * partial + reduce kernels (compact_attention.py:334-415, 537-603, 1116-1336).
 * Span addressing: base_offsets[b,h] + r (block_tables == NULL); paged:
 * block_tables[b,h,r/page_size]*page_size + r%page_size.  workspace holds
 * batch*num_kv_heads*num_splits*group_size*(head_dim+2) floats and counters
 * batch*num_kv_heads ints that must be zero before the first call (every call
 * leaves them zero).  Calls that share counters must not overlap in time.
 * rope_positions != NULL rotates q in-kernel with the decision lane zeroed
 * (B4, _compact_decode_grouped_splitk_partial_qrope_kernel, compact_attention.py:418-534).
 * The matrix-core kernel (bf16 q, FP8 K/V, group_size <= 4, head_dim 64 /
 * 128) runs a pair of at most split_rows live rows (rounded up to 64; 0 = one
 * 64-row group per wave of the workgroup) as one workgroup with no merge and
 * splits a longer one into ceil(live / h) workgroups, at most num_splits,
 * with h = split_rows / 2 at head_dim 64 for at most 128 (seq, kv head) pairs
 * and h = split_rows otherwise; the other kernels ignore
 * split_rows and divide every pair's live span evenly over num_splits.  Split
 * partials are handed over with agent-scope atomic stores / loads ordered
 * around the ticket (no L2 write-back or invalidate).  The matrix-core kernel
 * takes the live-count and block-table strides (and, fused, the slot_mapping
 * strides) as int32: larger ones are hipErrorInvalidValue. */
int fdms_compact_decode_attention(const void* q, int q_dtype, int64_t qs_b, int64_t qs_h, const void* compact_k,
                                  const void* compact_v, int kv_dtype, int64_t c_s, const int32_t* base_offsets,
                                  int64_t bo_b, int64_t bo_h, const int32_t* block_tables, int64_t bt_b,
                                  int64_t bt_h, int page_size, const int32_t* live_counts, int64_t lc_b,
                                  int64_t lc_h, void* out, int64_t os_b, int64_t os_h, float* workspace,
                                  int* counters, int batch, int num_kv_heads, int group_size, int head_dim,
                                  int num_splits, int split_rows, float scale, const float* rope_cos_sin,
                                  int64_t rcs_p, int64_t rcs_d, const int64_t* rope_positions, const float* k_scale,
                                  const float* v_scale, void* stream);

/* A9 + B2-B5 — decode preprocess and attention in one launch: the reference's
 * fused_dms_rope_store_compact_decode(store_q=False, store_transient_k=False)
 * (compact_attention.py:67-209, 1010-1113) followed by compact_decode_attention
 * with in-kernel q RoPE (418-534, 1116-1336), as llama.py:112-134 sequences them.
 * q / k / v are the step's raw bf16 rows (not written back).  The DMS decision
 * goes to evict_out, RoPE(k) and v are appended as FP8 at slot_mapping[b,h]
 * (skipped when < 0), and the appended token is rank live-1 of the flat span
 * (prepare_decode_metadata has already counted it).  Matrix-core path only:
 * FP8 compact K/V with 16-byte rows, group_size <= 4, head_dim 64 / 128.
 * Workspace, counters and split_rows as for fdms_compact_decode_attention.
 * q_norm / k_norm (bf16 [head_dim], or NULL): Qwen3's QK-norm, applied to each
 * raw q / k head first, bf16(bf16(x * rsqrt(mean(x^2) + norm_eps)) * w) as
 * the RMSNorm entry points compute it (qwen3.py:92-94, before the DMS
 * extraction and RoPE), replacing the two RMSNorm launches before this one. */
int fdms_fused_decode_attention(const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b,
                                int64_t ks_h, const void* v, int64_t vs_b, int64_t vs_h, const float* cos_sin,
                                int64_t cs_p, int64_t cs_d, const int64_t* positions, const int32_t* slot_mapping,
                                int64_t sm_b, int64_t sm_h, uint8_t* evict_out, int64_t ev_b, int64_t ev_h,
                                float alpha_scale, float alpha_offset, float threshold, int positive_scale,
                                void* compact_k, void* compact_v, int64_t c_s, const int32_t* base_offsets,
                                int64_t bo_b, int64_t bo_h, const int32_t* live_counts, int64_t lc_b, int64_t lc_h,
                                void* out, int64_t os_b, int64_t os_h, float* workspace, int* counters, int batch,
                                int num_kv_heads, int group_size, int head_dim, int num_splits, int split_rows,
                                float scale, const float* k_scale, const float* v_scale, const void* q_norm,
                                const void* k_norm, float norm_eps, void* stream);

/* Allocation-free fdms_fused_decode_attention (no reference counterpart): for
 * callers that cannot allocate (code under HIP graph capture, serving loops
 * that forbid hipMalloc).  Same arguments minus workspace / counters: the split
 * partials and tickets live in the library's own device array (one per GPU,
 * held until the process ends; looked up with hipGetSymbolAddress on the first
 * call on a device).  Limit: batch * num_kv_heads * num_splits * group_size *
 * (head_dim + 2) <= 2^21 floats and batch * num_kv_heads <= 16384, else
 * hipErrorInvalidValue.  Every call on a GPU shares that array and leaves its
 * tickets zero: calls that overlap in time on one GPU (other streams, other
 * threads) race and must not be issued. */
int fdms_fused_decode_attention_noalloc(const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b,
                                        int64_t ks_h, const void* v, int64_t vs_b, int64_t vs_h,
                                        const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
                                        const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, uint8_t* evict_out,
                                        int64_t ev_b, int64_t ev_h, float alpha_scale, float alpha_offset,
                                        float threshold, int positive_scale, void* compact_k, void* compact_v,
                                        int64_t c_s, const int32_t* base_offsets, int64_t bo_b, int64_t bo_h,
                                        const int32_t* live_counts, int64_t lc_b, int64_t lc_h, void* out,
                                        int64_t os_b, int64_t os_h, int batch, int num_kv_heads, int group_size,
                                        int head_dim, int num_splits, int split_rows, float scale,
                                        const float* k_scale, const float* v_scale, const void* q_norm,
                                        const void* k_norm, float norm_eps, void* stream);

/* A12/A13 — decode expiry, full (incremental = 0) or incremental (1).  Replaces
 * _dms_expiry_kernel / dms_expiry_one_layer and _dms_expiry_incremental_kernel /
 * dms_expiry_incremental_one_layer (compact_attention.py:690-965) and the
 * per-layer loops of compact_kv.py:1396-1560; semantics of the exact torch path
 * compact_kv.py:1263-1337.  Metadata is [layer, seq, head, slot] with strides;
 * arenas come from layer_k/layer_v (device tables of per-layer base addresses)
 * or, for num_layers == 1, compact_k/compact_v.  Rows move as row_bytes bytes
 * at a c_s_bytes slot stride.  Slots at or beyond live are expected to hold
 * (-1, 0) already, as the reference's append/record path leaves them. */
int fdms_dms_expiry(int incremental, int32_t* positions, int64_t ps_l, int64_t ps_s, int64_t ps_h, uint8_t* evict,
                    int64_t es_l, int64_t es_s, int64_t es_h, int32_t* live_counts, int64_t lc_l, int64_t lc_s,
                    int64_t lc_h, const int32_t* base_offsets, int64_t bo_l, int64_t bo_s, int64_t bo_h,
                    void* compact_k, void* compact_v, const uint64_t* layer_k, const uint64_t* layer_v,
                    int64_t row_bytes, int64_t c_s_bytes, const int64_t* current_positions, int num_layers,
                    int num_seqs, int num_kv_heads, int window, void* stream);

/* A15 — decode append slots.  Replaces prepare_decode_metadata
 * (compact_kv.py:1727-1770): slot_out[l,b,h] = base + live; live += 1.  Every
 * operand is a strided [layers, seqs, kv_heads] view. */
int fdms_prepare_decode_metadata(const int32_t* base, int64_t b_l, int64_t b_b, int64_t b_h, int32_t* live,
                                 int64_t l_l, int64_t l_b, int64_t l_h, int32_t* slot_out, int64_t s_l,
                                 int64_t s_b, int64_t s_h, int num_layers, int num_seqs, int num_kv_heads,
                                 void* stream);

/* A14 — record the appended token's decision.  Replaces
 * _record_dms_decisions_layer_major_kernel / record_appended_dms_decisions
 * (compact_kv.py:426-484, 1562-1725): positions[l,row,h,live-1] = pos[b],
 * evict[l,row,h,live-1] = evict_all[l,b,h]; row = meta_rows[b] or row_start + b. */
int fdms_record_dms_decisions(int32_t* positions, int64_t p_l, int64_t p_s, int64_t p_h, int64_t p_c,
                              uint8_t* evict, int64_t e_l, int64_t e_s, int64_t e_h, int64_t e_c,
                              const int32_t* live, int64_t l_l, int64_t l_s, int64_t l_h, const uint8_t* evict_all,
                              int64_t a_l, int64_t a_b, int64_t a_h, const void* cur_positions, int pos_is_64,
                              const int32_t* meta_rows, int row_start, int num_layers, int num_seqs,
                              int num_kv_heads, void* stream);

/* B1 — dense causal prefill attention over a ragged batch (bf16, head_dim 64
 * or 128, GQA).  Replaces the reference's flash_attn_varlen_func(causal=True)
 * call (fastdms/layers/attention.py:85-92).  Rows are 16-byte aligned;
 * cu_seqlens [num_seqs+1] on the device; max_seqlen bounds the grid. */
int fdms_prefill_attention(const void* q, int64_t qs_t, int64_t qs_h, const void* k, int64_t ks_t, int64_t ks_h,
                           const void* v, int64_t vs_t, int64_t vs_h, void* out, int64_t os_t, int64_t os_h,
                           const int32_t* cu_seqlens, int num_seqs, int max_seqlen, int num_q_heads,
                           int num_kv_heads, int head_dim, float scale, void* stream);

/* B1 with separate query and key ranges (the reference's
 * flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, causal=True),
 * attention.py:85-92): sequence s has query rows cu_seqlens_q[s] ..
 * cu_seqlens_q[s+1]-1 of q / out and keys cu_seqlens_k[s] .. cu_seqlens_k[s+1]-1
 * of k / v, the queries being the last of the keys (bottom-right causal
 * alignment: query i of n attends to keys 0 .. klen - n + i).  A chunk of a
 * long prompt passes the retained earlier chunks' K/V plus its own.  Needs
 * klen >= qlen for every sequence (a sequence with fewer keys than queries is
 * skipped and its rows are not written); max_seqlen_q bounds the grid. */
int fdms_prefill_attention_varlen(const void* q, int64_t qs_t, int64_t qs_h, const void* k, int64_t ks_t,
                                  int64_t ks_h, const void* v, int64_t vs_t, int64_t vs_h, void* out, int64_t os_t,
                                  int64_t os_h, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int num_seqs, int max_seqlen_q, int num_q_heads, int num_kv_heads, int head_dim,
                                  float scale, void* stream);

/* One v_mfma_f32_16x16x32_bf16 with the operand layout the attention kernels
 * assume (no reference counterpart: a lane-layout self-check for tests). */
int fdms_mfma_probe(const void* a, const void* b, float* c, void* stream);

/* Residual-add + RMSNorm, bf16 (fastdms/layers/layernorm.py:16-40).  Row r of the
 * input is at in + (r/heads)*in_stride + (r%heads)*in_head_stride (heads > 1
 * normalises each head of a strided [tokens, heads, D] view, Qwen3 QK-norm,
 * qwen3.py:92-94).  amax_out (optional, fp32 [rows]) = max |out[r, :]| (NaN if
 * the row holds a NaN): the row statistic of the consuming FP8 linear's
 * activation quantisation (fdms_linear_small_m's x_amax), so that linear
 * skips its own pass over x.  q_out (optional, with amax_out; e4m3fn [rows,
 * q_stride], 8-byte aligned) = that quantisation done here once:
 * e4m3fn(out * s), s = 448 / amax (1 if amax is 0 or NaN; q_mode 1 divides,
 * 2 rounds as reciprocal(amax) * 448), RNE with saturation
 * (linear.py:514-523, 683-694); the linear then reads the codes (x_dtype
 * FP8).  out may be null when q_out is given. */
int fdms_rmsnorm(const void* in, int64_t in_stride, int64_t in_head_stride, int heads, const void* residual,
                 const void* weight, void* out, int64_t out_stride, void* residual_out, int64_t rows, int hidden,
                 float eps, float* amax_out, void* q_out, int64_t q_stride, int q_mode, void* stream);

/* out = silu(x[:, :F]) * x[:, F:], bf16 (fastdms/layers/activation.py:8-11). */
int fdms_silu_mul(const void* x, void* out, int64_t rows, int f, void* stream);

/* (f)2 — FP8 embedding gather: out[i, :] = bf16(e4m3fn(table[ids[i], :]) *
 * bf16(scale_inv[ids[i]])), bf16 output [n, dim] (fastdms/layers/embed_head.py:
 * 422-432, the table shared with or quantised like the FP8 LM head,
 * 379-402).  ids int64 on the device; an id outside [0, vocab) gives a NaN
 * row.  dim % 8 == 0, table rows 8-byte aligned, out 16-byte aligned. */
int fdms_embedding_fp8(const int64_t* ids, int64_t n, const void* table, int64_t table_stride, const float* scale_inv,
                       int64_t vocab, void* out, int64_t out_stride, int dim, void* stream);

/* (f)2 / B9 — the decode step's bf16 embedding gather and its first RMSNorm in
 * one launch (F.embedding, fastdms/layers/embed_head.py:87-104, then the first
 * decoder layer's input_layernorm without residual, layernorm.py:16-28):
 * rows_out[i, :] = table[ids[i], :] (the first residual, contiguous rows:
 * rows_stride == hidden) and out[i, :] = RMSNorm(rows_out[i, :]) with
 * `weight` / `eps`, bit-identical to fdms_rmsnorm of the gathered rows.  An id
 * outside [0, vocab) gives NaN rows in both.  hidden % 8 == 0, 16-byte
 * aligned rows. */
int fdms_embedding_rmsnorm(const int64_t* ids, int64_t n, const void* table, int64_t table_stride, int64_t vocab,
                           const void* weight, float eps, void* out, int64_t out_stride, void* rows_out,
                           int64_t rows_stride, int hidden, void* stream);

/* RMSNorm (+ residual) whose input row r is bf16(sum over s < k_splits of
 * partials[s * split_stride + r * hidden + c]) in split order: the merge of a
 * split-K fdms_linear_small_m (epilogue 3) done by its consumer, as the
 * reference's RMSNorm(down_proj / o_proj output, residual) sequence
 * (layernorm.py:19-40; llama.py:248-266).  For an FP8 linear, row_scale [rows]
 * (its row_scale_out) and col_scale [hidden] (the weight's scale_inv) make the
 * input bf16((sum * row_scale[r]) * col_scale[c]), the linear's own
 * finalisation (either may be null: factor 1).  amax_out, q_out as
 * fdms_rmsnorm.
 * partials and col_scale 32-byte aligned, split_stride a multiple of 8;
 * residual / residual_out contiguous rows. */
int fdms_rmsnorm_partials(const float* partials, int k_splits, int64_t split_stride, const void* residual,
                          const void* weight, void* out, int64_t out_stride, void* residual_out, int64_t rows,
                          int hidden, float eps, const float* row_scale, const float* col_scale, float* amax_out,
                          void* q_out, int64_t q_stride, int q_mode, void* stream);

/* Row argmax, ties to the lowest index (fastdms/layers/embed_head.py:142, 160,
 * and the torch argmax of ParallelLMHead.greedy_token_ids, 491-543). */
int fdms_argmax_rows(const void* x, int dtype, int64_t stride, int64_t rows, int n, int64_t* out, void* stream);

/* C1 — per-row FP8 quantisation.  Replaces LinearBase.quantize_weight_to_fp8 /
 * _amax_to_scale (fastdms/layers/linear.py:386-388, 813-823) for weight rows
 * [N, K] and the per-row dynamic activation quantisation of the FP8 paths
 * (514-523, 683-694, 652-654): s = 448/amax(row) (1 if zero), out = e4m3fn(v*s)
 * (RNE), scale_inv[row] = 1/s.  in_dtype bf16 or f32.  torch_form = 1 rounds
 * 448/amax the way the reference's torch expressions evaluate it
 * (reciprocal(amax) * 448: weights, _fp8_linear); 0 divides directly (its
 * Triton kernels). */
int fdms_quantize_fp8_rows(const void* in, int in_dtype, int64_t in_stride, int64_t rows, int k, void* out,
                           int64_t out_stride, float* scale_inv, int torch_form, void* stream);

/* C2 / C3 / C6 (decode rows) — y[m,n] = a[m,:] . W[n,:] for m <= 16 rows.
 * Replaces _fp8_row1_matvec(_dot)_kernel and _fp8_small_m_linear_kernel
 * (linear.py:492-632, 665-763) for w_dtype FP8 (W row-major [N, K] = the
 * reference's column-major W8^T [K, N], per-row scale_inv [N]; quantize_x = the
 * per-row dynamic activation quantisation: 1 = 448/amax divided directly as its
 * Triton kernels do, 2 = reciprocal(amax) * 448 as _fp8_linear's torch
 * expression (635-662, the torch._scaled_mm path at rows <= 16), 0 = none;
 * y = bf16(acc/x_s*scale_inv), bias added in bf16), and the
 * BF16 F.linear of the decode step (linear.py:926; y = bf16(acc + bias)) for
 * w_dtype bf16.  prologue 1 = RMSNorm of x (+ residual, fp32 sum; the bf16 sum
 * goes to residual_out, written by one workgroup; layernorm.py:19-40).
 * epilogue 1 = W is [gate; up] (n rows), the output has n/2 columns
 * bf16(silu(gate) * up) (activation.py:8-11).  epilogue 3 (no bias, no
 * prologue) = no merge: split s writes its fp32 partial sums (before the FP8
 * scales) to workspace[(s * m + row) * n + col] and y is not written; the
 * consumer (fdms_rmsnorm_partials) adds the splits in order and applies
 * row_scale_out[row] (written here when given: 1/x_s, or 1 without activation
 * quantisation) and the weight's scale_inv.  x_amax (optional, prologue 0 with
 * quantize_x): row r's amax is the max of x_amax[r * x_amax_stride + p], p <
 * x_amax_n, supplied by x's producer (fdms_rmsnorm's amax_out, or this
 * function's amax_out) in place of the pass over x; the result is the same
 * (the amax must propagate NaN, as torch's does).  x_dtype FP8 (FP8 weights,
 * quantize_x 1 / 2, x_amax required): x holds the e4m3fn codes of the
 * quantised activation (fdms_rmsnorm's q_out, same quantize_x form), row
 * stride x_stride bytes.  amax_out (optional, epilogues 0 / 1) = per-strip max
 * |y|: amax_out[row * (n_out/16) + strip].  epilogue 4 (prologue 0, no
 * activation quantisation) = the residual add of the RMSNorm that follows
 * (layernorm.py:32-40): with v the finished bf16 output, y receives f =
 * fp32(v) + fp32(residual) as fp32 rows (y_stride in floats, 16-byte aligned),
 * residual_out = bf16(f) (it may be residual itself: updated in place), and
 * amax_out[row * (n/16) + strip] = the strip's sum of f^2.  prologue 2 (x_dtype
 * F32, quantize_x 0, epilogues 0 / 1) = that RMSNorm applied as x is loaded:
 * x holds f (fp32 rows, x_stride in floats), x_amax [m, x_amax_n = k/16] the
 * producer strips' sums of f^2 (x_amax_stride per row), norm_weight the norm's weight;
 * a = bf16(bf16(f * rsqrt(sum / k + eps)) * norm_weight).  k_splits > 1 splits K over
 * workgroups: workspace holds (n_out/16) * k_splits * 256 floats (x2 for
 * epilogue 1) and counters n_out/16 ints, zero before the first call and left
 * zero.  k / k_splits a multiple of 256, n_out of 16, 16-byte aligned rows; y
 * and residual_out must not alias x / residual (except epilogue 4's in-place
 * residual). */
int fdms_linear_small_m(const void* x, int64_t x_stride, int m, int k, const void* w, int w_dtype,
                        int64_t w_stride, const float* w_scale_inv, const void* bias, int n, int prologue,
                        const void* norm_weight, float eps, const void* residual, int64_t res_stride,
                        void* residual_out, int64_t res_out_stride, int quantize_x, int epilogue, int k_splits,
                        float* workspace, int* counters, void* y, int64_t y_stride, const float* x_amax,
                        int x_amax_n, int64_t x_amax_stride, float* amax_out, float* row_scale_out, int x_dtype,
                        void* stream);

/* C7 — greedy LM head: token[m] = argmax_n a[m,:] . W[n,:] for m <= 16 rows,
 * ties to the lowest index, NaN first (torch.argmax order).  Replaces
 * _fp8_row1_argmax_stage/reduce + _fp8_row1_argmax (fastdms/layers/embed_head.py:
 * 96-211; FP8 weights, per-row quantised activation, scores in fp32:
 * bf16_scores = 0) and greedy_token_ids' forward + argmax (491-598; bf16
 * logits: bf16_scores = 1, with FP8 weights the _fp8_linear scores rounded to
 * bf16).  One GEMV launch writes each strip's best (part_val / part_idx,
 * m * n/16 each), a second reduces them into out_tokens (int64).  Other
 * arguments as fdms_linear_small_m. */
int fdms_linear_argmax_small_m(const void* x, int64_t x_stride, int m, int k, const void* w, int w_dtype,
                               int64_t w_stride, const float* w_scale_inv, const void* bias, int n, int quantize_x,
                               int bf16_scores, int k_splits, float* workspace, int* counters, float* part_val,
                               int* part_idx, int64_t* out_tokens, void* stream);

/* C7 — FP8 re-ranking of the INT4 head's candidates.  Replaces
 * _fp8_row1_rerank_topk_kernel / _fp8_row1_rerank_topk (fastdms/layers/
 * embed_head.py:214-302): per row, score the candidate ids [rows, topk] (int64,
 * topk in {2, 4, 8, 16, 32}) with the FP8 rows (448/amax activation
 * quantisation, fp32 scores) and write the best id, the lowest on ties; ids
 * outside [0, n) score -inf.  k % 16 == 0, 16-byte aligned rows. */
int fdms_fp8_rerank_topk(const void* x, int64_t x_stride, int rows, int k, const void* w_fp8, int64_t w_stride,
                         const float* w_scale_inv, int n, const int64_t* candidates, int topk, int64_t* out_tokens,
                         void* stream);

/* C5 — W4A16 decode linear.  Replaces _int4_row1_matvec /
 * torch._weight_int4pack_mm (fastdms/layers/linear.py:462-478): y[m,n] =
 * x[m,:] . bf16((q[n,:] - 8) * scale + zero) with per-group bf16 scale / zero
 * in the reference's scale_zeros layout (linear.py:461-464): bf16 [k/group_size,
 * sz_stride >= n, 2], element (g, n, 0) the scale and (g, n, 1) the zero of
 * group g of weight row n (4-byte aligned).  The weight packing is this
 * library's own: w_packed[n, j] holds q[n, 2j] (low nibble) and q[n, 2j+1]
 * (high nibble).  epilogue 0 = bf16(acc + bias) into y, 1 = SiLU*up of [gate;
 * up] rows (as fdms_linear_small_m), 2 = greedy argmax into out_tokens (as
 * fdms_linear_argmax_small_m), 3 = fp32 split partials workspace[split][row][n]
 * (no bias; as fdms_linear_small_m's epilogue 3, summed by
 * fdms_rmsnorm_partials).  m <= 16. */
int fdms_linear_int4_small_m(const void* x, int64_t x_stride, int m, int k, const void* w_packed,
                             int64_t w_stride_bytes, const void* scale_zeros, int group_size, int64_t sz_stride,
                             const void* bias, int n, int epilogue, int k_splits, float* workspace, int* counters,
                             float* part_val, int* part_idx, int64_t* out_tokens, void* y, int64_t y_stride,
                             void* stream);

/* C5 — INT4 group quantisation of weight rows (linear.py:414-459, symmetric or
 * asymmetric); q is computed with the fp32 scale / zero, which are stored in
 * bf16 (456-458) as the reference's scale_zeros [k/group_size, sz_stride >=
 * rows, 2] (461-464).  Output packed as fdms_linear_int4_small_m reads it. */
int fdms_quantize_int4_groups(const void* w, int w_dtype, int64_t w_stride, int64_t rows, int k, int group_size,
                              int asymmetric, void* out_packed, int64_t out_stride, void* scale_zeros,
                              int64_t sz_stride, void* stream);

/* Paged compact KV (16-row pages from a device free stack per layer; no
 * reference counterpart: the reference packs into flat spans from a host
 * first-fit allocator, compact_kv.py:830-857, 955-1099).  Prefill side, one
 * layer: fdms_streaming_pack_prepare plus the page pop of every (seq, head):
 * ceil(live / 16) ids from page_stack[page_top - n .. page_top) (one atomic pop
 * per span) into block_table[row, h, 0 .. n) (other entries -1), n into
 * pages_held[row, h].  page_budget (required, one int of device memory, at
 * most *page_top): the launch's pops debit it first and fail when it is
 * short, which keeps pages on the stack for other sequences.  A span whose
 * pages do not fit gets none and live_out 0, and *overflow is raised to 1
 * (the caller frees the batch's spans and retries it later); 2 means the stack
 * was shorter than a debit that fitted (page_budget > *page_top: the pool
 * state is no longer valid).  Budget debits and stack pops are single atomic
 * subtracts, never retried: concurrent spans do not serialise. */
int fdms_paged_pack_prepare(const uint8_t* evict, int64_t es_t, int64_t es_h, const int32_t* cu_seqlens,
                            int num_seqs, int window, int num_kv_heads, int max_chunks, int32_t* live_out,
                            int64_t lo_b, int64_t lo_h, int32_t* block_offsets, int64_t of_b, int64_t of_h,
                            int64_t of_c, int32_t* positions, uint8_t* evict_meta, const int32_t* meta_rows,
                            int64_t tp_b, int64_t tp_h, int64_t em_b, int64_t em_h, int meta_cap,
                            int32_t* page_stack, int32_t* page_top, int32_t* page_budget, int32_t* block_table,
                            int64_t bt_b, int64_t bt_h, int32_t* pages_held, int64_t hd_b, int64_t hd_h,
                            int max_pages, int32_t* overflow, void* stream);

/* Paged prefill scatter: fdms_streaming_pack_rank_scatter with rank r of (seq,
 * head) stored at row block_table[row, h, r >> 4] * 16 + (r & 15). */
int fdms_paged_pack_scatter(const void* k, const void* v, int kv_dtype, int64_t ks_t, int64_t ks_h, int64_t vs_t,
                            int64_t vs_h, const uint8_t* evict, int64_t es_t, int64_t es_h,
                            const int32_t* cu_seqlens, int num_seqs, const int32_t* block_offsets, int64_t bo_b,
                            int64_t bo_h, int64_t bo_c, void* compact_k, void* compact_v, int compact_dtype,
                            int64_t cs_s, int32_t* positions, uint8_t* evict_meta, const int32_t* meta_rows,
                            int64_t tp_b, int64_t tp_h, int64_t tp_s, int64_t em_b, int64_t em_h, int64_t em_s,
                            const int32_t* block_table, int64_t bt_b, int64_t bt_h, int window, int num_kv_heads,
                            int head_dim, int max_chunks, int vec, const float* k_scale, const float* v_scale,
                            void* stream);

/* Paged decode append slots, all layers: when a span's pages are full (live ==
 * 16 * held) one page is popped from its layer's stack (page_stack[l *
 * stack_stride ...], page_top[l]) into the next table entry; then slot =
 * physical row of rank live and live += 1 (prepare_decode_metadata,
 * compact_kv.py:1727-1770, on pages).  A short pool gives slot -1 and sets
 * *overflow. */
int fdms_paged_prepare_decode(int32_t* live, int64_t l_l, int64_t l_b, int64_t l_h, int32_t* slot_out, int64_t s_l,
                              int64_t s_b, int64_t s_h, int32_t* block_table, int64_t bt_l, int64_t bt_b,
                              int64_t bt_h, int32_t* pages_held, int64_t hd_l, int64_t hd_b, int64_t hd_h,
                              const int32_t* page_stack, int64_t stack_stride, int32_t* page_top, int max_pages,
                              int32_t* overflow, int num_layers, int num_seqs, int num_kv_heads, void* stream);

/* Paged sequence free: every page of the spans of rows[0 .. num_rows) (all
 * layers and kv heads) back to its layer's stack; tables -1, held and live 0
 * (the reference frees host ranges, compact_kv.py:1772-1795). */
int fdms_paged_free(const int32_t* rows, int num_rows, int32_t* block_table, int64_t bt_l, int64_t bt_b,
                    int64_t bt_h, int32_t* pages_held, int64_t hd_l, int64_t hd_b, int64_t hd_h, int32_t* live,
                    int64_t l_l, int64_t l_b, int64_t l_h, int32_t* page_stack, int64_t stack_stride,
                    int32_t* page_top, int num_layers, int num_kv_heads, void* stream);

/* Paged decode expiry (A12 / A13 on pages): fdms_dms_expiry's re-compaction
 * with span slot r at row block_table[l, s, h, r >> 4] * 16 + (r & 15); each
 * span then keeps ceil(live / 16) pages and returns the rest to its layer's
 * stack. */
int fdms_paged_expiry(int incremental, int32_t* positions, int64_t ps_l, int64_t ps_s, int64_t ps_h, uint8_t* evict,
                      int64_t es_l, int64_t es_s, int64_t es_h, int32_t* live_counts, int64_t lc_l, int64_t lc_s,
                      int64_t lc_h, int32_t* block_table, int64_t bt_l, int64_t bt_s, int64_t bt_h,
                      int32_t* pages_held, int64_t hd_l, int64_t hd_s, int64_t hd_h, int32_t* page_stack,
                      int64_t stack_stride, int32_t* page_top, const uint64_t* layer_k, const uint64_t* layer_v,
                      int64_t row_bytes, int64_t c_s_bytes, const int64_t* current_positions, int num_layers,
                      int num_seqs, int num_kv_heads, int window, void* stream);

/* Paged fused decode attention: fdms_fused_decode_attention with rank r of (b,
 * h) at row block_tables[b, h, r / page_size] * page_size + r % page_size
 * (no base offsets); slot_mapping holds the appended token's row. */
int fdms_fused_decode_attention_paged(const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b,
                                      int64_t ks_h, const void* v, int64_t vs_b, int64_t vs_h, const float* cos_sin,
                                      int64_t cs_p, int64_t cs_d, const int64_t* positions,
                                      const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, uint8_t* evict_out,
                                      int64_t ev_b, int64_t ev_h, float alpha_scale, float alpha_offset,
                                      float threshold, int positive_scale, void* compact_k, void* compact_v,
                                      int64_t c_s, const int32_t* block_tables, int64_t bt_b, int64_t bt_h,
                                      int page_size, const int32_t* live_counts, int64_t lc_b, int64_t lc_h,
                                      void* out, int64_t os_b, int64_t os_h, float* workspace, int* counters,
                                      int batch, int num_kv_heads, int group_size, int head_dim, int num_splits,
                                      int split_rows, float scale, const float* k_scale, const float* v_scale,
                                      const void* q_norm, const void* k_norm, float norm_eps, void* stream);

/* The decode step's attention work plan (no reference counterpart): the
 * append rows of fdms_paged_prepare_decode (one workgroup per layer: the
 * layer's page pops take stack entries top-1, top-2, ... in (seq, head)
 * order, no atomics), then per layer one work item for every live workgroup
 * of that layer's fdms_fused_decode_attention_planned launch.  Layer l's
 * block starts at plan + l * plan_l: 4 ints (the last one: the number of
 * further splits), then the items, 72 int32 each: split 0 of pair p at item
 * p, the pairs' further splits packed after the pairs in (pair, split)
 * order.  A pair of live ranks (after the append) takes ns = 1 split if live
 * <= split_rows, else min(num_splits, ceil(live / heavy_rows)), of
 * ceil(live / ns) ranks rounded up to 64 (the unplanned launch's
 * partition).  An item holds pair, first rank, end rank (the appended rank
 * left out), split | (ns << 16), live, append row, position, flags (bit 0:
 * the item holds the appended rank), then the page id of each of its 16-rank
 * quarters (up to 64).  split_rows and heavy_rows multiples of 64,
 * heavy_rows <= split_rows <= 1024; plan 16-byte aligned, plan_l a multiple
 * of 4 and >= 4 + num_splits * num_seqs * num_kv_heads * 72; num_seqs *
 * num_kv_heads <= 8192. */
int fdms_paged_prepare_decode_plan(int32_t* live, int64_t l_l, int64_t l_b, int64_t l_h, int32_t* slot_out,
                                   int64_t s_l, int64_t s_b, int64_t s_h, int32_t* block_table, int64_t bt_l,
                                   int64_t bt_b, int64_t bt_h, int32_t* pages_held, int64_t hd_l, int64_t hd_b,
                                   int64_t hd_h, const int32_t* page_stack, int64_t stack_stride, int32_t* page_top,
                                   int max_pages, int32_t* overflow, const int64_t* positions, int32_t* plan,
                                   int64_t plan_l, int split_rows, int heavy_rows, int num_splits, int num_layers,
                                   int num_seqs, int num_kv_heads, void* stream);

/* A9 + B2-B5 on the step's plan (no reference counterpart as a launch form;
 * the computation is fdms_fused_decode_attention_paged's, i.e. the
 * reference's fused_dms_rope_store_compact_decode + compact_decode_attention,
 * compact_attention.py:67-209, 1010-1336): one layer, plan = that layer's
 * items from fdms_paged_prepare_decode_plan (its block + 4 ints: the count of
 * further splits is plan[-1]), positions the step's int64 positions.  The
 * grid holds num_splits x pairs workgroups of 8 waves: workgroup p < pairs
 * runs split 0 of pair p and loads the pair's raw rows and position with
 * its item; a later one runs a further split named by its item, or exits
 * past the layer's count; then its K/V rows (two 64-row groups per wave at
 * most, their page ids from the item).  The workspace holds batch * num_kv_heads *
 * num_splits * group_size * (head_dim + 2) floats and counters batch *
 * num_kv_heads zeros.  Planned with the unplanned launch's partition, the
 * decisions, appended rows and outputs are that launch's, bit for bit. */
int fdms_fused_decode_attention_planned(const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b,
                                        int64_t ks_h, const void* v, int64_t vs_b, int64_t vs_h,
                                        const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
                                        const int32_t* plan, uint8_t* evict_out, int64_t ev_b, int64_t ev_h,
                                        float alpha_scale, float alpha_offset, float threshold, int positive_scale,
                                        void* compact_k, void* compact_v, int64_t c_s, void* out, int64_t os_b,
                                        int64_t os_h, float* workspace, int* counters, int batch, int num_kv_heads,
                                        int group_size, int head_dim, int num_splits, float scale,
                                        const float* k_scale, const float* v_scale, const void* q_norm,
                                        const void* k_norm, float norm_eps, void* stream);

/* FP8 GEMM for prefill row counts (replaces the torch._scaled_mm call of
 * _fp8_linear, linear.py:635-662): y[m, n] = bf16((sum_k x[m, k] * w[n, k]) *
 * x_inv[m] * w_inv[n]), then bf16(y + bias[n]) when bias is not NULL.  x [M, K]
 * and w [N, K] e4m3fn rows with byte strides x_s / w_s (K, strides and
 * pointers multiples of 16); x_inv [M], w_inv [N] fp32; y [M, N] bf16 with row
 * stride y_s elements.  Runs on the FP8 matrix cores (fp32 accumulation). */
int fdms_fp8_gemm(const void* x, int64_t x_s, const float* x_inv, const void* w, int64_t w_s, const float* w_inv,
                  const void* bias, void* y, int64_t y_s, int M, int N, int K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTDMS_AMD_H */
