// Compact-KV GQA decode attention (reference: fastdms/layers/compact_attention.py
// split-K partial 334-415, reduce 537-603, wrapper 1116-1336, torch reference
// 1339-1364).
//
// out[b, h*G+g] = softmax(K_span . q * scale) . V_span over the live slots of
// (b, kv head h).  A slot r of a span is addressed either flat
// (base_offsets[b,h] + r, the reference layout) or paged
// (block_table[b,h,r >> log2 P] * P + (r & (P-1))).
//
// Work split: grid = (num_splits, B*Hkv).  Each (b,h) divides its *own* live
// count evenly over the splits, so no workgroup scans the padded capacity the
// reference launches over (cdiv(max_capacity, 256) splits).  Split partials
// (max, sum, acc) go to a workspace; the last workgroup of a (b,h) to finish
// (device-scope atomic ticket) merges them and writes the output, then resets
// its ticket to 0 so the next call (or graph replay) starts clean.  Softmax is
// computed in the log2 domain (q pre-scaled by scale*log2 e, exp2).
#include "fdms_common.h"

using namespace fdms;

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 256;
constexpr int kMaxG = 8;
constexpr int kMaxD = 256;
constexpr float kLog2e = 1.4426950408889634f;

struct SpanAddr {
  const int32_t* base;
  const int32_t* table;
  int64_t tb_b, tb_h;
  int page_shift;
  int paged;
  __device__ __forceinline__ int64_t row(int b, int h, int64_t bo, int r) const {
    if (paged) {
      const int32_t page = table[b * tb_b + h * tb_h + (r >> page_shift)];
      return ((int64_t)page << page_shift) + (r & ((1 << page_shift) - 1));
    }
    return bo + r;
  }
};

}  // namespace

template <typename QT, typename KT>
__global__ __launch_bounds__(kThreads) void decode_attn_generic_kernel(
    const QT* __restrict__ q, int64_t qs_b, int64_t qs_h, const KT* __restrict__ ck, const KT* __restrict__ cv,
    int64_t c_s, const int32_t* __restrict__ base_offsets, int64_t bo_b, int64_t bo_h,
    const int32_t* __restrict__ block_tables, int64_t bt_b, int64_t bt_h, int page_shift, int paged,
    const int32_t* __restrict__ live_counts, int64_t lc_b, int64_t lc_h, QT* __restrict__ out, int64_t os_b,
    int64_t os_h, float* __restrict__ ws, int* __restrict__ counters, int num_kv_heads, int group_size,
    int head_dim, int num_splits, float scale, const float* __restrict__ rope_cs, int64_t rcs_p, int64_t rcs_d,
    const int64_t* __restrict__ rope_pos) {
  __shared__ float s_q[kMaxG][kMaxD];
  __shared__ float s_p[kMaxG][kTile];
  __shared__ int64_t s_row[kTile];
  __shared__ float s_m[kMaxG], s_l[kMaxG], s_alpha[kMaxG];
  __shared__ int s_last;

  const int pair = blockIdx.y;
  const int split = blockIdx.x;
  const int b = pair / num_kv_heads;
  const int h = pair - b * num_kv_heads;
  const int tid = threadIdx.x;
  const int G = group_size;
  const int D = head_dim;
  const int live = live_counts[b * lc_b + h * lc_h];
  const int per = (live + num_splits - 1) / num_splits;
  const int t0 = min(live, split * per);
  const int t1 = min(live, t0 + per);
  const int64_t bo = paged ? 0 : (int64_t)base_offsets[b * bo_b + h * bo_h];
  const SpanAddr addr{base_offsets, block_tables, bt_b, bt_h, page_shift, paged};
  const float qscale = scale * kLog2e;

  if (rope_pos) {
    // inline q RoPE with the decision lane (g=0, d=D-1) zeroed
    // (compact_attention.py:454-488); rotated q stays fp32.
    const int half = D / 2;
    const int64_t pos = rope_pos[b];
    for (int i = tid; i < kMaxG * half; i += kThreads) {
      const int g = i / half, j = i - g * half;
      float y1 = 0.0f, y2 = 0.0f;
      if (g < G) {
        const QT* qh = q + b * qs_b + (int64_t)(h * G + g) * qs_h;
        const float x1 = ld<QT>(qh + j);
        const float x2 = (g == 0 && j == half - 1) ? 0.0f : ld<QT>(qh + j + half);
        const float c = rope_cs[pos * rcs_p + (int64_t)j * rcs_d];
        const float sn = rope_cs[pos * rcs_p + (int64_t)(j + half) * rcs_d];
        rope_f32(x1, x2, c, sn, &y1, &y2);
      }
      s_q[g][j] = y1 * qscale;
      s_q[g][j + half] = y2 * qscale;
    }
  } else {
    for (int i = tid; i < kMaxG * D; i += kThreads) {
      const int g = i / D, d = i - g * D;
      s_q[g][d] = (g < G) ? ld<QT>(q + b * qs_b + (int64_t)(h * G + g) * qs_h + d) * qscale : 0.0f;
    }
  }
  if (tid < kMaxG) {
    s_m[tid] = -INFINITY;
    s_l[tid] = 0.0f;
  }
  const int n_out = G * D;
  float acc[kMaxG];
#pragma unroll
  for (int k = 0; k < kMaxG; ++k) acc[k] = 0.0f;
  __syncthreads();

  for (int tile = t0; tile < t1; tile += kTile) {
    const int n = min(kTile, t1 - tile);
    // scores: one token per thread
    {
      const int i = tid;
      float s[kMaxG];
#pragma unroll
      for (int g = 0; g < kMaxG; ++g) s[g] = 0.0f;
      if (i < n) {
        const int64_t row = addr.row(b, h, bo, tile + i);
        s_row[i] = row;
        const KT* kr = ck + row * c_s;
        for (int d = 0; d < D; ++d) {
          const float kd = ld<KT>(kr + d);
#pragma unroll
          for (int g = 0; g < kMaxG; ++g) s[g] += s_q[g][d] * kd;
        }
      }
#pragma unroll
      for (int g = 0; g < kMaxG; ++g) s_p[g][i] = (i < n) ? s[g] : -INFINITY;
    }
    __syncthreads();
    // per-head tile max / exp / sum: wave w owns heads w and w+4
    {
      const int w = tid >> 6, lane = tid & 63;
      for (int g = w; g < G; g += kThreads / kWave) {
        float mx = -INFINITY;
        for (int i = lane; i < n; i += kWave) mx = fmaxf(mx, s_p[g][i]);
        mx = wave_max(mx);
        const float m_old = s_m[g];
        const float m_new = fmaxf(m_old, mx);
        float sum = 0.0f;
        for (int i = lane; i < n; i += kWave) {
          const float p = exp2f(s_p[g][i] - m_new);
          s_p[g][i] = p;
          sum += p;
        }
        sum = wave_sum(sum);
        if (lane == 0) {
          const float alpha = exp2f(m_old - m_new);
          s_alpha[g] = alpha;
          s_l[g] = s_l[g] * alpha + sum;
          s_m[g] = m_new;
        }
      }
    }
    __syncthreads();
    // acc[g][d] = acc*alpha + sum_i p[g][i] * V[row_i][d]
#pragma unroll
    for (int k = 0; k < kMaxG; ++k) {
      const int o = tid + k * kThreads;
      if (o < n_out) {
        const int g = o / D, d = o - g * D;
        float a = acc[k] * s_alpha[g];
        for (int i = 0; i < n; ++i) a += s_p[g][i] * ld<KT>(cv + s_row[i] * c_s + d);
        acc[k] = a;
      }
    }
    __syncthreads();
  }

  if (num_splits == 1) {
#pragma unroll
    for (int k = 0; k < kMaxG; ++k) {
      const int o = tid + k * kThreads;
      if (o < n_out) {
        const int g = o / D, d = o - g * D;
        st<QT>(out + b * os_b + (int64_t)(h * G + g) * os_h + d, acc[k] / s_l[g]);
      }
    }
    return;
  }

  const int64_t stride = (int64_t)G * (D + 2);
  float* mine = ws + ((int64_t)pair * num_splits + split) * stride;
  if (tid < G) {
    mine[tid] = s_m[tid];
    mine[G + tid] = s_l[tid];
  }
#pragma unroll
  for (int k = 0; k < kMaxG; ++k) {
    const int o = tid + k * kThreads;
    if (o < n_out) mine[2 * G + o] = acc[k];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = (atomicAdd(&counters[pair], 1) == num_splits - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* all = ws + (int64_t)pair * num_splits * stride;
#pragma unroll
  for (int k = 0; k < kMaxG; ++k) {
    const int o = tid + k * kThreads;
    if (o < n_out) {
      const int g = o / D;
      float M = -INFINITY;
      for (int s = 0; s < num_splits; ++s) M = fmaxf(M, (all + s * stride + g)[0]);
      float L = 0.0f, A = 0.0f;
      for (int s = 0; s < num_splits; ++s) {
        const float* ps = all + s * stride;
        const float ms = (ps + g)[0];
        const float wgt = (ms == -INFINITY) ? 0.0f : exp2f(ms - M);
        L += (ps + G + g)[0] * wgt;
        A += (ps + 2 * G + o)[0] * wgt;
      }
      const int d = o - g * D;
      st<QT>(out + b * os_b + (int64_t)(h * G + g) * os_h + d, A / L);
    }
  }
  if (tid == 0) counters[pair] = 0;
}

FDMS_EXPORT int fdms_compact_decode_attention(
    const void* q, int q_dtype, int64_t qs_b, int64_t qs_h, const void* compact_k, const void* compact_v,
    int kv_dtype, int64_t c_s, const int32_t* base_offsets, int64_t bo_b, int64_t bo_h, const int32_t* block_tables,
    int64_t bt_b, int64_t bt_h, int page_size, const int32_t* live_counts, int64_t lc_b, int64_t lc_h, void* out,
    int64_t os_b, int64_t os_h, float* workspace, int* counters, int batch, int num_kv_heads, int group_size,
    int head_dim, int num_splits, float scale, const float* rope_cos_sin, int64_t rcs_p, int64_t rcs_d,
    const int64_t* rope_positions, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || group_size <= 0 || group_size > kMaxG) return (int)hipErrorInvalidValue;
  if (head_dim <= 0 || head_dim > kMaxD || num_splits <= 0 || num_splits > 65535) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  if (!q || !compact_k || !compact_v || !live_counts || !out) return (int)hipErrorInvalidValue;
  int paged = 0, page_shift = 0;
  if (block_tables) {
    if (page_size <= 0 || (page_size & (page_size - 1))) return (int)hipErrorInvalidValue;
    paged = 1;
    while ((1 << page_shift) < page_size) ++page_shift;
  } else if (!base_offsets) {
    return (int)hipErrorInvalidValue;
  }
  if (num_splits > 1 && (!workspace || !counters)) return (int)hipErrorInvalidValue;
  if (rope_positions && (!rope_cos_sin || head_dim % 2)) return (int)hipErrorInvalidValue;
  const int pairs = batch * num_kv_heads;
  if (pairs > 65535) return (int)hipErrorInvalidValue;
  const dim3 grid(num_splits, pairs);
  FDMS_DISPATCH_FLOAT(q_dtype, QT,
    FDMS_DISPATCH_DTYPE(kv_dtype, KT,
      hipLaunchKernelGGL((decode_attn_generic_kernel<QT, KT>), grid, dim3(kThreads), 0, (hipStream_t)stream,
                         (const QT*)q, qs_b, qs_h, (const KT*)compact_k, (const KT*)compact_v, c_s, base_offsets,
                         bo_b, bo_h, block_tables, bt_b, bt_h, page_shift, paged, live_counts, lc_b, lc_h, (QT*)out,
                         os_b, os_h, workspace, counters, num_kv_heads, group_size, head_dim, num_splits, scale,
                         rope_cos_sin, rcs_p, rcs_d, rope_positions)));
  FDMS_LAUNCH_CHECK();
  return 0;
}
