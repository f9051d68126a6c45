// Element-wise model ops around the DMS path, fused so a decode layer issues
// few launches: residual-add + RMSNorm (reference layernorm.py:16-40) and
// SiLU(gate) * up (activation.py:8-11).  bf16 in/out, fp32 math; one block
// per row, 16-byte vector loads.  HBM-bound: 2-3 bf16 reads + 2 writes per
// element.
#include "fdms_vec.h"

using namespace fdms;

namespace {
constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum(float v, float* s_red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[w] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) t += s_red[i];
  __syncthreads();
  return t;
}
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, float* s_red) {
  v = wave_max_u32(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[w] = __uint_as_float(v);
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) t = max(t, __float_as_uint(s_red[i]));
  __syncthreads();
  return t;
}
}  // namespace

// x_out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w), where x = in (+ residual
// in fp32, and residual_out = bf16(x)) — layernorm.py:19-40.
// PART: the input is the fp32 split-K partial sums of the preceding linear,
// part[s * split_stride + row * hidden + c], s < k_splits, and x = bf16 of
// their sum taken in split order (the linear kernel's own merge).
// PART: the input is the fp32 split-K partials; KS > 0 is their count known
// at compile time, KS = 0 reads k_splits at run time.  With row_scale /
// col_scale (an FP8 linear's 1/x_s[row] and weight scale_inv[c]) the input is
// x = bf16(sum * row_scale[row] * col_scale[c]), the linear's own finalisation.
// amax_out[row] (optional) = max |out[row, :]| (NaN if the row holds one), the
// statistic the next FP8 linear's activation quantisation needs; q_out
// (optional, with amax_out) receives that quantisation itself, e4m3fn(out *
// s) with s = 448 / amax (q_mode 2: the torch rounding), and out may then be
// null.  PER = 8-column chunks
// per thread (hidden <= PER * 8 * kThreads).  Every load of the row goes out
// before the first use, with addresses clamped in bounds instead of loads
// under a condition (a conditional load makes the compiler wait for it at
// the end of its block, one memory round trip per load).
template <bool PART, int KS, int PER>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const bf16_t* __restrict__ in, const bf16_t* residual,
                                                           const bf16_t* __restrict__ weight, bf16_t* __restrict__ out,
                                                           bf16_t* residual_out, int hidden, int64_t in_stride,
                                                           int64_t in_head_stride, int heads, int64_t out_stride,
                                                           float eps, const float* __restrict__ part, int k_splits,
                                                           int64_t split_stride, const float* __restrict__ row_scale,
                                                           const float* __restrict__ col_scale,
                                                           float* __restrict__ amax_out, uint8_t* __restrict__ q_out,
                                                           int64_t q_stride, int q_mode,
                                                           const int64_t* __restrict__ ids, int64_t vocab) {
  __shared__ float s_red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  // ids (optional, embedding rows): input row r is table row ids[r] (in_stride
  // per row); an id outside [0, vocab) reads row 0 and yields NaN rows
  const int64_t id = ids ? ids[row] : 0;
  const bool id_ok = !ids || (id >= 0 && id < vocab);
  const bf16_t* x = PART ? nullptr
                         : ids ? in + (id_ok ? id : 0) * in_stride
                               : in + (row / heads) * in_stride + (row % heads) * in_head_stride;
  const bool has_res = residual != nullptr;  // uniform
  const bf16_t* rs = has_res ? residual + row * (int64_t)hidden : weight;  // a valid address either way
  constexpr int V = 8;
  constexpr int NS = KS > 0 ? KS : 1;
  Vec<bf16_t, V> wv[PER], xv[PER], rv[PER];
  Vec<float, V> pv[PER][NS], cs[PER];
  const float* csrc = (PART && col_scale) ? col_scale : part;  // a valid address either way (PART)
  const float rscale = (PART && row_scale) ? row_scale[row] : 1.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int cc = min(((int)threadIdx.x + j * kThreads) * V, hidden - V);  // int min (an unsigned operand picks the double overload)
    wv[j] = *reinterpret_cast<const Vec<bf16_t, V>*>(weight + cc);
    if constexpr (PART) cs[j] = *reinterpret_cast<const Vec<float, V>*>(csrc + cc);
    if constexpr (PART && KS > 0) {
#pragma unroll
      for (int sp = 0; sp < KS; ++sp)
        pv[j][sp] = *reinterpret_cast<const Vec<float, V>*>(part + sp * split_stride + row * hidden + cc);
    }
    if constexpr (!PART) xv[j] = *reinterpret_cast<const Vec<bf16_t, V>*>(x + cc);
    rv[j] = *reinterpret_cast<const Vec<bf16_t, V>*>(rs + cc);
  }
  float vals[PER][V];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = (threadIdx.x + j * kThreads) * V;
    const bool valid = c < hidden;
    float xf[V];
    if constexpr (PART) {
#pragma unroll
      for (int i = 0; i < V; ++i) xf[i] = 0.0f;
      if constexpr (KS > 0) {
#pragma unroll
        for (int sp = 0; sp < KS; ++sp)
#pragma unroll
          for (int i = 0; i < V; ++i) xf[i] += pv[j][sp].v[i];
      } else if (valid) {
        for (int sp = 0; sp < k_splits; ++sp) {
          const Vec<float, V> p = *reinterpret_cast<const Vec<float, V>*>(part + sp * split_stride + row * hidden + c);
#pragma unroll
          for (int i = 0; i < V; ++i) xf[i] += p.v[i];
        }
      }
      if (row_scale) {
#pragma unroll
        for (int i = 0; i < V; ++i) xf[i] *= rscale;
      }
      if (col_scale) {
#pragma unroll
        for (int i = 0; i < V; ++i) xf[i] *= cs[j].v[i];
      }
#pragma unroll
      for (int i = 0; i < V; ++i) xf[i] = bf16_to_f32(f32_to_bf16(xf[i]));
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) xf[i] = id_ok ? bf16_to_f32(xv[j].v[i].bits) : __builtin_nanf("");
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
      float f = xf[i];
      if (has_res) f += bf16_to_f32(rv[j].v[i].bits);
      vals[j][i] = f;
      ss += valid ? f * f : 0.0f;
    }
    if (residual_out && valid) {
      Vec<bf16_t, V> ro;
#pragma unroll
      for (int i = 0; i < V; ++i) ro.v[i].bits = (uint16_t)f32_to_bf16(vals[j][i]);
      *reinterpret_cast<Vec<bf16_t, V>*>(residual_out + row * (int64_t)hidden + c) = ro;
    }
  }
  const float total = block_sum(ss, s_red);
  const float inv = rsqrtf(total / (float)hidden + eps);  // torch.rsqrt (layernorm.py:24, 38)
  uint32_t amax = 0;
  float ov[PER][V];  // the bf16 outputs as fp32
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = (threadIdx.x + j * kThreads) * V;
    Vec<bf16_t, V> o;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float xn = bf16_to_f32(f32_to_bf16(vals[j][i] * inv));
      o.v[i].bits = (uint16_t)f32_to_bf16(xn * bf16_to_f32(wv[j].v[i].bits));
      ov[j][i] = bf16_to_f32(o.v[i].bits);
      if (c < hidden) amax = max(amax, abs_bits(ov[j][i]));
    }
    if (out && c < hidden) *reinterpret_cast<Vec<bf16_t, V>*>(out + row * out_stride + c) = o;
  }
  if (amax_out) {  // uniform
    amax = block_max_u32(amax, s_red);
    const float a = __uint_as_float(amax);
    if (threadIdx.x == 0) amax_out[row] = a;
    if (q_out) {
      const float qs = fp8_row_scale(a, q_mode == 2);
      const bool finite = fp8_row_finite(a, qs);
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int c = (threadIdx.x + j * kThreads) * V;
        if (c < hidden) {
          uint32_t w[V / 4];
#pragma unroll
          for (int i = 0; i < V / 4; ++i) {
            const float* f = &ov[j][4 * i];
            w[i] = finite ? f32x4_to_fp8x4_finite(f[0] * qs, f[1] * qs, f[2] * qs, f[3] * qs)
                          : f32x4_to_fp8x4_sw(f[0] * qs, f[1] * qs, f[2] * qs, f[3] * qs);
          }
          *reinterpret_cast<uint2*>(q_out + row * q_stride + c) = uint2{w[0], w[1]};
        }
      }
    }
  }
}

// Row r of the input is at in + (r / heads) * in_stride + (r % heads) * in_head_stride
// (heads = 1 for plain rows; heads > 1 normalises every head of a strided
// [tokens, heads, head_dim] view, as Qwen3's q_norm / k_norm do).  Output row r
// is at out + r * out_stride; residual / residual_out are contiguous rows.
// Short rows (hidden = 8 T, T = 4 .. 64 lanes, e.g. Qwen3's per-head q / k
// norms at head_dim 128): T lanes per row, 256 / T rows per workgroup, the
// row's sum of squares a segmented wave reduction; the same formula as
// rmsnorm_kernel, without residual or quantised outputs.  (One 256-thread
// workgroup per 128-element head row left 15 of 16 threads idle and launched
// millions of workgroups per prefill layer.)
template <int T>
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(const bf16_t* __restrict__ in, int64_t in_stride,
                                                                int64_t in_head_stride, int heads,
                                                                const bf16_t* __restrict__ weight,
                                                                bf16_t* __restrict__ out, int64_t out_stride,
                                                                int64_t rows, float eps) {
  constexpr int kRows = kThreads / T;
  const int64_t r = (int64_t)blockIdx.x * kRows + threadIdx.x / T;
  const int c = (threadIdx.x % T) * 8;
  const bool ok = r < rows;
  Vec<bf16_t, 8> xv{};
  if (ok) {
    const int64_t tok = r / heads, hd = r - tok * heads;
    xv = *reinterpret_cast<const Vec<bf16_t, 8>*>(in + tok * in_stride + hd * in_head_stride + c);
  }
  float xf[8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xf[i] = bf16_to_f32(xv.v[i].bits);
    ss += xf[i] * xf[i];
  }
  ss = segment_sum<T>(ss);  // every lane, rows past the end included
  if (!ok) return;
  const float inv = rsqrtf(ss / (float)(8 * T) + eps);  // torch.rsqrt (layernorm.py:24, 38)
  const Vec<bf16_t, 8> wv = *reinterpret_cast<const Vec<bf16_t, 8>*>(weight + c);
  Vec<bf16_t, 8> o;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float xn = bf16_to_f32(f32_to_bf16(xf[i] * inv));
    o.v[i].bits = (uint16_t)f32_to_bf16(xn * bf16_to_f32(wv.v[i].bits));
  }
  *reinterpret_cast<Vec<bf16_t, 8>*>(out + r * out_stride + c) = o;
}

FDMS_EXPORT int fdms_rmsnorm(const void* in, int64_t in_stride, int64_t in_head_stride, int heads,
                             const void* residual, const void* weight, void* out, int64_t out_stride,
                             void* residual_out, int64_t rows, int hidden, float eps, float* amax_out,
                             void* q_out, int64_t q_stride, int q_mode, void* stream) {
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > 8 * kThreads * 4 || heads <= 0) return (int)hipErrorInvalidValue;
  if (heads > 1 && (residual || residual_out)) return (int)hipErrorInvalidValue;
  if (q_out && (!amax_out || q_mode < 1 || q_mode > 2 || q_stride < hidden || q_stride % 8 || (uintptr_t)q_out % 8))
    return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!in || !weight || (!out && !q_out) || rows > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  // rows move as 16-byte vectors
  if (!fdms_aligned16(in, weight, out, residual, residual_out) || (in_stride | in_head_stride | out_stride) % 8)
    return (int)hipErrorInvalidValue;
  const int lanes = hidden / 8;
  if (!residual && !residual_out && !amax_out && !q_out && hidden <= 512 && lanes >= 4 && !(lanes & (lanes - 1))) {
    const int64_t blocks = (rows * lanes + kThreads - 1) / kThreads;
#define FDMS_RMSNORM_ROWS(TV)                                                                                   \
  hipLaunchKernelGGL((rmsnorm_rows_kernel<TV>), dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream,  \
                     (const bf16_t*)in, in_stride, in_head_stride, heads, (const bf16_t*)weight, (bf16_t*)out,       \
                     out_stride, rows, eps)
    switch (lanes) {
      case 4: FDMS_RMSNORM_ROWS(4); break;
      case 8: FDMS_RMSNORM_ROWS(8); break;
      case 16: FDMS_RMSNORM_ROWS(16); break;
      case 32: FDMS_RMSNORM_ROWS(32); break;
      default: FDMS_RMSNORM_ROWS(64); break;
    }
#undef FDMS_RMSNORM_ROWS
    FDMS_LAUNCH_CHECK();
    return 0;
  }
#define FDMS_RMSNORM(PERV)                                                                                      \
  hipLaunchKernelGGL((rmsnorm_kernel<false, 0, PERV>), dim3((unsigned)rows), dim3(kThreads), 0,                  \
                     (hipStream_t)stream, (const bf16_t*)in, (const bf16_t*)residual, (const bf16_t*)weight,        \
                     (bf16_t*)out, (bf16_t*)residual_out, hidden, in_stride, in_head_stride, heads, out_stride, eps, \
                     nullptr, 0, (int64_t)0, nullptr, nullptr, amax_out, (uint8_t*)q_out, q_stride, q_mode, nullptr,    \
                     (int64_t)0)
  const int per = (hidden + 8 * kThreads - 1) / (8 * kThreads);
  if (per == 1) FDMS_RMSNORM(1);
  else if (per == 2) FDMS_RMSNORM(2);
  else FDMS_RMSNORM(4);
#undef FDMS_RMSNORM
  FDMS_LAUNCH_CHECK();
  return 0;
}

// RMSNorm (+ residual) of x = bf16(sum of the k_splits fp32 partials
// partials[s * split_stride + r * hidden + c]) -- the consumer side of
// fdms_linear_small_m's epilogue 3.  residual / residual_out contiguous rows.
FDMS_EXPORT int fdms_rmsnorm_partials(const float* partials, int k_splits, int64_t split_stride,
                                      const void* residual, const void* weight, void* out, int64_t out_stride,
                                      void* residual_out, int64_t rows, int hidden, float eps,
                                      const float* row_scale, const float* col_scale, float* amax_out,
                                      void* q_out, int64_t q_stride, int q_mode, void* stream) {
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > 8 * kThreads * 4 || k_splits < 1) return (int)hipErrorInvalidValue;
  if (q_out && (!amax_out || q_mode < 1 || q_mode > 2 || q_stride < hidden || q_stride % 8 || (uintptr_t)q_out % 8))
    return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!partials || !weight || (!out && !q_out) || rows > 0x7FFFFFFF || split_stride < rows * (int64_t)hidden)
    return (int)hipErrorInvalidValue;
  if ((uintptr_t)partials % 32 || split_stride % 8 || (uintptr_t)col_scale % 32) return (int)hipErrorInvalidValue;
  if (!fdms_aligned16(weight, out, residual, residual_out) || out_stride % 8) return (int)hipErrorInvalidValue;
#define FDMS_RMSNORM_PART(KSV, PERV)                                                                              \
  hipLaunchKernelGGL((rmsnorm_kernel<true, KSV, PERV>), dim3((unsigned)rows), dim3(kThreads), 0,                   \
                     (hipStream_t)stream, nullptr, (const bf16_t*)residual, (const bf16_t*)weight, (bf16_t*)out,      \
                     (bf16_t*)residual_out, hidden, (int64_t)0, (int64_t)0, 1, out_stride, eps, partials, k_splits,   \
                     split_stride, row_scale, col_scale, amax_out, (uint8_t*)q_out, q_stride, q_mode, nullptr,        \
                     (int64_t)0)
#define FDMS_RMSNORM_PART_PER(PERV)                   \
  if (k_splits == 1) FDMS_RMSNORM_PART(1, PERV);      \
  else if (k_splits == 2) FDMS_RMSNORM_PART(2, PERV); \
  else if (k_splits == 4) FDMS_RMSNORM_PART(4, PERV); \
  else if (k_splits == 8) FDMS_RMSNORM_PART(8, PERV); \
  else FDMS_RMSNORM_PART(0, PERV)
  const int per = (hidden + 8 * kThreads - 1) / (8 * kThreads);
  if (per == 1) {
    FDMS_RMSNORM_PART_PER(1);
  } else if (per == 2) {
    FDMS_RMSNORM_PART_PER(2);
  } else {
    FDMS_RMSNORM_PART_PER(4);
  }
#undef FDMS_RMSNORM_PART_PER
#undef FDMS_RMSNORM_PART
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Embedding gather + RMSNorm of the gathered rows in one launch (the decode
// step's first layer: F.embedding, embed_head.py:87-104, then the first
// input_layernorm without residual, layernorm.py:16-28): rows_out[i] =
// table[ids[i]] (the first residual), out[i] = RMSNorm(rows_out[i]), the same
// bits as fdms_rmsnorm of the gathered rows.  An id outside [0, vocab) gives
// NaN rows in both (the reference's index_select raises there).
FDMS_EXPORT int fdms_embedding_rmsnorm(const int64_t* ids, int64_t n, const void* table, int64_t table_stride,
                                       int64_t vocab, const void* weight, float eps, void* out, int64_t out_stride,
                                       void* rows_out, int64_t rows_stride, int hidden, void* stream) {
  if (n < 0 || hidden <= 0 || hidden % 8 || hidden > 8 * kThreads * 4 || vocab <= 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  if (!ids || !table || !weight || !out || !rows_out || n > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  if (!fdms_aligned16(table, weight, out, rows_out) || (table_stride | out_stride | rows_stride) % 8 ||
      table_stride < hidden || out_stride < hidden || rows_stride != hidden)
    return (int)hipErrorInvalidValue;
#define FDMS_EMB_RMSNORM(PERV)                                                                                    \
  hipLaunchKernelGGL((rmsnorm_kernel<false, 0, PERV>), dim3((unsigned)n), dim3(kThreads), 0, (hipStream_t)stream,   \
                     (const bf16_t*)table, nullptr, (const bf16_t*)weight, (bf16_t*)out, (bf16_t*)rows_out, hidden,  \
                     table_stride, (int64_t)0, 1, out_stride, eps, nullptr, 0, (int64_t)0, nullptr, nullptr, nullptr, \
                     nullptr, (int64_t)0, 0, ids, vocab)
  const int per = (hidden + 8 * kThreads - 1) / (8 * kThreads);
  if (per == 1) FDMS_EMB_RMSNORM(1);
  else if (per == 2) FDMS_EMB_RMSNORM(2);
  else FDMS_EMB_RMSNORM(4);
#undef FDMS_EMB_RMSNORM
  FDMS_LAUNCH_CHECK();
  return 0;
}

// FP8 embedding rows: out[i, :] = bf16(e4m3fn(table[ids[i], :]) * bf16(scale_inv[ids[i]]))
// (embed_head.py:422-432: the FP8 row and its scale_inv, each in bf16, then
// multiplied).  One workgroup per id, 8 columns per thread; an id outside
// [0, vocab) yields a row of NaN (the reference's index_select raises there)
// and reads nothing.
__global__ __launch_bounds__(kThreads) void embedding_fp8_kernel(const int64_t* __restrict__ ids,
                                                                 const uint8_t* __restrict__ table, int64_t t_s,
                                                                 const float* __restrict__ scale_inv, int64_t vocab,
                                                                 bf16_t* __restrict__ out, int64_t o_s, int dim) {
  const int64_t i = blockIdx.x;
  const int64_t id = ids[i];
  const bool ok = id >= 0 && id < vocab;
  const float s = ok ? bf16_to_f32(f32_to_bf16(scale_inv[id])) : __builtin_nanf("");
  const uint8_t* src = table + (ok ? id : 0) * t_s;
  for (int c = threadIdx.x * 8; c < dim; c += kThreads * 8) {
    const uint2 v = ok ? *reinterpret_cast<const uint2*>(src + c) : uint2{0u, 0u};
    const uint32_t w[2] = {v.x, v.y};
    uint32_t o[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[h], false);  // exact
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[h], true);
      o[2 * h] = f32_to_bf16(lo[0] * s) | (f32_to_bf16(lo[1] * s) << 16);
      o[2 * h + 1] = f32_to_bf16(hi[0] * s) | (f32_to_bf16(hi[1] * s) << 16);
    }
    *reinterpret_cast<uint4*>(out + i * o_s + c) = uint4{o[0], o[1], o[2], o[3]};
  }
}

FDMS_EXPORT int fdms_embedding_fp8(const int64_t* ids, int64_t n, const void* table, int64_t table_stride,
                                   const float* scale_inv, int64_t vocab, void* out, int64_t out_stride, int dim,
                                   void* stream) {
  if (n < 0 || dim <= 0 || dim % 8 || vocab <= 0 || table_stride < dim || out_stride < dim) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  if (!ids || !table || !scale_inv || !out || n > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  if ((uintptr_t)table % 8 || table_stride % 8 || !fdms_aligned16(out) || out_stride % 8) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(embedding_fp8_kernel, dim3((unsigned)n), dim3(kThreads), 0, (hipStream_t)stream, ids,
                     (const uint8_t*)table, table_stride, scale_inv, vocab, (bf16_t*)out, out_stride, dim);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// out[r, j] = bf16(silu(x[r, j]) * x[r, F + j]) in fp32 (activation.py:8-11).
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const bf16_t* __restrict__ x, bf16_t* __restrict__ out,
                                                            int64_t rows, int f) {
  constexpr int V = 8;
  const int64_t per_row = f / V;
  const int64_t total = rows * per_row;
  for (int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x; u < total; u += (int64_t)gridDim.x * kThreads) {
    const int64_t r = u / per_row;
    const int64_t c = (u - r * per_row) * V;
    const Vec<bf16_t, V> g = *reinterpret_cast<const Vec<bf16_t, V>*>(x + r * 2 * f + c);
    const Vec<bf16_t, V> up = *reinterpret_cast<const Vec<bf16_t, V>*>(x + r * 2 * f + f + c);
    Vec<bf16_t, V> o;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float a = bf16_to_f32(g.v[i].bits);
      const float s = a / (1.0f + expf(-a));
      o.v[i].bits = (uint16_t)f32_to_bf16(s * bf16_to_f32(up.v[i].bits));
    }
    *reinterpret_cast<Vec<bf16_t, V>*>(out + r * f + c) = o;
  }
}

FDMS_EXPORT int fdms_silu_mul(const void* x, void* out, int64_t rows, int f, void* stream) {
  if (rows < 0 || f <= 0 || f % 8) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!x || !out) return (int)hipErrorInvalidValue;
  const int64_t units = rows * (f / 8);
  const int64_t want = (units + kThreads - 1) / kThreads;
  const int64_t blocks = want < 4096 ? want : 4096;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream,
                     (const bf16_t*)x, (bf16_t*)out, rows, f);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Row argmax with torch.argmax's semantics (embed_head.py:142, 160): ties go
// to the lowest index and NaN counts as larger than every number (the lowest
// NaN index wins), so a row always yields an index in [0, n).

// One 1024-thread block per row; 16-byte vector loads, four in flight per
// thread, when the row is 16-byte aligned; fp32 or bf16 logits; int64 output.
constexpr int kArgmaxThreads = 1024;

template <typename T>
struct ArgmaxVec;
template <>
struct ArgmaxVec<float> {
  static constexpr int kN = 4;
  static __device__ __forceinline__ void load(const float* p, float* v) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  }
};
template <>
struct ArgmaxVec<bf16_t> {
  static constexpr int kN = 8;
  static __device__ __forceinline__ void load(const bf16_t* p, float* v) {
    const uint4 x = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};

template <typename T, bool VEC>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const T* __restrict__ x, int64_t stride, int n,
                                                                     int64_t* __restrict__ out) {
  constexpr int kW = kArgmaxThreads / kWave;
  __shared__ float s_v[kW];
  __shared__ int s_i[kW];
  const T* row = x + (int64_t)blockIdx.x * stride;
  float best = -INFINITY;
  int bi = 0x7FFFFFFF;  // no element yet: loses every comparison
  auto take = [&](float v, int j) {
    if (bi == 0x7FFFFFFF || argmax_better(v, j, best, bi)) {
      best = v;
      bi = j;
    }
  };
  int tail = 0;
  if (VEC) {
    constexpr int N = ArgmaxVec<T>::kN;
    constexpr int kU = 4;  // vectors in flight per thread
    const int nvec = n / N;
    for (int v0 = threadIdx.x; v0 < nvec; v0 += kArgmaxThreads * kU) {
      float vals[kU][N];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int vi = v0 + u * kArgmaxThreads;
        if (vi < nvec) ArgmaxVec<T>::load(row + (int64_t)vi * N, vals[u]);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int vi = v0 + u * kArgmaxThreads;
        if (vi < nvec) {
#pragma unroll
          for (int e = 0; e < N; ++e) take(vals[u][e], vi * N + e);
        }
      }
    }
    tail = nvec * N;
  }
  for (int j = tail + threadIdx.x; j < n; j += kArgmaxThreads) take(ld<T>(row + j), j);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o);
    const int oi = __shfl_xor(bi, o);
    if (oi != 0x7FFFFFFF && (bi == 0x7FFFFFFF || argmax_better(ov, oi, best, bi))) {
      best = ov;
      bi = oi;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[w] = best;
    s_i[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kW; ++i) {
      if (s_i[i] != 0x7FFFFFFF && (bi == 0x7FFFFFFF || argmax_better(s_v[i], s_i[i], best, bi))) {
        best = s_v[i];
        bi = s_i[i];
      }
    }
    out[blockIdx.x] = bi;
  }
}

FDMS_EXPORT int fdms_argmax_rows(const void* x, int dtype, int64_t stride, int64_t rows, int n, int64_t* out,
                                 void* stream) {
  if (rows < 0 || n <= 0 || rows > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!x || !out) return (int)hipErrorInvalidValue;
  const int esz = dtype == kF32 ? 4 : 2;
  const bool vec = ((uintptr_t)x % 16) == 0 && (stride * esz) % 16 == 0;
  const dim3 grid((unsigned)rows), block(kArgmaxThreads);
  if (dtype == kF32) {
    if (vec) hipLaunchKernelGGL((argmax_rows_kernel<float, true>), grid, block, 0, (hipStream_t)stream, (const float*)x, stride, n, out);
    else hipLaunchKernelGGL((argmax_rows_kernel<float, false>), grid, block, 0, (hipStream_t)stream, (const float*)x, stride, n, out);
  } else if (dtype == kBF16) {
    if (vec) hipLaunchKernelGGL((argmax_rows_kernel<bf16_t, true>), grid, block, 0, (hipStream_t)stream, (const bf16_t*)x, stride, n, out);
    else hipLaunchKernelGGL((argmax_rows_kernel<bf16_t, false>), grid, block, 0, (hipStream_t)stream, (const bf16_t*)x, stride, n, out);
  } else {
    return (int)hipErrorInvalidValue;
  }
  FDMS_LAUNCH_CHECK();
  return 0;
}
