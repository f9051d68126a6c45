// Decode-shaped linear layers (M <= 16 rows): y[m, n] = sum_k a[m, k] * W[n, k]
// with W in bf16 or FP8 e4m3fn + per-output-channel scale.
//
// Reference semantics (fastdms/layers/linear.py):
//   bf16 weights: F.linear(x, W, bias) -> bf16(acc + bias)            (926)
//   FP8 weights (quantize_weight_to_fp8, 813-847): W8[n, k] = fp8(W[n, k] *
//     s[n]), s[n] = 448 / amax(W[n, :]) (1 if 0), scale_inv[n] = 1 / s[n];
//     small-M / row1 kernels (492-632, 665-763): per-row dynamic activation
//     quantisation x_s[m] = 448 / amax(x[m, :]), xq = fp8(x * x_s), then
//     y = bf16(sum_k xq * W8 * (1 / x_s[m]) * scale_inv[n]), bias added in bf16.
//
// The activation may be produced on the fly by a fused prologue:
//   PRO = 1: RMSNorm with the residual add of layernorm.py:19-40:
//            f = fp32(x) + fp32(residual) (residual optional), residual_out =
//            bf16(f) (written by workgroup 0), a = bf16(bf16(f * rsqrt(mean(f^2)
//            + eps)) * norm_w) -- the normalised value is the unrounded sum.
//   PRO = 2: the same RMSNorm on rows that an EPI 4 producer finished: x holds
//            f itself (fp32 rows) and x_amax the producer strips' sums of f^2
//            ([M, strips]); rsqrt(sum / K + eps) is taken from those, so a
//            workgroup reads only its own K range of f (no pass over the row).
// and the output may go through a fused epilogue:
//   EPI = 1: the weight holds [gate; up] (n = 2 * n_out rows, gate_up_proj) and
//            the output is bf16(silu(bf16 gate) * bf16 up) (activation.py:8-11).
//   EPI = 3: no bias: each K split writes its fp32 partial sums to
//            workspace[split][m][n]; the consumer adds them in split order and
//            applies the row scale 1/x_s[m] and the FP8 column scale (the merge
//            and scaling of EPI 0, moved into the next kernel).
//   EPI = 4: the residual add of the RMSNorm that follows (layernorm.py:32-40):
//            with v = the finalised bf16 output, y receives f = fp32(v) +
//            fp32(residual) as fp32 rows, residual_out = bf16(f) (it may be
//            the residual itself: each element is read, then written, by one
//            lane), and amax_out[m][strip] = the strip's sum of f^2 -- what a
//            PRO 2 consumer needs to apply the norm.
// The activation's per-row amax may come from its producer (x_amax: the
// RMSNorm's output amax, or the per-strip output amax that EPI 0 / 1 writes to
// amax_out) instead of a statistics pass over x.
//
// MI355X mapping: one workgroup per 16-column output strip (per gate/up strip
// pair for EPI 1) and K split; its NW waves split the workgroup's K range.  A
// k-block is 64 columns: a lane group of 16 lanes reads 32 contiguous bytes of
// 16 weight rows; each wave double-buffers groups of U k-blocks (the next
// group's loads are in flight while the current one runs
// v_mfma_f32_16x16x32_bf16 with A = 16 weight rows, B = the activation rows,
// M <= 16 padded with zeros, C = y^T).  FP8 weights are exact in bf16, so the
// FP8 path without activation quantisation converts in registers and uses the
// same MFMA; products are exact and accumulate in fp32 like the reference's
// FP8 dot.  FP8 weights with the quantised activation, and INT4 weights, read
// 128-column k-blocks (lane group g: columns 32g .. 32g + 31): the FP8 ones
// multiply on v_mfma_scale_f32_16x16x128_f8f6f4, the INT4 ones are
// dequantised to bf16 for four v_mfma_f32_16x16x32_bf16.  The waves' C fragments are
// summed through LDS.  When there are fewer strips than CUs, K is split across
// workgroups: each split publishes its fragment with agent-scope atomic stores
// and the last split of a strip to arrive (device-scope ticket) sums them and
// runs the epilogue, then resets its ticket.  HBM-bound on W.
#include <cstdlib>
#include <type_traits>

#include "fdms_vec.h"

using namespace fdms;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kKB = 64;       // k-block: columns per lane group step
constexpr int kMaxM = 16;
constexpr float kFp8Max = 448.0f;

// two fp32 -> bf16 (round to nearest even), a in the low half: one
// v_cvt_pk_bf16_f32 (two scalar conversions compile to two of them, a shift
// and an or)
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t r = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ float rbf(float a) { return (float)(__bf16)a; }  // round to bf16
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

template <typename WT> struct WBlock;
// bf16 weights: a lane group reads 16 bf16 = 32 B per k-block
template <> struct WBlock<bf16_t> {
  struct Raw { uint4 v[2]; };
  static __device__ __forceinline__ void load(const bf16_t* row, int k, Raw& r) {
    const uint4* p = reinterpret_cast<const uint4*>(row + k);
    r.v[0] = p[0];
    r.v[1] = p[1];
  }
  static __device__ __forceinline__ void to_ops(const Raw& r, uint4* op0, uint4* op1) {
    *op0 = r.v[0];
    *op1 = r.v[1];
  }
};
// FP8 weights: 16 fp8 = 16 B per k-block, converted to two bf16x8 operands
template <> struct WBlock<fp8_t> {
  using Raw = uint4;
  static __device__ __forceinline__ void load(const fp8_t* row, int k, Raw& r) {
    r = *reinterpret_cast<const uint4*>(row + k);
  }
  static __device__ __forceinline__ void to_ops(const Raw& r, uint4* op0, uint4* op1) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
      o[2 * i] = pack2(lo[0], lo[1]);   // fp8 values are exact in bf16
      o[2 * i + 1] = pack2(hi[0], hi[1]);
    }
    *op0 = uint4{o[0], o[1], o[2], o[3]};
    *op1 = uint4{o[4], o[5], o[6], o[7]};
  }
};
// the generic path's per-k-block weight registers (INT4 weights take the
// 128-column path, which keeps its codes in Buf::w4)
template <typename WT> struct WRaw { using type = typename WBlock<WT>::Raw; };
template <> struct WRaw<u4x2_t> { using type = uint32_t; };

template <typename WT> __device__ __forceinline__ constexpr bool is_fp8() { return false; }
template <> __device__ __forceinline__ constexpr bool is_fp8<fp8_t>() { return true; }
template <typename WT> __device__ __forceinline__ constexpr bool is_int4() { return false; }
template <> __device__ __forceinline__ constexpr bool is_int4<u4x2_t>() { return true; }

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// 8 bf16 of x (+ 8 of r when r != nullptr) as fp32 sums
__device__ __forceinline__ void load_sum8(const bf16_t* x, const bf16_t* r, float* f) {
  const uint4 v = *reinterpret_cast<const uint4*>(x);
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf_lo(u[i]);
    f[2 * i + 1] = bf_hi(u[i]);
  }
  if (r) {
    const uint4 q = *reinterpret_cast<const uint4*>(r);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] += bf_lo(w[i]);
      f[2 * i + 1] += bf_hi(w[i]);
    }
  }
}

constexpr int kXcds = 8;

__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Row statistics of the RMSNorm prologue / activation quantisation for row m,
// computed by one wave with every load of a batch in flight together.
template <int PRO, bool QX>
__device__ __forceinline__ void row_stats(const bf16_t* xr, const bf16_t* rr, const bf16_t* norm_w, int K, float eps,
                                          int qx_torch, int lane, bf16_t* res_out_row, float* inv_out,
                                          float* xs_out) {
  constexpr int kB = 8;  // 16-byte chunks per lane per batch
  float inv = 1.0f;
  if (PRO == 1) {
    float ss = 0.0f;
    for (int k0 = lane * 8; k0 < K; k0 += 64 * 8 * kB) {
      float f[kB][8];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int k = k0 + j * 64 * 8;
        if (k < K) load_sum8(xr + k, rr ? rr + k : nullptr, f[j]);
      }
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int k = k0 + j * 64 * 8;
        if (k < K) {
#pragma unroll
          for (int i = 0; i < 8; ++i) ss += f[j][i] * f[j][i];
          if (res_out_row) {
            *reinterpret_cast<uint4*>(res_out_row + k) =
                uint4{pack2(f[j][0], f[j][1]), pack2(f[j][2], f[j][3]), pack2(f[j][4], f[j][5]), pack2(f[j][6], f[j][7])};
          }
        }
      }
    }
    ss = wave_sum(ss);
    inv = rsqrtf(ss / (float)K + eps);  // torch.rsqrt (layernorm.py:24, 38)
  }
  float amax = 0.0f;
  if (QX) {
    for (int k0 = lane * 8; k0 < K; k0 += 64 * 8 * kB) {
      float f[kB][8];
      uint4 wv[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int k = k0 + j * 64 * 8;
        if (k < K) {
          load_sum8(xr + k, (PRO == 1 && rr) ? rr + k : nullptr, f[j]);
          if (PRO == 1) wv[j] = *reinterpret_cast<const uint4*>(norm_w + k);
        }
      }
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int k = k0 + j * 64 * 8;
        if (k < K) {
          const uint32_t uw[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float a = f[j][i];
            if (PRO == 1) a = rbf(rbf(a * inv) * ((i & 1) ? bf_hi(uw[i >> 1]) : bf_lo(uw[i >> 1])));
            amax = fmaxf(amax, fabsf(a));
          }
        }
      }
    }
    amax = wave_max(amax);
  }
  *inv_out = inv;
  // 448 / amax: the Triton kernels divide; torch's tensor expression
  // (_fp8_linear) multiplies the reciprocal of amax by 448 (two roundings)
  *xs_out = (amax > 0.0f) ? (qx_torch ? (1.0f / amax) * kFp8Max : kFp8Max / amax) : 1.0f;
}

}  // namespace

// y[m, n] = a[m, :] . W[n, :] for one 16-column strip (two for EPI 1) and one
// K split.  EPI 0: y = the finalised value.  EPI 1 (gate_up): the workgroup
// computes gate strip n0 and up strip n0 + n_out and writes
// bf16(silu(bf16 gate) * bf16 up) -- gate_up followed by SiluAndMul.
template <typename WT, int PRO, bool QX, int EPI, int NW, int U, bool XQ = false>
__global__ __launch_bounds__(NW * 64) void linear_small_m_kernel(
    const bf16_t* __restrict__ x, int64_t x_s, int M, int K, const WT* __restrict__ w, int64_t w_s,
    const float* __restrict__ w_scale_inv, const bf16_t* __restrict__ bias, const bf16_t* __restrict__ norm_w,
    float eps, const bf16_t* res, int64_t res_s, bf16_t* res_out, int64_t ro_s,
    bf16_t* __restrict__ y, int64_t y_s, int n_out, int strips, int ksplit, float* __restrict__ ws,
    int* __restrict__ counters, float* __restrict__ part_val, int* __restrict__ part_idx,
    const uint32_t* __restrict__ g_sz, int group, int64_t g_s, int qx_torch,
    int bf16_scores, const float* __restrict__ x_amax, int x_amax_n, int64_t x_amax_s, float* __restrict__ amax_out,
    float* __restrict__ row_scale_out) {
  constexpr int NA = EPI == 1 ? 2 : 1;  // accumulators (strips) per workgroup
  // FP8 weights with the quantised activation run on the FP8 matrix cores
  // (v_mfma_scale_f32_16x16x128_f8f6f4, unit scales): 128-column k-blocks,
  // lane group g holding columns 32g .. 32g + 31 of both operands, no
  // per-element conversion of the weights
  constexpr bool F8 = is_fp8<WT>() && QX && PRO == 0;
  // XQ: x already holds the e4m3fn codes of the quantised activation (its
  // producer quantised it with the row amax it hands over in x_amax)
  static_assert(!XQ || F8, "a pre-quantised activation needs FP8 weights");
  // INT4 weights use the same 128-column k-blocks: lane group g reads 16
  // bytes (32 codes) of its row for columns 32g .. 32g + 31 -- one group of
  // the scale_zeros layout (group >= 32) -- and dequantises them into four
  // bf16 operands for v_mfma_f32_16x16x32_bf16 (MFMA j: columns 32g + 8j ..)
  constexpr bool I4 = is_int4<WT>();
  static_assert(!I4 || (PRO == 0 && !QX), "INT4 weights take bf16 activations, no prologue");
  constexpr int KB = (F8 || I4) ? 2 * kKB : kKB;
  __shared__ float s_inv[kMaxM], s_xs[kMaxM];
  __shared__ f32x4 s_acc[NA][NW][64];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  // the wave index is uniform across the wave: saying so keeps the k-range
  // tests below scalar branches (a divergent branch around a load makes the
  // compiler wait for the load where the branches join)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  // XCD-aware (strip, split): the K splits of one strip run on the same XCD
  const int lin = blockIdx.x;
  const int xcd = lin % kXcds;
  const int slot = lin / kXcds;
  const int strip = (slot / ksplit) * kXcds + xcd;
  const int ks = slot - (slot / ksplit) * ksplit;
  if (strip >= strips) return;  // uniform per workgroup
  const int n0 = strip * 16;

  const int kc = K / ksplit;            // this workgroup's K range
  const int kw = kc / NW;               // this wave's part of it
  const int kw0 = ks * kc + wave * kw;
  const int kend = kw0 + kw;
  const int g = lane >> 4;
  const int c = lane & 15;
  const WT* wrow[NA];
  wrow[0] = w + (int64_t)(n0 + c) * w_s;
  if (EPI == 1) wrow[NA - 1] = w + (int64_t)(n0 + n_out + c) * w_s;
  const bool has_row = c < M;
  const bf16_t* xrow = x + (int64_t)(has_row ? c : 0) * x_s;
  const uint8_t* xqrow = reinterpret_cast<const uint8_t*>(x) + (int64_t)(has_row ? c : 0) * x_s;  // XQ
  const bf16_t* rrow = (PRO == 1 && res) ? res + (int64_t)(has_row ? c : 0) * res_s : nullptr;
  const float* frow0 = reinterpret_cast<const float*>(x);  // PRO 2: the fp32 rows
  float inv = 1.0f, xsc = 1.0f;  // row statistics, read after the stats pass below
  bool xfin = true;               // F8: x * xsc of this lane's row is finite and in range
  f32x4 acc[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};

  // PRO 2 stages each group's activation through this wave's slice of LDS:
  // the group's fp32 rows arrive as contiguous 16-byte chunks (lane l takes
  // columns 4 (l % kCq) .. + 3 of rows l / kCq, + kRq, ...), are normalised
  // once and stored as bf16, and the k-blocks read their B operands back
  // (rows padded by 16 bytes: the 16 rows of a lane group fall in distinct
  // banks).  Each wave reads only its own slice, so no workgroup barrier.
  constexpr int G = U * KB;                  // columns per group
  constexpr int kCq = G / 4;                 // 16-byte fp32 chunks per row and group
  constexpr int kRq = kCq >= 64 ? 1 : 64 / kCq;  // rows per load instruction
  constexpr int kActRows = kMaxM;
  constexpr int kFChunks = (kActRows + kRq - 1) / kRq;
  constexpr int kActStride = G + 8;          // bf16 per LDS row
  __shared__ __attribute__((aligned(16))) uint16_t s_act[PRO == 2 ? NW : 1][PRO == 2 ? kActRows : 1][PRO == 2 ? kActStride : 8];
  const int fq_row = lane / kCq, fq_col = 4 * (lane % kCq);
  float fq_inv[kFChunks];  // PRO 2: inv of rows fq_row + kRq * t (set after the statistics)

  struct Buf {
    typename WRaw<WT>::type w[NA][U];
    uint32_t gsz[NA][U];  // I4: the group's (scale, zero) as two bf16
    uint4 x[U][2];
    uint4 r[U][2];   // residual (PRO 1)
    uint4 nw[U][2];  // norm weight (PRO 1)
    uint4 fch[kFChunks];  // PRO 2: the group's fp32 rows, this lane's chunks
    uint2 fnw;            // PRO 2: norm weight of this lane's four columns
    uint4 w8[NA][U][2];  // F8: 32 weight bytes per lane per k-block
    uint4 x8[U][4];      // F8 / I4: 32 bf16 activations per lane per k-block
    uint4 w4[NA][U];     // I4: 32 weight codes per lane per k-block
  };
  auto load = [&](int kb0, Buf& b) {
    if constexpr (I4) {
      // activation chunks first (from L2), then codes and (scale, zero);
      // a last half block's lane groups 2 and 3 read clamped columns that
      // compute zeroes
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * KB < kend) {
          const int kl = min(kb0 + u * KB + 32 * g, kend - 32);
          const uint4* xp = reinterpret_cast<const uint4*>(xrow + kl);
#pragma unroll
          for (int i = 0; i < 4; ++i) b.x8[u][i] = xp[i];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * KB < kend) {
          const int kl = min(kb0 + u * KB + 32 * g, kend - 32);
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            b.w4[a][u] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(wrow[a]) + kl / 2);
            // group kl / group of weight row n: consecutive lanes read consecutive rows
            b.gsz[a][u] = g_sz[(int64_t)(kl / group) * g_s + (n0 + c + (a ? n_out : 0))];
          }
        }
      }
    } else if constexpr (F8) {
      // the group's activation loads go out before its weight loads: loads
      // complete in issue order, so the activation (from L2) is quantised
      // while the weights are still on their way from HBM.  Branch-free: a
      // last half block (64 columns) has nothing for lane groups 2 and 3,
      // whose loads are clamped in bounds and whose values (and those of rows
      // >= M, read from row 0) are zeroed in compute
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * KB < kend) {
          const int kl = min(kb0 + u * KB + 32 * g, kend - 32);
          if constexpr (XQ) {
            const uint4* xp = reinterpret_cast<const uint4*>(xqrow + kl);
            b.x8[u][0] = xp[0];
            b.x8[u][1] = xp[1];
          } else {
            const uint4* xp = reinterpret_cast<const uint4*>(xrow + kl);
#pragma unroll
            for (int i = 0; i < 4; ++i) b.x8[u][i] = xp[i];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * KB < kend) {
          const int kl = min(kb0 + u * KB + 32 * g, kend - 32);
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            const uint4* p = reinterpret_cast<const uint4*>(wrow[a] + kl);
            b.w8[a][u][0] = p[0];
            b.w8[a][u][1] = p[1];
          }
        }
      }
    } else {
      if constexpr (PRO == 2) {
        // chunks of rows < M only (uniform per t: rows fq_row + kRq t, clamped)
        const int col = min(kb0 + fq_col, kend - 4);
#pragma unroll
        for (int t = 0; t < kFChunks; ++t)
          if (kRq * t < M)
            b.fch[t] = *reinterpret_cast<const uint4*>(frow0 + (int64_t)min(fq_row + kRq * t, M - 1) * x_s + col);
        b.fnw = *reinterpret_cast<const uint2*>(norm_w + col);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kb0 + u * kKB + 16 * g;
        if (kb0 + u * kKB < kend) {
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            WBlock<WT>::load(wrow[a], k, b.w[a][u]);
          }
          b.x[u][0] = b.x[u][1] = b.r[u][0] = b.r[u][1] = uint4{0u, 0u, 0u, 0u};
          if (PRO != 2 && has_row) {
            const uint4* xp = reinterpret_cast<const uint4*>(xrow + k);
            b.x[u][0] = xp[0];
            b.x[u][1] = xp[1];
            if (PRO == 1) {
              const uint4* np = reinterpret_cast<const uint4*>(norm_w + k);
              b.nw[u][0] = np[0];
              b.nw[u][1] = np[1];
              if (rrow) {
                const uint4* rp = reinterpret_cast<const uint4*>(rrow + k);
                b.r[u][0] = rp[0];
                b.r[u][1] = rp[1];
              }
            }
          }
        }
      }
    }
  };
  auto compute = [&](int kb0, const Buf& b) {
    if constexpr (I4) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * KB >= kend) break;
        const bool xv = kb0 + u * KB + 32 * g < kend && has_row;  // this lane group's columns and row exist
        // the activation operands, zeroed where they do not exist, shared by both strips
        uint4 bxs[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bxs[j] = xv ? b.x8[u][j] : uint4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          // w = bf16((q - 8) * s + z) as one fma of the code: q * s + (z - 8s)
          // (z - 8s exact for the symmetric zero 0); each byte of the masked
          // word converts in one v_cvt_f32_ubyte, the high nibbles as 16q
          // (with s / 16)
          const float sc = bf_lo(b.gsz[a][u]), zc = bf_hi(b.gsz[a][u]);
          const float c8 = __builtin_fmaf(-8.0f, sc, zc), s16 = sc * 0.0625f;
          const uint32_t wd[4] = {b.w4[a][u].x, b.w4[a][u].y, b.w4[a][u].z, b.w4[a][u].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            uint32_t lo = wd[j] & 0x0F0F0F0Fu, hi = wd[j] & 0xF0F0F0F0u;
            // hide the masks' known zero bits from the compiler: it would
            // otherwise narrow (lo >> 8i) & 0xFF to a 4-bit field extract
            // plus a byte-0 conversion, two instructions instead of one
            // v_cvt_f32_ubyte<i> per code
            asm("" : "+v"(lo), "+v"(hi));
            const uint4 aw = uint4{
                pack2(__builtin_fmaf((float)(lo & 0xFFu), sc, c8),
                      __builtin_fmaf((float)(hi & 0xFFu), s16, c8)),
                pack2(__builtin_fmaf((float)((lo >> 8) & 0xFFu), sc, c8),
                      __builtin_fmaf((float)((hi >> 8) & 0xFFu), s16, c8)),
                pack2(__builtin_fmaf((float)((lo >> 16) & 0xFFu), sc, c8),
                      __builtin_fmaf((float)((hi >> 16) & 0xFFu), s16, c8)),
                pack2(__builtin_fmaf((float)((lo >> 24) & 0xFFu), sc, c8),
                      __builtin_fmaf((float)((hi >> 24) & 0xFFu), s16, c8))};
            acc[a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(aw), as_bf16x8(bxs[j]), acc[a], 0, 0, 0);
          }
        }
      }
    } else if constexpr (F8) {
      // every block's activation quantised first (it arrives before the
      // weights), then the MFMAs
      uint32_t qx[U][8];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * KB >= kend) break;
        if constexpr (XQ) {
          const uint4 a0 = b.x8[u][0], a1 = b.x8[u][1];
          qx[u][0] = a0.x; qx[u][1] = a0.y; qx[u][2] = a0.z; qx[u][3] = a0.w;
          qx[u][4] = a1.x; qx[u][5] = a1.y; qx[u][6] = a1.z; qx[u][7] = a1.w;
          continue;
        }
        // x * x_s quantised to e4m3fn, four columns per word: the clamped
        // hardware RNE conversion, or the software encoder for a row whose
        // amax or scale is not finite (NaN / inf elements)
        float f[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t v[4] = {b.x8[u][i].x, b.x8[u][i].y, b.x8[u][i].z, b.x8[u][i].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f[8 * i + 2 * e] = bf_lo(v[e]) * xsc;
            f[8 * i + 2 * e + 1] = bf_hi(v[e]) * xsc;
          }
        }
        if (__builtin_expect(xfin, 1)) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            qx[u][j] = f32x4_to_fp8x4_finite(f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3]);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) qx[u][j] = f32x4_to_fp8x4_sw(f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * KB >= kend) break;
        const bool gv = kb0 + u * KB + 32 * g < kend;  // this lane group's columns exist
        const uint32_t* q = qx[u];
        const bool xv = gv && has_row;
        const i32x8 bx = i32x8{xv ? (int)q[0] : 0, xv ? (int)q[1] : 0, xv ? (int)q[2] : 0, xv ? (int)q[3] : 0,
                               xv ? (int)q[4] : 0, xv ? (int)q[5] : 0, xv ? (int)q[6] : 0, xv ? (int)q[7] : 0};
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const uint4 w0 = b.w8[a][u][0], w1 = b.w8[a][u][1];
          const i32x8 aw = i32x8{gv ? (int)w0.x : 0, gv ? (int)w0.y : 0, gv ? (int)w0.z : 0, gv ? (int)w0.w : 0,
                                 gv ? (int)w1.x : 0, gv ? (int)w1.y : 0, gv ? (int)w1.z : 0, gv ? (int)w1.w : 0};
          acc[a] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aw, bx, acc[a], 0, 0, 0, 127, 0, 127);
        }
      }
    } else {
      if constexpr (PRO == 2) {
        // a = bf16(bf16(f * inv) * norm_w) of the group's rows into this wave's
        // LDS slice (the previous group's reads are done: LDS runs a wave's
        // instructions in order)
        const float nwf[4] = {bf_lo(b.fnw.x), bf_hi(b.fnw.x), bf_lo(b.fnw.y), bf_hi(b.fnw.y)};
#pragma unroll
        for (int t = 0; t < kFChunks; ++t) {
          const int row = fq_row + kRq * t;
          if (kRq * t < M && row < M) {
            const uint4 v = b.fch[t];
            const float f[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
            const float iv = fq_inv[t];
            *reinterpret_cast<uint2*>(&s_act[wave][row][fq_col]) =
                uint2{pack2(rbf(rbf(f[0] * iv) * nwf[0]), rbf(rbf(f[1] * iv) * nwf[1])),
                      pack2(rbf(rbf(f[2] * iv) * nwf[2]), rbf(rbf(f[3] * iv) * nwf[3]))};
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb0 + u * kKB >= kend) break;
        uint4 bo[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (PRO == 0 && !QX) {
            bo[h] = b.x[u][h];
          } else if (PRO == 2) {
            bo[h] = has_row ? *reinterpret_cast<const uint4*>(&s_act[wave][c][u * kKB + 16 * g + 8 * h])
                            : uint4{0u, 0u, 0u, 0u};
          } else {
            const uint32_t v[4] = {b.x[u][h].x, b.x[u][h].y, b.x[u][h].z, b.x[u][h].w};
            const uint32_t q[4] = {b.nw[u][h].x, b.nw[u][h].y, b.nw[u][h].z, b.nw[u][h].w};
            const uint32_t rs[4] = {b.r[u][h].x, b.r[u][h].y, b.r[u][h].z, b.r[u][h].w};
            uint32_t o[4];
            float f[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float lo = bf_lo(v[i]), hi = bf_hi(v[i]);
              if (PRO == 1) {
                lo = rbf(rbf((lo + bf_lo(rs[i])) * inv) * bf_lo(q[i]));
                hi = rbf(rbf((hi + bf_hi(rs[i])) * inv) * bf_hi(q[i]));
              }
              f[2 * i] = lo;
              f[2 * i + 1] = hi;
              o[i] = pack2(lo, hi);
            }
            if (QX) {  // fp8 quantised activation (exact in bf16), four values per conversion
#pragma unroll
              for (int i = 0; i < 2; ++i) {
                const uint32_t q8 = f32x4_to_fp8x4(f[4 * i] * xsc, f[4 * i + 1] * xsc, f[4 * i + 2] * xsc,
                                                   f[4 * i + 3] * xsc);
                o[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)q8, 1.0f, false));
                o[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)q8, 1.0f, true));
              }
            }
            bo[h] = uint4{o[0], o[1], o[2], o[3]};
          }
        }
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          uint4 a0, a1;
          WBlock<WT>::to_ops(b.w[a][u], &a0, &a1);
          acc[a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0), as_bf16x8(bo[0]), acc[a], 0, 0, 0);
          acc[a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1), as_bf16x8(bo[1]), acc[a], 0, 0, 0);
        }
      }
    }
  };

  // 448 / amax: the Triton kernels divide; torch's tensor expression
  // (_fp8_linear) multiplies the reciprocal of amax by 448 (two roundings)
  auto x_scale = [&](float a) { return fp8_row_scale(a, qx_torch != 0); };

  // Activation statistics (PRO 0 with QX): their loads go out before the
  // weight loads -- loads complete in issue order, so the statistics wait for
  // their own loads only -- and the first two weight groups are in flight
  // while the statistics are reduced.  Maxima are taken over abs_bits (NaN
  // propagates, as in the producers' amax).
  constexpr int NT = NW * 64;
  constexpr int kRowsPerWave = (kMaxM + NW - 1) / NW;
  __shared__ uint32_t s_am[kMaxM][NW];
  __shared__ float s_amax[kMaxM];
  const bool amax_one = PRO == 0 && QX && x_amax && x_amax_n == 1;  // uniform
  uint32_t a_one = 0;                // amax_one: row c's amax, one load per lane
  uint32_t av[kRowsPerWave][8];      // x_amax partials: rows wave, wave + NW, ...
  uint4 xv[kMaxM];                   // no x_amax: the first 8-column chunk of each row
  if (PRO == 0 && QX) {
    if (amax_one) {
      a_one = abs_bits(x_amax[(int64_t)min(c, M - 1) * x_amax_s]);
    } else if (x_amax) {
      // indices clamped in bounds: a repeated element cannot change a maximum
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const float* ap = x_amax + (int64_t)min(wave + rr * NW, M - 1) * x_amax_s;
#pragma unroll
        for (int j = 0; j < 8; ++j) av[rr][j] = abs_bits(ap[min(lane + 64 * j, x_amax_n - 1)]);
      }
    } else {
      // the whole workgroup reads every row at once, thread t the 8-column
      // chunks t, t + NT, ...; rows and columns clamped in bounds
      const int c0 = min(tid * 8, K - 8);
#pragma unroll
      for (int mm = 0; mm < kMaxM; ++mm) xv[mm] = *reinterpret_cast<const uint4*>(x + (int64_t)min(mm, M - 1) * x_s + c0);
    }
  }

  // PRO 2: the producer's strip sums go out first (loads complete in issue
  // order, so the reduction below waits for these alone), at most
  // kStatLoads per lane and row, the rest read after
  constexpr int kStatLoads = 4;
  float sv[kRowsPerWave][kStatLoads];
  if constexpr (PRO == 2) {
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const float* sp = x_amax + (int64_t)min(wave + rr * NW, M - 1) * x_amax_s;
#pragma unroll
      for (int j = 0; j < kStatLoads; ++j) sv[rr][j] = sp[min(lane + 64 * j, x_amax_n - 1)];  // masked below
    }
  }

  // with statistics to wait for, both first groups go out before them;
  // otherwise the loop below issues group 1 right after group 0
  constexpr bool kEarly2 = (PRO == 0 && QX) || PRO == 2;
  Buf b0, b1;                // even / odd groups (no register copies between them)
  if (kw0 < kend) load(kw0, b0);
  if (kEarly2 && kw0 + G < kend) load(kw0 + G, b1);

  // |bf16| of both halves of a word as abs_bits
  auto bf_abs_max = [](uint32_t m, uint32_t w) { return max(m, max((w << 16) & 0x7FFFFFFFu, w & 0x7FFF0000u)); };
  if (amax_one) {
    const float a = __uint_as_float(a_one);
    xsc = x_scale(a);
    xfin = fp8_row_finite(a, xsc);
    if (wave == 0 && lane < M) s_xs[lane] = xsc;  // the epilogue's copy (read after the reduction barrier)
  } else if (PRO == 0 && QX && x_amax) {
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int mm = wave + rr * NW;
      uint32_t a = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) a = max(a, av[rr][j]);
      const float* ap = x_amax + (int64_t)min(mm, M - 1) * x_amax_s;
      for (int p = lane + 64 * 8; p < x_amax_n; p += 64) a = max(a, abs_bits(ap[p]));  // beyond 512 partials
      a = wave_max_u32(a);
      if (lane == 0 && mm < M) {
        s_amax[mm] = __uint_as_float(a);
        s_xs[mm] = x_scale(__uint_as_float(a));
      }
    }
    __syncthreads();
  } else if (PRO == 0 && QX) {
    uint32_t am[kMaxM];
#pragma unroll
    for (int mm = 0; mm < kMaxM; ++mm) {
      const uint32_t w4[4] = {xv[mm].x, xv[mm].y, xv[mm].z, xv[mm].w};
      am[mm] = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) am[mm] = bf_abs_max(am[mm], w4[i]);
    }
    for (int cc = tid * 8 + NT * 8; cc < K; cc += NT * 8) {  // rows longer than one pass
      uint4 xr[kMaxM];
#pragma unroll
      for (int mm = 0; mm < kMaxM; ++mm)
        xr[mm] = *reinterpret_cast<const uint4*>(x + (int64_t)min(mm, M - 1) * x_s + cc);
#pragma unroll
      for (int mm = 0; mm < kMaxM; ++mm) {
        const uint32_t w4[4] = {xr[mm].x, xr[mm].y, xr[mm].z, xr[mm].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) am[mm] = bf_abs_max(am[mm], w4[i]);
      }
    }
#pragma unroll
    for (int mm = 0; mm < kMaxM; ++mm) {
      if (mm >= M) break;
      const uint32_t w = wave_max_u32(am[mm]);
      if (lane == 0) s_am[mm][wave] = w;
    }
    __syncthreads();
    if (tid < M) {
      uint32_t a = 0;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) a = max(a, s_am[tid][w2]);
      s_amax[tid] = __uint_as_float(a);
      s_xs[tid] = x_scale(__uint_as_float(a));
    }
    __syncthreads();
  } else if (PRO == 2) {
    // the row's sum of f^2 from the producer's strips (x_amax [M, strips]),
    // each lane summing strips lane, lane + 64, ..., then the wave
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int mm = wave + rr * NW;
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < kStatLoads; ++j) ss += (lane + 64 * j < x_amax_n) ? sv[rr][j] : 0.0f;
      const float* sp = x_amax + (int64_t)min(mm, M - 1) * x_amax_s;
      for (int s2 = lane + 64 * kStatLoads; s2 < x_amax_n; s2 += 64) ss += sp[s2];
      ss = wave_sum(ss);
      if (lane == 0 && mm < M) s_inv[mm] = rsqrtf(ss / (float)K + eps);  // torch.rsqrt (layernorm.py:38)
    }
    __syncthreads();
  } else if (PRO == 1 || QX) {
    for (int m = wave; m < M; m += NW) {
      float inv, xs;
      row_stats<PRO, QX>(x + (int64_t)m * x_s, (PRO == 1 && res) ? res + (int64_t)m * res_s : nullptr, norm_w, K,
                         eps, qx_torch, lane, (res_out && blockIdx.x == 0) ? res_out + (int64_t)m * ro_s : nullptr, &inv, &xs);
      if (lane == 0) {
        s_inv[m] = inv;
        s_xs[m] = xs;
      }
    }
    __syncthreads();
  }

  if (PRO == 1 && has_row) inv = s_inv[c];
  if constexpr (PRO == 2) {
#pragma unroll
    for (int t = 0; t < kFChunks; ++t) fq_inv[t] = s_inv[min(fq_row + kRq * t, kActRows - 1)];
  }
  if (QX && has_row && !amax_one) {
    xsc = s_xs[c];
    if constexpr (F8) xfin = fp8_row_finite(s_amax[c], xsc);
  }
  // group i + 1 loads while group i computes
  for (int kb0 = kw0; kb0 < kend; kb0 += 2 * G) {
    const bool odd = kb0 + G < kend;
    if (!kEarly2 && odd) load(kb0 + G, b1);
    compute(kb0, b0);
    if (kb0 + 2 * G < kend) load(kb0 + 2 * G, b0);
    if (odd) {
      compute(kb0 + G, b1);
      if (kEarly2 && kb0 + 3 * G < kend) load(kb0 + 3 * G, b1);
    }
  }

  // EPI 4: the residual of this lane's four columns, loaded before the
  // reduction and the split handoff (only the finishing workgroup uses it)
  // (rows clamped in bounds instead of a load under a lane-dependent branch)
  uint2 rv4 = uint2{0u, 0u};
  if (EPI == 4 && wave == 0)
    rv4 = *reinterpret_cast<const uint2*>(res + (int64_t)min(lane & 15, M - 1) * res_s + n0 + 4 * (lane >> 4));
  // ---- reduce the waves' C fragments; lane l holds C[n = 4*(l/16) + r][m = l%16]
#pragma unroll
  for (int a = 0; a < NA; ++a) s_acc[a][wave][lane] = acc[a];
  __syncthreads();
  if (wave != 0) return;
  f32x4 t[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    t[a] = s_acc[a][0][lane];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) {
      const f32x4 o = s_acc[a][w2][lane];
      t[a][0] += o[0];
      t[a][1] += o[1];
      t[a][2] += o[2];
      t[a][3] += o[3];
    }
  }
  if (EPI == 3) {
    // split partials for the consumer to sum (no merge here): ws[ks][m][n]; the
    // consumer applies the row scale 1/x_s[m] (one workgroup publishes it) and
    // the weight's column scale after the sum, as the merge below does
    const int mm = lane & 15;
    if (mm < M) {
      float* dst = ws + ((int64_t)ks * M + mm) * n_out + n0 + 4 * (lane >> 4);
      *reinterpret_cast<f32x4*>(dst) = t[0];
    }
    if (row_scale_out && strip == 0 && ks == 0 && lane < M) row_scale_out[lane] = QX ? 1.0f / s_xs[lane] : 1.0f;
    return;
  }
  if (ksplit > 1) {
    // split-K: publish this split's fragments (agent-coherent stores), the last
    // split of the strip to arrive sums them all
    float* mine = ws + ((int64_t)strip * ksplit + ks) * (NA * 256);
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r) store_agent(mine + a * 256 + lane * 4 + r, t[a][r]);
    // handoff (fdms_common.h): stores completed before the ticket, loads after it
    handoff_release();
    if (lane == 0) s_last = (ticket_add(&counters[strip]) == ksplit - 1);
    __builtin_amdgcn_wave_barrier();
    if (!s_last) return;
    handoff_acquire();
    const float* all = ws + (int64_t)strip * ksplit * (NA * 256);
#pragma unroll
    for (int a = 0; a < NA; ++a) t[a] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ksplit; s0 += 4) {
      float v[4][NA][4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[j][a][r] = (s0 + j < ksplit) ? load_agent(all + (s0 + j) * (NA * 256) + a * 256 + lane * 4 + r) : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int r = 0; r < 4; ++r) t[a][r] += v[j][a][r];
    }
    if (lane == 0) __hip_atomic_store(&counters[strip], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const int m = lane & 15;
  if (EPI == 2) {
    // greedy head: the strip's best score per row (torch.argmax order), as the
    // reference scores it -- bf16 logits for bf16 / INT4 weights and for FP8
    // weights at more than one row (forward().argmax(), embed_head.py:543-598),
    // fp32 scores for the FP8 row-1 argmax (embed_head.py:96-144)
    constexpr int kNone = 0x7FFFFFFF;
    float bv = 0.0f;
    int bi = kNone;
    if (m < M) {
      const float xsi2 = QX ? 1.0f / s_xs[m] : 1.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = n0 + 4 * (lane >> 4) + r;
        float v;
        if (is_fp8<WT>() && !bf16_scores) {
          v = t[0][r] * xsi2 * w_scale_inv[n];
          if (bias) v += ld<bf16_t>(bias + n);
        } else if (is_fp8<WT>()) {
          v = rbf(t[0][r] * xsi2 * w_scale_inv[n]);
          if (bias) v = rbf(v + ld<bf16_t>(bias + n));
        } else if (is_int4<WT>()) {
          // INT4 logits: the bf16 matmul result, then the bias in bf16
          // (linear.py:475-477)
          v = rbf(t[0][r]);
          if (bias) v = rbf(v + ld<bf16_t>(bias + n));
        } else {
          v = QX ? t[0][r] * xsi2 : t[0][r];
          v = rbf(v + (bias ? ld<bf16_t>(bias + n) : 0.0f));
        }
        if (bi == kNone || argmax_better(v, n, bv, bi)) {
          bv = v;
          bi = n;
        }
      }
    }
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (oi != kNone && (bi == kNone || argmax_better(ov, oi, bv, bi))) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane < 16 && m < M) {
      part_val[(int64_t)m * strips + strip] = bv;
      part_idx[(int64_t)m * strips + strip] = bi;
    }
    return;
  }
  const bool row_ok = m < M;
  const float xsi = (QX && row_ok) ? 1.0f / s_xs[m] : 1.0f;
  auto finalize = [&](float acc_v, int n) {
    float v;
    if (is_fp8<WT>() || is_int4<WT>() || QX) {  // matmul rounded to bf16, then the bias
      v = acc_v * xsi;
      if (is_fp8<WT>()) v *= w_scale_inv[n];
      v = rbf(v);
      if (bias) v = rbf(v + ld<bf16_t>(bias + n));
    } else {
      v = rbf(acc_v + (bias ? ld<bf16_t>(bias + n) : 0.0f));
    }
    return v;
  };
  if (EPI == 4) {
    // f = fp32(v) + fp32(residual): fp32 rows to y, bf16(f) to residual_out,
    // the strip's sum of f^2 per row to amax_out[m][strip].  Lane l holds
    // columns 4 (l / 16) .. + 3 of row l % 16: the sum runs over those four,
    // then over lanes l ^ 16 and l ^ 32
    const int nc = n0 + 4 * (lane >> 4);
    float f[4];
    const float rf[4] = {bf_lo(rv4.x), bf_hi(rv4.x), bf_lo(rv4.y), bf_hi(rv4.y)};
    float ss = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f[r] = finalize(t[0][r], nc + r) + rf[r];
      ss += f[r] * f[r];
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (row_ok) {
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(y) + (int64_t)m * y_s + nc) = f32x4{f[0], f[1], f[2], f[3]};
      *reinterpret_cast<uint2*>(res_out + (int64_t)m * ro_s + nc) = uint2{pack2(f[0], f[1]), pack2(f[2], f[3])};
      if (lane < 16) amax_out[(int64_t)m * strips + strip] = ss;
    }
    return;
  }
  uint32_t vmax = 0;  // the row's max |output| over this strip, as abs_bits (rows >= M hold x = 0)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int n = n0 + 4 * (lane >> 4) + r;
    float v;
    if (EPI == 1) {
      const float gt = finalize(t[0][r], n);
      const float up = finalize(t[NA - 1][r], n + n_out);
      v = rbf(silu(gt) * up);
    } else {
      v = finalize(t[0][r], n);
    }
    const __bf16 vb = (__bf16)v;
    vmax = max(vmax, abs_bits((float)vb));
    if (row_ok) y[(int64_t)m * y_s + n].bits = __builtin_bit_cast(uint16_t, vb);
  }
  if (EPI <= 1 && amax_out) {
    // per-strip row amax (NaN propagating) for the consumer's activation
    // quantisation: lanes l, l ^ 16, l ^ 32, l ^ 48 hold the same row
    vmax = max(vmax, (uint32_t)__shfl_xor((int)vmax, 16));
    vmax = max(vmax, (uint32_t)__shfl_xor((int)vmax, 32));
    if (lane < 16 && row_ok) amax_out[(int64_t)m * strips + strip] = __uint_as_float(vmax);
  }
}

namespace {

struct LinArgs {
  const bf16_t* x; int64_t x_s; int M, K; const void* w; int64_t w_s; const float* wsi; const bf16_t* bias;
  const bf16_t* norm_w; float eps; const bf16_t* res; int64_t res_s; bf16_t* res_out; int64_t ro_s;
  bf16_t* y; int64_t y_s; int n_out, strips, ksplit; float* ws; int* counters; float* pval; int* pidx;
  const uint32_t* g_sz = nullptr; int group = 1; int64_t g_s = 0;
  int qx_torch = 0; int bf16_scores = 1;
  const float* x_amax = nullptr; int x_amax_n = 0; int64_t x_amax_s = 0; float* amax_out = nullptr;
  float* row_scale_out = nullptr;
};

template <typename WT, int PRO, bool QX, int EPI, bool XQ = false>
void launch_linear(int nw, dim3 grid, hipStream_t st, const LinArgs& a) {
  const WT* w = (const WT*)a.w;
  // k-blocks per double-buffered group (register budget: the RMSNorm prologue
  // also holds the residual and norm weight of each k-block, the activation
  // statistics hold their loads while both first groups are in flight)
  constexpr int U = (PRO == 1 || PRO == 2 || (QX && PRO == 0) || std::is_same_v<WT, u4x2_t>) ? 2 : 4;
#define FDMS_LIN_ARGS a.x, a.x_s, a.M, a.K, w, a.w_s, a.wsi, a.bias, a.norm_w, a.eps, a.res, a.res_s, a.res_out, \
                      a.ro_s, a.y, a.y_s, a.n_out, a.strips, a.ksplit, a.ws, a.counters, a.pval, a.pidx, \
                      a.g_sz, a.group, a.g_s, a.qx_torch, a.bf16_scores, a.x_amax, a.x_amax_n, \
                      a.x_amax_s, a.amax_out, a.row_scale_out
  if (nw == 8) {
    hipLaunchKernelGGL((linear_small_m_kernel<WT, PRO, QX, EPI, 8, U, XQ>), grid, dim3(512), 0, st, FDMS_LIN_ARGS);
  } else {
    hipLaunchKernelGGL((linear_small_m_kernel<WT, PRO, QX, EPI, 4, U, XQ>), grid, dim3(256), 0, st, FDMS_LIN_ARGS);
  }
#undef FDMS_LIN_ARGS
}

template <typename WT>
void dispatch_linear(int prologue, int qx, int epi, int nw, dim3 grid, hipStream_t st, const LinArgs& a) {
#define FDMS_LIN_E(P, Q)                                    \
  if (epi == 2) launch_linear<WT, P, Q, 2>(nw, grid, st, a); \
  else if (epi) launch_linear<WT, P, Q, 1>(nw, grid, st, a); \
  else launch_linear<WT, P, Q, 0>(nw, grid, st, a)
#define FDMS_LIN_Q(P) \
  if (qx) { FDMS_LIN_E(P, true); } else { FDMS_LIN_E(P, false); }
  if (prologue == 1) {
    FDMS_LIN_Q(1);
  } else {
    FDMS_LIN_Q(0);
  }
#undef FDMS_LIN_E
#undef FDMS_LIN_Q
}

}  // namespace

FDMS_EXPORT int fdms_linear_small_m(const void* x, int64_t x_stride, int m, int k, const void* w, int w_dtype,
                                    int64_t w_stride, const float* w_scale_inv, const void* bias, int n, int prologue,
                                    const void* norm_weight, float eps, const void* residual, int64_t res_stride,
                                    void* residual_out, int64_t res_out_stride, int quantize_x, int epilogue,
                                    int k_splits, float* workspace, int* counters, void* y, int64_t y_stride,
                                    const float* x_amax, int x_amax_n, int64_t x_amax_stride, float* amax_out,
                                    float* row_scale_out, int x_dtype, void* stream) {
  if (m < 0 || m > kMaxM || k <= 0 || n < 0 || prologue < 0 || prologue > 2 || epilogue < 0 || epilogue > 4 ||
      epilogue == 2 || quantize_x < 0 || quantize_x > 2)
    return (int)hipErrorInvalidValue;
  if (epilogue == 3 && (prologue != 0 || bias || !workspace)) return (int)hipErrorInvalidValue;
  // prologue 2: fp32 rows f and their producer's per-strip sums of f^2 in x_amax
  const bool stats_in = prologue == 2;
  // (one sum per 16-column producer strip: x_amax_n = k / 16, all summed into the norm)
  if (stats_in && (x_dtype != kF32 || quantize_x != 0 || !x_amax || x_amax_n != k / 16 || k % 16 ||
                   (m > 1 && x_amax_stride < x_amax_n) || epilogue > 1))
    return (int)hipErrorInvalidValue;
  // the producer's row amax replaces the activation statistics pass (no prologue)
  if (x_amax && !stats_in && (prologue != 0 || quantize_x == 0 || x_amax_n < 1 || (m > 1 && x_amax_stride < x_amax_n)))
    return (int)hipErrorInvalidValue;
  // epilogue 4: the residual add (residual in, residual_out may be the same
  // rows), fp32 rows to y, the strips' sums of squares to amax_out
  const bool stats_out = epilogue == 4;
  if (stats_out && (prologue != 0 || quantize_x != 0 || !residual || !residual_out || !amax_out))
    return (int)hipErrorInvalidValue;
  if ((amax_out && epilogue > 1 && !stats_out) || (row_scale_out && epilogue != 3)) return (int)hipErrorInvalidValue;
  // an activation quantised by its producer: e4m3fn codes with their row amax
  const bool xq = x_dtype == kFP8;
  if ((x_dtype != kBF16 && !xq && !stats_in) || (xq && (w_dtype != kFP8 || quantize_x == 0 || !x_amax)))
    return (int)hipErrorInvalidValue;
  if (m == 0 || n == 0) return 0;
  if (!x || !w || !y || (prologue >= 1 && !norm_weight)) return (int)hipErrorInvalidValue;
  if (w_dtype != kBF16 && w_dtype != kFP8) return (int)hipErrorInvalidValue;
  if (w_dtype == kFP8 && !w_scale_inv) return (int)hipErrorInvalidValue;
  if (prologue != 1 && !stats_out && (residual || residual_out)) return (int)hipErrorInvalidValue;
  // other workgroups still read x / residual while workgroup 0 writes residual_out
  if (prologue == 1 && residual_out && (residual_out == residual || residual_out == x)) return (int)hipErrorInvalidValue;
  if (stats_out && (residual_out == x || residual == x)) return (int)hipErrorInvalidValue;
  if (y == x || (residual && y == residual) || (residual_out && y == residual_out)) return (int)hipErrorInvalidValue;
  // n = weight rows; epilogue 1 pairs row n0 with n0 + n/2 and writes n/2 columns
  const int n_out = epilogue == 1 ? n / 2 : n;
  if (n_out % 16 || (epilogue == 1 && n % 2)) return (int)hipErrorInvalidValue;
  if (k_splits < 1 || k_splits > 64) return (int)hipErrorInvalidValue;
  if (k_splits > 1 && epilogue != 3 && (!workspace || !counters)) return (int)hipErrorInvalidValue;
  const int kc = k / k_splits;
  if (k % k_splits) return (int)hipErrorInvalidValue;
  // four waves per workgroup (eight, the override, measured 5 % slower on
  // the 8B decode shapes and 0.8 % on the 1B ones)
  int nw = 4;
  if (const char* e = std::getenv("FASTDMS_AMD_LIN_WAVES")) {  // tuning override
    const int v = std::atoi(e);
    if ((v == 4 || v == 8) && kc % (kKB * v) == 0) nw = v;
  }
  if (kc % (kKB * nw)) return (int)hipErrorInvalidValue;  // whole k-blocks per wave
  const int wsz = w_dtype == kFP8 ? 1 : 2;
  auto al16 = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
  if (!al16(x) || !al16(w) || (x_stride * (xq ? 1 : stats_in ? 4 : 2)) % 16 || (w_stride * wsz) % 16)
    return (int)hipErrorInvalidValue;
  if (stats_in && !al16(norm_weight)) return (int)hipErrorInvalidValue;
  if (stats_out && (!al16(y) || y_stride % 4 || (uintptr_t)residual % 8 || (uintptr_t)residual_out % 8 ||
                    res_stride % 4 || res_out_stride % 4 || res_stride < n || res_out_stride < n))
    return (int)hipErrorInvalidValue;
  if (prologue == 1 && (!al16(norm_weight) || (residual && (!al16(residual) || (res_stride * 2) % 16)) ||
                        (residual_out && (!al16(residual_out) || (res_out_stride * 2) % 16))))
    return (int)hipErrorInvalidValue;
  if (x_stride < k || w_stride < k || y_stride < n_out) return (int)hipErrorInvalidValue;
  if (!stats_out && ((residual && res_stride < k) || (residual_out && res_out_stride < k)))
    return (int)hipErrorInvalidValue;
  const int strips = n_out / 16;
  const int64_t blocks = (int64_t)((strips + kXcds - 1) / kXcds) * kXcds * k_splits;
  if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks);
  LinArgs a{(const bf16_t*)x, x_stride, m, k, w, w_stride, w_scale_inv, (const bf16_t*)bias,
            (const bf16_t*)norm_weight, eps, (const bf16_t*)residual, res_stride, (bf16_t*)residual_out,
            res_out_stride, (bf16_t*)y, y_stride, n_out, strips, k_splits, workspace, counters, nullptr,
            nullptr};
  a.qx_torch = quantize_x == 2;
  a.x_amax = x_amax;
  a.x_amax_n = x_amax_n;
  a.x_amax_s = x_amax_stride;
  a.amax_out = amax_out;
  a.row_scale_out = row_scale_out;
  if (stats_in) {
    if (w_dtype == kFP8) {
      if (epilogue == 1) launch_linear<fp8_t, 2, false, 1>(nw, grid, (hipStream_t)stream, a);
      else launch_linear<fp8_t, 2, false, 0>(nw, grid, (hipStream_t)stream, a);
    } else {
      if (epilogue == 1) launch_linear<bf16_t, 2, false, 1>(nw, grid, (hipStream_t)stream, a);
      else launch_linear<bf16_t, 2, false, 0>(nw, grid, (hipStream_t)stream, a);
    }
  } else if (stats_out) {
    if (w_dtype == kFP8) launch_linear<fp8_t, 0, false, 4>(nw, grid, (hipStream_t)stream, a);
    else launch_linear<bf16_t, 0, false, 4>(nw, grid, (hipStream_t)stream, a);
  } else if (xq) {
    if (epilogue == 3) launch_linear<fp8_t, 0, true, 3, true>(nw, grid, (hipStream_t)stream, a);
    else if (epilogue == 1) launch_linear<fp8_t, 0, true, 1, true>(nw, grid, (hipStream_t)stream, a);
    else launch_linear<fp8_t, 0, true, 0, true>(nw, grid, (hipStream_t)stream, a);
  } else if (epilogue == 3) {
    if (w_dtype == kFP8 && quantize_x) launch_linear<fp8_t, 0, true, 3>(nw, grid, (hipStream_t)stream, a);
    else if (w_dtype == kFP8) launch_linear<fp8_t, 0, false, 3>(nw, grid, (hipStream_t)stream, a);
    else if (quantize_x) launch_linear<bf16_t, 0, true, 3>(nw, grid, (hipStream_t)stream, a);
    else launch_linear<bf16_t, 0, false, 3>(nw, grid, (hipStream_t)stream, a);
  } else if (w_dtype == kFP8) {
    dispatch_linear<fp8_t>(prologue, quantize_x, epilogue, nw, grid, (hipStream_t)stream, a);
  } else {
    dispatch_linear<bf16_t>(prologue, quantize_x, epilogue, nw, grid, (hipStream_t)stream, a);
  }
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Second stage of the greedy head: per row, the best of the strips' partial
// (score, index) pairs in torch.argmax order (embed_head.py:147-160).
__global__ __launch_bounds__(1024) void argmax_partials_kernel(const float* __restrict__ pval,
                                                               const int* __restrict__ pidx, int strips,
                                                               int64_t* __restrict__ out) {
  constexpr int kNone = 0x7FFFFFFF;
  __shared__ float s_v[1024 / kWave];
  __shared__ int s_i[1024 / kWave];
  const int64_t row = blockIdx.x;
  float bv = 0.0f;
  int bi = kNone;
  // kU strips per thread per pass, all loads issued before the first compare
  // (clamped to the last strip; the duplicates cannot change the argmax)
  constexpr int kU = 8;
  for (int j0 = threadIdx.x; j0 < strips; j0 += 1024 * kU) {
    float v[kU];
    int ix[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = min(j0 + u * 1024, strips - 1);
      v[u] = pval[row * strips + j];
      ix[u] = pidx[row * strips + j];
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (bi == kNone || argmax_better(v[u], ix[u], bv, bi)) {
        bv = v[u];
        bi = ix[u];
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (oi != kNone && (bi == kNone || argmax_better(ov, oi, bv, bi))) {
      bv = ov;
      bi = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = bv;
    s_i[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int wv = 1; wv < 1024 / kWave; ++wv) {
      if (s_i[wv] != kNone && (bi == kNone || argmax_better(s_v[wv], s_i[wv], bv, bi))) {
        bv = s_v[wv];
        bi = s_i[wv];
      }
    }
    out[row] = bi;
  }
}

FDMS_EXPORT int fdms_linear_argmax_small_m(const void* x, int64_t x_stride, int m, int k, const void* w,
                                           int w_dtype, int64_t w_stride, const float* w_scale_inv,
                                           const void* bias, int n, int quantize_x, int bf16_scores, int k_splits,
                                           float* workspace, int* counters, float* part_val, int* part_idx,
                                           int64_t* out_tokens, void* stream) {
  if (m < 0 || m > kMaxM || k <= 0 || n < 0 || quantize_x < 0 || quantize_x > 2) return (int)hipErrorInvalidValue;
  if (m == 0) return 0;
  if (n == 0 || !x || !w || !part_val || !part_idx || !out_tokens) return (int)hipErrorInvalidValue;
  if (w_dtype != kBF16 && w_dtype != kFP8) return (int)hipErrorInvalidValue;
  if (w_dtype == kFP8 && !w_scale_inv) return (int)hipErrorInvalidValue;
  if (n % 16 || k_splits < 1 || k_splits > 64 || k % k_splits) return (int)hipErrorInvalidValue;
  if (k_splits > 1 && (!workspace || !counters)) return (int)hipErrorInvalidValue;
  const int kc = k / k_splits;
  // four waves per workgroup (eight, the override, measured 5 % slower on
  // the 8B decode shapes and 0.8 % on the 1B ones)
  int nw = 4;
  if (const char* e = std::getenv("FASTDMS_AMD_LIN_WAVES")) {  // tuning override
    const int v = std::atoi(e);
    if ((v == 4 || v == 8) && kc % (kKB * v) == 0) nw = v;
  }
  if (kc % (kKB * nw)) return (int)hipErrorInvalidValue;
  const int wsz = w_dtype == kFP8 ? 1 : 2;
  if (((uintptr_t)x % 16) || ((uintptr_t)w % 16) || (x_stride * 2) % 16 || (w_stride * wsz) % 16 ||
      x_stride < k || w_stride < k)
    return (int)hipErrorInvalidValue;
  const int strips = n / 16;
  const int64_t blocks = (int64_t)((strips + kXcds - 1) / kXcds) * kXcds * k_splits;
  if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  LinArgs a{(const bf16_t*)x, x_stride, m, k, w, w_stride, w_scale_inv, (const bf16_t*)bias, nullptr, 0.0f,
            nullptr, 0, nullptr, 0, nullptr, 0, n, strips, k_splits, workspace, counters, part_val, part_idx};
  a.qx_torch = quantize_x == 2;
  a.bf16_scores = bf16_scores != 0;
  const dim3 grid((unsigned)blocks);
  if (w_dtype == kFP8) {
    dispatch_linear<fp8_t>(0, quantize_x, 2, nw, grid, (hipStream_t)stream, a);
  } else {
    dispatch_linear<bf16_t>(0, quantize_x, 2, nw, grid, (hipStream_t)stream, a);
  }
  FDMS_LAUNCH_CHECK();
  hipLaunchKernelGGL(argmax_partials_kernel, dim3((unsigned)m), dim3(1024), 0, (hipStream_t)stream, part_val,
                     part_idx, strips, out_tokens);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Re-ranking of the INT4 head's top-k candidates in FP8 (embed_head.py:214-302):
// one workgroup per row; the activation is quantised as the row-1 kernels do
// (448/amax divided, RNE to e4m3fn), each wave scores candidates t = wave,
// wave + 4, ... (fp32 products of e4m3 values are exact), and thread 0 picks
// the best, the lowest id on ties; an id outside [0, N) scores -inf.
__global__ __launch_bounds__(256) void fp8_rerank_topk_kernel(const bf16_t* __restrict__ x, int64_t x_s, int K,
                                                              const uint8_t* __restrict__ w, int64_t w_s,
                                                              const float* __restrict__ w_scale_inv, int N,
                                                              const int64_t* __restrict__ cand, int topk,
                                                              int64_t* __restrict__ out) {
  __shared__ float s_red[4];
  __shared__ float s_score[32];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const bf16_t* xr = x + row * x_s;
  float am = 0.0f;
  for (int k = tid * 8; k < K; k += 256 * 8) {
    float f[8];
    load_sum8(xr + k, nullptr, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(f[i]));
  }
  am = wave_max(am);
  if (lane == 0) s_red[wave] = am;
  __syncthreads();
  am = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  const float xs = am > 0.0f ? kFp8Max / am : 1.0f;
  const float xsi = 1.0f / xs;
  for (int t = wave; t < topk; t += 4) {
    const int64_t id = cand[row * topk + t];
    float score = -INFINITY;
    if (id >= 0 && id < N) {
      const uint8_t* wr = w + id * w_s;
      float acc = 0.0f;
      for (int k = lane * 16; k < K; k += 64 * 16) {
        const uint4 wv = *reinterpret_cast<const uint4*>(wr + k);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
        float f[16];
        load_sum8(xr + k, nullptr, f);
        load_sum8(xr + k + 8, nullptr, f + 8);
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const uint32_t q8 = f32x4_to_fp8x4(f[4 * i4] * xs, f[4 * i4 + 1] * xs, f[4 * i4 + 2] * xs,
                                             f[4 * i4 + 3] * xs);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc += fp8_to_f32((q8 >> (8 * i)) & 0xFFu) * fp8_to_f32((ww[i4] >> (8 * i)) & 0xFFu);
        }
      }
      score = wave_sum(acc) * xsi * w_scale_inv[id];
    }
    if (lane == 0) s_score[t] = score;
  }
  __syncthreads();
  if (tid == 0) {
    float best = -INFINITY;
    int64_t bid = N;
    for (int t = 0; t < topk; ++t) {
      const int64_t id = cand[row * topk + t];
      const float v = s_score[t];
      if (v > best || (v == best && id < bid)) {
        best = v;
        bid = id;
      }
    }
    out[row] = bid;
  }
}

FDMS_EXPORT int fdms_fp8_rerank_topk(const void* x, int64_t x_stride, int rows, int k, const void* w_fp8,
                                     int64_t w_stride, const float* w_scale_inv, int n, const int64_t* candidates,
                                     int topk, int64_t* out_tokens, void* stream) {
  if (rows < 0 || k <= 0 || n <= 0 || (topk != 2 && topk != 4 && topk != 8 && topk != 16 && topk != 32))
    return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!x || !w_fp8 || !w_scale_inv || !candidates || !out_tokens) return (int)hipErrorInvalidValue;
  if (k % 16 || ((uintptr_t)x % 16) || ((uintptr_t)w_fp8 % 16) || (x_stride * 2) % 16 || w_stride % 16 ||
      x_stride < k || w_stride < k)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(fp8_rerank_topk_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)x, x_stride, k, (const uint8_t*)w_fp8, w_stride, w_scale_inv, n, candidates,
                     topk, out_tokens);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// C5 — W4A16 decode linear: the small-M kernel with INT4 weights (no
// activation quantisation or prologue; epilogue 0 plain, 1 SiLU*up, 2 greedy,
// 3 fp32 split partials into workspace for the next RMSNorm to sum).
FDMS_EXPORT int fdms_linear_int4_small_m(const void* x, int64_t x_stride, int m, int k, const void* w_packed,
                                         int64_t w_stride_bytes, const void* scale_zeros, int group_size,
                                         int64_t sz_stride, const void* bias, int n, int epilogue,
                                         int k_splits, float* workspace, int* counters, float* part_val,
                                         int* part_idx, int64_t* out_tokens, void* y, int64_t y_stride,
                                         void* stream) {
  if (m < 0 || m > kMaxM || k <= 0 || n < 0 || epilogue < 0 || epilogue > 3) return (int)hipErrorInvalidValue;
  if (m == 0 || n == 0) return 0;
  if (!x || !w_packed || !scale_zeros || ((uintptr_t)scale_zeros % 4)) return (int)hipErrorInvalidValue;
  // epilogue 3: workspace[split][row][n] fp32 partials, no bias (the consumer adds in split order)
  if (epilogue == 3 && (bias || !workspace)) return (int)hipErrorInvalidValue;
  // a lane group's 32 columns of a 128-column k-block lie in one group
  if (group_size < 32 || (group_size & (group_size - 1)) || k % group_size || sz_stride < n)
    return (int)hipErrorInvalidValue;
  if (epilogue == 2 ? (!part_val || !part_idx || !out_tokens) : (epilogue != 3 && !y)) return (int)hipErrorInvalidValue;
  const int n_out = epilogue == 1 ? n / 2 : n;
  if (n_out % 16 || (epilogue == 1 && n % 2)) return (int)hipErrorInvalidValue;
  if (k_splits < 1 || k_splits > 64 || k % k_splits || (k_splits > 1 && epilogue != 3 && (!workspace || !counters)))
    return (int)hipErrorInvalidValue;
  const int kc = k / k_splits;
  // four waves per workgroup (eight, the override, measured 5 % slower on
  // the 8B decode shapes and 0.8 % on the 1B ones)
  int nw = 4;
  if (const char* e = std::getenv("FASTDMS_AMD_LIN_WAVES")) {  // tuning override
    const int v = std::atoi(e);
    if ((v == 4 || v == 8) && kc % (kKB * v) == 0) nw = v;
  }
  if (kc % (kKB * nw)) return (int)hipErrorInvalidValue;
  if (((uintptr_t)x % 16) || ((uintptr_t)w_packed % 16) || (x_stride * 2) % 16 || w_stride_bytes % 16 ||
      x_stride < k || w_stride_bytes * 2 < k || (epilogue < 2 && y_stride < n_out))
    return (int)hipErrorInvalidValue;
  if (y && (y == x)) return (int)hipErrorInvalidValue;
  const int strips = n_out / 16;
  const int64_t blocks = (int64_t)((strips + kXcds - 1) / kXcds) * kXcds * k_splits;
  if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  LinArgs a{(const bf16_t*)x, x_stride, m, k, w_packed, w_stride_bytes, nullptr, (const bf16_t*)bias, nullptr, 0.0f,
            nullptr, 0, nullptr, 0, (bf16_t*)y, y_stride, n_out, strips, k_splits, workspace, counters, part_val,
            part_idx};
  a.g_sz = (const uint32_t*)scale_zeros;
  a.group = group_size;
  a.g_s = sz_stride;
  const dim3 grid((unsigned)blocks);
  const hipStream_t st = (hipStream_t)stream;
  if (epilogue == 3) launch_linear<u4x2_t, 0, false, 3>(nw, grid, st, a);
  else if (epilogue == 2) launch_linear<u4x2_t, 0, false, 2>(nw, grid, st, a);
  else if (epilogue == 1) launch_linear<u4x2_t, 0, false, 1>(nw, grid, st, a);
  else launch_linear<u4x2_t, 0, false, 0>(nw, grid, st, a);
  FDMS_LAUNCH_CHECK();
  if (epilogue == 2) {
    hipLaunchKernelGGL(argmax_partials_kernel, dim3((unsigned)m), dim3(1024), 0, st, part_val, part_idx, strips,
                       out_tokens);
    FDMS_LAUNCH_CHECK();
  }
  return 0;
}

// C5 — INT4 group quantisation of weight rows [N, K] (linear.py:414-459):
// symmetric s = amax/7 (1 for a zero group), zero = 0, q = clamp(rint(w/s), -8, 7) + 8;
// asymmetric s = (max-min)/15 (1 if flat), zero = min + 8s (min if flat),
// q = clamp(rint((w - zero)/s + 8), 0, 15); q uses the fp32 scale / zero, the
// stored scale / zero are rounded to bf16 and written as the reference's
// scale_zeros [groups, N, 2] (linear.py:461-464; sz_s pairs between groups).
// One wave per (row, group).
template <typename TI>
__global__ __launch_bounds__(256) void quantize_int4_kernel(const TI* __restrict__ w, int64_t w_s, int k, int group,
                                                            int asym, uint8_t* __restrict__ out, int64_t out_s,
                                                            uint32_t* __restrict__ sz, int64_t sz_s,
                                                            int64_t total_groups) {
  const int64_t gid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gid >= total_groups) return;
  const int lane = threadIdx.x & 63;
  const int groups_per_row = k / group;
  const int64_t row = gid / groups_per_row;
  const int gi = (int)(gid - row * groups_per_row);
  const TI* src = w + row * w_s + (int64_t)gi * group;
  float mn = INFINITY, mx = -INFINITY, am = 0.0f;
  for (int j = lane; j < group; j += 64) {
    const float v = ld<TI>(src + j);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
    am = fmaxf(am, fabsf(v));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o));
    mx = fmaxf(mx, __shfl_xor(mx, o));
    am = fmaxf(am, __shfl_xor(am, o));
  }
  // amax / 7.0 and span / 15.0 as torch evaluates them on a GPU: a multiply by
  // the fp32 reciprocal of the scalar.
  float s, z;
  if (asym) {
    const float span = mx - mn;
    s = span > 0.0f ? span * (1.0f / 15.0f) : 1.0f;
    z = span > 0.0f ? mn + 8.0f * s : mn;
  } else {
    s = am > 0.0f ? am * (1.0f / 7.0f) : 1.0f;
    z = 0.0f;
  }
  uint8_t* dst = out + row * out_s + (int64_t)gi * (group / 2);
  for (int j = lane; j < group / 2; j += 64) {
    int q[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float v = ld<TI>(src + 2 * j + h);
      float r;
      if (asym) r = fminf(fmaxf(rintf((v - z) / s + 8.0f), 0.0f), 15.0f);
      else r = fminf(fmaxf(rintf(v / s), -8.0f), 7.0f) + 8.0f;
      q[h] = (int)r;
    }
    dst[j] = (uint8_t)(q[0] | (q[1] << 4));
  }
  if (lane == 0) sz[(int64_t)gi * sz_s + row] = f32_to_bf16(s) | (f32_to_bf16(z) << 16);
}

FDMS_EXPORT int fdms_quantize_int4_groups(const void* w, int w_dtype, int64_t w_stride, int64_t rows, int k,
                                          int group_size, int asymmetric, void* out_packed, int64_t out_stride,
                                          void* scale_zeros, int64_t sz_stride, void* stream) {
  if (rows < 0 || k <= 0 || group_size < 2 || group_size % 2 || k % group_size) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!w || !out_packed || !scale_zeros || ((uintptr_t)scale_zeros % 4) || w_stride < k || out_stride * 2 < k ||
      sz_stride < rows)
    return (int)hipErrorInvalidValue;
  const int64_t total = rows * (k / group_size);
  const int64_t blocks = (total + 3) / 4;
  if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  if (w_dtype == kBF16) {
    hipLaunchKernelGGL(quantize_int4_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)w, w_stride, k, group_size, asymmetric, (uint8_t*)out_packed, out_stride,
                       (uint32_t*)scale_zeros, sz_stride, total);
  } else if (w_dtype == kF32) {
    hipLaunchKernelGGL(quantize_int4_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const float*)w, w_stride, k, group_size, asymmetric, (uint8_t*)out_packed, out_stride,
                       (uint32_t*)scale_zeros, sz_stride, total);
  } else {
    return (int)hipErrorInvalidValue;
  }
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Per-row FP8 quantisation (linear.py:386-388, 813-823 for weight rows;
// 514-523, 683-694, 652-654 for activation rows): s = 448 / amax(row) (1 when
// the row is all zero), q = e4m3fn(v * s) rounded to nearest even, scale_inv =
// 1 / s.  torch_form selects how 448 / amax is rounded: the reference's torch
// expressions (weights, _fp8_linear) evaluate reciprocal(amax) * 448; its
// Triton kernels divide directly.  One workgroup per row.
template <typename TI>
__global__ __launch_bounds__(256) void quantize_fp8_rows_kernel(const TI* __restrict__ in, int64_t in_s, int k,
                                                                uint8_t* __restrict__ out, int64_t out_s,
                                                                float* __restrict__ scale_inv, int torch_form) {
  __shared__ float s_red[256 / kWave];
  const int64_t row = blockIdx.x;
  const TI* r = in + row * in_s;
  float amax = 0.0f;
  for (int j = threadIdx.x; j < k; j += 256) amax = fmaxf(amax, fabsf(ld<TI>(r + j)));
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  // torch's tensor expression 448 / amax is reciprocal(amax) * 448 (two roundings)
  const float sc = amax > 0.0f ? (torch_form ? (1.0f / amax) * kFp8Max : kFp8Max / amax) : 1.0f;
  uint8_t* o = out + row * out_s;
  if (k % 4 == 0 && (reinterpret_cast<uintptr_t>(o) & 3) == 0) {  // four codes per converter call
    for (int j = 4 * threadIdx.x; j < k; j += 4 * 256)
      *reinterpret_cast<uint32_t*>(o + j) = f32x4_to_fp8x4(ld<TI>(r + j) * sc, ld<TI>(r + j + 1) * sc,
                                                           ld<TI>(r + j + 2) * sc, ld<TI>(r + j + 3) * sc);
  } else {
    for (int j = threadIdx.x; j < k; j += 256) o[j] = (uint8_t)f32_to_fp8(ld<TI>(r + j) * sc);
  }
  if (threadIdx.x == 0) scale_inv[row] = 1.0f / sc;
}

// The same quantisation of bf16 rows in one pass: each thread holds C
// 16-byte chunks of the row (k <= 2048 C) in registers, loaded with clamped
// indices (a repeated chunk cannot change the maximum), and stores 8 codes
// per chunk; identical results to quantize_fp8_rows_kernel.
template <int C>
__global__ __launch_bounds__(256) void quantize_fp8_rows_vec_kernel(const bf16_t* __restrict__ in, int64_t in_s,
                                                                    int k, uint8_t* __restrict__ out, int64_t out_s,
                                                                    float* __restrict__ scale_inv, int torch_form) {
  __shared__ float s_red[256 / kWave];
  const int64_t row = blockIdx.x;
  const bf16_t* r = in + row * in_s;
  uint4 v[C];
#pragma unroll
  for (int c = 0; c < C; ++c)
    v[c] = *reinterpret_cast<const uint4*>(r + min(((int)threadIdx.x + c * 256) * 8, k - 8));
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      amax = fmaxf(fmaxf(amax, fabsf(__uint_as_float(w[i] << 16))), fabsf(__uint_as_float(w[i] & 0xFFFF0000u)));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  const float sc = amax > 0.0f ? (torch_form ? (1.0f / amax) * kFp8Max : kFp8Max / amax) : 1.0f;
  uint8_t* o = out + row * out_s;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int j = ((int)threadIdx.x + c * 256) * 8;
    if (j < k) {
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
      float f[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16) * sc;
        f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u) * sc;
      }
      *reinterpret_cast<uint2*>(o + j) = uint2{f32x4_to_fp8x4(f[0], f[1], f[2], f[3]), f32x4_to_fp8x4(f[4], f[5], f[6], f[7])};
    }
  }
  if (threadIdx.x == 0) scale_inv[row] = 1.0f / sc;
}

FDMS_EXPORT int fdms_quantize_fp8_rows(const void* in, int in_dtype, int64_t in_stride, int64_t rows, int k,
                                       void* out, int64_t out_stride, float* scale_inv, int torch_form,
                                       void* stream) {
  if (rows < 0 || k <= 0 || rows > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!in || !out || !scale_inv || in_stride < k || out_stride < k) return (int)hipErrorInvalidValue;
  // bf16 rows of 16-byte chunks up to 16384 columns: the one-pass kernel
  const bool vec = in_dtype == kBF16 && k % 8 == 0 && k <= 8 * 256 * 8 && (uintptr_t)in % 16 == 0 &&
                   in_stride % 8 == 0 && (uintptr_t)out % 8 == 0 && out_stride % 8 == 0;
  if (vec) {
    const int chunks = (k + 8 * 256 - 1) / (8 * 256);
#define FDMS_QFP8_VEC(CC)                                                                                        \
  hipLaunchKernelGGL(quantize_fp8_rows_vec_kernel<CC>, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, \
                     (const bf16_t*)in, in_stride, k, (uint8_t*)out, out_stride, scale_inv, torch_form)
    if (chunks == 1) FDMS_QFP8_VEC(1);
    else if (chunks == 2) FDMS_QFP8_VEC(2);
    else if (chunks <= 4) FDMS_QFP8_VEC(4);
    else FDMS_QFP8_VEC(8);
#undef FDMS_QFP8_VEC
  } else if (in_dtype == kBF16) {
    hipLaunchKernelGGL(quantize_fp8_rows_kernel<bf16_t>, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)in, in_stride, k, (uint8_t*)out, out_stride, scale_inv, torch_form);
  } else if (in_dtype == kF32) {
    hipLaunchKernelGGL(quantize_fp8_rows_kernel<float>, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                       (const float*)in, in_stride, k, (uint8_t*)out, out_stride, scale_inv, torch_form);
  } else {
    return (int)hipErrorInvalidValue;
  }
  FDMS_LAUNCH_CHECK();
  return 0;
}
