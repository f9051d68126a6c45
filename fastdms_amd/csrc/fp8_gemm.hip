// FP8 GEMM for prefill row counts on the gfx950 FP8 matrix cores: the
// reference's _fp8_linear for rows above the small-M kernels
// (fastdms/layers/linear.py:635-662: x quantised per row to e4m3fn, then
// torch._scaled_mm(xq, W8^T, scale_a = x_scale_inv, scale_b = w_scale_inv,
// out_dtype = bf16), bias added in bf16):
//
//   y[m, n] = bf16((sum_k xq[m, k] * w8[n, k]) * x_inv[m] * w_inv[n])
//   y[m, n] = bf16(y[m, n] + bias[n])                       (with a bias)
//
// The products of two e4m3 values are exact in fp32; the matrix cores
// accumulate them in fp32 (v_mfma_scale_f32_16x16x128_f8f6f4 with unit E8M0
// block scales), so the result differs from torch's only in summation order.
//
// Tiling: a workgroup computes a 128 x 128 tile of y with 4 waves of 64 x 64
// (4 x 4 MFMA tiles of 16 x 16 each, K = 128 per instruction).  Operands go
// straight from global memory into registers in the MFMA layout (lane group
// g of lane (g, c) holds bytes 32 g .. 32 g + 31 of a 128-byte k-block of row
// c), double-buffered: the next k-block is in flight while the current one
// multiplies.  Tiles are assigned XCD by XCD (block ids are dispatched round
// robin over the 8 XCDs), each XCD taking a contiguous run of tiles with n
// fastest, so an x row block is read into one XCD's L2 and reused there.
#include <cstdlib>

#include "fdms_common.h"

using namespace fdms;

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kGemmXcds = 8;

struct Frag {
  uint4 w[4][2];  // four 16-row weight tiles: 32 bytes of this lane's row
  uint4 x[4][2];  // four 16-row activation tiles
};

__device__ __forceinline__ i32x8 as_i32x8(const uint4& a, const uint4& b) {
  return i32x8{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// Bytes k .. k + 31 of each of the lane's rows (k = block start + 32 g).
// TAIL: the last, partial k-block; 16-byte chunks at or past K read as zero
// (their addresses are clamped to chunk 0, in bounds).
template <bool TAIL>
__device__ __forceinline__ void load_frag(Frag& f, const uint8_t* const* wp, const uint8_t* const* xp, int k,
                                          int K) {
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int kk = k + 16 * hh;
    const bool ok = !TAIL || kk < K;
    const int ka = ok ? kk : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 vw = *reinterpret_cast<const uint4*>(wp[i] + ka);
      const uint4 vx = *reinterpret_cast<const uint4*>(xp[i] + ka);
      f.w[i][hh] = ok ? vw : uint4{0u, 0u, 0u, 0u};
      f.x[i][hh] = ok ? vx : uint4{0u, 0u, 0u, 0u};
    }
  }
}

__device__ __forceinline__ void mma(f32x4 (&acc)[4][4], const Frag& f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const i32x8 a = as_i32x8(f.w[i][0], f.w[i][1]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, as_i32x8(f.x[j][0], f.x[j][1]), acc[i][j], 0,
                                                                   0, 0, 127, 0, 127);
  }
}

}  // namespace

template <bool BIAS, bool VEC_OUT>
__global__ __launch_bounds__(kThreads) void fp8_gemm_kernel(
    const uint8_t* __restrict__ x, int64_t x_s, const float* __restrict__ x_inv, const uint8_t* __restrict__ w,
    int64_t w_s, const float* __restrict__ w_inv, const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
    int64_t y_s, int M, int N, int K, int tiles_n, int total, int per_xcd) {
  const int lin = blockIdx.x;
  const int t = (lin % kGemmXcds) * per_xcd + lin / kGemmXcds;
  if (t >= total) return;  // uniform per workgroup
  const int tm = t / tiles_n, tn = t - (t / tiles_n) * tiles_n;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const int m0 = tm * kBM + (wave >> 1) * 64;
  const int n0 = tn * kBN + (wave & 1) * 64;
  // rows past M / N are read from the last row (in bounds) and never stored
  const uint8_t* wp[4];
  const uint8_t* xp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wp[i] = w + (int64_t)min(n0 + 16 * i + c, N - 1) * w_s;
    xp[i] = x + (int64_t)min(m0 + 16 * i + c, M - 1) * x_s;
  }
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kfull = K & ~(kBK - 1);
  const int kl = 32 * g;
  Frag fa, fb;
  if (kfull > 0) load_frag<false>(fa, wp, xp, kl, K);
  for (int k0 = 0; k0 < kfull; k0 += 2 * kBK) {  // two buffers, no register copies
    if (k0 + kBK < kfull) load_frag<false>(fb, wp, xp, k0 + kBK + kl, K);
    mma(acc, fa);
    if (k0 + kBK >= kfull) break;
    if (k0 + 2 * kBK < kfull) load_frag<false>(fa, wp, xp, k0 + 2 * kBK + kl, K);
    mma(acc, fb);
  }
  if (kfull < K) {
    load_frag<true>(fa, wp, xp, kfull + kl, K);
    mma(acc, fa);
  }

  // lane (g, c) holds C[n = n0 + 16 i + 4 g + r][m = m0 + 16 j + c]
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + 16 * j + c;
    if (m >= M) continue;
    const float xs = x_inv[m];
    bf16_t* yr = y + (int64_t)m * y_s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nb = n0 + 16 * i + 4 * g;
      if (nb >= N) continue;
      uint32_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = min(nb + r, N - 1);
        float v = acc[i][j][r] * xs * w_inv[n];
        if (BIAS) v = bf16_to_f32(f32_to_bf16(v)) + bf16_to_f32(bias[n].bits);
        o[r] = f32_to_bf16(v);
      }
      if (VEC_OUT && nb + 3 < N) {
        *reinterpret_cast<uint2*>(yr + nb) = uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) yr[nb + r].bits = (uint16_t)o[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large problems: 256 x 256 workgroup tiles, 4 waves of 128 x 128 (8 x 8 MFMA
// tiles, the accumulators in AGPRs), operands staged through LDS.  Each
// k-block (128 bytes of 256 x rows and 256 w rows, 64 KiB) is loaded by all
// 256 threads with coalesced 16-byte loads (8 threads per row), written to
// one of two LDS buffers, and read back by the waves in the MFMA layout; the
// global loads of block t + 2 are in flight while block t multiplies.  LDS
// rows are 128 bytes with the 16-byte chunks XOR-swizzled by row (chunk q of
// row r at slot q ^ (r & 7)), so the 16 rows a fragment read touches spread
// over the banks.
// ---------------------------------------------------------------------------
namespace {
constexpr int kBT = 256;      // workgroup tile, rows of x and of w
constexpr int kRowBytes = 128;  // one k-block of a row

struct Staging {
  uint4 x[8];
  uint4 w[8];
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * kRowBytes + ((chunk ^ (row & 7)) << 4); }

// FASTDMS_AMD_FP8_GEMM_BIG=0 keeps every problem on the 128 x 128 kernel
bool big_tiles_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("FASTDMS_AMD_FP8_GEMM_BIG");
    return !(e && e[0] == '0');
  }();
  return on;
}
}  // namespace

template <bool BIAS, bool VEC_OUT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void fp8_gemm_big_kernel(
    const uint8_t* __restrict__ x, int64_t x_s, const float* __restrict__ x_inv, const uint8_t* __restrict__ w,
    int64_t w_s, const float* __restrict__ w_inv, const bf16_t* __restrict__ bias, bf16_t* __restrict__ y,
    int64_t y_s, int M, int N, int K, int tiles_n, int total, int per_xcd) {
  __shared__ __attribute__((aligned(16))) uint8_t s_x[2][kBT * kRowBytes];
  __shared__ __attribute__((aligned(16))) uint8_t s_w[2][kBT * kRowBytes];
  const int lin = blockIdx.x;
  const int t = (lin % kGemmXcds) * per_xcd + lin / kGemmXcds;
  if (t >= total) return;  // uniform per workgroup
  const int tm = t / tiles_n, tn = t - (t / tiles_n) * tiles_n;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int mb = tm * kBT, nb0 = tn * kBT;

  // staging: element u of this thread is row (tid + 256 u) / 8, chunk tid % 8
  const int srow0 = tid >> 3, schunk = tid & 7;
  const uint8_t* xs_row[8];
  const uint8_t* ws_row[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    xs_row[u] = x + (int64_t)min(mb + srow0 + 32 * u, M - 1) * x_s;
    ws_row[u] = w + (int64_t)min(nb0 + srow0 + 32 * u, N - 1) * w_s;
  }
  auto load_stage = [&](Staging& st, int blk) {
    const int kk = blk * kRowBytes + schunk * 16;
    const bool ok = kk < K;
    const int ka = ok ? kk : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint4 vx = *reinterpret_cast<const uint4*>(xs_row[u] + ka);
      const uint4 vw = *reinterpret_cast<const uint4*>(ws_row[u] + ka);
      st.x[u] = ok ? vx : uint4{0u, 0u, 0u, 0u};
      st.w[u] = ok ? vw : uint4{0u, 0u, 0u, 0u};
    }
  };
  auto store_stage = [&](const Staging& st, int buf) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int r = srow0 + 32 * u;
      *reinterpret_cast<uint4*>(&s_x[buf][swz(r, schunk)]) = st.x[u];
      *reinterpret_cast<uint4*>(&s_w[buf][swz(r, schunk)]) = st.w[u];
    }
  };

  // wave (wy, wx): x rows wy * 128 .. + 127, w rows wx * 128 .. + 127 of the tile
  const int xr0 = (wave >> 1) * 128, wr0 = (wave & 1) * 128;
  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf) {
    i32x8 xf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = xr0 + 16 * j + c;
      const uint4 lo = *reinterpret_cast<const uint4*>(&s_x[buf][swz(r, 2 * g)]);
      const uint4 hi = *reinterpret_cast<const uint4*>(&s_x[buf][swz(r, 2 * g + 1)]);
      xf[j] = as_i32x8(lo, hi);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = wr0 + 16 * i + c;
      const uint4 lo = *reinterpret_cast<const uint4*>(&s_w[buf][swz(r, 2 * g)]);
      const uint4 hi = *reinterpret_cast<const uint4*>(&s_w[buf][swz(r, 2 * g + 1)]);
      const i32x8 wf = as_i32x8(lo, hi);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, xf[j], acc[i][j], 0, 0, 0, 127, 0, 127);
    }
  };

  const int nblk = (K + kRowBytes - 1) / kRowBytes;
  Staging st;
  load_stage(st, 0);
  store_stage(st, 0);
  __syncthreads();
  if (nblk > 1) load_stage(st, 1);
  for (int b = 0; b < nblk; ++b) {
    compute(b & 1);
    if (b + 1 < nblk) {
      // buffer (b + 1) & 1 was last read in iteration b - 1, before its barrier
      store_stage(st, (b + 1) & 1);
      if (b + 2 < nblk) load_stage(st, b + 2);
    }
    __syncthreads();
  }

  // lane (g, c) holds C[n = wr0 + 16 i + 4 g + r][m = xr0 + 16 j + c] of the tile
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int m = mb + xr0 + 16 * j + c;
    if (m >= M) continue;
    const float xsc = x_inv[m];
    bf16_t* yr = y + (int64_t)m * y_s;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int nb = nb0 + wr0 + 16 * i + 4 * g;
      if (nb >= N) continue;
      uint32_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = min(nb + r, N - 1);
        float v = acc[i][j][r] * xsc * w_inv[n];
        if (BIAS) v = bf16_to_f32(f32_to_bf16(v)) + bf16_to_f32(bias[n].bits);
        o[r] = f32_to_bf16(v);
      }
      if (VEC_OUT && nb + 3 < N) {
        *reinterpret_cast<uint2*>(yr + nb) = uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) yr[nb + r].bits = (uint16_t)o[r];
      }
    }
  }
}

// y [M, N] bf16 (row stride y_s elements) = the FP8 product above.  x, w:
// e4m3fn rows [M, K] / [N, K] with byte strides x_s / w_s; K, the strides and
// the pointers 16-byte multiples.  x_inv [M], w_inv [N] fp32; bias [N] bf16 or
// NULL.
FDMS_EXPORT int fdms_fp8_gemm(const void* x, int64_t x_s, const float* x_inv, const void* w, int64_t w_s,
                              const float* w_inv, const void* bias, void* y, int64_t y_s, int M, int N, int K,
                              void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || (K & 15) || (x_s & 15) || (w_s & 15) || x_s < K || w_s < K || y_s < N)
    return (int)hipErrorInvalidValue;
  if (M == 0) return 0;
  if (!x || !x_inv || !w || !w_inv || !y) return (int)hipErrorInvalidValue;
  if (((uintptr_t)x | (uintptr_t)w) & 15) return (int)hipErrorInvalidValue;
  const bool vec = (y_s % 4) == 0 && ((uintptr_t)y % 8) == 0;
  // 256 x 256 tiles when they fill the chip
  const int64_t big_m = (M + kBT - 1) / kBT, big_n = (N + kBT - 1) / kBT;
  if (big_m * big_n >= 256 && big_tiles_enabled()) {
    const int64_t total = big_m * big_n;
    if (total > (int64_t)0x7FFFFFFF - kGemmXcds) return (int)hipErrorInvalidValue;
    const int per_xcd = (int)((total + kGemmXcds - 1) / kGemmXcds);
    const dim3 grid((unsigned)(per_xcd * kGemmXcds));
#define FDMS_GEMM_BIG(B, V)                                                                                       \
  hipLaunchKernelGGL((fp8_gemm_big_kernel<B, V>), grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint8_t*)x, \
                     x_s, x_inv, (const uint8_t*)w, w_s, w_inv, (const bf16_t*)bias, (bf16_t*)y, y_s, M, N, K,      \
                     (int)big_n, (int)total, per_xcd)
    if (bias) {
      if (vec) FDMS_GEMM_BIG(true, true); else FDMS_GEMM_BIG(true, false);
    } else {
      if (vec) FDMS_GEMM_BIG(false, true); else FDMS_GEMM_BIG(false, false);
    }
#undef FDMS_GEMM_BIG
    FDMS_LAUNCH_CHECK();
    return 0;
  }
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const int64_t total = (int64_t)tiles_m * tiles_n;
  if (total > (int64_t)0x7FFFFFFF - kGemmXcds) return (int)hipErrorInvalidValue;
  const int per_xcd = (int)((total + kGemmXcds - 1) / kGemmXcds);
  const dim3 grid((unsigned)(per_xcd * kGemmXcds));
#define FDMS_GEMM_LAUNCH(B, V)                                                                                    \
  hipLaunchKernelGGL((fp8_gemm_kernel<B, V>), grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint8_t*)x, x_s, \
                     x_inv, (const uint8_t*)w, w_s, w_inv, (const bf16_t*)bias, (bf16_t*)y, y_s, M, N, K, tiles_n,  \
                     (int)total, per_xcd)
  if (bias) {
    if (vec) FDMS_GEMM_LAUNCH(true, true); else FDMS_GEMM_LAUNCH(true, false);
  } else {
    if (vec) FDMS_GEMM_LAUNCH(false, true); else FDMS_GEMM_LAUNCH(false, false);
  }
#undef FDMS_GEMM_LAUNCH
  FDMS_LAUNCH_CHECK();
  return 0;
}
