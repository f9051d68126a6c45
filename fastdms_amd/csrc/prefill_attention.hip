// Dense causal prefill attention over a ragged batch (the reference calls
// flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, causal=True),
// attention.py:85-92: evictions act only at pack time, so prefill attends to
// the full prompt).  A sequence's query rows are the last of its keys
// (flash-attn's bottom-right causal alignment): a chunk of a long prompt
// attends to the retained earlier chunks plus itself.
//
// bf16 in/out, fp32 softmax, GQA.  One workgroup = 64 query rows of one query
// head (4 waves x 16 rows); key/value blocks of 64 tokens are staged in LDS
// (K row-major, V transposed) and shared by the 4 waves.  Per wave:
//   S^T (keys x queries) = K . Q^T   with v_mfma_f32_16x16x32_bf16
//   online softmax in the log2 domain (row max across 4 lane groups)
//   O (queries x d) += P . V         with v_mfma_f32_16x16x32_bf16
// MFMA 16x16x32 bf16 operand layout (lane l, 8 values each):
//   A[row = l%16][k = 8*(l/16) + i],  B[k = 8*(l/16) + i][col = l%16],
//   C[row = 4*(l/16) + r][col = l%16], r = 0..3.
// S^T's C layout gives lane l the scores of query l%16 for keys
// 16t + 4*(l/16) + r, which is directly the A operand of P.V once the key
// order inside each 32-key MFMA step is permuted the same way for V.
#include <cstdlib>

#include "fdms_common.h"

using namespace fdms;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kQRows = 64;   // query rows per workgroup
constexpr int kKeys = 64;    // keys per LDS block
constexpr int kThreads = 256;

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
  bf16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return f32_to_bf16(a) | (f32_to_bf16(b) << 16);
}

// Two fp32 -> bf16 (round to nearest even) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t r = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace

// FASTDMS_AMD_PREFILL_GQA=0 selects the per-head kernel for every shape
// (comparison / testing).
static bool fdms_prefill_gqa_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("FASTDMS_AMD_PREFILL_GQA");
    return !(e && e[0] == '0');
  }();
  return on;
}

template <int D>
__global__ __launch_bounds__(kThreads) void prefill_attn_kernel(
    const bf16_t* __restrict__ q, int64_t qs_t, int64_t qs_h, const bf16_t* __restrict__ k, int64_t ks_t,
    int64_t ks_h, const bf16_t* __restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t* __restrict__ out, int64_t os_t,
    int64_t os_h, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int group,
    float scale_log2) {
  constexpr int KPAD = D + 8;       // sK row stride (bf16)
  constexpr int VPAD = kKeys + 8;   // sVt row stride (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t sK[kKeys * KPAD];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[D * VPAD];

  const int seq = blockIdx.z;
  const int qh = blockIdx.y;
  const int kvh = qh / group;
  // query rows are the last qlen of the sequence's klen keys (bottom-right
  // causal alignment): row i is position off + i and sees keys 0 .. off + i
  const int start = cu_q[seq];
  const int len = cu_q[seq + 1] - start;
  const int kstart = cu_k[seq];
  const int klen = cu_k[seq + 1] - kstart;
  const int off = klen - len;
  if (off < 0) return;  // rejected: more queries than keys
  const int nqb = (len + kQRows - 1) / kQRows;
  if ((int)blockIdx.x >= nqb) return;
  const int qb = nqb - 1 - (int)blockIdx.x;  // heaviest (diagonal-last) blocks first
  const int q0 = qb * kQRows;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lg = lane >> 4;   // lane group 0..3
  const int lc = lane & 15;   // lane column 0..15
  const int my_q = q0 + wave * 16 + lc;  // query row this lane's S^T column belongs to

  // Q^T as the B operand of S^T = K.Q^T: lane holds Q[my_q][32j + 8*lg + i]
  bf16x8 qop[D / 32];
  {
    const int qrow = min(my_q, len - 1);
    const bf16_t* qp = q + (int64_t)(start + qrow) * qs_t + (int64_t)qh * qs_h;
#pragma unroll
    for (int j = 0; j < D / 32; ++j) qop[j] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 32 * j + 8 * lg));
  }

  float m_run = -INFINITY;  // running max of query my_q (same in the 4 lane groups)
  float l_part = 0.0f;      // this lane's partial softmax denominator
  f32x4 o[D / 16];          // O[q = 4*lg + r][d = 16c + lc] of this wave's 16 rows
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nkb = min((klen + kKeys - 1) / kKeys, (off + q0 + kQRows - 1) / kKeys + 1);
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * kKeys;
    __syncthreads();
    // stage K (row-major) and V (transposed) for keys k0..k0+63; zero beyond len
    for (int u = tid; u < kKeys * D / 8; u += kThreads) {
      const int key = u / (D / 8);
      const int d0 = (u - key * (D / 8)) * 8;
      uint4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
      if (k0 + key < klen) {
        kv = *reinterpret_cast<const uint4*>(k + (int64_t)(kstart + k0 + key) * ks_t + (int64_t)kvh * ks_h + d0);
        vv = *reinterpret_cast<const uint4*>(v + (int64_t)(kstart + k0 + key) * vs_t + (int64_t)kvh * vs_h + d0);
      }
      *reinterpret_cast<uint4*>(&sK[key * KPAD + d0]) = kv;
      const uint16_t* vh = reinterpret_cast<const uint16_t*>(&vv);
#pragma unroll
      for (int i = 0; i < 8; ++i) sVt[(d0 + i) * VPAD + key] = vh[i];
    }
    __syncthreads();

    // S^T for the 4 key tiles of 16: lane gets keys 16t + 4*lg + r for query my_q
    float s[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < D / 32; ++j) {
        const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(&sK[(16 * t + lc) * KPAD + 32 * j + 8 * lg]));
        acc = mfma16x16x32(a, qop[j], acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 16 * t + 4 * lg + r;
        const bool ok = key <= off + my_q && key < klen;
        s[t][r] = ok ? acc[r] * scale_log2 : -INFINITY;
      }
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) bmax = fmaxf(bmax, s[t][r]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    const float m_new = fmaxf(m_run, bmax);
    const float alpha = (m_run == -INFINITY) ? 0.0f : exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = (s[t][r] == -INFINITY) ? 0.0f : exp2f(s[t][r] - m_new);
        s[t][r] = p;
        psum += p;
      }
    l_part = l_part * alpha + psum;
    // rescale O rows q = 4*lg + r by alpha of that query (held by lane 4*lg + r)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * lg + r);
#pragma unroll
      for (int c = 0; c < D / 16; ++c) o[c][r] *= ar;
    }
    // O += P.V over two 32-key steps; k index i of lane group lg = key 32*st + 16*(i/4) + 4*lg + i%4
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      uint4 pa;
      pa.x = pack_bf16x2(s[2 * st][0], s[2 * st][1]);
      pa.y = pack_bf16x2(s[2 * st][2], s[2 * st][3]);
      pa.z = pack_bf16x2(s[2 * st + 1][0], s[2 * st + 1][1]);
      pa.w = pack_bf16x2(s[2 * st + 1][2], s[2 * st + 1][3]);
      const bf16x8 a = as_bf16x8(pa);
      const int key_a = 32 * st + 4 * lg;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        const uint16_t* vr = &sVt[(16 * c + lc) * VPAD];
        uint4 b;
        const uint2 lo = *reinterpret_cast<const uint2*>(vr + key_a);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + key_a + 16);
        b.x = lo.x;
        b.y = lo.y;
        b.z = hi.x;
        b.w = hi.y;
        o[c] = mfma16x16x32(a, as_bf16x8(b), o[c]);
      }
    }
  }

  float l_tot = l_part;
  l_tot += __shfl_xor(l_tot, 16);
  l_tot += __shfl_xor(l_tot, 32);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float inv = 1.0f / __shfl(l_tot, 4 * lg + r);
    const int row = q0 + wave * 16 + 4 * lg + r;
    if (row < len) {
      bf16_t* op = out + (int64_t)(start + row) * os_t + (int64_t)qh * os_h;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) op[16 * c + lc].bits = (uint16_t)f32_to_bf16(o[c][r] * inv);
    }
  }
}

// GQA-packed variant for group sizes 1, 2 and 4: a workgroup takes P =
// 64·QT/G query positions of one KV head for all G query heads that share it,
// so one staged K/V block feeds 64·QT query rows (wave w: head w % G,
// positions 16·QT·(w / G) .. +16·QT-1, QT 16-row MFMA tiles; QT = 2: QT = 4
// halves the LDS reads per MFMA but costs an occupancy step (3 -> 2 waves per
// SIMD at head_dim 64) and measured no faster).  K/V blocks of 64 keys are
// double-buffered in LDS: the next block's global loads are in flight while
// the current one is computed, and one barrier separates blocks.  V is
// transposed in registers (4 keys x 8 dims per thread, byte permutes) so the
// LDS stores are 8-byte vectors.  Every K fragment read from LDS feeds both
// query tiles of a wave, as does every V fragment.  The softmax row sums come
// from the matrix cores (P . 1, an extra output tile).  Softmax rescaling is
// lazy: the running max only moves (and O / the sums are rescaled) when a block raises it
// by more than 8 in the log2 domain, so p = exp2(s - m) stays below 256.  The
// running max starts at a finite floor (-1e30) instead of -inf: the first
// block with a visible key then takes the same grow test as every later one,
// its rescale factor exp2((floor - m) * scale) is exactly 0, and a row whose
// keys so far are all masked keeps the floor with p = exp2(-inf) = 0 -- the
// same results as special-casing -inf, with fewer VALU instructions per block.
template <int D, int G, int QT>
__global__ __launch_bounds__(kThreads) void prefill_attn_gqa_kernel(
    const bf16_t* __restrict__ q, int64_t qs_t, int64_t qs_h, const bf16_t* __restrict__ k, int64_t ks_t,
    int64_t ks_h, const bf16_t* __restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t* __restrict__ out, int64_t os_t,
    int64_t os_h, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, float scale_log2) {
  constexpr int RW = 16 * QT;       // query rows per wave (QT 16-row MFMA tiles)
  constexpr int P = 4 * RW / G;     // query positions per workgroup
  constexpr int KPAD = D + 8;       // sK row stride (bf16)
  // sVt row stride (bf16): 136 B = 34 dwords, so the 16 lanes of one 8-byte
  // B-operand read (rows 16c + lc) land on 16 distinct bank pairs
  constexpr int VPAD = kKeys + 4;
  constexpr int UNITS = 4 * D;      // staging units per block: 2D V quads (4 keys x 8 dims) + 2D K quads (4 chunks)
  constexpr int UPT = UNITS / kThreads;
  static_assert(UNITS % kThreads == 0, "staging units must divide over the workgroup");
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kKeys * KPAD];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[2][D * VPAD];

  const int seq = blockIdx.z;
  const int kvh = blockIdx.y;
  // query rows are the last len of the klen keys (bottom-right causal
  // alignment, as the per-head kernel); positions below are query rows
  const int start = cu_q[seq];
  const int len = cu_q[seq + 1] - start;
  const int kstart = cu_k[seq];
  const int klen = cu_k[seq + 1] - kstart;
  const int off = klen - len;
  if (off < 0) return;  // rejected: more queries than keys
  const int nqb = (len + P - 1) / P;
  if ((int)blockIdx.x >= nqb) return;
  const int q0 = (nqb - 1 - (int)blockIdx.x) * P;  // heaviest (diagonal-last) blocks first
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lg = lane >> 4;
  const int lc = lane & 15;
  const int qh = kvh * G + wave % G;
  const int wq0 = q0 + (wave / G) * RW;            // first position of this wave
  const int wq_last = min(wq0 + RW - 1, len - 1);  // last valid position of this wave

  bf16x8 qop[QT][D / 32];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qrow = min(wq0 + 16 * qt + lc, len - 1);
    const bf16_t* qp = q + (int64_t)(start + qrow) * qs_t + (int64_t)qh * qs_h;
#pragma unroll
    for (int j = 0; j < D / 32; ++j) qop[qt][j] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 32 * j + 8 * lg));
  }

  const bf16_t* kb_base = k + (int64_t)kstart * ks_t + (int64_t)kvh * ks_h;
  const bf16_t* vb_base = v + (int64_t)kstart * vs_t + (int64_t)kvh * vs_h;
  uint4 stage[UPT][4];
  // unit u < 2D: V quad (keys 4*(u % 16) .. +3, dims 8*(u / 16) .. +7: the 16
  // lanes of a row store 128 contiguous bytes of one transposed row);
  // u >= 2D: K chunks (u - 2D) + 2D*r, r = 0..3 (chunk c = key * (D/8) + dim / 8:
  // consecutive lanes move consecutive 16-byte chunks).
  // Row r of unit i is key k0 + krow[i][r] at element offset koff[i][r] +
  // key * stride; rows past the sequence end are clamped (their scores are
  // masked).
  // Whether unit i is a V or a K unit is uniform per wave (2D is a multiple
  // of 64), so a block's row base is a scalar and each lane adds a fixed
  // 32-bit element offset: the loads of a block cost no vector address math.
  int krow[UPT][4], koff[UPT][4], eoff[UPT][4];
  const bf16_t* kvp[UPT];
  int64_t kvs[UPT];
#pragma unroll
  for (int i = 0; i < UPT; ++i) {
    const int u = tid + i * kThreads;
    const bool is_v = __builtin_amdgcn_readfirstlane((int)(u < 2 * D)) != 0;
    kvp[i] = is_v ? vb_base : kb_base;
    kvs[i] = is_v ? vs_t : ks_t;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = (u - 2 * D) + 2 * D * r;
      krow[i][r] = is_v ? 4 * (u % 16) + r : c / (D / 8);
      koff[i][r] = is_v ? 8 * (u / 16) : 8 * (c % (D / 8));
      eoff[i][r] = krow[i][r] * (int)kvs[i] + koff[i][r];  // < 64 rows: within int range for any real stride
    }
  }
  auto load_block = [&](int k0) {
    if (k0 + kKeys <= klen) {  // uniform
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const bf16_t* base = kvp[i] + (int64_t)k0 * kvs[i];  // scalar
#pragma unroll
        for (int r = 0; r < 4; ++r) stage[i][r] = *reinterpret_cast<const uint4*>(base + eoff[i][r]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < UPT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = min(k0 + krow[i][r], klen - 1);  // rows past the end clamped (their scores are masked)
          stage[i][r] = *reinterpret_cast<const uint4*>(kvp[i] + (int64_t)key * kvs[i] + koff[i][r]);
        }
    }
  };
  auto store_block = [&](int buf) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * kThreads;
      if (u < 2 * D) {
        const int kq = u % 16, dc = u / 16;
        const uint32_t w0[4] = {stage[i][0].x, stage[i][0].y, stage[i][0].z, stage[i][0].w};
        const uint32_t w1[4] = {stage[i][1].x, stage[i][1].y, stage[i][1].z, stage[i][1].w};
        const uint32_t w2[4] = {stage[i][2].x, stage[i][2].y, stage[i][2].z, stage[i][2].w};
        const uint32_t w3[4] = {stage[i][3].x, stage[i][3].y, stage[i][3].z, stage[i][3].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          uint2 t;
          t.x = __builtin_amdgcn_perm(w1[e >> 1], w0[e >> 1], sel);  // keys 4kq, 4kq+1 of dim 8dc+e
          t.y = __builtin_amdgcn_perm(w3[e >> 1], w2[e >> 1], sel);  // keys 4kq+2, 4kq+3
          *reinterpret_cast<uint2*>(&sVt[buf][(8 * dc + e) * VPAD + 4 * kq]) = t;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = (u - 2 * D) + 2 * D * r;
          *reinterpret_cast<uint4*>(&sK[buf][(c / (D / 8)) * KPAD + 8 * (c % (D / 8))]) = stage[i][r];
        }
      }
    }
  };

  constexpr float kMaxFloor = -1e30f;  // below any score; see the rescale note above
  float m_run[QT];  // raw-score running max of query lc of each tile
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) m_run[qt] = kMaxFloor;
  // o[qt][D/16] accumulates P . 1 on the matrix cores: column-replicated row
  // sums of the same bf16 P as the numerator, in the O layout (no shuffles)
  f32x4 o[QT][D / 16 + 1];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int c = 0; c <= D / 16; ++c) o[qt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16x8 ones = as_bf16x8(uint4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

  const int kend = min(klen, off + q0 + P);  // keys 0 .. kend-1 are visible to some row of the workgroup
  const int nkb = (kend + kKeys - 1) / kKeys;
  load_block(0);
  store_block(0);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * kKeys;
    const int buf = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) load_block(k0 + kKeys);
    if (k0 <= off + wq_last) {  // wave-uniform: this block holds keys visible to the wave
      f32x4 acc[QT][4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) acc[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
          const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(&sK[buf][(16 * t + lc) * KPAD + 32 * j + 8 * lg]));
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) acc[qt][t] = mfma16x16x32(a, qop[qt][j], acc[qt][t]);
        }
      }
      const bool masked = k0 + kKeys - 1 > off + wq0 || k0 + kKeys > klen;  // wave-uniform
      if (masked) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const int lim = off + min(wq0 + 16 * qt + lc, len - 1);
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int key = k0 + 16 * t + 4 * lg + r;
              acc[qt][t][r] = key > lim ? -INFINITY : acc[qt][t][r];
            }
        }
      }
      uint4 pa[QT][2];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        float bmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) bmax = fmaxf(bmax, acc[qt][t][r]);
        bmax = rows_max(bmax);
        // lazy rescale: move the max only when it grows by more than 2^8 in p
        const bool grow = (bmax - m_run[qt]) * scale_log2 > 8.0f;  // bmax = -inf (all masked): false
        if (__builtin_amdgcn_ballot_w64(grow)) {  // wave-uniform
          const float m_new = fmaxf(m_run[qt], bmax);
          const float alpha = __builtin_amdgcn_exp2f((m_run[qt] - m_new) * scale_log2);  // 0 from the floor
          m_run[qt] = m_new;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * lg + r);
#pragma unroll
            for (int c = 0; c <= D / 16; ++c) o[qt][c][r] *= ar;
          }
        }
        const float mb = m_run[qt] * scale_log2;
        float p[4][4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) p[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[qt][t][r], scale_log2, -mb));
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          pa[qt][st].x = cvt_pk_bf16(p[2 * st][0], p[2 * st][1]);
          pa[qt][st].y = cvt_pk_bf16(p[2 * st][2], p[2 * st][3]);
          pa[qt][st].z = cvt_pk_bf16(p[2 * st + 1][0], p[2 * st + 1][1]);
          pa[qt][st].w = cvt_pk_bf16(p[2 * st + 1][2], p[2 * st + 1][3]);
        }
      }
      // O += P.V; k index i of lane group lg = key 32*st + 16*(i/4) + 4*lg + i%4
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int key_a = 32 * st + 4 * lg;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const uint16_t* vr = &sVt[buf][(16 * c + lc) * VPAD];
          const uint2 lo = *reinterpret_cast<const uint2*>(vr + key_a);
          const uint2 hi = *reinterpret_cast<const uint2*>(vr + key_a + 16);
          const bf16x8 b = as_bf16x8(uint4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) o[qt][c] = mfma16x16x32(as_bf16x8(pa[qt][st]), b, o[qt][c]);
        }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][D / 16] = mfma16x16x32(as_bf16x8(pa[qt][st]), ones, o[qt][D / 16]);
      }
    }
    if (more) store_block(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float inv = 1.0f / o[qt][D / 16][r];  // row sum of query 4*lg + r
      const int row = wq0 + 16 * qt + 4 * lg + r;
      if (row < len) {
        bf16_t* op = out + (int64_t)(start + row) * os_t + (int64_t)qh * os_h;
#pragma unroll
        for (int c = 0; c < D / 16; ++c) op[16 * c + lc].bits = (uint16_t)f32_to_bf16(o[qt][c][r] * inv);
      }
    }
  }
}

FDMS_EXPORT int fdms_prefill_attention_varlen(const void* q, int64_t qs_t, int64_t qs_h, const void* k,
                                              int64_t ks_t, int64_t ks_h, const void* v, int64_t vs_t, int64_t vs_h,
                                              void* out, int64_t os_t, int64_t os_h, const int32_t* cu_seqlens_q,
                                              const int32_t* cu_seqlens_k, int num_seqs, int max_seqlen_q,
                                              int num_q_heads, int num_kv_heads, int head_dim, float scale,
                                              void* stream) {
  if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return (int)hipErrorInvalidValue;
  if (num_seqs == 0 || max_seqlen_q <= 0) return 0;
  if (!q || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k) return (int)hipErrorInvalidValue;
  if (num_seqs > 65535 || num_q_heads > 65535) return (int)hipErrorInvalidValue;
  // token strides in elements: 64 rows of either stay in 32-bit offsets
  if (ks_t < 0 || vs_t < 0 || ks_t >= (1 << 24) || vs_t >= (1 << 24)) return (int)hipErrorInvalidValue;
  const float sl2 = scale * 1.4426950408889634f;
  const int group = num_q_heads / num_kv_heads;
  const int32_t* cq = cu_seqlens_q;
  const int32_t* ck = cu_seqlens_k;
  if ((group == 1 || group == 2 || group == 4) && (head_dim == 64 || head_dim == 128) &&
      fdms_prefill_gqa_enabled()) {
    // 16-row query tiles per wave.  Four (head_dim 64 only) measured within
    // 1 % of two on the Llama-3.2-1B c=8 prompts and 15 % slower on one
    // 8192-token prompt, so two is the default
    int qt = 2;
    if (const char* e = std::getenv("FASTDMS_AMD_PREFILL_QT")) {  // comparison / testing
      if (e[0] == '4' && head_dim == 64) qt = 4;
    }
    const int pos = 64 * qt / group;  // query positions per workgroup
    const dim3 ggrid((max_seqlen_q + pos - 1) / pos, num_kv_heads, num_seqs);
#define FDMS_PREFILL_GQA(DD, GG, QQ)                                                                               \
  hipLaunchKernelGGL((prefill_attn_gqa_kernel<DD, GG, QQ>), ggrid, dim3(kThreads), 0, (hipStream_t)stream,          \
                     (const bf16_t*)q, qs_t, qs_h, (const bf16_t*)k, ks_t, ks_h, (const bf16_t*)v, vs_t, vs_h,       \
                     (bf16_t*)out, os_t, os_h, cq, ck, sl2)
    if (head_dim == 64 && qt == 4) {
      if (group == 1) FDMS_PREFILL_GQA(64, 1, 4); else if (group == 2) FDMS_PREFILL_GQA(64, 2, 4); else FDMS_PREFILL_GQA(64, 4, 4);
    } else if (head_dim == 64) {
      if (group == 1) FDMS_PREFILL_GQA(64, 1, 2); else if (group == 2) FDMS_PREFILL_GQA(64, 2, 2); else FDMS_PREFILL_GQA(64, 4, 2);
    } else {
      if (group == 1) FDMS_PREFILL_GQA(128, 1, 2); else if (group == 2) FDMS_PREFILL_GQA(128, 2, 2); else FDMS_PREFILL_GQA(128, 4, 2);
    }
#undef FDMS_PREFILL_GQA
    FDMS_LAUNCH_CHECK();
    return 0;
  }
  const dim3 grid((max_seqlen_q + kQRows - 1) / kQRows, num_q_heads, num_seqs);
  if (head_dim == 64) {
    hipLaunchKernelGGL(prefill_attn_kernel<64>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const bf16_t*)q, qs_t,
                       qs_h, (const bf16_t*)k, ks_t, ks_h, (const bf16_t*)v, vs_t, vs_h, (bf16_t*)out, os_t, os_h,
                       cq, ck, group, sl2);
  } else if (head_dim == 128) {
    hipLaunchKernelGGL(prefill_attn_kernel<128>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const bf16_t*)q,
                       qs_t, qs_h, (const bf16_t*)k, ks_t, ks_h, (const bf16_t*)v, vs_t, vs_h, (bf16_t*)out, os_t,
                       os_h, cq, ck, group, sl2);
  } else {
    return (int)hipErrorInvalidValue;
  }
  FDMS_LAUNCH_CHECK();
  return 0;
}

FDMS_EXPORT int fdms_prefill_attention(const void* q, int64_t qs_t, int64_t qs_h, const void* k, int64_t ks_t,
                                       int64_t ks_h, const void* v, int64_t vs_t, int64_t vs_h, void* out,
                                       int64_t os_t, int64_t os_h, const int32_t* cu_seqlens, int num_seqs,
                                       int max_seqlen, int num_q_heads, int num_kv_heads, int head_dim, float scale,
                                       void* stream) {
  return fdms_prefill_attention_varlen(q, qs_t, qs_h, k, ks_t, ks_h, v, vs_t, vs_h, out, os_t, os_h, cu_seqlens,
                                       cu_seqlens, num_seqs, max_seqlen, num_q_heads, num_kv_heads, head_dim, scale,
                                       stream);
}

// One v_mfma_f32_16x16x32_bf16 of a 16x32 A and a 32x16 B (row-major bf16)
// loaded with the operand layout the kernels above assume; C row-major fp32.
// Exists so a test can confirm that layout against a host matmul.
__global__ void mfma_probe_kernel(const bf16_t* __restrict__ a, const bf16_t* __restrict__ b, float* __restrict__ c) {
  const int l = threadIdx.x;
  uint16_t av[8], bv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = a[(l % 16) * 32 + 8 * (l / 16) + i].bits;
    bv[i] = b[(8 * (l / 16) + i) * 16 + (l % 16)].bits;
  }
  uint4 ua, ub;
  __builtin_memcpy(&ua, av, 16);
  __builtin_memcpy(&ub, bv, 16);
  const f32x4 r = mfma16x16x32(as_bf16x8(ua), as_bf16x8(ub), f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
  for (int i = 0; i < 4; ++i) c[(4 * (l / 16) + i) * 16 + (l % 16)] = r[i];
}

FDMS_EXPORT int fdms_mfma_probe(const void* a, const void* b, float* c, void* stream) {
  if (!a || !b || !c) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (const bf16_t*)a,
                     (const bf16_t*)b, c);
  FDMS_LAUNCH_CHECK();
  return 0;
}
