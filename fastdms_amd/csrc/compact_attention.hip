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
#include <algorithm>
#include <climits>
#include <cstdlib>
#include <mutex>

#include "fdms_common.h"
#include "fdms_plan.h"

using namespace fdms;

// FASTDMS_AMD_ATTN_GENERIC=1 routes every call to the generic kernel (read per
// call on the host; used to compare the two kernels on the same inputs).
static bool fdms_force_generic_attention() {
  const char* e = std::getenv("FASTDMS_AMD_ATTN_GENERIC");
  return e && e[0] == '1';
}

// Matrix-core kernel launch shape: FASTDMS_AMD_ATTN_WAVES = 4 or 8 waves per workgroup for the
// fused head_dim-64 kernel (default: 8 for 17 to 128 (seq, kv head) pairs,
// where a launch has few workgroups and each pair's rows go to more waves,
// else 4: three workgroups fit per CU, and at 16 pairs or fewer smaller
// splits spread the rows over more CUs).  Read per call; tuning switches
// that change speed, never results.
static int fdms_attn_fused_waves(int head_dim, int pairs) {
  if (head_dim == 128) return 8;  // the preprocess needs 2.5 * head_dim threads
  const char* e = std::getenv("FASTDMS_AMD_ATTN_WAVES");
  if (e && (e[0] == '4' || e[0] == '8') && !e[1]) return e[0] - '0';
  return (pairs > 16 && pairs <= 128) ? 8 : 4;
}

static bool fits_i32(int64_t v) { return v >= INT32_MIN && v <= INT32_MAX; }

// Rows per split of a pair longer than split_rows: split_rows / div rounded
// up to 64, div = 2 at head_dim 64 with at most 128 (seq, kv head) pairs
// (the launch time there is set by the heavy pairs, which pay the merge
// chain: half-size splits shorten their loops, 9.45 -> 8.74 us at c = 8),
// else 1 (measured slower: head_dim 128 19.9 vs 17.2 us, 128 sequences
// 0.40 vs 0.42 of HBM).  FASTDMS_AMD_ATTN_SPLIT_DIV = 1, 2 or 4 overrides
// (tuning only).
static int fdms_attn_heavy_rows(int rows, int head_dim, int pairs) {
  const char* e = std::getenv("FASTDMS_AMD_ATTN_SPLIT_DIV");
  int div = (head_dim == 64 && pairs <= 128) ? 2 : 1;
  if (e && (e[0] == '1' || e[0] == '2' || e[0] == '4') && !e[1]) div = e[0] - '0';
  return std::max(64, ((rows / div) + 63) & ~63);
}

// FASTDMS_AMD_ATTN_MFMA=0 keeps FP8 calls off the matrix-core kernel (read per
// call; used to compare kernels on the same inputs).
static bool fdms_mfma_attention_enabled() {
  const char* e = std::getenv("FASTDMS_AMD_ATTN_MFMA");
  return !(e && e[0] == '0');
}

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

__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-merge handoff of a workgroup (handoff_release / handoff_acquire in
// fdms_common.h): every thread's partials (relaxed agent-scope atomic stores)
// have completed before one thread takes the pair's ticket; the workgroup that
// takes ticket n-1 (the last of the pair's n workgroups) orders its partial
// loads (relaxed agent-scope atomic loads) after it.  Correct wherever the
// pair's workgroups run (any XCD).
__device__ __forceinline__ bool take_last_ticket(int* counter, int n, int* s_flag) {
  handoff_release();
  __syncthreads();
  if (threadIdx.x == 0) *s_flag = ticket_add(counter) == n - 1;
  __syncthreads();
  const bool last = *s_flag;
  if (last) handoff_acquire();
  return last;
}

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
    store_agent(mine + tid, s_m[tid]);
    store_agent(mine + G + tid, s_l[tid]);
  }
#pragma unroll
  for (int k = 0; k < kMaxG; ++k) {
    const int o = tid + k * kThreads;
    if (o < n_out) store_agent(mine + 2 * G + o, acc[k]);
  }
  if (!take_last_ticket(&counters[pair], num_splits, &s_last)) return;
  const float* all = ws + (int64_t)pair * num_splits * stride;
#pragma unroll
  for (int k = 0; k < kMaxG; ++k) {
    const int o = tid + k * kThreads;
    if (o < n_out) {
      const int g = o / D;
      float M = -INFINITY;
      for (int s = 0; s < num_splits; ++s) M = fmaxf(M, load_agent(all + s * stride + g));
      float L = 0.0f, A = 0.0f;
      for (int s = 0; s < num_splits; ++s) {
        const float* ps = all + s * stride;
        const float ms = load_agent(ps + g);
        const float wgt = (ms == -INFINITY) ? 0.0f : exp2f(ms - M);
        L += load_agent(ps + G + g) * wgt;
        A += load_agent(ps + 2 * G + o) * wgt;
      }
      const int d = o - g * D;
      st<QT>(out + b * os_b + (int64_t)(h * G + g) * os_h + d, A / L);
    }
  }
  if (tid == 0) __hip_atomic_store(&counters[pair], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Tiled fast path: bf16 q, FP8 or bf16 K/V rows of 16-byte-aligned D = 64 / 128
// elements, G in {1, 2, 4, 8}.
//
// A tile of T rows is read with lane-contiguous 16-byte loads (C = row bytes /
// 16 lanes per row, RP = 256 / C rows per pass, NP passes in flight per
// thread), so every wave instruction covers 1 KiB of one contiguous span.
//   scores: each lane dots its 16-byte chunk with q (kept in LDS, pre-scaled
//           by scale*log2 e) and the C lanes of a row reduce with xor shuffles;
//   V:      the same lanes convert their chunk to bf16 into an LDS tile;
//   P.V:    lane l of wave w owns DPL = G*D/64 outputs (head g = l / (64/G... ))
//           over rows w, w+4, ...; the four waves' partial sums are reduced
//           once after the last tile (the online-softmax rescale is applied
//           per tile to every wave's partials alike).
// FP8 is decoded with v_cvt_pk_f32_fp8 (OCP e4m3fn on gfx950).
// Workgroups are dispatched round-robin over the 8 XCDs; the linear block id
// is remapped so all splits of one (b, h) run on the same XCD and their
// partials meet in that XCD's L2.
// ---------------------------------------------------------------------------
namespace {

constexpr int kXcds = 8;
constexpr int kMergeBatch = 8;  // split partials loaded per round trip in the merge

template <typename KT> struct RowLoad;
template <> struct RowLoad<fp8_t> {
  static constexpr int kEpc = 16;  // elements per 16-byte chunk
  static __device__ __forceinline__ void to_f32(const uint4& c, float* f) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
      f[4 * i + 0] = lo[0];
      f[4 * i + 1] = lo[1];
      f[4 * i + 2] = hi[0];
      f[4 * i + 3] = hi[1];
    }
  }
};
template <> struct RowLoad<bf16_t> {
  static constexpr int kEpc = 8;
  static __device__ __forceinline__ void to_f32(const uint4& c, float* f) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};

template <int D, int G, typename KT>
struct TiledCfg {
  static constexpr int kEpc = RowLoad<KT>::kEpc;
  static constexpr int kC = D / kEpc;            // lanes per row
  static constexpr int kRP = kThreads / kC;      // rows per pass
  static constexpr int kNP = 4;                  // passes per tile
  static constexpr int kT = kRP * kNP;           // rows per tile
  static constexpr int kDPL = G * D / 64;        // P.V outputs per lane
  static constexpr int kLanesPerHead = 64 / G;   // P.V lanes per head
};

}  // namespace

template <int D, int G, typename KT>
__global__ __launch_bounds__(kThreads) void decode_attn_tiled_kernel(
    const bf16_t* __restrict__ q, int64_t qs_b, int64_t qs_h, const KT* __restrict__ ck, const KT* __restrict__ cv,
    int64_t c_s, const int32_t* __restrict__ base_offsets, int64_t bo_b, int64_t bo_h,
    const int32_t* __restrict__ block_tables, int64_t bt_b, int64_t bt_h, int page_shift, int paged,
    const int32_t* __restrict__ live_counts, int64_t lc_b, int64_t lc_h, bf16_t* __restrict__ out, int64_t os_b,
    int64_t os_h, float* __restrict__ ws, int* __restrict__ counters, int num_kv_heads, int num_pairs,
    int num_splits, float scale, const float* __restrict__ rope_cs, int64_t rcs_p, int64_t rcs_d,
    const int64_t* __restrict__ rope_pos) {
  using Cfg = TiledCfg<D, G, KT>;
  constexpr int C = Cfg::kC, RP = Cfg::kRP, NP = Cfg::kNP, T = Cfg::kT, EPC = Cfg::kEpc;
  constexpr int DPL = Cfg::kDPL, LPH = Cfg::kLanesPerHead;
  __shared__ __attribute__((aligned(16))) float s_q[G][D];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[T][D];   // bf16 bits
  __shared__ float s_p[G][T];
  __shared__ __attribute__((aligned(16))) float s_red[kThreads / kWave][64][DPL];
  __shared__ float s_m[G], s_l[G], s_alpha[G];
  __shared__ int s_last;

  // XCD-aware (pair, split) of this workgroup
  const int lin = blockIdx.x;
  const int xcd = lin % kXcds;
  const int slot = lin / kXcds;
  const int pair = (slot / num_splits) * kXcds + xcd;
  const int split = slot - (slot / num_splits) * num_splits;
  if (pair >= num_pairs) return;  // uniform per workgroup
  const int b = pair / num_kv_heads;
  const int h = pair - b * num_kv_heads;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;

  const int live = live_counts[b * lc_b + h * lc_h];
  const int per = (live + num_splits - 1) / num_splits;
  const int t0 = min(live, split * per);
  const int t1 = min(live, t0 + per);
  const int64_t bo = paged ? 0 : (int64_t)base_offsets[b * bo_b + h * bo_h];
  const SpanAddr addr{base_offsets, block_tables, bt_b, bt_h, page_shift, paged};
  const float qscale = scale * kLog2e;

  // q -> LDS (fp32, pre-scaled), optional inline RoPE with the decision lane zeroed
  if (rope_pos) {
    constexpr int half = D / 2;
    const int64_t pos = rope_pos[b];
    for (int i = tid; i < G * half; i += kThreads) {
      const int g = i / half, j = i - g * half;
      const bf16_t* qh = q + b * qs_b + (int64_t)(h * G + g) * qs_h;
      const float x1 = ld<bf16_t>(qh + j);
      const float x2 = (g == 0 && j == half - 1) ? 0.0f : ld<bf16_t>(qh + j + half);
      float y1, y2;
      rope_f32(x1, x2, rope_cs[pos * rcs_p + (int64_t)j * rcs_d], rope_cs[pos * rcs_p + (int64_t)(j + half) * rcs_d],
               &y1, &y2);
      s_q[g][j] = y1 * qscale;
      s_q[g][j + half] = y2 * qscale;
    }
  } else {
    for (int i = tid; i < G * D; i += kThreads) {
      const int g = i / D, d = i - g * D;
      s_q[g][d] = ld<bf16_t>(q + b * qs_b + (int64_t)(h * G + g) * qs_h + d) * qscale;
    }
  }
  if (tid < G) {
    s_m[tid] = -INFINITY;
    s_l[tid] = 0.0f;
  }
  __syncthreads();

  const int chunk = tid % C;        // this lane's 16-byte chunk of a row
  const int prow = tid / C;         // this lane's row within a pass
  const int pv_g = lane / LPH;      // P.V: head and output columns of this lane
  const int pv_d0 = (lane - pv_g * LPH) * DPL;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;

  for (int tile = t0; tile < t1; tile += T) {
    const int n = min(T, t1 - tile);
    uint4 kr[NP], vr[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int r = p * RP + prow;
      kr[p] = uint4{0u, 0u, 0u, 0u};
      vr[p] = uint4{0u, 0u, 0u, 0u};
      if (r < n) {
        const int64_t row = addr.row(b, h, bo, tile + r);
        kr[p] = *reinterpret_cast<const uint4*>(ck + row * c_s + chunk * EPC);
        vr[p] = *reinterpret_cast<const uint4*>(cv + row * c_s + chunk * EPC);
      }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int r = p * RP + prow;
      float kf[EPC];
      RowLoad<KT>::to_f32(kr[p], kf);
      float sc[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4* qg = reinterpret_cast<const float4*>(&s_q[g][chunk * EPC]);
        float a = 0.0f;
#pragma unroll
        for (int e4 = 0; e4 < EPC / 4; ++e4) {
          const float4 qq = qg[e4];
          a += qq.x * kf[4 * e4] + qq.y * kf[4 * e4 + 1] + qq.z * kf[4 * e4 + 2] + qq.w * kf[4 * e4 + 3];
        }
        sc[g] = a;
      }
#pragma unroll
      for (int o = 1; o < C; o <<= 1)
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g] += __shfl_xor(sc[g], o);
      if (chunk == 0 && r < T) {
#pragma unroll
        for (int g = 0; g < G; ++g) s_p[g][r] = (r < n) ? sc[g] : -INFINITY;
      }
      // V chunk -> LDS as bf16
      float vf[EPC];
      RowLoad<KT>::to_f32(vr[p], vf);
      uint32_t packed[EPC / 2];
#pragma unroll
      for (int e = 0; e < EPC / 2; ++e)
        packed[e] = f32_to_bf16(vf[2 * e]) | (f32_to_bf16(vf[2 * e + 1]) << 16);
      uint4* dst = reinterpret_cast<uint4*>(&s_v[r][chunk * EPC]);
#pragma unroll
      for (int e = 0; e < EPC / 8; ++e) dst[e] = uint4{packed[4 * e], packed[4 * e + 1], packed[4 * e + 2], packed[4 * e + 3]};
    }
    __syncthreads();
    // online softmax over the tile, one wave per head (heads w, w+4)
    for (int g = wave; g < G; g += kThreads / kWave) {
      float mx = -INFINITY;
      for (int i = lane; i < n; i += kWave) mx = fmaxf(mx, s_p[g][i]);
      mx = wave_max(mx);
      const float m_old = s_m[g];
      const float m_new = fmaxf(m_old, mx);
      float sum = 0.0f;
      for (int i = lane; i < n; i += kWave) {
        const float pr = exp2f(s_p[g][i] - m_new);
        s_p[g][i] = pr;
        sum += pr;
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        const float alpha = exp2f(m_old - m_new);
        s_alpha[g] = alpha;
        s_l[g] = s_l[g] * alpha + sum;
        s_m[g] = m_new;
      }
    }
    __syncthreads();
    // P.V over rows wave, wave+4, ...
    {
      const float alpha = s_alpha[pv_g];
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[i] *= alpha;
      for (int r = wave; r < n; r += kThreads / kWave) {
        const float pr = s_p[pv_g][r];
        const uint16_t* vrow = &s_v[r][pv_d0];
#pragma unroll
        for (int i2 = 0; i2 < DPL / 2; ++i2) {
          const uint32_t w2 = *reinterpret_cast<const uint32_t*>(vrow + 2 * i2);
          acc[2 * i2] += pr * __uint_as_float(w2 << 16);
          acc[2 * i2 + 1] += pr * __uint_as_float(w2 & 0xFFFF0000u);
        }
        if (DPL == 1) acc[0] += pr * __uint_as_float((uint32_t)vrow[0] << 16);
      }
    }
    __syncthreads();
  }

  // reduce the four waves' partial sums
#pragma unroll
  for (int i = 0; i < DPL; ++i) s_red[wave][lane][i] = acc[i];
  __syncthreads();
  // thread tid < 64 (wave 0) now owns (pv_g, pv_d0 .. pv_d0 + DPL)
  float tot[DPL];
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) tot[i] = s_red[0][lane][i] + s_red[1][lane][i] + s_red[2][lane][i] + s_red[3][lane][i];
  }
  if (num_splits == 1) {
    if (wave == 0) {
      const float inv = 1.0f / s_l[pv_g];
      bf16_t* op = out + b * os_b + (int64_t)(h * G + pv_g) * os_h + pv_d0;
#pragma unroll
      for (int i = 0; i < DPL; ++i) op[i].bits = (uint16_t)f32_to_bf16(tot[i] * inv);
    }
    return;
  }
  constexpr int64_t kStride = (int64_t)G * (D + 2);
  float* mine = ws + ((int64_t)pair * num_splits + split) * kStride;
  if (tid < G) {
    store_agent(mine + tid, s_m[tid]);
    store_agent(mine + G + tid, s_l[tid]);
  }
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) store_agent(mine + 2 * G + pv_g * D + pv_d0 + i, tot[i]);
  }
  if (!take_last_ticket(&counters[pair], num_splits, &s_last)) return;
  const float* all = ws + (int64_t)pair * num_splits * kStride;
  for (int o = tid; o < G * D; o += kThreads) {
    const int g = o / D;
    float M = -INFINITY;
    for (int s2 = 0; s2 < num_splits; ++s2) M = fmaxf(M, load_agent(all + s2 * kStride + g));
    float L = 0.0f, A = 0.0f;
    for (int s2 = 0; s2 < num_splits; ++s2) {
      const float* ps = all + s2 * kStride;
      const float ms = load_agent(ps + g);
      const float wgt = (ms == -INFINITY) ? 0.0f : exp2f(ms - M);
      L += load_agent(ps + G + g) * wgt;
      A += load_agent(ps + 2 * G + o) * wgt;
    }
    out[b * os_b + (int64_t)(h * G + g) * os_h + (o - g * D)].bits = (uint16_t)f32_to_bf16(A / L);
  }
  if (tid == 0) __hip_atomic_store(&counters[pair], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Wave-local fast path (G <= 4): each wave owns a contiguous run of the
// workgroup's rows and streams it in wave tiles of RT = NP * 64 / C rows, the
// next tile's K/V already in flight while the current one is computed.  C
// lanes share a row (one 16-byte chunk each): their partial dots are summed
// with DPP, so every lane of the row holds the row's score and can apply its
// probability to its own V chunk -- P.V accumulates in registers with a
// per-lane running max and no barrier or LDS traffic inside the loop.  Lanes
// and waves are combined once at the end (DPP row rotations, then LDS), and
// split partials are merged by the last workgroup of a (b, h) pair.  The
// partials travel as agent-scope atomic stores / loads (coherent across XCDs
// without an L2 write-back), ordered by a wait for their completion before
// the ticket increment.
// ---------------------------------------------------------------------------
namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// sum over the C consecutive lanes of a row group (C = 4, 8, 16)
template <int C>
__device__ __forceinline__ float row_group_sum(float v) {
  v += dpp_f<0xB1>(v);                       // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);                       // quad_perm [2,3,0,1]
  if constexpr (C >= 8) v += dpp_f<0x141>(v);   // row_half_mirror
  if constexpr (C >= 16) v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

// sum over the lanes of a 16-lane row that hold the same chunk (lane % C)
template <int C>
__device__ __forceinline__ float same_chunk_row_sum(float v) {
  if constexpr (C <= 4) v += dpp_f<0x124>(v);   // row_ror:4
  if constexpr (C <= 8) v += dpp_f<0x128>(v);   // row_ror:8
  return v;
}


}  // namespace

template <int D, int G, typename KT, int NP>
__global__ __launch_bounds__(kThreads) void decode_attn_wave_kernel(
    const bf16_t* __restrict__ q, int64_t qs_b, int64_t qs_h, const KT* __restrict__ ck, const KT* __restrict__ cv,
    int64_t c_s, const int32_t* __restrict__ base_offsets, int64_t bo_b, int64_t bo_h,
    const int32_t* __restrict__ block_tables, int64_t bt_b, int64_t bt_h, int page_shift, int paged,
    const int32_t* __restrict__ live_counts, int64_t lc_b, int64_t lc_h, bf16_t* __restrict__ out, int64_t os_b,
    int64_t os_h, float* __restrict__ ws, int* __restrict__ counters, int num_kv_heads, int num_pairs,
    int num_splits, float scale, const float* __restrict__ rope_cs, int64_t rcs_p, int64_t rcs_d,
    const int64_t* __restrict__ rope_pos) {
  constexpr int EPC = RowLoad<KT>::kEpc;
  constexpr int C = D / EPC;       // lanes per row
  constexpr int RPI = 64 / C;      // rows per load instruction (per wave)
  constexpr int RT = RPI * NP;     // rows per wave tile
  constexpr int kWaves = kThreads / kWave;
  constexpr int kRows16 = 4;       // 16-lane rows per wave
  static_assert(C == 4 || C == 8 || C == 16, "row split");
  __shared__ __attribute__((aligned(16))) float s_q[G][D];
  __shared__ float s_wm[kWaves][G], s_wl[kWaves][G];
  __shared__ __attribute__((aligned(16))) float s_buf[kWaves][kRows16][C][G][EPC];
  __shared__ float s_M[G], s_L[G];
  __shared__ int s_last;

  const int lin = blockIdx.x;
  const int xcd = lin % kXcds;
  const int slot = lin / kXcds;
  const int pair = (slot / num_splits) * kXcds + xcd;
  const int split = slot - (slot / num_splits) * num_splits;
  if (pair >= num_pairs) return;  // uniform per workgroup
  const int b = pair / num_kv_heads;
  const int h = pair - b * num_kv_heads;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;

  const int live = live_counts[b * lc_b + h * lc_h];
  const int per = (live + num_splits - 1) / num_splits;
  const int t0 = min(live, split * per);
  const int t1 = min(live, t0 + per);
  const int wq = (t1 - t0 + kWaves - 1) / kWaves;
  const int w0 = min(t1, t0 + wave * wq);
  const int w1 = min(t1, w0 + wq);
  const int64_t bo = paged ? 0 : (int64_t)base_offsets[b * bo_b + h * bo_h];
  const SpanAddr addr{base_offsets, block_tables, bt_b, bt_h, page_shift, paged};
  const float qscale = scale * kLog2e;

  if (rope_pos) {
    constexpr int half = D / 2;
    const int64_t pos = rope_pos[b];
    for (int i = tid; i < G * half; i += kThreads) {
      const int g = i / half, j = i - g * half;
      const bf16_t* qh = q + b * qs_b + (int64_t)(h * G + g) * qs_h;
      const float x1 = ld<bf16_t>(qh + j);
      const float x2 = (g == 0 && j == half - 1) ? 0.0f : ld<bf16_t>(qh + j + half);
      float y1, y2;
      rope_f32(x1, x2, rope_cs[pos * rcs_p + (int64_t)j * rcs_d], rope_cs[pos * rcs_p + (int64_t)(j + half) * rcs_d],
               &y1, &y2);
      s_q[g][j] = y1 * qscale;
      s_q[g][j + half] = y2 * qscale;
    }
  } else {
    for (int i = tid; i < G * D; i += kThreads) {
      const int g = i / D, d = i - g * D;
      s_q[g][d] = ld<bf16_t>(q + b * qs_b + (int64_t)(h * G + g) * qs_h + d) * qscale;
    }
  }
  __syncthreads();

  const int chunk = lane % C;
  const int rowi = lane / C;
  float qf[G][EPC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < EPC; ++e) qf[g][e] = s_q[g][chunk * EPC + e];

  float m[G], l[G], acc[G][EPC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[g][e] = 0.0f;
  }

  uint4 kc[NP], vc[NP], kn[NP], vn[NP];
  auto load_tile = [&](int ts, uint4* kk, uint4* vv) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int r = ts + p * RPI + rowi;
      kk[p] = uint4{0u, 0u, 0u, 0u};
      vv[p] = uint4{0u, 0u, 0u, 0u};
      if (r < w1) {
        const int64_t row = addr.row(b, h, bo, r);
        kk[p] = *reinterpret_cast<const uint4*>(ck + row * c_s + chunk * EPC);
        vv[p] = *reinterpret_cast<const uint4*>(cv + row * c_s + chunk * EPC);
      }
    }
  };
  if (w0 < w1) load_tile(w0, kc, vc);
  for (int ts = w0; ts < w1; ts += RT) {
    const bool more = ts + RT < w1;
    if (more) load_tile(ts + RT, kn, vn);
    float sc[NP][G];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float kf[EPC];
      RowLoad<KT>::to_f32(kc[p], kf);
      const bool valid = ts + p * RPI + rowi < w1;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < EPC; ++e) a += qf[g][e] * kf[e];
        a = row_group_sum<C>(a);
        sc[p][g] = valid ? a : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = sc[0][g];
#pragma unroll
      for (int p = 1; p < NP; ++p) mx = fmaxf(mx, sc[p][g]);
      const float m_new = fmaxf(m[g], mx);
      if (m_new != -INFINITY) {  // lanes whose rows are all past the end keep their state
        const float alpha = exp2f(m[g] - m_new);
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[g][e] *= alpha;
        m[g] = m_new;
      }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float vf[EPC];
      RowLoad<KT>::to_f32(vc[p], vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = (sc[p][g] == -INFINITY) ? 0.0f : exp2f(sc[p][g] - m[g]);
        l[g] += (chunk == 0) ? pr : 0.0f;
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[g][e] += pr * vf[e];
      }
    }
    if (more) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        kc[p] = kn[p];
        vc[p] = vn[p];
      }
    }
  }

  // workgroup max per head, then rescale every lane to it
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float wm = wave_max(m[g]);
    if (lane == 0) s_wm[wave][g] = wm;
  }
  __syncthreads();
  if (tid < G) {
    float M = s_wm[0][tid];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_wm[w][tid]);
    s_M[tid] = M;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float M = s_M[g];
    const float f = (m[g] == -INFINITY || M == -INFINITY) ? 0.0f : exp2f(m[g] - M);
    const float lw = wave_sum(l[g] * f);
    if (lane == 0) s_wl[wave][g] = lw;
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[g][e] = same_chunk_row_sum<C>(acc[g][e] * f);
  }
  // lanes 0..C-1 of each 16-lane row now hold that row's sums for their chunk
  if ((lane & 15) < C) {
    const int r16 = lane >> 4;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < EPC; ++e) s_buf[wave][r16][lane & 15][g][e] = acc[g][e];
  }
  __syncthreads();
  if (tid < G) {
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) L += s_wl[w][tid];
    s_L[tid] = L;
  }
  __syncthreads();

  constexpr int kOut = G * D;
  if (num_splits == 1) {
    for (int o = tid; o < kOut; o += kThreads) {
      const int g = o / D, d = o - g * D;
      const int cidx = d / EPC, e = d - cidx * EPC;
      float A = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w)
#pragma unroll
        for (int r = 0; r < kRows16; ++r) A += s_buf[w][r][cidx][g][e];
      out[b * os_b + (int64_t)(h * G + g) * os_h + d].bits = (uint16_t)f32_to_bf16(A / s_L[g]);
    }
    return;
  }
  constexpr int64_t kStride = (int64_t)G * (D + 2);
  float* mine = ws + ((int64_t)pair * num_splits + split) * kStride;
  if (tid < G) {
    store_agent(mine + tid, s_M[tid]);
    store_agent(mine + G + tid, s_L[tid]);
  }
  for (int o = tid; o < kOut; o += kThreads) {
    const int g = o / D, d = o - g * D;
    const int cidx = d / EPC, e = d - cidx * EPC;
    float A = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
#pragma unroll
      for (int r = 0; r < kRows16; ++r) A += s_buf[w][r][cidx][g][e];
    store_agent(mine + 2 * G + o, A);
  }
  if (!take_last_ticket(&counters[pair], num_splits, &s_last)) return;
  const float* all = ws + (int64_t)pair * num_splits * kStride;
  for (int o = tid; o < kOut; o += kThreads) {
    const int g = o / D;
    float M = -INFINITY, L = 0.0f, A = 0.0f;
    for (int s0 = 0; s0 < num_splits; s0 += kMergeBatch) {
      // issue the batch's loads together: one memory round trip per batch
      float mv[kMergeBatch], lv[kMergeBatch], av[kMergeBatch];
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) {
        mv[j] = -INFINITY;
        lv[j] = av[j] = 0.0f;
        if (s0 + j < num_splits) {
          const float* ps = all + (s0 + j) * kStride;
          mv[j] = load_agent(ps + g);
          lv[j] = load_agent(ps + G + g);
          av[j] = load_agent(ps + 2 * G + o);
        }
      }
      float bm = M;
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) bm = fmaxf(bm, mv[j]);
      const float f = (M == -INFINITY || bm == -INFINITY) ? 0.0f : exp2f(M - bm);
      L *= f;
      A *= f;
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) {
        const float wgt = (mv[j] == -INFINITY) ? 0.0f : exp2f(mv[j] - bm);
        L += lv[j] * wgt;
        A += av[j] * wgt;
      }
      M = bm;
    }
    out[b * os_b + (int64_t)(h * G + g) * os_h + (o - g * D)].bits = (uint16_t)f32_to_bf16(A / L);
  }
  if (tid == 0) __hip_atomic_store(&counters[pair], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Matrix-core path (FP8 K/V, bf16 q, G <= 4, D = 64 / 128).
//
// Both products run on the 16-block 4x4x4 MFMA (v_mfma_f32_4x4x4_16b_*).  A
// wave takes its tokens in groups of 64; lane l = 4*s + k (s = 0..15,
// k = 0..3) owns token s + 16*k of the group.
//   QK^T: block s, A = K rows of the lane's token, D/4 dims at a time
//         (fp8 -> bf16 is exact), B = Q[head j][dims] (bf16).  Register r of
//         lane (s, j) ends up holding S[token s + 16*r][head j].
//   P.V:  16 steps; at step s every block multiplies block s's A -- lane
//         (s, i)'s four probabilities P[head i][tokens s + 16*k], broadcast
//         by the instruction itself (CBSZ = 4, ABID = s) -- with
//         B = V[tokens s + 16*k][dim 4*b + j] (fp8 -> f16, exact).  Each
//         lane (b, j) accumulates O[heads 0..3][dim 4*b + j] (+ 64 for
//         D = 128): no reduction across lanes is needed afterwards.
//         The B operands come from a per-wave transposed copy of the group's
//         V in LDS (VT[dim][s] = bytes of tokens s, s+16, s+32, s+48), made
//         with byte permutes from the lane's own 16-byte row slices.
// Scores are scaled (scale * log2 e) in fp32 after the product; the softmax
// is online per group with a wave-wide maximum per head, so a rescale costs
// four multiplies.  P enters the P.V product rounded to f16 (relative error
// <= 2^-11); the denominator sums the fp32 values.  A workgroup covers one
// (seq, kv head) pair, or one 64-aligned split of it; splits are merged by
// the last workgroup of the pair as in the kernels above.
// ---------------------------------------------------------------------------
namespace {

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef _Float16 v4f16_t __attribute__((ext_vector_type(4)));
typedef float v4f32_t __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v4i16_t fp8x4_to_bf16x4(uint32_t w) {
  const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false));
  const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true));
  return __builtin_bit_cast(v4i16_t, v2u32_t{lo, hi});
}
__device__ __forceinline__ v4f16_t fp8x4_to_f16x4(uint32_t w) {
  const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, false));
  const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, true));
  return __builtin_bit_cast(v4f16_t, v2u32_t{lo, hi});
}

// Sum / max over the 16 lanes of a wave that share lane % 4.
__device__ __forceinline__ float blocks_sum(float v) {
  v += dpp_f<0x128>(v);  // row_ror:8
  v += dpp_f<0x124>(v);  // row_ror:4
  return rows_sum(v);    // lanes l^16, l^32
}
__device__ __forceinline__ float blocks_max(float v) {
  v = fmaxf(v, dpp_f<0x128>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  return rows_max(v);
}
// value of lane (l & ~3) + I (quad broadcast)
template <int I>
__device__ __forceinline__ float quad_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), I * 0x55, 0xF, 0xF, true));
}

// A group's K row words (the lane's token) and V row slices (tokens s + 16*kk,
// bytes [D/4 * q, D/4 * (q + 1)) with q = lane % 4), zero past `end`.
template <int D>
struct MfmaGroup {
  static constexpr int kW = D / 4;   // words of K per lane, and of V per lane
  uint32_t k[kW];
  uint32_t v[4][kW / 4];
};

// Row of span rank r (flat: bo + r; paged: through the block table).
template <bool PAGED>
__device__ __forceinline__ int64_t span_row(const SpanAddr& addr, int b, int h, int64_t bo, int r) {
  if constexpr (PAGED) {
    const int32_t page = addr.table[b * addr.tb_b + h * addr.tb_h + (r >> addr.page_shift)];
    return ((int64_t)page << addr.page_shift) + (r & ((1 << addr.page_shift) - 1));
  } else {
    return bo + r;
  }
}

// Loads are unconditional: ranks past `end` read row end-1 (live, so finite)
// instead, which keeps the wait counters exact across the loop.  Their
// scores are masked to -inf, so their K and V never reach the output.
// Flat spans address rows from the span's first row (kspan / vspan, uniform)
// with 32-bit offsets; paged spans go through the block table.  The address
// step and the load step are separate so that the table reads of several
// groups share one scalar-memory wait.
template <int D>
struct MfmaGroupAddr {
  const uint4* k;
  const uint4* v[4];
};

// Paged group with its quarters' page rows known (qrow[kk] = physical row of
// the first row of the page holding rows g0 + 16 kk .. g0 + 16 kk + 15,
// clamped to `end` - 1).
template <int D>
__device__ __forceinline__ void mfma_group_addr_paged(MfmaGroupAddr<D>& ga, const uint8_t* __restrict__ kspan,
                                                      const uint8_t* __restrict__ vspan, int64_t c_s,
                                                      const int64_t (&qrow)[4], int page_shift, int g0, int end,
                                                      int lane) {
  const int s = lane >> 2, q = lane & 3;
  const int last = end - 1;
  const int mask = (1 << page_shift) - 1;
  const int64_t kq = q == 0 ? qrow[0] : q == 1 ? qrow[1] : q == 2 ? qrow[2] : qrow[3];
  ga.k = reinterpret_cast<const uint4*>(kspan + (kq + (min(g0 + s + 16 * q, last) & mask)) * c_s);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    ga.v[kk] = reinterpret_cast<const uint4*>(vspan + (qrow[kk] + (min(g0 + s + 16 * kk, last) & mask)) * c_s +
                                              q * (D / 4));
}

template <int D, bool PAGED>
__device__ __forceinline__ void mfma_group_addr(MfmaGroupAddr<D>& ga, const uint8_t* __restrict__ kspan,
                                                const uint8_t* __restrict__ vspan, int64_t c_s,
                                                const SpanAddr& addr, int b, int h, int g0, int end, int lane) {
  const int s = lane >> 2, q = lane & 3;
  if constexpr (PAGED) {
    // A group starts 64-row aligned and pages hold >= 16 rows (the host
    // checks), so each 16-row quarter of the group lies in one page: its id
    // is a wave-uniform value, read through the scalar cache (the tables are
    // not written during the launch), instead of a table load per lane.
    using const_i32 = const __attribute__((address_space(4))) int32_t;
    const_i32* trow = (const_i32*)(addr.table + b * addr.tb_b + h * addr.tb_h);
    const int last = end - 1;
    int64_t qrow[4];  // physical row of the first row of each quarter's page
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int r0 = __builtin_amdgcn_readfirstlane(min(g0 + 16 * kk, last));
      qrow[kk] = (int64_t)trow[r0 >> addr.page_shift] << addr.page_shift;
    }
    mfma_group_addr_paged<D>(ga, kspan, vspan, c_s, qrow, addr.page_shift, g0, end, lane);
    (void)s;
    (void)q;
  } else {
    const uint32_t cs = (uint32_t)c_s;
    ga.k = reinterpret_cast<const uint4*>(kspan + __umul24((uint32_t)min(g0 + s + 16 * q, end - 1), cs));
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      ga.v[kk] = reinterpret_cast<const uint4*>(vspan + (__umul24((uint32_t)min(g0 + s + 16 * kk, end - 1), cs) +
                                                         (uint32_t)(q * (D / 4))));
  }
}

template <int D>
__device__ __forceinline__ void mfma_issue_group(MfmaGroup<D>& g, const MfmaGroupAddr<D>& ga) {
  constexpr int KQ = D / 16;  // 16-byte chunks per K row
  constexpr int VQ = D / 64;  // 16-byte chunks per V slice
#pragma unroll
  for (int m = 0; m < KQ; ++m) {
    const uint4 x = ga.k[m];
    g.k[4 * m] = x.x;
    g.k[4 * m + 1] = x.y;
    g.k[4 * m + 2] = x.z;
    g.k[4 * m + 3] = x.w;
  }
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int m = 0; m < VQ; ++m) {
      const uint4 x = ga.v[kk][m];
      g.v[kk][4 * m] = x.x;
      g.v[kk][4 * m + 1] = x.y;
      g.v[kk][4 * m + 2] = x.z;
      g.v[kk][4 * m + 3] = x.w;
    }
}

template <int D, bool PAGED>
__device__ __forceinline__ void mfma_load_group(MfmaGroup<D>& g, const uint8_t* __restrict__ kspan,
                                                const uint8_t* __restrict__ vspan, int64_t c_s,
                                                const SpanAddr& addr, int b, int h, int g0, int end, int lane) {
  MfmaGroupAddr<D> ga;
  mfma_group_addr<D, PAGED>(ga, kspan, vspan, c_s, addr, b, h, g0, end, lane);
  mfma_issue_group<D>(g, ga);
}

constexpr int kVtStride = 20;  // dwords per dim row of the transposed V tile (16 steps + pad)

}  // namespace

// Inputs of the decode preprocess fused in front of the attention (the
// reference's fused_dms_rope_store_compact_decode, compact_attention.py:67-209):
// raw k / v rows of the step, RoPE table and positions, append slots, DMS
// decision output and threshold.
struct DecodePre {
  const bf16_t* k;
  int64_t ks_b, ks_h;
  const bf16_t* v;
  int64_t vs_b, vs_h;
  const float* cos_sin;
  int64_t cs_p, cs_d;
  const int64_t* positions;
  const int32_t* slot;
  int64_t sm_b, sm_h;
  uint8_t* evict_out;
  int64_t ev_b, ev_h;
  float alpha_scale, alpha_offset, threshold;
  int positive_scale;
  // Qwen3 QK-norm (or NULL): q / k rows are RMS-normalised per head with
  // these [head_dim] bf16 weights before the decision and RoPE
  const bf16_t* q_norm;
  const bf16_t* k_norm;
  float norm_eps;
};


// The first ten arguments are what a workgroup needs before its first
// loads (the planned launch's work plan; its pair, live count, and for the
// fused kernel the step's append slot and position); this file is built with
// them preloaded into SGPRs at
// wave launch (-amdgpu-kernarg-preload-count), which takes one scalar memory
// round trip off that chain (the page table is read only after the live
// count, by when the other arguments have landed).  Strides are int32 (the
// hosts check the range).
// Four waves per SIMD asked for (at most 128 VGPRs; met at head_dim 64, not
// at 128, which stays at 130 without spilling): once a launch fills the chip
// the kernel is bound by how many rows are in flight (7 % faster at 128
// sequences than at the unconstrained 130 VGPRs).
template <int D, int NW, bool PAGED, bool FUSED, bool PLANNED = false>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(4))) void decode_attn_mfma_kernel(
    const int32_t* __restrict__ plan, const int32_t* __restrict__ live_counts, int lc_b, int lc_h, const int32_t* __restrict__ fslot, int sm_b,
    int sm_h, const int64_t* __restrict__ fpositions, int num_pairs, int num_kv_heads,
    const bf16_t* __restrict__ q, int64_t qs_b, int64_t qs_h, uint8_t* __restrict__ ck,
    uint8_t* __restrict__ cv, int64_t c_s, const int32_t* __restrict__ base_offsets, int64_t bo_b,
    int64_t bo_h, const int32_t* __restrict__ block_tables, int bt_b, int bt_h, int page_shift, int paged,
    bf16_t* __restrict__ out, int64_t os_b,
    int64_t os_h, float* __restrict__ ws, int* __restrict__ counters, int group_size,
    int num_splits, int split_rows, int heavy_rows, float scale, const float* __restrict__ rope_cs, int64_t rcs_p,
    int64_t rcs_d, const int64_t* __restrict__ rope_pos, const DecodePre pre, const float* __restrict__ k_scale,
    const float* __restrict__ v_scale) {
  constexpr int NT = NW * kWave;
  constexpr int NWX = FUSED ? NW + 1 : NW;  // combine slots: the waves (+ the appended token)
  constexpr int KW = MfmaGroup<D>::kW;
  constexpr int VW = KW / 4;    // V words per token slice
  constexpr int NA = D / 64;    // accumulator quads per lane
  __shared__ __attribute__((aligned(16))) uint16_t s_q[4][D];  // bf16 q, heads >= G zero
  __shared__ __attribute__((aligned(16))) uint32_t s_vt[NW][D * kVtStride];
  __shared__ float s_wm[NWX][4], s_wl[NWX][4];
  __shared__ __attribute__((aligned(16))) float s_wacc[NWX][4][D];
  __shared__ float s_knew[FUSED ? D : 1], s_vnew[FUSED ? D : 1];  // appended row as stored (FP8 values)
  __shared__ int s_last;

  // Work split: workgroup (pair, split), split-major: block ids are
  // dispatched in order, so split 0 of every pair goes out first and the
  // workgroups past a pair's split count (the grid holds the host's bound
  // for the batch; they exit after one load) come last instead of between
  // the working ones.  The padded pair count is a multiple of the 8 XCDs
  // (block ids go round-robin over them), so all splits of a pair run on one
  // XCD and their partials meet in its L2.  Pair (b, h) takes ns =
  // ceil(live / split_rows) splits (at most num_splits) of at most
  // split_rows rows each.
  static_assert(!PLANNED || (PAGED && FUSED && NW == kPlanWaves), "a plan item is two groups per wave at most");
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps the group loop scalar
  const int lane = tid & 63;
  const int jj = lane & 3, ss = lane >> 2;
  const int G = group_size;
  int split, pair, b, h, live;
  int64_t fpos = 0;
  int32_t app_slot = -1;
  [[maybe_unused]] int plan_ns = 1, plan_t0 = 0, plan_t1 = 0;
  [[maybe_unused]] bool plan_new = false;
  [[maybe_unused]] int64_t plan_qrow[4] = {0, 0, 0, 0}, plan_qrow2[4] = {0, 0, 0, 0};
  if constexpr (PLANNED) {
    // Workgroup p < num_pairs runs split 0 of pair p: its raw rows and
    // position load at once, beside its plan item (fdms_plan.h); a later
    // workgroup runs a further split, named by its item, up to the layer's
    // count of those.  The item arrives as one 16-byte word per lane (lanes
    // past the item re-read its last word) with everything the K/V loads need.
    const int lin = blockIdx.x;
    const bool first = lin < num_pairs;  // uniform per workgroup
    const int extra = first ? 0 : plan[-1];  // the layer's further splits, stored before its items
    const uint4 w = reinterpret_cast<const uint4*>(plan + (int64_t)lin * kPlanInts)[min(lane, kPlanInts / 4 - 1)];
    if (!first && lin >= num_pairs + extra) return;  // uniform: past the step's items
    pair = first ? lin : __builtin_amdgcn_readlane((int)w.x, 0);
    b = pair / num_kv_heads;
    h = pair - b * num_kv_heads;
    fpos = fpositions[b];
    plan_t0 = __builtin_amdgcn_readlane((int)w.y, 0);
    plan_t1 = __builtin_amdgcn_readlane((int)w.z, 0);
    split = __builtin_amdgcn_readlane((int)w.w, 0) & 0xFFFF;
    plan_ns = __builtin_amdgcn_readlane((int)w.w, 0) >> 16;
    live = __builtin_amdgcn_readlane((int)w.x, 1);
    app_slot = __builtin_amdgcn_readlane((int)w.y, 1);
    plan_new = (__builtin_amdgcn_readlane((int)w.w, 1) & 1) != 0;
    // this wave's groups w and w + 8: the page ids of their 16-row quarters
    const int pl = kPlanHeader / 4 + wave;
    plan_qrow[0] = (int64_t)__builtin_amdgcn_readlane((int)w.x, pl) << kPlanPageShift;
    plan_qrow[1] = (int64_t)__builtin_amdgcn_readlane((int)w.y, pl) << kPlanPageShift;
    plan_qrow[2] = (int64_t)__builtin_amdgcn_readlane((int)w.z, pl) << kPlanPageShift;
    plan_qrow[3] = (int64_t)__builtin_amdgcn_readlane((int)w.w, pl) << kPlanPageShift;
    plan_qrow2[0] = (int64_t)__builtin_amdgcn_readlane((int)w.x, pl + kPlanWaves) << kPlanPageShift;
    plan_qrow2[1] = (int64_t)__builtin_amdgcn_readlane((int)w.y, pl + kPlanWaves) << kPlanPageShift;
    plan_qrow2[2] = (int64_t)__builtin_amdgcn_readlane((int)w.z, pl + kPlanWaves) << kPlanPageShift;
    plan_qrow2[3] = (int64_t)__builtin_amdgcn_readlane((int)w.w, pl + kPlanWaves) << kPlanPageShift;
  } else {
    const int lin = blockIdx.x;
    const int padded_pairs = ((num_pairs + kXcds - 1) / kXcds) * kXcds;
    split = lin / padded_pairs;
    pair = lin - split * padded_pairs;
    if (pair >= num_pairs) return;  // uniform per workgroup
    b = pair / num_kv_heads;
    h = pair - b * num_kv_heads;

    // Prologue order (each step issues what does not depend on the step after
    // it, so the first K/V rows arrive after three memory latencies: live
    // count, page ids, rows): the per-pair scalars (live count, the fused
    // step's position and append slot), then the raw rows as bits (no use
    // before the span loads are out), then the RoPE table row.
    if constexpr (FUSED) fpos = fpositions[b];
    live = live_counts[(int64_t)b * lc_b + (int64_t)h * lc_h];
    if constexpr (FUSED) {
      app_slot = fslot[(int64_t)b * sm_b + (int64_t)h * sm_h];
      // the three loads share one wait: keeps the position load from being
      // sunk past the early exit below into a round trip of its own
      asm volatile("" ::"s"(fpos), "s"(live), "s"(app_slot));
    }
  }

  // q elements of this thread (non-fused path without RoPE)
  constexpr int QPT = (4 * D + NT - 1) / NT;  // q elements per thread
  uint32_t qraw[QPT];
#pragma unroll
  for (int x = 0; x < QPT; ++x) {
    const int i = tid + x * NT;
    const int g = i / D, d = i - g * D;
    qraw[x] = (i < 4 * D && g < G) ? (uint32_t)q[b * qs_b + (int64_t)(h * G + g) * qs_h + d].bits : 0u;
  }

  // fused preprocess: this thread's raw q pair, k pair or v element (bf16
  // bits, from one load site so that no load waits for another) and its
  // RoPE cos / sin
  constexpr int kHalf = D / 2;
  uint32_t fb1 = 0u, fb2 = 0u;  // raw pair / element
  uint32_t fw1 = 0u, fw2 = 0u;  // QK-norm weights of the pair (bf16 bits)
  float fc = 0.0f, fsn = 0.0f;  // RoPE cos and sin
  if constexpr (FUSED) {
    static_assert(NT >= 5 * kHalf + D, "one preprocess item per thread");
    // threads without an item (and q heads past G) read the pair's first q
    // element and ignore it
    const bf16_t* src = q + b * qs_b + (int64_t)(h * G) * qs_h;
    int second = 0;  // offset of the pair's second element (0: a v element, read twice)
    if (tid < 4 * kHalf) {
      const int g = tid / kHalf, jx = tid - g * kHalf;
      if (g < G) {
        src += (int64_t)g * qs_h + jx;
        second = kHalf;
      }
    } else if (tid < 5 * kHalf) {
      src = pre.k + b * pre.ks_b + h * pre.ks_h + (tid - 4 * kHalf);
      second = kHalf;
    } else if (tid < 5 * kHalf + D) {
      src = pre.v + b * pre.vs_b + h * pre.vs_h + (tid - 5 * kHalf);
    }
    fb1 = src[0].bits;
    fb2 = src[second].bits;
    if (tid < 5 * kHalf) {
      const int jx = tid % kHalf;
      const float* cs = pre.cos_sin + fpos * pre.cs_p;
      fc = cs[(int64_t)jx * pre.cs_d];
      fsn = cs[(int64_t)(jx + kHalf) * pre.cs_d];
      const bf16_t* nw = tid < 4 * kHalf ? pre.q_norm : pre.k_norm;
      if (nw) {
        fw1 = nw[jx].bits;
        fw2 = nw[jx + kHalf].bits;
      }
    }
  }

  const int64_t bo = PAGED ? 0 : (int64_t)base_offsets[b * bo_b + h * bo_h];
  const SpanAddr addr{base_offsets, block_tables, bt_b, bt_h, page_shift, paged};
  // a pair up to split_rows rows is one workgroup (no merge); a longer one
  // takes splits of heavy_rows rows (<= split_rows), so the pairs that pay
  // the merge chain get shorter loops
  int ns, t0, t1;
  bool new_tok = false;
  if constexpr (PLANNED) {
    ns = plan_ns;
    t0 = plan_t0;
    t1 = plan_t1;  // the plan already leaves the appended rank out
    new_tok = plan_new;
  } else {
    ns = live <= split_rows ? 1 : min(num_splits, (live + heavy_rows - 1) / heavy_rows);
    if (split >= ns) return;  // uniform per workgroup
    const int per = (((live + ns - 1) / ns) + 63) & ~63;
    t0 = min(live, split * per);
    t1 = min(live, t0 + per);
    // Fused preprocess: the step's token is rank live - 1 (slot >= 0); its row is
    // being written by this launch, so no workgroup reads it back -- the split
    // holding that rank adds the token from the values it computes itself.
    if constexpr (FUSED) {
      if (app_slot >= 0 && live > 0) {
        new_tok = t0 < live && t1 == live;
        t1 = min(t1, live - 1);
      }
    }
  }
  const int ngroups = max(0, (t1 - t0 + 63) >> 6);

  const uint8_t* kspan = PAGED ? ck : ck + bo * c_s;  // flat: the span's first row
  const uint8_t* vspan = PAGED ? cv : cv + bo * c_s;
  // The wave's first group goes in flight now.  Its loads are unconditional
  // once the split has a group: a wave past the end reads row t1 - 1 (live
  // and finite) and never processes it, which keeps the wait counts exact.
  // Its four page ids are read first (lanes 0-3, one vector load); the raw
  // rows issued above are waited for before the span loads go out (they have
  // had the live-count and page-id latencies to land), so the preprocess
  // below never waits for span rows.
  MfmaGroup<D> cur;
  if constexpr (PLANNED) {
    // the page ids came with the item: the group's K/V loads go out right
    // behind the raw rows (the preprocess waits for those only)
    if (ngroups > 0) {
      MfmaGroupAddr<D> ga;
      mfma_group_addr_paged<D>(ga, ck, cv, c_s, plan_qrow, kPlanPageShift, t0 + wave * 64, t1, lane);
      mfma_issue_group<D>(cur, ga);
    }
  } else {
  int32_t pid = 0;  // paged: lane kk reads the page id of quarter kk
  if constexpr (PAGED) {
    if (ngroups > 0 && lane < 4) {
      const int r0 = min(t0 + wave * 64 + 16 * lane, t1 - 1);
      pid = block_tables[(int64_t)b * bt_b + (int64_t)h * bt_h + (r0 >> page_shift)];
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): raw rows, RoPE row and page ids have landed
  if (ngroups > 0) {
    MfmaGroupAddr<D> ga;
    const int g0 = t0 + wave * 64;
    if constexpr (PAGED) {
      int64_t qrow[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qrow[kk] = (int64_t)__builtin_amdgcn_readlane(pid, kk) << page_shift;
      mfma_group_addr_paged<D>(ga, kspan, vspan, c_s, qrow, page_shift, g0, t1, lane);
    } else {
      mfma_group_addr<D, false>(ga, kspan, vspan, c_s, addr, b, h, g0, t1, lane);
    }
    mfma_issue_group<D>(cur, ga);
  }
  }
  [[maybe_unused]] float fx1 = __uint_as_float(fb1 << 16), fx2 = __uint_as_float(fb2 << 16);
  if constexpr (FUSED) {
    // QK-norm (layernorm.py:19-40 on each q / k head, qwen3.py:92-94, before
    // the DMS extraction): x_out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w).
    // A head's kHalf pair threads are an aligned lane segment; the sum runs
    // on every lane (no divergent shuffles) and only q / k threads use it.
    if (pre.q_norm || pre.k_norm) {
      const float ss = segment_sum<kHalf>(fx1 * fx1 + fx2 * fx2);
      const bool on = tid < 4 * kHalf ? pre.q_norm != nullptr : (tid < 5 * kHalf && pre.k_norm != nullptr);
      if (on) {
        const float inv = rsqrtf(ss / (float)D + pre.norm_eps);
        fx1 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(fx1 * inv)) * __uint_as_float(fw1 << 16)));
        fx2 = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(fx2 * inv)) * __uint_as_float(fw2 << 16)));
      }
    }
  }

  if constexpr (FUSED) {
    // decode preprocess: q pairs (decision lane read, then zeroed), the key
    // pair j and the value element d of the step's row; the workgroup of split
    // 0 writes the decision and appends the FP8 row at the slot
    if (tid < 4 * kHalf) {
      const int g = tid / kHalf, jx = tid - g * kHalf;
      uint32_t y1b = 0u, y2b = 0u;
      if (g < G) {
        float x2 = fx2;
        if (g == 0 && jx == kHalf - 1) {
          if (split == 0)
            pre.evict_out[b * pre.ev_b + h * pre.ev_h] =
                dms_decide(x2, pre.alpha_scale, pre.alpha_offset, pre.threshold, pre.positive_scale) ? 1 : 0;
          x2 = 0.0f;
        }
        float y1, y2;
        rope_f32(fx1, x2, fc, fsn, &y1, &y2);
        y1b = f32_to_bf16(y1);
        y2b = f32_to_bf16(y2);
      }
      s_q[g][jx] = (uint16_t)y1b;
      s_q[g][jx + kHalf] = (uint16_t)y2b;
    } else if (tid < 5 * kHalf) {
      const int jx = tid - 4 * kHalf;
      float y1, y2;
      rope_f32(fx1, fx2, fc, fsn, &y1, &y2);
      const float km = k_scale ? 1.0f / k_scale[h] : 1.0f;  // per-head FP8 scale: stored = x / scale
      const uint32_t k1 = f32_to_fp8(y1 * km), k2 = f32_to_fp8(y2 * km);
      s_knew[jx] = fp8_to_f32(k1);
      s_knew[jx + kHalf] = fp8_to_f32(k2);
      if (split == 0 && app_slot >= 0) {
        ck[(int64_t)app_slot * c_s + jx] = (uint8_t)k1;
        ck[(int64_t)app_slot * c_s + jx + kHalf] = (uint8_t)k2;
      }
    } else if (tid < 5 * kHalf + D) {
      const int d = tid - 5 * kHalf;
      const uint32_t v8 = f32_to_fp8(fx1 * (v_scale ? 1.0f / v_scale[h] : 1.0f));
      s_vnew[d] = fp8_to_f32(v8);
      if (split == 0 && app_slot >= 0) cv[(int64_t)app_slot * c_s + d] = (uint8_t)v8;
    }
  } else if (rope_pos) {
    // rotate q here (decision lane zeroed), rounded to bf16 like a stored q
    constexpr int half = D / 2;
    const int64_t pos = rope_pos[b];
    for (int i = tid; i < 4 * half; i += NT) {
      const int g = i / half, jx = i - g * half;
      uint32_t y1b = 0u, y2b = 0u;
      if (g < G) {
        const bf16_t* qh = q + b * qs_b + (int64_t)(h * G + g) * qs_h;
        const float x1 = ld<bf16_t>(qh + jx);
        const float x2 = (g == 0 && jx == half - 1) ? 0.0f : ld<bf16_t>(qh + jx + half);
        float y1, y2;
        rope_f32(x1, x2, rope_cs[pos * rcs_p + (int64_t)jx * rcs_d], rope_cs[pos * rcs_p + (int64_t)(jx + half) * rcs_d],
                 &y1, &y2);
        y1b = f32_to_bf16(y1);
        y2b = f32_to_bf16(y2);
      }
      s_q[g][jx] = (uint16_t)y1b;
      s_q[g][jx + half] = (uint16_t)y2b;
    }
  } else {
#pragma unroll
    for (int x = 0; x < QPT; ++x) {
      const int i = tid + x * NT;
      if (i < 4 * D) s_q[i / D][i % D] = (uint16_t)qraw[x];
    }
  }
  __syncthreads();

  // FP8 dequant in registers: the per-head K scale folds into the score scale,
  // the V scale multiplies the output
  const float qscale = scale * kLog2e * (k_scale ? k_scale[h] : 1.0f);
  const float oscale = v_scale ? v_scale[h] : 1.0f;
  if constexpr (FUSED) {
    // the appended token as one more partial (m = its score, l = 1, acc = v),
    // by the last wave, which has the fewest groups
    if (wave == NW - 1) {
      float sg[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float part = 0.0f;
#pragma unroll
        for (int d = lane; d < D; d += kWave) part += bf16_to_f32(s_q[g][d]) * s_knew[d];
        sg[g] = wave_sum(part);
      }
      if (lane < 4) {
        const float sl = lane == 0 ? sg[0] : lane == 1 ? sg[1] : lane == 2 ? sg[2] : sg[3];
        s_wm[NW][lane] = new_tok ? sl * qscale : -INFINITY;
        s_wl[NW][lane] = 1.0f;
      }
#pragma unroll
      for (int d = lane; d < D; d += kWave)
#pragma unroll
        for (int g = 0; g < 4; ++g) s_wacc[NW][g][d] = s_vnew[d];
    }
  }
  float m_j = -INFINITY;  // running max of head jj (same in every lane of that head)
  float l_j = 0.0f;       // this lane's share of the denominator of head jj
  v4f32_t acc[NA][2];  // even / odd P.V steps (two independent chains)
#pragma unroll
  for (int a = 0; a < NA; ++a) acc[a][0] = acc[a][1] = v4f32_t{0.f, 0.f, 0.f, 0.f};
  uint32_t* vt = s_vt[wave];

  // One group: QK^T, V -> transposed LDS tile, online softmax, P.V; the
  // wave's next group (gidx + NW) goes in flight in grp's registers as soon
  // as they are consumed.
  auto process = [&](MfmaGroup<D>& grp, int gidx) {
    // S^T for the group: register r of lane (s, j) = S[token s + 16r][head j]
    v4f32_t sq[2];  // two independent chains
    sq[0] = sq[1] = v4f32_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < KW; ++n) {
      const v4i16_t qn = *reinterpret_cast<const v4i16_t*>(&s_q[jj][4 * n]);
      sq[n & 1] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(fp8x4_to_bf16x4(grp.k[n]), qn, sq[n & 1], 0, 0, 0);
    }
    // V slices -> transposed tile: VT[dim][s] = bytes of tokens s, s+16, s+32, s+48
#pragma unroll
    for (int w = 0; w < VW; ++w) {
      const uint32_t x01l = __builtin_amdgcn_perm(grp.v[1][w], grp.v[0][w], 0x05010400u);
      const uint32_t x01h = __builtin_amdgcn_perm(grp.v[1][w], grp.v[0][w], 0x07030602u);
      const uint32_t x23l = __builtin_amdgcn_perm(grp.v[3][w], grp.v[2][w], 0x05010400u);
      const uint32_t x23h = __builtin_amdgcn_perm(grp.v[3][w], grp.v[2][w], 0x07030602u);
      const int d0 = jj * (D / 4) + 4 * w;  // dim of byte 0 of word w of this lane's slice
      vt[(d0 + 0) * kVtStride + ss] = __builtin_amdgcn_perm(x23l, x01l, 0x05040100u);
      vt[(d0 + 1) * kVtStride + ss] = __builtin_amdgcn_perm(x23l, x01l, 0x07060302u);
      vt[(d0 + 2) * kVtStride + ss] = __builtin_amdgcn_perm(x23h, x01h, 0x05040100u);
      vt[(d0 + 3) * kVtStride + ss] = __builtin_amdgcn_perm(x23h, x01h, 0x07060302u);
    }
    // the registers are free again: the wave's next group goes in flight now
    // and lands while the softmax and P.V below run
    if (gidx + NW < ngroups) {
      if constexpr (PLANNED) {  // at most two groups per wave: the second's page ids came with the item
        MfmaGroupAddr<D> ga;
        mfma_group_addr_paged<D>(ga, ck, cv, c_s, plan_qrow2, kPlanPageShift, t0 + (gidx + NW) * 64, t1, lane);
        mfma_issue_group<D>(grp, ga);
      } else {
        mfma_load_group<D, PAGED>(grp, kspan, vspan, c_s, addr, b, h, t0 + (gidx + NW) * 64, t1, lane);
      }
    }
    // scores, online softmax per head
    const int tb = t0 + gidx * 64 + ss;
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sc[r] = (tb + 16 * r < t1) ? (sq[0][r] + sq[1][r]) * qscale : -INFINITY;
    const float gmax = blocks_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float m_new = fmaxf(m_j, gmax);
    const float alpha_j = (m_j == m_new) ? 1.0f : __builtin_amdgcn_exp2f(m_j - m_new);
    m_j = m_new;
    const float al[4] = {quad_bcast<0>(alpha_j), quad_bcast<1>(alpha_j), quad_bcast<2>(alpha_j),
                         quad_bcast<3>(alpha_j)};
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[a][0][i] *= al[i];
        acc[a][1][i] *= al[i];
      }
    v4f16_t pa;
    float lsum = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = __builtin_amdgcn_exp2f(sc[r] - m_new);  // -inf -> 0
      pa[r] = (_Float16)p;
      lsum += p;
    }
    l_j = l_j * alpha_j + lsum;
    __builtin_amdgcn_wave_barrier();  // VT writes of the wave before its reads (LDS is in order per wave)
    // P.V: step s broadcasts block s's probabilities
#define FDMS_PV_STEP(S)                                                                                            \
    {                                                                                                              \
      _Pragma("unroll") for (int a = 0; a < NA; ++a) {                                                             \
        const uint32_t vw = vt[(64 * a + lane) * kVtStride + (S)];                                                 \
        acc[a][(S) & 1] = __builtin_amdgcn_mfma_f32_4x4x4f16(pa, fp8x4_to_f16x4(vw), acc[a][(S) & 1], 4, (S), 0);  \
      }                                                                                                            \
    }
    FDMS_PV_STEP(0) FDMS_PV_STEP(1) FDMS_PV_STEP(2) FDMS_PV_STEP(3) FDMS_PV_STEP(4) FDMS_PV_STEP(5)
    FDMS_PV_STEP(6) FDMS_PV_STEP(7) FDMS_PV_STEP(8) FDMS_PV_STEP(9) FDMS_PV_STEP(10) FDMS_PV_STEP(11)
    FDMS_PV_STEP(12) FDMS_PV_STEP(13) FDMS_PV_STEP(14) FDMS_PV_STEP(15)
#undef FDMS_PV_STEP
    __builtin_amdgcn_wave_barrier();  // reads done before the next group's writes
  };
  for (int gi = wave; gi < ngroups; gi += NW) process(cur, gi);  // wave-uniform

  // per wave: max, denominator, accumulators -> LDS; combine the waves
  const float lw = blocks_sum(l_j);
  if (lane < 4) {
    s_wm[wave][lane] = m_j;
    s_wl[wave][lane] = lw;
  }
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_wacc[wave][i][64 * a + lane] = acc[a][0][i] + acc[a][1][i];
  __syncthreads();
  const int n_out = G * D;
  const int64_t stride = (int64_t)G * (D + 2);
  float* mine = ws + ((int64_t)pair * num_splits + split) * stride;
  for (int o = tid; o < n_out; o += NT) {
    const int og = o / D, od = o - og * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWX; ++w) M = fmaxf(M, s_wm[w][og]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < NWX; ++w) {
      const float mw = s_wm[w][og];
      const float f = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      L += s_wl[w][og] * f;
      A += s_wacc[w][og][od] * f;
    }
    if (ns == 1) {
      out[b * os_b + (int64_t)(h * G + og) * os_h + od].bits = (uint16_t)f32_to_bf16(A / L * oscale);
    } else {
      store_agent(mine + 2 * G + o, A);
      if (od == 0) {
        store_agent(mine + og, M);
        store_agent(mine + G + og, L);
      }
    }
  }
  if (ns == 1) return;
  if (!take_last_ticket(&counters[pair], ns, &s_last)) return;
  const float* all = ws + (int64_t)pair * num_splits * stride;
  for (int o = tid; o < n_out; o += NT) {
    const int og = o / D, od = o - og * D;
    float M = -INFINITY, L = 0.0f, Acc = 0.0f;
    for (int s0 = 0; s0 < ns; s0 += kMergeBatch) {
      float mv[kMergeBatch], lv[kMergeBatch], av[kMergeBatch];
#pragma unroll
      for (int x = 0; x < kMergeBatch; ++x) {
        mv[x] = -INFINITY;
        lv[x] = av[x] = 0.0f;
        if (s0 + x < ns) {
          const float* ps = all + (s0 + x) * stride;
          mv[x] = load_agent(ps + og);
          lv[x] = load_agent(ps + G + og);
          av[x] = load_agent(ps + 2 * G + o);
        }
      }
      float bm = M;
#pragma unroll
      for (int x = 0; x < kMergeBatch; ++x) bm = fmaxf(bm, mv[x]);
      const float f = (M == -INFINITY || bm == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(M - bm);
      L *= f;
      Acc *= f;
#pragma unroll
      for (int x = 0; x < kMergeBatch; ++x) {
        const float wgt = (mv[x] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mv[x] - bm);
        L += lv[x] * wgt;
        Acc += av[x] * wgt;
      }
      M = bm;
    }
    out[b * os_b + (int64_t)(h * G + og) * os_h + od].bits = (uint16_t)f32_to_bf16(Acc / L * oscale);
  }
  if (tid == 0) __hip_atomic_store(&counters[pair], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

namespace {

template <int D, typename KT>
bool launch_tiled_d(int G, dim3 grid, hipStream_t stream, const bf16_t* q, int64_t qs_b, int64_t qs_h, const KT* ck,
                    const KT* cv, int64_t c_s, const int32_t* bo, int64_t bo_b, int64_t bo_h, const int32_t* bt,
                    int64_t bt_b, int64_t bt_h, int page_shift, int paged, const int32_t* lc, int64_t lc_b,
                    int64_t lc_h, bf16_t* out, int64_t os_b, int64_t os_h, float* ws, int* counters, int hkv,
                    int pairs, int splits, float scale, const float* rcs, int64_t rcs_p, int64_t rcs_d,
                    const int64_t* rpos) {
#define FDMS_TILED(GG)                                                                                          \
  hipLaunchKernelGGL((decode_attn_tiled_kernel<D, GG, KT>), grid, dim3(kThreads), 0, stream, q, qs_b, qs_h, ck, cv, \
                     c_s, bo, bo_b, bo_h, bt, bt_b, bt_h, page_shift, paged, lc, lc_b, lc_h, out, os_b, os_h, ws,      \
                     counters, hkv, pairs, splits, scale, rcs, rcs_p, rcs_d, rpos)
#define FDMS_WAVE(GG)                                                                                          \
  hipLaunchKernelGGL((decode_attn_wave_kernel<D, GG, KT, 2>), grid, dim3(kThreads), 0, stream, q, qs_b, qs_h, ck, cv, \
                     c_s, bo, bo_b, bo_h, bt, bt_b, bt_h, page_shift, paged, lc, lc_b, lc_h, out, os_b, os_h, ws,      \
                     counters, hkv, pairs, splits, scale, rcs, rcs_p, rcs_d, rpos)
  const char* e = std::getenv("FASTDMS_AMD_ATTN_TILED");
  const bool tiled = e && e[0] == '1';
  switch (G) {
    case 1: if (tiled) FDMS_TILED(1); else FDMS_WAVE(1); return true;
    case 2: if (tiled) FDMS_TILED(2); else FDMS_WAVE(2); return true;
    case 4: if (tiled) FDMS_TILED(4); else FDMS_WAVE(4); return true;
    case 8: FDMS_TILED(8); return true;
    default: return false;
  }
#undef FDMS_TILED
#undef FDMS_WAVE
}

}  // namespace

FDMS_EXPORT int fdms_compact_decode_attention(
    const void* q, int q_dtype, int64_t qs_b, int64_t qs_h, const void* compact_k, const void* compact_v,
    int kv_dtype, int64_t c_s, const int32_t* base_offsets, int64_t bo_b, int64_t bo_h, const int32_t* block_tables,
    int64_t bt_b, int64_t bt_h, int page_size, const int32_t* live_counts, int64_t lc_b, int64_t lc_h, void* out,
    int64_t os_b, int64_t os_h, float* workspace, int* counters, int batch, int num_kv_heads, int group_size,
    int head_dim, int num_splits, int split_rows, float scale, const float* rope_cos_sin, int64_t rcs_p,
    int64_t rcs_d, const int64_t* rope_positions, const float* k_scale, const float* v_scale, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || group_size <= 0 || group_size > kMaxG) return (int)hipErrorInvalidValue;
  if (head_dim <= 0 || head_dim > kMaxD || num_splits <= 0 || num_splits > 65535 || split_rows < 0)
    return (int)hipErrorInvalidValue;
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
  // tiled fast path: bf16 q, FP8 / bf16 K/V, D = 64 / 128, 16-byte aligned rows
  const int kv_size = kv_dtype == kFP8 ? 1 : (kv_dtype == kBF16 ? 2 : 0);
  const bool tiled_ok = q_dtype == kBF16 && kv_size > 0 && (head_dim == 64 || head_dim == 128) &&
                        (c_s * kv_size) % 16 == 0 && ((uintptr_t)compact_k % 16) == 0 &&
                        ((uintptr_t)compact_v % 16) == 0 && (group_size == 1 || group_size == 2 ||
                        group_size == 4 || group_size == 8) && !fdms_force_generic_attention();
  // matrix-core path: pages (if any) of at least 16 rows, so a 64-row group's
  // quarters each lie in one page
  const bool mfma_ok = tiled_ok && kv_dtype == kFP8 && group_size <= 4 && fdms_mfma_attention_enabled() &&
                       (!paged || page_shift >= 4);
  if (mfma_ok) {
    // split_rows: rows per split (rounded up to 64; 0 = one 64-row group per wave)
    const int nw = 4;
    const int rows = split_rows > 0 ? ((split_rows + 63) & ~63) : nw * 64;
    const int64_t blocks = (int64_t)((pairs + kXcds - 1) / kXcds) * kXcds * num_splits;
    if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    if (!fits_i32(lc_b) || !fits_i32(lc_h) || !fits_i32(bt_b) || !fits_i32(bt_h)) return (int)hipErrorInvalidValue;
#define FDMS_MFMA_ARGS                                                                                          \
  nullptr, live_counts, (int)lc_b, (int)lc_h, nullptr, 0, 0, nullptr, pairs, num_kv_heads,                         \
      (const bf16_t*)q, qs_b, qs_h,                                                                                   \
      (uint8_t*)compact_k, (uint8_t*)compact_v, c_s, base_offsets, bo_b, bo_h, block_tables, (int)bt_b, (int)bt_h,   \
      page_shift, paged, (bf16_t*)out, os_b, os_h, workspace, counters, group_size, num_splits, rows,              \
      fdms_attn_heavy_rows(rows, head_dim, pairs), scale,                                                                            \
      rope_cos_sin, rcs_p, rcs_d, rope_positions, DecodePre{}, k_scale, v_scale
#define FDMS_MFMA_LAUNCH(DD, PG)                                                                            \
  hipLaunchKernelGGL((decode_attn_mfma_kernel<DD, 4, PG, false>), dim3((unsigned)blocks), dim3(4 * kWave), 0, \
                     (hipStream_t)stream, FDMS_MFMA_ARGS)
    if (head_dim == 64) {
      if (paged) FDMS_MFMA_LAUNCH(64, true); else FDMS_MFMA_LAUNCH(64, false);
    } else {
      if (paged) FDMS_MFMA_LAUNCH(128, true); else FDMS_MFMA_LAUNCH(128, false);
    }
#undef FDMS_MFMA_LAUNCH
#undef FDMS_MFMA_ARGS
    FDMS_LAUNCH_CHECK();
    return 0;
  }
  // per-head FP8 scales: matrix-core kernel only
  if (k_scale || v_scale) return (int)hipErrorInvalidValue;
  if (tiled_ok) {
    const int64_t blocks = (int64_t)((pairs + kXcds - 1) / kXcds) * kXcds * num_splits;
    if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
    const dim3 tgrid((unsigned)blocks);
    bool done = false;
#define FDMS_TILED_ARGS(KT)                                                                                         group_size, tgrid, (hipStream_t)stream, (const bf16_t*)q, qs_b, qs_h, (const KT*)compact_k, (const KT*)compact_v,       c_s, base_offsets, bo_b, bo_h, block_tables, bt_b, bt_h, page_shift, paged, live_counts, lc_b, lc_h,                (bf16_t*)out, os_b, os_h, workspace, counters, num_kv_heads, pairs, num_splits, scale, rope_cos_sin, rcs_p,         rcs_d, rope_positions
    if (kv_dtype == kFP8) {
      done = head_dim == 64 ? launch_tiled_d<64, fp8_t>(FDMS_TILED_ARGS(fp8_t))
                            : launch_tiled_d<128, fp8_t>(FDMS_TILED_ARGS(fp8_t));
    } else {
      done = head_dim == 64 ? launch_tiled_d<64, bf16_t>(FDMS_TILED_ARGS(bf16_t))
                            : launch_tiled_d<128, bf16_t>(FDMS_TILED_ARGS(bf16_t));
    }
#undef FDMS_TILED_ARGS
    if (done) {
      FDMS_LAUNCH_CHECK();
      return 0;
    }
  }
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

// Decode preprocess + attention in one launch: the reference's
// fused_dms_rope_store_compact_decode(store_q=False, store_transient_k=False)
// followed by compact_decode_attention with in-kernel q RoPE
// (compact_attention.py:67-209, 418-534, 1010-1336; llama.py:112-134).  q, k,
// v are the step's raw rows; q and k are not written back.  The appended token
// is rank live-1 of span (b, h) (prepare_decode_metadata: slot = base + live,
// then live += 1).  Matrix-core path only: bf16 q/k/v, FP8 flat spans,
// group_size <= 4, head_dim 64 / 128, 16-byte aligned rows.
static int fused_decode_attention(
    const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b, int64_t ks_h, const void* v,
    int64_t vs_b, int64_t vs_h, const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
    const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, uint8_t* evict_out, int64_t ev_b, int64_t ev_h,
    float alpha_scale, float alpha_offset, float threshold, int positive_scale, void* compact_k, void* compact_v,
    int64_t c_s, const int32_t* base_offsets, int64_t bo_b, int64_t bo_h, const int32_t* live_counts, int64_t lc_b,
    int64_t lc_h, void* out, int64_t os_b, int64_t os_h, float* workspace, int* counters, int batch,
    int num_kv_heads, int group_size, int head_dim, int num_splits, int split_rows, float scale, const float* k_scale,
    const float* v_scale, const void* q_norm, const void* k_norm, float norm_eps, void* stream,
    const int32_t* block_tables = nullptr, int64_t bt_b = 0, int64_t bt_h = 0, int page_size = 0) {
  if (batch < 0 || num_kv_heads <= 0 || group_size <= 0 || group_size > 4) return (int)hipErrorInvalidValue;
  if ((head_dim != 64 && head_dim != 128) || num_splits <= 0 || num_splits > 65535 || split_rows < 0)
    return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  if (!q || !k || !v || !cos_sin || !positions || !slot_mapping || !evict_out || !compact_k || !compact_v ||
      !live_counts || !out)
    return (int)hipErrorInvalidValue;
  int page_shift = 0;
  if (block_tables) {  // pages of at least 16 rows (see mfma_load_group)
    if (page_size < 16 || (page_size & (page_size - 1))) return (int)hipErrorInvalidValue;
    while ((1 << page_shift) < page_size) ++page_shift;
  } else if (!base_offsets) {
    return (int)hipErrorInvalidValue;
  }
  const int paged = block_tables ? 1 : 0;
  if (c_s % 16 || ((uintptr_t)compact_k % 16) || ((uintptr_t)compact_v % 16)) return (int)hipErrorInvalidValue;
  if (num_splits > 1 && (!workspace || !counters)) return (int)hipErrorInvalidValue;
  const int pairs = batch * num_kv_heads;
  if (pairs > 65535) return (int)hipErrorInvalidValue;
  if ((q_norm && ((uintptr_t)q_norm & 1)) || (k_norm && ((uintptr_t)k_norm & 1)) || !(norm_eps >= 0.0f))
    return (int)hipErrorInvalidValue;
  const DecodePre pre{(const bf16_t*)k, ks_b, ks_h, (const bf16_t*)v, vs_b, vs_h, cos_sin, cs_p, cs_d, positions,
                      slot_mapping, sm_b, sm_h, evict_out, ev_b, ev_h, alpha_scale, alpha_offset, threshold,
                      positive_scale, (const bf16_t*)q_norm, (const bf16_t*)k_norm, norm_eps};
  // 4 waves (or 8), 8 for head_dim 128 (the preprocess needs 2.5 * head_dim
  // threads); split_rows as for fdms_compact_decode_attention
  const int nw = fdms_attn_fused_waves(head_dim, pairs);
  const int rows = split_rows > 0 ? ((split_rows + 63) & ~63) : nw * 64;
  const int heavy = fdms_attn_heavy_rows(rows, head_dim, pairs);
  const int64_t blocks = (int64_t)((pairs + kXcds - 1) / kXcds) * kXcds * num_splits;
  if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  if (!fits_i32(lc_b) || !fits_i32(lc_h) || !fits_i32(bt_b) || !fits_i32(bt_h) || !fits_i32(sm_b) ||
      !fits_i32(sm_h))
    return (int)hipErrorInvalidValue;
#define FDMS_FUSED_LAUNCH(DD, NWV, PG)                                                                               \
  hipLaunchKernelGGL((decode_attn_mfma_kernel<DD, NWV, PG, true>), dim3((unsigned)blocks), dim3(NWV * kWave), 0,     \
                     (hipStream_t)stream, nullptr, live_counts, (int)lc_b, (int)lc_h, slot_mapping,                   \
                     (int)sm_b, (int)sm_h,                                                                            \
                     positions, pairs, num_kv_heads, (const bf16_t*)q, qs_b, qs_h, (uint8_t*)compact_k,               \
                     (uint8_t*)compact_v, c_s, base_offsets, bo_b, bo_h, block_tables, (int)bt_b, (int)bt_h,          \
                     page_shift, paged, (bf16_t*)out, os_b, os_h,                                                     \
                     workspace, counters, group_size, num_splits, rows, heavy, scale, nullptr, 0, 0, nullptr, pre,     \
                     k_scale,                                                                                          \
                     v_scale)
  if (head_dim == 64 && nw == 4) {
    if (paged) FDMS_FUSED_LAUNCH(64, 4, true); else FDMS_FUSED_LAUNCH(64, 4, false);
  } else if (head_dim == 64) {
    if (paged) FDMS_FUSED_LAUNCH(64, 8, true); else FDMS_FUSED_LAUNCH(64, 8, false);
  } else {
    if (paged) FDMS_FUSED_LAUNCH(128, 8, true); else FDMS_FUSED_LAUNCH(128, 8, false);
  }
#undef FDMS_FUSED_LAUNCH
  FDMS_LAUNCH_CHECK();
  return 0;
}

FDMS_EXPORT int fdms_fused_decode_attention(
    const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b, int64_t ks_h, const void* v,
    int64_t vs_b, int64_t vs_h, const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
    const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, uint8_t* evict_out, int64_t ev_b, int64_t ev_h,
    float alpha_scale, float alpha_offset, float threshold, int positive_scale, void* compact_k, void* compact_v,
    int64_t c_s, const int32_t* base_offsets, int64_t bo_b, int64_t bo_h, const int32_t* live_counts, int64_t lc_b,
    int64_t lc_h, void* out, int64_t os_b, int64_t os_h, float* workspace, int* counters, int batch,
    int num_kv_heads, int group_size, int head_dim, int num_splits, int split_rows, float scale, const float* k_scale,
    const float* v_scale, const void* q_norm, const void* k_norm, float norm_eps, void* stream) {
  return fused_decode_attention(q, qs_b, qs_h, k, ks_b, ks_h, v, vs_b, vs_h, cos_sin, cs_p, cs_d, positions,
                                slot_mapping, sm_b, sm_h, evict_out, ev_b, ev_h, alpha_scale, alpha_offset, threshold,
                                positive_scale, compact_k, compact_v, c_s, base_offsets, bo_b, bo_h, live_counts, lc_b,
                                lc_h, out, os_b, os_h, workspace, counters, batch, num_kv_heads, group_size, head_dim,
                                num_splits, split_rows, scale, k_scale, v_scale, q_norm, k_norm, norm_eps, stream);
}

// Paged-layout fused decode attention (no reference counterpart: the reference
// reads flat spans): fdms_fused_decode_attention with rank r of (b, h) at row
// block_tables[b, h, r / page_size] * page_size + r % page_size instead of
// base_offsets[b, h] + r; slot_mapping holds the appended token's row (from
// fdms_paged_prepare_decode).
FDMS_EXPORT int fdms_fused_decode_attention_paged(
    const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b, int64_t ks_h, const void* v,
    int64_t vs_b, int64_t vs_h, const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
    const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, uint8_t* evict_out, int64_t ev_b, int64_t ev_h,
    float alpha_scale, float alpha_offset, float threshold, int positive_scale, void* compact_k, void* compact_v,
    int64_t c_s, const int32_t* block_tables, int64_t bt_b, int64_t bt_h, int page_size, const int32_t* live_counts,
    int64_t lc_b, int64_t lc_h, void* out, int64_t os_b, int64_t os_h, float* workspace, int* counters, int batch,
    int num_kv_heads, int group_size, int head_dim, int num_splits, int split_rows, float scale, const float* k_scale,
    const float* v_scale, const void* q_norm, const void* k_norm, float norm_eps, void* stream) {
  if (!block_tables) return (int)hipErrorInvalidValue;
  return fused_decode_attention(q, qs_b, qs_h, k, ks_b, ks_h, v, vs_b, vs_h, cos_sin, cs_p, cs_d, positions,
                                slot_mapping, sm_b, sm_h, evict_out, ev_b, ev_h, alpha_scale, alpha_offset, threshold,
                                positive_scale, compact_k, compact_v, c_s, nullptr, 0, 0, live_counts, lc_b, lc_h,
                                out, os_b, os_h, workspace, counters, batch, num_kv_heads, group_size, head_dim,
                                num_splits, split_rows, scale, k_scale, v_scale, q_norm, k_norm, norm_eps, stream,
                                block_tables, bt_b, bt_h, page_size);
}

// Planned form of fdms_fused_decode_attention_paged (no reference
// counterpart): the layer's work plan from fdms_paged_prepare_decode_plan
// (`plan` = that layer's items, its count of further splits in the int
// before them) replaces the live counts, append rows and block tables.  The
// grid holds num_splits x pairs workgroups: workgroup i runs item i, those
// past the layer's items exit after one load.  With the partition the
// unplanned launch uses (the same split_rows, heavy_rows and num_splits given
// to the plan) the decisions, appended rows and outputs are the unplanned
// launch's, bit for bit.
FDMS_EXPORT int fdms_fused_decode_attention_planned(
    const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b, int64_t ks_h, const void* v,
    int64_t vs_b, int64_t vs_h, const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
    const int32_t* plan, uint8_t* evict_out, int64_t ev_b, int64_t ev_h, float alpha_scale, float alpha_offset,
    float threshold, int positive_scale, void* compact_k, void* compact_v, int64_t c_s, void* out, int64_t os_b,
    int64_t os_h, float* workspace, int* counters, int batch, int num_kv_heads, int group_size, int head_dim,
    int num_splits, float scale, const float* k_scale, const float* v_scale, const void* q_norm, const void* k_norm,
    float norm_eps, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || group_size <= 0 || group_size > 4) return (int)hipErrorInvalidValue;
  if ((head_dim != 64 && head_dim != 128) || num_splits <= 0 || num_splits > 65535) return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  if (!q || !k || !v || !cos_sin || !positions || !plan || !evict_out || !compact_k || !compact_v || !out)
    return (int)hipErrorInvalidValue;
  if ((uintptr_t)plan % 16 || c_s % 16 || ((uintptr_t)compact_k % 16) || ((uintptr_t)compact_v % 16))
    return (int)hipErrorInvalidValue;
  if (num_splits > 1 && (!workspace || !counters)) return (int)hipErrorInvalidValue;
  const int pairs = batch * num_kv_heads;
  if (pairs > 65535) return (int)hipErrorInvalidValue;
  if ((q_norm && ((uintptr_t)q_norm & 1)) || (k_norm && ((uintptr_t)k_norm & 1)) || !(norm_eps >= 0.0f))
    return (int)hipErrorInvalidValue;
  const int64_t blocks = (int64_t)pairs * num_splits;
  if (blocks > 0x7FFFFFFF) return (int)hipErrorInvalidValue;
  const DecodePre pre{(const bf16_t*)k, ks_b, ks_h, (const bf16_t*)v, vs_b, vs_h, cos_sin, cs_p, cs_d, positions,
                      nullptr, 0, 0, evict_out, ev_b, ev_h, alpha_scale, alpha_offset, threshold,
                      positive_scale, (const bf16_t*)q_norm, (const bf16_t*)k_norm, norm_eps};
#define FDMS_PLANNED_LAUNCH(DD)                                                                                    \
  hipLaunchKernelGGL((decode_attn_mfma_kernel<DD, kPlanWaves, true, true, true>), dim3((unsigned)blocks),       \
                     dim3(kPlanWaves * kWave), 0, (hipStream_t)stream, plan, nullptr, 0, 0, nullptr, 0, 0,         \
                     positions, pairs, num_kv_heads, (const bf16_t*)q, qs_b, qs_h, (uint8_t*)compact_k,       \
                     (uint8_t*)compact_v, c_s, nullptr, 0, 0, nullptr, 0, 0, kPlanPageShift, 1, (bf16_t*)out,      \
                     os_b, os_h, workspace, counters, group_size, num_splits, kPlanRows, kPlanRows, scale,         \
                     nullptr, 0, 0, nullptr, pre, k_scale, v_scale)
  if (head_dim == 64) FDMS_PLANNED_LAUNCH(64); else FDMS_PLANNED_LAUNCH(128);
#undef FDMS_PLANNED_LAUNCH
  FDMS_LAUNCH_CHECK();
  return 0;
}

// ---------------------------------------------------------------------------
// Allocation-free variant of fdms_fused_decode_attention: the split partials
// and tickets live in the library's own device array `scratch` (one copy per
// GPU, held until the process ends), so a caller that cannot allocate (HIP
// graph capture, a serving loop that forbids hipMalloc) passes only inputs and
// outputs.  Host code must never pass the array's name to a kernel (in host
// code it is a stand-in, not a device address): the address comes from
// hipGetSymbolAddress, once per device with that device current, and is kept
// per device.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kScratchFloats = int64_t(2) << 20;  // 8 MiB of split partials
constexpr int kScratchCounters = 16384;                // tickets (ints) after the partials
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) float scratch[kScratchFloats + kScratchCounters];

__global__ void zero_ints_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device (looked up and its tickets
// zeroed on the first call there); nullptr with *err set on failure.
static float* scratch_on_current_device(hipStream_t stream, int* err) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = (int)e;
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *err = (int)hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = (int)(e != hipSuccess ? e : hipErrorInvalidSymbol);
      return nullptr;
    }
    // the tickets must start at zero (every call leaves them zero); a fill
    // kernel, not hipMemsetAsync, so a first call under graph capture is fine
    hipLaunchKernelGGL(zero_ints_kernel, dim3(16), dim3(256), 0, stream,
                       reinterpret_cast<int*>(static_cast<float*>(p) + kScratchFloats), kScratchCounters);
    e = hipGetLastError();
    if (e != hipSuccess) {
      *err = (int)e;
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}

FDMS_EXPORT int fdms_fused_decode_attention_noalloc(
    const void* q, int64_t qs_b, int64_t qs_h, const void* k, int64_t ks_b, int64_t ks_h, const void* v,
    int64_t vs_b, int64_t vs_h, const float* cos_sin, int64_t cs_p, int64_t cs_d, const int64_t* positions,
    const int32_t* slot_mapping, int64_t sm_b, int64_t sm_h, uint8_t* evict_out, int64_t ev_b, int64_t ev_h,
    float alpha_scale, float alpha_offset, float threshold, int positive_scale, void* compact_k, void* compact_v,
    int64_t c_s, const int32_t* base_offsets, int64_t bo_b, int64_t bo_h, const int32_t* live_counts, int64_t lc_b,
    int64_t lc_h, void* out, int64_t os_b, int64_t os_h, int batch, int num_kv_heads, int group_size, int head_dim,
    int num_splits, int split_rows, float scale, const float* k_scale, const float* v_scale, const void* q_norm, const void* k_norm, float norm_eps, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || group_size <= 0 || group_size > 4 || num_splits <= 0)
    return (int)hipErrorInvalidValue;
  // the scratch limit: pairs * num_splits * group_size * (head_dim + 2)
  // partial floats and one ticket per pair
  const int64_t pairs = (int64_t)batch * num_kv_heads;
  if (pairs * num_splits * group_size * (int64_t)(head_dim + 2) > kScratchFloats || pairs > kScratchCounters)
    return (int)hipErrorInvalidValue;
  if (batch == 0) return 0;
  int err = 0;
  float* ws = scratch_on_current_device((hipStream_t)stream, &err);
  if (!ws) return err;
  return fused_decode_attention(q, qs_b, qs_h, k, ks_b, ks_h, v, vs_b, vs_h, cos_sin, cs_p, cs_d, positions,
                                slot_mapping, sm_b, sm_h, evict_out, ev_b, ev_h, alpha_scale, alpha_offset, threshold,
                                positive_scale, compact_k, compact_v, c_s, base_offsets, bo_b, bo_h, live_counts, lc_b,
                                lc_h, out, os_b, os_h, ws, reinterpret_cast<int*>(ws + kScratchFloats), batch,
                                num_kv_heads, group_size, head_dim, num_splits, split_rows, scale, k_scale, v_scale,
                                q_norm, k_norm, norm_eps, stream);
}
