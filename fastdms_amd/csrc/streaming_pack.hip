// Streaming prefill pack into compact K/V spans (reference:
// fastdms/engine/compact_kv.py:38-296 and streaming_pack_layer 915-1099).
//
// keep[t,h] = ~evict[t,h] | t >= max(0, len-1-W); rank = exclusive prefix of
// keep down the token axis; kept rows land at compact[base[b,h] + rank].
//
// MI355X layout of the work: one launch covers every sequence of a ragged
// prefill batch (cu_seqlens), grid = (chunk, seq*head).  A 256-token chunk is
// ranked with wave ballots (64-bit masks + popcount) and an LDS prefix over
// the 4 waves; kept rows are listed in LDS and copied cooperatively, VEC
// elements per lane, so each row moves as whole 16-byte vectors.  HBM-bound:
// only kept rows are read (2*D*in_bytes per kept token per head) and written
// (2*D*out_bytes), plus one evict byte per token per head.
#include "fdms_pool.h"
#include "fdms_vec.h"

using namespace fdms;

namespace {

constexpr int kChunk = 256;  // compact_kv.py:276, 318 (chunk the block offsets index)

__device__ __forceinline__ int block_rank(bool keep, int* s_wave, int* total) {
  const uint64_t m = __ballot(keep);
  const int lane = __lane_id();
  const int wave = threadIdx.x >> 6;
  const int prefix = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) s_wave[wave] = __popcll(m);
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kChunk / kWave; ++w) {
    const int c = s_wave[w];
    off += (w < wave) ? c : 0;
    tot += c;
  }
  *total = tot;
  return off + prefix;
}

struct SeqSpan {
  int64_t tok0;  // first token of the sequence in k/v
  int64_t ev0;   // first token of the sequence in the evict array
  int len;
};

__device__ __forceinline__ SeqSpan seq_span(const int32_t* cu, int b, int single_start, int single_len) {
  SeqSpan s;
  if (cu) {
    s.tok0 = cu[b];
    s.ev0 = cu[b];
    s.len = cu[b + 1] - cu[b];
  } else {
    s.tok0 = single_start;
    s.ev0 = 0;
    s.len = single_len;
  }
  return s;
}

}  // namespace

// One block per (seq, head): chunk keep counts -> exclusive chunk offsets and
// live count (compact_kv.py:140-165 + the torch scan at 294-295).  Optionally
// resets the (seq, head) metadata row to (-1, False) first (compact_kv.py:1031-1032).
// The evict bytes of kPrepBatch chunks are loaded together (one memory round
// trip per batch, not per chunk); each wave counts its 64 tokens of every
// chunk with a ballot, and the running offset is accumulated uniformly.
constexpr int kPrepBatch = 32;
static_assert(kPrepBatch <= 64 && (kPrepBatch & (kPrepBatch - 1)) == 0, "one chunk per lane of a wave");

// Page pool of one layer (paged compact KV): the free page ids are
// stack[0 .. *top); a (seq, head) span owns pages bt[row * bt_b + h * bt_h + j],
// j < held[row * hd_b + h * hd_h], rank r living at row bt[r >> 4] * 16 + (r & 15).
struct PagePool {
  int32_t* stack;
  int32_t* top;
  int32_t* budget;  // pages this launch may still take (debited before the stack; at most the stack top)
  int32_t* bt;
  int64_t bt_b, bt_h;
  int32_t* held;
  int64_t hd_b, hd_h;
  int max_pages;
  int32_t* overflow;  // 1: a span's pages did not fit the budget; 2: the stack was short (broken pool)
};
constexpr int kPageShift = 4;  // 16-row pages
constexpr int kPackXcds = 8;

// (seq, head) workgroups of the count / scan kernel, padded to whole XCD rounds
inline dim3 prepare_grid(int num_seqs, int num_kv_heads) {
  return dim3((unsigned)(((num_seqs + kPackXcds - 1) / kPackXcds) * kPackXcds * num_kv_heads));
}

template <bool PAGED>
__global__ __launch_bounds__(kChunk) void pack_prepare_kernel(
    const uint8_t* __restrict__ evict, int64_t es_t, int64_t es_h, const int32_t* __restrict__ cu,
    int single_len, int window, int num_kv_heads, int max_chunks, int32_t* __restrict__ live_out, int64_t lo_b,
    int64_t lo_h, int32_t* __restrict__ offsets, int64_t of_b, int64_t of_h, int64_t of_c,
    int32_t* __restrict__ positions, uint8_t* __restrict__ evict_meta, const int32_t* __restrict__ meta_rows,
    int64_t tp_b, int64_t tp_h, int64_t em_b, int64_t em_h, int meta_cap, const PagePool pool, int num_seqs) {
  __shared__ int s_cnt[kPrepBatch][kChunk / kWave];
  __shared__ int s_p0;
  // every kv head of a sequence on one XCD (block ids are dispatched round
  // robin over the 8 XCDs): the heads read the same evict rows, which then
  // come from HBM into one L2 instead of eight
  const int xcd = blockIdx.x % kPackXcds, slot = blockIdx.x / kPackXcds;
  const int b = xcd + kPackXcds * (slot / num_kv_heads);
  const int h = slot - (slot / num_kv_heads) * num_kv_heads;
  if (b >= num_seqs) return;  // uniform per workgroup
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const SeqSpan sp = seq_span(cu, b, 0, single_len);
  const int thresh = max(0, sp.len - 1 - window);
  if (positions) {
    const int64_t row = meta_rows ? meta_rows[b] : b;
    int32_t* pr = positions + row * tp_b + h * tp_h;
    uint8_t* er = evict_meta + row * em_b + h * em_h;
    for (int s = tid; s < meta_cap; s += kChunk) {
      pr[s] = -1;
      er[s] = 0;
    }
  }
  const uint8_t* ev = evict + sp.ev0 * es_t + h * es_h;
  int running = 0;
  for (int c0 = 0; c0 < max_chunks; c0 += kPrepBatch) {
    // branch-free loads from clamped rows (a select on a predicated load would
    // wait for it on the spot); rows past the end are masked in the ballot
    uint8_t e[kPrepBatch];
    if (sp.len > 0) {
#pragma unroll
      for (int j = 0; j < kPrepBatch; ++j) {
        const int t = min((c0 + j) * kChunk + tid, sp.len - 1);
        e[j] = ev[(int64_t)t * es_t];
      }
    }
#pragma unroll
    for (int j = 0; j < kPrepBatch; ++j) {
      const int t = (c0 + j) * kChunk + tid;
      const bool keep = t < sp.len && (e[j] == 0 || t >= thresh);
      const uint64_t m = __ballot(keep);
      if (lane == 0) s_cnt[j][wave] = __popcll(m);
    }
    __syncthreads();
    // lane j < kPrepBatch of every wave: chunk c0 + j's kept count, then an
    // inclusive scan over the lanes (every wave computes the same running
    // offset; wave 0 stores the chunk offsets) -- one LDS round trip per
    // batch instead of one per chunk
    int tot = 0;
    if (lane < kPrepBatch) {
#pragma unroll
      for (int w = 0; w < kChunk / kWave; ++w) tot += s_cnt[lane][w];
    }
    int incl = tot;
#pragma unroll
    for (int o = 1; o < kPrepBatch; o <<= 1) {
      const int up = __shfl_up(incl, o);
      if (lane >= o) incl += up;
    }
    if (wave == 0 && lane < kPrepBatch && c0 + lane < max_chunks)
      offsets[b * of_b + h * of_h + (c0 + lane) * of_c] = running + incl - tot;
    running += __shfl(incl, kPrepBatch - 1);
    if (c0 + kPrepBatch < max_chunks) __syncthreads();  // s_cnt is reused by the next batch
  }
  if (tid == 0) live_out[b * lo_b + h * lo_h] = running;
  if constexpr (PAGED) {
    // ceil(live / 16) pages from the layer's free stack: one atomic pop per
    // (seq, head) (distinct ranges), then the span's block-table row
    const int64_t row = meta_rows ? meta_rows[b] : b;
    const int n = (running + (1 << kPageShift) - 1) >> kPageShift;
    if (tid == 0) {
      int p0 = -1;
      int flag = 1;
      if (n > 0 && n <= pool.max_pages && debit_budget(pool.budget, n, DeviceSub{}, DeviceAdd{})) {
        // the debit fitted, so (budget <= top) the stack holds the pages
        p0 = pop_pages(pool.top, n, DeviceSub{});
        flag = 2;  // only reached with p0 < 0: the budget exceeded the stack
      }
      if (p0 < 0 && n > 0) {
        // no pages: the span is left empty (live 0) and the launch flagged
        // (1: the budget was short; 2: the pool's precondition was broken)
        atomicMax(pool.overflow, flag);
        live_out[b * lo_b + h * lo_h] = 0;
      }
      s_p0 = p0;
    }
    __syncthreads();
    const int p0 = s_p0;
    int32_t* btr = pool.bt + row * pool.bt_b + h * pool.bt_h;
    for (int j = tid; j < pool.max_pages; j += kChunk) btr[j] = (p0 >= 0 && j < n) ? pool.stack[p0 + j] : -1;
    if (tid == 0) pool.held[row * pool.hd_b + h * pool.hd_h] = p0 >= 0 ? n : 0;
  }
}

template <typename TI, typename TO, int VEC, bool FUSED, bool PAGED>
__global__ __launch_bounds__(kChunk) void pack_scatter_kernel(
    const TI* __restrict__ k, const TI* __restrict__ v, int64_t ks_t, int64_t ks_h, int64_t vs_t, int64_t vs_h,
    const uint8_t* __restrict__ evict, int64_t es_t, int64_t es_h, const int32_t* __restrict__ cu, int single_start,
    int single_len, const int32_t* __restrict__ block_offsets, int64_t bo_b, int64_t bo_h, int64_t bo_c,
    const uint8_t* __restrict__ keep_in, int64_t kp_t, int64_t kp_h, const int32_t* __restrict__ rank_in,
    int64_t rk_t, int64_t rk_h, const int32_t* __restrict__ base, int64_t bs_b, int64_t bs_h, TO* __restrict__ ck,
    TO* __restrict__ cv, int64_t cs_s, int32_t* __restrict__ positions, uint8_t* __restrict__ evict_meta,
    const int32_t* __restrict__ meta_rows, int64_t tp_b, int64_t tp_h, int64_t tp_s, int64_t em_b, int64_t em_h,
    int64_t em_s, int window, int num_kv_heads, int head_dim, const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, const int32_t* __restrict__ bt, int64_t bt_b, int64_t bt_h) {
  __shared__ int s_wave[kChunk / kWave];
  __shared__ int64_t s_src[kChunk];
  __shared__ int64_t s_dst[kChunk];
  const int c = blockIdx.x;
  const int h = blockIdx.y % num_kv_heads;
  const int b = blockIdx.y / num_kv_heads;
  const SeqSpan sp = seq_span(cu, b, single_start, single_len);
  if (c * kChunk >= sp.len) return;  // uniform per block
  // per-block scalars first: their loads overlap the evict load
  const int64_t row = meta_rows ? meta_rows[b] : b;
  const int64_t span0 = PAGED ? 0 : base[b * bs_b + h * bs_h];
  const int32_t* btr = PAGED ? bt + row * bt_b + h * bt_h : nullptr;
  const float kmul = inv_scale(k_scale, h), vmul = inv_scale(v_scale, h);
  const int chunk0 = FUSED ? block_offsets[b * bo_b + h * bo_h + c * bo_c] : 0;
  const int t = c * kChunk + threadIdx.x;
  const bool valid = t < sp.len;
  uint8_t e = 0;
  if (valid) e = evict[(sp.ev0 + t) * es_t + h * es_h];
  bool keep;
  if (FUSED) {
    keep = valid && ((e == 0) || (t >= max(0, sp.len - 1 - window)));
  } else {
    keep = valid && keep_in[(int64_t)t * kp_t + h * kp_h] != 0;
  }
  int total = 0;
  const int local = block_rank(keep, s_wave, &total);
  int64_t rank = 0;
  if (keep) {
    rank = FUSED ? (int64_t)chunk0 + local : (int64_t)rank_in[(int64_t)t * rk_t + h * rk_h];
    s_src[local] = sp.tok0 + t;
    if constexpr (PAGED) {
      const int32_t page = btr[rank >> kPageShift];  // -1: the span got no pages (pool short)
      s_dst[local] = page < 0 ? -1 : ((int64_t)page << kPageShift) + (rank & ((1 << kPageShift) - 1));
    } else {
      s_dst[local] = span0 + rank;
    }
  }
  __syncthreads();
  // metadata stores after the barrier, so the barrier does not wait for them
  if (keep) {
    positions[row * tp_b + h * tp_h + rank * tp_s] = t;
    evict_meta[row * em_b + h * em_h + rank * em_s] = e;
  }
  // kU vectors of K and of V per thread are loaded before any is stored, so a
  // chunk of kept rows moves in one memory round trip per batch
  constexpr int kU = 8;
  const int units = head_dim / VEC;
  const int n = total * units;
  for (int u0 = threadIdx.x; u0 < n; u0 += kChunk * kU) {
    Vec<TI, VEC> kr[kU], vr[kU];
    int64_t dst[kU];
#pragma unroll
    for (int i = 0; i < kU; ++i) {
      const int u = min(u0 + i * kChunk, n - 1);  // clamped: loads stay unpredicated
      const int r = u / units;
      const int j = (u - r * units) * VEC;
      const int64_t src = s_src[r];
      dst[i] = s_dst[r] < 0 ? -1 : s_dst[r] * cs_s + j;
      kr[i] = *reinterpret_cast<const Vec<TI, VEC>*>(k + src * ks_t + h * ks_h + j);
      vr[i] = *reinterpret_cast<const Vec<TI, VEC>*>(v + src * vs_t + h * vs_h + j);
    }
#pragma unroll
    for (int i = 0; i < kU; ++i) {
      if (u0 + i * kChunk < n && dst[i] >= 0) {
        *reinterpret_cast<Vec<TO, VEC>*>(ck + dst[i]) = convert_vec_scaled<TI, TO, VEC>(kr[i], kmul);
        *reinterpret_cast<Vec<TO, VEC>*>(cv + dst[i]) = convert_vec_scaled<TI, TO, VEC>(vr[i], vmul);
      }
    }
  }
}

FDMS_EXPORT int fdms_streaming_pack_prepare(const uint8_t* evict, int64_t es_t, int64_t es_h, const int32_t* cu_seqlens,
                                            int single_len, int num_seqs, int window, int num_kv_heads,
                                            int max_chunks, int32_t* live_out, int64_t lo_b, int64_t lo_h,
                                            int32_t* block_offsets, int64_t of_b, int64_t of_h, int64_t of_c,
                                            int32_t* positions, uint8_t* evict_meta, const int32_t* meta_rows,
                                            int64_t tp_b, int64_t tp_h, int64_t em_b, int64_t em_h, int meta_cap,
                                            void* stream) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || max_chunks < 0) return (int)hipErrorInvalidValue;
  if (!evict || !live_out || (max_chunks > 0 && !block_offsets)) return (int)hipErrorInvalidValue;
  if (positions && !evict_meta) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_prepare_kernel<false>, prepare_grid(num_seqs, num_kv_heads), dim3(kChunk), 0,
                     (hipStream_t)stream, evict, es_t, es_h, cu_seqlens, single_len, window, num_kv_heads, max_chunks,
                     live_out, lo_b, lo_h, block_offsets, of_b, of_h, of_c, positions, evict_meta, meta_rows, tp_b,
                     tp_h, em_b, em_h, meta_cap, PagePool{}, num_seqs);
  FDMS_LAUNCH_CHECK();
  return 0;
}

template <bool FUSED, bool PAGED = false>
static int launch_scatter(const void* k, const void* v, int kv_dtype, int64_t ks_t, int64_t ks_h, int64_t vs_t,
                          int64_t vs_h, const uint8_t* evict, int64_t es_t, int64_t es_h, const int32_t* cu,
                          int single_start, int single_len, int num_seqs, const int32_t* bo, int64_t bo_b,
                          int64_t bo_h, int64_t bo_c, const uint8_t* keep, int64_t kp_t, int64_t kp_h,
                          const int32_t* rank, int64_t rk_t, int64_t rk_h, const int32_t* base, int64_t bs_b,
                          int64_t bs_h, void* ck, void* cv, int compact_dtype, int64_t cs_s, int32_t* positions,
                          uint8_t* evict_meta, const int32_t* meta_rows, int64_t tp_b, int64_t tp_h, int64_t tp_s,
                          int64_t em_b, int64_t em_h, int64_t em_s, int window, int num_kv_heads, int head_dim,
                          int max_chunks, int vec, const float* k_scale, const float* v_scale, void* stream,
                          const int32_t* bt = nullptr, int64_t bt_b = 0, int64_t bt_h = 0) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_chunks <= 0) return (int)hipErrorInvalidValue;
  if (vec <= 0 || head_dim % vec != 0) return (int)hipErrorInvalidValue;
  if (!k || !v || !evict || !ck || !cv || !positions || !evict_meta) return (int)hipErrorInvalidValue;
  if (PAGED ? !bt : !base) return (int)hipErrorInvalidValue;
  const dim3 grid(max_chunks, num_seqs * num_kv_heads);
  FDMS_DISPATCH_DTYPE(kv_dtype, TI,
    FDMS_DISPATCH_DTYPE(compact_dtype, TO,
      FDMS_DISPATCH_VEC(vec, V,
        hipLaunchKernelGGL((pack_scatter_kernel<TI, TO, V, FUSED, PAGED>), grid, dim3(kChunk), 0, (hipStream_t)stream,
                           (const TI*)k, (const TI*)v, ks_t, ks_h, vs_t, vs_h, evict, es_t, es_h, cu, single_start,
                           single_len, bo, bo_b, bo_h, bo_c, keep, kp_t, kp_h, rank, rk_t, rk_h, base, bs_b, bs_h,
                           (TO*)ck, (TO*)cv, cs_s, positions, evict_meta, meta_rows, tp_b, tp_h, tp_s, em_b, em_h,
                           em_s, window, num_kv_heads, head_dim, k_scale, v_scale, bt, bt_b, bt_h))));
  FDMS_LAUNCH_CHECK();
  return 0;
}

FDMS_EXPORT int fdms_streaming_pack_rank_scatter(
    const void* k, const void* v, int kv_dtype, int64_t ks_t, int64_t ks_h, int64_t vs_t, int64_t vs_h,
    const uint8_t* evict, int64_t es_t, int64_t es_h, const int32_t* cu_seqlens, int single_start, int single_len,
    int num_seqs, const int32_t* block_offsets, int64_t bo_b, int64_t bo_h, int64_t bo_c, const int32_t* base,
    int64_t bs_b, int64_t bs_h, void* compact_k, void* compact_v, int compact_dtype, int64_t cs_s,
    int32_t* positions, uint8_t* evict_meta, const int32_t* meta_rows, int64_t tp_b, int64_t tp_h, int64_t tp_s,
    int64_t em_b, int64_t em_h, int64_t em_s, int window, int num_kv_heads, int head_dim, int max_chunks, int vec,
    const float* k_scale, const float* v_scale, void* stream) {
  if (!block_offsets) return (int)hipErrorInvalidValue;
  return launch_scatter<true>(k, v, kv_dtype, ks_t, ks_h, vs_t, vs_h, evict, es_t, es_h, cu_seqlens, single_start,
                              single_len, num_seqs, block_offsets, bo_b, bo_h, bo_c, nullptr, 0, 0, nullptr, 0, 0,
                              base, bs_b, bs_h, compact_k, compact_v, compact_dtype, cs_s, positions, evict_meta,
                              meta_rows, tp_b, tp_h, tp_s, em_b, em_h, em_s, window, num_kv_heads, head_dim,
                              max_chunks, vec, k_scale, v_scale, stream);
}

FDMS_EXPORT int fdms_streaming_pack_scatter(
    const void* k, const void* v, int kv_dtype, int64_t ks_t, int64_t ks_h, int64_t vs_t, int64_t vs_h,
    const uint8_t* keep, int64_t kp_t, int64_t kp_h, const int32_t* rank, int64_t rk_t, int64_t rk_h,
    const uint8_t* seq_evict, int64_t es_t, int64_t es_h, const int32_t* base, int64_t bs_h, void* compact_k,
    void* compact_v, int compact_dtype, int64_t cs_s, int32_t* positions, int64_t tp_h, int64_t tp_s,
    uint8_t* evict_meta, int64_t em_h, int64_t em_s, int start, int seq_len, int num_kv_heads, int head_dim, int vec,
    const float* k_scale, const float* v_scale, void* stream) {
  if (!keep || !rank) return (int)hipErrorInvalidValue;
  if (seq_len <= 0) return 0;
  const int max_chunks = (seq_len + kChunk - 1) / kChunk;
  return launch_scatter<false>(k, v, kv_dtype, ks_t, ks_h, vs_t, vs_h, seq_evict, es_t, es_h, nullptr, start,
                               seq_len, 1, nullptr, 0, 0, 0, keep, kp_t, kp_h, rank, rk_t, rk_h, base, 0, bs_h,
                               compact_k, compact_v, compact_dtype, cs_s, positions, evict_meta, nullptr, 0, tp_h,
                               tp_s, 0, em_h, em_s, 0, num_kv_heads, head_dim, max_chunks, vec, k_scale, v_scale,
                               stream);
}

// Paged compact KV, prefill side (no reference counterpart: the reference packs
// into flat spans from a host first-fit allocator, compact_kv.py:830-857,
// 955-1099).  Prepare = fdms_streaming_pack_prepare plus the page pop of every
// (seq, head): ceil(live / 16) pages from the layer's free stack into the
// span's block-table row (other entries -1) and held[row, h].  Each pop first
// debits page_budget (one counter per layer, required, at most the stack top:
// the pages not kept for other sequences' decode appends), then takes the
// pages off the stack; neither is retried (fdms_pool.h).  A span whose pages
// do not fit the budget gets none and live 0, and *overflow is raised to 1:
// the caller then gives up the batch (frees its spans).  A stack shorter than
// a fitted debit (budget > top: a caller error) raises it to 2.
// One layer per call; pops use atomics, so which page ids a span gets depends
// on the order the workgroups run in (the rows a rank lands in follow the
// table).
FDMS_EXPORT int fdms_paged_pack_prepare(const uint8_t* evict, int64_t es_t, int64_t es_h, const int32_t* cu_seqlens,
                                        int num_seqs, int window, int num_kv_heads, int max_chunks,
                                        int32_t* live_out, int64_t lo_b, int64_t lo_h, int32_t* block_offsets,
                                        int64_t of_b, int64_t of_h, int64_t of_c, int32_t* positions,
                                        uint8_t* evict_meta, const int32_t* meta_rows, int64_t tp_b, int64_t tp_h,
                                        int64_t em_b, int64_t em_h, int meta_cap, int32_t* page_stack,
                                        int32_t* page_top, int32_t* page_budget, int32_t* block_table,
                                        int64_t bt_b, int64_t bt_h, int32_t* pages_held, int64_t hd_b, int64_t hd_h,
                                        int max_pages, int32_t* overflow, void* stream) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || max_chunks <= 0 || max_pages <= 0) return (int)hipErrorInvalidValue;
  if (!evict || !cu_seqlens || !live_out || !block_offsets || !positions || !evict_meta) return (int)hipErrorInvalidValue;
  if (!page_stack || !page_top || !page_budget || !block_table || !pages_held || !overflow)
    return (int)hipErrorInvalidValue;
  const PagePool pool{page_stack, page_top, page_budget, block_table, bt_b, bt_h, pages_held, hd_b, hd_h, max_pages,
                      overflow};
  hipLaunchKernelGGL(pack_prepare_kernel<true>, prepare_grid(num_seqs, num_kv_heads), dim3(kChunk), 0,
                     (hipStream_t)stream,
                     evict, es_t, es_h, cu_seqlens, 0, window, num_kv_heads, max_chunks, live_out, lo_b, lo_h,
                     block_offsets, of_b, of_h, of_c, positions, evict_meta, meta_rows, tp_b, tp_h, em_b, em_h,
                     meta_cap, pool, num_seqs);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Paged compact KV, prefill side: fdms_streaming_pack_rank_scatter with rank r
// of (seq, head) stored at row block_table[row, h, r >> 4] * 16 + (r & 15)
// (the table written by fdms_paged_pack_prepare).
FDMS_EXPORT int fdms_paged_pack_scatter(
    const void* k, const void* v, int kv_dtype, int64_t ks_t, int64_t ks_h, int64_t vs_t, int64_t vs_h,
    const uint8_t* evict, int64_t es_t, int64_t es_h, const int32_t* cu_seqlens, int num_seqs,
    const int32_t* block_offsets, int64_t bo_b, int64_t bo_h, int64_t bo_c, void* compact_k, void* compact_v,
    int compact_dtype, int64_t cs_s, int32_t* positions, uint8_t* evict_meta, const int32_t* meta_rows, int64_t tp_b,
    int64_t tp_h, int64_t tp_s, int64_t em_b, int64_t em_h, int64_t em_s, const int32_t* block_table, int64_t bt_b,
    int64_t bt_h, int window, int num_kv_heads, int head_dim, int max_chunks, int vec, const float* k_scale,
    const float* v_scale, void* stream) {
  if (!block_offsets || !cu_seqlens) return (int)hipErrorInvalidValue;
  return launch_scatter<true, true>(k, v, kv_dtype, ks_t, ks_h, vs_t, vs_h, evict, es_t, es_h, cu_seqlens, 0, 0,
                                    num_seqs, block_offsets, bo_b, bo_h, bo_c, nullptr, 0, 0, nullptr, 0, 0, nullptr,
                                    0, 0, compact_k, compact_v, compact_dtype, cs_s, positions, evict_meta, meta_rows,
                                    tp_b, tp_h, tp_s, em_b, em_h, em_s, window, num_kv_heads, head_dim, max_chunks,
                                    vec, k_scale, v_scale, stream, block_table, bt_b, bt_h);
}
