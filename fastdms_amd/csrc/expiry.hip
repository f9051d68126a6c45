// DMS decode-time expiry of compact spans (reference:
// fastdms/layers/compact_attention.py:690-858 kernels, 861-965 wrappers;
// fastdms/engine/compact_kv.py:1263-1337 exact torch path, 1396-1560 per-layer
// drivers).
//
// full:        keep = (slot < live) & (~evict | cur - pos <= W); kept slots move to
//              their cumsum rank, trailing metadata -> (-1, False), live = #kept.
// incremental: the first slot with evict & pos < cur - W is removed and the
//              tail shifted left by one; live -= 1.
//
// One block per (layer, sequence, kv head); one launch covers every layer
// (per-layer arena pointers come from a device pointer table), where the
// reference launches once per layer.  Slots are scanned in 256-slot chunks
// with ballot ranks.  Moves are in place with dst <= src, so every chunk (and
// every register-sized pass inside it) reads all of its sources before any
// thread writes: a destination can only alias a source that an earlier pass
// already read.  Only rows whose rank changes are touched (the reference's
// full kernel rewrites every kept row).  Rows move as raw bytes, so one kernel
// serves every arena dtype.
#include "fdms_vec.h"

using namespace fdms;

namespace {

constexpr int kThreads = 256;
constexpr int kUnitsPerThread = 8;

__device__ __forceinline__ int block_rank(bool keep, int* s_wave, int* total) {
  const uint64_t m = __ballot(keep);
  const int lane = __lane_id();
  const int wave = threadIdx.x >> 6;
  const int prefix = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) s_wave[wave] = __popcll(m);
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) {
    const int c = s_wave[w];
    off += (w < wave) ? c : 0;
    tot += c;
  }
  *total = tot;
  return off + prefix;
}

// Copy n_moves rows (src slot s_src[i] -> dst slot s_dst[i], both relative to
// the span base) for K and V, in passes that read everything before writing.
// Physical arena row of span slot r: base + r (flat spans) or, paged,
// table[r >> 4] * 16 + (r & 15).
__device__ __forceinline__ int64_t slot_row(int64_t base, const int32_t* table, int r) {
  return table ? ((int64_t)table[r >> 4] << 4) + (r & 15) : base + r;
}

template <int UNIT>
__device__ void move_rows(uint8_t* ck, uint8_t* cv, int64_t base, int64_t c_s_bytes, int64_t row_bytes,
                          const int* s_src, const int* s_dst, int n_moves, const int32_t* table) {
  const int units_per_row = (int)(row_bytes / UNIT);
  const int total = n_moves * units_per_row * 2;
  for (int p0 = 0; p0 < total; p0 += kThreads * kUnitsPerThread) {
    Vec<uint8_t, UNIT> buf[kUnitsPerThread];
    int64_t dst_off[kUnitsPerThread];
    uint8_t* dst_arena[kUnitsPerThread];
#pragma unroll
    for (int j = 0; j < kUnitsPerThread; ++j) {
      const int u = p0 + j * kThreads + threadIdx.x;
      dst_arena[j] = nullptr;
      if (u < total) {
        const int which = u / (n_moves * units_per_row);  // 0 = K, 1 = V
        const int uu = u - which * n_moves * units_per_row;
        const int r = uu / units_per_row;
        const int64_t off = (int64_t)(uu - r * units_per_row) * UNIT;
        uint8_t* arena = which ? cv : ck;
        buf[j] = *reinterpret_cast<const Vec<uint8_t, UNIT>*>(arena + slot_row(base, table, s_src[r]) * c_s_bytes +
                                                              off);
        dst_arena[j] = arena;
        dst_off[j] = slot_row(base, table, s_dst[r]) * c_s_bytes + off;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kUnitsPerThread; ++j) {
      if (dst_arena[j]) *reinterpret_cast<Vec<uint8_t, UNIT>*>(dst_arena[j] + dst_off[j]) = buf[j];
    }
    __syncthreads();
  }
}

// Paged spans of the expiry launch (table == nullptr: flat spans).  After the
// re-compaction a span keeps ceil(live / 16) pages; the rest go back to the
// layer's free stack (atomic add: distinct ranges).
struct PagedSpans {
  int32_t* table;
  int64_t bt_l, bt_s, bt_h;
  int32_t* held;
  int64_t hd_l, hd_s, hd_h;
  int32_t* stack;
  int64_t stack_stride;
  int32_t* top;
};

__device__ void release_pages(const PagedSpans& pg, int l, int32_t* table, int32_t* held, int live_after) {
  const int keep = (live_after + 15) >> 4;
  const int n = *held;
  if (n > keep) {
    const int32_t at = atomicAdd(pg.top + l, n - keep);
    for (int j = keep; j < n; ++j) {
      pg.stack[l * pg.stack_stride + at + (j - keep)] = table[j];
      table[j] = -1;
    }
    *held = keep;
  }
}

}  // namespace

template <int UNIT, bool INCREMENTAL>
__global__ __launch_bounds__(kThreads) void dms_expiry_kernel(
    int32_t* __restrict__ positions, int64_t ps_l, int64_t ps_s, int64_t ps_h, uint8_t* __restrict__ evict,
    int64_t es_l, int64_t es_s, int64_t es_h, int32_t* __restrict__ live_counts, int64_t lc_l, int64_t lc_s,
    int64_t lc_h, const int32_t* __restrict__ base_offsets, int64_t bo_l, int64_t bo_s, int64_t bo_h,
    uint8_t* compact_k, uint8_t* compact_v, const uint64_t* __restrict__ layer_k, const uint64_t* __restrict__ layer_v,
    int64_t row_bytes, int64_t c_s_bytes, const int64_t* __restrict__ current_positions, int num_kv_heads,
    int window, const PagedSpans pg) {
  __shared__ int s_wave[kThreads / kWave];
  __shared__ int s_wave_mv[kThreads / kWave];
  __shared__ int s_src[kThreads];
  __shared__ int s_dst[kThreads];
  __shared__ int s_first;

  const int l = blockIdx.y;
  const int s = blockIdx.x / num_kv_heads;
  const int h = blockIdx.x - s * num_kv_heads;
  int32_t* pos = positions + l * ps_l + s * ps_s + h * ps_h;
  uint8_t* ev = evict + l * es_l + s * es_s + h * es_h;
  int32_t* live_p = live_counts + l * lc_l + s * lc_s + h * lc_h;
  const int64_t base = pg.table ? 0 : base_offsets[l * bo_l + s * bo_s + h * bo_h];
  int32_t* table = pg.table ? pg.table + l * pg.bt_l + s * pg.bt_s + h * pg.bt_h : nullptr;
  int32_t* held = pg.table ? pg.held + l * pg.hd_l + s * pg.hd_s + h * pg.hd_h : nullptr;
  uint8_t* ck = layer_k ? reinterpret_cast<uint8_t*>(layer_k[l]) : compact_k;
  uint8_t* cv = layer_v ? reinterpret_cast<uint8_t*>(layer_v[l]) : compact_v;
  const int64_t cur = current_positions[s];
  const int live = *live_p;
  const int tid = threadIdx.x;

  if (!INCREMENTAL) {
    int running = 0;
    for (int c0 = 0; c0 < live; c0 += kThreads) {
      const int slot = c0 + tid;
      const bool valid = slot < live;
      int32_t p = -1;
      uint8_t e = 0;
      if (valid) {
        p = pos[slot];
        e = ev[slot];
      }
      const bool keep = valid && ((e == 0) || (cur - (int64_t)p) <= (int64_t)window);
      int total = 0;
      const int r = running + block_rank(keep, s_wave, &total);  // barrier: all reads done
      const bool move = keep && r != slot;
      const uint64_t mm = __ballot(move);
      // compact list of moves (ordered by slot) for the row copy
      {
        const int lane = __lane_id();
        const int wave = tid >> 6;
        if (lane == 0) s_wave_mv[wave] = __popcll(mm);
        __syncthreads();
        int off = 0, nmv = 0;
#pragma unroll
        for (int w = 0; w < kThreads / kWave; ++w) {
          off += (w < wave) ? s_wave_mv[w] : 0;
          nmv += s_wave_mv[w];
        }
        if (move) {
          const int idx = off + __popcll(mm & ((1ull << lane) - 1ull));
          s_src[idx] = slot;
          s_dst[idx] = r;
          pos[r] = p;
          ev[r] = e;
        }
        __syncthreads();
        if (nmv) move_rows<UNIT>(ck, cv, base, c_s_bytes, row_bytes, s_src, s_dst, nmv, table);
      }
      running += total;
      __syncthreads();
    }
    for (int slot = running + tid; slot < live; slot += kThreads) {
      pos[slot] = -1;
      ev[slot] = 0;
    }
    if (tid == 0) {
      *live_p = running;
      if (table) release_pages(pg, l, table, held, running);
    }
    return;
  }

  // incremental: first expired slot
  const int64_t cutoff = cur - (int64_t)window;
  if (tid == 0) s_first = live;
  __syncthreads();
  for (int c0 = 0; c0 < live; c0 += kThreads) {
    const int slot = c0 + tid;
    bool hit = false;
    if (slot < live) hit = ev[slot] != 0 && (int64_t)pos[slot] < cutoff;
    const uint64_t m = __ballot(hit);
    if (m && __lane_id() == 0) atomicMin(&s_first, c0 + (tid & ~63) + (int)__ffsll((unsigned long long)m) - 1);
    __syncthreads();
    const int f = s_first;
    __syncthreads();
    if (f < live) break;
  }
  const int first = s_first;
  if (first >= live) return;
  for (int c0 = first; c0 < live - 1; c0 += kThreads) {
    const int slot = c0 + tid;
    const bool move = slot < live - 1;
    int32_t p = -1;
    uint8_t e = 0;
    if (move) {
      p = pos[slot + 1];
      e = ev[slot + 1];
    }
    const int n = min(kThreads, live - 1 - c0);
    if (tid < n) {
      s_src[tid] = slot + 1;
      s_dst[tid] = slot;
    }
    __syncthreads();  // all metadata reads of this chunk done
    if (move) {
      pos[slot] = p;
      ev[slot] = e;
    }
    move_rows<UNIT>(ck, cv, base, c_s_bytes, row_bytes, s_src, s_dst, n, table);
  }
  if (tid == 0) {
    pos[live - 1] = -1;
    ev[live - 1] = 0;
    *live_p = live - 1;
    if (table) release_pages(pg, l, table, held, live - 1);
  }
}

static int launch_expiry(int incremental, int32_t* positions, int64_t ps_l, int64_t ps_s, int64_t ps_h,
                         uint8_t* evict, int64_t es_l, int64_t es_s, int64_t es_h, int32_t* live_counts,
                         int64_t lc_l, int64_t lc_s, int64_t lc_h, const int32_t* base_offsets, int64_t bo_l,
                         int64_t bo_s, int64_t bo_h, void* compact_k, void* compact_v, const uint64_t* layer_k,
                         const uint64_t* layer_v, int64_t row_bytes, int64_t c_s_bytes,
                         const int64_t* current_positions, int num_layers, int num_seqs, int num_kv_heads,
                         int window, void* stream, const PagedSpans pg) {
  if (num_layers <= 0 || num_seqs < 0 || num_kv_heads <= 0 || row_bytes <= 0) return (int)hipErrorInvalidValue;
  if (num_seqs == 0) return 0;
  if (!positions || !evict || !live_counts || !current_positions) return (int)hipErrorInvalidValue;
  if (pg.table ? (!pg.held || !pg.stack || !pg.top) : !base_offsets) return (int)hipErrorInvalidValue;
  if (!(layer_k && layer_v) && !(compact_k && compact_v)) return (int)hipErrorInvalidValue;
  if ((int64_t)num_seqs * num_kv_heads > 0x7FFFFFFF || num_layers > 65535) return (int)hipErrorInvalidValue;
  const dim3 grid(num_seqs * num_kv_heads, num_layers);
  int unit = 1;
  if (row_bytes % 16 == 0 && c_s_bytes % 16 == 0) unit = 16;
  else if (row_bytes % 4 == 0 && c_s_bytes % 4 == 0) unit = 4;
#define FDMS_EXPIRY_LAUNCH(U, INC)                                                                              \
  hipLaunchKernelGGL((dms_expiry_kernel<U, INC>), grid, dim3(kThreads), 0, (hipStream_t)stream, positions, ps_l, \
                     ps_s, ps_h, evict, es_l, es_s, es_h, live_counts, lc_l, lc_s, lc_h, base_offsets, bo_l, bo_s, \
                     bo_h, (uint8_t*)compact_k, (uint8_t*)compact_v, layer_k, layer_v, row_bytes, c_s_bytes,       \
                     current_positions, num_kv_heads, window, pg)
  if (incremental) {
    if (unit == 16) FDMS_EXPIRY_LAUNCH(16, true);
    else if (unit == 4) FDMS_EXPIRY_LAUNCH(4, true);
    else FDMS_EXPIRY_LAUNCH(1, true);
  } else {
    if (unit == 16) FDMS_EXPIRY_LAUNCH(16, false);
    else if (unit == 4) FDMS_EXPIRY_LAUNCH(4, false);
    else FDMS_EXPIRY_LAUNCH(1, false);
  }
#undef FDMS_EXPIRY_LAUNCH
  FDMS_LAUNCH_CHECK();
  return 0;
}

FDMS_EXPORT int fdms_dms_expiry(int incremental, int32_t* positions, int64_t ps_l, int64_t ps_s, int64_t ps_h,
                                uint8_t* evict, int64_t es_l, int64_t es_s, int64_t es_h, int32_t* live_counts,
                                int64_t lc_l, int64_t lc_s, int64_t lc_h, const int32_t* base_offsets, int64_t bo_l,
                                int64_t bo_s, int64_t bo_h, void* compact_k, void* compact_v, const uint64_t* layer_k,
                                const uint64_t* layer_v, int64_t row_bytes, int64_t c_s_bytes,
                                const int64_t* current_positions, int num_layers, int num_seqs, int num_kv_heads,
                                int window, void* stream) {
  return launch_expiry(incremental, positions, ps_l, ps_s, ps_h, evict, es_l, es_s, es_h, live_counts, lc_l, lc_s,
                       lc_h, base_offsets, bo_l, bo_s, bo_h, compact_k, compact_v, layer_k, layer_v, row_bytes,
                       c_s_bytes, current_positions, num_layers, num_seqs, num_kv_heads, window, stream, PagedSpans{});
}

// Paged-layout expiry (no reference counterpart: the reference re-compacts
// flat spans, compact_attention.py:690-965): the same re-compaction with span
// slot r at row block_table[l, s, h, r >> 4] * 16 + (r & 15), after which each
// span keeps ceil(live / 16) pages and returns the rest to its layer's free
// stack (page_stack[l * stack_stride ...], page_top[l]).
FDMS_EXPORT int fdms_paged_expiry(int incremental, int32_t* positions, int64_t ps_l, int64_t ps_s, int64_t ps_h,
                                  uint8_t* evict, int64_t es_l, int64_t es_s, int64_t es_h, int32_t* live_counts,
                                  int64_t lc_l, int64_t lc_s, int64_t lc_h, int32_t* block_table, int64_t bt_l,
                                  int64_t bt_s, int64_t bt_h, int32_t* pages_held, int64_t hd_l, int64_t hd_s,
                                  int64_t hd_h, int32_t* page_stack, int64_t stack_stride, int32_t* page_top,
                                  const uint64_t* layer_k, const uint64_t* layer_v, int64_t row_bytes,
                                  int64_t c_s_bytes, const int64_t* current_positions, int num_layers, int num_seqs,
                                  int num_kv_heads, int window, void* stream) {
  if (!block_table || !layer_k || !layer_v) return (int)hipErrorInvalidValue;
  const PagedSpans pg{block_table, bt_l, bt_s, bt_h, pages_held, hd_l, hd_s, hd_h, page_stack, stack_stride, page_top};
  return launch_expiry(incremental, positions, ps_l, ps_s, ps_h, evict, es_l, es_s, es_h, live_counts, lc_l, lc_s,
                       lc_h, nullptr, 0, 0, 0, nullptr, nullptr, layer_k, layer_v, row_bytes, c_s_bytes,
                       current_positions, num_layers, num_seqs, num_kv_heads, window, stream, pg);
}
