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
// reference launches once per layer.  The span's metadata is read in chunks of
// 2048 slots (slot c0 + 256 j + thread: every load instruction reads
// contiguous slots); keep / move ranks in slot order come from per-(j, wave)
// ballot counts behind one barrier.  Only rows whose rank changes move (the
// reference's full kernel rewrites every kept row), in passes of 32 KB per
// workgroup: a pass reads all of its sources before any thread writes (a
// destination may alias a source of the same pass), and the next pass's reads
// go out with this pass's writes -- every destination lies below every later
// source (dst = rank <= src, sources ascend).  Rows move as raw bytes, so one
// kernel serves every arena dtype.
#include "fdms_vec.h"

using namespace fdms;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kSlots = 8;                      // metadata slots per thread and chunk
constexpr int kChunk = kThreads * kSlots;      // 2048
constexpr int kMoveBytes = 128;                // row bytes per thread and pass (32 KB per workgroup)
constexpr int kLdsPages = 2048;                // page-table entries staged in LDS (spans up to 32768 rows)

// Physical arena row of span slot r: base + r (flat spans) or, paged,
// table[r >> 4] * 16 + (r & 15).
__device__ __forceinline__ int64_t slot_row(int64_t base, const int32_t* table, int r) {
  return table ? ((int64_t)table[r >> 4] << 4) + (r & 15) : base + r;
}

// The register type of one UNIT-byte access (a plain vector type: the HIP
// uint4 struct kept the move buffers in scratch memory).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
template <int UNIT> struct UnitReg;
template <> struct UnitReg<16> { using type = u32x4_t; };
template <> struct UnitReg<4> { using type = uint32_t; };
template <> struct UnitReg<1> { using type = uint8_t; };

// Global-memory pointers: the arenas arrive as integers (a per-layer pointer
// table), and through a generic pointer every row access would be a flat
// access, which also counts against the LDS counter -- each LDS read of the
// move list or page table would then wait for all row loads in flight.
#define FDMS_GLOBAL __attribute__((address_space(1)))

// Row-move passes over the chunk's move list (s_src / s_dst, ascending
// sources): K rows then V rows, UNIT bytes per access.  A pass's loads are
// unconditional (the units past the end repeat the last one) so that none
// of them waits for its data before the next is issued, and the units stay
// in registers.  TBL: 0 flat spans (row = base + slot), 1 paged with the
// span's page table staged in LDS, 2 paged with the table read from global
// memory (spans longer than the staging).
template <int UNIT, int TBL>
struct Mover {
  static constexpr int kU = kMoveBytes / UNIT < 16 ? kMoveBytes / UNIT : 16;  // units per thread and pass
  using U = typename UnitReg<UNIT>::type;
  FDMS_GLOBAL uint8_t* ck;
  FDMS_GLOBAL uint8_t* cv;
  int64_t base, c_s_bytes;
  const int32_t* table;  // TBL 1: the kernel's LDS copy; TBL 2: global
  int units_per_row, n_moves, total;
  const int* s_src;
  const int* s_dst;

  __device__ __forceinline__ int64_t row(int r) const {
    if constexpr (TBL == 0) {
      return base + r;
    } else if constexpr (TBL == 1) {
      return ((int64_t)table[r >> 4] << 4) + (r & 15);
    } else {
      return ((int64_t)((const FDMS_GLOBAL int32_t*)table)[r >> 4] << 4) + (r & 15);
    }
  }
  __device__ __forceinline__ void read(int p0, U* buf, int64_t* dst_off, int* which) const {
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int u0 = p0 + j * kThreads + (int)threadIdx.x;
      const int u = min(u0, total - 1);  // total > 0
      const int w = u / (n_moves * units_per_row);  // 0 = K, 1 = V
      const int uu = u - w * n_moves * units_per_row;
      const int r = uu / units_per_row;
      const int64_t off = (int64_t)(uu - r * units_per_row) * UNIT;
      const FDMS_GLOBAL uint8_t* arena = w ? cv : ck;
      buf[j] = *reinterpret_cast<const FDMS_GLOBAL U*>(arena + row(s_src[r]) * c_s_bytes + off);
      dst_off[j] = row(s_dst[r]) * c_s_bytes + off;
      which[j] = u0 < total ? w : -1;
    }
  }
  __device__ __forceinline__ void write(const U* buf, const int64_t* dst_off, const int* which) const {
#pragma unroll
    for (int j = 0; j < kU; ++j)
      if (which[j] >= 0) *reinterpret_cast<FDMS_GLOBAL U*>((which[j] ? cv : ck) + dst_off[j]) = buf[j];
  }
  // every pass: its reads, a barrier (all reads of the pass done), its
  // writes; pass p + 1's reads are issued before pass p's writes
  __device__ __forceinline__ void run() const {
    constexpr int kPass = kThreads * kU;
    if (total <= 0) return;
    U b0[kU], b1[kU];
    int64_t o0[kU], o1[kU];
    int w0[kU], w1[kU];
    read(0, b0, o0, w0);
    for (int p0 = 0; p0 < total; p0 += 2 * kPass) {
      __syncthreads();
      if (p0 + kPass < total) read(p0 + kPass, b1, o1, w1);
      write(b0, o0, w0);
      if (p0 + kPass >= total) break;
      __syncthreads();
      if (p0 + 2 * kPass < total) read(p0 + 2 * kPass, b0, o0, w0);
      write(b1, o1, w1);
    }
  }
};

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
  __shared__ int s_cnt[kSlots][kWaves];  // kept, then moved, slots per (j, wave)
  __shared__ int s_hit[kSlots][kWaves];  // INCREMENTAL: first hit of (j, wave), or kChunk
  __shared__ int s_src[kChunk];
  __shared__ int s_dst[kChunk];
  __shared__ int32_t s_table[kLdsPages];  // paged: the span's page ids, read once

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
  const int lane = tid & 63, wave = tid >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t cutoff = cur - (int64_t)window;

  // paged: the span's block-table row into LDS (its loads go out with the
  // first chunk's metadata loads), so a row move waits for one memory round
  // trip, not two
  const int n_pages = (live + 15) >> 4;
  const int32_t* tbl = table;
  if (table && n_pages <= kLdsPages) {
    for (int i = tid; i < n_pages; i += kThreads) s_table[i] = table[i];
    tbl = s_table;  // made visible by the first chunk's barriers
  }
  int running = 0;       // slots kept before this chunk
  int first = live;      // INCREMENTAL: the removed slot, once found
  for (int c0 = 0; c0 < live; c0 += kChunk) {
    int32_t p[kSlots];
    uint8_t e[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const int slot = min(c0 + j * kThreads + tid, live - 1);  // clamped: every load in bounds
      p[j] = pos[slot];
      e[j] = ev[slot];
    }
    bool keep[kSlots];
    if (INCREMENTAL) {
      if (first == live) {  // uniform: look for the first expired slot in this chunk
#pragma unroll
        for (int j = 0; j < kSlots; ++j) {
          const int slot = c0 + j * kThreads + tid;
          const uint64_t m = __ballot(slot < live && e[j] != 0 && (int64_t)p[j] < cutoff);
          if (lane == 0) s_hit[j][wave] = m ? j * kThreads + wave * 64 + (int)__ffsll((unsigned long long)m) - 1 : kChunk;
        }
        __syncthreads();
        int f = kChunk;
#pragma unroll
        for (int j = 0; j < kSlots; ++j)
#pragma unroll
          for (int w = 0; w < kWaves; ++w) f = min(f, s_hit[j][w]);
        if (f < kChunk) first = c0 + f;
      }
#pragma unroll
      for (int j = 0; j < kSlots; ++j) keep[j] = c0 + j * kThreads + tid < live && c0 + j * kThreads + tid != first;
    } else {
#pragma unroll
      for (int j = 0; j < kSlots; ++j)
        keep[j] = c0 + j * kThreads + tid < live && (e[j] == 0 || (cur - (int64_t)p[j]) <= (int64_t)window);
    }
    // ranks in slot order (j-major, then thread): kept and moved counts per (j, wave)
    uint64_t km[kSlots], mm[kSlots];
    int rank_in[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      km[j] = __ballot(keep[j]);
      rank_in[j] = __popcll(km[j] & below);
    }
    // a slot moves when it is kept and slots before it (in this chunk or
    // earlier) were removed: its rank differs from its slot
    int kept_before_wave[kSlots];
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < kSlots; ++j) s_cnt[j][wave] = __popcll(km[j]);
    }
    __syncthreads();  // all metadata reads of the chunk done; counts published
    int acc = 0, tot = 0;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int c = s_cnt[j][w];
        if (w == wave) kept_before_wave[j] = acc;
        acc += c;
      }
    }
    tot = acc;
    int rank[kSlots];
    bool mv[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      rank[j] = running + kept_before_wave[j] + rank_in[j];
      mv[j] = keep[j] && rank[j] != c0 + j * kThreads + tid;
      mm[j] = __ballot(mv[j]);
    }
    __syncthreads();  // the kept counts are read: reuse s_cnt for the move counts
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < kSlots; ++j) s_cnt[j][wave] = __popcll(mm[j]);
    }
    __syncthreads();
    int macc = 0;
    int moved_before_wave[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        if (w == wave) moved_before_wave[j] = macc;
        macc += s_cnt[j][w];
      }
    }
    const int n_moves = macc;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      if (mv[j]) {
        const int idx = moved_before_wave[j] + __popcll(mm[j] & below);
        s_src[idx] = c0 + j * kThreads + tid;
        s_dst[idx] = rank[j];
        pos[rank[j]] = p[j];
        ev[rank[j]] = e[j];
      }
    }
    __syncthreads();  // the move list is complete
    if (n_moves) {
      auto* gk = (FDMS_GLOBAL uint8_t*)ck;
      auto* gv = (FDMS_GLOBAL uint8_t*)cv;
      const int upr = (int)(row_bytes / UNIT), total = n_moves * upr * 2;
      if (!table) {
        Mover<UNIT, 0>{gk, gv, base, c_s_bytes, nullptr, upr, n_moves, total, s_src, s_dst}.run();
      } else if (tbl == s_table) {  // uniform
        Mover<UNIT, 1>{gk, gv, base, c_s_bytes, s_table, upr, n_moves, total, s_src, s_dst}.run();
      } else {
        Mover<UNIT, 2>{gk, gv, base, c_s_bytes, table, upr, n_moves, total, s_src, s_dst}.run();
      }
    }
    running += tot;
    __syncthreads();  // s_src / s_dst / s_cnt are reused by the next chunk
  }
  for (int slot = running + tid; slot < live; slot += kThreads) {
    pos[slot] = -1;
    ev[slot] = 0;
  }
  if (tid == 0) {
    *live_p = running;
    if (table) release_pages(pg, l, table, held, running);
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
