// Decode-step metadata (reference: fastdms/engine/compact_kv.py:1727-1770
// prepare_decode_metadata, 426-484 + 1562-1725 record_appended_dms_decisions).
//
// prepare: slot[l,b,h] = base + live; live += 1 (the append slot of this step,
//          reserved before the forward).
// record:  positions[l,row_b,h,live-1] = pos[b]; evict[...] = evict_all[l,b,h]
//          (the appended token's DMS decision, after the forward).
// One thread per (layer, seq, head); one launch for all layers.  Launch-bound.
#include "fdms_common.h"
#include "fdms_plan.h"
#include "fdms_pool.h"

using namespace fdms;

__global__ void prepare_decode_kernel(const int32_t* __restrict__ base, int64_t b_l, int64_t b_b, int64_t b_h,
                                      int32_t* __restrict__ live, int64_t l_l, int64_t l_b, int64_t l_h,
                                      int32_t* __restrict__ slot, int64_t s_l, int64_t s_b, int64_t s_h, int num_seqs,
                                      int num_kv_heads, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int h = i % num_kv_heads;
  const int b = (i / num_kv_heads) % num_seqs;
  const int l = i / (num_kv_heads * num_seqs);
  int32_t* lp = live + l * l_l + b * l_b + h * l_h;
  const int32_t old = *lp;
  slot[l * s_l + b * s_b + h * s_h] = base[l * b_l + b * b_b + h * b_h] + old;
  *lp = old + 1;
}

FDMS_EXPORT int fdms_prepare_decode_metadata(const int32_t* base, int64_t b_l, int64_t b_b, int64_t b_h,
                                             int32_t* live, int64_t l_l, int64_t l_b, int64_t l_h,
                                             int32_t* slot_out, int64_t s_l, int64_t s_b, int64_t s_h,
                                             int num_layers, int num_seqs, int num_kv_heads, void* stream) {
  if (num_layers <= 0 || num_seqs < 0 || num_kv_heads <= 0) return (int)hipErrorInvalidValue;
  const int total = num_layers * num_seqs * num_kv_heads;
  if (total == 0) return 0;
  if (!base || !live || !slot_out) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(prepare_decode_kernel, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream, base, b_l,
                     b_b, b_h, live, l_l, l_b, l_h, slot_out, s_l, s_b, s_h, num_seqs, num_kv_heads, total);
  FDMS_LAUNCH_CHECK();
  return 0;
}

__global__ void record_decisions_kernel(int32_t* __restrict__ positions, int64_t p_l, int64_t p_s, int64_t p_h,
                                        int64_t p_c, uint8_t* __restrict__ evict, int64_t e_l, int64_t e_s,
                                        int64_t e_h, int64_t e_c, const int32_t* __restrict__ live, int64_t l_l,
                                        int64_t l_s, int64_t l_h, const uint8_t* __restrict__ evict_all, int64_t a_l,
                                        int64_t a_b, int64_t a_h, const void* __restrict__ cur_positions,
                                        int pos_is_64, const int32_t* __restrict__ meta_rows, int row_start,
                                        int num_seqs, int num_kv_heads, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int h = i % num_kv_heads;
  const int b = (i / num_kv_heads) % num_seqs;
  const int l = i / (num_kv_heads * num_seqs);
  const int64_t row = meta_rows ? meta_rows[b] : (int64_t)row_start + b;
  const int64_t idx = (int64_t)live[l * l_l + row * l_s + h * l_h] - 1;
  const int32_t p = pos_is_64 ? (int32_t)((const int64_t*)cur_positions)[b] : ((const int32_t*)cur_positions)[b];
  positions[l * p_l + row * p_s + h * p_h + idx * p_c] = p;
  evict[l * e_l + row * e_s + h * e_h + idx * e_c] = evict_all[l * a_l + b * a_b + h * a_h];
}

FDMS_EXPORT int fdms_record_dms_decisions(int32_t* positions, int64_t p_l, int64_t p_s, int64_t p_h, int64_t p_c,
                                          uint8_t* evict, int64_t e_l, int64_t e_s, int64_t e_h, int64_t e_c,
                                          const int32_t* live, int64_t l_l, int64_t l_s, int64_t l_h,
                                          const uint8_t* evict_all, int64_t a_l, int64_t a_b, int64_t a_h,
                                          const void* cur_positions, int pos_is_64, const int32_t* meta_rows,
                                          int row_start, int num_layers, int num_seqs, int num_kv_heads,
                                          void* stream) {
  if (num_layers <= 0 || num_seqs < 0 || num_kv_heads <= 0) return (int)hipErrorInvalidValue;
  const int total = num_layers * num_seqs * num_kv_heads;
  if (total == 0) return 0;
  if (!positions || !evict || !live || !evict_all || !cur_positions) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(record_decisions_kernel, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     positions, p_l, p_s, p_h, p_c, evict, e_l, e_s, e_h, e_c, live, l_l, l_s, l_h, evict_all, a_l,
                     a_b, a_h, cur_positions, pos_is_64, meta_rows, row_start, num_seqs, num_kv_heads, total);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// ---------------------------------------------------------------------------
// Paged compact KV (no reference counterpart: the reference appends into flat
// spans, slot = base + live, compact_kv.py:1727-1770).  Per layer l the pool
// holds free page ids stack[l * stack_stride + 0 .. top[l]); span (l, b, h)
// owns pages bt[l, b, h, 0 .. held[l, b, h]) of 16 rows each.
// ---------------------------------------------------------------------------
constexpr int kPagedShift = 4;

// Decode append slot with on-demand pages: when the span's pages are full
// (live == 16 * held) one page is popped from the layer's stack (atomic,
// distinct per thread) and appended to the span's table; then slot = the
// physical row of rank live, and live += 1.  A pool that is short gives slot
// -1 (no append) and sets *overflow.
__global__ void paged_prepare_decode_kernel(int32_t* __restrict__ live, int64_t l_l, int64_t l_b, int64_t l_h,
                                            int32_t* __restrict__ slot, int64_t s_l, int64_t s_b, int64_t s_h,
                                            int32_t* __restrict__ bt, int64_t bt_l, int64_t bt_b, int64_t bt_h,
                                            int32_t* __restrict__ held, int64_t hd_l, int64_t hd_b, int64_t hd_h,
                                            const int32_t* __restrict__ stack, int64_t stack_stride,
                                            int32_t* __restrict__ top, int max_pages, int32_t* __restrict__ overflow,
                                            int num_seqs, int num_kv_heads, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int h = i % num_kv_heads;
  const int b = (i / num_kv_heads) % num_seqs;
  const int l = i / (num_kv_heads * num_seqs);
  int32_t* lp = live + l * l_l + b * l_b + h * l_h;
  int32_t* hp = held + l * hd_l + b * hd_b + h * hd_h;
  int32_t* btr = bt + l * bt_l + b * bt_b + h * bt_h;
  int32_t* sp = slot + l * s_l + b * s_b + h * s_h;
  const int32_t n = *lp;
  int32_t np = *hp;
  if (n >= (np << kPagedShift)) {
    int32_t got = -1;
    if (np < max_pages) {
      const int32_t t = fdms::claim_units(top + l, 1);  // compare-and-swap: a failed claim writes nothing
      if (t >= 0) got = stack[l * stack_stride + t];
    }
    if (got < 0) {
      atomicExch(overflow, 1);
      *sp = -1;
      return;
    }
    btr[np] = got;
    *hp = ++np;
  }
  *sp = (btr[n >> kPagedShift] << kPagedShift) + (n & ((1 << kPagedShift) - 1));
  *lp = n + 1;
}

FDMS_EXPORT int fdms_paged_prepare_decode(int32_t* live, int64_t l_l, int64_t l_b, int64_t l_h, int32_t* slot_out,
                                          int64_t s_l, int64_t s_b, int64_t s_h, int32_t* block_table, int64_t bt_l,
                                          int64_t bt_b, int64_t bt_h, int32_t* pages_held, int64_t hd_l,
                                          int64_t hd_b, int64_t hd_h, const int32_t* page_stack,
                                          int64_t stack_stride, int32_t* page_top, int max_pages, int32_t* overflow,
                                          int num_layers, int num_seqs, int num_kv_heads, void* stream) {
  if (num_layers <= 0 || num_seqs < 0 || num_kv_heads <= 0 || max_pages <= 0) return (int)hipErrorInvalidValue;
  const int total = num_layers * num_seqs * num_kv_heads;
  if (total == 0) return 0;
  if (!live || !slot_out || !block_table || !pages_held || !page_stack || !page_top || !overflow)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(paged_prepare_decode_kernel, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     live, l_l, l_b, l_h, slot_out, s_l, s_b, s_h, block_table, bt_l, bt_b, bt_h, pages_held, hd_l,
                     hd_b, hd_h, page_stack, stack_stride, page_top, max_pages, overflow, num_seqs, num_kv_heads,
                     total);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// The same slot assignment with the step's attention work plan (fdms_plan.h):
// one workgroup per layer, so the layer's page pops need no atomics -- the
// spans that need a page take stack entries top-1, top-2, ... in (seq, head)
// order of a block prefix count (pops past the stack fail: slot -1, overflow).
// Then each span's items go to their fixed grid positions split *
// padded_pairs + pair: rank range, split count, live count, append row,
// position and page ids; split 0 of pair p at item p, the further splits
// after the pairs at the block prefix of their counts, and their number in
// the int before the layer's items.
constexpr int kPlanThreads = 1024;
constexpr int kPlanMaxPairsPerThread = 8;  // pairs per layer <= 8192

// Exclusive prefix over the block of one value per thread; returns the
// thread's prefix, *total the block's sum.  Every thread must call it.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_buf, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_buf[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
  const int nw = blockDim.x >> 6;
  for (int w = 0; w < nw; ++w) {
    const int t = s_buf[w];
    before += w < wave ? t : 0;
    all += t;
  }
  __syncthreads();  // s_buf is reused by the next scan
  *total = all;
  return before + x - v;
}

__global__ __launch_bounds__(kPlanThreads) void paged_prepare_decode_plan_kernel(
    int32_t* __restrict__ live, int64_t l_l, int64_t l_b, int64_t l_h, int32_t* __restrict__ slot, int64_t s_l,
    int64_t s_b, int64_t s_h, int32_t* __restrict__ bt, int64_t bt_l, int64_t bt_b, int64_t bt_h,
    int32_t* __restrict__ held, int64_t hd_l, int64_t hd_b, int64_t hd_h, const int32_t* __restrict__ stack,
    int64_t stack_stride, int32_t* __restrict__ top, int max_pages, int32_t* __restrict__ overflow,
    const int64_t* __restrict__ positions, int32_t* __restrict__ plan, int64_t plan_l, int split_rows,
    int heavy_rows, int num_splits, int num_seqs, int num_kv_heads) {
  __shared__ int s_buf[kPlanThreads / 64];
  const int l = blockIdx.x;
  const int tid = threadIdx.x;
  const int pairs = num_seqs * num_kv_heads;
  const int top0 = top[l];
  int pops = 0, extra_before = 0;
  int32_t* lp = plan + l * plan_l + kPlanLead;  // the layer's items; its further-split count at lp[-1]
  const int nt = blockDim.x;  // a multiple of 64: the batch's pairs rounded up, at most kPlanThreads
#pragma unroll
  for (int k = 0; k < kPlanMaxPairsPerThread; ++k) {
    if (k * nt >= pairs) break;  // uniform
    const int p = tid + k * nt;
    int n = 0, np = 0;
    bool need = false;
    int b = 0, h = 0;
    if (p < pairs) {
      b = p / num_kv_heads;
      h = p - b * num_kv_heads;
      n = live[l * l_l + b * l_b + h * l_h];
      np = held[l * hd_l + b * hd_b + h * hd_h];
      need = n >= (np << kPagedShift);
    }
    // pops in (seq, head) order: pair p = tid + k * nt ranks among the
    // needers of this round after those of the earlier rounds
    int tot = 0;
    const int j = block_exclusive_scan(need ? 1 : 0, s_buf, &tot) + pops;
    pops += tot;
    int32_t* btr = bt + l * bt_l + b * bt_b + h * bt_h;
    bool ok = true;
    if (need) {
      ok = np < max_pages && j < top0;
      if (ok) {
        btr[np] = stack[l * stack_stride + top0 - 1 - j];
        held[l * hd_l + b * hd_b + h * hd_h] = np + 1;
      } else {
        atomicExch(overflow, 1);
      }
    }
    int32_t app = -1;
    if (p < pairs && ok) {
      app = (btr[n >> kPagedShift] << kPagedShift) + (n & ((1 << kPagedShift) - 1));
      live[l * l_l + b * l_b + h * l_h] = n + 1;
      n += 1;
    }
    if (p < pairs) slot[l * s_l + b * s_b + h * s_h] = app;
    // the pair's items: split 0 at p, the further ones packed after the pairs
    const int ns = (p < pairs && n > 0) ? plan_splits(n, split_rows, heavy_rows, num_splits) : 1;
    int extra_tot = 0;
    const int extra = block_exclusive_scan(p < pairs ? ns - 1 : 0, s_buf, &extra_tot) + extra_before;
    extra_before += extra_tot;
    if (p >= pairs) continue;
    const int per = plan_split_rows(n, ns);
    const int pos = (int)positions[b];
    for (int sp = 0; sp < ns; ++sp) {
      int32_t* it = lp + (int64_t)(sp == 0 ? p : pairs + extra + sp - 1) * kPlanInts;
      const int r0 = min(n, sp * per);
      int r1 = min(n, r0 + per);
      int flags = 0;
      if (app >= 0 && r0 < n && r1 == n) {
        flags = 1;
        r1 = n - 1;
      }
      reinterpret_cast<int4*>(it)[0] = make_int4(p, r0, r1, sp | (ns << 16));
      reinterpret_cast<int4*>(it)[1] = make_int4(n, app, pos, flags);
      const int last = max(r1 - 1, r0);
      const int used = r1 > r0 ? (r1 - r0 + 63) / 64 * 4 : 0;  // quarters of the item's groups
      // the item's page ids are table entries r0 / 16 .. (clamped at the
      // page of its last rank): every load goes out before the first store
      // (unconditional, indices in bounds), one memory latency per item
      if (n > 0) {
        const int q0 = r0 >> kPagedShift, ql = min(last, n - 1) >> kPagedShift;  // a held page, even for an empty item
        int32_t ids[kPlanPages];
#pragma unroll
        for (int j = 0; j < kPlanPages; ++j) ids[j] = btr[min(q0 + j, ql)];
#pragma unroll
        for (int j4 = 0; j4 < kPlanPages; j4 += 4)
          if (j4 < used)
            reinterpret_cast<int4*>(it + kPlanHeader)[j4 / 4] = make_int4(ids[j4], ids[j4 + 1], ids[j4 + 2], ids[j4 + 3]);
      }
    }
  }
  if (tid == 0) {
    top[l] = max(0, top0 - pops);
    lp[-1] = extra_before;
  }
}

FDMS_EXPORT int fdms_paged_prepare_decode_plan(int32_t* live, int64_t l_l, int64_t l_b, int64_t l_h,
                                               int32_t* slot_out, int64_t s_l, int64_t s_b, int64_t s_h,
                                               int32_t* block_table, int64_t bt_l, int64_t bt_b, int64_t bt_h,
                                               int32_t* pages_held, int64_t hd_l, int64_t hd_b, int64_t hd_h,
                                               const int32_t* page_stack, int64_t stack_stride, int32_t* page_top,
                                               int max_pages, int32_t* overflow, const int64_t* positions,
                                               int32_t* plan, int64_t plan_l, int split_rows, int heavy_rows,
                                               int num_splits, int num_layers, int num_seqs, int num_kv_heads,
                                               void* stream) {
  if (num_layers <= 0 || num_seqs < 0 || num_kv_heads <= 0 || max_pages <= 0 || num_splits <= 0)
    return (int)hipErrorInvalidValue;
  if (split_rows < 64 || split_rows > kPlanRows || heavy_rows < 64 || heavy_rows > split_rows ||
      (split_rows % 64) || (heavy_rows % 64))
    return (int)hipErrorInvalidValue;
  if ((int64_t)num_seqs * num_kv_heads > (int64_t)kPlanThreads * kPlanMaxPairsPerThread)
    return (int)hipErrorInvalidValue;
  if (!live || !slot_out || !block_table || !pages_held || !page_stack || !page_top || !overflow || !positions ||
      !plan)
    return (int)hipErrorInvalidValue;
  if (num_seqs == 0) return 0;
  const int64_t items = (int64_t)num_splits * num_seqs * num_kv_heads;
  if (((uintptr_t)plan % 16) || plan_l % 4 || plan_l < kPlanLead + items * kPlanInts) return (int)hipErrorInvalidValue;
  const int pairs = num_seqs * num_kv_heads;
  const int threads = pairs >= kPlanThreads ? kPlanThreads : ((pairs + 63) / 64) * 64;
  hipLaunchKernelGGL(paged_prepare_decode_plan_kernel, dim3(num_layers), dim3(threads), 0, (hipStream_t)stream,
                     live, l_l, l_b, l_h, slot_out, s_l, s_b, s_h, block_table, bt_l, bt_b, bt_h, pages_held, hd_l,
                     hd_b, hd_h, page_stack, stack_stride, page_top, max_pages, overflow, positions, plan, plan_l,
                     split_rows, heavy_rows, num_splits, num_seqs, num_kv_heads);
  FDMS_LAUNCH_CHECK();
  return 0;
}

// Return every page of the spans of rows[0 .. num_rows) (all layers, all kv
// heads) to the layers' stacks and clear their tables (the sequence-free of
// the paged layout; the span layout's is the host free list).  One thread per
// (layer, row, head); pushes take distinct stack ranges with an atomic add.
__global__ void paged_free_kernel(const int32_t* __restrict__ rows, int num_rows, int32_t* __restrict__ bt,
                                  int64_t bt_l, int64_t bt_b, int64_t bt_h, int32_t* __restrict__ held, int64_t hd_l,
                                  int64_t hd_b, int64_t hd_h, int32_t* __restrict__ live, int64_t l_l, int64_t l_b,
                                  int64_t l_h, int32_t* __restrict__ stack, int64_t stack_stride,
                                  int32_t* __restrict__ top, int num_kv_heads, int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int h = i % num_kv_heads;
  const int r = (i / num_kv_heads) % num_rows;
  const int l = i / (num_kv_heads * num_rows);
  const int64_t row = rows[r];
  int32_t* hp = held + l * hd_l + row * hd_b + h * hd_h;
  int32_t* btr = bt + l * bt_l + row * bt_b + h * bt_h;
  const int32_t n = *hp;
  if (n > 0) {
    const int32_t at = atomicAdd(top + l, n);
    for (int j = 0; j < n; ++j) {
      stack[l * stack_stride + at + j] = btr[j];
      btr[j] = -1;
    }
  }
  *hp = 0;
  live[l * l_l + row * l_b + h * l_h] = 0;
}

FDMS_EXPORT int fdms_paged_free(const int32_t* rows, int num_rows, int32_t* block_table, int64_t bt_l, int64_t bt_b,
                                int64_t bt_h, int32_t* pages_held, int64_t hd_l, int64_t hd_b, int64_t hd_h,
                                int32_t* live, int64_t l_l, int64_t l_b, int64_t l_h, int32_t* page_stack,
                                int64_t stack_stride, int32_t* page_top, int num_layers, int num_kv_heads,
                                void* stream) {
  if (num_layers <= 0 || num_rows < 0 || num_kv_heads <= 0) return (int)hipErrorInvalidValue;
  const int total = num_layers * num_rows * num_kv_heads;
  if (total == 0) return 0;
  if (!rows || !block_table || !pages_held || !live || !page_stack || !page_top) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(paged_free_kernel, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream, rows, num_rows,
                     block_table, bt_l, bt_b, bt_h, pages_held, hd_l, hd_b, hd_h, live, l_l, l_b, l_h, page_stack,
                     stack_stride, page_top, num_kv_heads, total);
  FDMS_LAUNCH_CHECK();
  return 0;
}
