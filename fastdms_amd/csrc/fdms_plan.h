// The decode step's attention work plan (paged compact KV).
//
// fdms_paged_prepare_decode_plan writes, per layer, a list of work items --
// one per workgroup of that layer's fdms_fused_decode_attention_planned
// launch -- after it has assigned the step's append rows.  An item covers at
// most kPlanRows consecutive ranks of one (seq, kv head) span, 64-row aligned,
// so each of the attention workgroup's eight waves holds at most one 64-row
// group, and it carries everything the workgroup needs before its first K/V
// load: the pair, the rank range, the split index and count of the pair, the
// live count, the append row and position, and the page id of every 16-row
// quarter it reads.  The attention kernel then needs one memory round trip
// (the item) before its K/V loads, instead of live count -> page ids -> rows.
#pragma once

namespace fdms {

constexpr int kPlanRows = 512;                        // ranks per item: 8 waves x one 64-row group
constexpr int kPlanPage = 16;                         // rows per page (the paged layout's)
constexpr int kPlanPageShift = 4;
constexpr int kPlanPages = kPlanRows / kPlanPage;     // page ids per item
constexpr int kPlanHeader = 8;                        // header ints
constexpr int kPlanInts = kPlanHeader + kPlanPages;   // 40 ints = 160 bytes, ten 16-byte words

// header fields (int32)
enum PlanField : int {
  kPlanPair = 0,   // b * num_kv_heads + h
  kPlanR0 = 1,     // first rank (a multiple of 64)
  kPlanR1 = 2,     // end rank (exclusive) of the span rows to read; the appended rank is never read back
  kPlanSplit = 3,  // split index | (splits of the pair << 16)
  kPlanLive = 4,   // live count after the append
  kPlanSlot = 5,   // physical row of the append (-1: no append)
  kPlanPos = 6,    // the step's position of the sequence
  kPlanFlags = 7,  // bit 0: this item holds the appended rank (adds that token from registers)
};
// Page ids start at kPlanHeader: entry j is the page holding rank
// min(r0 + 16 j, r1 - 1) (unused when the item reads no rows).

// Items of a pair with `live` ranks: ceil(live / kPlanRows), 64-row aligned
// splits of equal size (the last one shorter).
__host__ __device__ inline int plan_items_of(int live) { return (live + kPlanRows - 1) / kPlanRows; }
__host__ __device__ inline int plan_split_rows(int live, int items) {
  return (((live + items - 1) / items) + 63) & ~63;
}

}  // namespace fdms
