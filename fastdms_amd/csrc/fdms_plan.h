// The decode step's attention work plan (paged compact KV).
//
// fdms_paged_prepare_decode_plan writes, per layer, one work item for every
// live workgroup of that layer's fdms_fused_decode_attention_planned launch,
// after it has assigned the step's append rows.  A pair of `live` ranks takes
// ns = 1 split when live <= split_rows, else min(num_splits, ceil(live /
// heavy_rows)); split s covers ranks [s * per, (s + 1) * per) with per =
// ceil(live / ns) rounded up to 64 (the in-kernel partition of
// fdms_fused_decode_attention_paged).  Item order: split 0 of pair p at
// index p (so that workgroup knows its pair, and loads the pair's raw q / k /
// v rows, before its item arrives; most pairs have one split), then the
// pairs' further splits packed after the pairs in (pair, split) order; the
// layer's count of those further splits ends the list, and the launch's
// workgroups past it exit.  An item carries everything its workgroup needs
// before its first K/V load: the rank range, the split index and count, the
// live count, the append row and position, and the page id of every 16-rank
// quarter it reads (at most kPlanRows ranks: two 64-row groups per wave of
// the 8-wave workgroup).
#pragma once

namespace fdms {

constexpr int kPlanRows = 1024;                       // ranks per item at most: 8 waves x two 64-row groups
constexpr int kPlanWaves = 8;
constexpr int kPlanPage = 16;                         // rows per page (the paged layout's)
constexpr int kPlanPageShift = 4;
constexpr int kPlanPages = kPlanRows / kPlanPage;     // page ids per item
constexpr int kPlanHeader = 8;                        // header ints
constexpr int kPlanInts = kPlanHeader + kPlanPages;   // 72 ints = 288 bytes, eighteen 16-byte words
// A layer's plan block: kPlanLead ints (the last one: the count of further
// splits), then its items (16-byte aligned).
constexpr int kPlanLead = 4;

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

// Splits of a pair (the unplanned kernel's rule).
__host__ __device__ inline int plan_splits(int live, int split_rows, int heavy_rows, int num_splits) {
  return live <= split_rows ? 1 : (num_splits < (live + heavy_rows - 1) / heavy_rows
                                       ? num_splits : (live + heavy_rows - 1) / heavy_rows);
}
__host__ __device__ inline int plan_split_rows(int live, int splits) {
  return (((live + splits - 1) / splits) + 63) & ~63;
}

}  // namespace fdms
