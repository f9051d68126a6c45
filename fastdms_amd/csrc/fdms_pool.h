// Taking pages from a layer's free-page pool: the stack top (the number of
// free page ids on the stack) and, for a prefill's packs, a page budget.
//
// Two forms:
//
// * claim_units (decode appends, one page at a time): a compare-and-swap of
//   the value the claimant saw, retried with the fresher value a failed swap
//   returns.  A claim that fails writes nothing.
// * debit_budget + pop_pages (a prefill's packs, ceil(live / 16) pages per
//   span, every span of a layer at once): one atomic subtract each, no
//   retries, so 64+ concurrent claimants do not serialise.  The budget is
//   debited first; a debit that finds the budget short adds its amount back.
//   That transient deficit can refuse another, concurrent debit that would
//   have fit -- but only while a debit is failing, and the first failing
//   debit of a launch saw no deficit, so it was short for real: a launch
//   with a spurious refusal always holds a genuine one (and the caller then
//   gives up the whole batch).  Successful debits never sum to more than the
//   budget, so with budget <= top (the caller's precondition: the budget is
//   the pool minus every running sequence's page bound) a pop after a
//   successful debit always finds its pages: the stack top is only ever
//   subtracted from, never undone, and no page id is handed out twice.
//   (A multi-page subtract-then-undo on the stack top itself could hand one
//   page out twice; tests/pool_claim_replay.cpp replays that interleaving.)
//
// The helpers are templates over the atomic operations so the same code runs
// on the device and in a host test that replays chosen interleavings.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define FDMS_HOST_DEVICE __host__ __device__
#else
#define FDMS_HOST_DEVICE
#endif

namespace fdms {

// Claims n > 0 units by compare-and-swap.  `seen` is a value of the counter
// read by the caller (a stale one only costs a retry).  Returns the counter's
// value after the claim (the units [result, result + n) of a stack whose top
// the counter is), or -1 when fewer than n units are left.
// cas(counter, expected, desired) stores `desired` if the counter equals
// `expected` and returns the value it found.
template <class Cas>
FDMS_HOST_DEVICE inline int claim_units(int* counter, int n, int seen, Cas cas) {
  while (seen >= n) {
    const int found = cas(counter, seen, seen - n);
    if (found == seen) return seen - n;
    seen = found;
  }
  return -1;
}

// Debits n > 0 pages from a budget counter: true when they fit.
// sub / add(counter, n) are atomic and return the value before the operation.
template <class Sub, class Add>
FDMS_HOST_DEVICE inline bool debit_budget(int* budget, int n, Sub sub, Add add) {
  if (sub(budget, n) >= n) return true;
  add(budget, n);
  return false;
}

// Pops n > 0 page ids after a successful debit: returns the stack index of the
// first (the ids are stack[result .. result + n)), or -1 if the stack was
// short, which the budget precondition rules out (the counter is then left
// as it is and the caller reports a broken pool).
template <class Sub>
FDMS_HOST_DEVICE inline int pop_pages(int* top, int n, Sub sub) {
  const int old = sub(top, n);
  return old >= n ? old - n : -1;
}

#if defined(__HIPCC__)
struct DeviceCas {
  __device__ int operator()(int* p, int expected, int desired) const { return atomicCAS(p, expected, desired); }
};
struct DeviceSub {
  __device__ int operator()(int* p, int n) const { return atomicSub(p, n); }
};
struct DeviceAdd {
  __device__ int operator()(int* p, int n) const { return atomicAdd(p, n); }
};
// Device form of claim_units: one relaxed load for the first guess.
__device__ inline int claim_units(int* counter, int n) {
  const int seen = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return claim_units(counter, n, seen, DeviceCas{});
}
#endif

}  // namespace fdms
