// Claiming units from a shared counter of free units (the page pool's stack
// top and its per-layer page budget).
//
// A claim of n units succeeds only when the counter holds at least n, and a
// claim that fails never writes the counter: the update is a compare-and-swap
// of the value the claimant saw, retried with the fresher value the failed
// swap returns.  (A subtract-then-undo claim lets a failed claim's transient
// deficit hide units from, or hand the same units to, concurrent claimants;
// see tests/pool_claim_replay.cpp for that interleaving.)
//
// The helper is a template over the compare-and-swap so the same code runs on
// the device (atomicCAS on global memory) and in a host test that replays
// chosen interleavings.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define FDMS_HOST_DEVICE __host__ __device__
#else
#define FDMS_HOST_DEVICE
#endif

namespace fdms {

// Claims n > 0 units.  `seen` is a value of the counter read by the caller
// (any earlier value: a stale one only costs a retry).  Returns the counter's
// value after the claim (the claimed units are [result, result + n) of a
// stack whose top the counter is), or -1 when fewer than n units are left.
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

#if defined(__HIPCC__)
struct DeviceCas {
  __device__ int operator()(int* p, int expected, int desired) const { return atomicCAS(p, expected, desired); }
};
// Device form: one relaxed load for the first guess, then compare-and-swap.
__device__ inline int claim_units(int* counter, int n) {
  const int seen = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return claim_units(counter, n, seen, DeviceCas{});
}
#endif

}  // namespace fdms
