// Host replay of the page pool's claim logic (fastdms_amd/csrc/fdms_pool.h).
// Built with g++ by tests/test_pool_claim.py; prints "ok" and exits 0 when
// every check holds.
//
// 1. The interleaving in which a subtract-then-undo pop hands one page out
//    twice (the scheme the pool used before claim_units): replayed step by
//    step on that scheme it must show the double hand-out (a control that the
//    replay can see the failure), and replayed on claim_units it must not.
// 2. A compare-and-swap that finds the counter moved (another claim between
//    the caller's read and its swap) retries with the value it found.
// 3. Many host threads claiming from one counter with real atomics: the
//    claimed ranges are disjoint and, with the counter's final value, cover
//    the pool exactly; every refused claim asked for more than was left at
//    some point.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#include "fdms_pool.h"

static int failures = 0;
#define CHECK(c, msg)                                         \
  do {                                                        \
    if (!(c)) {                                               \
      std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, msg); \
      ++failures;                                             \
    }                                                         \
  } while (0)

struct PlainCas {
  int operator()(int* p, int expected, int desired) const {
    const int found = *p;
    if (found == expected) *p = desired;
    return found;
  }
};

// Marks the stack slots [lo, lo + n) as handed out; returns false when one of
// them already was.
static bool take(std::vector<int>& owner, int lo, int n, int who) {
  bool fresh = true;
  for (int i = lo; i < lo + n; ++i) {
    if (owner[i] >= 0) fresh = false;
    owner[i] = who;
  }
  return fresh;
}

// The ADVICE interleaving on a subtract-then-undo pop: A pops 4, B asks 8 and
// C asks 1 (both fail and leave their subtraction in place), B undoes, D pops
// 5, C undoes.  Each step is one atomic operation of the old scheme.
static void replay_subtract_undo() {
  int top = 10;
  std::vector<int> owner(10, -1);
  bool fresh = true;
  int a = (top -= 4);                      // A: old 10 -> its pages [6, 10)
  fresh &= take(owner, a, 4, 0);
  int b = (top -= 8);                      // B: -2, failed
  int c = (top -= 1);                      // C: -3, failed
  CHECK(b < 0 && c < 0, "control: B and C fail");
  top += 8;                                // B undoes: 5
  int d = (top -= 5);                      // D: 0 -> pages [0, 5)
  CHECK(d >= 0, "control: D succeeds");
  fresh &= take(owner, d, 5, 3);
  top += 1;                                // C undoes: 1
  // the pool now says stack[0] is free while D holds it, and stack[5] is lost
  const bool consistent = fresh && top == 10 - 4 - 5 && owner[5] >= 0;
  CHECK(!consistent, "control: the subtract-then-undo replay must show the inconsistency");
}

// The same requests on claim_units, in the same order.
static void replay_claim_units() {
  int top = 10;
  std::vector<int> owner(10, -1);
  const int a = fdms::claim_units(&top, 4, top, PlainCas{});
  const int b = fdms::claim_units(&top, 8, top, PlainCas{});
  const int c = fdms::claim_units(&top, 1, top, PlainCas{});
  const int d = fdms::claim_units(&top, 5, top, PlainCas{});
  CHECK(a == 6 && b == -1 && c == 5 && d == 0 && top == 0, "claim_units replay values");
  CHECK(take(owner, a, 4, 0) && take(owner, c, 1, 2) && take(owner, d, 5, 3), "claim_units: no page twice");
  for (int i = 0; i < 10; ++i) CHECK(owner[i] >= 0, "claim_units: every page accounted for");
  // a failed claim leaves the counter untouched
  int t2 = 3;
  CHECK(fdms::claim_units(&t2, 4, t2, PlainCas{}) == -1 && t2 == 3, "failed claim writes nothing");
  CHECK(fdms::claim_units(&t2, 3, t2, PlainCas{}) == 0 && t2 == 0, "exact claim empties the counter");
}

// A swap that finds the counter moved: another claimant takes 3 units between
// this claimant's read (10) and its swap.
static void replay_interference() {
  int top = 10;
  int calls = 0;
  auto racing = [&](int* p, int expected, int desired) {
    if (calls++ == 0) *p -= 3;  // the other claim lands first
    return PlainCas{}(p, expected, desired);
  };
  const int got = fdms::claim_units(&top, 4, 10, racing);
  CHECK(got == 3 && top == 3 && calls == 2, "retry with the value the failed swap returned");
  // the counter moved below n: the retry gives up without writing
  top = 5;
  calls = 0;
  auto draining = [&](int* p, int expected, int desired) {
    if (calls++ == 0) *p -= 4;
    return PlainCas{}(p, expected, desired);
  };
  CHECK(fdms::claim_units(&top, 3, 5, draining) == -1 && top == 1, "give up once fewer units are left");
}

struct AtomicCas {
  int operator()(int* p, int expected, int desired) const {
    __atomic_compare_exchange_n(p, &expected, desired, false, __ATOMIC_ACQ_REL, __ATOMIC_ACQUIRE);
    return expected;  // the value found (unchanged when the swap succeeded)
  }
};

static void stress() {
  constexpr int kPool = 20000, kThreads = 8, kPerThread = 4000;
  int top = kPool;
  std::vector<std::atomic<int>> owner(kPool);
  for (auto& o : owner) o.store(-1);
  std::atomic<int> dup{0}, claimed{0};
  std::vector<std::thread> ts;
  for (int w = 0; w < kThreads; ++w) {
    ts.emplace_back([&, w] {
      std::mt19937 rng(1234 + w);
      std::uniform_int_distribution<int> size(1, 9);
      for (int i = 0; i < kPerThread; ++i) {
        const int n = size(rng);
        const int seen = __atomic_load_n(&top, __ATOMIC_ACQUIRE);
        const int lo = fdms::claim_units(&top, n, seen, AtomicCas{});
        if (lo < 0) continue;
        claimed += n;
        for (int j = lo; j < lo + n; ++j) {
          int expect = -1;
          if (!owner[j].compare_exchange_strong(expect, w)) ++dup;
        }
      }
    });
  }
  for (auto& t : ts) t.join();
  CHECK(dup.load() == 0, "stress: no page handed out twice");
  CHECK(claimed.load() + top == kPool, "stress: claimed + left == pool");
  int held = 0;
  for (int i = 0; i < kPool; ++i) held += owner[i].load() >= 0;
  CHECK(held == claimed.load(), "stress: claimed pages are exactly the handed-out slots");
  for (int i = 0; i < top; ++i) CHECK(owner[i].load() < 0, "stress: the slots below top are free");
}

int main() {
  replay_subtract_undo();
  replay_claim_units();
  replay_interference();
  stress();
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
