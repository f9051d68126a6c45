// Host replay of the page pool's claim logic (fastdms_amd/csrc/fdms_pool.h).
// Built with g++ by tests/test_pool_claim.py; prints "ok" and exits 0 when
// every check holds.
//
// 1. The interleaving in which a subtract-then-undo pop on the stack top
//    hands one page out twice: replayed step by step on that scheme it must
//    show the double hand-out (a control that the replay can see the
//    failure); replayed on claim_units, and on debit_budget + pop_pages with
//    the same requests, it must not.
// 2. A compare-and-swap that finds the counter moved (another claim between
//    the caller's read and its swap) retries with the value it found.
// 3. Many host threads claiming with real atomics, through claim_units and
//    through debit_budget + pop_pages (budget <= top): the claimed ranges are
//    disjoint and, with the counter's final value, cover the pool exactly;
//    no pop after a fitted debit finds the stack short.
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

// An interleaving of subtract-then-undo pops: A pops 4, B asks 8 and
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

// The same requests through the pack's scheme: each claimant debits the
// budget (subtract; add back on failure), then pops the stack (subtract).
// The budget starts equal to the stack top, the steps interleave as above.
static void replay_debit_pop() {
  int top = 10, budget = 10;
  std::vector<int> owner(10, -1);
  auto sub = [](int* p, int n) { const int o = *p; *p -= n; return o; };
  auto add = [](int* p, int n) { const int o = *p; *p += n; return o; };
  // A debits 4 and pops
  CHECK(sub(&budget, 4) >= 4, "A debit");
  const int a = fdms::pop_pages(&top, 4, sub);
  // B (8) and C (1) subtract from the budget: both find it short
  const bool b_ok = sub(&budget, 8) >= 8;
  const bool c_ok = sub(&budget, 1) >= 1;  // refused while B's deficit is in flight
  CHECK(!b_ok && !c_ok, "B refused for real, C refused while B is failing");
  add(&budget, 8);  // B adds back
  // D debits 5 and pops
  CHECK(fdms::debit_budget(&budget, 5, sub, add), "D debit");
  const int d = fdms::pop_pages(&top, 5, sub);
  add(&budget, 1);  // C adds back
  CHECK(a == 6 && d == 1 && top == 1 && budget == 1, "debit/pop replay values");
  CHECK(take(owner, a, 4, 0) && take(owner, d, 5, 3), "debit/pop: no page twice");
  CHECK(owner[0] < 0, "debit/pop: the page below top is still free");
  // a pop with the stack shorter than the debit (budget > top: the caller's
  // precondition broken) reports -1 and the caller flags the pool
  int t2 = 2;
  CHECK(fdms::pop_pages(&t2, 3, sub) == -1, "short stack reported");
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

static void stress_debit_pop() {
  constexpr int kPool = 20000, kBudget = 15000, kThreads = 8, kPerThread = 3000;
  int top = kPool, budget = kBudget;
  std::vector<std::atomic<int>> owner(kPool);
  for (auto& o : owner) o.store(-1);
  std::atomic<int> dup{0}, claimed{0}, short_pops{0};
  auto sub = [](int* p, int n) { return __atomic_fetch_sub(p, n, __ATOMIC_ACQ_REL); };
  auto add = [](int* p, int n) { return __atomic_fetch_add(p, n, __ATOMIC_ACQ_REL); };
  std::vector<std::thread> ts;
  for (int w = 0; w < kThreads; ++w) {
    ts.emplace_back([&, w] {
      std::mt19937 rng(777 + w);
      std::uniform_int_distribution<int> size(1, 12);
      for (int i = 0; i < kPerThread; ++i) {
        const int n = size(rng);
        if (!fdms::debit_budget(&budget, n, sub, add)) continue;
        const int lo = fdms::pop_pages(&top, n, sub);
        if (lo < 0) {
          ++short_pops;
          continue;
        }
        claimed += n;
        for (int j = lo; j < lo + n; ++j) {
          int expect = -1;
          if (!owner[j].compare_exchange_strong(expect, w)) ++dup;
        }
      }
    });
  }
  for (auto& t : ts) t.join();
  CHECK(short_pops.load() == 0, "debit/pop stress: no pop after a fitted debit finds the stack short");
  CHECK(dup.load() == 0, "debit/pop stress: no page handed out twice");
  CHECK(claimed.load() <= kBudget, "debit/pop stress: never more than the budget");
  CHECK(claimed.load() + top == kPool && claimed.load() + budget == kBudget, "debit/pop stress: counters agree");
  for (int i = 0; i < top; ++i) CHECK(owner[i].load() < 0, "debit/pop stress: the slots below top are free");
}

int main() {
  replay_subtract_undo();
  replay_claim_units();
  replay_interference();
  replay_debit_pop();
  stress();
  stress_debit_pop();
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
