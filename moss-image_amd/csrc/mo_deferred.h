// Deferred host work of the engine: pinned host ranges that copies may still touch, returned to
// the pool only once those copies have finished, and the coded byte counts of wire-coded copies,
// read from the first u64 of their host range once the copy has finished.
//
// Copies finish out of order: a D2H of 2 MiB or more runs as halves on two DMA engines, a
// smaller one on the first engine alone, and H2D on an engine of its own. So every finished
// count is settled, not only the oldest, and before a host range is freed every count that
// reads inside it is settled (or dropped, when its copy did not finish: a range is freed only
// after its own copies, which include the one a count waits for). A count therefore never
// reads a range that went back to the pool, and a range that `trim` handed back to the driver
// is never read.
//
// Kept free of HIP and HSA so it can be tested on the host (tests/native/deferred_test.cpp).
#pragma once

#include <stdint.h>

#include <deque>

namespace mo {

template <class Ref>
struct DeferredHost {
  struct Free {
    char* host;
    uint64_t bytes;
    Ref copies[2];
  };
  struct Count {
    const char* host;
    Ref copy;
    bool d2h;
    uint64_t group;
    uint32_t seg;
  };

  std::deque<Free> frees;
  std::deque<Count> counts;

  // `done(ref)`: the copy has finished (a null ref counts as finished).
  // `count(c)`: read and account the count `c` (its copy has finished).
  template <class Done, class OnCount>
  void settle_counts(Done done, OnCount count) {
    for (auto it = counts.begin(); it != counts.end();) {
      if (done(it->copy)) {
        count(*it);
        it = counts.erase(it);
      } else {
        ++it;
      }
    }
  }

  // Settles every finished count, then frees every range whose copies have finished, settling
  // the counts inside it first. `release(host, bytes)` returns a range to the pool.
  template <class Done, class OnCount, class OnRelease>
  void settle(Done done, OnCount count, OnRelease release) {
    settle_counts(done, count);
    for (auto it = frees.begin(); it != frees.end();) {
      if (!done(it->copies[0]) || !done(it->copies[1])) {
        ++it;
        continue;
      }
      const char* lo = it->host;
      const char* hi = it->host + it->bytes;
      for (auto c = counts.begin(); c != counts.end();) {
        if (c->host >= lo && c->host < hi) {
          if (done(c->copy)) count(*c);
          c = counts.erase(c);
        } else {
          ++c;
        }
      }
      release(it->host, it->bytes);
      it = frees.erase(it);
    }
  }

  // Whether every copy still referenced has finished.
  template <class Done>
  bool all_done(Done done) const {
    for (const Count& c : counts)
      if (!done(c.copy)) return false;
    for (const Free& f : frees)
      if (!done(f.copies[0]) || !done(f.copies[1])) return false;
    return true;
  }

  void clear() {
    frees.clear();
    counts.clear();
  }
};

}  // namespace mo
