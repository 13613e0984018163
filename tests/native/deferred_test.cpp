// Host test of mo::DeferredHost (moss-image_amd/csrc/mo_deferred.h): coded byte counts are read
// only from host ranges still held, whatever order the copies finish in, and every count whose
// copy finished is read exactly once. Prints "ok" and exits 0 when every check holds.
#include <stdio.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "mo_deferred.h"

struct Copy {
  std::string name;
  bool done = false;
  int flip_after = -1;  // becomes done on this query (a copy finishing between two loops)
  int queries = 0;
};
using Ref = std::shared_ptr<Copy>;

static int failures = 0;
static std::map<const char*, uint64_t> held;  // host ranges still in the pool's hands of the engine
static std::vector<std::string> counted;

static void check(bool ok, const std::string& what) {
  if (!ok) {
    printf("FAIL %s\n", what.c_str());
    ++failures;
  }
}

static bool is_held(const char* p) {
  for (auto& kv : held)
    if (p >= kv.first && p < kv.first + kv.second) return true;
  return false;
}

static bool done(const Ref& r) {
  if (!r) return true;
  ++r->queries;
  if (r->flip_after >= 0 && r->queries >= r->flip_after) r->done = true;
  return r->done;
}

static Ref copy(const char* name, bool finished) {
  Ref r = std::make_shared<Copy>();
  r->name = name;
  r->done = finished;
  return r;
}

using D = mo::DeferredHost<Ref>;

static void settle(D& d) {
  d.settle(
      done,
      [](const D::Count& c) {
        check(is_held(c.host), "count of copy " + c.copy->name + " read a host range already freed");
        counted.push_back(c.copy->name);
      },
      [](char* host, uint64_t bytes) {
        check(held.count(host) && held[host] == bytes, "freed a range that is not held whole");
        held.erase(host);
      });
}

int main() {
  static char arena[1 << 16];
  char* a = arena;
  char* b = arena + 4096;
  char* c = arena + 8192;

  // 1. Out of order: the older count's D2H (split over two engines) is still running when a
  //    younger group's D2H has landed and that group is released; then the pool trims.
  {
    D d;
    held = {{a, 4096}, {b, 4096}};
    counted.clear();
    Ref da = copy("a-d2h", false), db = copy("b-d2h", true);
    d.counts.push_back({a, da, true, 1, 0});
    d.counts.push_back({b, db, true, 2, 0});
    d.frees.push_back({b, 4096, {db, nullptr}});  // group 2 released
    settle(d);
    check(counted.size() == 1 && counted[0] == "b-d2h", "the finished younger count is read before its range is freed");
    check(!held.count(b), "the released range is freed once its copy finished");
    check(d.counts.size() == 1, "the older count waits for its copy");
    da->done = true;
    settle(d);
    check(counted.size() == 2 && counted[1] == "a-d2h", "the older count is read once its copy finished");
    check(d.counts.empty() && d.frees.empty(), "nothing left");
  }

  // 2. A copy that finishes between the count loop and the free loop: its count is read inside
  //    the free loop, before the range goes back.
  {
    D d;
    held = {{c, 4096}};
    counted.clear();
    Ref dc = copy("c-d2h", false);
    dc->flip_after = 2;  // busy for the count loop, finished for the free loop
    d.counts.push_back({c, dc, true, 3, 0});
    d.frees.push_back({c, 4096, {dc, nullptr}});
    settle(d);
    check(counted.size() == 1 && counted[0] == "c-d2h", "a count finishing between the loops is still read");
    check(!held.count(c) && d.counts.empty(), "then the range is freed and the count gone");
  }

  // 3. A range whose own copies are still running is kept with its counts; an H2D count of a
  //    fetched segment is read once the H2D finished, while the segment's range is held.
  {
    D d;
    held = {{a, 4096}};
    counted.clear();
    Ref d2h = copy("a-d2h", true), h2d = copy("a-h2d", false);
    d.counts.push_back({a, h2d, false, 0, 0});
    d.frees.push_back({a, 4096, {d2h, h2d}});
    settle(d);
    check(counted.empty() && held.count(a) && d.frees.size() == 1, "a range is held while a copy of it runs");
    h2d->done = true;
    settle(d);
    check(counted.size() == 1 && counted[0] == "a-h2d" && !held.count(a), "H2D count read, then the range freed");
  }

  // 4. A count inside a range being freed whose copy did not finish is dropped, never read
  //    (its range is freed only once the range's own copies finished).
  {
    D d;
    held = {{b, 4096}};
    counted.clear();
    Ref stray = copy("stray", false);
    d.counts.push_back({b + 64, stray, true, 4, 0});
    d.frees.push_back({b, 4096, {nullptr, nullptr}});
    settle(d);
    check(counted.empty() && d.counts.empty() && !held.count(b), "an unfinished count inside a freed range is dropped");
  }

  // 5. all_done sees every copy referenced.
  {
    D d;
    Ref x = copy("x", true), y = copy("y", false);
    d.counts.push_back({a, x, true, 0, 0});
    d.frees.push_back({a, 16, {x, y}});
    check(!d.all_done(done), "all_done: a free's second copy still runs");
    y->done = true;
    check(d.all_done(done), "all_done once every copy finished");
  }

  if (failures) return 1;
  printf("ok\n");
  return 0;
}
