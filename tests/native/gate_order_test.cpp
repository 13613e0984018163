// Host test of mo::GateOrder (moss-image_amd/csrc/mo_gate_order.h): which earlier copies through
// a gate each new copy waits for, and what must finish before a kernel overwrites the slot.
// Prints "ok" and exits 0 when every check holds.
#include <stdio.h>

#include <algorithm>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "mo_gate_order.h"

struct Copy {
  std::string name;
  bool done = false;
};
using Ref = std::shared_ptr<Copy>;

static int failures = 0;

static bool is_done(const Ref& c) { return !c || c->done; }

static std::string names(const std::vector<Ref>& refs) {
  std::vector<std::string> v;
  for (const Ref& r : refs) v.push_back(r ? r->name : "nothing");
  std::sort(v.begin(), v.end());
  std::string out;
  for (const std::string& n : v) out += (out.empty() ? "" : ",") + n;
  return out.empty() ? "nothing" : out;
}

static void expect(const std::vector<Ref>& got, const std::vector<Ref>& want, const char* what) {
  if (names(got) != names(want)) {
    printf("FAIL %s: waits for %s, expected %s\n", what, names(got).c_str(), names(want).c_str());
    ++failures;
  }
}

static void expect1(const Ref& got, const Ref& want, const char* what) {
  expect(got ? std::vector<Ref>{got} : std::vector<Ref>{}, want ? std::vector<Ref>{want} : std::vector<Ref>{}, what);
}

static Ref copy(const char* name) { return std::make_shared<Copy>(Copy{name}); }

int main() {
  // A restore slot: fills only. Each fill waits for the previous one (a fill released or
  // evicted before its unpack may still be in flight on another engine).
  {
    mo::GateOrder<Ref> g;
    Ref f1 = copy("fill1"), f2 = copy("fill2"), f3 = copy("fill3");
    expect(g.on_write(f1), {}, "first fill of a restore slot");
    expect(g.on_write(f2), {f1}, "second fill");
    expect(g.on_write(f3), {f2}, "third fill");
    expect1(g.last, f3, "gate's last copy after fills");
    expect(g.outstanding(), {f3}, "a kernel overwriting the restore slot waits for the last fill");
  }
  // A staging slot: D2H reads only, written by kernels. Reads wait for no copy and may overlap,
  // and a kernel that overwrites the slot must wait for all of them: a D2H split over two
  // engines can still be running its second half after a later D2H on the first engine ended.
  {
    mo::GateOrder<Ref> g;
    Ref d1 = copy("d2h1"), d2 = copy("d2h2"), d3 = copy("d2h3");
    expect1(g.on_read(d1, is_done), Ref(), "first D2H of a staging slot");
    expect1(g.on_read(d2, is_done), Ref(), "second D2H of a staging slot");
    expect1(g.last, d2, "gate's last copy after D2H");
    d2->done = true;  // the later copy finished first
    expect(g.outstanding(), {d1, d2}, "slot reuse waits for every D2H, not only the last");
    d1->done = true;
    expect1(g.on_read(d3, is_done), Ref(), "third D2H");
    expect(g.outstanding(), {d3}, "finished reads are pruned");
  }
  // A streamer slot: fill, write-back, fill, fill, two write-backs, fill.
  {
    mo::GateOrder<Ref> g;
    Ref f1 = copy("fill1"), w1 = copy("writeback1"), f2 = copy("fill2"), f3 = copy("fill3"),
        w2 = copy("writeback2"), w3 = copy("writeback3"), f4 = copy("fill4");
    expect(g.on_write(f1), {}, "first fill");
    expect1(g.on_read(w1, is_done), f1, "write-back after a fill (read after write)");
    expect(g.on_write(f2), {w1, f1}, "fill after a write-back (write after read)");
    expect(g.on_write(f3), {f2}, "fill after a fill (write after write)");
    expect1(g.on_read(w2, is_done), f3, "write-back reads the latest fill");
    expect1(g.on_read(w3, is_done), f3, "a second write-back reads the same fill");
    expect(g.on_write(f4), {w2, w3, f3}, "fill after two write-backs waits for both");
    g.clear();
    expect(g.on_write(f1), {}, "fill after clear");
  }
  if (failures) return 1;
  printf("ok\n");
  return 0;
}
