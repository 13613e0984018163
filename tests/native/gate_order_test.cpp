// Host test of mo::GateOrder (moss-image_amd/csrc/mo_gate_order.h): which earlier copy through
// a gate each new copy waits for. Prints "ok" and exits 0 when every check holds.
#include <stdio.h>

#include <memory>
#include <string>

#include "mo_gate_order.h"

using Ref = std::shared_ptr<std::string>;

static int failures = 0;

static void expect(const Ref& got, const Ref& want, const char* what) {
  if (got != want) {
    printf("FAIL %s: waits for %s, expected %s\n", what, got ? got->c_str() : "nothing",
           want ? want->c_str() : "nothing");
    ++failures;
  }
}

static Ref copy(const char* name) { return std::make_shared<std::string>(name); }

int main() {
  // A restore slot: fills only. Each fill waits for the previous one (a fill released or
  // evicted before its unpack may still be in flight on another engine).
  {
    mo::GateOrder<Ref> g;
    Ref f1 = copy("fill1"), f2 = copy("fill2"), f3 = copy("fill3");
    expect(g.on_write(f1), Ref(), "first fill of a restore slot");
    expect(g.on_write(f2), f1, "second fill");
    expect(g.on_write(f3), f2, "third fill");
    expect(g.last, f3, "gate's last copy after fills");
  }
  // A staging slot: D2H reads only, written by kernels. Reads wait for no copy and may overlap.
  {
    mo::GateOrder<Ref> g;
    Ref d1 = copy("d2h1"), d2 = copy("d2h2");
    expect(g.on_read(d1), Ref(), "first D2H of a staging slot");
    expect(g.on_read(d2), Ref(), "second D2H of a staging slot");
    expect(g.last, d2, "gate's last copy after D2H");
  }
  // A streamer slot: fill, write-back, fill, fill, write-back.
  {
    mo::GateOrder<Ref> g;
    Ref f1 = copy("fill1"), w1 = copy("writeback1"), f2 = copy("fill2"), f3 = copy("fill3"),
        w2 = copy("writeback2");
    expect(g.on_write(f1), Ref(), "first fill");
    expect(g.on_read(w1), f1, "write-back after a fill (read after write)");
    expect(g.on_write(f2), w1, "fill after a write-back (write after read)");
    expect(g.on_write(f3), f2, "fill after a fill (write after write)");
    expect(g.on_read(w2), f3, "write-back reads the latest fill");
    g.clear();
    expect(g.on_write(f1), Ref(), "fill after clear");
  }
  if (failures) return 1;
  printf("ok\n");
  return 0;
}
