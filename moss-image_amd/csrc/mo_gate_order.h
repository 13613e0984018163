// Copy-to-copy ordering through one gate (the ordering point of one device slot).
//
// A transport may run two copies of one direction at once, on different DMA engines or as
// halves split across two engines, so the order in which copies are issued says nothing about
// the order in which their bytes land: a later copy on one engine can finish while an earlier
// copy's half on the other engine still runs. Every copy that touches a slot therefore names
// all the earlier copies through the same gate that it must wait for:
//   - a copy that writes the slot (an H2D fill) waits for the gate's last write (write after
//     write: a fill released or evicted before its unpack can be overtaken by the next one)
//     and for every read since that write (write after read: write-backs still reading it);
//   - a copy that reads the slot (a D2H or a write-back) waits for the gate's last write into
//     it (read after write). Staging slots are written by kernels, not copies, so their D2H
//     copies wait for nothing here and overlap freely.
// Before a kernel overwrites the slot, everything in `outstanding()` must have finished: the
// last write and every read since, not only the last copy.
// The HIP events of the slot's consumers on compute streams are tracked by the transport
// itself; this header is only the copy-to-copy part, kept free of HIP and HSA so it can be
// tested on the host.
#pragma once

#include <utility>
#include <vector>

namespace mo {

template <class Ref>
struct GateOrder {
  Ref last;                // the last copy through the gate, of any kind
  Ref last_write;          // the last copy that wrote the gate's slot
  std::vector<Ref> reads;  // copies that read the slot since `last_write` (finished ones pruned)

  // `c` writes the slot; returns the copies it must wait for.
  std::vector<Ref> on_write(const Ref& c) {
    std::vector<Ref> deps = std::move(reads);
    reads.clear();
    if (last_write) deps.push_back(last_write);
    last = c;
    last_write = c;
    return deps;
  }

  // `c` reads the slot; returns the copy it must wait for (empty if none). `done(ref)` tells
  // which earlier reads have finished, so the list stays as short as the copies in flight.
  template <class Done>
  Ref on_read(const Ref& c, Done done) {
    prune(done);
    reads.push_back(c);
    last = c;
    return last_write;
  }

  // Every copy that may still access the slot: the last write and the reads since.
  std::vector<Ref> outstanding() const {
    std::vector<Ref> all = reads;
    if (last_write) all.push_back(last_write);
    return all;
  }

  template <class Done>
  void prune(Done done) {
    size_t keep = 0;
    for (size_t i = 0; i < reads.size(); ++i)
      if (!done(reads[i])) reads[keep++] = reads[i];
    reads.resize(keep);
  }

  void clear() {
    last = Ref();
    last_write = Ref();
    reads.clear();
  }
};

}  // namespace mo
