// Copy-to-copy ordering through one gate (the ordering point of one device slot).
//
// A transport may run two copies of one direction at once, on different DMA engines or as
// halves split across two engines, so the order in which copies are issued says nothing about
// the order in which their bytes land. Every copy that touches a slot therefore names the
// earlier copies through the same gate that it must wait for:
//   - a copy that writes the slot (an H2D fill) waits for the gate's last copy of any kind: a
//     fill still in flight (write after write: a fill released or evicted before its unpack
//     can be overtaken by the next one) or a write-back still reading the slot (write after
//     read);
//   - a copy that reads the slot (a D2H or a write-back) waits for the gate's last write into
//     it (read after write). Staging slots are written by kernels, not copies, so their D2H
//     copies wait for nothing here and overlap freely.
// The HIP events of the slot's consumers on compute streams are tracked by the transport
// itself; this header is only the copy-to-copy part, kept free of HIP and HSA so it can be
// tested on the host.
#pragma once

namespace mo {

template <class Ref>
struct GateOrder {
  Ref last;        // the last copy through the gate, of any kind
  Ref last_write;  // the last copy that wrote the gate's slot

  // `c` writes the slot; returns the copy it must wait for (empty if none).
  Ref on_write(const Ref& c) {
    Ref dep = last;
    last = c;
    last_write = c;
    return dep;
  }

  // `c` reads the slot; returns the copy it must wait for (empty if none).
  Ref on_read(const Ref& c) {
    Ref dep = last_write;
    last = c;
    return dep;
  }

  void clear() {
    last = Ref();
    last_write = Ref();
  }
};

}  // namespace mo
