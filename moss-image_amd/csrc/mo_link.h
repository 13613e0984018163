// Host-link transport of the engine: how a staging segment gets to pinned host memory and
// back, and how the compute stream is ordered against those copies.
//
// Two implementations:
//   SdmaLink    (default) the MI355X's SDMA copy engines through the HSA runtime
//               (hsa_amd_memory_async_copy_on_engine). No compute unit is used, so copies
//               overlap GEMM-heavy compute without slowing it. Ordering with HIP streams:
//                 compute -> copy : an issuer thread queries the HIP event recorded after the
//                                   producing kernels, then issues the copy,
//                 copy -> copy    : the issuer holds a copy until the one it depends on finished,
//                 copy -> compute : the host waits for the copy's HSA signal before it enqueues
//                                   the dependent kernels (wait()).
//               No GPU queue ever waits on host-written memory, and every wait is bounded.
//   StreamLink  copies on dedicated HIP streams, ordered with HIP events only (every wait is a
//               hipStreamWaitEvent; the host never blocks for a copy). Two methods:
//                 DMA          hipMemcpyAsync with hipMemcpyDeviceToDeviceNoCU between pinned
//                              host and device memory, which the HIP runtime runs on the SDMA
//                              engines; D2H optionally split in halves over two streams,
//                 copy kernel  the engine's copy kernel (comparison: contends for CUs).
//
// A "gate" is the ordering point of one device slot (staging or restore): copies into or out
// of the slot go through its gate, and the compute stream waits on the gate before it touches
// the slot again.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <memory>
#include <string>

namespace mo {

// Completion state of one copy, shared between segment bookkeeping and the transport.
struct CopyState {
  virtual ~CopyState() = default;
  // The copy finished (or failed) and the transport holds no more references to it.
  virtual bool done() const = 0;
  virtual bool failed() const = 0;
  // The copy no longer waits for anything but the transport itself: waiting for it takes at
  // most the transfer time of what is queued ahead of it on its engine.
  virtual bool started() const { return done(); }
};
using CopyRef = std::shared_ptr<CopyState>;

struct LinkStats {
  uint64_t d2h_bytes = 0, h2d_bytes = 0;        // issued (sized copies: their largest size)
  uint64_t d2h_done_bytes = 0, h2d_done_bytes = 0;  // completed and timed
  double d2h_ms = 0, h2d_ms = 0;                // engine-busy time of completed copies
  uint64_t failures = 0;
  uint64_t host_blocks = 0;                     // wait() calls that had to block the host
  double host_block_ms = 0;                     // time spent blocked in them
};

class Link {
 public:
  virtual ~Link() = default;
  virtual int new_gate(int* gate) = 0;
  // Copy device `src` to pinned host `dst` once the work enqueued so far on `compute` is done.
  // Completion is published through `gate`.
  virtual int d2h(void* dst, const void* src, uint64_t bytes, hipStream_t compute, int gate, CopyRef* out) = 0;
  // Copy pinned host `src` to device `dst` once `after` (the D2H that filled src) finished and
  // the gate's last consumer (see consumed()) finished. Completion is published through `gate`.
  virtual int h2d(void* dst, const void* src, uint64_t bytes, const CopyRef& after, int gate, CopyRef* out) = 0;
  // Copy the slot behind `gate` (device `src`) to pinned host `dst` once the gate's last
  // consumer (see consumed()) finished. The gate's next h2d (given this copy as `after`) and
  // wait() are ordered behind it.
  virtual int writeback(void* dst, const void* src, uint64_t bytes, int gate, CopyRef* out) = 0;
  // Order work enqueued on `compute` after this call behind the gate's last copy (no-op if
  // none): SdmaLink blocks the host until the copy finished; StreamLink makes the stream wait.
  virtual int wait(int gate, hipStream_t compute) = 0;
  // Record that the slot behind `gate` is free for the next copy once `compute` reaches here.
  virtual int consumed(int gate, hipStream_t compute) = 0;
  // Block until every copy issued so far finished.
  virtual int synchronize() = 0;
  // Sized copies: the byte count is read from pinned host memory at `size` when the copy is
  // issued, which is after its dependencies finished (for d2h_sized: the work enqueued on
  // `compute`, which writes *size; for h2d_sized: `after`, whose bytes begin with it), and is
  // clamped to [1, max_bytes]. Only a transport that issues copies after their dependencies
  // can take them (sized_copies()).
  virtual bool sized_copies() const { return false; }
  virtual int d2h_sized(void* dst, const void* src, const volatile uint64_t* size, uint64_t max_bytes,
                        hipStream_t compute, int gate, CopyRef* out) {
    (void)dst, (void)src, (void)size, (void)max_bytes, (void)compute, (void)gate, (void)out;
    return (int)hipErrorNotSupported;
  }
  virtual int h2d_sized(void* dst, const void* src, const volatile uint64_t* size, uint64_t max_bytes,
                        const CopyRef& after, int gate, CopyRef* out) {
    (void)dst, (void)src, (void)size, (void)max_bytes, (void)after, (void)gate, (void)out;
    return (int)hipErrorNotSupported;
  }
  // Whether the gate's last copy is on the copy engines (its dependencies were met and it was
  // issued) and has not finished: the link, not the work it waits for, holds the gate.
  virtual bool link_busy(int gate) = 0;
  // Time copies by the DMA engine's own start and end stamps instead of the host clock at
  // issue and completion. False if the transport cannot (it keeps the host clock).
  virtual bool use_dma_timestamps() { return false; }
  virtual void stats(LinkStats* out) = 0;
  virtual void reset_stats() = 0;
  virtual const char* name() const = 0;
};

// `status`/`err` receive the failure when a factory returns null.
std::unique_ptr<Link> make_sdma_link(int device, uint32_t d2h_engine, uint32_t h2d_engine, std::string& err,
                                     int* status);
// `alias` maps a pinned host pointer to its device-visible address for the copy kernel.
std::unique_ptr<Link> make_stream_link(int device, uint32_t copy_blocks, bool timing, char* (*alias)(void*, char*),
                                       void* alias_ctx, std::string& err, int* status);
// SDMA copies through HIP streams (StreamLink, DMA method); split_d2h: D2H copies of 2 MiB or
// more go out as two halves on two streams while no H2D is pending.
std::unique_ptr<Link> make_hip_dma_link(int device, bool split_d2h, bool timing, std::string& err, int* status);

}  // namespace mo
