// Frozen-block streaming: the native side of moss_offload.memory.AsyncBlockStreamer.
//
// Replaces what training/memory.py does on its copy stream (AsyncBlockStreamer._stage,
// memory.py:157-191, and the ready/reusable events of :193-225, :246-247): the frozen
// parameters and buffers of one block live in one pinned host master, and a fill copies it
// into a device staging slot. Here the copy runs on an SDMA engine (no compute units, no
// interference with the step's GEMMs), ordered like the activation engine's copies:
//   release -> fill : the issuer thread holds the fill until the HIP event recorded at the
//                     slot's last release has completed (the slot's previous contents are no
//                     longer read by the GPU);
//   fill -> acquire : the host waits for the fill's completion before it enqueues the
//                     kernels that read the slot;
//   release -> write-back -> fill : a slot whose contents were updated on the device (the
//                     trainable ring, training/trainable_offload.py:245-260) is copied back to its
//                     master after the release point, and the slot's next fill waits for that
//                     copy.
// No GPU queue waits on host memory, and every wait is bounded.
#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/moss_offload.h"
#include "mo_internal.h"
#include "mo_link.h"

namespace mo {
// Defined in mo_engine.cpp: thread-local error message and its setters.
int set_error(int code, const std::string& msg);
int set_hip_error(int e, const char* what);
}  // namespace mo

struct mo_streamer {
  std::mutex mu;
  int device = 0;
  std::unique_ptr<mo::Link> link;
  std::vector<int> gates;        // one per slot
  std::vector<mo::CopyRef> pending_writeback;  // per slot: the next fill waits for it
  uint64_t fills = 0, bytes = 0, writebacks = 0, writeback_bytes = 0;
};

namespace {

class StreamerDevice {
 public:
  explicit StreamerDevice(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != device) (void)hipSetDevice(device);
    dev_ = device;
  }
  ~StreamerDevice() {
    if (prev_ >= 0 && prev_ != dev_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = -1, dev_ = -1;
};

// Runs `body` (a braced block returning int) under the streamer's mutex with its device
// current; no C++ exception leaves the C ABI.
#define MO_STREAMER_CALL(s, body)                                                     \
  if (!(s)) return mo::set_error(MO_E_INVALID, "null streamer");                      \
  try {                                                                               \
    std::lock_guard<std::mutex> lock((s)->mu);                                        \
    StreamerDevice guard((s)->device);                                                \
    return [&]() -> int body();                                                       \
  } catch (const std::exception& ex) {                                                \
    return mo::set_error(MO_E_STATE, std::string("internal error: ") + ex.what());    \
  } catch (...) {                                                                     \
    return mo::set_error(MO_E_STATE, "internal error");                               \
  }

int check_slot(mo_streamer* s, uint32_t slot) {
  if (slot >= s->gates.size())
    return mo::set_error(MO_E_INVALID, "slot " + std::to_string(slot) + " out of range (" +
                                           std::to_string(s->gates.size()) + " slots)");
  return 0;
}

}  // namespace

extern "C" {

int mo_pinned_alloc(uint64_t bytes, uint64_t* host) {
  if (!host) return mo::set_error(MO_E_INVALID, "null output");
  *host = 0;
  const uint64_t size = ((bytes ? bytes : 1) + 4095) & ~4095ull;
  void* p = nullptr;
  const hipError_t e = hipHostMalloc(&p, size, hipHostMallocDefault);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "hipHostMalloc (pinned block master)");
  *host = (uint64_t)p;
  return 0;
}

int mo_pinned_free(uint64_t host) {
  if (!host) return 0;
  const hipError_t e = hipHostFree((void*)host);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "hipHostFree (pinned block master)");
  return 0;
}

int mo_streamer_create(int device, uint32_t slots, uint32_t h2d_engine, mo_streamer** out) {
  if (!out) return mo::set_error(MO_E_INVALID, "null output");
  *out = nullptr;
  if (slots == 0 || slots > 64) return mo::set_error(MO_E_INVALID, "slots must be 1..64");
  try {
    auto s = std::make_unique<mo_streamer>();
    s->device = device;
    StreamerDevice guard(device);
    std::string err;
    int status = 0;
    s->link = mo::make_sdma_link(device, 0, h2d_engine, err, &status);
    if (!s->link) return mo::set_error(status ? status : MO_E_STATE, "SDMA link: " + err);
    for (uint32_t i = 0; i < slots; ++i) {
      int g = 0;
      if (int rc = s->link->new_gate(&g)) return mo::set_hip_error(rc, "slot gate");
      s->gates.push_back(g);
    }
    s->pending_writeback.resize(slots);
    *out = s.release();
    return 0;
  } catch (const std::exception& ex) {
    return mo::set_error(MO_E_STATE, std::string("internal error: ") + ex.what());
  }
}

int mo_streamer_destroy(mo_streamer* s) {
  if (!s) return 0;
  int rc = 0;
  {
    std::lock_guard<std::mutex> lock(s->mu);
    StreamerDevice guard(s->device);
    if (s->link) rc = s->link->synchronize();
    s->link.reset();
  }
  delete s;
  return rc ? mo::set_error(MO_E_STATE, "streamer copies did not finish in time") : 0;
}

int mo_streamer_fill(mo_streamer* s, uint32_t slot, uint64_t dst, uint64_t src, uint64_t bytes) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    if (!dst || !src) return mo::set_error(MO_E_INVALID, "null fill address");
    if (bytes == 0) return 0;
    mo::CopyRef copy;
    if (int rc = s->link->h2d((void*)dst, (const void*)src, bytes, s->pending_writeback[slot], s->gates[slot], &copy))
      return mo::set_hip_error(rc, "slot fill (SDMA H2D)");
    s->pending_writeback[slot].reset();
    s->fills++;
    s->bytes += bytes;
    return 0;
  });
}

int mo_streamer_writeback(mo_streamer* s, uint32_t slot, uint64_t dst, uint64_t src, uint64_t bytes) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    if (!dst || !src) return mo::set_error(MO_E_INVALID, "null write-back address");
    if (bytes == 0) return 0;
    mo::CopyRef copy;
    if (int rc = s->link->writeback((void*)dst, (const void*)src, bytes, s->gates[slot], &copy))
      return mo::set_hip_error(rc, "slot write-back (SDMA D2H)");
    s->pending_writeback[slot] = std::move(copy);
    s->writebacks++;
    s->writeback_bytes += bytes;
    return 0;
  });
}

int mo_streamer_acquire(mo_streamer* s, uint32_t slot, uint64_t stream) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    if (int rc = s->link->wait(s->gates[slot], (hipStream_t)stream))
      return mo::set_error(rc, "slot fill failed or did not finish in time");
    return 0;
  });
}

int mo_streamer_release(mo_streamer* s, uint32_t slot, uint64_t stream) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    if (int rc = s->link->consumed(s->gates[slot], (hipStream_t)stream)) return mo::set_hip_error(rc, "slot release");
    return 0;
  });
}

int mo_streamer_synchronize(mo_streamer* s) {
  MO_STREAMER_CALL(s, {
    if (s->link->synchronize()) return mo::set_error(MO_E_STATE, "streamer copies did not finish in time");
    return 0;
  });
}

int mo_streamer_get_stats(mo_streamer* s, mo_streamer_stats* out) {
  MO_STREAMER_CALL(s, {
    if (!out) return mo::set_error(MO_E_INVALID, "null output");
    mo::LinkStats ls;
    s->link->stats(&ls);
    *out = mo_streamer_stats{};
    out->fills = s->fills;
    out->bytes = s->bytes;
    out->timed_bytes = ls.h2d_done_bytes;
    out->busy_ms = ls.h2d_ms;
    out->writebacks = s->writebacks;
    out->writeback_bytes = s->writeback_bytes;
    out->timed_writeback_bytes = ls.d2h_done_bytes;
    out->writeback_busy_ms = ls.d2h_ms;
    out->host_blocks = ls.host_blocks;
    out->host_block_ms = ls.host_block_ms;
    out->copy_failures = ls.failures;
    return 0;
  });
}

int mo_streamer_reset_stats(mo_streamer* s) {
  MO_STREAMER_CALL(s, {
    s->link->reset_stats();
    s->fills = s->bytes = s->writebacks = s->writeback_bytes = 0;
    return 0;
  });
}

}  // extern "C"
