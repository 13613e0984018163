// Block streaming: the native side of moss_offload.memory.AsyncBlockStreamer (frozen blocks)
// and moss_offload.trainable_offload.TrainableBlockStreamer (blocks updated in place).
//
// The ring (mo_streamer_stage .. mo_streamer_slot_info) decides residency: which block each
// device slot holds, how many running executions still read it (pins), whether it was written
// on the device since its fill (dirty: copied back to its master before the slot is reused), and
// which slot a new block replaces (an empty one, else the least recently staged that is neither
// pinned nor kept for the block about to run beside it). Python only asks for a block and gets
// a slot and its fill generation, which every later call on that slot must present.
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

// Residency of one device slot in the block ring (mo_streamer_stage and the calls after it).
struct RingSlot {
  uint64_t dev = 0, capacity = 0;  // the caller's device buffer (mo_streamer_attach)
  int64_t block = -1;              // block held, -1 = none
  uint64_t host = 0, bytes = 0;    // that block's pinned master
  uint32_t pins = 0;               // executions still reading the slot
  bool dirty = false;              // written on the device since its fill
  uint64_t generation = 0;         // bumped by every fill
  uint64_t last_use = 0;           // tick of the last stage that returned this slot
};

struct mo_streamer {
  std::mutex mu;
  int device = 0;
  std::unique_ptr<mo::Link> link;
  std::vector<int> gates;        // one per slot
  std::vector<mo::CopyRef> pending_writeback;  // per slot: the next fill waits for it
  std::vector<RingSlot> ring;    // per slot
  uint64_t tick = 0;
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

int issue_fill(mo_streamer* s, uint32_t slot, uint64_t dst, uint64_t src, uint64_t bytes) {
  mo::CopyRef copy;
  if (int rc = s->link->h2d((void*)dst, (const void*)src, bytes, s->pending_writeback[slot], s->gates[slot], &copy))
    return mo::set_hip_error(rc, "slot fill (SDMA H2D)");
  s->pending_writeback[slot].reset();
  s->fills++;
  s->bytes += bytes;
  return 0;
}

int issue_writeback(mo_streamer* s, uint32_t slot, uint64_t dst, uint64_t src, uint64_t bytes) {
  mo::CopyRef copy;
  if (int rc = s->link->writeback((void*)dst, (const void*)src, bytes, s->gates[slot], &copy))
    return mo::set_hip_error(rc, "slot write-back (SDMA D2H)");
  s->pending_writeback[slot] = std::move(copy);
  s->writebacks++;
  s->writeback_bytes += bytes;
  return 0;
}

// The slot's block leaves it: a dirty slot is first copied back to the block's master, after
// the slot's last release point; its next fill is ordered behind that copy.
int vacate(mo_streamer* s, uint32_t k) {
  RingSlot& r = s->ring[k];
  if (r.block >= 0 && r.dirty && r.bytes)
    if (int rc = issue_writeback(s, k, r.host, r.dev, r.bytes)) return rc;
  r.block = -1;
  r.host = r.bytes = 0;
  r.dirty = false;
  r.pins = 0;
  return 0;
}

int check_generation(mo_streamer* s, uint32_t slot, uint64_t generation, const char* what) {
  if (int rc = check_slot(s, slot)) return rc;
  const RingSlot& r = s->ring[slot];
  if (r.block < 0 || r.generation != generation)
    return mo::set_error(MO_E_STATE, std::string(what) + ": slot " + std::to_string(slot) +
                                         " no longer holds the block it held at generation " +
                                         std::to_string(generation));
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
    s->ring.resize(slots);
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
    return issue_fill(s, slot, dst, src, bytes);
  });
}

int mo_streamer_writeback(mo_streamer* s, uint32_t slot, uint64_t dst, uint64_t src, uint64_t bytes) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    if (!dst || !src) return mo::set_error(MO_E_INVALID, "null write-back address");
    if (bytes == 0) return 0;
    return issue_writeback(s, slot, dst, src, bytes);
  });
}

int mo_streamer_attach(mo_streamer* s, uint32_t slot, uint64_t dev, uint64_t capacity) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    RingSlot& r = s->ring[slot];
    if (r.block >= 0) return mo::set_error(MO_E_STATE, "mo_streamer_attach: slot " + std::to_string(slot) + " holds a block");
    r.dev = dev;
    r.capacity = dev ? capacity : 0;
    return 0;
  });
}

int mo_streamer_stage(mo_streamer* s, int64_t block, uint64_t host, uint64_t bytes, int64_t keep, uint32_t* slot,
                      uint64_t* generation, int* filled) {
  MO_STREAMER_CALL(s, {
    if (!slot || !generation || !filled) return mo::set_error(MO_E_INVALID, "null output");
    if (block < 0 || !host) return mo::set_error(MO_E_INVALID, "mo_streamer_stage: bad block or master");
    *filled = 0;
    const uint64_t now = ++s->tick;
    for (uint32_t k = 0; k < s->ring.size(); ++k) {
      RingSlot& r = s->ring[k];
      if (r.block == block) {
        if (r.host != host || r.bytes != bytes)
          return mo::set_error(MO_E_INVALID, "mo_streamer_stage: block " + std::to_string(block) +
                                                 " staged with a different master");
        r.last_use = now;
        *slot = k;
        *generation = r.generation;
        return 0;
      }
    }
    // the victim: an attached slot large enough, not pinned, not holding `keep`; an empty one
    // first, else the one used longest ago
    int best = -1;
    for (uint32_t k = 0; k < s->ring.size(); ++k) {
      const RingSlot& r = s->ring[k];
      if (!r.dev || r.capacity < bytes || r.pins || (keep >= 0 && r.block == keep)) continue;
      if (best < 0) {
        best = (int)k;
        continue;
      }
      const RingSlot& b = s->ring[best];
      const bool empty = r.block < 0;
      const bool bempty = b.block < 0;
      if ((empty && !bempty) || (empty == bempty && r.last_use < b.last_use)) best = (int)k;
    }
    if (best < 0)
      return mo::set_error(MO_E_STATE, "no staging slot can take block " + std::to_string(block) +
                                           ": every slot is in use by a running block or holds the block kept beside it");
    if (int rc = vacate(s, (uint32_t)best)) return rc;
    RingSlot& r = s->ring[best];
    if (bytes)
      if (int rc = issue_fill(s, (uint32_t)best, r.dev, host, bytes)) return rc;
    r.block = block;
    r.host = host;
    r.bytes = bytes;
    r.generation++;
    r.last_use = now;
    *slot = (uint32_t)best;
    *generation = r.generation;
    *filled = 1;
    return 0;
  });
}

int mo_streamer_pin(mo_streamer* s, uint32_t slot, uint64_t generation) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_generation(s, slot, generation, "mo_streamer_pin")) return rc;
    s->ring[slot].pins++;
    return 0;
  });
}

int mo_streamer_unpin(mo_streamer* s, uint32_t slot, uint64_t generation, uint64_t stream) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_generation(s, slot, generation, "mo_streamer_unpin")) return rc;
    RingSlot& r = s->ring[slot];
    if (!r.pins) return mo::set_error(MO_E_STATE, "mo_streamer_unpin: slot " + std::to_string(slot) + " is not pinned");
    if (int rc = s->link->consumed(s->gates[slot], (hipStream_t)stream)) return mo::set_hip_error(rc, "slot release");
    r.pins--;
    return 0;
  });
}

int mo_streamer_mark_dirty(mo_streamer* s, uint32_t slot, uint64_t generation, int dirty) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_generation(s, slot, generation, "mo_streamer_mark_dirty")) return rc;
    s->ring[slot].dirty = dirty != 0;
    return 0;
  });
}

int mo_streamer_evict(mo_streamer* s, uint32_t slot) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    if (s->ring[slot].pins)
      return mo::set_error(MO_E_STATE, "mo_streamer_evict: slot " + std::to_string(slot) + " is in use by a running block");
    return vacate(s, slot);
  });
}

int mo_streamer_slot_info(mo_streamer* s, uint32_t slot, int64_t* block, uint32_t* pins, int* dirty,
                          uint64_t* generation) {
  MO_STREAMER_CALL(s, {
    if (int rc = check_slot(s, slot)) return rc;
    const RingSlot& r = s->ring[slot];
    if (block) *block = r.block;
    if (pins) *pins = r.pins;
    if (dirty) *dirty = r.dirty ? 1 : 0;
    if (generation) *generation = r.generation;
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
