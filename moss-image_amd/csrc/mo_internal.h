// Host-side declarations shared by the launchers (mo_launch.cpp) and the engine (mo_engine.cpp).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <string>

#include "mo_kdesc.h"
#include "mo_layout.h"
#include "mo_wire.h"

namespace mo {

int make_kdesc(const Canon& c, uint64_t tensor_base, uint64_t first, uint64_t nbytes, uint64_t payload,
               KDesc& kd, std::string& err);

// Optional observer of kernel launches: supplies the HIP events a launch records its own
// start and end into (the timestamps of the dispatch itself, the same interval a kernel trace
// reports), and is told the payload bytes of each timed launch.
class LaunchTimer {
 public:
  virtual ~LaunchTimer() = default;
  // *start/*stop stay null when the next launch is not timed.
  virtual int events(hipEvent_t* start, hipEvent_t* stop) = 0;
  // bytes: payload bytes of the launch; hbm: device-memory bytes it reads and writes
  virtual void launched(uint64_t bytes, uint64_t hbm) = 0;
};

// Accumulates pieces and launches the pack (or unpack) kernel in batches of kMaxDesc.
class Launcher {
 public:
  Launcher(bool pack, hipStream_t stream, LaunchTimer* timer = nullptr);
  void add(const KDesc& kd);
  int flush();
  int status() const { return status_; }
  uint64_t launches() const { return launches_; }
  uint64_t bytes() const { return bytes_; }
  bool full() const { return args_.ndesc == (uint32_t)kMaxDesc; }  // the next add launches

 private:
  bool pack_;
  hipStream_t stream_;
  LaunchTimer* timer_;
  LaunchArgs args_;
  uint32_t tiles_ = 0;
  int status_ = 0;
  uint64_t launches_ = 0;
  uint64_t bytes_ = 0;          // all bytes added
  uint64_t pending_bytes_ = 0;  // bytes of the batch not launched yet
  uint64_t pending_hbm_ = 0;    // device-memory bytes the batch reads and writes
  bool has_elem_ = false;       // the pending batch holds an ELEM piece (LDS-staged kernel)
};

int launch_link_copy(void* dst, const void* src, uint64_t bytes, uint32_t blocks, hipStream_t stream);

// Device address and size of the current device's mo_noalloc_scratch (loads the code object on
// first use on the device).
int noalloc_scratch(uint64_t* ptr, uint64_t* bytes);

// mo_equal_kernel over nbytes at a and b (16-byte aligned); writes 1 to *flag on a difference.
int launch_equal(const void* a, const void* b, uint64_t nbytes, uint32_t* flag, hipStream_t stream);

// Wire coding of a segment (format and sizes in mo_wire.h). wire_encode codes `raw_bytes` at
// `raw` into `wire` (capacity at least wire_capacity(raw_bytes)) with three launches on
// `stream`, and also writes the coded size to pinned host memory at `host_total` (0: not).
// wire_decode restores the raw bytes from a coded stream of at most `wire_bytes`. Both buffers
// 16-byte aligned (wire_check).
// At most 512 MiB: the coder addresses the wire buffer, about 2.1x the raw bytes with its working
// space, through 32-bit buffer offsets.
constexpr uint64_t kWireMaxRaw = 1ull << 29;
int wire_check(uint64_t raw, uint64_t raw_bytes, uint64_t wire, uint64_t wire_bytes, std::string& err);
int wire_encode(uint64_t raw, uint64_t raw_bytes, uint64_t wire, uint64_t capacity, uint64_t host_total,
                hipStream_t stream);
int wire_decode(uint64_t wire, uint64_t wire_bytes, uint64_t raw, uint64_t raw_bytes, hipStream_t stream);

}  // namespace mo
