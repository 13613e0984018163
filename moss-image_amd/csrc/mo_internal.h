// Internal declarations shared by the kernels (mo_kernels.hip) and the engine (mo_engine.cpp).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "mo_layout.h"

namespace mo {

constexpr int kThreads = 256;                 // lanes per workgroup (4 wave64)
constexpr int kUnroll = 4;                    // 16-byte transfers in flight per lane
constexpr uint32_t kTileBytes = kThreads * kUnroll * 16;  // 16 KiB of payload per workgroup
constexpr int kMaxOuter = MO_MAX_DIMS - 1;    // canonical dims beyond the innermost run
constexpr int kMaxDesc = 16;                  // pieces per launch (kernel-argument budget)
constexpr uint32_t kMaxTilesPerLaunch = 1u << 22;

enum : uint8_t { kPathContig = 0, kPathRuns = 1, kPathElem = 2 };

struct KFastDiv {
  uint32_t d, m, s;
};

// One piece: a byte range of one tensor's storage-order payload.
struct KDesc {
  uint64_t tensor = 0;        // tensor-side base address (element (0,...,0))
  uint64_t payload = 0;       // payload-side address of the piece's first byte
  uint64_t first = 0;         // piece start in path units: bytes | 16-B chunks | elements
  uint64_t nbytes = 0;        // piece length in bytes
  uint64_t inner_stride = 0;  // bytes between consecutive units of the innermost run
  uint32_t tile0 = 0;         // first tile of this piece within the launch
  uint8_t path = 0;
  uint8_t eb = 0;
  uint8_t nouter = 0;
  uint8_t pad = 0;
  KFastDiv inner{1, 1, 0};    // units per innermost run
  KFastDiv outer[kMaxOuter]{};  // sizes of the outer dims, innermost first
  uint64_t ostride[kMaxOuter]{};  // byte strides of the outer dims
};

struct LaunchArgs {
  uint32_t ndesc = 0;
  uint32_t pad = 0;
  KDesc d[kMaxDesc];
};
static_assert(sizeof(LaunchArgs) <= 4096, "kernel arguments must fit in 4 KiB");

int make_kdesc(const Canon& c, uint64_t tensor_base, uint64_t first, uint64_t nbytes, uint64_t payload,
               KDesc& kd, std::string& err);

// Optional observer that brackets each kernel launch (e.g. with timing events).
class LaunchTimer {
 public:
  virtual ~LaunchTimer() = default;
  virtual int before(hipStream_t stream) = 0;
  virtual int after(hipStream_t stream, uint64_t bytes) = 0;
};

// Accumulates pieces and launches the pack (or unpack) kernel in batches of kMaxDesc.
class Launcher {
 public:
  Launcher(bool pack, hipStream_t stream, LaunchTimer* timer = nullptr)
      : pack_(pack), stream_(stream), timer_(timer) {}
  void add(const KDesc& kd);
  int flush();
  int status() const { return status_; }
  uint64_t launches() const { return launches_; }
  uint64_t bytes() const { return bytes_; }

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
};

int launch_link_copy(void* dst, const void* src, uint64_t bytes, uint32_t blocks, hipStream_t stream);

}  // namespace mo
