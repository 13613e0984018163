// Kernel-argument structures shared by the device code (mo_device.hip) and the host launchers.
// Plain data only: no HIP headers, so the host side compiles with any C++17 compiler.
#pragma once

#include <stdint.h>

#include "../../include/moss_offload.h"

namespace mo {

constexpr int kThreads = 256;                 // lanes per workgroup (4 wave64)
constexpr int kUnroll = 4;                    // 16-byte transfers in flight per lane
constexpr uint32_t kTileBytes = kThreads * kUnroll * 16;  // 16 KiB of payload per workgroup
constexpr int kMaxOuter = MO_MAX_DIMS - 1;    // canonical dims beyond the innermost run
constexpr int kMaxDesc = 16;                  // pieces per launch (kernel-argument budget)
constexpr uint32_t kMaxTilesPerLaunch = 1u << 22;
constexpr int kLinkUnroll = 8;                // 16-byte transfers in flight per lane (link copy)
// Device scratch of mo_pack_to_host (the entry point that allocates nothing): a payload gathered
// there waits for its DMA to the caller's pinned host buffer. One array per device, part of the
// code object, so it is reserved when the code object is loaded and kept until the process ends.
constexpr uint64_t kNoAllocScratchBytes = 64ull << 20;

// NARROW: contiguous float32 on the tensor side, its high halves (bfloat16 bits) as the
// payload; `first` and `nbytes` count payload bytes, the tensor side is twice that.
enum : uint8_t { kPathContig = 0, kPathRuns = 1, kPathElem = 2, kPathNarrow = 3 };

// Cache policy of a piece (KDesc::cache): non-temporal loads of the side read (the tensor when
// packing, the payload when unpacking) and non-temporal stores of the side written. Streaming
// accesses do not allocate in the GPU caches, which suits bytes that are read or written once.
enum : uint8_t { kCacheNtLoad = 1, kCacheNtStore = 2 };

struct KFastDiv {
  uint32_t d, m, s;
};

// One piece: a byte range of one tensor's storage-order payload.
struct KDesc {
  uint64_t tensor;        // tensor-side base address (element (0,...,0))
  uint64_t payload;       // payload-side address of the piece's first byte
  uint64_t first;         // piece start in path units: bytes | 16-B chunks | elements
  uint64_t nbytes;        // piece length in bytes
  uint64_t inner_stride;  // bytes between consecutive units of the innermost run
  uint32_t tile0;         // first tile of this piece within the launch
  uint8_t path;
  uint8_t eb;
  uint8_t nouter;
  uint8_t cache;          // kCache* bits for the CONTIG and NARROW paths
  KFastDiv inner;               // units per innermost run
  KFastDiv outer[kMaxOuter];    // sizes of the outer dims, innermost first
  uint64_t ostride[kMaxOuter];  // byte strides of the outer dims
};

struct LaunchArgs {
  uint32_t ndesc;
  uint32_t pad;
  // d[i].tile0 for i < ndesc, UINT32_MAX after: contiguous, so a workgroup finds its piece with
  // one 64-byte scalar load instead of a chain of dependent loads over the descriptors
  uint32_t tile0[kMaxDesc];
  KDesc d[kMaxDesc];
};
static_assert(sizeof(LaunchArgs) <= 4096, "kernel arguments must fit in 4 KiB");

}  // namespace mo
