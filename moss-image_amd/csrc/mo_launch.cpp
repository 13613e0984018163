// Host side of the kernels: piece -> kernel descriptor, batched launches, and the loader of
// the embedded gfx950 code object (mo_device.hip compiled with hipcc --genco).
//
// The device code is loaded with hipModuleLoadData on first use on each device and its
// kernels are launched with hipModuleLaunchKernel. The library therefore registers no fat
// binary with the HIP runtime at load time and unregisters none at process exit; the runtime
// shared with the host application (torch's) owns the module like any other.
#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <string>

#include "mo_internal.h"

extern "C" const unsigned char mo_device_code[];
extern "C" const uint64_t mo_device_code_size;

// Exported by libamdhip64 (declared in hip/hip_ext.h, which only hipcc can parse): a module
// launch that records its own dispatch start and end into two HIP events. Grid sizes are in
// work-items.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ,
                                               size_t sharedMemBytes, hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent, hipEvent_t stopEvent,
                                               uint32_t flags);

namespace mo {

namespace {

struct DeviceModule {
  hipModule_t module = nullptr;
  hipFunction_t pack = nullptr, unpack = nullptr, link = nullptr;
  hipFunction_t pack1 = nullptr, unpack1 = nullptr;  // single-piece launches
  // the same four with ELEM pieces in the launch (they reserve the LDS staging buffer)
  hipFunction_t pack_elem = nullptr, unpack_elem = nullptr, pack1_elem = nullptr, unpack1_elem = nullptr;
  hipFunction_t equal = nullptr;
  hipFunction_t wire_sizes = nullptr, wire_scan = nullptr, wire_encode = nullptr, wire_decode = nullptr;
  // this device's copy of mo_noalloc_scratch (every device holds its own, at its own address)
  uint64_t scratch = 0, scratch_bytes = 0;
};

std::mutex g_modules_mu;
std::map<int, DeviceModule> g_modules;

int load_functions(DeviceModule& m) {
  hipError_t e = hipModuleLoadData(&m.module, mo_device_code);
  if (e != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.pack, m.module, "mo_pack_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.unpack, m.module, "mo_unpack_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.link, m.module, "mo_link_copy_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.pack1, m.module, "mo_pack1_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.unpack1, m.module, "mo_unpack1_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.pack_elem, m.module, "mo_pack_elem_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.unpack_elem, m.module, "mo_unpack_elem_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.pack1_elem, m.module, "mo_pack1_elem_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.unpack1_elem, m.module, "mo_unpack1_elem_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.equal, m.module, "mo_equal_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.wire_sizes, m.module, "mo_wire_sizes_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.wire_scan, m.module, "mo_wire_scan_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.wire_encode, m.module, "mo_wire_encode_kernel")) != hipSuccess) return (int)e;
  if ((e = hipModuleGetFunction(&m.wire_decode, m.module, "mo_wire_decode_kernel")) != hipSuccess) return (int)e;
  // Set-up of the allocation-free entry point, once per device with that device current: the
  // device address of this module's scratch array. From here on only this address is used.
  hipDeviceptr_t scratch = nullptr;
  size_t bytes = 0;
  if ((e = hipModuleGetGlobal(&scratch, &bytes, m.module, "mo_noalloc_scratch")) != hipSuccess) return (int)e;
  if (!scratch || bytes != kNoAllocScratchBytes || (uint64_t)scratch % 256) return (int)hipErrorInvalidSymbol;
  m.scratch = (uint64_t)scratch;
  m.scratch_bytes = bytes;
  return 0;
}

}  // namespace

// Kernels of the current device, loading the code object on first use.
static int module_of_device(DeviceModule* out) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lock(g_modules_mu);
  auto it = g_modules.find(device);
  if (it == g_modules.end()) {
    DeviceModule m;
    if (int rc = load_functions(m)) return rc;
    it = g_modules.emplace(device, m).first;
  }
  *out = it->second;
  return 0;
}

// The current device's scratch of mo_pack_to_host (its code object loaded on first use).
int noalloc_scratch(uint64_t* ptr, uint64_t* bytes) {
  DeviceModule m;
  if (int rc = module_of_device(&m)) return rc;
  *ptr = m.scratch;
  *bytes = m.scratch_bytes;
  return 0;
}

static int kernels(hipFunction_t* pack, hipFunction_t* unpack, hipFunction_t* link) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lock(g_modules_mu);
  auto it = g_modules.find(device);
  if (it == g_modules.end()) {
    DeviceModule m;
    if (int rc = load_functions(m)) return rc;
    it = g_modules.emplace(device, m).first;
  }
  if (pack) *pack = it->second.pack;
  if (unpack) *unpack = it->second.unpack;
  if (link) *link = it->second.link;
  return 0;
}

// ------------------------------------------------------------------------------------------
// piece -> kernel descriptor

int make_kdesc(const Canon& c, uint64_t tensor_base, uint64_t first, uint64_t nbytes, uint64_t payload,
               KDesc& kd, std::string& err) {
  kd = KDesc();
  kd.tensor = tensor_base;
  kd.payload = payload;
  kd.nbytes = nbytes;
  kd.eb = (uint8_t)c.eb;
  kd.inner = KFastDiv{1, 1, 0};
  if (payload % 16 != 0 || first % 16 != 0) {
    err = "piece payload and offset must be 16-byte aligned";
    return MO_E_INVALID;
  }
  // Canonical dims, innermost last. A unit-stride innermost dim is a contiguous run.
  const int nd = c.nd;
  const bool inner_contig = nd == 0 || (uint64_t)c.stride[nd - 1] == c.eb;
  const uint64_t run_bytes = nd == 0 ? c.eb : (inner_contig ? (uint64_t)c.size[nd - 1] * c.eb : c.eb);
  const int nouter = inner_contig ? (nd > 0 ? nd - 1 : 0) : nd;  // dims outside the run
  if (c.bf16_high) {
    // canonicalize admits only contiguous tensors with this flag
    if (nouter != 0 || tensor_base % 16 != 0) {
      err = "a bf16-high tensor must be contiguous and 16-byte aligned";
      return MO_E_INVALID;
    }
    kd.path = kPathNarrow;
    kd.first = first;
    return 0;
  }
  if (nouter == 0 && tensor_base % 16 == 0) {
    kd.path = kPathContig;
    kd.first = first;
    return 0;
  }
  bool runs16 = run_bytes % 16 == 0 && tensor_base % 16 == 0 && nouter <= kMaxOuter;
  for (int k = 0; k < nouter && runs16; ++k) runs16 = c.stride[k] % 16 == 0;
  if (runs16) {
    const uint64_t run_chunks = run_bytes / 16;
    const uint64_t total_chunks = c.nbytes / 16;
    if (run_chunks >= (1ull << 32) || total_chunks >= (1ull << 32)) {
      err = "tensor too large for 32-bit chunk indexing";
      return MO_E_INVALID;
    }
    kd.path = kPathRuns;
    kd.first = first / 16;
    const FastDiv f = make_fastdiv((uint32_t)run_chunks);
    kd.inner = KFastDiv{f.d, f.m, f.s};
    kd.inner_stride = 16;
    kd.nouter = (uint8_t)nouter;
    for (int k = 0; k < nouter; ++k) {  // kernel order: innermost outer dim first
      const int dim = nouter - 1 - k;
      const FastDiv g = make_fastdiv((uint32_t)c.size[dim]);
      kd.outer[k] = KFastDiv{g.d, g.m, g.s};
      kd.ostride[k] = (uint64_t)c.stride[dim];
    }
    return 0;
  }
  // ELEM path: units are elements; the innermost canonical dim is the inner run.
  if (c.numel >= (1ull << 32)) {
    err = "tensor too large for 32-bit element indexing";
    return MO_E_INVALID;
  }
  const int eouter = nd > 0 ? nd - 1 : 0;
  kd.path = kPathElem;
  kd.first = first / c.eb;
  if (nd == 0) {
    kd.inner_stride = c.eb;
    return 0;
  }
  const FastDiv f = make_fastdiv((uint32_t)c.size[nd - 1]);
  kd.inner = KFastDiv{f.d, f.m, f.s};
  kd.inner_stride = (uint64_t)c.stride[nd - 1];
  kd.nouter = (uint8_t)eouter;
  for (int k = 0; k < eouter; ++k) {
    const int dim = eouter - 1 - k;
    const FastDiv g = make_fastdiv((uint32_t)c.size[dim]);
    kd.outer[k] = KFastDiv{g.d, g.m, g.s};
    kd.ostride[k] = (uint64_t)c.stride[dim];
  }
  return 0;
}

// ------------------------------------------------------------------------------------------
// batched launches

Launcher::Launcher(bool pack, hipStream_t stream, LaunchTimer* timer) : pack_(pack), stream_(stream), timer_(timer) {
  args_.ndesc = 0;
  args_.pad = 0;
  for (auto& t : args_.tile0) t = UINT32_MAX;
}

void Launcher::add(const KDesc& kd) {
  if (kd.nbytes == 0) return;
  if (args_.ndesc == (uint32_t)kMaxDesc) flush();
  KDesc& slot = args_.d[args_.ndesc];
  slot = kd;
  slot.tile0 = tiles_;
  args_.tile0[args_.ndesc] = tiles_;
  const uint64_t t = (kd.nbytes + kTileBytes - 1) / kTileBytes;
  tiles_ += (uint32_t)t;
  bytes_ += kd.nbytes;
  pending_bytes_ += kd.nbytes;
  pending_hbm_ += kd.nbytes * (kd.path == kPathNarrow ? 3 : 2);  // narrow: 2 B tensor-side per payload B
  has_elem_ = has_elem_ || kd.path == kPathElem;
  args_.ndesc++;
  if (tiles_ > kMaxTilesPerLaunch) flush();
}

int Launcher::flush() {
  if (args_.ndesc == 0) return 0;
  hipFunction_t fn = nullptr;
  const bool single = args_.ndesc == 1;  // tile0 == 0: the single-descriptor kernel
  if (status_ == 0) {
    DeviceModule m;
    status_ = module_of_device(&m);
    if (has_elem_) fn = single ? (pack_ ? m.pack1_elem : m.unpack1_elem) : (pack_ ? m.pack_elem : m.unpack_elem);
    else fn = single ? (pack_ ? m.pack1 : m.unpack1) : (pack_ ? m.pack : m.unpack);
  }
  hipEvent_t t0 = nullptr, t1 = nullptr;
  if (status_ == 0 && timer_) status_ = timer_->events(&t0, &t1);
  if (status_ == 0) {
    void* params[] = {single ? (void*)&args_.d[0] : (void*)&args_};
    // The extended launch takes the grid in work-items (tiles_ <= kMaxTilesPerLaunch + kMaxDesc,
    // so tiles_ * kThreads stays far below 2^32).
    const hipError_t e = t0 ? hipExtModuleLaunchKernel(fn, tiles_ * kThreads, 1, 1, kThreads, 1, 1, 0, stream_,
                                                       params, nullptr, t0, t1, 0)
                            : hipModuleLaunchKernel(fn, tiles_, 1, 1, kThreads, 1, 1, 0, stream_, params, nullptr);
    if (e != hipSuccess) status_ = (int)e;
    launches_++;
    if (e == hipSuccess && t0) timer_->launched(pending_bytes_, pending_hbm_);
  }
  for (uint32_t k = 0; k < args_.ndesc; ++k) args_.tile0[k] = UINT32_MAX;
  args_.ndesc = 0;
  tiles_ = 0;
  pending_bytes_ = 0;
  pending_hbm_ = 0;
  has_elem_ = false;
  return status_;
}

int launch_link_copy(void* dst, const void* src, uint64_t bytes, uint32_t blocks, hipStream_t stream) {
  if (bytes == 0) return 0;
  if (blocks == 0) blocks = 64;
  const uint64_t max_blocks = (bytes / 16 + kThreads - 1) / kThreads;
  if (blocks > max_blocks) blocks = (uint32_t)(max_blocks ? max_blocks : 1);
  hipFunction_t fn = nullptr;
  if (int rc = kernels(nullptr, nullptr, &fn)) return rc;
  void* d = dst;
  const void* s = src;
  uint64_t n = bytes;
  void* params[] = {&d, &s, &n};
  return (int)hipModuleLaunchKernel(fn, blocks, 1, 1, kThreads, 1, 1, 0, stream, params, nullptr);
}

int launch_equal(const void* a, const void* b, uint64_t nbytes, uint32_t* flag, hipStream_t stream) {
  if (nbytes == 0) return 0;
  const uint64_t tiles = (nbytes + kTileBytes - 1) / kTileBytes;
  if (tiles * kThreads > UINT32_MAX) return (int)hipErrorInvalidValue;
  DeviceModule m;
  if (int rc = module_of_device(&m)) return rc;
  const void* x = a;
  const void* y = b;
  uint64_t n = nbytes;
  uint32_t* f = flag;
  void* params[] = {&x, &y, &n, &f};
  return (int)hipModuleLaunchKernel(m.equal, (uint32_t)tiles, 1, 1, kThreads, 1, 1, 0, stream, params, nullptr);
}

// Wire coding (mo_wire.h). The caller checks sizes and alignment (wire_check).
int wire_check(uint64_t raw, uint64_t raw_bytes, uint64_t wire, uint64_t wire_bytes, std::string& err) {
  if (raw_bytes > kWireMaxRaw) {
    err = "segment too large for wire coding (at most " + std::to_string(kWireMaxRaw) + " bytes)";
    return MO_E_INVALID;
  }
  if ((raw % 16) || (wire % 16)) {
    err = "wire coding needs 16-byte aligned buffers";
    return MO_E_INVALID;
  }
  if ((raw_bytes && !raw) || !wire) {
    err = "null buffer";
    return MO_E_INVALID;
  }
  (void)wire_bytes;
  return 0;
}

int wire_encode(uint64_t raw, uint64_t raw_bytes, uint64_t wire, uint64_t capacity, uint64_t host_total,
                hipStream_t stream) {
  DeviceModule m;
  if (int rc = module_of_device(&m)) return rc;
  const uint64_t tiles = wire_tiles(raw_bytes);
  const uint32_t groups = (uint32_t)((tiles + kWireTilesPerGroup - 1) / kWireTilesPerGroup);  // one wave per tile
  const void* r = (const void*)raw;
  void* w = (void*)wire;
  uint64_t n = raw_bytes, cap = capacity;
  void* ht = (void*)host_total;
  hipError_t e;
  if (tiles) {
    void* params[] = {&r, &n, &w, &cap};
    if ((e = hipModuleLaunchKernel(m.wire_sizes, groups, 1, 1, kThreads, 1, 1, 0, stream, params, nullptr)) !=
        hipSuccess)
      return (int)e;
  }
  {
    void* params[] = {&r, &n, &w, &cap, &ht};
    if ((e = hipModuleLaunchKernel(m.wire_scan, 1, 1, 1, kWireScanThreads, 1, 1, 0, stream, params, nullptr)) !=
        hipSuccess)
      return (int)e;
  }
  if (tiles) {
    void* params[] = {&r, &n, &w, &cap};
    if ((e = hipModuleLaunchKernel(m.wire_encode, groups, 1, 1, kThreads, 1, 1, 0, stream, params,
                                   nullptr)) != hipSuccess)
      return (int)e;
  }
  return 0;
}

int wire_decode(uint64_t wire, uint64_t wire_bytes, uint64_t raw, uint64_t raw_bytes, hipStream_t stream) {
  DeviceModule m;
  if (int rc = module_of_device(&m)) return rc;
  const uint64_t tiles = wire_tiles(raw_bytes);
  const void* w = (const void*)wire;
  void* r = (void*)raw;
  uint64_t wb = wire_bytes, n = raw_bytes;
  void* params[] = {&w, &wb, &n, &r};
  const uint32_t groups = (uint32_t)((tiles + kWireTilesPerGroup - 1) / kWireTilesPerGroup);  // one wave per tile
  return (int)hipModuleLaunchKernel(m.wire_decode, groups ? groups : 1, 1, 1, kThreads, 1, 1, 0, stream,
                                    params, nullptr);
}

}  // namespace mo
