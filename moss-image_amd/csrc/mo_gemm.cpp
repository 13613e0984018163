// Host side of the int8 weight-only GEMMs (csrc/mo_gemm.hip): argument checks, module loading
// from the embedded gfx950 code object, the launch plan. C ABI: mo_int8_linear_forward/backward.
//
// Launch plan: the large tile (256 x 256) carries the work; when its grid would leave the GPU's
// last round of workgroups less than half full, the rows of that partial round go to a second
// launch with the small tile (128 x 128, two workgroups a CU), and a grid smaller than one
// round of large tiles uses the small tile throughout. Every output element is computed by one
// workgroup with the same reduction order in either tile, so the plan does not change results.
#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>

#include "../../include/moss_offload.h"

extern "C" const unsigned char mo_gemm_code[];

namespace mo {
int set_error(int code, const std::string& msg);
int set_hip_error(int e, const char* what);
}  // namespace mo

namespace {

constexpr uint32_t kLarge = 256, kSmall = 128;  // output tile edges (mo_gemm.hip Cfg)

struct Kernel {
  hipFunction_t fn = nullptr;
  uint32_t threads = 0, tile = 0;
};

struct GemmModule {
  hipModule_t module = nullptr;
  int cus = 0;
  // [backward][small][tail]
  Kernel k[2][2][2];
  hipFunction_t decode = nullptr;     // mo_int8_decode_kernel
  hipFunction_t ws_fwd = nullptr;     // mo_int8_ws_fwd: weight in registers, column scales
  hipFunction_t ws_kscale = nullptr;  // mo_int8_ws_kscale: the same on a transposed weight, per-k scales
  hipFunction_t transpose = nullptr;  // mo_int8_transpose_kernel
};

// Which kernel takes the large-tile rows of a launch plan (mo_int8_set_kernel).
std::atomic<uint32_t> g_kernel{MO_INT8_KERNEL_REGISTERS};

std::mutex g_mu;
std::map<int, GemmModule> g_modules;

int gemm_module(GemmModule* out) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_modules.find(device);
  if (it == g_modules.end()) {
    GemmModule m;
    if ((e = hipModuleLoadData(&m.module, mo_gemm_code)) != hipSuccess)
      return mo::set_hip_error((int)e, "hipModuleLoadData (int8 GEMM code object)");
    if ((e = hipDeviceGetAttribute(&m.cus, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess)
      return mo::set_hip_error((int)e, "hipDeviceGetAttribute (CU count)");
    for (int bwd = 0; bwd < 2; ++bwd)
      for (int small = 0; small < 2; ++small)
        for (int tail = 0; tail < 2; ++tail) {
          const std::string name = std::string("mo_int8_linear_") + (bwd ? "bwd" : "fwd") + (small ? "_small" : "_large") +
                                   (tail ? "_tail" : "");
          Kernel& k = m.k[bwd][small][tail];
          if ((e = hipModuleGetFunction(&k.fn, m.module, name.c_str())) != hipSuccess)
            return mo::set_hip_error((int)e, "hipModuleGetFunction (int8 GEMM)");
          k.tile = small ? kSmall : kLarge;
          k.threads = small ? 256 : (bwd ? 256 : 512);  // waves of each configuration x 64
        }
    if ((e = hipModuleGetFunction(&m.decode, m.module, "mo_int8_decode_kernel")) != hipSuccess)
      return mo::set_hip_error((int)e, "hipModuleGetFunction (int8 decode)");
    if ((e = hipModuleGetFunction(&m.ws_fwd, m.module, "mo_int8_ws_fwd")) != hipSuccess ||
        (e = hipModuleGetFunction(&m.ws_kscale, m.module, "mo_int8_ws_kscale")) != hipSuccess ||
        (e = hipModuleGetFunction(&m.transpose, m.module, "mo_int8_transpose_kernel")) != hipSuccess)
      return mo::set_hip_error((int)e, "hipModuleGetFunction (int8 weight-in-registers kernels)");
    it = g_modules.emplace(device, m).first;
  }
  *out = it->second;
  return 0;
}

int check(uint64_t a, uint64_t w, uint64_t scale, uint64_t c, uint32_t rows, uint32_t in_f, uint32_t out_f) {
  if (!a || !w || !scale || !c) return mo::set_error(MO_E_INVALID, "null matrix pointer");
  if (rows == 0 || in_f == 0 || out_f == 0) return mo::set_error(MO_E_INVALID, "empty matrix");
  if (in_f % 16 || out_f % 16)
    return mo::set_error(MO_E_INVALID, "in_features and out_features must be multiples of 16 (got " +
                                           std::to_string(in_f) + ", " + std::to_string(out_f) + ")");
  if ((a | w | c) % 16) return mo::set_error(MO_E_INVALID, "matrix pointers must be 16-byte aligned");
  if (scale % 4) return mo::set_error(MO_E_INVALID, "scale pointer must be 4-byte aligned");
  // 32-bit buffer offsets: one tile's rows of either activation, and the whole weight
  if (in_f > (1u << 20) || out_f > (1u << 20) || (uint64_t)in_f * out_f >= (1ull << 31))
    return mo::set_error(MO_E_INVALID, "weight too large (in_features, out_features <= 2^20 and in * out < 2^31)");
  if ((uint64_t)rows * (out_f > in_f ? out_f : in_f) >= (1ull << 40)) return mo::set_error(MO_E_INVALID, "matrix too large");
  return 0;
}

struct Part {
  bool small;
  uint32_t row0, rows;
};

// Split [0, rows) between the large and the small tile (see the file comment).
int plan(uint32_t rows, uint32_t cols, int cus, Part parts[2]) {
  const uint64_t tm = (rows + kLarge - 1) / kLarge, tc = (cols + kLarge - 1) / kLarge, total = tm * tc;
  const uint64_t rounds = total / (uint64_t)cus, rem = total % (uint64_t)cus;
  if (rounds == 0) {
    parts[0] = {true, 0, rows};
    return 1;
  }
  if (rem == 0 || 2 * rem >= (uint64_t)cus) {
    parts[0] = {false, 0, rows};
    return 1;
  }
  const uint64_t main_rows = (rounds * (uint64_t)cus / tc) * kLarge;
  if (main_rows == 0) {
    parts[0] = {true, 0, rows};
    return 1;
  }
  if (main_rows >= rows) {
    parts[0] = {false, 0, rows};
    return 1;
  }
  parts[0] = {false, 0, (uint32_t)main_rows};
  parts[1] = {true, (uint32_t)main_rows, rows - (uint32_t)main_rows};
  return 2;
}

int launch(const Kernel& k, void** params, uint32_t rows, uint32_t cols, uint64_t stream) {
  const uint64_t tiles_m = (rows + k.tile - 1) / k.tile, tiles_c = (cols + k.tile - 1) / k.tile;
  const uint64_t grid = tiles_m * tiles_c;
  if (grid >= (1ull << 31)) return mo::set_error(MO_E_INVALID, "grid too large");
  const hipError_t e =
      hipModuleLaunchKernel(k.fn, (uint32_t)grid, 1, 1, k.threads, 1, 1, 0, (hipStream_t)stream, params, nullptr);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "int8 GEMM launch");
  return 0;
}

// The weight-in-registers kernels: 256 x 256 tiles, four waves.
Kernel registers_kernel(hipFunction_t fn) { return Kernel{fn, 256, kLarge}; }

}  // namespace

extern "C" {

int mo_int8_decode(uint64_t w, uint64_t scale, uint64_t out, uint32_t out_features, uint32_t in_features,
                   uint64_t stream) {
  if (!w || !scale || !out) return mo::set_error(MO_E_INVALID, "null pointer");
  if (out_features == 0 || in_features == 0) return mo::set_error(MO_E_INVALID, "empty weight");
  if (in_features % 16) return mo::set_error(MO_E_INVALID, "in_features must be a multiple of 16");
  if ((w | out) % 16 || scale % 4) return mo::set_error(MO_E_INVALID, "misaligned pointer");
  if ((uint64_t)in_features * out_features >= (1ull << 31)) return mo::set_error(MO_E_INVALID, "weight too large");
  GemmModule m;
  if (int rc = gemm_module(&m)) return rc;
  const uint64_t chunks = (uint64_t)out_features * (in_features / 16);
  const void* q = (const void*)w;
  const void* sc = (const void*)scale;
  void* o = (void*)out;
  uint32_t rows = out_features, cols = in_features;
  void* params[] = {&q, &sc, &o, &rows, &cols};
  const hipError_t e = hipModuleLaunchKernel(m.decode, (uint32_t)((chunks + 255) / 256), 1, 1, 256, 1, 1, 0,
                                             (hipStream_t)stream, params, nullptr);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "int8 decode launch");
  return 0;
}

int mo_int8_linear_forward(uint64_t x, uint64_t w, uint64_t scale, uint64_t bias, uint64_t y, uint32_t rows,
                           uint32_t in_features, uint32_t out_features, uint64_t stream) {
  if (int rc = check(x, w, scale, y, rows, in_features, out_features)) return rc;
  if (bias % 2) return mo::set_error(MO_E_INVALID, "bias pointer must be 2-byte aligned");
  GemmModule m;
  if (int rc = gemm_module(&m)) return rc;
  Part parts[2];
  const int n = plan(rows, out_features, m.cus, parts);
  const int tail = in_features % 64 != 0;
  const bool registers = !tail && g_kernel.load() == MO_INT8_KERNEL_REGISTERS;
  for (int p = 0; p < n; ++p) {
    const Kernel k = !parts[p].small && registers ? registers_kernel(m.ws_fwd) : m.k[0][parts[p].small][tail];
    const void* A = (const void*)(x + (uint64_t)parts[p].row0 * in_features * 2);
    const void* B = (const void*)w;
    const void* S = (const void*)scale;
    const void* Bi = (const void*)bias;
    void* C = (void*)(y + (uint64_t)parts[p].row0 * out_features * 2);
    int M = (int)parts[p].rows, NC = (int)out_features, R = (int)in_features;
    int tiles_m = (int)((parts[p].rows + k.tile - 1) / k.tile);
    void* params[] = {&A, &B, &S, &Bi, &C, &M, &NC, &R, &tiles_m};
    if (int rc = launch(k, params, parts[p].rows, out_features, stream)) return rc;
  }
  return 0;
}

uint64_t mo_int8_backward_workspace_bytes(uint32_t in_features, uint32_t out_features) {
  return (uint64_t)in_features * out_features;
}

int mo_int8_linear_backward(uint64_t dy, uint64_t w, uint64_t scale, uint64_t dx, uint32_t rows, uint32_t in_features,
                            uint32_t out_features, uint64_t workspace, uint64_t workspace_bytes, uint64_t stream) {
  if (int rc = check(dy, w, scale, dx, rows, in_features, out_features)) return rc;
  if (workspace % 16) return mo::set_error(MO_E_INVALID, "workspace pointer must be 16-byte aligned");
  GemmModule m;
  if (int rc = gemm_module(&m)) return rc;
  Part parts[2];
  const int n = plan(rows, in_features, m.cus, parts);
  const int tail = out_features % 64 != 0;
  const bool registers = !tail && g_kernel.load() == MO_INT8_KERNEL_REGISTERS && workspace &&
                         workspace_bytes >= mo_int8_backward_workspace_bytes(in_features, out_features);
  bool transposed = false;
  for (int p = 0; p < n; ++p) {
    const bool ws = !parts[p].small && registers;
    if (ws && !transposed) {
      // the weight with the reduction (out) contiguous, for the weight-in-registers kernel
      const void* src = (const void*)w;
      void* dst = (void*)workspace;
      uint32_t r = out_features, c = in_features;
      void* tparams[] = {&src, &dst, &r, &c};
      const uint64_t threads = (uint64_t)(out_features / 16) * (in_features / 4);
      const hipError_t e = hipModuleLaunchKernel(m.transpose, (uint32_t)((threads + 255) / 256), 1, 1, 256, 1, 1, 0,
                                                 (hipStream_t)stream, tparams, nullptr);
      if (e != hipSuccess) return mo::set_hip_error((int)e, "int8 transpose launch");
      transposed = true;
    }
    const Kernel k = ws ? registers_kernel(m.ws_kscale) : m.k[1][parts[p].small][tail];
    const void* A = (const void*)(dy + (uint64_t)parts[p].row0 * out_features * 2);
    const void* B = ws ? (const void*)workspace : (const void*)w;
    const void* S = (const void*)scale;
    void* C = (void*)(dx + (uint64_t)parts[p].row0 * in_features * 2);
    int M = (int)parts[p].rows, NC = (int)in_features, R = (int)out_features;
    int tiles_m = (int)((parts[p].rows + k.tile - 1) / k.tile);
    void* params[] = {&A, &B, &S, &C, &M, &NC, &R, &tiles_m};
    if (int rc = launch(k, params, parts[p].rows, in_features, stream)) return rc;
  }
  return 0;
}

int mo_int8_set_kernel(uint32_t kernel) {
  if (kernel != MO_INT8_KERNEL_REGISTERS && kernel != MO_INT8_KERNEL_LDS)
    return mo::set_error(MO_E_INVALID, "unknown int8 kernel selection");
  g_kernel.store(kernel);
  return 0;
}

}  // extern "C"
