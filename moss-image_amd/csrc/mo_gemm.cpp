// Host side of the int8 weight-only GEMMs (csrc/mo_gemm.hip): argument checks, module loading
// from the embedded gfx950 code object, launches. C ABI: mo_int8_linear_forward/backward.
#include <hip/hip_runtime_api.h>
#include <stdint.h>

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

constexpr int kThreads = 256;
constexpr int kTile = 128;

struct GemmModule {
  hipModule_t module = nullptr;
  hipFunction_t fwd = nullptr, bwd = nullptr;
};

std::mutex g_mu;
std::map<int, GemmModule> g_modules;

int gemm_kernels(GemmModule* out) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_modules.find(device);
  if (it == g_modules.end()) {
    GemmModule m;
    if ((e = hipModuleLoadData(&m.module, mo_gemm_code)) != hipSuccess)
      return mo::set_hip_error((int)e, "hipModuleLoadData (int8 GEMM code object)");
    if ((e = hipModuleGetFunction(&m.fwd, m.module, "mo_int8_linear_fwd_kernel")) != hipSuccess ||
        (e = hipModuleGetFunction(&m.bwd, m.module, "mo_int8_linear_bwd_kernel")) != hipSuccess)
      return mo::set_hip_error((int)e, "hipModuleGetFunction (int8 GEMM)");
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
  if ((uint64_t)rows * (out_f > in_f ? out_f : in_f) >= (1ull << 40))
    return mo::set_error(MO_E_INVALID, "matrix too large");
  return 0;
}

int launch(hipFunction_t fn, void** params, uint32_t rows, uint32_t cols, uint64_t stream) {
  const uint64_t tiles_m = (rows + kTile - 1) / kTile, tiles_c = (cols + kTile - 1) / kTile;
  const uint64_t grid = tiles_m * tiles_c;
  if (grid >= (1ull << 31)) return mo::set_error(MO_E_INVALID, "grid too large");
  const hipError_t e = hipModuleLaunchKernel(fn, (uint32_t)grid, 1, 1, kThreads, 1, 1, 0, (hipStream_t)stream, params,
                                             nullptr);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "int8 GEMM launch");
  return 0;
}

}  // namespace

extern "C" {

int mo_int8_linear_forward(uint64_t x, uint64_t w, uint64_t scale, uint64_t bias, uint64_t y, uint32_t rows,
                           uint32_t in_features, uint32_t out_features, uint64_t stream) {
  if (int rc = check(x, w, scale, y, rows, in_features, out_features)) return rc;
  if (bias % 2) return mo::set_error(MO_E_INVALID, "bias pointer must be 2-byte aligned");
  GemmModule m;
  if (int rc = gemm_kernels(&m)) return rc;
  const void* A = (const void*)x;
  const void* B = (const void*)w;
  const void* S = (const void*)scale;
  const void* Bi = (const void*)bias;
  void* C = (void*)y;
  int M = (int)rows, NC = (int)out_features, R = (int)in_features;
  int tiles_m = (int)((rows + kTile - 1) / kTile);
  void* params[] = {&A, &B, &S, &Bi, &C, &M, &NC, &R, &tiles_m};
  return launch(m.fwd, params, rows, out_features, stream);
}

int mo_int8_linear_backward(uint64_t dy, uint64_t w, uint64_t scale, uint64_t dx, uint32_t rows, uint32_t in_features,
                            uint32_t out_features, uint64_t stream) {
  if (int rc = check(dy, w, scale, dx, rows, in_features, out_features)) return rc;
  GemmModule m;
  if (int rc = gemm_kernels(&m)) return rc;
  const void* A = (const void*)dy;
  const void* B = (const void*)w;
  const void* S = (const void*)scale;
  void* C = (void*)dx;
  int M = (int)rows, NC = (int)in_features, R = (int)out_features;
  int tiles_m = (int)((rows + kTile - 1) / kTile);
  void* params[] = {&A, &B, &S, &C, &M, &NC, &R, &tiles_m};
  return launch(m.bwd, params, rows, in_features, stream);
}

}  // extern "C"
