// Host side of the int8 weight-only GEMMs (csrc/mo_gemm.hip): argument checks, module loading
// from the embedded gfx950 code object, the launch plan. C ABI: mo_int8_linear_forward/backward.
//
// Launch plan: the large tile (256 x 256) carries the work; when its grid would leave the GPU's
// last round of workgroups less than half full, the rows of that partial round go to a second
// launch, and a grid smaller than one round of large tiles is such a launch alone. That launch
// uses the small tile (128 x 128, two workgroups a CU), or, with the weight-in-registers kernel
// and a workspace, the large tile with its reduction split: `splits` workgroups per tile, each
// over a contiguous part of the reduction, write fp32 planes to the workspace, and
// mo_int8_split_reduce adds them in split order and rounds. The large and small tiles add the
// same products in the same order, so moving rows between them does not change results; a
// split reduction rounds its sum differently, and the rows it computes are the same for any
// call with the same row count in that launch, features and device.
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
  hipFunction_t ws_fwd_split = nullptr, ws_kscale_split = nullptr, split_reduce = nullptr;
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
        (e = hipModuleGetFunction(&m.transpose, m.module, "mo_int8_transpose_kernel")) != hipSuccess ||
        (e = hipModuleGetFunction(&m.ws_fwd_split, m.module, "mo_int8_ws_fwd_split")) != hipSuccess ||
        (e = hipModuleGetFunction(&m.ws_kscale_split, m.module, "mo_int8_ws_kscale_split")) != hipSuccess ||
        (e = hipModuleGetFunction(&m.split_reduce, m.module, "mo_int8_split_reduce")) != hipSuccess)
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

enum class Tile { Large, Small, Split };

struct Part {
  Tile tile;
  uint32_t row0, rows;
  uint32_t splits, split_steps;  // Split: workgroups per tile, reduction steps (of 64) each
};

constexpr uint32_t kMinSplitSteps = 12;  // a split covers at least 12 x 64 of the reduction
constexpr uint32_t kLoopSteps = 6;       // the register kernel's loop runs steps in sixes

// The launch for rows [row0, row0 + n) that do not fill a round of large tiles: a split
// reduction on the large tile when `steps` (the reduction in steps of 64; 0 = no split) allows
// at least two splits of kMinSplitSteps, the tiles times the splits fit one round, and the
// rows fill at least three quarters of their large tiles; the small tile otherwise. A split's
// length is rounded up to whole loop iterations (the last split takes what remains), which
// keeps the time of the longest split and launches fewer workgroups.
Part short_part(uint32_t row0, uint32_t n, uint32_t cols, uint32_t steps, int cus) {
  const uint64_t tm = (n + kLarge - 1) / kLarge, tiles = tm * ((cols + kLarge - 1) / kLarge);
  if (steps && 4ull * n >= 3ull * tm * kLarge && tiles <= (uint64_t)cus / 2) {
    uint64_t s = (uint64_t)cus / tiles;
    if (s > steps / kMinSplitSteps) s = steps / kMinSplitSteps;
    if (s >= 2) {
      uint32_t per = (uint32_t)((steps + s - 1) / s);
      per = (per + kLoopSteps - 1) / kLoopSteps * kLoopSteps;
      const uint32_t splits = (steps + per - 1) / per;
      if (splits >= 2) return {Tile::Split, row0, n, splits, per};
    }
  }
  return {Tile::Small, row0, n, 1, 0};
}

// Split [0, rows) between the large tile and a short launch (see the file comment).
int plan(uint32_t rows, uint32_t cols, uint32_t steps, int cus, Part parts[2]) {
  const uint64_t tm = (rows + kLarge - 1) / kLarge, tc = (cols + kLarge - 1) / kLarge, total = tm * tc;
  const uint64_t rounds = total / (uint64_t)cus, rem = total % (uint64_t)cus;
  if (rounds == 0) {
    parts[0] = short_part(0, rows, cols, steps, cus);
    return 1;
  }
  if (rem == 0 || 2 * rem >= (uint64_t)cus) {
    parts[0] = {Tile::Large, 0, rows, 1, 0};
    return 1;
  }
  const uint64_t main_rows = (rounds * (uint64_t)cus / tc) * kLarge;
  if (main_rows == 0) {
    parts[0] = {Tile::Small, 0, rows, 1, 0};
    return 1;
  }
  if (main_rows >= rows) {
    parts[0] = {Tile::Large, 0, rows, 1, 0};
    return 1;
  }
  parts[0] = {Tile::Large, 0, (uint32_t)main_rows, 1, 0};
  parts[1] = short_part((uint32_t)main_rows, rows - (uint32_t)main_rows, cols, steps, cus);
  return 2;
}

// fp32 planes of a plan's split launch (0 if it has none), rounded up to 256 bytes.
uint64_t split_bytes(const Part* parts, int n, uint32_t cols) {
  uint64_t b = 0;
  for (int p = 0; p < n; ++p)
    if (parts[p].tile == Tile::Split) b = (uint64_t)parts[p].splits * parts[p].rows * cols * 4;
  return (b + 255) & ~uint64_t(255);
}

// Reduction steps a split may use: the weight-in-registers kernel takes reductions of whole
// steps of 64 only.
uint32_t split_steps_of(uint32_t reduction) { return reduction % 64 ? 0 : reduction / 64; }

int cu_count(int* cus) {
  GemmModule m;
  if (int rc = gemm_module(&m)) return rc;
  *cus = m.cus;
  return 0;
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

// A split part: `splits` x tiles workgroups of the split kernel writing fp32 planes to `planes`,
// then the reduction into C (rows of the part, `cols` wide; bias may be 0).
int launch_split(const GemmModule& m, hipFunction_t fn, const Part& part, uint64_t a, uint64_t b, uint64_t scale,
                 uint64_t bias, uint64_t c, uint64_t planes, uint32_t cols, uint32_t reduction, uint64_t stream) {
  const uint64_t tiles_m = (part.rows + kLarge - 1) / kLarge, tiles_c = (cols + kLarge - 1) / kLarge;
  const void* A = (const void*)a;
  const void* B = (const void*)b;
  const void* S = (const void*)scale;
  void* P = (void*)planes;
  int M = (int)part.rows, N = (int)cols, K = (int)reduction, tm = (int)tiles_m, splits = (int)part.splits,
      per = (int)part.split_steps;
  void* params[] = {&A, &B, &S, &P, &M, &N, &K, &tm, &splits, &per};
  hipError_t e = hipModuleLaunchKernel(fn, (uint32_t)(tiles_m * tiles_c * part.splits), 1, 1, 256, 1, 1, 0,
                                       (hipStream_t)stream, params, nullptr);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "int8 GEMM split launch");
  const void* Pc = (const void*)planes;
  const void* Bi = (const void*)bias;
  void* C = (void*)c;
  uint32_t rows = part.rows, n = cols, sp = part.splits;
  void* rparams[] = {&Pc, &Bi, &C, &rows, &n, &sp};
  const uint64_t lanes = (uint64_t)part.rows * (cols / 8);
  e = hipModuleLaunchKernel(m.split_reduce, (uint32_t)((lanes + 255) / 256), 1, 1, 256, 1, 1, 0, (hipStream_t)stream,
                            rparams, nullptr);
  if (e != hipSuccess) return mo::set_hip_error((int)e, "int8 split reduction launch");
  return 0;
}

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

uint64_t mo_int8_forward_workspace_bytes(uint32_t rows, uint32_t in_features, uint32_t out_features) {
  int cus = 0;
  if (cu_count(&cus)) return 0;
  Part parts[2];
  const int n = plan(rows, out_features, split_steps_of(in_features), cus, parts);
  return split_bytes(parts, n, out_features);
}

int mo_int8_linear_forward(uint64_t x, uint64_t w, uint64_t scale, uint64_t bias, uint64_t y, uint32_t rows,
                           uint32_t in_features, uint32_t out_features, uint64_t workspace, uint64_t workspace_bytes,
                           uint64_t stream) {
  if (int rc = check(x, w, scale, y, rows, in_features, out_features)) return rc;
  if (bias % 2) return mo::set_error(MO_E_INVALID, "bias pointer must be 2-byte aligned");
  if (workspace % 16) return mo::set_error(MO_E_INVALID, "workspace pointer must be 16-byte aligned");
  GemmModule m;
  if (int rc = gemm_module(&m)) return rc;
  const int tail = in_features % 64 != 0;
  const bool registers = !tail && g_kernel.load() == MO_INT8_KERNEL_REGISTERS;
  Part parts[2];
  const int n = plan(rows, out_features, registers && workspace ? split_steps_of(in_features) : 0, m.cus, parts);
  if (workspace && workspace_bytes < split_bytes(parts, n, out_features))
    return mo::set_error(MO_E_INVALID, "workspace smaller than mo_int8_forward_workspace_bytes");
  for (int p = 0; p < n; ++p) {
    const uint64_t a = x + (uint64_t)parts[p].row0 * in_features * 2;
    const uint64_t c = y + (uint64_t)parts[p].row0 * out_features * 2;
    if (parts[p].tile == Tile::Split) {
      if (int rc = launch_split(m, m.ws_fwd_split, parts[p], a, w, scale, bias, c, workspace, out_features,
                                in_features, stream))
        return rc;
      continue;
    }
    const bool small = parts[p].tile == Tile::Small;
    const Kernel k = !small && registers ? registers_kernel(m.ws_fwd) : m.k[0][small][tail];
    const void* A = (const void*)a;
    const void* B = (const void*)w;
    const void* S = (const void*)scale;
    const void* Bi = (const void*)bias;
    void* C = (void*)c;
    int M = (int)parts[p].rows, NC = (int)out_features, R = (int)in_features;
    int tiles_m = (int)((parts[p].rows + k.tile - 1) / k.tile);
    void* params[] = {&A, &B, &S, &Bi, &C, &M, &NC, &R, &tiles_m};
    if (int rc = launch(k, params, parts[p].rows, out_features, stream)) return rc;
  }
  return 0;
}

// The transposed int8 weight, then (when the plan splits a reduction) the fp32 planes.
uint64_t mo_int8_backward_workspace_bytes(uint32_t rows, uint32_t in_features, uint32_t out_features) {
  const uint64_t transposed = ((uint64_t)in_features * out_features + 255) & ~uint64_t(255);
  int cus = 0;
  if (cu_count(&cus)) return transposed;
  Part parts[2];
  const int n = plan(rows, in_features, split_steps_of(out_features), cus, parts);
  return transposed + split_bytes(parts, n, in_features);
}

int mo_int8_linear_backward(uint64_t dy, uint64_t w, uint64_t scale, uint64_t dx, uint32_t rows, uint32_t in_features,
                            uint32_t out_features, uint64_t workspace, uint64_t workspace_bytes, uint64_t stream) {
  if (int rc = check(dy, w, scale, dx, rows, in_features, out_features)) return rc;
  if (workspace % 16) return mo::set_error(MO_E_INVALID, "workspace pointer must be 16-byte aligned");
  GemmModule m;
  if (int rc = gemm_module(&m)) return rc;
  const int tail = out_features % 64 != 0;
  const bool registers = !tail && g_kernel.load() == MO_INT8_KERNEL_REGISTERS && workspace;
  const uint64_t transposed_bytes = ((uint64_t)in_features * out_features + 255) & ~uint64_t(255);
  Part parts[2];
  const int n = plan(rows, in_features, registers ? split_steps_of(out_features) : 0, m.cus, parts);
  if (workspace && workspace_bytes < transposed_bytes + split_bytes(parts, n, in_features))
    return mo::set_error(MO_E_INVALID, "workspace smaller than mo_int8_backward_workspace_bytes");
  bool transposed = false;
  for (int p = 0; p < n; ++p) {
    const bool small = parts[p].tile == Tile::Small;
    const bool ws = !small && registers;
    if (ws && !transposed) {
      // the weight with the reduction (out) contiguous, for the weight-in-registers kernels
      const void* src = (const void*)w;
      void* dst = (void*)workspace;
      uint32_t r = out_features, c = in_features;
      void* tparams[] = {&src, &dst, &r, &c};
      const uint64_t blocks = (uint64_t)((out_features + 127) / 128) * ((in_features + 127) / 128);
      const hipError_t e = hipModuleLaunchKernel(m.transpose, (uint32_t)blocks, 1, 1, 256, 1, 1, 0,
                                                 (hipStream_t)stream, tparams, nullptr);
      if (e != hipSuccess) return mo::set_hip_error((int)e, "int8 transpose launch");
      transposed = true;
    }
    const uint64_t a = dy + (uint64_t)parts[p].row0 * out_features * 2;
    const uint64_t c = dx + (uint64_t)parts[p].row0 * in_features * 2;
    if (parts[p].tile == Tile::Split) {
      if (int rc = launch_split(m, m.ws_kscale_split, parts[p], a, workspace, scale, 0, c,
                                workspace + transposed_bytes, in_features, out_features, stream))
        return rc;
      continue;
    }
    const Kernel k = ws ? registers_kernel(m.ws_kscale) : m.k[1][small][tail];
    const void* A = (const void*)a;
    const void* B = ws ? (const void*)workspace : (const void*)w;
    const void* S = (const void*)scale;
    void* C = (void*)c;
    int M = (int)parts[p].rows, NC = (int)in_features, R = (int)out_features;
    int tiles_m = (int)((parts[p].rows + k.tile - 1) / k.tile);
    void* params[] = {&A, &B, &S, &C, &M, &NC, &R, &tiles_m};
    if (int rc = launch(k, params, parts[p].rows, in_features, stream)) return rc;
  }
  return 0;
}

int mo_int8_launch_plan(uint32_t rows, uint32_t cols, uint32_t reduction, uint32_t cus, uint32_t kernel,
                        uint32_t* n_parts, uint32_t* parts) {
  if (!n_parts || !parts) return mo::set_error(MO_E_INVALID, "null output pointer");
  if (rows == 0 || cols == 0 || reduction == 0 || cus == 0) return mo::set_error(MO_E_INVALID, "empty shape");
  if (kernel != MO_INT8_KERNEL_REGISTERS && kernel != MO_INT8_KERNEL_LDS)
    return mo::set_error(MO_E_INVALID, "unknown int8 kernel selection");
  Part p[2];
  const uint32_t steps = kernel == MO_INT8_KERNEL_REGISTERS ? split_steps_of(reduction) : 0;
  const int n = plan(rows, cols, steps, (int)cus, p);
  for (int i = 0; i < n; ++i) {
    parts[5 * i + 0] = p[i].tile == Tile::Large ? 0u : p[i].tile == Tile::Small ? 1u : 2u;
    parts[5 * i + 1] = p[i].row0;
    parts[5 * i + 2] = p[i].rows;
    parts[5 * i + 3] = p[i].splits;
    parts[5 * i + 4] = p[i].split_steps;
  }
  *n_parts = (uint32_t)n;
  return 0;
}

int mo_int8_set_kernel(uint32_t kernel) {
  if (kernel != MO_INT8_KERNEL_REGISTERS && kernel != MO_INT8_KERNEL_LDS)
    return mo::set_error(MO_E_INVALID, "unknown int8 kernel selection");
  g_kernel.store(kernel);
  return 0;
}

}  // extern "C"
