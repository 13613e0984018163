// Host-side layout logic shared by the kernel launchers and the engine.
//
// A saved tensor view is reduced to a canonical description of its storage footprint:
// dimensions of size > 1, sorted by stride (largest first), with mergeable neighbours
// merged. The non-overlap rule is the one the reference applies before it offloads a view
// (training/activation_offload.py:49-60): walking dimensions by increasing stride, each
// stride must be at least the extent covered so far. Stride-0 dimensions must already have
// been narrowed to one element by the caller (activation_offload.py:45-47).
#pragma once

#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <string>

#include "../../include/moss_offload.h"

namespace mo {

constexpr uint64_t kPayloadAlign = 256;

inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Canonical storage-order description of a tensor view (all strides in BYTES).
struct Canon {
  uint64_t base = 0;     // address of logical element (0,...,0)
  uint32_t eb = 0;       // element bytes
  int nd = 0;            // canonical dims, outermost first
  int64_t size[MO_MAX_DIMS] = {};
  int64_t stride[MO_MAX_DIMS] = {};  // bytes
  uint64_t numel = 0;
  uint64_t nbytes = 0;   // payload bytes: numel * eb, or numel * 2 for a bf16-high tensor
  bool bf16_high = false;  // MO_TENSOR_BF16_HIGH: payload = the high halves of float32 elements
};

// Returns 0 or an MO_E_* code with a message in `err`.
inline int canonicalize(const mo_tensor& t, Canon& c, std::string& err) {
  c = Canon();
  if (t.ndim > MO_MAX_DIMS) {
    err = "tensor has more than MO_MAX_DIMS dimensions";
    return MO_E_INVALID;
  }
  const uint32_t eb = t.elem_bytes;
  if (!(eb == 1 || eb == 2 || eb == 4 || eb == 8 || eb == 16)) {
    err = "element size must be 1, 2, 4, 8 or 16 bytes";
    return MO_E_INVALID;
  }
  c.base = t.ptr;
  c.eb = eb;
  uint64_t numel = 1;
  for (uint32_t i = 0; i < t.ndim; ++i) {
    if (t.size[i] < 0) {
      err = "negative size";
      return MO_E_INVALID;
    }
    if (t.stride[i] < 0) {
      err = "negative stride (the reference keeps such views resident)";
      return MO_E_LAYOUT;
    }
    numel *= (uint64_t)t.size[i];
  }
  c.numel = numel;
  c.nbytes = numel * eb;
  if (t.flags & ~(uint32_t)MO_TENSOR_BF16_HIGH) {
    err = "unknown tensor flags";
    return MO_E_INVALID;
  }
  if (t.flags & MO_TENSOR_BF16_HIGH) {
    if (eb != 4) {
      err = "MO_TENSOR_BF16_HIGH needs 4-byte (float32) elements";
      return MO_E_INVALID;
    }
    c.bf16_high = true;
    c.nbytes = numel * 2;
  }
  if (numel == 0) return 0;
  if (t.ptr % eb != 0) {
    err = "tensor address is not aligned to its element size";
    return MO_E_INVALID;
  }
  // Dimensions that move the address.
  struct Dim { int64_t stride, size; };
  Dim dims[MO_MAX_DIMS];
  int nd = 0;
  for (uint32_t i = 0; i < t.ndim; ++i) {
    if (t.size[i] <= 1) continue;
    if (t.stride[i] == 0) {
      err = "expanded (stride-0) dimension must be narrowed before packing";
      return MO_E_LAYOUT;
    }
    dims[nd++] = Dim{t.stride[i], t.size[i]};
  }
  // Increasing stride for the overlap walk; stable so equal strides keep their order.
  std::stable_sort(dims, dims + nd, [](const Dim& a, const Dim& b) { return a.stride < b.stride; });
  int64_t extent = 1;
  for (int i = 0; i < nd; ++i) {
    if (dims[i].stride < extent) {
      err = "overlapping layout (the reference keeps such views resident)";
      return MO_E_LAYOUT;
    }
    extent += (dims[i].size - 1) * dims[i].stride;
  }
  // Merge from the innermost outwards: outer.stride == inner.size * inner.stride.
  Dim merged[MO_MAX_DIMS];
  int nm = 0;
  for (int i = 0; i < nd; ++i) {
    if (nm > 0 && dims[i].stride == merged[nm - 1].size * merged[nm - 1].stride) {
      merged[nm - 1].size *= dims[i].size;
    } else {
      merged[nm++] = dims[i];
    }
  }
  c.nd = nm;
  for (int i = 0; i < nm; ++i) {  // outermost first
    c.size[i] = merged[nm - 1 - i].size;
    c.stride[i] = merged[nm - 1 - i].stride * (int64_t)eb;
  }
  if (c.bf16_high && !(nm == 0 || (nm == 1 && merged[0].stride == 1))) {
    err = "MO_TENSOR_BF16_HIGH needs a contiguous tensor";
    return MO_E_LAYOUT;
  }
  return 0;
}

// Highest address touched + 1, relative to base (0 for empty tensors).
inline uint64_t canon_extent_bytes(const Canon& c) {
  if (c.numel == 0) return 0;
  uint64_t last = 0;
  for (int i = 0; i < c.nd; ++i) last += (uint64_t)(c.size[i] - 1) * (uint64_t)c.stride[i];
  return last + c.eb;
}

// ---------------------------------------------------------------------------------------
// Division by a run-time invariant 32-bit divisor with one multiply-high and a shift
// (Granlund & Montgomery, "Division by invariant integers using multiplication", PLDI 1994,
// round-up multiplier; the 33-bit sum is formed in 64 bits). Exact for all n < 2^32.
struct FastDiv {
  uint32_t d = 1, m = 1, s = 0;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t l = 0;
  while (l < 32 && (uint64_t(1) << l) < d) ++l;
  f.s = l;
  // m = floor(2^32 * (2^l - d) / d) + 1
  f.m = (uint32_t)(((((uint64_t)1 << l) - d) << 32) / d + 1);
  return f;
}

inline uint32_t fastdiv_host(uint32_t n, const FastDiv& f) {
  uint64_t t = ((uint64_t)f.m * n) >> 32;
  return (uint32_t)((t + n) >> f.s);
}

}  // namespace mo
