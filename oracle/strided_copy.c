/*
 * Plain-C restatement of the dense-payload copies of the reference offload hooks.
 * TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
 *
 * RyukoMatoiFan/MOSS-Image training/activation_offload.py
 *   :123-124  cpu = empty(payload_shape); cpu.copy_(source)   -> oracle_gather, logical order
 *   :75-76    restored = empty_strided(payload_shape, stride); restored.copy_(payload)
 *                                                             -> oracle_scatter, logical order
 * Tensor.copy_ between a strided view and a contiguous tensor visits elements in row-major
 * (logical) order. The engine's payload is the same set of elements in storage order; passing
 * the stride-descending permutation (oracle_storage_perm) makes these routines produce and
 * consume that order, so one routine checks both formats.
 *
 * Build: make -C oracle   (outputs oracle/_build/liboracle_copy.so)
 */
#include <stdint.h>
#include <string.h>

#define ORACLE_MAX_DIMS 16

/* Dimension visiting order of a storage-order payload: by stride, largest first; ties keep
 * their logical order (stable). Writes ndim indices into perm. */
void oracle_storage_perm(int ndim, const int64_t* size, const int64_t* stride, int* perm) {
  (void)size;
  for (int i = 0; i < ndim; ++i) perm[i] = i;
  /* insertion sort, stable */
  for (int i = 1; i < ndim; ++i) {
    int p = perm[i];
    int j = i - 1;
    while (j >= 0 && stride[perm[j]] < stride[p]) {
      perm[j + 1] = perm[j];
      --j;
    }
    perm[j + 1] = p;
  }
}

/* Walk every logical element of (size, stride) with dimensions nested in `perm` order
 * (perm[0] outermost; NULL = logical order) and call copy for each. Returns the count. */
static int64_t walk(const int64_t* size, const int64_t* stride, int ndim, const int* perm, char* base,
                    char* dense, int64_t eb, int to_dense) {
  int order[ORACLE_MAX_DIMS];
  int64_t idx[ORACLE_MAX_DIMS];
  int64_t total = 1;
  if (ndim > ORACLE_MAX_DIMS) return -1;
  for (int i = 0; i < ndim; ++i) {
    order[i] = perm ? perm[i] : i;
    idx[i] = 0;
    total *= size[i];
  }
  for (int64_t n = 0; n < total; ++n) {
    int64_t off = 0;
    for (int i = 0; i < ndim; ++i) off += idx[i] * stride[order[i]];
    if (to_dense) memcpy(dense + n * eb, base + off * eb, (size_t)eb);
    else memcpy(base + off * eb, dense + n * eb, (size_t)eb);
    for (int i = ndim - 1; i >= 0; --i) { /* odometer, innermost = last in order */
      if (++idx[i] < size[order[i]]) break;
      idx[i] = 0;
    }
  }
  return total;
}

/* Gather the logical elements of a strided view into `out` (dense). */
int64_t oracle_gather(const void* base, int64_t elem_bytes, int ndim, const int64_t* size, const int64_t* stride,
                      const int* perm, void* out) {
  return walk(size, stride, ndim, perm, (char*)base, (char*)out, elem_bytes, 1);
}

/* Scatter a dense payload back into a strided view (inverse of oracle_gather). */
int64_t oracle_scatter(void* base, int64_t elem_bytes, int ndim, const int64_t* size, const int64_t* stride,
                       const int* perm, const void* in) {
  return walk(size, stride, ndim, perm, (char*)base, (char*)in, elem_bytes, 0);
}
