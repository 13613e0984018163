/*
 * moss_offload.h - C ABI of the MI355X activation-offload engine and block streamer.
 *
 * The engine replaces the per-tensor work that MOSS-Image's saved-tensor hooks do in
 * training/activation_offload.py (reference repository RyukoMatoiFan/MOSS-Image):
 *
 *   pack   (activation_offload.py:116-134)  pinned torch.empty + copy_(non_blocking) + Event
 *   unpack (activation_offload.py:136-147)  wait_event + _restore_layout
 *   _restore_layout (activation_offload.py:64-77)  empty_strided + copy_ + as_strided
 *
 * The reference is pure Python and exposes no foreign-function interface of its own; the
 * Python shim in moss-image_amd/moss_offload binds this header through ctypes and keeps the
 * reference's Python API (activation_cpu_offload, _offload_view, _restore_layout).
 *
 * Conventions
 *   - Every function returns 0 on success and a non-zero status otherwise (a hipError_t value,
 *     or MO_E_* below). mo_last_error() returns a thread-local message for the last failure.
 *   - Device pointers and streams cross the boundary as uint64_t (data_ptr(), cuda_stream).
 *   - No C++ exception crosses the boundary. All engine calls are serialised by an engine mutex.
 *
 * Payload format (shared by every entry point)
 *   A tensor's payload is its logical elements in STORAGE order: dimensions of size > 1 sorted
 *   by stride, largest first, so the copy reads and writes memory in address order and never
 *   transposes. Restoring into a tensor with the same strides is the exact inverse. Each
 *   payload starts at a 256-byte aligned offset of its staging buffer.
 */
#ifndef MOSS_OFFLOAD_H
#define MOSS_OFFLOAD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MO_ABI_VERSION 21
#define MO_MAX_DIMS 8

/* Error codes outside the hipError_t range. */
#define MO_E_INVALID 1001   /* bad argument, descriptor or handle          */
#define MO_E_LAYOUT 1002    /* overlapping / negative-stride layout         */
#define MO_E_HOST_OOM 1003  /* pinned host pool limit reached               */
#define MO_E_STATE 1004     /* call not valid in the engine's current state */

/* Flags for mo_config.flags. */
#define MO_FLAG_TIMING 0x1         /* time every copy: HIP events (KERNEL_COPY link), or the
                                      SDMA engines' own start/end stamps (SDMA link)      */
#define MO_FLAG_KERNEL_COPY 0x2    /* move D2H/H2D with a copy kernel on HIP streams instead
                                      of the SDMA engines (comparison; contends for CUs)   */
#define MO_FLAG_KERNEL_TIMING 0x4  /* time every pack/unpack launch with HIP events       */
#define MO_FLAG_NO_STAGED_RESTORE 0x8 /* always restore through H2D, even when a segment is
                                         still intact in its staging slot                  */
#define MO_FLAG_EAGER_PACK 0x10    /* launch each mo_pack call's gather kernels before it
                                      returns instead of batching them per segment        */
#define MO_FLAG_HIP_DMA 0x20       /* move D2H/H2D with hipMemcpyAsync on dedicated HIP copy
                                      streams (the runtime runs them on the SDMA engines),
                                      ordered by hipStreamWaitEvent only: an unpack enqueues
                                      a stream wait and never blocks the host. D2H copies of
                                      2 MiB or more are split over two copy streams while no
                                      H2D is pending, unless d2h_engine has exactly one bit */

/* Cache policy of the kernels. Default: pack reads saved tensors with ordinary loads and writes
   the staging slot with streaming (non-temporal) stores; unpack reads the restore slot with
   non-temporal loads and writes restored tensors with streaming stores. */
#define MO_FLAG_PACK_NT_LOAD 0x40  /* the pack kernel reads saved tensors with non-temporal
                                      (streaming) loads; the Python layer sets it by default
                                      (faster in every measured step once gathers are
                                      batched per segment)                                */
#define MO_FLAG_UNPACK_CACHED_LOAD 0x80 /* the unpack kernel reads the payload with ordinary
                                           loads instead of non-temporal ones             */
#define MO_FLAG_UNPACK_CACHED_STORE 0x100 /* the unpack kernel writes restored tensors with
                                             ordinary stores instead of streaming ones      */
#define MO_FLAG_WIRE_CODING 0x200 /* code every staging segment of at least 256 KiB with the
                                     lossless wire coding (mo_wire_encode) before its D2H and
                                     decode it after its H2D: bfloat16 activations cross the
                                     host link in about 0.66 of their bytes. SDMA link only
                                     (the coded length is read when the copy is issued);
                                     costs one wire buffer per staging and restore slot     */
#define MO_FLAG_WIRE_AUTO 0x400   /* the same, only for segments that close while the D2H
                                     copies queued or in flight hold at least two staging
                                     slots of bytes (the link is the bottleneck)            */

/*
 * A strided tensor view on the device. `ptr` is the address of logical element (0,...,0),
 * which is the lowest address because all strides are non-negative. Strides are in
 * elements. This is the information the reference reads at activation_offload.py:40-61
 * (shape, stride) plus data_ptr() and element_size().
 */
typedef struct mo_tensor {
  uint64_t ptr;
  uint32_t elem_bytes; /* 1, 2, 4, 8 or 16 */
  uint32_t ndim;       /* 0..MO_MAX_DIMS */
  int64_t size[MO_MAX_DIMS];
  int64_t stride[MO_MAX_DIMS];
  uint32_t flags;      /* MO_TENSOR_*                                                    */
  uint32_t reserved;   /* 0                                                              */
} mo_tensor;

/* Flags for mo_tensor.flags.
 * MO_TENSOR_BF16_HIGH: a contiguous float32 tensor whose values are exactly bfloat16 (the low
 * 16 bits of every element are zero, as for the output of a bfloat16 -> float32 cast). Its
 * payload keeps the high 16 bits of each element (numel x 2 bytes), and restoring it writes
 * them back with the low bits zero: the same float32 bits, over half the bytes. No reference
 * counterpart: the reference copies the float32 tensor as it is. */
#define MO_TENSOR_BF16_HIGH 0x1

/* Engine configuration (mo_create). Zero fields take the defaults in brackets. */
typedef struct mo_config {
  uint64_t stage_slot_bytes;    /* [128 MiB] device staging and restore slot size      */
  uint32_t stage_slots;         /* [4] slots in the forward staging ring               */
  uint32_t restore_slots;       /* [16] slots in the backward restore ring, each of
                                   stage_slot_bytes (with restore_small_slots set, those
                                   past the first two get their memory at first use)  */
  uint64_t host_limit_bytes;    /* [0 = no limit] cap on pinned host memory             */
  uint64_t host_chunk_bytes;    /* [1 GiB] granularity of hipHostMalloc reservations   */
  uint32_t flags;               /* MO_FLAG_*                                          */
  uint32_t copy_kernel_blocks;  /* [16] workgroups of the copy kernel (KERNEL_COPY)  */
  uint32_t d2h_engine;          /* [0 = the two lowest available] SDMA engine bits for
                                   D2H; with two, a copy of 2 MiB or more is split in
                                   halves, one per engine                              */
  uint32_t h2d_engine;          /* [0 = the lowest available not used by D2H] SDMA
                                   engine bits for H2D (two bits: split the same way)  */
  uint64_t wire_device_limit;   /* [0 = no limit] cap on the device bytes of the wire
                                   buffers; where they would pass it, or their
                                   allocation fails, segments cross raw and the engine
                                   tries again at the next forward                    */
  uint64_t commit_batch_bytes;  /* [0 = off] a segment closed by mo_commit waits, with its
                                   gathers, for later commits until this many bytes of
                                   such segments (or the staging slot) are full; then one
                                   launch gathers them all and their D2Hs follow. No
                                   reference counterpart (the reference copies each save
                                   at its hook)                                         */
  uint32_t stage_slots_max;     /* [0 = stage_slots: fixed] the staging ring grows, at the
                                   commit of a group of n segments, to ceil(n / 3) slots,
                                   at most this many                                   */
  uint32_t restore_slots_max;   /* [0 = restore_slots: fixed] the restore ring grows, at
                                   the same commit, to n + 2 slots, at most this many.
                                   A slot that cannot be allocated (or whose wire buffer
                                   would pass wire_device_limit) ends the growth; the
                                   engine runs on with the slots it has                  */
  uint32_t restore_small_slots; /* [0 = off] restore slots of a quarter of
                                   stage_slot_bytes for raw segments that fit one: the
                                   ring gains up to this many once 8 groups in a row were
                                   committed with only such segments (a checkpointed
                                   block's inputs). Nonzero also allocates every restore
                                   slot past the first two at its first use, and mo_trim
                                   frees them again once no group is live. stage_slots_max
                                   + restore_slots_max + this: 64 at most              */
} mo_config;

/* Where one packed tensor lives: its group (one block's saves) and index in the group. */
typedef struct mo_ref {
  uint64_t group;
  uint32_t entry;
  uint32_t reserved;
} mo_ref;

typedef struct mo_stats {
  uint64_t groups_created, groups_live, entries_live;
  uint64_t bytes_packed, bytes_unpacked;  /* payload bytes through pack / unpack kernels */
  uint64_t bytes_d2h, bytes_h2d;          /* bytes over the host link                  */
  uint64_t pack_launches, unpack_launches, d2h_copies, h2d_copies;
  uint64_t host_bytes_in_use, host_bytes_peak, host_bytes_reserved;  /* pinned pool; the peak since
                                                                         creation or mo_reset_stats */
  uint64_t stage_slot_waits;   /* staging slots reused (each ordered after its last D2H) */
  uint64_t host_blocks;        /* engine calls that blocked the host for a copy          */
  double host_block_ms;        /* time spent blocked in them                             */
  uint64_t prefetch_issued;    /* segments fetched ahead of their unpack              */
  uint64_t prefetch_hits;      /* segments already resident when unpack asked          */
  uint64_t restore_fetches;    /* segments fetched on demand by unpack                 */
  uint64_t staged_hits;        /* segments unpacked from their staging slot (no H2D)   */
  uint64_t bytes_staged;       /* bytes of those segments                              */
  double d2h_ms, h2d_ms;       /* copy-engine busy time of completed copies (SDMA: host
                                  clock at issue/completion; KERNEL_COPY: HIP events)  */
  uint64_t timed_d2h_bytes, timed_h2d_bytes; /* bytes of those completed copies          */
  uint64_t copy_failures;      /* copies the runtime reported as failed                 */
  double pack_ms, unpack_ms;   /* summed kernel durations (MO_FLAG_KERNEL_TIMING)         */
  uint64_t timed_pack_bytes, timed_unpack_bytes; /* payload bytes of those launches      */
  uint64_t timed_pack_launches, timed_unpack_launches;
  uint64_t timed_pack_hbm_bytes, timed_unpack_hbm_bytes; /* device-memory bytes read + written
                                                            by those launches                */
  uint64_t wire_segments;      /* segments sent wire-coded (MO_FLAG_WIRE_*)               */
  uint64_t wire_raw_bytes;     /* their payload bytes                                     */
  uint64_t wire_bytes;         /* their coded bytes, counted as each D2H completes; bytes_d2h
                                  and bytes_h2d count coded bytes for coded segments        */
  uint64_t device_ring_bytes;  /* device memory the engine holds: staging and restore slots,
                                  plus their wire buffers once wire coding has run          */
  uint64_t wire_fallbacks;     /* segments meant for wire coding that crossed raw because the
                                  wire buffers could not be allocated (or would pass
                                  wire_device_limit)                                        */
  uint64_t ahead_restored;     /* further groups of mo_unpack_groups restored               */
  uint64_t ahead_not_resident; /* further groups left: a segment was not in a restore slot  */
  uint64_t ahead_in_flight;    /* further groups left: a segment's H2D had not started      */
  uint64_t restore_slots_big;   /* restore slots of stage_slot_bytes holding device memory  */
  uint64_t restore_slots_small; /* restore slots of a quarter of that (restore_small_slots) */
} mo_stats;

typedef struct mo_engine mo_engine;

/* ---- library ---------------------------------------------------------------------------- */
int mo_abi_version(void);
const char* mo_last_error(void);

/* ---- kernels alone (microbenchmarks, parity tests, _restore_layout) ---------------------- */

/* Payload layout of n tensors: offsets[i] (256-byte aligned) and the total bytes. Host only. */
int mo_payload_layout(const mo_tensor* tensors, int n, uint64_t* offsets, uint64_t* total_bytes);

/* Pack kernel: gather n tensor views into `payload` at `offsets` (NULL = mo_payload_layout).
 * Replaces the device side of cpu.copy_(source) at activation_offload.py:124. */
int mo_gather(const mo_tensor* tensors, int n, uint64_t payload, const uint64_t* offsets,
              uint64_t stream);

/* Unpack kernel: scatter payloads back into n tensor views with the same strides.
 * Replaces restored.copy_(payload) at activation_offload.py:75-76. */
int mo_scatter(const mo_tensor* tensors, int n, uint64_t payload, const uint64_t* offsets,
               uint64_t stream);

/* Wire coding of a payload (lossless; no counterpart in the reference, which copies raw bytes).
 * The engine codes staging segments with it before their D2H when MO_FLAG_WIRE_CODING (or
 * MO_FLAG_WIRE_AUTO) is set. Sixteen-bit words keep their sign and mantissa as a byte; the
 * 8-bit exponents of each 32 KiB tile are coded with interleaved rANS (64 states, the tile's
 * exponent frequencies normalised to 4096), and a tile that would not shrink is stored raw;
 * bfloat16 activations shrink to about 0.66 of their bytes. Format in csrc/mo_wire.h.
 * mo_wire_capacity: the largest coded size of raw_bytes plus the coder's working space (the
 * wire buffer to provide). mo_wire_encode codes raw_bytes at device `raw` into device `wire`
 * (3 launches on `stream`); the coded size is the stream's first u64 and is also written to
 * pinned host memory at `host_total` (0: not). mo_wire_decode restores raw_bytes bytes from a
 * coded stream of at most wire_bytes. Buffers 16-byte aligned, raw_bytes at most 2^29. */
uint64_t mo_wire_capacity(uint64_t raw_bytes);
int mo_wire_encode(uint64_t raw, uint64_t raw_bytes, uint64_t wire, uint64_t wire_capacity, uint64_t host_total,
                   uint64_t stream);
int mo_wire_decode(uint64_t wire, uint64_t wire_bytes, uint64_t raw, uint64_t raw_bytes, uint64_t stream);

/* Gather n tensor views, in the payload format of mo_gather, into pinned host memory at `host`
 * (host_bytes long) on `stream`, allocating nothing. offsets[i] (may be NULL) receives each
 * payload's offset, as mo_payload_layout gives it; bytes between payloads are unspecified. The
 * pack kernel gathers into a device scratch array that is part of the library's code object
 * (64 MiB per device, reserved when the code object loads on that device and held until the
 * process ends), then a DMA copies the payload to `host`. Payloads larger than the scratch are
 * rejected with MO_E_INVALID, as is a host buffer that is too small or not pinned.
 * No counterpart in the reference (it pins a fresh tensor per save, activation_offload.py:123):
 * a variant of mo_pack for callers that cannot allocate, such as code under HIP graph capture or
 * a serving loop that must not touch the allocator. The first call on a device loads the code
 * object (set-up, not capturable); later calls only enqueue a kernel and a copy. Every call on
 * one device shares its scratch: calls that overlap on that device (different streams with no
 * order between them) race. */
int mo_pack_to_host(const mo_tensor* tensors, int n, uint64_t host, uint64_t host_bytes, uint64_t* offsets,
                    uint64_t stream);

/* Copy `bytes` between device and pinned host memory with the engine's link-copy kernel
 * (direction 0 = device->host, 1 = host->device). Measures the copy-kernel alternative to
 * the DMA engines. */
int mo_link_copy(uint64_t dst, uint64_t src, uint64_t bytes, int direction, uint32_t blocks,
                 uint64_t stream);

/* ---- engine (the activation_cpu_offload hook pair, activation_offload.py:80-149) --------- */
int mo_create(int device, const mo_config* config, mo_engine** out);
int mo_destroy(mo_engine* engine);

/* Pack n saved tensors into the open group (a new group opens if none is). Each tensor is
 * gathered into the staging ring on `stream` and refs[i] says where it went. Replaces
 * pack(), activation_offload.py:116-134.
 *
 * The gather kernels of consecutive calls on one stream are batched: they are launched, in
 * stream order, as one kernel per staging segment when the segment closes (its slot fills, or
 * mo_commit / mo_unpack of the group closes it; with commit_batch_bytes, commits' segments
 * gather together up to that many bytes or the slot's end, and any unpack, prefetch, release
 * or synchronize launches them first), before a call on another stream, and at
 * mo_synchronize or mo_pack_flush. The caller therefore keeps the memory of every tensor it
 * passed valid (not freed, not written) until mo_pack_progress reports the call as launched;
 * after that the usual stream-ordered reuse applies. MO_FLAG_EAGER_PACK launches every call's
 * kernels before it returns. Releasing the open group drops its gathers not yet launched. */
int mo_pack(mo_engine* engine, const mo_tensor* tensors, int n, uint64_t stream, mo_ref* refs);

/* *calls = mo_pack calls made so far; every call numbered (from 1) at most *launched has all
 * of its gather kernels enqueued. No reference counterpart: the reference copies at once. */
int mo_pack_progress(mo_engine* engine, uint64_t* calls, uint64_t* launched);

/* Launch every pending gather kernel now (on the stream of the calls that made them), and
 * issue the D2H of every committed segment that was waiting for them. */
int mo_pack_flush(mo_engine* engine);

/* Byte equality of nbytes at device addresses a and b (both 16-byte aligned), checked by a
 * kernel on `stream` after the work already queued there; nothing blocks. *ticket receives a
 * handle for the result, or 0 when all 64 result slots are taken (no check was started).
 * The caller keeps both ranges unchanged until the result is known.
 * No reference counterpart: the hooks use it to store a saved tensor that equals an earlier
 * save (two casts of one tensor, for instance) once, where the reference copies both. */
int mo_equal(mo_engine* engine, uint64_t a, uint64_t b, uint64_t nbytes, uint64_t stream, uint64_t* ticket);

/* *state = 0 while the check runs (wait == 0), 1 if the ranges were equal, 2 if they differed.
 * wait != 0 blocks until the result is known. A ticket reports 1 or 2 once and is then freed. */
int mo_equal_result(mo_engine* engine, uint64_t ticket, int wait, int* state);

/* Give up a ticket whose result is no longer wanted; its slot is reused once the check ends. */
int mo_equal_discard(mo_engine* engine, uint64_t ticket);

/* Close the open group: the compute stream records an event, the D2H stream waits for it and
 * streams the group's staging segments into pinned host memory. *group receives the id
 * (UINT64_MAX if no group was open). Replaces the Event().record at activation_offload.py:125. */
int mo_commit(mo_engine* engine, uint64_t stream, uint64_t* group);

/* Enqueue H2D copies of a committed group into free restore slots (as many segments as fit),
 * so a later mo_unpack on `stream` finds them resident. Segments still intact in their staging
 * slot (and packed on `stream`) are skipped: unpack reads them there. Never blocks the host. */
int mo_prefetch(mo_engine* engine, uint64_t group, uint64_t stream);

/* The same for the segments that hold entry `entry` of the group only: a save that later blocks
 * share, which backward needs while the rest of its (older) group is not due yet. No reference
 * counterpart: the reference prefetches nothing; the H2D it brings forward is the one the
 * reference's unpack (activation_offload.py:136-147) waits for. */
int mo_prefetch_entry(mo_engine* engine, uint64_t group, uint32_t entry, uint64_t stream);

/* Prefetch several groups, given in the order backward will need them: the first as
 * mo_prefetch does; each later one only if every segment it still needs gets a free restore
 * slot now (a farther group never takes a slot a nearer one will need); stops at the first
 * that does not fit. No reference counterpart: the reference prefetches nothing. */
int mo_prefetch_groups(mo_engine* engine, const uint64_t* groups, uint32_t n, uint64_t stream);

/* Restore entries of a group: dst[i] is the device address for entry i (0 = skip it), laid out
 * with the strides the entry was packed with. H2D copies any missing segment, makes `stream`
 * wait for it, and launches the unpack kernel on `stream`. Replaces unpack(),
 * activation_offload.py:136-147. */
int mo_unpack(mo_engine* engine, uint64_t group, const uint64_t* dst, uint32_t n,
              uint64_t stream);

/* Restore groups[0] as mo_unpack does (its entries' addresses are dst[0 .. counts[0])), then
 * each further groups[k] (the next counts[k] addresses) only if every segment it needs can be
 * read now with at most a short wait: resident in a restore slot with its H2D landed or handed
 * to the copy engine, or still in its staging slot. unpacked[k] is set to 1 for each group
 * restored. The first group's last segment and the further groups are scattered together, in
 * as few kernel launches as their
 * pieces allow (small groups, such as the inputs of checkpointed blocks, then share one large
 * launch). No reference counterpart: the reference restores one saved tensor per unpack
 * (activation_offload.py:136-147). */
int mo_unpack_groups(mo_engine* engine, const uint64_t* groups, const uint64_t* dst,
                     const uint32_t* counts, uint32_t n, uint64_t stream, uint32_t* unpacked);

/* Drop a group: its pinned host memory returns to the pool once every copy using it ended. */
int mo_release(mo_engine* engine, uint64_t group);

/* Number of entries in a group and whether its D2H completed (host query, non-blocking). */
int mo_group_info(mo_engine* engine, uint64_t group, uint32_t* entries, uint64_t* payload_bytes,
                  int* d2h_complete);

/* Block the host until every copy the engine enqueued has finished. */
int mo_synchronize(mo_engine* engine);

int mo_get_stats(mo_engine* engine, mo_stats* stats);
int mo_reset_stats(mo_engine* engine);

/* Release pinned chunks that hold no live payload. With no group live, also free the wire
 * buffers (after waiting for every copy and for the device; the next coded segment allocates
 * them again) and, with restore_small_slots set, the memory of every restore slot past the
 * first two (given again at the slot's next use). */
int mo_trim(mo_engine* engine);

/* Name of the host-link transport in use: "sdma" or "kernel". */
const char* mo_link_name(mo_engine* engine);

/* ---- block streaming (AsyncBlockStreamer, training/memory.py:93-361; TrainableBlockStreamer,
 * training/trainable_offload.py:89-477) --------------------------------------------------- */

/* Pinned host memory of `bytes` rounded up to a page, for the block masters of a streamed
 * model (replaces torch.empty(..., pin_memory=True) at memory.py:461, which rounds each pin up to
 * a power of two). Independent of any engine; free with mo_pinned_free. */
int mo_pinned_alloc(uint64_t bytes, uint64_t* host);
int mo_pinned_free(uint64_t host);

typedef struct mo_streamer mo_streamer;

typedef struct mo_streamer_stats {
  uint64_t fills, bytes;        /* slot fills issued and their bytes                        */
  uint64_t timed_bytes;         /* bytes of completed fills                                 */
  double busy_ms;               /* SDMA busy time of completed fills (host clock)           */
  uint64_t host_blocks;         /* acquires that had to block the host for a fill           */
  double host_block_ms;
  uint64_t copy_failures;
  uint64_t writebacks, writeback_bytes;  /* slot write-backs issued and their bytes          */
  uint64_t timed_writeback_bytes;        /* bytes of completed write-backs                  */
  double writeback_busy_ms;              /* SDMA busy time of completed write-backs         */
} mo_streamer_stats;

/* A streamer with `slots` device staging slots (the buffers themselves belong to the caller)
 * and its own SDMA queues (h2d_engine: SDMA engine bits for fills, 0 = the lowest available
 * other than the two write-back engines; with two bits, copies of 2 MiB or more are split). Replaces the copy stream and slot events of AsyncBlockStreamer
 * (memory.py:109-119) and TrainableBlockStreamer (trainable_offload.py:128-179). */
int mo_streamer_create(int device, uint32_t slots, uint32_t h2d_engine, mo_streamer** out);
int mo_streamer_destroy(mo_streamer* streamer);

/* Copy `bytes` from pinned host `src` to device `dst` (the slot's buffer) once the GPU has
 * passed the slot's last mo_streamer_release point. Never blocks the host. Replaces
 * target.copy_(block.cpu_buffer, non_blocking=True) on the copy stream, memory.py:163-174. */
int mo_streamer_fill(mo_streamer* streamer, uint32_t slot, uint64_t dst, uint64_t src, uint64_t bytes);

/* Copy the slot's device contents `src` back to its pinned master `dst` once the GPU has passed
 * the slot's last mo_streamer_release point; the slot's next fill waits for this copy. Never
 * blocks the host. Replaces the dirty-slot eviction of TrainableBlockStreamer
 * (training/trainable_offload.py:245-260). */
int mo_streamer_writeback(mo_streamer* streamer, uint32_t slot, uint64_t dst, uint64_t src, uint64_t bytes);

/* Work enqueued on `stream` after this call sees the slot's last fill complete: the host waits
 * for the copy (bounded). Replaces compute_stream.wait_event(slot.ready), memory.py:246-247. */
int mo_streamer_acquire(mo_streamer* streamer, uint32_t slot, uint64_t stream);

/* The slot may be refilled once `stream` reaches this point. Replaces the slot.reusable events
 * of memory.py:193-225. */
int mo_streamer_release(mo_streamer* streamer, uint32_t slot, uint64_t stream);

/* ---- block ring: residency decided by the streamer (no reference counterpart as an ABI: the
 * reference keeps this state in Python, training/memory.py:142-191 and
 * training/trainable_offload.py:194-287). A block is identified by the caller's integer id and
 * its pinned master (host address and size); every slot is a device buffer the caller attaches.
 * A slot's generation counts its fills: calls naming a slot present the generation that
 * mo_streamer_stage returned and fail with MO_E_STATE once the slot holds another block. */

/* Give slot `slot` its device buffer of `capacity` bytes (dev 0 detaches an empty slot). */
int mo_streamer_attach(mo_streamer* streamer, uint32_t slot, uint64_t dev, uint64_t capacity);

/* Make block `block` resident: if a slot holds it, *slot names that slot and nothing is
 * copied (*filled = 0). Otherwise a slot is chosen (an empty one, else the least recently
 * staged one that is not pinned, does not hold `keep` and is large enough), its block is
 * written back first if the slot is dirty, and a fill of `bytes` from `host` is issued behind
 * the slot's last release point (*filled = 1). MO_E_STATE when no slot can be chosen. Never
 * blocks the host. Replaces AsyncBlockStreamer._stage (memory.py:157-191) and the eviction and
 * refill of TrainableBlockStreamer (trainable_offload.py:245-287). */
int mo_streamer_stage(mo_streamer* streamer, int64_t block, uint64_t host, uint64_t bytes, int64_t keep,
                      uint32_t* slot, uint64_t* generation, int* filled);

/* A running execution reads the slot: while pinned it is never chosen for another block. */
int mo_streamer_pin(mo_streamer* streamer, uint32_t slot, uint64_t generation);

/* The execution is done with the slot once `stream` gets here: drops one pin and records the
 * slot's release point (write-back and refill wait for it). */
int mo_streamer_unpin(mo_streamer* streamer, uint32_t slot, uint64_t generation, uint64_t stream);

/* Whether the slot's contents were updated on the device since its fill (copied back to the
 * block's master before the slot takes another block, or at mo_streamer_evict). */
int mo_streamer_mark_dirty(mo_streamer* streamer, uint32_t slot, uint64_t generation, int dirty);

/* Empty an unpinned slot (writing a dirty block back first). */
int mo_streamer_evict(mo_streamer* streamer, uint32_t slot);

/* The slot's block (-1 = none), pins, dirty flag and generation (any output may be NULL). */
int mo_streamer_slot_info(mo_streamer* streamer, uint32_t slot, int64_t* block, uint32_t* pins, int* dirty,
                          uint64_t* generation);

int mo_streamer_synchronize(mo_streamer* streamer);
int mo_streamer_get_stats(mo_streamer* streamer, mo_streamer_stats* stats);
int mo_streamer_reset_stats(mo_streamer* streamer);

/* ---- int8 weight-only linear (training/quant_kernels.py:100-228, quantization.py:27-65) ----- */

/* The decoded weight bf16(q * bf16(scale)) of an int8 weight [out_features][in_features] (fp32
 * per-row scale) written to `out` (bf16, same shape), on `stream`; in_features a multiple of 16,
 * weight and out 16-byte aligned. This is one pass in place of the reference eager path's decode
 * (quant_kernels.py:126-131, cast then scale). Calls with many rows take it and a library GEMM
 * instead of the fused kernels below. */
int mo_int8_decode(uint64_t w, uint64_t scale, uint64_t out, uint32_t out_features, uint32_t in_features,
                   uint64_t stream);

/* y[rows][out] = x[rows][in] . decode(w)^T (+ bias), on bf16 MFMA with fp32 accumulation, where
 * decode(w)[n][k] = bf16(w[n][k] * bf16(scale[n])), the decode of quant_kernels.py:126-131.
 * x, y, bias: bf16 (bias may be 0); w: int8 [out][in] row-major; scale: fp32 [out].
 * in_features and out_features multiples of 16, each at most 2^20, in * out < 2^31; x, w, y
 * 16-byte aligned. `workspace` (device, 16-byte aligned, at least
 * mo_int8_forward_workspace_bytes(rows, in, out) bytes; 0 = none) holds the fp32 partial sums
 * of the rows whose reduction the launch plan splits over several workgroups (rows that do not
 * fill a round of large tiles, on the default kernel); without one those rows take the small
 * tile. Enqueued on `stream` (one to three kernel launches), no allocation, no host
 * synchronisation. Replaces _int8_linear_forward_kernel (quant_kernels.py:100-157). */
int mo_int8_linear_forward(uint64_t x, uint64_t w, uint64_t scale, uint64_t bias, uint64_t y, uint32_t rows,
                           uint32_t in_features, uint32_t out_features, uint64_t workspace,
                           uint64_t workspace_bytes, uint64_t stream);
/* Bytes of workspace the forward's plan uses for this shape on the current device (0: none). */
uint64_t mo_int8_forward_workspace_bytes(uint32_t rows, uint32_t in_features, uint32_t out_features);

/* dx[rows][in] = dy[rows][out] . decode(w): the input gradient of the frozen int8 linear (no
 * weight gradient). Same layouts and constraints. `workspace` (device, 16-byte aligned, at
 * least mo_int8_backward_workspace_bytes(rows, in, out); 0 = none) receives the transposed int8
 * weight, which the large-tile kernel reads with the reduction contiguous, followed by the
 * partial sums of split reductions as in the forward; without one the large tile decodes the
 * weight through LDS instead (slower) and no reduction is split. Replaces
 * _int8_linear_backward_kernel (quant_kernels.py:160-209). */
int mo_int8_linear_backward(uint64_t dy, uint64_t w, uint64_t scale, uint64_t dx, uint32_t rows,
                            uint32_t in_features, uint32_t out_features, uint64_t workspace,
                            uint64_t workspace_bytes, uint64_t stream);
uint64_t mo_int8_backward_workspace_bytes(uint32_t rows, uint32_t in_features, uint32_t out_features);

/* Which kernel takes the large (256 x 256) tiles of the two calls above, process-wide:
 * MO_INT8_KERNEL_REGISTERS (default; reduction a multiple of 64): each wave decodes its columns'
 * int8 weights in registers into the MFMA operand, and the LDS carries only the activations;
 * MO_INT8_KERNEL_LDS: the weight tile is decoded into LDS and shared by the waves. Both give
 * the same results bit for bit on the rows the large tile computes; only the default splits
 * reductions (see mo_int8_linear_forward). The switch exists to measure one kernel against the
 * other. No reference counterpart (the reference has one Triton kernel per direction). */
enum { MO_INT8_KERNEL_REGISTERS = 0, MO_INT8_KERNEL_LDS = 1 };
int mo_int8_set_kernel(uint32_t kernel);

/* The launch plan of a call with a workspace, host only: `cols` output columns (out for the
 * forward, in for the input gradient) from a `reduction` (in, or out), on a device of `cus`
 * CUs with `kernel` taking the large tiles. Writes *n_parts (1 or 2) and, per part, five
 * values to parts[5 i ..]: tile (0 large, 1 small, 2 large with a split reduction), first row,
 * rows, splits, reduction steps of 64 per split. No reference counterpart: it describes this
 * library's launches, for tests and tools. */
int mo_int8_launch_plan(uint32_t rows, uint32_t cols, uint32_t reduction, uint32_t cus, uint32_t kernel,
                        uint32_t* n_parts, uint32_t* parts);

/* ---- host gradient accumulation (training/fused_adafactor.py:327-369) -------------------- */

/* Gradient element types: the reference's value-kind codes (quant_kernels.py:280-287). */
enum { MO_DTYPE_F16 = 0, MO_DTYPE_BF16 = 1, MO_DTYPE_F32 = 2 };

typedef struct mo_gradacc mo_gradacc;

typedef struct mo_gradacc_stats {
  uint64_t calls;          /* mo_gradacc_accumulate calls */
  uint64_t chunks;         /* staging-slot copies they issued */
  uint64_t bytes;          /* gradient bytes issued over the link */
  uint64_t elements;       /* elements accumulated on the host */
  uint64_t d2h_done_bytes; /* completed, timed D2H bytes */
  double d2h_ms;           /* SDMA busy time of those copies */
  double accumulate_ms;    /* host time converting and adding */
  uint64_t host_blocks;    /* calls that blocked the host (no free slot, or mo_gradacc_wait) */
  double host_block_ms;
  uint64_t pending_chunks; /* copies not yet accumulated */
  uint64_t copy_failures;
} mo_gradacc_stats;

/* An accumulator on `device`: `slots` device staging slots of `slot_bytes` (a multiple of 4096)
 * each with a pinned host twin, an SDMA D2H link on engines `d2h_engine` (bits, 0 = the two
 * lowest available; copies of 2 MiB or more are split across two), and `host_threads`
 * threads for the host additions. Replaces the blocking pinned copy of
 * FusedAdafactor._stash_gradient_on_host (fused_adafactor.py:337-346). */
int mo_gradacc_create(int device, uint32_t slots, uint64_t slot_bytes, uint32_t host_threads, uint32_t d2h_engine,
                      mo_gradacc** out);
/* Waits (bounded) for every pending accumulation, then frees the accumulator. */
int mo_gradacc_destroy(mo_gradacc* acc);
/* dst[i] = x[i] (first != 0) or dst[i] += x[i], i < count, where x = fp32(src) and src is a
 * device gradient of `dtype` and dst a host fp32 buffer (pinned or pageable). The gradient is
 * copied into staging slots on `stream` before the call returns, so the caller may free it
 * afterwards under the stream's ordering; the D2H and the host additions run in the
 * background, in call order, one IEEE fp32 add per element and call (the reference's
 * accumulated.add_(host_gradient), fused_adafactor.py:347-352). Blocks the host only while
 * every slot is in flight. `dst` must not be read or written until mo_gradacc_wait(acc, dst). */
int mo_gradacc_accumulate(mo_gradacc* acc, uint64_t dst, uint32_t first, uint64_t src, uint32_t dtype,
                          uint64_t count, uint64_t stream);
/* Block until every accumulation into `dst` (the `dst` a call passed; 0 = all) is complete. */
int mo_gradacc_wait(mo_gradacc* acc, uint64_t dst);
int mo_gradacc_get_stats(mo_gradacc* acc, mo_gradacc_stats* out);
int mo_gradacc_reset_stats(mo_gradacc* acc);

#ifdef __cplusplus
}
#endif

#endif /* MOSS_OFFLOAD_H */
