// Activation-offload engine: staging ring, pinned host pool, restore ring and the C ABI
// declared in include/moss_offload.h.
//
// Forward (replaces activation_offload.py:116-134, one pinned tensor + copy per save):
//   mo_pack gathers each saved tensor into the open segment of the device staging ring on the
//   caller's compute stream. A segment closes when its slot fills or its group (one block's
//   saves) is committed; the link then copies the whole segment to pinned host memory in one
//   transfer (SDMA engine by default). Pack kernels that refill a slot are enqueued only once
//   that slot's last D2H finished.
// Backward (replaces activation_offload.py:136-147, wait_event + _restore_layout):
//   mo_prefetch copies a group's segments into free restore slots ahead of use. mo_unpack
//   fetches whatever is missing, orders the unpack kernel after that copy, and scatters each
//   entry into its destination. Segments still intact in their staging slot skip the H2D.
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/moss_offload.h"
#include "mo_deferred.h"
#include "mo_internal.h"
#include "mo_link.h"

namespace mo {
namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int hip_fail(int e, const char* what) {
  g_error = std::string(what) + ": " + hipGetErrorName((hipError_t)e) + " (" + hipGetErrorString((hipError_t)e) + ")";
  return e;
}

}  // namespace

// Error setters shared with the other C-ABI translation units (mo_streamer.cpp).
int set_error(int code, const std::string& msg) { return fail(code, msg); }
int set_hip_error(int e, const char* what) { return hip_fail(e, what); }

namespace {

#define MO_HIP(call)                                       \
  do {                                                     \
    hipError_t _e = (call);                                \
    if (_e != hipSuccess) return hip_fail((int)_e, #call); \
  } while (0)

#define MO_LINK(call)                          \
  do {                                         \
    int _rc = (call);                          \
    if (_rc != 0) return hip_fail(_rc, #call); \
  } while (0)

constexpr uint64_t kNone = UINT64_MAX;
constexpr uint64_t kMinPiece = 1ull << 20;  // do not start a piece in less slot space than this
constexpr uint64_t kPieceAlign = 4096;      // split pieces at page multiples
constexpr uint64_t kHostAlign = 4096;

class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != device) (void)hipSetDevice(device);
    dev_ = device;
  }
  ~DeviceGuard() {
    if (prev_ >= 0 && prev_ != dev_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = -1, dev_ = -1;
};

// ------------------------------------------------------------------------------------------
// Pinned host pool: hipHostMalloc chunks, first-fit with coalescing, page-aligned blocks.
class HostPool {
 public:
  struct Chunk {
    char* base = nullptr;
    char* dev = nullptr;  // device-visible alias (for the copy kernel)
    uint64_t size = 0;
    uint64_t used = 0;
    std::map<uint64_t, uint64_t> free;  // offset -> size
  };

  void configure(uint64_t limit, uint64_t chunk) {
    limit_ = limit;
    chunk_ = chunk;
  }
  ~HostPool() { release_all(); }

  int alloc(uint64_t bytes, char** out) {
    bytes = align_up(bytes ? bytes : 1, kHostAlign);
    for (auto& c : chunks_) {
      for (auto it = c->free.begin(); it != c->free.end(); ++it) {
        if (it->second >= bytes) {
          const uint64_t off = it->first, sz = it->second;
          c->free.erase(it);
          if (sz > bytes) c->free.emplace(off + bytes, sz - bytes);
          c->used += bytes;
          account(bytes);
          *out = c->base + off;
          return 0;
        }
      }
    }
    const uint64_t size = align_up(std::max(bytes, chunk_), 2ull << 20);
    if (limit_ && reserved_ + size > limit_) {
      return fail(MO_E_HOST_OOM, "pinned host pool limit reached: reserved " + std::to_string(reserved_) + " B + " +
                                     std::to_string(size) + " B > limit " + std::to_string(limit_) +
                                     " B (raise host_limit_bytes or offload less)");
    }
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, size, hipHostMallocDefault);
    if (e != hipSuccess || !p) {
      return fail(MO_E_HOST_OOM, std::string("hipHostMalloc of ") + std::to_string(size) +
                                     " B failed: " + hipGetErrorString(e) + " (pinned host memory exhausted)");
    }
    void* dp = nullptr;
    if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess) dp = p;
    auto c = std::make_unique<Chunk>();
    c->base = (char*)p;
    c->dev = (char*)dp;
    c->size = size;
    if (size > bytes) c->free.emplace(bytes, size - bytes);
    c->used = bytes;
    reserved_ += size;
    account(bytes);
    *out = c->base;
    chunks_.push_back(std::move(c));
    return 0;
  }

  void free(char* p, uint64_t bytes) {
    bytes = align_up(bytes ? bytes : 1, kHostAlign);
    for (auto& c : chunks_) {
      if (p >= c->base && p < c->base + c->size) {
        uint64_t off = (uint64_t)(p - c->base), sz = bytes;
        auto next = c->free.lower_bound(off);
        if (next != c->free.end() && off + sz == next->first) {
          sz += next->second;
          next = c->free.erase(next);
        }
        if (next != c->free.begin()) {
          auto prev = std::prev(next);
          if (prev->first + prev->second == off) {
            off = prev->first;
            sz += prev->second;
            c->free.erase(prev);
          }
        }
        c->free.emplace(off, sz);
        c->used -= bytes;
        in_use_ -= bytes;
        return;
      }
    }
  }

  char* device_alias(char* p) const {
    for (auto& c : chunks_)
      if (p >= c->base && p < c->base + c->size) return c->dev + (p - c->base);
    return p;
  }

  void trim() {
    for (auto it = chunks_.begin(); it != chunks_.end();) {
      if ((*it)->used == 0) {
        (void)hipHostFree((*it)->base);
        reserved_ -= (*it)->size;
        it = chunks_.erase(it);
      } else {
        ++it;
      }
    }
  }

  void release_all() {
    for (auto& c : chunks_) (void)hipHostFree(c->base);
    chunks_.clear();
    reserved_ = in_use_ = 0;
  }

  uint64_t in_use() const { return in_use_; }
  uint64_t peak() const { return peak_; }
  void reset_peak() { peak_ = in_use_; }
  uint64_t reserved() const { return reserved_; }

 private:
  void account(uint64_t b) {
    in_use_ += b;
    peak_ = std::max(peak_, in_use_);
  }
  std::vector<std::unique_ptr<Chunk>> chunks_;
  uint64_t limit_ = 0, chunk_ = 1ull << 30;
  uint64_t reserved_ = 0, in_use_ = 0, peak_ = 0;
};

char* host_alias(void* ctx, char* p) { return ((HostPool*)ctx)->device_alias(p); }

// ------------------------------------------------------------------------------------------
struct Piece {
  uint32_t entry;
  uint64_t first;    // byte offset within the entry's payload
  uint64_t nbytes;
  uint64_t seg_off;  // byte offset within the segment
};

struct Segment {
  int stage_slot = -1;
  uint64_t stage_off = 0;
  uint64_t stage_gen = 0;          // fill generation of the staging slot when packed
  hipStream_t pack_stream = nullptr;
  bool one_stream = true;          // every piece was packed on pack_stream
  uint64_t bytes = 0;
  std::vector<Piece> pieces;
  char* host = nullptr;
  CopyRef d2h;  // the copy that filled `host`
  CopyRef h2d;  // the last copy that read `host`
  bool committed = false;
  bool prefetched = false;
  int restore_slot = -1;
  uint64_t restore_gen = 0;
  // Wire-coded: the host copy (host_bytes long, wire_max_coded(bytes)) holds the coded stream,
  // whose first u64 is its length; a fetch brings it into the restore slot's wire buffer and
  // the unpack decodes it into the slot first.
  bool wire = false;
  uint64_t host_bytes = 0;
};

struct Entry {
  Canon canon;
};

struct Group {
  uint64_t id = 0;
  bool open = true;
  uint64_t payload_bytes = 0;
  std::vector<Entry> entries;
  std::vector<Segment> segs;
};

struct StageSlot {
  char* dev = nullptr;
  uint64_t used = 0;
  uint64_t fill_gen = 0;  // bumped every time the slot is reset for refilling
  int gate = -1;
  char* wire = nullptr;    // coded streams of the slot's segments (wire coding)
  uint64_t wire_used = 0;  // reset with `used`
};

struct RestoreSlot {
  char* dev = nullptr;   // null until the slot is first used (restore_small_slots), or after mo_trim
  uint64_t cap = 0;      // bytes of `dev`: stage_slot_bytes, or small_cap for a small slot
  bool small = false;    // holds only raw segments of at most small_cap bytes
  bool dead = false;     // its allocation failed: not used again until mo_trim
  uint64_t group = kNone;
  uint32_t seg = 0;
  uint64_t gen = 0;
  uint64_t tick = 0;
  bool consumed = true;  // scattered at least once since fetched (or empty)
  int gate = -1;
  char* wire = nullptr;  // a coded segment's stream as fetched (wire coding)
  bool decoded = true;   // dev holds the fetched segment's raw bytes (once `join` completes)
  // Recorded on `used_on` after the slot's last decode and scatter: an unpack of the slot on
  // another stream waits for it first. Compared by handle only, never used as a stream.
  hipEvent_t join = nullptr;
  hipStream_t used_on = nullptr;
};

// Host ranges freed once their copies finish, and coded byte counts read once theirs finish
// (mo_deferred.h). A count's bytes are the first u64 of the host copy, known only after the
// coding kernels ran; a D2H names its segment, whose host copy then shrinks to the stream's
// length.
using Deferred = mo::DeferredHost<CopyRef>;
using PendingFree = Deferred::Free;
using PendingCount = Deferred::Count;

struct Timing {
  hipEvent_t start, end;
  uint64_t bytes;
  uint64_t hbm;
  bool pack;
};

bool idle(const CopyRef& c) { return !c || c->done(); }

}  // namespace

struct Engine {
  int device = 0;
  mo_config cfg{};
  std::mutex mu;
  std::unique_ptr<Link> link;
  std::vector<StageSlot> stage;
  std::vector<RestoreSlot> restore;
  int stage_cur = 0;
  HostPool pool;
  std::unordered_map<uint64_t, std::unique_ptr<Group>> groups;
  Group* open_group = nullptr;
  int open_seg = -1;  // index into open_group->segs, or -1
  uint64_t next_group = 0;
  uint64_t gen_counter = 0, tick = 0;
  std::vector<hipEvent_t> timing_pool;
  Deferred deferred;  // host frees and coded-byte counts waiting for their copies
  uint64_t wire_slot_bytes = 0;     // each staging slot's wire buffer, once allocated
  uint64_t wire_restore_bytes = 0;  // each restore slot's wire buffer, once allocated
  std::deque<Timing> timings;
  mo_stats st{};

  // ---- equality checks (mo_equal): a result word in pinned host memory + an event each ----
  static constexpr uint32_t kEqualSlots = 64;
  enum { kFree = 0, kRunning = 1, kAbandoned = 2 };
  struct EqualSlot {
    hipEvent_t ev = nullptr;
    uint64_t gen = 0;
    int state = kFree;
  };
  uint32_t* eq_flags = nullptr;  // kEqualSlots words, written by mo_equal_kernel
  EqualSlot eq[kEqualSlots];
  uint64_t eq_gen = 0;

  int equal(uint64_t a, uint64_t b, uint64_t nbytes, hipStream_t stream, uint64_t* ticket) {
    *ticket = 0;
    if (a % 16 || b % 16) return fail(MO_E_INVALID, "mo_equal: addresses must be 16-byte aligned");
    if (!eq_flags) {
      void* p = nullptr;
      MO_HIP(hipHostMalloc(&p, kEqualSlots * sizeof(uint32_t), hipHostMallocDefault));
      eq_flags = (uint32_t*)p;
    }
    int slot = -1;
    for (uint32_t i = 0; i < kEqualSlots && slot < 0; ++i) {
      if (eq[i].state == kAbandoned && hipEventQuery(eq[i].ev) == hipSuccess) eq[i].state = kFree;
      if (eq[i].state == kFree) slot = (int)i;
    }
    if (slot < 0) return 0;  // every slot waits for a result: no check, ticket 0
    EqualSlot& q = eq[slot];
    if (!q.ev) MO_HIP(hipEventCreateWithFlags(&q.ev, hipEventDisableTiming));
    eq_flags[slot] = 0;
    uint32_t* flag = nullptr;
    MO_HIP(hipHostGetDevicePointer((void**)&flag, eq_flags, 0));
    if (int rc = launch_equal((const void*)a, (const void*)b, nbytes, flag + slot, stream))
      return hip_fail(rc, "equality kernel launch");
    MO_HIP(hipEventRecord(q.ev, stream));
    q.gen = ++eq_gen;
    q.state = kRunning;
    *ticket = (q.gen << 8) | (uint64_t)slot;
    return 0;
  }

  EqualSlot* equal_slot(uint64_t ticket) {
    const uint64_t slot = ticket & 0xff;
    if (ticket == 0 || slot >= kEqualSlots || eq[slot].state != kRunning || eq[slot].gen != (ticket >> 8))
      return nullptr;
    return &eq[slot];
  }

  int equal_result(uint64_t ticket, int wait, int* state) {
    EqualSlot* q = equal_slot(ticket);
    if (!q) return fail(MO_E_INVALID, "mo_equal_result: unknown ticket " + std::to_string(ticket));
    if (wait) {
      MO_HIP(hipEventSynchronize(q->ev));
    } else {
      const hipError_t e = hipEventQuery(q->ev);
      if (e == hipErrorNotReady) {
        *state = 0;
        return 0;
      }
      if (e != hipSuccess) return hip_fail((int)e, "hipEventQuery (equality check)");
    }
    *state = eq_flags[q - eq] ? 2 : 1;
    q->state = kFree;
    return 0;
  }

  int equal_discard(uint64_t ticket) {
    EqualSlot* q = equal_slot(ticket);
    if (!q) return fail(MO_E_INVALID, "mo_equal_discard: unknown ticket " + std::to_string(ticket));
    q->state = kAbandoned;  // reused once its kernel has finished
    return 0;
  }

  // ---- pack/unpack kernel timing (MO_FLAG_KERNEL_TIMING) ----
  struct KernelTimer : LaunchTimer {
    Engine* e;
    bool pack;
    Timing cur{};
    KernelTimer(Engine* engine, bool p) : e(engine), pack(p) {}
    int events(hipEvent_t* start, hipEvent_t* stop) override {
      cur = Timing{nullptr, nullptr, 0, 0, pack};
      if (!(e->cfg.flags & MO_FLAG_KERNEL_TIMING)) return 0;
      for (hipEvent_t* ev : {&cur.start, &cur.end}) {
        if (!e->timing_pool.empty()) {
          *ev = e->timing_pool.back();
          e->timing_pool.pop_back();
        } else {
          hipError_t err = hipEventCreate(ev);
          if (err != hipSuccess) return (int)err;
        }
      }
      *start = cur.start;
      *stop = cur.end;
      return 0;
    }
    void launched(uint64_t bytes, uint64_t hbm) override {
      cur.bytes = bytes;
      cur.hbm = hbm;
      e->timings.push_back(cur);
      cur = Timing{nullptr, nullptr, 0, 0, pack};
    }
  };

  // ---- batched pack launches ----
  // Gather descriptors of consecutive mo_pack calls on one stream wait here and go out as one
  // launch when the open segment closes (before its D2H is issued), when a call comes on
  // another stream, or on synchronize / mo_pack_flush. The caller keeps each call's sources
  // valid until pack_launched reaches the call's number (mo_pack_progress).
  KernelTimer pack_timer{this, true};
  std::unique_ptr<Launcher> pend;
  hipStream_t pend_stream = nullptr;
  uint64_t pack_calls = 0;     // mo_pack calls so far (1-based numbers)
  uint64_t pack_launched = 0;  // every call numbered <= this has all its kernels enqueued
  bool in_pack = false;        // a flush inside a call leaves that call's later pieces pending

  // Launch the pending gathers, then issue the D2H of the committed segments that waited for
  // them (commit_batch_bytes), in commit order.
  int flush_packs() {
    if (pend) {
      const int rc = pend->flush();
      st.pack_launches += pend->launches();
      pend.reset();
      if (rc) return hip_fail(rc, "pack kernel launch");
    }
    pack_launched = in_pack ? pack_calls - 1 : pack_calls;
    std::vector<Closing> waiting;
    waiting.swap(closing);
    closing_bytes = 0;
    for (const Closing& c : waiting) {
      Group* g = find(c.group);
      if (!g) continue;  // release() flushes first, so this does not happen
      if (int rc = issue_d2h(*g, c.seg, c.stream)) return rc;
    }
    return 0;
  }

  // Segments closed by mo_commit whose gathers (and so D2H) wait for later commits.
  struct Closing {
    uint64_t group;
    uint32_t seg;
    hipStream_t stream;
  };
  std::vector<Closing> closing;
  uint64_t closing_bytes = 0;

  // The open group is released before its D2H: its pending gathers never need to run.
  void discard_packs() {
    if (pend) st.pack_launches += pend->launches();
    pend.reset();
    pack_launched = pack_calls;
  }

  Launcher& pack_launcher(hipStream_t stream) {
    if (!pend) {
      pend.reset(new Launcher(true, stream, &pack_timer));
      pend_stream = stream;
    }
    return *pend;
  }

  void process_timings(bool wait) {
    while (!timings.empty()) {
      Timing& t = timings.front();
      if (wait) (void)hipEventSynchronize(t.end);
      else if (hipEventQuery(t.end) != hipSuccess) break;
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, t.start, t.end) == hipSuccess) {
        if (t.pack) {
          st.pack_ms += ms;
          st.timed_pack_bytes += t.bytes;
          st.timed_pack_hbm_bytes += t.hbm;
          st.timed_pack_launches++;
        } else {
          st.unpack_ms += ms;
          st.timed_unpack_bytes += t.bytes;
          st.timed_unpack_hbm_bytes += t.hbm;
          st.timed_unpack_launches++;
        }
      }
      timing_pool.push_back(t.start);
      timing_pool.push_back(t.end);
      timings.pop_front();
    }
  }

  // A failed copy still releases whoever waits on it (no hang); report it at the next call.
  uint64_t seen_failures = 0;
  int check_link() {
    LinkStats ls;
    link->stats(&ls);
    if (ls.failures > seen_failures) {
      seen_failures = ls.failures;
      return fail(MO_E_STATE, "a host-link copy failed; offloaded data may be lost");
    }
    return 0;
  }

  // ---- deferred host frees ----
  // Count the coded bytes of every wire-coded copy that has completed. With `wait`, first wait
  // (at most 300 s) for all of them.
  void process_counts(bool wait) {
    if (wait) wait_copies(false);
    deferred.settle_counts(idle, [this](const PendingCount& c) { count(c); });
  }

  void count(const PendingCount& c) {
    if (c.copy && c.copy->failed()) return;
    uint64_t total = 0;
    memcpy(&total, c.host, sizeof(total));
    (c.d2h ? st.bytes_d2h : st.bytes_h2d) += total;
    if (c.d2h) {
      st.wire_bytes += total;
      shrink_host(c, total);
    }
  }

  // Poll until every copy the deferred work refers to has finished (only the counts' copies
  // unless `frees`); false after 300 s.
  bool wait_copies(bool frees) {
    const auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(300);
    auto busy = [&] {
      if (frees) return !deferred.all_done(idle);
      for (const PendingCount& c : deferred.counts)
        if (!idle(c.copy)) return true;
      return false;
    };
    while (busy()) {
      if (std::chrono::steady_clock::now() > deadline) return false;
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    return true;
  }

  // A coded segment's host copy was sized for its largest stream; once the stream's length is
  // known the rest of the copy goes back to the pool. The D2H (issued once the coding kernels
  // have run) and any fetch copy only the stream's length, so neither touches what is freed.
  // The length is known when the coding kernels have completed (early_shrinks), long before
  // the D2H lands on a link-bound forward, whose queue holds several segments: shrunk only at
  // D2H completion, each copy left a hole of a third of a slot behind the next segment's copy,
  // and config 4 not checkpointed reserved 62 GiB of pinned memory for 42.6 GiB in use.
  void shrink_host(const PendingCount& c, uint64_t total) {
    Group* g = find(c.group);
    if (!g || c.seg >= g->segs.size()) return;  // released meanwhile: freed whole
    Segment& seg = g->segs[c.seg];
    if (seg.host != c.host || !seg.wire || total > seg.host_bytes) return;
    const uint64_t held = align_up(seg.host_bytes, kHostAlign);
    const uint64_t keep = align_up(std::max<uint64_t>(total, 16), kHostAlign);
    if (keep >= held) return;
    pool.free(seg.host + keep, held - keep);
    seg.host_bytes = keep;
  }

  // Coded segments whose host copy still has its largest size, with an event recorded after
  // their coding kernels: once it has completed, the stream's length is in the copy's first u64.
  struct PendingShrink {
    uint64_t group;
    uint32_t seg;
    const char* host;
    hipEvent_t coded;
  };
  std::deque<PendingShrink> shrinks;
  std::vector<hipEvent_t> shrink_events;  // idle events for PendingShrink::coded
  void early_shrinks() {
    for (auto it = shrinks.begin(); it != shrinks.end();) {
      const hipError_t q = hipEventQuery(it->coded);
      if (q == hipErrorNotReady) {
        ++it;
        continue;
      }
      if (q == hipSuccess) {
        // the group and its host copy must still be there before the copy is read
        const Group* g = find(it->group);
        if (g && it->seg < g->segs.size() && g->segs[it->seg].host == it->host && g->segs[it->seg].wire) {
          uint64_t total = 0;
          memcpy(&total, it->host, sizeof(total));
          shrink_host(PendingCount{it->host, CopyRef{}, true, it->group, it->seg}, total);
        }
      } else {
        (void)hipGetLastError();  // a failed query only forgoes the early shrink
      }
      shrink_events.push_back(it->coded);
      it = shrinks.erase(it);
    }
  }

  // Settle the counts and free the host ranges whose copies have finished; with `wait`, all of
  // them (at most 300 s).
  int process_pending(bool wait) {
    early_shrinks();
    const bool finished = !wait || wait_copies(true);
    deferred.settle(idle, [this](const PendingCount& c) { count(c); },
                    [this](char* host, uint64_t bytes) { pool.free(host, bytes); });
    return finished ? 0 : fail(MO_E_STATE, "copies did not finish in 300 s");
  }

  // ---- forward ----
  // Close the open segment and send it: launch the pending gathers, then its D2H. With
  // `deferrable` (a commit), while the link is not behind and no coding is asked for, the
  // segment may instead wait, gathers and all, for later commits' (commit_batch_bytes); a
  // later flush sends them together. *deferred says which happened.
  int close_segment(hipStream_t stream, bool deferrable = false, bool* deferred = nullptr) {
    if (deferred) *deferred = false;
    if (!open_group || open_seg < 0) return 0;
    const uint32_t si = (uint32_t)open_seg;
    Segment& seg = open_group->segs[si];
    seg.bytes = stage[seg.stage_slot].used - seg.stage_off;
    open_seg = -1;
    if (deferrable && cfg.commit_batch_bytes && pend && pend_stream == stream && !link_behind &&
        !(cfg.flags & MO_FLAG_WIRE_CODING) && closing_bytes + seg.bytes < cfg.commit_batch_bytes) {
      closing.push_back(Closing{open_group->id, si, stream});
      closing_bytes += seg.bytes;
      if (deferred) *deferred = true;
      return 0;
    }
    if (int rc = flush_packs()) return rc;
    return issue_d2h(*open_group, si, stream);
  }

  // The D2H of a closed segment whose gathers are launched (coded first if the link is behind).
  int issue_d2h(Group& g, uint32_t si, hipStream_t stream) {
    Segment& seg = g.segs[si];
    StageSlot& slot = stage[seg.stage_slot];
    const uint64_t gid = g.id;
    if (wire_wanted(seg.bytes) && wire_ready()) {
      const uint64_t cap = wire_capacity(seg.bytes);
      if (slot.wire_used + cap <= wire_slot_bytes) {
        char* w = slot.wire + slot.wire_used;
        const uint64_t most = wire_max_coded(seg.bytes);  // the stream; the working space stays on the device
        early_shrinks();  // earlier segments' unused tails go back before this copy is placed
        if (int rc = pool.alloc(most, &seg.host)) return rc;
        seg.host_bytes = most;
        // the coded length goes straight to the host copy's first u64, where the copy engine's
        // issuer reads it once the coding kernels have completed
        MO_HIP((hipError_t)wire_encode((uint64_t)(slot.dev + seg.stage_off), seg.bytes, (uint64_t)w, cap,
                                        (uint64_t)seg.host, stream));
        {
          hipEvent_t ev = nullptr;
          if (!shrink_events.empty()) {
            ev = shrink_events.back();
            shrink_events.pop_back();
          } else if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
            ev = nullptr;
            (void)hipGetLastError();  // no early shrink for this one: it shrinks when its D2H lands
          }
          if (ev && hipEventRecord(ev, stream) == hipSuccess) {
            shrinks.push_back(PendingShrink{gid, si, seg.host, ev});
          } else if (ev) {
            (void)hipGetLastError();
            shrink_events.push_back(ev);
          }
        }
        MO_LINK(link->d2h_sized(seg.host, w, (const volatile uint64_t*)seg.host, most, stream, slot.gate, &seg.d2h));
        slot.wire_used += (cap + 255) & ~uint64_t(255);
        seg.wire = true;
        seg.committed = true;
        st.d2h_copies++;
        st.wire_segments++;
        st.wire_raw_bytes += seg.bytes;
        deferred.counts.push_back(PendingCount{seg.host, seg.d2h, true, gid, si});
        return 0;
      }
    }
    if (int rc = pool.alloc(seg.bytes, &seg.host)) return rc;
    seg.host_bytes = seg.bytes;
    MO_LINK(link->d2h(seg.host, slot.dev + seg.stage_off, seg.bytes, stream, slot.gate, &seg.d2h));
    seg.committed = true;
    st.d2h_copies++;
    st.bytes_d2h += seg.bytes;
    return 0;
  }

  // Whether to code a closing segment: MO_FLAG_WIRE_CODING codes every segment of at least
  // kWireMinBytes; MO_FLAG_WIRE_AUTO once the link is behind in this forward: the staging ring
  // came round, twice in a row, to a slot whose D2H was still on the copy engines (issued, not
  // finished), so the pack had to wait for the link, not for the GPU to reach the copy. It
  // stays on until the next unpack (the backward has begun). A checkpointed step's few MB per
  // block leave the ring idle (at most a lone wrap lands on a copy just issued) and are not
  // coded; a non-checkpointed forward fills the ring within a few blocks and codes from then
  // on. Only a transport that sizes copies at issue can carry coded segments.
  static constexpr uint64_t kWireMinBytes = 256ull << 10;
  bool link_behind = false;
  int busy_wraps = 0;  // consecutive slot advances that found the slot's D2H on the engines
  bool wire_wanted(uint64_t bytes) {
    if (!(cfg.flags & (MO_FLAG_WIRE_CODING | MO_FLAG_WIRE_AUTO)) || bytes < kWireMinBytes || bytes > kWireMaxRaw)
      return false;
    if (!link->sized_copies()) return false;
    if (!(cfg.flags & MO_FLAG_WIRE_CODING) && !link_behind) return false;
    if (wire_unavailable) {
      st.wire_fallbacks++;
      return false;
    }
    return true;
  }

  // Wire buffers, allocated on first use: one per staging slot (the coded streams of its
  // segments, each followed by the coder's working space) and one per restore slot (a fetched
  // stream, at most wire_max_coded of a slot).
  // They are an optimisation, so the step never fails for want of them: where they would pass
  // cfg.wire_device_limit or an allocation fails (the HIP error is cleared, the buffers made so
  // far stay for the next attempt), segments cross raw until the next forward tries again.
  bool wire_unavailable = false;
  bool wire_ready() {
    if (wire_slot_bytes) return true;
    const uint64_t bytes = ((wire_capacity(cfg.stage_slot_bytes) + cfg.stage_slot_bytes / 64 + (2ull << 20)) + 4095) &
                           ~uint64_t(4095);
    const uint64_t fetched = (wire_max_coded(cfg.stage_slot_bytes) + 4095) & ~uint64_t(4095);
    bool ok = !cfg.wire_device_limit || bytes * stage.size() + fetched * big_slots() <= cfg.wire_device_limit;
    for (auto& s : stage)
      if (ok && !s.wire && hipMalloc(&s.wire, bytes) != hipSuccess) {
        s.wire = nullptr;
        ok = false;
      }
    // full-size restore slots that hold memory; one given its memory later gets its wire
    // buffer with it (alloc_restore)
    for (auto& r : restore)
      if (ok && r.dev && !r.small && !r.wire && hipMalloc(&r.wire, fetched) != hipSuccess) {
        r.wire = nullptr;
        ok = false;
      }
    if (!ok) {
      (void)hipGetLastError();
      wire_unavailable = true;
      st.wire_fallbacks++;
      return false;
    }
    wire_slot_bytes = bytes;
    wire_restore_bytes = fetched;
    return true;
  }

  int advance_slot(hipStream_t stream) {
    // segments waiting for their gathers (commit_batch_bytes) go out before the ring moves on:
    // the slot reached next may hold some of them, and its wait below covers only copies
    // already issued
    if (!closing.empty())
      if (int rc = flush_packs()) return rc;
    stage_cur = (stage_cur + 1) % (int)stage.size();
    StageSlot& s = stage[stage_cur];
    st.stage_slot_waits++;
    busy_wraps = link->link_busy(s.gate) ? busy_wraps + 1 : 0;
    if (busy_wraps >= 2) link_behind = true;
    MO_LINK(link->wait(s.gate, stream));
    s.used = 0;
    s.wire_used = 0;
    s.fill_gen++;
    return 0;
  }

  // A committed segment whose staging bytes have not been overwritten since it was packed on
  // `stream` can be unpacked from the staging slot itself: no H2D needed. (Its D2H still ran,
  // so the host copy remains the reference once the slot is refilled.)
  bool staged(const Segment& seg, hipStream_t stream) const {
    return (cfg.flags & MO_FLAG_NO_STAGED_RESTORE) == 0 && seg.committed && seg.stage_slot >= 0 &&
           stage[seg.stage_slot].fill_gen == seg.stage_gen && seg.one_stream && seg.pack_stream == stream;
  }

  // Cache policy of the pack and unpack kernels (KDesc::cache). Pack writes the staging slot
  // with streaming stores (read next by a DMA engine). Unpack reads the restore slot with
  // non-temporal loads (read once) and writes the restored tensors with streaming stores.
  // Measured on the config-2 block set and in the config-3 step: non-temporal unpack loads
  // raise unpack by 3-4 % in both; non-temporal pack loads help the isolated block set but
  // slow pack in the step, where the saves are read while the forward still uses them.
  // The flags flip each choice for measurement.
  uint8_t pack_cache() const {
    return kCacheNtStore | ((cfg.flags & MO_FLAG_PACK_NT_LOAD) ? kCacheNtLoad : 0);
  }
  uint8_t unpack_cache() const {
    return ((cfg.flags & MO_FLAG_UNPACK_CACHED_LOAD) ? 0 : kCacheNtLoad) |
           ((cfg.flags & MO_FLAG_UNPACK_CACHED_STORE) ? 0 : kCacheNtStore);
  }

  int pack(const mo_tensor* ts, int n, hipStream_t stream, mo_ref* refs) {
    if (int rc = check_link()) return rc;
    process_pending(false);
    std::vector<Canon> canons(n);
    std::string err;
    for (int i = 0; i < n; ++i) {
      if (int rc = canonicalize(ts[i], canons[i], err))
        return fail(rc, "mo_pack: tensor " + std::to_string(i) + ": " + err);
    }
    if (!open_group) {
      auto g = std::make_unique<Group>();
      g->id = next_group++;
      open_group = g.get();
      groups.emplace(g->id, std::move(g));
      open_seg = -1;
      st.groups_created++;
    }
    Group& g = *open_group;
    if (pend && pend_stream != stream)
      if (int rc = flush_packs()) return rc;
    ++pack_calls;
    in_pack = true;
    const int rc = pack_into(g, canons, stream, refs);
    in_pack = false;
    if (rc) return rc;
    if (cfg.flags & MO_FLAG_EAGER_PACK) return flush_packs();
    if (!pend) pack_launched = pack_calls;  // nothing of this call is pending
    return 0;
  }

  int pack_into(Group& g, const std::vector<Canon>& canons, hipStream_t stream, mo_ref* refs) {
    std::string err;
    const int n = (int)canons.size();
    const uint64_t slot_bytes = cfg.stage_slot_bytes;
    for (int i = 0; i < n; ++i) {
      const Canon& c = canons[i];
      const uint32_t idx = (uint32_t)g.entries.size();
      g.entries.push_back(Entry{c});
      g.payload_bytes += c.nbytes;
      refs[i].group = g.id;
      refs[i].entry = idx;
      refs[i].reserved = 0;
      uint64_t remaining = c.nbytes, first = 0;
      while (remaining > 0) {
        StageSlot& s = stage[stage_cur];
        const uint64_t pos = align_up(s.used, kPayloadAlign);
        const uint64_t space = pos < slot_bytes ? slot_bytes - pos : 0;
        if (space == 0 || (space < remaining && space < kMinPiece)) {
          if (int rc = close_segment(stream)) return rc;
          if (int rc = advance_slot(stream)) return rc;
          continue;
        }
        if (open_seg < 0) {
          Segment seg;
          seg.stage_slot = stage_cur;
          seg.stage_off = pos;
          seg.stage_gen = s.fill_gen;
          seg.pack_stream = stream;
          g.segs.push_back(std::move(seg));
          open_seg = (int)g.segs.size() - 1;
        }
        Segment& seg = g.segs[open_seg];
        if (seg.pack_stream != stream) seg.one_stream = false;
        uint64_t take = std::min(remaining, space);
        if (take < remaining) take = take / kPieceAlign * kPieceAlign;
        KDesc kd;
        if (int rc = make_kdesc(c, c.base, first, take, (uint64_t)(s.dev + pos), kd, err))
          return fail(rc, "mo_pack: " + err);
        kd.cache = pack_cache();
        if (pend && pend->full())  // launch through flush_packs so pack_launched stays exact
          if (int rc = flush_packs()) return rc;
        Launcher& L = pack_launcher(stream);
        L.add(kd);
        if (L.status()) return hip_fail(L.status(), "pack kernel launch");
        seg.pieces.push_back(Piece{idx, first, take, pos - seg.stage_off});
        s.used = pos + take;
        first += take;
        remaining -= take;
        st.bytes_packed += take;
      }
    }
    return 0;
  }

  int commit(hipStream_t stream, uint64_t* gid) {
    *gid = kNone;
    // no open group: nothing to close; committed segments that wait keep waiting
    if (!open_group) return closing.empty() ? flush_packs() : 0;
    bool waits = false;
    if (int rc = close_segment(stream, true, &waits)) return rc;
    // a group with no segment yet launches what is pending, unless commits are gathering
    if (!waits && closing.empty())
      if (int rc = flush_packs()) return rc;
    open_group->open = false;
    *gid = open_group->id;
    grow_rings(*open_group);
    open_group = nullptr;
    open_seg = -1;
    return 0;
  }

  // ---- backward ----
  Group* find(uint64_t gid) {
    auto it = groups.find(gid);
    return it == groups.end() ? nullptr : it->second.get();
  }

  bool resident(const Group& g, uint32_t si) const {
    const Segment& seg = g.segs[si];
    if (seg.restore_slot < 0) return false;
    const RestoreSlot& r = restore[seg.restore_slot];
    return r.group == g.id && r.seg == si && r.gen == seg.restore_gen;
  }

  // Restore slots a segment of `g` may take: all of them for raw segments; for wire-coded ones
  // the first max(kCodedSlotsMin, segments of g + 2). Measured on MI355X with sixteen slots,
  // non-checkpointed steps, alternating runs on one box: at 1024² (about six coded segments a
  // block) eight slots for coded segments run 0.653 s/it against 0.665 with all sixteen; at
  // 2048² (about 25 a block, more than the ring) all sixteen run 2.60 against 2.88 with eight.
  // Checkpointed steps code nothing and keep the whole ring.
  // (Counted over the full-size slots in ring order; small slots never hold coded segments.)
  static constexpr int kCodedSlotsMin = 8;
  int slot_limit(const Group& g, uint32_t si) const {
    if (!g.segs[si].wire) return kMaxSlots;
    return std::max(kCodedSlotsMin, (int)g.segs.size() + 2);
  }

  // Small restore slots (restore_small_slots): a checkpointed block's inputs (28 MB at 1024^2)
  // in a 32 MiB slot rather than a 128 MiB one.
  uint64_t small_cap = 0;  // bytes of a small slot; 0: no small slots
  bool small_fit(const Segment& seg) const { return small_cap && !seg.wire && seg.bytes <= small_cap; }
  size_t big_slots() const {
    size_t n = 0;
    for (const RestoreSlot& r : restore) n += !r.small;
    return n;
  }

  // Give restore slot k its device memory (and its wire buffer while coding's buffers exist).
  // On failure the HIP error is cleared and the slot is left alone until mo_trim.
  bool alloc_restore(int k) {
    RestoreSlot& r = restore[k];
    DeviceGuard guard(device);
    if (hipMalloc(&r.dev, r.cap) != hipSuccess) r.dev = nullptr;
    if (r.dev && !r.small && wire_restore_bytes && hipMalloc(&r.wire, wire_restore_bytes) != hipSuccess) {
      r.wire = nullptr;
      (void)hipFree(r.dev);
      r.dev = nullptr;
    }
    if (r.dev) return true;
    (void)hipGetLastError();
    r.dead = true;
    return false;
  }

  // Choose a restore slot for segment `si` of group `g`: a small slot only for a segment that
  // fits one, a full-size one only among the first slot_limit of them. By rank, then least
  // recently used:
  //   a segment that fits a small slot: small and empty, small without memory yet, full-size
  //     and empty, small in use, full-size in use, full-size without memory yet;
  //   any other: empty, without memory yet, in use.
  // A slot without memory gets it here. for_prefetch: only slots that are empty or already
  // consumed (a prefetch never evicts data that is still waiting for use), and no full-size
  // slot is given memory for a segment that fits a small one.
  int pick_slot(const Group& g, uint32_t si, bool for_prefetch) {
    const bool fits_small = small_fit(g.segs[si]);
    const int limit = slot_limit(g, si);
    auto rank = [&](const RestoreSlot& r) -> int {
      if (!r.dev) return r.small ? 1 : fits_small ? (for_prefetch ? -1 : 5) : 1;
      if (r.group == kNone) return r.small ? 0 : fits_small ? 2 : 0;
      if (for_prefetch && !r.consumed) return -1;
      return r.small ? 3 : fits_small ? 4 : 2;
    };
    for (;;) {
      int best = -1, best_rank = 0, big = 0;
      for (int k = 0; k < (int)restore.size(); ++k) {
        const RestoreSlot& r = restore[k];
        if (r.small ? !fits_small : big++ >= limit) continue;
        if (r.dead) continue;
        if (r.group == g.id && r.seg > si && !r.consumed) continue;  // a later segment of g, still to be read
        const int rk = rank(r);
        if (rk < 0) continue;
        if (best < 0 || rk < best_rank || (rk == best_rank && r.tick < restore[best].tick)) {
          best = k;
          best_rank = rk;
        }
      }
      if (best < 0 && !for_prefetch) {
        // Every slot it may take holds a later, unconsumed segment of g: evict the furthest one.
        uint32_t far = 0;
        big = 0;
        for (int k = 0; k < (int)restore.size(); ++k) {
          const RestoreSlot& r = restore[k];
          if (r.small ? !fits_small : big++ >= limit) continue;
          if (r.dev && r.group == g.id && r.seg >= far) {
            far = r.seg;
            best = k;
          }
        }
      }
      if (best < 0 || restore[best].dev || alloc_restore(best)) return best;
      // that slot could not be given memory (now dead): choose again
    }
  }

  int fetch(Group& g, uint32_t si, int k) {
    Segment& seg = g.segs[si];
    RestoreSlot& r = restore[k];
    if (!seg.committed || !seg.host)
      return fail(MO_E_STATE, "group " + std::to_string(g.id) + " segment " + std::to_string(si) +
                                  " has no host copy (its D2H was never issued)");
    if (!r.dev || seg.bytes > r.cap || (seg.wire && !r.wire))
      return fail(MO_E_STATE, "restore slot " + std::to_string(k) + " cannot hold group " + std::to_string(g.id) +
                                  " segment " + std::to_string(si));
    CopyRef copy;
    if (seg.wire) {
      MO_LINK(link->h2d_sized(r.wire, seg.host, (const volatile uint64_t*)seg.host, seg.host_bytes, seg.d2h, r.gate,
                              &copy));
      deferred.counts.push_back(PendingCount{seg.host, copy, false, 0, 0});
      r.decoded = false;
    } else {
      MO_LINK(link->h2d(r.dev, seg.host, seg.bytes, seg.d2h, r.gate, &copy));
      st.bytes_h2d += seg.bytes;
      r.decoded = true;
    }
    seg.h2d = std::move(copy);
    r.used_on = nullptr;  // the H2D was ordered after the slot's consumed point
    r.group = g.id;
    r.seg = si;
    r.gen = ++gen_counter;
    r.tick = ++tick;
    r.consumed = false;
    seg.restore_slot = k;
    seg.restore_gen = r.gen;
    st.h2d_copies++;
    return 0;
  }

  // entry: only the segments holding a piece of that entry (kAllEntries: every segment).
  static constexpr uint32_t kAllEntries = 0xffffffffu;
  int prefetch(uint64_t gid, hipStream_t stream, uint32_t entry = kAllEntries) {
    if (!closing.empty())
      if (int rc = flush_packs()) return rc;
    process_pending(false);
    Group* g = find(gid);
    if (!g) return fail(MO_E_INVALID, "mo_prefetch: unknown group " + std::to_string(gid));
    if (entry != kAllEntries && entry >= g->entries.size())
      return fail(MO_E_INVALID, "mo_prefetch_entry: group " + std::to_string(gid) + " has no entry " +
                                    std::to_string(entry));
    if (g->open) return 0;
    for (uint32_t si = 0; si < g->segs.size(); ++si) {
      if (entry != kAllEntries) {
        bool holds = false;
        for (const Piece& p : g->segs[si].pieces) holds = holds || p.entry == entry;
        if (!holds) continue;
      }
      if (resident(*g, si) || staged(g->segs[si], stream)) continue;
      const int k = pick_slot(*g, si, true);
      if (k < 0) break;
      if (int rc = fetch(*g, si, k)) return rc;
      g->segs[si].prefetched = true;
      st.prefetch_issued++;
    }
    return 0;
  }

  // Groups in the order backward will need them: the first as far as free slots allow (as
  // prefetch), each later one only if every segment it still needs gets a free slot now, so a
  // farther group never takes a slot a nearer one will need. Stops at the first that does not.
  int prefetch_groups(const uint64_t* gids, uint32_t n, hipStream_t stream) {
    if (n == 0) return 0;
    if (int rc = prefetch(gids[0], stream)) return rc;
    for (uint32_t k = 1; k < n; ++k) {
      Group* g = find(gids[k]);
      if (!g) return fail(MO_E_INVALID, "mo_prefetch_groups: unknown group " + std::to_string(gids[k]));
      if (g->open) return 0;
      // segments to fetch: `small` that fit a small slot, `big` that do not, of them `coded`
      // confined to the first `low` full-size slots
      uint32_t small = 0, big = 0, coded = 0;
      int low = kMaxSlots;
      for (uint32_t si = 0; si < g->segs.size(); ++si) {
        const Segment& seg = g->segs[si];
        if (resident(*g, si) || staged(seg, stream)) continue;
        if (small_fit(seg)) {
          ++small;
          continue;
        }
        ++big;
        if (seg.wire) {
          ++coded;
          low = std::min(low, slot_limit(*g, si));
        }
      }
      // free slots (empty or consumed): small ones, full-size ones (a prefetch gives memory to a
      // full-size slot only for a segment that needs one), of those with memory and of the
      // first `low`
      uint32_t free_small = 0, free_big = 0, free_big_mem = 0, free_low = 0;
      int nbig = 0;
      for (const RestoreSlot& r : restore) {
        const bool free = !r.dead && (r.group == kNone || r.consumed);
        if (r.small) {
          free_small += free;
          continue;
        }
        if (free) {
          ++free_big;
          free_big_mem += r.dev != nullptr;
          free_low += nbig < low;
        }
        ++nbig;
      }
      // small segments take small slots, then full-size ones with memory the others leave
      const uint32_t big_left = free_big_mem > big ? free_big_mem - big : 0;
      if (big > free_big || coded > free_low || small > free_small + big_left) return 0;
      if (int rc = prefetch(gids[k], stream)) return rc;
    }
    return 0;
  }

  // Restore group gids[0] into dst[0 .. counts[0]) (an entry with a zero address is skipped),
  // fetching what is missing; then each further group gids[k], into the next counts[k]
  // addresses, if every segment it needs can be read right now without a wait: resident in a
  // restore slot with its H2D landed, or still in its staging slot. unpacked[k] says which were.
  // The first group's segments are scattered one by one, each flushed and its slot released
  // before the next segment may fetch (and so take a slot); its last segment's pieces and the
  // further groups' go out together, in as few launches as the pieces allow. The further
  // groups never fetch, so no slot with a scatter still pending is ever refilled.
  int unpack_groups(const uint64_t* gids, const uint64_t* dst, const uint32_t* counts, uint32_t n,
                    hipStream_t stream, uint32_t* unpacked) {
    if (int rc = check_link()) return rc;
    if (!closing.empty())  // segments waiting for their gathers go out before any is read
      if (int rc = flush_packs()) return rc;
    link_behind = false;
    busy_wraps = 0;
    wire_unavailable = false;  // the next forward may try to allocate the wire buffers again
    process_pending(false);
    for (uint32_t k = 0; k < n; ++k) {
      unpacked[k] = 0;
      const Group* g = find(gids[k]);
      if (!g) return fail(MO_E_INVALID, "mo_unpack: unknown group " + std::to_string(gids[k]));
      if (counts[k] != g->entries.size())
        return fail(MO_E_INVALID, "mo_unpack: group " + std::to_string(gids[k]) + " has " +
                                      std::to_string(g->entries.size()) + " entries, got " + std::to_string(counts[k]));
    }
    KernelTimer timer(this, false);
    Launcher L(false, stream, &timer);
    std::vector<RestoreSlot*> pending;  // slots whose scatter is added but not yet released
    auto release_pending = [&]() -> int {
      const int rc = L.flush();
      for (RestoreSlot* r : pending) {
        MO_LINK(link->consumed(r->gate, stream));
        if (!r->join) MO_HIP(hipEventCreateWithFlags(&r->join, hipEventDisableTiming));
        MO_HIP(hipEventRecord(r->join, stream));
        r->used_on = stream;
        r->consumed = true;
        r->tick = ++tick;
      }
      pending.clear();
      return rc ? hip_fail(rc, "unpack kernel launch") : 0;
    };
    int rc = 0;
    uint64_t off = 0;
    for (uint32_t k = 0; k < n && !rc; off += counts[k], ++k) {
      Group* g = find(gids[k]);
      if (k > 0) {
        const int why = not_ready(*g, dst + off, stream);
        if (why == 1) st.ahead_not_resident++;
        if (why == 2) st.ahead_in_flight++;
        if (why) continue;
        st.ahead_restored++;
      }
      if (g->open) {
        uint64_t id;
        if ((rc = commit(stream, &id))) break;
      }
      for (uint32_t si = 0; si < g->segs.size() && !rc; ++si) {
        if (k == 0 && !pending.empty() && (rc = release_pending())) break;
        rc = scatter_segment(*g, si, dst + off, stream, k == 0, L, pending);
      }
      if (!rc) unpacked[k] = 1;
    }
    const int rc2 = release_pending();
    st.unpack_launches += L.launches();
    return rc ? rc : rc2;
  }

  // 0 when every segment of `g` with a destination in `dst` can be scattered on `stream` now,
  // with at most a short wait: staged, or resident with its H2D landed or started (on the
  // SDMA link: handed to the engine, so the wait is at most the transfer of what is queued
  // ahead of it; on HIP streams: the GPU waits); else 1 (open, or a segment not in a restore
  // slot) or 2 (a segment's H2D still waiting for the GPU to free its slot).
  int not_ready(const Group& g, const uint64_t* dst, hipStream_t stream) const {
    if (g.open) return 1;
    int why = 0;
    for (uint32_t si = 0; si < g.segs.size(); ++si) {
      const Segment& seg = g.segs[si];
      bool any = false;
      for (const Piece& p : seg.pieces) any = any || dst[p.entry] != 0;
      if (!any || staged(seg, stream)) continue;
      if (!resident(g, si)) return 1;
      if (seg.h2d && !seg.h2d->started()) why = 2;
    }
    return why;
  }

  // Add the pieces of segment `si` of `g` that have a destination to `L`, after making its
  // bytes readable on `stream`: from the staging slot, or from a restore slot (fetched first if
  // `fetch` allows, waited for, decoded if coded). The restore slot goes to `pending`.
  int scatter_segment(Group& g, uint32_t si, const uint64_t* dst, hipStream_t stream, bool fetch_allowed,
                      Launcher& L, std::vector<RestoreSlot*>& pending) {
    Segment& seg = g.segs[si];
    bool any = false;
    for (const Piece& p : seg.pieces) any = any || dst[p.entry] != 0;
    if (!any) return 0;
    RestoreSlot* r = nullptr;
    const char* src = nullptr;
    if (resident(g, si)) {
      if (seg.prefetched) st.prefetch_hits++;
      r = &restore[seg.restore_slot];
    } else if (staged(seg, stream)) {
      // Still in the staging slot, stream-ordered after its pack kernels: no H2D.
      src = stage[seg.stage_slot].dev + seg.stage_off;
      st.staged_hits++;
      st.bytes_staged += seg.bytes;
    } else {
      if (!fetch_allowed) return fail(MO_E_STATE, "mo_unpack: a further group's segment is not resident");
      const int k = pick_slot(g, si, false);
      if (k < 0) return fail(MO_E_STATE, "mo_unpack: no restore slot available");
      if (int rc = fetch(g, si, k)) return rc;
      st.restore_fetches++;
      r = &restore[k];
    }
    seg.prefetched = false;
    if (r) {
      MO_LINK(link->wait(r->gate, stream));
      // Last decoded or read on another stream: this stream reads the slot after that work,
      // and so the consumed point recorded after the scatter covers both streams' reads.
      if (r->used_on && r->used_on != stream) MO_HIP(hipStreamWaitEvent(stream, r->join, 0));
      if (!r->decoded) {
        // the coded stream has landed (wait): decode it into the slot on this stream, ahead
        // of the unpack kernels that read the slot
        MO_HIP((hipError_t)wire_decode((uint64_t)r->wire, seg.host_bytes, (uint64_t)r->dev, seg.bytes, stream));
        r->decoded = true;
      }
      src = r->dev;
    }
    std::string err;
    for (const Piece& p : seg.pieces) {
      if (!dst[p.entry]) continue;
      KDesc kd;
      const Canon& c = g.entries[p.entry].canon;
      if (dst[p.entry] % c.eb != 0) return fail(MO_E_INVALID, "mo_unpack: misaligned destination");
      if (int rc = make_kdesc(c, dst[p.entry], p.first, p.nbytes, (uint64_t)(src + p.seg_off), kd, err))
        return fail(rc, "mo_unpack: " + err);
      kd.cache = unpack_cache();
      L.add(kd);
      st.bytes_unpacked += p.nbytes;
    }
    if (r) pending.push_back(r);
    return L.status() ? hip_fail(L.status(), "unpack kernel launch") : 0;
  }

  int release(uint64_t gid) {
    Group* g = find(gid);
    if (!g) return fail(MO_E_INVALID, "mo_release: unknown group " + std::to_string(gid));
    if (!closing.empty()) {
      // Committed segments wait for gathers pending beside this group's: launch them all (the
      // open group's too, while their sources still live) and send the waiting segments.
      if (int rc = flush_packs()) return rc;
    }
    if (g == open_group) {
      // No D2H was issued: abandon the staging space and the gathers not launched yet
      // (their sources may be freed as soon as this returns).
      discard_packs();
      open_group = nullptr;
      open_seg = -1;
    }
    for (Segment& seg : g->segs) {
      if (seg.host) deferred.frees.push_back(PendingFree{seg.host, seg.host_bytes, {seg.d2h, seg.h2d}});
      if (seg.restore_slot >= 0) {
        RestoreSlot& r = restore[seg.restore_slot];
        if (r.group == g->id && r.gen == seg.restore_gen) {
          r.group = kNone;
          r.consumed = true;
        }
      }
    }
    groups.erase(gid);
    return process_pending(false);
  }

  // Pinned chunks that hold no live payload go back to the driver. With no group left (open or
  // committed), the wire buffers are freed too, after every copy and every kernel on the device
  // has finished (the next coded segment allocates them again); the restore slots then hold
  // nothing.
  // Where restore slots get their memory at first use (restore_small_slots), those past the
  // first two give it back too, and the count of small groups in a row starts again.
  int trim() {
    if (int rc = process_pending(false)) return rc;
    pool.trim();
    bool any = false;
    for (const auto& s : stage) any = any || s.wire;
    for (size_t k = 0; k < restore.size(); ++k) {
      const RestoreSlot& r = restore[k];
      any = any || r.wire || (lazy_restore() && k >= kEagerRestore && (r.dev || r.dead));
    }
    if (!any || open_group || !groups.empty()) return 0;
    MO_LINK(link->synchronize());
    MO_HIP(hipDeviceSynchronize());
    hipError_t first = hipSuccess;
    auto give_back = [&](char*& p) {
      const hipError_t e = p ? hipFree(p) : hipSuccess;
      if (first == hipSuccess) first = e;
      p = nullptr;
    };
    for (auto& s : stage) {
      give_back(s.wire);
      s.wire_used = 0;
    }
    for (size_t k = 0; k < restore.size(); ++k) {
      RestoreSlot& r = restore[k];
      give_back(r.wire);
      if (lazy_restore() && k >= kEagerRestore) {
        give_back(r.dev);
        r.dead = false;
      }
      r.group = kNone;
      r.consumed = true;
      r.decoded = true;
      r.used_on = nullptr;
    }
    wire_slot_bytes = 0;
    wire_restore_bytes = 0;
    small_run = 0;
    MO_HIP(first);
    return 0;
  }

  int synchronize() {
    if (int rc = flush_packs()) return rc;
    MO_LINK(link->synchronize());
    if (int rc = process_pending(true)) return rc;
    process_timings(true);
    return 0;
  }

  void fill_stats(mo_stats* out) {
    process_timings(false);
    process_counts(false);
    LinkStats ls;
    link->stats(&ls);
    st.d2h_ms = ls.d2h_ms;
    st.h2d_ms = ls.h2d_ms;
    st.timed_d2h_bytes = ls.d2h_done_bytes;
    st.timed_h2d_bytes = ls.h2d_done_bytes;
    st.copy_failures = ls.failures;
    st.host_blocks = ls.host_blocks;
    st.host_block_ms = ls.host_block_ms;
    st.groups_live = groups.size();
    uint64_t e = 0;
    for (auto& kv : groups) e += kv.second->entries.size();
    st.entries_live = e;
    st.host_bytes_in_use = pool.in_use();
    st.host_bytes_peak = pool.peak();
    st.host_bytes_reserved = pool.reserved();
    st.device_ring_bytes = stage.size() * (cfg.stage_slot_bytes + wire_slot_bytes);
    st.restore_slots_big = st.restore_slots_small = 0;
    for (const RestoreSlot& r : restore) {
      if (r.dev) {
        st.device_ring_bytes += r.cap;
        ++(r.small ? st.restore_slots_small : st.restore_slots_big);
      }
      if (r.wire) st.device_ring_bytes += wire_restore_bytes;
    }
    *out = st;
  }

  void reset_stats() {
    process_timings(false);
    link->reset_stats();
    pool.reset_peak();  // the pinned peak counts from here, like the other statistics
    st = mo_stats{};
  }

  int init(int dev, const mo_config* c) {
    device = dev;
    if (c) cfg = *c;
    if (!cfg.stage_slot_bytes) cfg.stage_slot_bytes = 128ull << 20;
    if (!cfg.stage_slots) cfg.stage_slots = 4;
    if (!cfg.restore_slots) cfg.restore_slots = 16;
    if (!cfg.host_chunk_bytes) cfg.host_chunk_bytes = 1ull << 30;
    if (!cfg.copy_kernel_blocks) cfg.copy_kernel_blocks = 16;
    if (cfg.stage_slot_bytes < 2 * kMinPiece || cfg.stage_slot_bytes % kPieceAlign)
      return fail(MO_E_INVALID, "stage_slot_bytes must be a multiple of 4096 and at least 2 MiB");
    if (!cfg.stage_slots_max) cfg.stage_slots_max = cfg.stage_slots;
    if (!cfg.restore_slots_max) cfg.restore_slots_max = cfg.restore_slots;
    if (cfg.stage_slots < 2 || cfg.restore_slots < 2 || cfg.stage_slots + cfg.restore_slots > kMaxSlots)
      return fail(MO_E_INVALID, "need at least 2 stage and 2 restore slots, 64 in total at most");
    if (cfg.stage_slots_max < cfg.stage_slots || cfg.restore_slots_max < cfg.restore_slots ||
        (uint64_t)cfg.stage_slots_max + cfg.restore_slots_max + cfg.restore_small_slots > kMaxSlots)
      return fail(MO_E_INVALID, "stage_slots_max and restore_slots_max must be at least the slot counts, "
                                "64 in total at most with restore_small_slots");
    small_cap = cfg.restore_small_slots ? align_up(cfg.stage_slot_bytes / 4, 4096) : 0;
    pool.configure(cfg.host_limit_bytes, cfg.host_chunk_bytes);
    DeviceGuard guard(device);
    std::string err;
    int status = 0;
    if (cfg.flags & MO_FLAG_KERNEL_COPY) {
      link = make_stream_link(device, cfg.copy_kernel_blocks, (cfg.flags & MO_FLAG_TIMING) != 0, host_alias, &pool,
                              err, &status);
    } else if (cfg.flags & MO_FLAG_HIP_DMA) {
      const bool split = __builtin_popcount(cfg.d2h_engine) != 1;
      link = make_hip_dma_link(device, split, (cfg.flags & MO_FLAG_TIMING) != 0, err, &status);
    } else {
      link = make_sdma_link(device, cfg.d2h_engine, cfg.h2d_engine, err, &status);
    }
    if (!link) return fail(status ? status : MO_E_STATE, "creating the host link failed: " + err);
    if (cfg.flags & MO_FLAG_TIMING) (void)link->use_dma_timestamps();
    // the rings never reallocate (a grown slot is appended in place)
    stage.reserve(cfg.stage_slots_max);
    restore.reserve(cfg.restore_slots_max + cfg.restore_small_slots);
    stage.resize(cfg.stage_slots);
    for (auto& s : stage) {
      MO_HIP(hipMalloc(&s.dev, cfg.stage_slot_bytes));
      MO_LINK(link->new_gate(&s.gate));
    }
    restore.resize(cfg.restore_slots);
    for (size_t k = 0; k < restore.size(); ++k) {
      RestoreSlot& r = restore[k];
      r.cap = cfg.stage_slot_bytes;
      if (!lazy_restore() || k < kEagerRestore) MO_HIP(hipMalloc(&r.dev, r.cap));
      MO_LINK(link->new_gate(&r.gate));
    }
    return 0;
  }

  // Ring growth at the commit of a group of n segments (stage_slots_max, restore_slots_max):
  //   - the restore ring to n + 2 slots, so that the next group backward needs can be fetched
  //     whole while this one is scattered (a group larger than the ring has its last segments
  //     fetched one by one at its restore, each waiting for an earlier one's scatter);
  //   - the staging ring to ceil(n / 3) slots, so that the D2H queue still holds bytes while a
  //     long kernel keeps the next segment's gather waiting (attention grows with the square
  //     of the tokens, the block's saves with the tokens).
  // Measured on MI355X, config 4 not checkpointed (2048^2, 24 blocks, about 23 coded segments
  // a block), fixed rings: 4 + 16 slots 2.60 s/it, 4 + 32 slots 2.45, 8 + 32 slots 2.33,
  // 12 + 32 slots 2.33; 4 + 48 was no faster than 4 + 32. At 1024^2 (at most about 12
  // segments a block) nothing grows: a fixed eight-slot staging ring there ran 0.663 s/it
  // against 0.650 with four (coding starts once the ring has come round twice, later on a
  // longer ring, so more of the forward crosses uncoded). The growth happens at the first
  // large commit, when coding is on already.
  //   - small restore slots (restore_small_slots), all of them once kSmallRun groups in a row
  //     were committed with only segments that fit one.
  // A slot joins the ring at its end: the staging ring's next advance reaches it after the
  // slots in use, and the restore ring's slot choice sees it empty. A restore slot joins
  // without memory where slots get it at first use (restore_small_slots), else with it. Growth
  // stops for good at the first slot whose memory cannot be had (the HIP error is cleared) or
  // whose wire buffer would pass wire_device_limit; the engine runs on with what it has.
  static constexpr int kMaxSlots = 64;
  static constexpr int kSmallRun = 8;
  static constexpr size_t kEagerRestore = 2;  // restore slots that get memory at init when the rest wait
  bool ring_growth_stopped = false;
  int small_run = 0;  // groups committed in a row with only segments that fit a small slot
  bool lazy_restore() const { return cfg.restore_small_slots != 0; }
  void grow_rings(const Group& g) {
    bool all_small = small_cap && !g.segs.empty();
    for (const Segment& seg : g.segs) all_small = all_small && small_fit(seg);
    small_run = all_small ? small_run + 1 : 0;
    if (ring_growth_stopped) return;
    const size_t n = g.segs.size();
    size_t big = big_slots(), small = restore.size() - big;
    const size_t stage_want = std::min<size_t>(cfg.stage_slots_max, std::max(stage.size(), (n + 2) / 3));
    const size_t big_want = std::min<size_t>(cfg.restore_slots_max, std::max(big, n + 2));
    const size_t small_want = small_run >= kSmallRun ? std::max<size_t>(small, cfg.restore_small_slots) : small;
    if (stage_want == stage.size() && big_want == big && small_want == small) return;
    DeviceGuard guard(device);
    auto wire_room = [&](uint64_t more) {
      const uint64_t now = stage.size() * wire_slot_bytes + big * wire_restore_bytes;
      return !cfg.wire_device_limit || now + more <= cfg.wire_device_limit;
    };
    auto get = [&](char** p, uint64_t bytes) {
      if (hipMalloc(p, bytes) == hipSuccess) return true;
      *p = nullptr;
      (void)hipGetLastError();
      return false;
    };
    while (!ring_growth_stopped && (stage.size() < stage_want || big < big_want || small < small_want)) {
      const bool is_stage = stage.size() < stage_want;
      const bool is_small = !is_stage && big >= big_want;
      const uint64_t wire_bytes = is_stage ? wire_slot_bytes : is_small ? 0 : wire_restore_bytes;
      const bool now = is_stage || !lazy_restore();  // memory now, or at first use
      char *dev = nullptr, *wire = nullptr;
      int gate = -1;
      if (!wire_room(wire_bytes) || (now && !get(&dev, cfg.stage_slot_bytes)) ||
          (now && wire_bytes && !get(&wire, wire_bytes)) || link->new_gate(&gate) != 0) {
        if (dev) (void)hipFree(dev);
        if (wire) (void)hipFree(wire);
        ring_growth_stopped = true;
        break;
      }
      if (is_stage) {
        StageSlot s;
        s.dev = dev;
        s.wire = wire;
        s.gate = gate;
        stage.push_back(s);
      } else {
        RestoreSlot r;
        r.dev = dev;
        r.wire = wire;
        r.gate = gate;
        r.small = is_small;
        r.cap = is_small ? small_cap : cfg.stage_slot_bytes;
        restore.push_back(r);
        ++(is_small ? small : big);
      }
    }
  }

  void teardown() {
    DeviceGuard guard(device);
    // Drain the link first: compute streams may wait on copies that are still queued.
    if (link) (void)link->synchronize();
    discard_packs();
    (void)hipDeviceSynchronize();
    groups.clear();
    (void)process_pending(true);
    deferred.clear();
    link.reset();
    for (auto& t : timings) {
      (void)hipEventDestroy(t.start);
      (void)hipEventDestroy(t.end);
    }
    timings.clear();
    for (hipEvent_t e : timing_pool) (void)hipEventDestroy(e);
    timing_pool.clear();
    for (auto& sh : shrinks) (void)hipEventDestroy(sh.coded);
    shrinks.clear();
    for (hipEvent_t e : shrink_events) (void)hipEventDestroy(e);
    shrink_events.clear();
    for (auto& q : eq) {
      if (q.ev) (void)hipEventDestroy(q.ev);
      q = EqualSlot{};
    }
    if (eq_flags) (void)hipHostFree(eq_flags);
    eq_flags = nullptr;
    for (auto& s : stage) {
      if (s.dev) (void)hipFree(s.dev);
      if (s.wire) (void)hipFree(s.wire);
    }
    for (auto& r : restore) {
      if (r.dev) (void)hipFree(r.dev);
      if (r.wire) (void)hipFree(r.wire);
      if (r.join) (void)hipEventDestroy(r.join);
    }
    stage.clear();
    restore.clear();
    pool.release_all();
  }
};

// ------------------------------------------------------------------------------------------
// kernels alone

static int build_layout(const mo_tensor* ts, int n, std::vector<Canon>& cs, std::vector<uint64_t>& offs,
                        uint64_t* total) {
  cs.resize(n);
  offs.resize(n);
  std::string err;
  uint64_t pos = 0;
  for (int i = 0; i < n; ++i) {
    if (int rc = canonicalize(ts[i], cs[i], err)) return fail(rc, "tensor " + std::to_string(i) + ": " + err);
    pos = align_up(pos, kPayloadAlign);
    offs[i] = pos;
    pos += cs[i].nbytes;
  }
  *total = pos;
  return 0;
}

static int run_copy(bool pack, const mo_tensor* ts, int n, uint64_t payload, const uint64_t* offsets,
                    uint64_t stream) {
  if (n < 0 || (n > 0 && !ts)) return fail(MO_E_INVALID, "bad tensor array");
  std::vector<Canon> cs;
  std::vector<uint64_t> offs;
  uint64_t total = 0;
  if (int rc = build_layout(ts, n, cs, offs, &total)) return rc;
  if (offsets)
    for (int i = 0; i < n; ++i) offs[i] = offsets[i];
  Launcher L(pack, (hipStream_t)stream);
  std::string err;
  for (int i = 0; i < n; ++i) {
    // Pieces of at most one launch's worth of tiles, so a launch grid never exceeds
    // kMaxTilesPerLaunch + kMaxDesc workgroups.
    const uint64_t chunk = (uint64_t)kMaxTilesPerLaunch * kTileBytes;
    for (uint64_t first = 0; first < cs[i].nbytes; first += chunk) {
      const uint64_t take = std::min(chunk, cs[i].nbytes - first);
      KDesc kd;
      if (int rc = make_kdesc(cs[i], cs[i].base, first, take, payload + offs[i] + first, kd, err))
        return fail(rc, "tensor " + std::to_string(i) + ": " + err);
      kd.cache = kCacheNtStore;  // the engine's default policy in both directions
      L.add(kd);
    }
  }
  if (int rc = L.flush()) return hip_fail(rc, pack ? "pack kernel launch" : "unpack kernel launch");
  return 0;
}

}  // namespace mo

// ------------------------------------------------------------------------------------------
// C ABI

struct mo_engine {
  mo::Engine e;
};

#define MO_GUARD_BEGIN try {
#define MO_GUARD_END                                                          \
  }                                                                           \
  catch (const std::exception& ex) {                                          \
    return mo::fail(MO_E_STATE, std::string("internal error: ") + ex.what()); \
  }                                                                           \
  catch (...) {                                                               \
    return mo::fail(MO_E_STATE, "internal error");                            \
  }

#define MO_ENGINE_CALL(engine, expr)                           \
  MO_GUARD_BEGIN                                               \
  if (!(engine)) return mo::fail(MO_E_INVALID, "null engine"); \
  std::lock_guard<std::mutex> lock((engine)->e.mu);            \
  mo::DeviceGuard guard((engine)->e.device);                   \
  return (expr);                                               \
  MO_GUARD_END

extern "C" {

int mo_abi_version(void) { return MO_ABI_VERSION; }

const char* mo_last_error(void) { return mo::g_error.c_str(); }

int mo_payload_layout(const mo_tensor* tensors, int n, uint64_t* offsets, uint64_t* total_bytes) {
  MO_GUARD_BEGIN
  if (n < 0 || (n > 0 && (!tensors || !offsets)) || !total_bytes) return mo::fail(MO_E_INVALID, "bad arguments");
  std::vector<mo::Canon> cs;
  std::vector<uint64_t> offs;
  if (int rc = mo::build_layout(tensors, n, cs, offs, total_bytes)) return rc;
  for (int i = 0; i < n; ++i) offsets[i] = offs[i];
  return 0;
  MO_GUARD_END
}

int mo_gather(const mo_tensor* tensors, int n, uint64_t payload, const uint64_t* offsets, uint64_t stream) {
  MO_GUARD_BEGIN
  return mo::run_copy(true, tensors, n, payload, offsets, stream);
  MO_GUARD_END
}

int mo_scatter(const mo_tensor* tensors, int n, uint64_t payload, const uint64_t* offsets, uint64_t stream) {
  MO_GUARD_BEGIN
  return mo::run_copy(false, tensors, n, payload, offsets, stream);
  MO_GUARD_END
}

uint64_t mo_wire_capacity(uint64_t raw_bytes) { return mo::wire_capacity(raw_bytes); }

int mo_wire_encode(uint64_t raw, uint64_t raw_bytes, uint64_t wire, uint64_t wire_capacity, uint64_t host_total,
                   uint64_t stream) {
  MO_GUARD_BEGIN
  std::string err;
  if (int rc = mo::wire_check(raw, raw_bytes, wire, wire_capacity, err)) return mo::set_error(rc, "mo_wire_encode: " + err);
  if (wire_capacity < mo::wire_capacity(raw_bytes))
    return mo::set_error(MO_E_INVALID, "mo_wire_encode: wire buffer smaller than mo_wire_capacity(raw_bytes)");
  if (host_total % 8) return mo::set_error(MO_E_INVALID, "mo_wire_encode: host_total must be 8-byte aligned");
  if (int rc = mo::wire_encode(raw, raw_bytes, wire, wire_capacity, host_total, (hipStream_t)stream))
    return mo::set_hip_error(rc, "mo_wire_encode launch");
  return 0;
  MO_GUARD_END
}

int mo_wire_decode(uint64_t wire, uint64_t wire_bytes, uint64_t raw, uint64_t raw_bytes, uint64_t stream) {
  MO_GUARD_BEGIN
  std::string err;
  if (int rc = mo::wire_check(raw, raw_bytes, wire, wire_bytes, err)) return mo::set_error(rc, "mo_wire_decode: " + err);
  if (int rc = mo::wire_decode(wire, wire_bytes, raw, raw_bytes, (hipStream_t)stream))
    return mo::set_hip_error(rc, "mo_wire_decode launch");
  return 0;
  MO_GUARD_END
}

int mo_pack_to_host(const mo_tensor* tensors, int n, uint64_t host, uint64_t host_bytes, uint64_t* offsets,
                    uint64_t stream) {
  MO_GUARD_BEGIN
  if (n < 0 || (n > 0 && !tensors) || !host) return mo::fail(MO_E_INVALID, "mo_pack_to_host: bad arguments");
  std::vector<mo::Canon> cs;
  std::vector<uint64_t> offs;
  uint64_t total = 0;
  if (int rc = mo::build_layout(tensors, n, cs, offs, &total)) return rc;
  if (total > mo::kNoAllocScratchBytes)
    return mo::fail(MO_E_INVALID, "mo_pack_to_host: a payload of " + std::to_string(total) +
                                      " bytes exceeds its device scratch of " +
                                      std::to_string(mo::kNoAllocScratchBytes) +
                                      " bytes; split the tensors over several calls");
  if (total > host_bytes)
    return mo::fail(MO_E_INVALID, "mo_pack_to_host: the host buffer holds " + std::to_string(host_bytes) +
                                      " bytes, the payload needs " + std::to_string(total));
  // The DMA needs page-locked memory: a pageable buffer would make the runtime stage the copy
  // through memory of its own.
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, (const void*)host) != hipSuccess || attr.type != hipMemoryTypeHost) {
    (void)hipGetLastError();
    return mo::fail(MO_E_INVALID, "mo_pack_to_host: the host buffer must be pinned (hipHostMalloc or pin_memory)");
  }
  uint64_t scratch = 0, scratch_bytes = 0;
  if (int rc = mo::noalloc_scratch(&scratch, &scratch_bytes)) return mo::hip_fail(rc, "loading the device code object");
  if (total) {
    if (int rc = mo::run_copy(true, tensors, n, scratch, offs.data(), stream)) return rc;
    hipError_t e = hipMemcpyAsync((void*)host, (const void*)scratch, total, hipMemcpyDeviceToHost, (hipStream_t)stream);
    if (e != hipSuccess) return mo::hip_fail((int)e, "mo_pack_to_host: D2H copy of the payload");
  }
  if (offsets)
    for (int i = 0; i < n; ++i) offsets[i] = offs[i];
  return 0;
  MO_GUARD_END
}

int mo_link_copy(uint64_t dst, uint64_t src, uint64_t bytes, int direction, uint32_t blocks, uint64_t stream) {
  MO_GUARD_BEGIN
  (void)direction;
  int rc = mo::launch_link_copy((void*)dst, (const void*)src, bytes, blocks, (hipStream_t)stream);
  if (rc) return mo::hip_fail(rc, "link copy kernel launch");
  return 0;
  MO_GUARD_END
}

int mo_create(int device, const mo_config* config, mo_engine** out) {
  MO_GUARD_BEGIN
  if (!out) return mo::fail(MO_E_INVALID, "null output");
  *out = nullptr;
  auto* h = new mo_engine();
  int rc = h->e.init(device, config);
  if (rc) {
    const std::string msg = mo::g_error;
    h->e.teardown();
    delete h;
    mo::g_error = msg;
    return rc;
  }
  *out = h;
  return 0;
  MO_GUARD_END
}

int mo_destroy(mo_engine* engine) {
  MO_GUARD_BEGIN
  if (!engine) return 0;
  {
    std::lock_guard<std::mutex> lock(engine->e.mu);
    engine->e.teardown();
  }
  delete engine;
  return 0;
  MO_GUARD_END
}

int mo_pack(mo_engine* engine, const mo_tensor* tensors, int n, uint64_t stream, mo_ref* refs) {
  if (n < 0 || (n > 0 && (!tensors || !refs))) return mo::fail(MO_E_INVALID, "mo_pack: bad arguments");
  MO_ENGINE_CALL(engine, engine->e.pack(tensors, n, (hipStream_t)stream, refs));
}

int mo_pack_progress(mo_engine* engine, uint64_t* calls, uint64_t* launched) {
  if (!calls || !launched) return mo::fail(MO_E_INVALID, "mo_pack_progress: null output");
  MO_ENGINE_CALL(engine, (*calls = engine->e.pack_calls, *launched = engine->e.pack_launched, 0));
}

int mo_pack_flush(mo_engine* engine) { MO_ENGINE_CALL(engine, engine->e.flush_packs()); }

int mo_equal(mo_engine* engine, uint64_t a, uint64_t b, uint64_t nbytes, uint64_t stream, uint64_t* ticket) {
  if (!ticket) return mo::fail(MO_E_INVALID, "mo_equal: null output");
  MO_ENGINE_CALL(engine, engine->e.equal(a, b, nbytes, (hipStream_t)stream, ticket));
}

int mo_equal_result(mo_engine* engine, uint64_t ticket, int wait, int* state) {
  if (!state) return mo::fail(MO_E_INVALID, "mo_equal_result: null output");
  MO_ENGINE_CALL(engine, engine->e.equal_result(ticket, wait, state));
}

int mo_equal_discard(mo_engine* engine, uint64_t ticket) { MO_ENGINE_CALL(engine, engine->e.equal_discard(ticket)); }

int mo_commit(mo_engine* engine, uint64_t stream, uint64_t* group) {
  if (!group) return mo::fail(MO_E_INVALID, "mo_commit: null output");
  MO_ENGINE_CALL(engine, engine->e.commit((hipStream_t)stream, group));
}

int mo_prefetch(mo_engine* engine, uint64_t group, uint64_t stream) {
  MO_ENGINE_CALL(engine, engine->e.prefetch(group, (hipStream_t)stream));
}

int mo_prefetch_entry(mo_engine* engine, uint64_t group, uint32_t entry, uint64_t stream) {
  if (entry == mo::Engine::kAllEntries) return mo::fail(MO_E_INVALID, "mo_prefetch_entry: bad entry index");
  MO_ENGINE_CALL(engine, engine->e.prefetch(group, (hipStream_t)stream, entry));
}

int mo_prefetch_groups(mo_engine* engine, const uint64_t* groups, uint32_t n, uint64_t stream) {
  if (n && !groups) return mo::fail(MO_E_INVALID, "mo_prefetch_groups: null group list");
  MO_ENGINE_CALL(engine, engine->e.prefetch_groups(groups, n, (hipStream_t)stream));
}

int mo_unpack(mo_engine* engine, uint64_t group, const uint64_t* dst, uint32_t n, uint64_t stream) {
  if (n > 0 && !dst) return mo::fail(MO_E_INVALID, "mo_unpack: null destination array");
  uint32_t unpacked = 0;
  MO_ENGINE_CALL(engine, engine->e.unpack_groups(&group, dst, &n, 1, (hipStream_t)stream, &unpacked));
}

int mo_unpack_groups(mo_engine* engine, const uint64_t* groups, const uint64_t* dst, const uint32_t* counts,
                     uint32_t n, uint64_t stream, uint32_t* unpacked) {
  if (n == 0) return mo::fail(MO_E_INVALID, "mo_unpack_groups: no group");
  if (!groups || !counts || !unpacked) return mo::fail(MO_E_INVALID, "mo_unpack_groups: null array");
  uint64_t total = 0;
  for (uint32_t k = 0; k < n; ++k) total += counts[k];
  if (total > 0 && !dst) return mo::fail(MO_E_INVALID, "mo_unpack_groups: null destination array");
  MO_ENGINE_CALL(engine, engine->e.unpack_groups(groups, dst, counts, n, (hipStream_t)stream, unpacked));
}

int mo_release(mo_engine* engine, uint64_t group) { MO_ENGINE_CALL(engine, engine->e.release(group)); }

int mo_group_info(mo_engine* engine, uint64_t group, uint32_t* entries, uint64_t* payload_bytes, int* d2h_complete) {
  MO_GUARD_BEGIN
  if (!engine) return mo::fail(MO_E_INVALID, "null engine");
  std::lock_guard<std::mutex> lock(engine->e.mu);
  mo::Group* g = engine->e.find(group);
  if (!g) return mo::fail(MO_E_INVALID, "mo_group_info: unknown group " + std::to_string(group));
  if (entries) *entries = (uint32_t)g->entries.size();
  if (payload_bytes) *payload_bytes = g->payload_bytes;
  if (d2h_complete) {
    int done = g->open ? 0 : 1;
    for (auto& seg : g->segs)
      if (!seg.committed || !mo::idle(seg.d2h)) done = 0;  // not committed: waits for its gathers
    *d2h_complete = done;
  }
  return 0;
  MO_GUARD_END
}

int mo_synchronize(mo_engine* engine) { MO_ENGINE_CALL(engine, engine->e.synchronize()); }

int mo_get_stats(mo_engine* engine, mo_stats* stats) {
  if (!stats) return mo::fail(MO_E_INVALID, "null stats");
  MO_ENGINE_CALL(engine, (engine->e.fill_stats(stats), 0));
}

int mo_reset_stats(mo_engine* engine) { MO_ENGINE_CALL(engine, (engine->e.reset_stats(), 0)); }

int mo_trim(mo_engine* engine) {
  MO_ENGINE_CALL(engine, engine->e.trim());
}

const char* mo_link_name(mo_engine* engine) {
  if (!engine || !engine->e.link) return "";
  return engine->e.link->name();
}

}  // extern "C"
