// Host-link transports (see mo_link.h): SDMA engines through HSA, and a copy kernel on HIP
// streams.
#include "mo_link.h"

#include <hip/hip_runtime_api.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <stdint.h>

#include <sys/prctl.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <thread>
#include <vector>

#include "mo_gate_order.h"
#include "mo_internal.h"

namespace mo {

namespace {

int64_t now_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

constexpr int64_t kWaitLimitNs = 300ll * 1000000000ll;  // a copy that takes longer is reported as failed

// H2D copies enqueued and not finished per device, over every SDMA link of the process
// (engine, streamer).
constexpr int kMaxDevices = 64;
std::atomic<int> g_h2d_inflight[kMaxDevices];

// The HSA runtime is shared with HIP (and with a profiler's interception layer when one is
// loaded). The library takes one reference on it, the first time a link is made, and never
// gives it back: an hsa_shut_down from a library's teardown can run while HIP and the
// profiler still use the runtime (at interpreter exit, for instance), and the runtime ends
// with the process anyway.
bool hsa_reference() {
  static const bool ok = hsa_init() == HSA_STATUS_SUCCESS;
  return ok;
}

// Process-wide pool of copy-completion signals. A signal handed to the runtime as a copy's
// completion signal is never destroyed: a profiler that intercepts the copy API may wrap it and
// still touch it after the copy is reported complete, or in its own exit handlers. Links
// return their signals here and later links reuse them; the process end reclaims them.
std::mutex g_signal_mu;
std::vector<hsa_signal_t> g_signals;

bool signal_pool_take(hsa_signal_t* sig) {
  {
    std::lock_guard<std::mutex> lock(g_signal_mu);
    if (!g_signals.empty()) {
      *sig = g_signals.back();
      g_signals.pop_back();
      return true;
    }
  }
  return hsa_signal_create(1, 0, nullptr, sig) == HSA_STATUS_SUCCESS;
}

void signal_pool_give(hsa_signal_t sig) {
  std::lock_guard<std::mutex> lock(g_signal_mu);
  g_signals.push_back(sig);
}

// Short polling sleep. The default 50 us timer slack of a Linux thread would dominate a 5 us
// sleep, so each polling thread lowers its own slack once.
void short_sleep() {
  thread_local bool tuned = false;
  if (!tuned) {
    prctl(PR_SET_TIMERSLACK, 1000UL, 0, 0, 0);
    tuned = true;
  }
  std::this_thread::sleep_for(std::chrono::microseconds(5));
}

// ==========================================================================================
// SDMA link
//
// Ordering uses only host-visible completion: HIP events (queried) for GPU work, HSA signal
// values (loaded) for SDMA copies. No GPU queue ever waits on memory the host writes, so a
// missed wake-up can only delay the host, never stall the GPU; every host wait is bounded.

class SdmaLink;

// A HIP event recorded once and never re-recorded; returned to the pool when the last holder
// (a gate or a pending job) drops it.
struct EventHold {
  hipEvent_t ev = nullptr;
  SdmaLink* owner = nullptr;
  ~EventHold();
};
using EventRef = std::shared_ptr<EventHold>;

struct SdmaCopy : CopyState {
  std::atomic<bool> finished{false};
  std::atomic<bool> fail{false};
  std::atomic<bool> issued{false};  // handed to the copy engines
  bool to_host = true;
  uint64_t bytes = 0;
  int64_t issue_ns = 0;
  int parts_left = 0;        // halves still in flight (worker thread only)
  bool counted_h2d = false;  // counted in g_h2d_inflight until finished
  bool counted_d2h = false;  // counted in d2h_inflight_ until finished (worker thread only)
  bool part_failed = false;  // a half failed or timed out (worker thread only)
  // DMA-engine stamps over the copy's parts, HSA system clock (worker thread only)
  uint64_t dma_start = UINT64_MAX, dma_end = 0;
  bool dma_stamped = true;  // every part completed with stamps
  bool done() const override { return finished.load(std::memory_order_acquire); }
  bool failed() const override { return fail.load(std::memory_order_acquire); }
  // handed to the engines: its compute-stream event and copy dependencies have passed
  bool started() const override { return done() || issued.load(std::memory_order_acquire); }
};
using SdmaRef = std::shared_ptr<SdmaCopy>;

struct Job {
  SdmaRef copy;
  void* dst = nullptr;
  const void* src = nullptr;
  EventRef wait;  // issue after this HIP event completed
  // and after these copies completed: the D2H that filled an H2D's source, and the earlier
  // copies through the same gate that this one must follow (GateOrder)
  std::vector<SdmaRef> deps;
  // sized copy: the byte count is read from here at issue, clamped to [1, max_bytes]
  const volatile uint64_t* size = nullptr;
  uint64_t max_bytes = 0;
  // Polling of `wait` backs off while the compute stream is far behind (hipEventQuery is a
  // runtime call that competes with the application's own launches).
  int64_t next_query_ns = 0;
  int64_t query_gap_ns = 0;
};

constexpr int64_t kQueryGapMinNs = 5000;
constexpr int64_t kQueryGapMaxNs = 100000;

struct InFlight {
  SdmaRef copy;
  hsa_signal_t sig;
};

struct GateState {
  GateOrder<SdmaRef> order;  // copy-to-copy ordering; order.last is the gate's last copy
  EventRef consumed;         // the slot's last consumer on a compute stream
};

struct AgentSearch {
  uint32_t bus = 0, dev = 0, domain = 0;
  bool found_gpu = false, found_cpu = false;
  int gpu_index = 0, want_index = 0;
  hsa_agent_t gpu{0}, fallback_gpu{0}, cpu{0};
};

hsa_status_t find_agents(hsa_agent_t agent, void* data) {
  auto* s = (AgentSearch*)data;
  hsa_device_type_t type;
  if (hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &type) != HSA_STATUS_SUCCESS) return HSA_STATUS_SUCCESS;
  if (type == HSA_DEVICE_TYPE_CPU && !s->found_cpu) {
    s->cpu = agent;
    s->found_cpu = true;
  }
  if (type == HSA_DEVICE_TYPE_GPU) {
    uint32_t bdf = 0, domain = 0;
    hsa_agent_get_info(agent, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_BDFID, &bdf);
    hsa_agent_get_info(agent, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_DOMAIN, &domain);
    if (((bdf >> 8) & 0xff) == s->bus && ((bdf >> 3) & 0x1f) == s->dev && domain == s->domain) {
      s->gpu = agent;
      s->found_gpu = true;
    }
    if (s->gpu_index++ == s->want_index) s->fallback_gpu = agent;
  }
  return HSA_STATUS_SUCCESS;
}

class SdmaLink : public Link {
 public:
  ~SdmaLink() override { shutdown(); }

  int init(int device, uint32_t d2h_engine, uint32_t h2d_engine, std::string& err) {
    device_ = device;
    if (!hsa_reference()) {
      err = "hsa_init failed";
      return MO_E_STATE;
    }
    // Match the HIP device to its HSA agent by PCI location (falls back to the ordinal).
    AgentSearch s;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributePciBusId, device) == hipSuccess) s.bus = (uint32_t)v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributePciDeviceId, device) == hipSuccess) s.dev = (uint32_t)v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributePciDomainID, device) == hipSuccess) s.domain = (uint32_t)v;
    s.want_index = device;
    hsa_iterate_agents(find_agents, &s);
    if (!s.found_cpu) {
      err = "no HSA CPU agent";
      return MO_E_STATE;
    }
    gpu_ = s.found_gpu ? s.gpu : s.fallback_gpu;
    cpu_ = s.cpu;
    if (!gpu_.handle) {
      err = "no HSA agent for the HIP device";
      return MO_E_STATE;
    }
    uint32_t d2h_mask = 0, h2d_mask = 0;
    if (hsa_amd_memory_copy_engine_status(cpu_, gpu_, &d2h_mask) != HSA_STATUS_SUCCESS || !d2h_mask ||
        hsa_amd_memory_copy_engine_status(gpu_, cpu_, &h2d_mask) != HSA_STATUS_SUCCESS || !h2d_mask) {
      err = "no SDMA engine available between host and device";
      return MO_E_STATE;
    }
    // D2H's first engine, then H2D's, then D2H's second from what is left: the lowest two
    // engines make the fastest pair while both directions run (block microbench: H2D on the
    // second-lowest engine 57.2 GB/s, on the third-lowest 53.3 GB/s beside the same D2H).
    uint32_t first[2] = {0, 0};
    const int n_first = pick(d2h_mask, d2h_engine, 0, 1, first);
    n_h2d_ = pick(h2d_mask, h2d_engine, first[0], 1, e_h2d_);
    if (d2h_engine) {
      n_d2h_ = pick(d2h_mask, d2h_engine, 0, 2, e_d2h_);
    } else {
      e_d2h_[0] = first[0];
      n_d2h_ = n_first;
      uint32_t second[2] = {0, 0};
      if (pick(d2h_mask & ~(first[0] | e_h2d_[0]), 0, 0, 1, second) && second[0]) {
        e_d2h_[1] = second[0];
        n_d2h_ = 2;
      }
    }
    worker_ = std::thread([this] { run(); });
    return 0;
  }

  int new_gate(int* gate) override {
    gates_.emplace_back();
    *gate = (int)gates_.size() - 1;
    return 0;
  }

  int d2h(void* dst, const void* src, uint64_t bytes, hipStream_t compute, int gate, CopyRef* out) override {
    return d2h_job(dst, src, bytes, compute, gate, out, nullptr);
  }

  int h2d(void* dst, const void* src, uint64_t bytes, const CopyRef& after, int gate, CopyRef* out) override {
    return h2d_job(dst, src, bytes, after, gate, out, nullptr);
  }

  // `size` null: a copy of `bytes`; else a sized copy of at most `bytes` (see Link).
  int d2h_job(void* dst, const void* src, uint64_t bytes, hipStream_t compute, int gate, CopyRef* out,
              const volatile uint64_t* size) {
    EventRef ev;
    if (int rc = take_event(&ev)) return rc;
    hipError_t e = hipEventRecord(ev->ev, compute);
    if (e != hipSuccess) return (int)e;
    auto copy = make_copy(true, bytes);
    Job job;
    job.copy = copy;
    job.dst = dst;
    job.src = src;
    job.wait = std::move(ev);
    add_dep(job, gates_[gate].order.on_read(copy, copy_done));
    job.size = size;
    job.max_bytes = bytes;
    enqueue(std::move(job));
    d2h_bytes_ += bytes;
    *out = copy;
    return 0;
  }

  int h2d_job(void* dst, const void* src, uint64_t bytes, const CopyRef& after, int gate, CopyRef* out,
              const volatile uint64_t* size) {
    auto copy = make_copy(false, bytes);
    h2d_inflight().fetch_add(1, std::memory_order_relaxed);
    copy->counted_h2d = true;
    Job job;
    job.copy = copy;
    job.dst = dst;
    job.src = src;
    job.wait = gates_[gate].consumed;
    add_dep(job, std::dynamic_pointer_cast<SdmaCopy>(after));
    for (const SdmaRef& dep : gates_[gate].order.on_write(copy)) add_dep(job, dep);
    job.size = size;
    job.max_bytes = bytes;
    enqueue(std::move(job));
    h2d_bytes_ += bytes;
    *out = copy;
    return 0;
  }

  bool sized_copies() const override { return true; }

  int d2h_sized(void* dst, const void* src, const volatile uint64_t* size, uint64_t max_bytes, hipStream_t compute,
                int gate, CopyRef* out) override {
    return d2h_job(dst, src, max_bytes, compute, gate, out, size);
  }

  int h2d_sized(void* dst, const void* src, const volatile uint64_t* size, uint64_t max_bytes, const CopyRef& after,
                int gate, CopyRef* out) override {
    return h2d_job(dst, src, max_bytes, after, gate, out, size);
  }

  bool link_busy(int gate) override {
    const SdmaRef& c = gates_[gate].order.last;
    return c && !c->done() && c->issued.load(std::memory_order_acquire);
  }

  int writeback(void* dst, const void* src, uint64_t bytes, int gate, CopyRef* out) override {
    auto copy = make_copy(true, bytes);
    Job job;
    job.copy = copy;
    job.dst = dst;
    job.src = src;
    job.wait = gates_[gate].consumed;
    add_dep(job, gates_[gate].order.on_read(copy, copy_done));
    enqueue(std::move(job));
    d2h_bytes_ += bytes;
    *out = copy;
    return 0;
  }

  // Host-side: return once every copy that may still access the gate's slot finished (its
  // last write and all reads since: two D2H copies of one staging slot may run on different
  // engines and finish out of order). The caller enqueues the dependent GPU work afterwards,
  // so stream order does the rest.
  int wait(int gate, hipStream_t compute) override {
    (void)compute;
    GateOrder<SdmaRef>& order = gates_[gate].order;
    bool blocked = false, failed = false;
    const int64_t t0 = now_ns();
    for (const SdmaRef& c : order.outstanding()) {
      if (!c) continue;
      while (!c->done()) {
        if (now_ns() - t0 > kWaitLimitNs) return MO_E_STATE;
        blocked = true;
        short_sleep();
      }
      failed = failed || c->failed();
    }
    order.prune(copy_done);
    if (blocked) {
      host_blocks_++;
      host_block_ns_ += (uint64_t)(now_ns() - t0);
    }
    return failed ? MO_E_STATE : 0;
  }

  int consumed(int gate, hipStream_t compute) override {
    EventRef ev;
    if (int rc = take_event(&ev)) return rc;
    hipError_t e = hipEventRecord(ev->ev, compute);
    if (e != hipSuccess) return (int)e;
    gates_[gate].consumed = std::move(ev);
    return 0;
  }

  int synchronize() override {
    const int64_t t0 = now_ns();
    for (;;) {
      {
        std::lock_guard<std::mutex> lock(mu_);
        if (queue_[0].empty() && queue_[1].empty() && holding_ == 0 && inflight_count_.load() == 0) break;
      }
      if (now_ns() - t0 > kWaitLimitNs) return MO_E_STATE;
      short_sleep();
    }
    return 0;
  }

  bool use_dma_timestamps() override {
    // Async-copy profiling is a process-wide switch of the HSA runtime; the stamps land in each
    // copy's completion signal.
    static std::once_flag once;
    static bool enabled = false;
    std::call_once(once, [] { enabled = hsa_amd_profiling_async_copy_enable(true) == HSA_STATUS_SUCCESS; });
    uint64_t hz = 0;
    if (!enabled || hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &hz) != HSA_STATUS_SUCCESS || !hz)
      return false;
    ns_per_tick_ = 1e9 / (double)hz;
    dma_time_.store(true, std::memory_order_release);
    return true;
  }

  void stats(LinkStats* out) override {
    out->d2h_bytes = d2h_bytes_;
    out->h2d_bytes = h2d_bytes_;
    out->d2h_done_bytes = done_bytes_[0].load();
    out->h2d_done_bytes = done_bytes_[1].load();
    out->d2h_ms = busy_ns_[0].load() / 1e6;
    out->h2d_ms = busy_ns_[1].load() / 1e6;
    out->failures = failures_.load();
    out->host_blocks = host_blocks_;
    out->host_block_ms = host_block_ns_ / 1e6;
  }

  void reset_stats() override {
    d2h_bytes_ = h2d_bytes_ = 0;
    host_blocks_ = host_block_ns_ = 0;
    for (int i = 0; i < 2; ++i) {
      done_bytes_[i] = 0;
      busy_ns_[i] = 0;
    }
  }

  const char* name() const override { return "sdma"; }

  void return_event(hipEvent_t ev) {
    std::lock_guard<std::mutex> lock(ev_mu_);
    ev_pool_.push_back(ev);
  }

 private:
  // Engines of one direction, as bits: the available bits of `want` (at most two), else the
  // `automatic` lowest available bits outside `avoid`, else the lowest available ones. Returns
  // how many. Automatic choice: two for D2H, one for H2D. A second H2D engine gains nothing
  // (H2D writes HBM and holds 55-57 GB/s under load), and while both directions run it takes
  // the host link from D2H (block microbench: D2H 53 -> 34 GB/s).
  static int pick(uint32_t mask, uint32_t want, uint32_t avoid, int automatic, uint32_t out[2]) {
    int n = 0, limit = 2;
    auto take = [&](uint32_t bits) {
      for (int i = 0; i < 32 && n < limit; ++i)
        if (bits & (1u << i)) out[n++] = 1u << i;
    };
    if (want) take(want & mask);
    limit = n ? limit : automatic;
    if (!n) take(mask & ~avoid);
    if (!n) take(mask);
    return n;
  }

  // A copy of at least kSplitBytes with two engines in its direction goes out as two halves,
  // one per engine. One SDMA engine keeps too few reads in flight to cover HBM latency while
  // HBM-bound kernels run (28 MB D2H: 41.6 GB/s alone, 56-57 GB/s as two halves). A D2H is
  // split only while no H2D is pending on the device (enqueued, even if still waiting for its
  // dependencies): with both directions busy the host link is the limit, and a split D2H takes
  // it from the H2D (block microbench: D2H 53 -> 55, H2D 57 -> 53 GB/s, iteration 43.7 ->
  // 45.5 ms).
  static constexpr uint64_t kSplitBytes = 2ull << 20;
  std::atomic<int>& h2d_inflight() { return g_h2d_inflight[device_ < kMaxDevices && device_ >= 0 ? device_ : 0]; }

  static bool copy_done(const SdmaRef& c) { return !c || c->done(); }
  static void add_dep(Job& job, const SdmaRef& dep) {
    if (dep) job.deps.push_back(dep);
  }

  SdmaRef make_copy(bool to_host, uint64_t bytes) {
    auto c = std::make_shared<SdmaCopy>();
    c->to_host = to_host;
    c->bytes = bytes;
    return c;
  }

  int take_event(EventRef* out) {
    hipEvent_t ev = nullptr;
    {
      std::lock_guard<std::mutex> lock(ev_mu_);
      if (!ev_pool_.empty()) {
        ev = ev_pool_.back();
        ev_pool_.pop_back();
      }
    }
    if (!ev) {
      hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (e != hipSuccess) return (int)e;
    }
    auto hold = std::make_shared<EventHold>();
    hold->ev = ev;
    hold->owner = this;
    *out = std::move(hold);
    return 0;
  }

  void enqueue(Job job) {
    {
      std::lock_guard<std::mutex> lock(mu_);
      queue_[job.copy->to_host ? 0 : 1].push_back(std::move(job));
    }
    cv_.notify_one();
  }

  // Worker-owned signal pool: a signal goes back to the pool as soon as its copy finished. The
  // pool is filled from, and returned to, the process-wide pool (signal_pool_take/give).
  bool take_signal(hsa_signal_t* sig) {
    if (sig_pool_.empty() && !signal_pool_take(sig)) return false;
    if (!sig_pool_.empty()) {
      *sig = sig_pool_.back();
      sig_pool_.pop_back();
    }
    hsa_signal_store_screlease(*sig, 1);
    return true;
  }

  void finish(const SdmaRef& c, bool failed) {
    const int dir = c->to_host ? 0 : 1;
    if (c->counted_d2h) {
      c->counted_d2h = false;
      d2h_inflight_--;
    }
    if (c->counted_h2d) {
      c->counted_h2d = false;
      h2d_inflight().fetch_sub(1, std::memory_order_relaxed);
    }

    const int64_t t = now_ns();
    if (failed) {
      c->fail.store(true, std::memory_order_release);
      failures_++;
    } else {
      if (dma_time_.load(std::memory_order_acquire) && c->dma_stamped && c->dma_end > c->dma_start) {
        // Engine-busy time from the engines' own stamps: the part of [start, end] not already
        // counted for the direction (copies of one direction may overlap on two engines).
        const uint64_t s = std::max(c->dma_start, last_dma_end_[dir]);
        busy_ns_[dir] += c->dma_end > s ? (uint64_t)((double)(c->dma_end - s) * ns_per_tick_) : 0;
        last_dma_end_[dir] = std::max(last_dma_end_[dir], c->dma_end);
      } else {
        // Host clock: copies on one engine run back to back, so a copy starts at the later of
        // its issue and the previous completion in its direction.
        const int64_t start = c->issue_ns > last_done_ns_[dir] ? c->issue_ns : last_done_ns_[dir];
        busy_ns_[dir] += t > start ? (uint64_t)(t - start) : 0;
      }
      done_bytes_[dir] += c->bytes;
      last_done_ns_[dir] = t;
    }
    c->finished.store(true, std::memory_order_release);
  }

  // Issue `job` if its dependencies are met. Returns true if the job left the queue.
  bool try_issue(Job& job) {
    if (job.wait) {
      const int64_t now = now_ns();
      if (now < job.next_query_ns) return false;
      const hipError_t q = hipEventQuery(job.wait->ev);
      if (q == hipErrorNotReady) {
        job.query_gap_ns = job.query_gap_ns ? std::min(2 * job.query_gap_ns, kQueryGapMaxNs) : kQueryGapMinNs;
        job.next_query_ns = now + job.query_gap_ns;
        return false;
      }
      job.wait.reset();
      if (q != hipSuccess) {
        finish(job.copy, true);
        return true;
      }
    }
    while (!job.deps.empty()) {
      const SdmaRef& dep = job.deps.back();
      if (!dep->done()) return false;
      const bool bad = dep->failed();
      job.deps.pop_back();
      if (bad) {
        finish(job.copy, true);
        return true;
      }
    }
    SdmaCopy& c = *job.copy;
    if (job.size) {
      // The dependency that produced *size has completed (its HIP event, or the D2H whose
      // bytes begin with it): read the coded size now.
      std::atomic_thread_fence(std::memory_order_acquire);
      const uint64_t n = *job.size;
      c.bytes = n == 0 ? 1 : (n > job.max_bytes ? job.max_bytes : n);
    }
    const uint32_t* engines = c.to_host ? e_d2h_ : e_h2d_;
    const bool quiet = !c.to_host || h2d_inflight().load(std::memory_order_relaxed) == 0;
    const int parts = (c.to_host ? n_d2h_ : n_h2d_) > 1 && c.bytes >= kSplitBytes && quiet ? 2 : 1;
    const uint64_t half = parts == 2 ? c.bytes / 2 / 4096 * 4096 : c.bytes;
    c.parts_left = parts;
    c.issue_ns = now_ns();
    c.issued.store(true, std::memory_order_release);
    if (c.to_host) {
      c.counted_d2h = true;
      d2h_inflight_++;
    }
    for (int k = 0; k < parts; ++k) {
      const uint64_t off = k ? half : 0;
      const uint64_t len = k ? c.bytes - half : half;
      hsa_signal_t sig{0};
      hsa_status_t st = HSA_STATUS_ERROR;
      if (take_signal(&sig)) {
        st = hsa_amd_memory_async_copy_on_engine(
            (char*)job.dst + off, c.to_host ? cpu_ : gpu_, (const char*)job.src + off, c.to_host ? gpu_ : cpu_, len,
            0, nullptr, sig, (hsa_amd_sdma_engine_id_t)engines[k], true);
        if (st != HSA_STATUS_SUCCESS) sig_pool_.push_back(sig);
      }
      if (st != HSA_STATUS_SUCCESS) {
        part_done(job.copy, true);  // the other half, if issued, still completes through its signal
        continue;
      }
      inflight_.push_back(InFlight{job.copy, sig});
      inflight_count_++;
    }
    return true;
  }

  // One half (or the whole) of a copy ended; the copy finishes with its last part.
  void part_done(const SdmaRef& c, bool failed) {
    if (failed) c->part_failed = true;
    if (--c->parts_left == 0) finish(c, c->part_failed);
  }

  // Completed copies leave the in-flight list (in issue order per engine, but checked all).
  bool poll_inflight() {
    bool progress = false;
    for (auto it = inflight_.begin(); it != inflight_.end();) {
      const hsa_signal_value_t v = hsa_signal_load_scacquire(it->sig);
      if (v < 1) {
        if (v == 0 && dma_time_.load(std::memory_order_acquire)) {
          // read before the signal is reused: it holds the stamps of its last copy
          SdmaCopy& c = *it->copy;
          hsa_amd_profiling_async_copy_time_t tm{};
          if (hsa_amd_profiling_get_async_copy_time(it->sig, &tm) == HSA_STATUS_SUCCESS && tm.start &&
              tm.end >= tm.start) {
            c.dma_start = std::min<uint64_t>(c.dma_start, tm.start);
            c.dma_end = std::max<uint64_t>(c.dma_end, tm.end);
          } else {
            c.dma_stamped = false;
          }
        }
        part_done(it->copy, v < 0);
        sig_pool_.push_back(it->sig);
        it = inflight_.erase(it);
        inflight_count_--;
        progress = true;
      } else if (now_ns() - it->copy->issue_ns > kWaitLimitNs) {
        // Give up on a copy the engine never completed: report it, keep the signal alive.
        part_done(it->copy, true);
        it = inflight_.erase(it);
        inflight_count_--;
        progress = true;
      } else {
        ++it;
      }
    }
    return progress;
  }

  // Issuer thread. Jobs of one direction issue in FIFO order; the two directions issue
  // independently (an H2D that needs a D2H names it as `after`, and a slot's copies order
  // through its gate). At most kD2hDepth D2H copies are in flight, so a D2H is issued about one
  // copy before the engines reach it and its split decision sees the H2D work pending by then.
  // Every event a job waits for was recorded on a compute stream before the job was enqueued,
  // and no GPU queue waits on the host, so every dependency eventually completes.
  static constexpr int kD2hDepth = 2;
  void run() {
    (void)hipSetDevice(device_);
    for (;;) {
      bool progress = poll_inflight();
      {
        std::unique_lock<std::mutex> lock(mu_);
        if (queue_[0].empty() && queue_[1].empty() && inflight_.empty()) {
          if (stop_) return;
          cv_.wait_for(lock, std::chrono::milliseconds(2),
                       [this] { return stop_ || !queue_[0].empty() || !queue_[1].empty(); });
          continue;
        }
      }
      for (int d = 0; d < 2; ++d) {
        if (d == 0 && d2h_inflight_ >= kD2hDepth) continue;
        Job job;
        {
          std::lock_guard<std::mutex> lock(mu_);
          if (queue_[d].empty()) continue;
          job = std::move(queue_[d].front());
          queue_[d].pop_front();
          holding_++;
        }
        const bool issued = try_issue(job);
        std::lock_guard<std::mutex> lock(mu_);
        if (issued) progress = true;
        else queue_[d].push_front(std::move(job));
        holding_--;
      }
      if (!progress) short_sleep();
    }
  }

  void shutdown() {
    if (worker_.joinable()) {
      {
        std::lock_guard<std::mutex> lock(mu_);
        stop_ = true;
      }
      cv_.notify_all();
      worker_.join();  // returns once the queue is drained and nothing is in flight
    }
    gates_.clear();
    for (hsa_signal_t s : sig_pool_) signal_pool_give(s);
    sig_pool_.clear();
    {
      std::lock_guard<std::mutex> lock(ev_mu_);
      for (hipEvent_t e : ev_pool_) (void)hipEventDestroy(e);
      ev_pool_.clear();
    }
    // No hsa_shut_down: the HSA reference taken in init() is held until the process ends (see
    // hsa_reference()).
  }

  int device_ = 0;
  hsa_agent_t gpu_{0}, cpu_{0};
  uint32_t e_d2h_[2] = {0, 0}, e_h2d_[2] = {0, 0};  // engine bits per direction
  int n_d2h_ = 0, n_h2d_ = 0;
  std::vector<GateState> gates_;  // API threads only (engine mutex)
  uint64_t d2h_bytes_ = 0, h2d_bytes_ = 0, host_blocks_ = 0, host_block_ns_ = 0;  // API threads only

  std::mutex ev_mu_;
  std::vector<hipEvent_t> ev_pool_;

  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<Job> queue_[2];  // by direction: 0 = D2H (and write-back), 1 = H2D
  bool stop_ = false;
  int holding_ = 0;  // jobs popped by the worker and not yet issued or put back
  int d2h_inflight_ = 0;  // D2H copies issued and not finished (worker thread only)
  std::thread worker_;

  // worker thread only
  std::vector<InFlight> inflight_;
  std::vector<hsa_signal_t> sig_pool_;
  int64_t last_done_ns_[2] = {0, 0};
  std::atomic<bool> dma_time_{false};
  double ns_per_tick_ = 1.0;
  uint64_t last_dma_end_[2] = {0, 0};

  std::atomic<int> inflight_count_{0};
  std::atomic<uint64_t> failures_{0};
  std::atomic<uint64_t> busy_ns_[2]{{0}, {0}};
  std::atomic<uint64_t> done_bytes_[2]{{0}, {0}};
};

EventHold::~EventHold() {
  if (owner && ev) owner->return_event(ev);
}

// ==========================================================================================
// Stream link: copies on dedicated HIP streams, ordered with HIP events only
//
// Two ways to move the bytes:
//   kDma         hipMemcpyAsync(..., hipMemcpyDeviceToDeviceNoCU) between pinned host memory and
//                device memory: the HIP runtime runs it on the SDMA engines (no compute unit).
//   kCopyKernel  the engine's own copy kernel (a comparison point: it contends for CUs).
// Every dependency is a hipStreamWaitEvent on a stream: compute -> copy (the copy stream waits
// for an event recorded after the producing kernels), copy -> copy (GateOrder), and copy ->
// compute (wait() makes the compute stream wait for the gate's last copy). The host never
// waits for a copy on this path; it only enqueues.

struct StreamCopy : CopyState {
  hipEvent_t ev[2] = {nullptr, nullptr};  // one per part (a split D2H has two)
  int parts = 0;
  std::vector<hipEvent_t>* pool = nullptr;
  std::mutex* pool_mu = nullptr;
  ~StreamCopy() override {
    std::lock_guard<std::mutex> lock(*pool_mu);
    for (int k = 0; k < parts; ++k) pool->push_back(ev[k]);
  }
  bool done() const override {
    for (int k = 0; k < parts; ++k)
      if (hipEventQuery(ev[k]) != hipSuccess) return false;
    return true;
  }
  bool failed() const override { return false; }
  // enqueued on a copy stream, which a consumer waits for on the GPU (hipStreamWaitEvent)
  bool started() const override { return true; }
};
using StreamRef = std::shared_ptr<StreamCopy>;

class StreamLink : public Link {
 public:
  enum Method { kCopyKernel, kDma };

  ~StreamLink() override {
    (void)synchronize();
    for (auto& g : gates_) {
      g.order.clear();
      if (g.consumed) (void)hipEventDestroy(g.consumed);
    }
    last_h2d_.reset();
    for (auto& t : timings_) {
      (void)hipEventDestroy(t.start);
      (void)hipEventDestroy(t.end);
    }
    for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
    if (tmp_) (void)hipEventDestroy(tmp_);
    if (base_) (void)hipEventDestroy(base_);
    for (hipStream_t s : d2h_)
      if (s) (void)hipStreamDestroy(s);
    if (h2d_) (void)hipStreamDestroy(h2d_);
  }

  int init(Method method, uint32_t blocks, bool timing, bool split_d2h, char* (*alias)(void*, char*), void* ctx) {
    method_ = method;
    blocks_ = blocks ? blocks : 16;
    timing_ = timing;
    alias_ = alias;
    alias_ctx_ = ctx;
    n_d2h_ = split_d2h ? 2 : 1;
    hipError_t e;
    for (int k = 0; k < n_d2h_; ++k)
      if ((e = hipStreamCreateWithFlags(&d2h_[k], hipStreamNonBlocking)) != hipSuccess) return (int)e;
    if ((e = hipStreamCreateWithFlags(&h2d_, hipStreamNonBlocking)) != hipSuccess) return (int)e;
    if ((e = hipEventCreateWithFlags(&tmp_, hipEventDisableTiming)) != hipSuccess) return (int)e;
    if (timing_) {
      if ((e = hipEventCreate(&base_)) != hipSuccess) return (int)e;
      if ((e = hipEventRecord(base_, d2h_[0])) != hipSuccess) return (int)e;
    }
    return 0;
  }

  int new_gate(int* gate) override {
    gates_.emplace_back();
    *gate = (int)gates_.size() - 1;
    return 0;
  }

  int d2h(void* dst, const void* src, uint64_t bytes, hipStream_t compute, int gate, CopyRef* out) override {
    hipError_t e;
    if ((e = hipEventRecord(tmp_, compute)) != hipSuccess) return (int)e;
    // Split in halves over the two D2H streams only while no H2D is pending: with both
    // directions busy the host link is the limit and a split D2H takes it from the H2D.
    const int parts = n_d2h_ == 2 && bytes >= kSplitBytes && !h2d_pending() ? 2 : 1;
    StreamRef copy;
    if (int rc = make_copy(parts, &copy)) return rc;
    const StreamRef dep = std::static_pointer_cast<StreamCopy>(gates_[gate].order.on_read(copy, copy_done));
    const uint64_t half = parts == 2 ? bytes / 2 / 4096 * 4096 : bytes;
    for (int k = 0; k < parts; ++k) {
      hipStream_t s = d2h_[k];
      if ((e = hipStreamWaitEvent(s, tmp_, 0)) != hipSuccess) return (int)e;
      if (int rc = wait_for(s, dep)) return rc;
      const uint64_t off = k ? half : 0, len = k ? bytes - half : half;
      if (int rc = move(s, host(dst) + off, (const char*)src + off, len, true, copy->ev[k])) return rc;
    }
    st_.d2h_bytes += bytes;
    *out = copy;
    return 0;
  }

  int h2d(void* dst, const void* src, uint64_t bytes, const CopyRef& after, int gate, CopyRef* out) override {
    StreamRef copy;
    if (int rc = make_copy(1, &copy)) return rc;
    Gate& g = gates_[gate];
    hipError_t e;
    if (g.consumed && (e = hipStreamWaitEvent(h2d_, g.consumed, 0)) != hipSuccess) return (int)e;
    if (int rc = wait_for(h2d_, std::static_pointer_cast<StreamCopy>(after))) return rc;
    for (const CopyRef& dep : g.order.on_write(copy))
      if (int rc = wait_for(h2d_, std::static_pointer_cast<StreamCopy>(dep))) return rc;
    if (int rc = move(h2d_, (char*)dst, host(src), bytes, false, copy->ev[0])) return rc;
    st_.h2d_bytes += bytes;
    last_h2d_ = copy;
    *out = copy;
    return 0;
  }

  int writeback(void* dst, const void* src, uint64_t bytes, int gate, CopyRef* out) override {
    StreamRef copy;
    if (int rc = make_copy(1, &copy)) return rc;
    Gate& g = gates_[gate];
    hipError_t e;
    if (g.consumed && (e = hipStreamWaitEvent(d2h_[0], g.consumed, 0)) != hipSuccess) return (int)e;
    if (int rc = wait_for(d2h_[0], std::static_pointer_cast<StreamCopy>(g.order.on_read(copy, copy_done)))) return rc;
    if (int rc = move(d2h_[0], host(dst), (const char*)src, bytes, true, copy->ev[0])) return rc;
    st_.d2h_bytes += bytes;
    *out = copy;
    return 0;
  }

  // Copies on HIP streams are enqueued at once; whether one has started is not known here.
  bool link_busy(int gate) override {
    const auto& c = gates_[gate].order.last;
    return c && !c->done();
  }

  // The compute stream waits for every copy that may still access the gate's slot (its last
  // write and all reads since, which may run on both D2H streams): GPU-side, the host does not
  // block.
  int wait(int gate, hipStream_t compute) override {
    for (const CopyRef& c : gates_[gate].order.outstanding())
      if (int rc = wait_for(compute, std::static_pointer_cast<StreamCopy>(c))) return rc;
    return 0;
  }

  int consumed(int gate, hipStream_t compute) override {
    Gate& g = gates_[gate];
    hipError_t e;
    if (!g.consumed && (e = hipEventCreateWithFlags(&g.consumed, hipEventDisableTiming)) != hipSuccess) return (int)e;
    return (int)hipEventRecord(g.consumed, compute);
  }

  int synchronize() override {
    hipError_t e;
    for (hipStream_t s : d2h_)
      if (s && (e = hipStreamSynchronize(s)) != hipSuccess) return (int)e;
    if (h2d_ && (e = hipStreamSynchronize(h2d_)) != hipSuccess) return (int)e;
    process_timings(true);
    return 0;
  }

  void stats(LinkStats* out) override {
    process_timings(false);
    *out = st_;
  }

  void reset_stats() override {
    process_timings(false);
    st_ = LinkStats();
    last_end_ms_[0] = last_end_ms_[1] = -1.0;
    if (base_ && timings_.empty()) {
      // re-base the interval clock so float milliseconds stay precise over long runs
      (void)hipEventRecord(base_, d2h_[0]);
    }
  }

  const char* name() const override { return method_ == kDma ? "hipdma" : "kernel"; }

 private:
  static constexpr uint64_t kSplitBytes = 2ull << 20;

  struct Gate {
    GateOrder<CopyRef> order;       // order.last: the gate's last copy
    hipEvent_t consumed = nullptr;  // the slot's last consumer on a compute stream
  };
  struct Timing {
    hipEvent_t start, end;
    uint64_t bytes;
    bool d2h;
  };

  char* host(const void* p) {
    return method_ == kCopyKernel ? alias_(alias_ctx_, (char*)p) : (char*)p;
  }

  bool h2d_pending() const { return last_h2d_ && !last_h2d_->done(); }

  int make_copy(int parts, StreamRef* out) {
    auto c = std::make_shared<StreamCopy>();
    c->pool = &pool_;
    c->pool_mu = &pool_mu_;
    for (int k = 0; k < parts; ++k) {
      {
        std::lock_guard<std::mutex> lock(pool_mu_);
        if (!pool_.empty()) {
          c->ev[k] = pool_.back();
          pool_.pop_back();
        }
      }
      if (!c->ev[k]) {
        hipError_t e = hipEventCreateWithFlags(&c->ev[k], hipEventDisableTiming);
        if (e != hipSuccess) return (int)e;
      }
      c->parts = k + 1;
    }
    *out = std::move(c);
    return 0;
  }

  static bool copy_done(const CopyRef& c) { return !c || c->done(); }

  static int wait_for(hipStream_t s, const StreamRef& c) {
    if (!c) return 0;
    for (int k = 0; k < c->parts; ++k) {
      hipError_t e = hipStreamWaitEvent(s, c->ev[k], 0);
      if (e != hipSuccess) return (int)e;
    }
    return 0;
  }

  // Enqueue one copy on `s` and record `done` after it.
  int move(hipStream_t s, char* dst, const char* src, uint64_t bytes, bool to_host, hipEvent_t done) {
    hipError_t e;
    Timing t{nullptr, nullptr, bytes, to_host};
    if (timing_) {
      if ((e = hipEventCreate(&t.start)) != hipSuccess) return (int)e;
      if ((e = hipEventCreate(&t.end)) != hipSuccess) return (int)e;
      if ((e = hipEventRecord(t.start, s)) != hipSuccess) return (int)e;
    }
    if (method_ == kDma) {
      if ((e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDeviceNoCU, s)) != hipSuccess) return (int)e;
    } else if (int rc = launch_link_copy(dst, src, bytes, blocks_, s)) {
      return rc;
    }
    if (timing_) {
      if ((e = hipEventRecord(t.end, s)) != hipSuccess) return (int)e;
      timings_.push_back(t);
    }
    return (int)hipEventRecord(done, s);
  }

  // Busy time per direction: the union of the copies' [start, end] intervals, measured against
  // one base event (copies of one direction may overlap on the two D2H streams).
  void process_timings(bool wait) {
    while (!timings_.empty()) {
      Timing& t = timings_.front();
      if (wait) (void)hipEventSynchronize(t.end);
      else if (hipEventQuery(t.end) != hipSuccess) break;
      float a = 0, b = 0;
      if (hipEventElapsedTime(&a, base_, t.start) == hipSuccess && hipEventElapsedTime(&b, base_, t.end) == hipSuccess) {
        const int d = t.d2h ? 0 : 1;
        const double s = std::max<double>(a, last_end_ms_[d]);
        const double busy = b > s ? b - s : 0.0;
        (t.d2h ? st_.d2h_ms : st_.h2d_ms) += busy;
        (t.d2h ? st_.d2h_done_bytes : st_.h2d_done_bytes) += t.bytes;
        last_end_ms_[d] = std::max<double>(last_end_ms_[d], b);
      }
      (void)hipEventDestroy(t.start);
      (void)hipEventDestroy(t.end);
      timings_.pop_front();
    }
  }

  Method method_ = kDma;
  uint32_t blocks_ = 16;
  bool timing_ = false;
  char* (*alias_)(void*, char*) = nullptr;
  void* alias_ctx_ = nullptr;
  int n_d2h_ = 1;
  hipStream_t d2h_[2] = {nullptr, nullptr};
  hipStream_t h2d_ = nullptr;
  hipEvent_t tmp_ = nullptr, base_ = nullptr;
  std::vector<Gate> gates_;
  StreamRef last_h2d_;
  std::mutex pool_mu_;
  std::vector<hipEvent_t> pool_;
  std::deque<Timing> timings_;
  double last_end_ms_[2] = {-1.0, -1.0};
  LinkStats st_;
};

}  // namespace

std::unique_ptr<Link> make_sdma_link(int device, uint32_t d2h_engine, uint32_t h2d_engine, std::string& err,
                                     int* status) {
  auto link = std::make_unique<SdmaLink>();
  *status = link->init(device, d2h_engine, h2d_engine, err);
  if (*status) return nullptr;
  return link;
}

std::unique_ptr<Link> make_stream_link(int device, uint32_t copy_blocks, bool timing, char* (*alias)(void*, char*),
                                       void* alias_ctx, std::string& err, int* status) {
  (void)device;
  auto link = std::make_unique<StreamLink>();
  *status = link->init(StreamLink::kCopyKernel, copy_blocks, timing, false, alias, alias_ctx);
  if (*status) {
    err = "creating the copy streams failed";
    return nullptr;
  }
  return link;
}

std::unique_ptr<Link> make_hip_dma_link(int device, bool split_d2h, bool timing, std::string& err, int* status) {
  (void)device;
  auto link = std::make_unique<StreamLink>();
  *status = link->init(StreamLink::kDma, 0, timing, split_d2h, nullptr, nullptr);
  if (*status) {
    err = "creating the copy streams failed";
    return nullptr;
  }
  return link;
}

}  // namespace mo
