// Host-link transports (see mo_link.h): SDMA engines through HSA, and a copy kernel on HIP
// streams.
#include "mo_link.h"

#include <hip/hip_runtime_api.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <stdint.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <thread>
#include <vector>

#include "mo_internal.h"

namespace mo {

namespace {

int64_t now_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

constexpr int kMaxGates = 64;
constexpr int kFlagStride = 16;  // uint32 per gate: one 64-byte line each

// Atomically raise *flag to at least `value` (flags only move forward).
void publish(uint32_t* flag, uint32_t value) {
  uint32_t cur = __atomic_load_n(flag, __ATOMIC_RELAXED);
  while (cur < value && !__atomic_compare_exchange_n(flag, &cur, value, true, __ATOMIC_RELEASE, __ATOMIC_RELAXED)) {
  }
}

// ==========================================================================================
// SDMA link

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
  hsa_signal_t sig{0};
  std::atomic<bool> handled{false};
  std::atomic<bool> fail{false};
  bool to_host = true;
  uint64_t bytes = 0;
  int64_t issue_ns = 0;
  uint32_t* flag = nullptr;
  uint32_t value = 0;
  SdmaLink* link = nullptr;
  std::shared_ptr<SdmaCopy> self;  // keeps the copy alive until its completion handler ran
  int64_t retired_ns = 0;
  ~SdmaCopy() override {
    if (sig.handle) hsa_signal_destroy(sig);
  }
  bool done() const override { return handled.load(std::memory_order_acquire); }
  bool failed() const override { return fail.load(std::memory_order_acquire); }
};

struct Job {
  std::shared_ptr<SdmaCopy> copy;
  void* dst = nullptr;
  const void* src = nullptr;
  EventRef wait;                    // issue after this HIP event completed
  std::shared_ptr<SdmaCopy> after;  // and after this copy completed
};

struct GateState {
  uint32_t gen = 0;
  EventRef consumed;
};

hsa_status_t find_agents(hsa_agent_t agent, void* data);

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
    if (hsa_init() != HSA_STATUS_SUCCESS) {
      err = "hsa_init failed";
      return MO_E_STATE;
    }
    hsa_inited_ = true;
    AgentSearch s;
    // Match the HIP device to its HSA agent by PCI location (falls back to the ordinal).
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
    e_d2h_ = pick(d2h_mask, d2h_engine, 0);
    e_h2d_ = pick(h2d_mask, h2d_engine, e_d2h_);
    void* p = nullptr;
    if (hipHostMalloc(&p, sizeof(uint32_t) * kFlagStride * kMaxGates, hipHostMallocCoherent) != hipSuccess) {
      err = "hipHostMalloc of gate flags failed";
      return MO_E_STATE;
    }
    flags_ = (uint32_t*)p;
    for (int i = 0; i < kFlagStride * kMaxGates; ++i) flags_[i] = 0;
    worker_ = std::thread([this] { run(); });
    return 0;
  }

  uint32_t d2h_engine() const { return e_d2h_; }
  uint32_t h2d_engine() const { return e_h2d_; }

  int new_gate(int* gate) override {
    if ((int)gates_.size() >= kMaxGates) return MO_E_INVALID;
    gates_.emplace_back();
    *gate = (int)gates_.size() - 1;
    return 0;
  }

  int d2h(void* dst, const void* src, uint64_t bytes, hipStream_t compute, int gate, CopyRef* out) override {
    EventRef ev;
    if (int rc = take_event(&ev)) return rc;
    hipError_t e = hipEventRecord(ev->ev, compute);
    if (e != hipSuccess) return (int)e;
    auto copy = make_copy(true, bytes, gate);
    if (!copy) return MO_E_STATE;
    Job job;
    job.copy = copy;
    job.dst = dst;
    job.src = src;
    job.wait = std::move(ev);
    enqueue(std::move(job));
    d2h_bytes_ += bytes;
    *out = copy;
    return 0;
  }

  int h2d(void* dst, const void* src, uint64_t bytes, const CopyRef& after, int gate, CopyRef* out) override {
    auto copy = make_copy(false, bytes, gate);
    if (!copy) return MO_E_STATE;
    Job job;
    job.copy = copy;
    job.dst = dst;
    job.src = src;
    job.wait = gates_[gate].consumed;
    job.after = std::dynamic_pointer_cast<SdmaCopy>(after);
    enqueue(std::move(job));
    h2d_bytes_ += bytes;
    *out = copy;
    return 0;
  }

  int wait(int gate, hipStream_t compute) override {
    const uint32_t gen = gates_[gate].gen;
    if (gen == 0) return 0;
    return (int)hipStreamWaitValue32(compute, flag(gate), gen, hipStreamWaitValueGte, 0xFFFFFFFFu);
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
    const int64_t deadline = now_ns() + 300ll * 1000000000ll;
    for (;;) {
      {
        std::lock_guard<std::mutex> lock(mu_);
        if (queue_.empty() && busy_ == 0 && completed_.load() == issued_.load()) break;
      }
      if (now_ns() > deadline) return MO_E_STATE;
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    sweep();
    return 0;
  }

  void stats(LinkStats* out) override {
    out->d2h_bytes = d2h_bytes_;
    out->h2d_bytes = h2d_bytes_;
    out->d2h_done_bytes = done_bytes_[0].load();
    out->h2d_done_bytes = done_bytes_[1].load();
    out->d2h_ms = busy_ns_[0].load() / 1e6;
    out->h2d_ms = busy_ns_[1].load() / 1e6;
    out->failures = failures_.load();
  }

  void reset_stats() override {
    d2h_bytes_ = h2d_bytes_ = 0;
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

  // Completion handler (HSA async-event thread): publish, account, retire. No HIP calls.
  static bool on_done(hsa_signal_value_t value, void* arg) {
    auto* c = (SdmaCopy*)arg;
    SdmaLink* link = c->link;
    if (value < 0) {
      c->fail.store(true, std::memory_order_release);
      link->failures_++;
    }
    const int dir = c->to_host ? 0 : 1;
    const int64_t t = now_ns();
    const int64_t prev = link->last_done_ns_[dir].exchange(t);
    const int64_t start = c->issue_ns > prev ? c->issue_ns : prev;
    link->busy_ns_[dir] += t > start ? (uint64_t)(t - start) : 0;
    link->done_bytes_[dir] += c->bytes;
    if (c->flag) publish(c->flag, c->value);
    c->handled.store(true, std::memory_order_release);
    {
      std::lock_guard<std::mutex> lock(link->retire_mu_);
      c->retired_ns = t;
      link->retired_.push_back(std::move(c->self));
    }
    link->completed_++;
    return false;  // one-shot
  }

 private:
  static uint32_t pick(uint32_t mask, uint32_t want, uint32_t avoid) {
    if (want && (mask & want)) return want & (~want + 1);
    for (int i = 0; i < 32; ++i)
      if ((mask & (1u << i)) && (1u << i) != avoid) return 1u << i;
    return mask & (~mask + 1);
  }

  uint32_t* flag(int gate) { return flags_ + gate * kFlagStride; }

  std::shared_ptr<SdmaCopy> make_copy(bool to_host, uint64_t bytes, int gate) {
    auto c = std::make_shared<SdmaCopy>();
    if (hsa_signal_create(1, 0, nullptr, &c->sig) != HSA_STATUS_SUCCESS) return nullptr;
    c->to_host = to_host;
    c->bytes = bytes;
    c->link = this;
    c->flag = flag(gate);
    c->value = ++gates_[gate].gen;
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
      hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming | hipEventBlockingSync);
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
      queue_.push_back(std::move(job));
    }
    cv_.notify_one();
  }

  // Issuer thread: jobs in FIFO order. Every event a job waits for was recorded before the job
  // was enqueued, and every stream wait on a job's gate is enqueued after the job, so waiting
  // here can never depend on a job behind this one.
  void run() {
    if (hipSetDevice(device_) != hipSuccess) {
      // Still drain the queue below so no stream waits forever.
    }
    for (;;) {
      Job job;
      {
        std::unique_lock<std::mutex> lock(mu_);
        cv_.wait_for(lock, std::chrono::milliseconds(5), [this] { return stop_ || !queue_.empty(); });
        if (queue_.empty()) {
          if (stop_) return;
          lock.unlock();
          sweep();
          continue;
        }
        job = std::move(queue_.front());
        queue_.pop_front();
        busy_++;
      }
      issue(job);
      {
        std::lock_guard<std::mutex> lock(mu_);
        busy_--;
      }
      sweep();
    }
  }

  void issue(Job& job) {
    if (job.wait) {
      (void)hipEventSynchronize(job.wait->ev);
      job.wait.reset();
    }
    auto& c = job.copy;
    bool ok = true;
    if (job.after) {
      // The host bytes must have arrived before they leave again.
      const int64_t deadline = now_ns() + 120ll * 1000000000ll;
      while (!job.after->done() && now_ns() < deadline) std::this_thread::sleep_for(std::chrono::microseconds(20));
      ok = job.after->done() && !job.after->failed();
      job.after.reset();
    }
    c->issue_ns = now_ns();
    c->self = c;
    issued_++;
    hsa_status_t st = HSA_STATUS_ERROR;
    if (ok) {
      st = hsa_amd_memory_async_copy_on_engine(job.dst, c->to_host ? cpu_ : gpu_, job.src, c->to_host ? gpu_ : cpu_,
                                               c->bytes, 0, nullptr, c->sig,
                                               (hsa_amd_sdma_engine_id_t)(c->to_host ? e_d2h_ : e_h2d_), true);
    }
    if (st == HSA_STATUS_SUCCESS) {
      st = hsa_amd_signal_async_handler(c->sig, HSA_SIGNAL_CONDITION_LT, 1, on_done, c.get());
      if (st == HSA_STATUS_SUCCESS) return;
      // No handler: wait here and complete inline.
      hsa_signal_value_t v = 1;
      while ((v = hsa_signal_wait_scacquire(c->sig, HSA_SIGNAL_CONDITION_LT, 1, 1000000, HSA_WAIT_STATE_BLOCKED)) >= 1) {
      }
      on_done(v, c.get());
      return;
    }
    // Never leave a stream waiting on a copy that will not happen: complete it as failed.
    on_done(-1, c.get());
  }

  // Destroy retired copies a while after their handler ran (their signals are then idle).
  void sweep() {
    std::vector<std::shared_ptr<SdmaCopy>> drop;
    {
      std::lock_guard<std::mutex> lock(retire_mu_);
      const int64_t limit = now_ns() - 5000000;  // 5 ms
      while (!retired_.empty() && retired_.front()->retired_ns < limit) {
        drop.push_back(std::move(retired_.front()));
        retired_.pop_front();
      }
    }
  }

  void shutdown() {
    if (worker_.joinable()) {
      {
        std::lock_guard<std::mutex> lock(mu_);
        stop_ = true;
      }
      cv_.notify_all();
      worker_.join();  // drains the queue first
      (void)synchronize();
      std::this_thread::sleep_for(std::chrono::milliseconds(10));
    }
    gates_.clear();
    {
      std::lock_guard<std::mutex> lock(retire_mu_);
      retired_.clear();
    }
    {
      std::lock_guard<std::mutex> lock(ev_mu_);
      for (hipEvent_t e : ev_pool_) (void)hipEventDestroy(e);
      ev_pool_.clear();
    }
    if (flags_) {
      (void)hipHostFree(flags_);
      flags_ = nullptr;
    }
    if (hsa_inited_) {
      hsa_shut_down();
      hsa_inited_ = false;
    }
  }

  int device_ = 0;
  bool hsa_inited_ = false;
  hsa_agent_t gpu_{0}, cpu_{0};
  uint32_t e_d2h_ = 0, e_h2d_ = 0;
  uint32_t* flags_ = nullptr;
  std::vector<GateState> gates_;  // touched by API threads only (engine mutex)

  std::mutex ev_mu_;
  std::vector<hipEvent_t> ev_pool_;

  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<Job> queue_;
  int busy_ = 0;
  bool stop_ = false;
  std::thread worker_;

  std::mutex retire_mu_;
  std::deque<std::shared_ptr<SdmaCopy>> retired_;

  std::atomic<uint64_t> issued_{0}, completed_{0}, failures_{0};
  std::atomic<int64_t> last_done_ns_[2]{{0}, {0}};
  std::atomic<uint64_t> busy_ns_[2]{{0}, {0}};
  std::atomic<uint64_t> done_bytes_[2]{{0}, {0}};
  uint64_t d2h_bytes_ = 0, h2d_bytes_ = 0;
};

EventHold::~EventHold() {
  if (owner && ev) owner->return_event(ev);
}

// ==========================================================================================
// Stream link: copy kernel on dedicated HIP streams

struct StreamCopy : CopyState {
  hipEvent_t ev = nullptr;
  std::vector<hipEvent_t>* pool = nullptr;
  std::mutex* pool_mu = nullptr;
  ~StreamCopy() override {
    if (ev) {
      std::lock_guard<std::mutex> lock(*pool_mu);
      pool->push_back(ev);
    }
  }
  bool done() const override { return hipEventQuery(ev) == hipSuccess; }
  bool failed() const override { return false; }
};

class StreamLink : public Link {
 public:
  ~StreamLink() override {
    (void)synchronize();
    for (auto& g : gates_) {
      if (g.ready) (void)hipEventDestroy(g.ready);
      if (g.consumed) (void)hipEventDestroy(g.consumed);
    }
    for (auto& t : timings_) {
      (void)hipEventDestroy(t.start);
      (void)hipEventDestroy(t.end);
    }
    for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
    if (tmp_) (void)hipEventDestroy(tmp_);
    if (d2h_) (void)hipStreamDestroy(d2h_);
    if (h2d_) (void)hipStreamDestroy(h2d_);
  }

  int init(uint32_t blocks, bool timing, char* (*alias)(void*, char*), void* ctx) {
    blocks_ = blocks ? blocks : 16;
    timing_ = timing;
    alias_ = alias;
    alias_ctx_ = ctx;
    hipError_t e;
    if ((e = hipStreamCreateWithFlags(&d2h_, hipStreamNonBlocking)) != hipSuccess) return (int)e;
    if ((e = hipStreamCreateWithFlags(&h2d_, hipStreamNonBlocking)) != hipSuccess) return (int)e;
    if ((e = hipEventCreateWithFlags(&tmp_, hipEventDisableTiming)) != hipSuccess) return (int)e;
    return 0;
  }

  int new_gate(int* gate) override {
    Gate g;
    hipError_t e;
    if ((e = hipEventCreateWithFlags(&g.ready, hipEventDisableTiming)) != hipSuccess) return (int)e;
    if ((e = hipEventCreateWithFlags(&g.consumed, hipEventDisableTiming)) != hipSuccess) return (int)e;
    gates_.push_back(g);
    *gate = (int)gates_.size() - 1;
    return 0;
  }

  int d2h(void* dst, const void* src, uint64_t bytes, hipStream_t compute, int gate, CopyRef* out) override {
    hipError_t e;
    if ((e = hipEventRecord(tmp_, compute)) != hipSuccess) return (int)e;
    if ((e = hipStreamWaitEvent(d2h_, tmp_, 0)) != hipSuccess) return (int)e;
    return copy(d2h_, alias_(alias_ctx_, (char*)dst), src, bytes, true, gate, out);
  }

  int h2d(void* dst, const void* src, uint64_t bytes, const CopyRef& after, int gate, CopyRef* out) override {
    hipError_t e;
    Gate& g = gates_[gate];
    if (g.consumed_recorded && (e = hipStreamWaitEvent(h2d_, g.consumed, 0)) != hipSuccess) return (int)e;
    auto prev = std::dynamic_pointer_cast<StreamCopy>(after);
    if (prev && (e = hipStreamWaitEvent(h2d_, prev->ev, 0)) != hipSuccess) return (int)e;
    return copy(h2d_, dst, alias_(alias_ctx_, (char*)src), bytes, false, gate, out);
  }

  int wait(int gate, hipStream_t compute) override {
    Gate& g = gates_[gate];
    if (!g.used) return 0;
    return (int)hipStreamWaitEvent(compute, g.ready, 0);
  }

  int consumed(int gate, hipStream_t compute) override {
    Gate& g = gates_[gate];
    hipError_t e = hipEventRecord(g.consumed, compute);
    g.consumed_recorded = e == hipSuccess;
    return (int)e;
  }

  int synchronize() override {
    hipError_t e;
    if (d2h_ && (e = hipStreamSynchronize(d2h_)) != hipSuccess) return (int)e;
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
  }
  const char* name() const override { return "kernel"; }

 private:
  struct Gate {
    hipEvent_t ready = nullptr, consumed = nullptr;
    bool used = false, consumed_recorded = false;
  };
  struct Timing {
    hipEvent_t start, end;
    uint64_t bytes;
    bool d2h;
  };

  int copy(hipStream_t s, void* dst, const void* src, uint64_t bytes, bool to_host, int gate, CopyRef* out) {
    hipError_t e;
    Timing t{nullptr, nullptr, bytes, to_host};
    if (timing_) {
      if ((e = hipEventCreate(&t.start)) != hipSuccess) return (int)e;
      if ((e = hipEventCreate(&t.end)) != hipSuccess) return (int)e;
      if ((e = hipEventRecord(t.start, s)) != hipSuccess) return (int)e;
    }
    if (int rc = launch_link_copy(dst, src, bytes, blocks_, s)) return rc;
    if (timing_) {
      if ((e = hipEventRecord(t.end, s)) != hipSuccess) return (int)e;
      timings_.push_back(t);
    }
    auto c = std::make_shared<StreamCopy>();
    {
      std::lock_guard<std::mutex> lock(pool_mu_);
      if (!pool_.empty()) {
        c->ev = pool_.back();
        pool_.pop_back();
      }
    }
    if (!c->ev && (e = hipEventCreateWithFlags(&c->ev, hipEventDisableTiming)) != hipSuccess) return (int)e;
    c->pool = &pool_;
    c->pool_mu = &pool_mu_;
    if ((e = hipEventRecord(c->ev, s)) != hipSuccess) return (int)e;
    Gate& g = gates_[gate];
    if ((e = hipEventRecord(g.ready, s)) != hipSuccess) return (int)e;
    g.used = true;
    (to_host ? st_.d2h_bytes : st_.h2d_bytes) += bytes;
    *out = c;
    return 0;
  }

  void process_timings(bool wait) {
    while (!timings_.empty()) {
      Timing& t = timings_.front();
      if (wait) (void)hipEventSynchronize(t.end);
      else if (hipEventQuery(t.end) != hipSuccess) break;
      float ms = 0;
      if (hipEventElapsedTime(&ms, t.start, t.end) == hipSuccess) {
        if (t.d2h) {
          st_.d2h_ms += ms;
          st_.d2h_done_bytes += t.bytes;
        } else {
          st_.h2d_ms += ms;
          st_.h2d_done_bytes += t.bytes;
        }
      }
      (void)hipEventDestroy(t.start);
      (void)hipEventDestroy(t.end);
      timings_.pop_front();
    }
  }

  uint32_t blocks_ = 16;
  bool timing_ = false;
  char* (*alias_)(void*, char*) = nullptr;
  void* alias_ctx_ = nullptr;
  hipStream_t d2h_ = nullptr, h2d_ = nullptr;
  hipEvent_t tmp_ = nullptr;
  std::vector<Gate> gates_;
  std::mutex pool_mu_;
  std::vector<hipEvent_t> pool_;
  std::deque<Timing> timings_;
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
  *status = link->init(copy_blocks, timing, alias, alias_ctx);
  if (*status) {
    err = "creating the copy streams failed";
    return nullptr;
  }
  return link;
}

}  // namespace mo
