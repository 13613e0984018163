// Host gradient accumulation without a blocking copy: the native side of
// moss_offload.host_gradients.HostGradientAccumulator.
//
// Replaces what FusedAdafactor._stash_gradient_on_host does for a device gradient
// (training/fused_adafactor.py:327-355): the reference allocates an fp32 pinned tensor, copies
// the gradient into it with a blocking copy_ (the hook returns only once the GPU has finished
// reading the gradient), then adds it on the host into the parameter's fp32 accumulator. Here:
//   1. on the caller's stream the gradient is copied into a device staging slot (so the
//      caller may release the gradient at once: its storage is reused only by later work on
//      that stream);
//   2. an SDMA engine copies the slot to a pinned host staging buffer once the stream has
//      passed step 1 (the issuer thread of the link, no GPU wait on host memory);
//   3. one worker thread takes the copies in issue order and converts + accumulates each into
//      the destination fp32 buffer (dst = x for the first contribution of a step, dst += x
//      after), split over a small pool of host threads, then frees the slot.
// The fp32 additions are the reference's (x converted exactly from bf16/fp16/fp32, one IEEE
// single-precision add per element and contribution, contributions in issue order), so the
// accumulated values are bitwise the reference's. The link carries the gradient in its own
// dtype (bf16: half the reference's bytes, which converts on the device first).
// Backpressure: when every slot is in flight, a call blocks the host until the oldest slot is
// free; every wait is bounded.
#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/moss_offload.h"
#include "mo_link.h"

namespace mo {
int set_error(int code, const std::string& msg);
int set_hip_error(int e, const char* what);
}  // namespace mo

namespace {

using Clock = std::chrono::steady_clock;
constexpr double kWaitLimitS = 300.0;  // bound on every host wait
constexpr uint64_t kParallelMin = 1 << 18;  // elements below which one thread accumulates

double ms_since(Clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

float from_half(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {  // subnormal: mant * 2^-24, exact in fp32
      float f = (float)mant * 5.9604644775390625e-8f;
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    // infinities keep their sign; NaNs come out quiet with their payload, as the device's
    // conversion (the reference converts on the device before its copy) makes them
    bits = sign | 0x7f800000u | (mant ? (mant | 0x200u) << 13 : 0u);
  } else {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

template <int kDtype>
void accumulate_range(float* dst, const void* src, uint64_t lo, uint64_t hi, bool first) {
  for (uint64_t i = lo; i < hi; ++i) {
    float x;
    if (kDtype == MO_DTYPE_BF16) {
      const uint32_t bits = (uint32_t)((const uint16_t*)src)[i] << 16;
      memcpy(&x, &bits, 4);
    } else if (kDtype == MO_DTYPE_F16) {
      x = from_half(((const uint16_t*)src)[i]);
    } else {
      x = ((const float*)src)[i];
    }
    dst[i] = first ? x : dst[i] + x;
  }
}

void accumulate(float* dst, const void* src, int dtype, uint64_t lo, uint64_t hi, bool first) {
  switch (dtype) {
    case MO_DTYPE_BF16: accumulate_range<MO_DTYPE_BF16>(dst, src, lo, hi, first); break;
    case MO_DTYPE_F16: accumulate_range<MO_DTYPE_F16>(dst, src, lo, hi, first); break;
    default: accumulate_range<MO_DTYPE_F32>(dst, src, lo, hi, first); break;
  }
}

uint32_t dtype_size(uint32_t dtype) { return dtype == MO_DTYPE_F32 ? 4 : 2; }

// A fixed pool that runs one ranged task at a time: the caller and the pool's threads take
// chunks of [0, n) from an atomic counter.
class RangePool {
 public:
  explicit RangePool(uint32_t threads) {
    for (uint32_t i = 0; i + 1 < threads; ++i) threads_.emplace_back([this] { loop(); });
  }
  ~RangePool() {
    {
      std::lock_guard<std::mutex> lock(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : threads_) t.join();
  }
  uint32_t size() const { return (uint32_t)threads_.size() + 1; }
  // fn(lo, hi) over [0, n) in chunks; returns when every chunk is done.
  void run(uint64_t n, uint64_t chunk, const std::function<void(uint64_t, uint64_t)>& fn) {
    if (threads_.empty() || n <= chunk) {
      fn(0, n);
      return;
    }
    {
      std::lock_guard<std::mutex> lock(mu_);
      fn_ = &fn;
      n_ = n;
      chunk_ = chunk;
      next_.store(0);
      active_ = (uint32_t)threads_.size();
      ++generation_;
    }
    cv_.notify_all();
    work();
    std::unique_lock<std::mutex> lock(mu_);
    done_cv_.wait(lock, [this] { return active_ == 0; });
    fn_ = nullptr;
  }

 private:
  void work() {
    for (;;) {
      const uint64_t lo = next_.fetch_add(chunk_);
      if (lo >= n_) return;
      (*fn_)(lo, lo + chunk_ < n_ ? lo + chunk_ : n_);
    }
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lock(mu_);
        cv_.wait(lock, [&] { return stop_ || generation_ != seen; });
        if (stop_) return;
        seen = generation_;
      }
      work();
      {
        std::lock_guard<std::mutex> lock(mu_);
        --active_;
      }
      done_cv_.notify_all();
    }
  }

  std::vector<std::thread> threads_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  bool stop_ = false;
  uint64_t generation_ = 0;
  const std::function<void(uint64_t, uint64_t)>* fn_ = nullptr;
  uint64_t n_ = 0, chunk_ = 1;
  std::atomic<uint64_t> next_{0};
  uint32_t active_ = 0;
};

class DeviceGuard {
 public:
  explicit DeviceGuard(int device) : dev_(device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != device) (void)hipSetDevice(device);
  }
  ~DeviceGuard() {
    if (prev_ >= 0 && prev_ != dev_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = -1, dev_ = -1;
};

}  // namespace

struct mo_gradacc {
  struct Slot {
    void* dev = nullptr;
    void* host = nullptr;
    int gate = 0;
    bool busy = false;
  };
  struct Job {
    uint32_t slot;
    mo::CopyRef copy;
    uint64_t key;  // the destination buffer of the call (what mo_gradacc_wait names)
    float* dst;
    uint64_t count;
    uint32_t dtype;
    bool first;
  };

  std::mutex mu;
  std::condition_variable cv;  // slot freed, job queued, job finished
  int device = 0;
  uint64_t slot_bytes = 0;
  std::unique_ptr<mo::Link> link;
  std::vector<Slot> slots;
  std::deque<Job> queue;  // issue order; the front is the worker's current job
  std::map<uint64_t, uint64_t> pending;  // key -> queued jobs
  std::unique_ptr<RangePool> pool;
  std::thread worker;
  bool stop = false;
  int error = 0;  // latched status of a failed copy or wait
  std::string error_msg;
  // stats (under mu)
  uint64_t calls = 0, chunks = 0, bytes = 0, elements = 0;
  uint64_t host_blocks = 0;
  double host_block_ms = 0, accumulate_ms = 0;

  void run_worker();
};

void mo_gradacc::run_worker() {
  for (;;) {
    Job job;
    {
      std::unique_lock<std::mutex> lock(mu);
      cv.wait(lock, [&] { return stop || !queue.empty(); });
      if (queue.empty()) return;  // stop with nothing left
      job = queue.front();
    }
    // wait for the SDMA copy of this slot (bounded, backing off from 5 to 100 us)
    const auto t0 = Clock::now();
    auto gap = std::chrono::microseconds(5);
    bool failed = false;
    while (!job.copy->done()) {
      if (std::chrono::duration<double>(Clock::now() - t0).count() > kWaitLimitS) {
        failed = true;
        break;
      }
      std::this_thread::sleep_for(gap);
      if (gap < std::chrono::microseconds(100)) gap *= 2;
    }
    failed = failed || job.copy->failed();
    double acc_ms = 0;
    if (!failed) {
      const auto a0 = Clock::now();
      const void* src = slots[job.slot].host;
      const uint64_t chunk = job.count < kParallelMin ? job.count : (job.count + pool->size() - 1) / pool->size();
      pool->run(job.count, chunk ? chunk : 1, [&](uint64_t lo, uint64_t hi) {
        accumulate(job.dst, src, (int)job.dtype, lo, hi, job.first);
      });
      acc_ms = ms_since(a0);
    }
    {
      std::lock_guard<std::mutex> lock(mu);
      if (failed && !error) {
        error = MO_E_STATE;
        error_msg = "gradient D2H copy failed or did not finish within the time limit";
      }
      slots[job.slot].busy = false;
      queue.pop_front();
      if (--pending[job.key] == 0) pending.erase(job.key);
      accumulate_ms += acc_ms;
      elements += failed ? 0 : job.count;
    }
    cv.notify_all();
  }
}

namespace {

#define MO_GRADACC_CHECK(g) \
  if (!(g)) return mo::set_error(MO_E_INVALID, "null gradient accumulator")

int latched(mo_gradacc* g) { return g->error ? mo::set_error(g->error, g->error_msg) : 0; }

// Wait (holding `lock`) until `ready()`; bounded. Counts as a host block when it had to wait.
template <class Pred>
int bounded_wait(mo_gradacc* g, std::unique_lock<std::mutex>& lock, Pred ready, const char* what) {
  if (ready()) return 0;
  const auto t0 = Clock::now();
  const bool ok = g->cv.wait_for(lock, std::chrono::duration<double>(kWaitLimitS), ready);
  g->host_blocks += 1;
  g->host_block_ms += ms_since(t0);
  if (!ok) return mo::set_error(MO_E_STATE, std::string(what) + " did not finish within the time limit");
  return 0;
}

}  // namespace

extern "C" {

int mo_gradacc_create(int device, uint32_t slots, uint64_t slot_bytes, uint32_t host_threads, uint32_t d2h_engine,
                      mo_gradacc** out) {
  if (!out) return mo::set_error(MO_E_INVALID, "null output");
  *out = nullptr;
  if (slots == 0 || slots > 64) return mo::set_error(MO_E_INVALID, "slots must be 1..64");
  if (slot_bytes < 4096 || slot_bytes % 4096) return mo::set_error(MO_E_INVALID, "slot_bytes must be a positive multiple of 4096");
  if (host_threads == 0 || host_threads > 256) return mo::set_error(MO_E_INVALID, "host_threads must be 1..256");
  try {
    auto g = std::make_unique<mo_gradacc>();
    g->device = device;
    g->slot_bytes = slot_bytes;
    DeviceGuard guard(device);
    std::string err;
    int status = 0;
    g->link = mo::make_sdma_link(device, d2h_engine, 0, err, &status);
    if (!g->link) return mo::set_error(status ? status : MO_E_STATE, "SDMA link: " + err);
    g->slots.resize(slots);
    for (auto& s : g->slots) {
      hipError_t e = hipMalloc(&s.dev, slot_bytes);
      if (e != hipSuccess) return mo::set_hip_error((int)e, "hipMalloc (gradient staging slot)");
      e = hipHostMalloc(&s.host, slot_bytes, hipHostMallocDefault);
      if (e != hipSuccess) return mo::set_hip_error((int)e, "hipHostMalloc (gradient host staging)");
      if (int rc = g->link->new_gate(&s.gate)) return mo::set_hip_error(rc, "slot gate");
    }
    g->pool = std::make_unique<RangePool>(host_threads);
    mo_gradacc* raw = g.get();
    g->worker = std::thread([raw] { raw->run_worker(); });
    *out = g.release();
    return 0;
  } catch (const std::exception& ex) {
    return mo::set_error(MO_E_STATE, std::string("internal error: ") + ex.what());
  }
}

int mo_gradacc_destroy(mo_gradacc* g) {
  if (!g) return 0;
  int rc = 0;
  {
    std::unique_lock<std::mutex> lock(g->mu);
    if (bounded_wait(g, lock, [&] { return g->queue.empty(); }, "pending gradient accumulation")) rc = MO_E_STATE;
    g->stop = true;
  }
  g->cv.notify_all();
  if (g->worker.joinable()) g->worker.join();
  {
    DeviceGuard guard(g->device);
    if (g->link && g->link->synchronize()) rc = MO_E_STATE;
    g->link.reset();
    for (auto& s : g->slots) {
      if (s.dev) (void)hipFree(s.dev);
      if (s.host) (void)hipHostFree(s.host);
    }
  }
  g->pool.reset();
  delete g;
  return rc ? mo::set_error(MO_E_STATE, "gradient accumulator did not drain in time") : 0;
}

int mo_gradacc_accumulate(mo_gradacc* g, uint64_t dst_host, uint32_t first, uint64_t src_device, uint32_t dtype,
                          uint64_t count, uint64_t stream) {
  MO_GRADACC_CHECK(g);
  if (!dst_host || !src_device) return mo::set_error(MO_E_INVALID, "null buffer");
  if (dtype != MO_DTYPE_BF16 && dtype != MO_DTYPE_F16 && dtype != MO_DTYPE_F32)
    return mo::set_error(MO_E_INVALID, "gradient dtype must be fp16, bf16 or fp32");
  if (dst_host % 4 || src_device % dtype_size(dtype)) return mo::set_error(MO_E_INVALID, "misaligned buffer");
  if (count == 0) return 0;
  try {
    std::unique_lock<std::mutex> lock(g->mu);
    if (int rc = latched(g)) return rc;
    DeviceGuard guard(g->device);
    const uint64_t esize = dtype_size(dtype);
    const uint64_t per_slot = g->slot_bytes / esize;
    g->calls += 1;
    for (uint64_t off = 0; off < count; off += per_slot) {
      const uint64_t n = count - off < per_slot ? count - off : per_slot;
      uint32_t slot = 0;
      auto free_slot = [&] {
        for (uint32_t i = 0; i < g->slots.size(); ++i)
          if (!g->slots[i].busy) {
            slot = i;
            return true;
          }
        return g->error != 0;
      };
      if (int rc = bounded_wait(g, lock, free_slot, "a gradient staging slot")) return rc;
      if (int rc = latched(g)) return rc;
      auto& s = g->slots[slot];
      // the slot is free: its previous host accumulation (and so its previous D2H) finished
      const hipError_t e = hipMemcpyAsync(s.dev, (const char*)src_device + off * esize, n * esize,
                                          hipMemcpyDeviceToDevice, (hipStream_t)stream);
      if (e != hipSuccess) return mo::set_hip_error((int)e, "hipMemcpyAsync (gradient -> staging slot)");
      mo::CopyRef copy;
      if (int rc = g->link->d2h(s.host, s.dev, n * esize, (hipStream_t)stream, s.gate, &copy))
        return mo::set_hip_error(rc, "gradient D2H");
      s.busy = true;
      g->queue.push_back({slot, copy, dst_host, (float*)dst_host + off, n, dtype, first != 0});
      g->pending[dst_host] += 1;
      g->chunks += 1;
      g->bytes += n * esize;
      g->cv.notify_all();
    }
    return 0;
  } catch (const std::exception& ex) {
    return mo::set_error(MO_E_STATE, std::string("internal error: ") + ex.what());
  }
}

int mo_gradacc_wait(mo_gradacc* g, uint64_t dst_host) {
  MO_GRADACC_CHECK(g);
  try {
    std::unique_lock<std::mutex> lock(g->mu);
    auto ready = [&] { return dst_host ? g->pending.count(dst_host) == 0 : g->queue.empty(); };
    if (int rc = bounded_wait(g, lock, ready, "gradient accumulation")) return rc;
    return latched(g);
  } catch (const std::exception& ex) {
    return mo::set_error(MO_E_STATE, std::string("internal error: ") + ex.what());
  }
}

int mo_gradacc_get_stats(mo_gradacc* g, mo_gradacc_stats* out) {
  MO_GRADACC_CHECK(g);
  if (!out) return mo::set_error(MO_E_INVALID, "null output");
  std::lock_guard<std::mutex> lock(g->mu);
  mo::LinkStats ls;
  g->link->stats(&ls);
  out->calls = g->calls;
  out->chunks = g->chunks;
  out->bytes = g->bytes;
  out->elements = g->elements;
  out->d2h_done_bytes = ls.d2h_done_bytes;
  out->d2h_ms = ls.d2h_ms;
  out->accumulate_ms = g->accumulate_ms;
  out->host_blocks = g->host_blocks;
  out->host_block_ms = g->host_block_ms;
  out->pending_chunks = g->queue.size();
  out->copy_failures = ls.failures;
  return 0;
}

int mo_gradacc_reset_stats(mo_gradacc* g) {
  MO_GRADACC_CHECK(g);
  std::lock_guard<std::mutex> lock(g->mu);
  g->link->reset_stats();
  g->calls = g->chunks = g->bytes = g->elements = g->host_blocks = 0;
  g->host_block_ms = g->accumulate_ms = 0;
  return 0;
}

}  // extern "C"
