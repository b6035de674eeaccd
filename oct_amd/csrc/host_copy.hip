// Host <-> device copies of caller-owned (pageable) host buffers.
//
// The host-pointer entry points (prometheus_reactor_runtime_sgemm and the
// other calls that take host arrays, reactor_sgemm.cpp:4152-4191) receive
// ordinary pageable memory.  HIP copies such memory through its own staging
// at 8-23 GB/s host-to-device and ~17 GB/s device-to-host on MI355X, while
// DMA from pinned memory runs at ~57 GB/s both ways.  Large copies therefore
// go through a ring of pinned chunks: the host threads copy chunk i into a
// pinned slot while the DMA engine moves chunk i-1, and the reverse for
// downloads.  Four host threads (the caller and three workers) copy
// pageable <-> pinned at 70-95 GB/s; the pipelined upload measured 47 GB/s.
// Copies below kPipeMin bytes, or when pinned memory is unavailable, keep
// hipMemcpyAsync.  host_memcpy lends the same threads to the async and batch
// entries' copies between caller buffers and their own pinned staging.
// Nothing here changes what is copied, only how.
#include <string.h>

#include <condition_variable>
#include <mutex>
#include <new>
#include <system_error>
#include <thread>

#include "reactor_internal.h"

namespace prom {
namespace {

constexpr size_t kPipeChunk = 8u << 20;
constexpr int kPipeSlots = 4;
constexpr size_t kPipeMin = 4u << 20;
constexpr int kCopyThreads = 4;
constexpr size_t kParallelMin = 1u << 20;

// memcpy split over the calling thread and kCopyThreads - 1 persistent
// workers.  One job at a time (callers hold the pipe's mutex).  The workers
// are never joined: they wait on the condition variable until the process
// ends, and the pool is never destroyed, so no exit-time destructor races
// them.
class CopyPool {
 public:
  void copy(char* dst, const char* src, size_t bytes) {
    if (bytes < kParallelMin || !start()) {
      memcpy(dst, src, bytes);
      return;
    }
    {
      std::lock_guard<std::mutex> g(mu_);
      dst_ = dst;
      src_ = src;
      bytes_ = bytes;
      per_ = ((bytes + threads_ - 1) / threads_ + 63) & ~(size_t)63;
      pending_ = threads_ - 1;
      ++generation_;
    }
    work_.notify_all();
    part(0);
    std::unique_lock<std::mutex> g(mu_);
    done_.wait(g, [&] { return pending_ == 0; });
  }

 private:
  bool start() {
    if (started_) return threads_ > 1;
    started_ = true;
    for (int id = 1; id < kCopyThreads; ++id) {
      try {
        std::thread([this, id] { worker(id); }).detach();
        threads_ = id + 1;
      } catch (const std::system_error&) {
        break;
      }
    }
    return threads_ > 1;
  }
  void part(int id) {
    const size_t off = (size_t)id * per_;
    if (off < bytes_) memcpy(dst_ + off, src_ + off, std::min(per_, bytes_ - off));
  }
  void worker(int id) {
    uint64_t seen = 0;
    std::unique_lock<std::mutex> g(mu_);
    for (;;) {
      work_.wait(g, [&] { return generation_ != seen; });
      seen = generation_;
      // A job started before this worker existed is not its to run.
      if (id >= threads_) continue;
      g.unlock();
      part(id);
      g.lock();
      if (--pending_ == 0) done_.notify_one();
    }
  }

  std::mutex mu_;
  std::condition_variable work_, done_;
  bool started_ = false;
  int threads_ = 1;
  uint64_t generation_ = 0;
  int pending_ = 0;
  char* dst_ = nullptr;
  const char* src_ = nullptr;
  size_t bytes_ = 0, per_ = 0;
};

struct Pipe {
  std::mutex mu;
  bool tried = false;
  bool ready = false;
  char* slot[kPipeSlots] = {};
  hipEvent_t done[kPipeSlots] = {};
  bool busy[kPipeSlots] = {};  // a DMA was recorded on done[i] and not yet waited for
  CopyPool pool;

  // Pinned slots and their events, once per process; on failure the copies
  // fall back to hipMemcpyAsync.
  bool init() {
    if (tried) return ready;
    tried = true;
    for (int i = 0; i < kPipeSlots; ++i) {
      if (hipHostMalloc(reinterpret_cast<void**>(&slot[i]), kPipeChunk, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        return false;
      }
    }
    ready = true;
    return true;
  }
  hipError_t wait(int s) {
    if (!busy[s]) return hipSuccess;
    const hipError_t e = hipEventSynchronize(done[s]);
    if (e == hipSuccess) busy[s] = false;
    return e;
  }
};

Pipe& pipe() {
  static Pipe* p = new Pipe();  // never destroyed (its workers outlive static destruction)
  return *p;
}

}  // namespace

void host_memcpy(void* dst, const void* src, size_t bytes) {
  if (bytes < kParallelMin) {
    memcpy(dst, src, bytes);
    return;
  }
  Pipe& p = pipe();
  std::lock_guard<std::mutex> g(p.mu);
  p.pool.copy(static_cast<char*>(dst), static_cast<const char*>(src), bytes);
}

hipError_t upload_host(void* dst, const void* src, size_t bytes, hipStream_t stream) {
  if (bytes < kPipeMin) return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream);
  Pipe& p = pipe();
  std::lock_guard<std::mutex> g(p.mu);
  if (!p.init()) return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream);
  const char* s8 = static_cast<const char*>(src);
  char* d8 = static_cast<char*>(dst);
  int s = 0;
  for (size_t off = 0; off < bytes; off += kPipeChunk, s = (s + 1) % kPipeSlots) {
    hipError_t e = p.wait(s);
    if (e != hipSuccess) return e;
    const size_t len = std::min(kPipeChunk, bytes - off);
    p.pool.copy(p.slot[s], s8 + off, len);
    e = hipMemcpyAsync(d8 + off, p.slot[s], len, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return e;
    e = hipEventRecord(p.done[s], stream);
    if (e != hipSuccess) return e;
    p.busy[s] = true;
  }
  return hipSuccess;
}

hipError_t download_host(void* dst, const void* src, size_t bytes, hipStream_t stream) {
  auto direct = [&] {
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream);
    return e != hipSuccess ? e : hipStreamSynchronize(stream);
  };
  if (bytes < kPipeMin) return direct();
  Pipe& p = pipe();
  std::lock_guard<std::mutex> g(p.mu);
  if (!p.init()) return direct();
  const char* s8 = static_cast<const char*>(src);
  char* d8 = static_cast<char*>(dst);
  const size_t chunks = (bytes + kPipeChunk - 1) / kPipeChunk;
  // Chunk i travels through slot i % kPipeSlots; up to kPipeSlots DMAs are
  // queued ahead of the host copies.
  auto enqueue = [&](size_t i) -> hipError_t {
    const int s = (int)(i % kPipeSlots);
    hipError_t e = p.wait(s);
    if (e != hipSuccess) return e;
    const size_t off = i * kPipeChunk;
    e = hipMemcpyAsync(p.slot[s], s8 + off, std::min(kPipeChunk, bytes - off), hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return e;
    e = hipEventRecord(p.done[s], stream);
    if (e == hipSuccess) p.busy[s] = true;
    return e;
  };
  for (size_t i = 0; i < chunks && i < (size_t)kPipeSlots; ++i) {
    const hipError_t e = enqueue(i);
    if (e != hipSuccess) return e;
  }
  for (size_t i = 0; i < chunks; ++i) {
    const int s = (int)(i % kPipeSlots);
    hipError_t e = p.wait(s);
    if (e != hipSuccess) return e;
    const size_t off = i * kPipeChunk;
    p.pool.copy(d8 + off, p.slot[s], std::min(kPipeChunk, bytes - off));
    if (i + kPipeSlots < chunks) {
      e = enqueue(i + kPipeSlots);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

}  // namespace prom
