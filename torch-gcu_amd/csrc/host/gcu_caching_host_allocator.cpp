// Caching allocator of pinned host memory (the reference's TOPSHostAllocator,
// torch_gcu/csrc/gcu/gcu_caching_host_allocator.cpp:133-369, rebuilt on HIP).
//
// Why cache: hipHostMalloc page-locks the memory and maps it into every
// device's address space, which costs far more than the copy that usually
// follows (milliseconds for a few MiB), so staging buffers of non-blocking
// copies and DataLoader pin_memory() batches are recycled instead.
//
// Blocks are sized in classes: a power of two from 4 KiB up to 64 MiB, then
// multiples of 2 MiB.  A request takes the smallest cached block of at least
// its class and at most twice it, so one huge cached block is not spent on a
// small request.  A block freed while asynchronous copies that used it may
// still be in flight (record_event named their streams) gets one event per
// stream, recorded at free time; it returns to the cache when all of them
// have completed.  Completed events are collected, oldest first, at the start
// of every allocation and by empty_cache.  A block whose copy was recorded
// into a graph under capture is never handed out again, since any replay may
// read or write it.
//
// One mutex guards the bookkeeping; hipHostMalloc and hipHostFree run outside
// it.
#include "gcu_caching_host_allocator.h"

#include <c10/core/Device.h>
#include <c10/util/Exception.h>

#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "gcu_runtime.h"

namespace torch_gcu {
namespace host_allocator {
namespace {

constexpr size_t kMinBlock = 4096;
constexpr size_t kPow2Limit = size_t(64) << 20;
constexpr size_t kLargeStep = size_t(2) << 20;

size_t size_class(size_t n) {
  if (n <= kMinBlock) return kMinBlock;
  if (n <= kPow2Limit) {
    size_t c = kMinBlock;
    while (c < n) c <<= 1;
    return c;
  }
  return (n + kLargeStep - 1) / kLargeStep * kLargeStep;
}

struct Use {
  int device;
  hipStream_t stream;
  bool operator==(const Use& o) const { return device == o.device && stream == o.stream; }
};

struct Block {
  void* ptr = nullptr;
  size_t size = 0;
  bool allocated = false;
  bool captured = false;  // recorded into a graph: never reused
  int pending = 0;        // events recorded at free time, not yet complete
  std::vector<Use> uses;  // streams named by record_event since allocation
};

struct Pending {
  hipEvent_t event;
  int device;
  Block* block;
};

class HostAllocator {
 public:
  std::pair<void*, Block*> allocate(size_t n) {
    if (n == 0) return {nullptr, nullptr};
    const size_t sz = size_class(n);
    {
      std::lock_guard<std::mutex> g(mu_);
      collect_locked();
      auto it = free_.lower_bound(sz);
      if (it != free_.end() && it->first <= 2 * sz) {
        Block* b = it->second;
        free_.erase(it);
        b->allocated = true;
        stats_.allocated_bytes += (int64_t)b->size;
        stats_.num_cache_hits += 1;
        return {b->ptr, b};
      }
    }
    void* p = pin(sz);
    if (p == nullptr) {
      empty_cache();
      p = pin(sz);
    }
    TORCH_CHECK(p != nullptr, "gcu: out of pinned host memory allocating ", sz,
                " bytes (hipHostMalloc failed; ", stats().reserved_bytes,
                " bytes are pinned by the host caching allocator)");
    auto* b = new Block();
    b->ptr = p;
    b->size = sz;
    b->allocated = true;
    std::lock_guard<std::mutex> g(mu_);
    by_addr_[(uintptr_t)p] = b;
    stats_.allocated_bytes += (int64_t)sz;
    stats_.reserved_bytes += (int64_t)sz;
    stats_.num_blocks += 1;
    stats_.num_host_alloc += 1;
    return {p, b};
  }

  void free(Block* b) {
    if (b == nullptr) return;
    std::lock_guard<std::mutex> g(mu_);
    b->allocated = false;
    stats_.allocated_bytes -= (int64_t)b->size;
    for (const Use& u : b->uses) {
      if (stream_is_capturing(u.stream)) {
        b->captured = true;
        continue;
      }
      // runs inside a deleter: failures keep the block out of the cache
      // instead of raising
      hipEvent_t e = take_event_locked(u.device);
      if (e == nullptr) {
        b->captured = true;
        continue;
      }
      if (hipEventRecord(e, u.stream) != hipSuccess) {
        (void)hipGetLastError();
        events_[u.device].push_back(e);
        b->captured = true;
        continue;
      }
      pending_.push_back(Pending{e, u.device, b});
      b->pending += 1;
    }
    b->uses.clear();
    if (!b->captured && b->pending == 0) free_.emplace(b->size, b);
  }

  bool record_event(const void* ptr, Block* ctx, hipStream_t stream, int device) {
    if (plain_) return false;
    std::lock_guard<std::mutex> g(mu_);
    // Found by address: a slice or a from_blob view of a block lies inside
    // it, and a context from another allocator is never dereferenced.
    (void)ctx;
    Block* b = find_locked(ptr);
    if (b == nullptr) return false;
    TORCH_INTERNAL_ASSERT(b->allocated, "record_event on a freed pinned block");
    const Use u{device, stream};
    for (const Use& v : b->uses)
      if (v == u) return true;
    b->uses.push_back(u);
    return true;
  }

  void empty_cache() {
    std::vector<Block*> drop;
    {
      std::lock_guard<std::mutex> g(mu_);
      collect_locked();
      for (auto& kv : free_) drop.push_back(kv.second);
      free_.clear();
      for (Block* b : drop) {
        by_addr_.erase((uintptr_t)b->ptr);
        stats_.reserved_bytes -= (int64_t)b->size;
        stats_.num_blocks -= 1;
        stats_.num_host_free += 1;
      }
    }
    for (Block* b : drop) {
      unpin(b->ptr);
      delete b;
    }
  }

  bool owns(const void* ptr) {
    std::lock_guard<std::mutex> g(mu_);
    return find_locked(ptr) != nullptr;
  }

  Stats stats() {
    std::lock_guard<std::mutex> g(mu_);
    Stats s = stats_;
    s.pending_events = (int64_t)pending_.size();
    return s;
  }

  void use_plain_memory() {
    std::lock_guard<std::mutex> g(mu_);
    TORCH_CHECK(by_addr_.empty(), "the host allocator's backing must be chosen before it allocates");
    plain_ = true;
  }

 private:
  void* pin(size_t sz) {
    if (plain_) return std::aligned_alloc(kMinBlock, sz);
    void* p = nullptr;
    const hipError_t e = hipHostMalloc(&p, sz, hipHostMallocDefault);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      if (e != hipErrorOutOfMemory && e != hipErrorMemoryAllocation)
        TORCH_CHECK(false, "gcu: hipHostMalloc(", sz, ") failed: ", hipGetErrorString(e));
      return nullptr;
    }
    return p;
  }

  void unpin(void* p) {
    if (plain_) {
      std::free(p);
      return;
    }
    GCU_HIP_CHECK(hipHostFree(p));
  }

  // the block whose range holds ptr
  Block* find_locked(const void* ptr) {
    auto it = by_addr_.upper_bound((uintptr_t)ptr);
    if (it == by_addr_.begin()) return nullptr;
    --it;
    Block* b = it->second;
    return (uintptr_t)ptr < it->first + b->size ? b : nullptr;
  }

  hipEvent_t take_event_locked(int device) {
    if ((int)events_.size() <= device) events_.resize(device + 1);
    auto& pool = events_[device];
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    // nullptr on failure (no exception: called from deleters)
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess || (prev != device && hipSetDevice(device) != hipSuccess)) {
      (void)hipGetLastError();
      return nullptr;
    }
    hipEvent_t e = nullptr;
    const hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (prev != device) (void)hipSetDevice(prev);
    if (err != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    return e;
  }

  // Returns the blocks whose events have all completed to the cache, oldest
  // event first; stops at the first event still in flight.
  void collect_locked() {
    while (!pending_.empty()) {
      Pending& p = pending_.front();
      const hipError_t err = hipEventQuery(p.event);
      if (err == hipErrorNotReady) {
        (void)hipGetLastError();
        return;
      }
      GCU_HIP_CHECK(err);
      Block* b = p.block;
      events_[p.device].push_back(p.event);
      pending_.pop_front();
      b->pending -= 1;
      if (b->pending == 0 && !b->allocated && !b->captured) free_.emplace(b->size, b);
    }
  }

  std::mutex mu_;
  bool plain_ = false;
  std::map<uintptr_t, Block*> by_addr_;    // every block, by base address
  std::multimap<size_t, Block*> free_;     // cached blocks, by size
  std::deque<Pending> pending_;            // oldest first
  std::vector<std::vector<hipEvent_t>> events_;  // idle events per device
  Stats stats_;
};

HostAllocator& instance() {
  // leaked: blocks can be freed by tensors that outlive static destruction
  static auto* a = new HostAllocator();
  return *a;
}

void delete_block(void* ctx) { instance().free(static_cast<Block*>(ctx)); }

struct PinnedAllocator final : public c10::Allocator {
  c10::DataPtr allocate(size_t n) override {
    auto pc = instance().allocate(n);
    return {pc.first, pc.second, &delete_block, c10::Device(c10::DeviceType::CPU)};
  }
  c10::DeleterFnPtr raw_deleter() const override { return nullptr; }
  void copy_data(void* dest, const void* src, std::size_t count) const override {
    if (count > 0) std::memcpy(dest, src, count);
  }
};

PinnedAllocator g_pinned;

}  // namespace

c10::Allocator* get() { return &g_pinned; }

bool record_event(const void* ptr, void* ctx, hipStream_t stream, int device) {
  return instance().record_event(ptr, static_cast<Block*>(ctx), stream, device);
}

void empty_cache() { instance().empty_cache(); }

bool owns(const void* ptr) { return ptr != nullptr && instance().owns(ptr); }

Stats stats() { return instance().stats(); }

void use_plain_memory_for_tests() { instance().use_plain_memory(); }

}  // namespace host_allocator
}  // namespace torch_gcu
