// Caching allocator of the "gcu" device.
//
// Memory is obtained from hipMalloc in segments and carved into blocks:
//   - requests up to 1 MiB ("small") are served from 2 MiB segments;
//   - requests between 1 MiB and 10 MiB get 20 MiB segments;
//   - larger requests get a segment rounded up to 2 MiB.
// Free blocks are cached per (pool, stream) in a set ordered by (stream,
// size, address); a request takes the best fit on its own stream, so reuse
// is stream ordered without synchronisation.  A block used on other streams
// (recordStream) is returned only after an event recorded on each of those
// streams has completed.  Adjacent free blocks of a segment are merged.
// While a graph is being captured, allocations on the capturing stream go to
// the graph's private pool, no event is queried, and no segment is freed
// (hipFree would synchronise inside the capture).
//
// These are the semantics of the reference's allocator
// (torch_gcu/csrc/gcu/gcu_caching_allocator.cpp: constants :50-64, malloc
// :593-731, split :733-813, free :815-859, recordStream :909-918, pools
// :1353-1413 and :1704-1728, events :2199-2270), implemented on HIP without
// hipMallocAsync.  The segment sizes suit a 288 GB device: large requests
// are not over-rounded, so fragmentation stays below one 2 MiB page per
// segment.
#include "gcu_caching_allocator.h"

#include <c10/core/Allocator.h>
#include <c10/util/Exception.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <unordered_map>
#include <unordered_set>

#include "gcu_runtime.h"

namespace torch_gcu {
namespace allocator {

namespace {

constexpr size_t kMinBlockSize = 512;
constexpr size_t kSmallSize = 1u << 20;
constexpr size_t kSmallBuffer = 2u << 20;
constexpr size_t kLargeBuffer = 20u << 20;
constexpr size_t kMinLargeAlloc = 10u << 20;
constexpr size_t kRoundLarge = 2u << 20;

struct BlockPool;
struct PrivatePool;

struct Block {
  int device = 0;
  hipStream_t stream = nullptr;
  size_t size = 0;
  size_t requested = 0;
  void* ptr = nullptr;
  BlockPool* pool = nullptr;
  bool allocated = false;
  Block* prev = nullptr;
  Block* next = nullptr;
  std::vector<hipStream_t> stream_uses;
  int event_count = 0;
  Context context;      // stack of the allocation (history with context on)
  Context seg_context;  // on a segment's first block: stack of the segment's creation
  bool is_split() const { return prev != nullptr || next != nullptr; }
};

struct BlockLess {
  bool operator()(const Block* a, const Block* b) const {
    if (a->stream != b->stream) return (uintptr_t)a->stream < (uintptr_t)b->stream;
    if (a->size != b->size) return a->size < b->size;
    return (uintptr_t)a->ptr < (uintptr_t)b->ptr;
  }
};

struct BlockPool {
  BlockPool(bool small, PrivatePool* o) : is_small(small), owner(o) {}
  std::set<Block*, BlockLess> blocks;
  bool is_small;
  PrivatePool* owner;
};

struct PrivatePool {
  PrivatePool() : large(false, this), small(true, this) {}
  int use_count = 1;
  int allocation_count = 0;
  BlockPool large;
  BlockPool small;
};

Config g_config;
std::once_flag g_config_once;

// Host-memory stand-in for HIP, used by the CPU tests of the allocator's
// bookkeeping: segments come from the C heap, events complete at once and
// no device call is made.
bool g_fake = false;
size_t g_fake_capacity = 0;
size_t g_fake_used = 0;

// History settings shared by every device: read outside the device locks
// (to gather a stack before taking one), so kept in atomics.
std::atomic<bool> g_hist_on{false};
std::atomic<int> g_hist_when{(int)RecordContext::NEVER};
std::atomic<ContextFn> g_hist_fn{nullptr};
std::atomic<size_t> g_hist_max{1};

Context gather_if(RecordContext level) {
  if (!g_hist_on.load() || g_hist_when.load() < (int)level) return nullptr;
  const ContextFn fn = g_hist_fn.load();
  return fn ? fn() : nullptr;
}

int64_t now_us() {
  return std::chrono::duration_cast<std::chrono::microseconds>(
             std::chrono::system_clock::now().time_since_epoch())
      .count();
}

size_t stat_index(bool small) { return small ? 1 : 2; }

std::string fmt_bytes(size_t n) {
  std::ostringstream os;
  if (n < 1024) os << n << " bytes";
  else if (n < (1u << 20)) os << (n / 1024.0) << " KiB";
  else if (n < (1ull << 30)) os << (n / 1048576.0) << " MiB";
  else os << (n / 1073741824.0) << " GiB";
  return os.str();
}

size_t round_power2_divisions(size_t size, size_t divisions) {
  if ((size & (size - 1)) == 0) return size;
  size_t floor2 = 1;
  while (floor2 * 2 <= size) floor2 *= 2;
  size_t div_log = 0;
  while (((size_t)1 << (div_log + 1)) <= divisions) ++div_log;
  const size_t step = floor2 >> div_log;
  if (step == 0) return floor2 * 2;
  const size_t down = size & ~(step - 1);
  return down == size ? size : down + step;
}

class DeviceAllocator {
 public:
  explicit DeviceAllocator(int device)
      : device_(device), large_(false, nullptr), small_(true, nullptr), trace_max_(g_hist_max.load()) {}

  // `ctx`: the caller's stack, gathered before the lock when history keeps
  // contexts (null otherwise).
  Block* malloc(size_t orig, hipStream_t stream, Context ctx = nullptr) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    OpContext oc(this, ctx);
    if (capturing_.empty()) process_events();
    const size_t size = round_size(orig);
    BlockPool& pool = get_pool(size, stream);
    const size_t alloc_size = allocation_size(size);
    Block* block = find_free(pool, stream, size);
    if (block == nullptr) {
      maybe_collect_garbage();
      block = new_segment(alloc_size, stream, pool);
      if (block == nullptr && capturing_.empty()) {
        ++stats_.num_alloc_retries;
        release_cached();
        block = new_segment(alloc_size, stream, pool);
      }
      if (block == nullptr) raise_oom(orig, alloc_size);
    } else {
      take_free(pool, block);
    }
    // split off the remainder when it is worth keeping
    const size_t remaining = block->size - size;
    const bool split = pool.is_small ? remaining >= kMinBlockSize
                                     : (remaining > kSmallSize && size < g_config.max_split_size);
    if (split) split_block(pool, block, size);
    mark_allocated(pool, block, orig, stream);
    record(TraceAction::ALLOC, block->ptr, (int64_t)orig, stream, RecordContext::ALLOC);
    return block;
  }

  bool owns(void* p) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    return active_.count(p) != 0;
  }

  void free(void* p, Context ctx = nullptr) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    OpContext oc(this, ctx);
    auto it = active_.find(p);
    TORCH_CHECK(it != active_.end(), "gcu allocator: invalid device pointer ", p);
    Block* b = it->second;
    record(TraceAction::FREE_REQUESTED, b->ptr, (int64_t)b->requested, b->stream,
           RecordContext::ALL);
    active_.erase(it);
    b->allocated = false;
    const bool small = b->pool->is_small;
    stat_sub(stats_.allocation, small, 1);
    stat_sub(stats_.allocated_bytes, small, (int64_t)b->size);
    stat_sub(stats_.requested_bytes, small, (int64_t)b->requested);
    if (b->pool->owner) b->pool->owner->allocation_count--;
    if (!b->stream_uses.empty()) {
      if (!capturing_.empty()) {
        // no event record/query inside a capture: keep the block until the
        // capture ends
        deferred_.push_back(b);
      } else {
        insert_events(b);
      }
      return;
    }
    free_block(b);
  }

  void record_stream(void* p, hipStream_t s) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    auto it = active_.find(p);
    if (it == active_.end()) return;  // not from this allocator (e.g. offset view)
    Block* b = it->second;
    if (s == b->stream) return;
    if (std::find(b->stream_uses.begin(), b->stream_uses.end(), s) == b->stream_uses.end())
      b->stream_uses.push_back(s);
  }

  void empty_cache(Context ctx = nullptr) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    OpContext oc(this, ctx);
    if (!capturing_.empty()) return;
    release_cached();
  }

  void set_fraction(double f) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    size_t free_b = 0, total = 0;
    device_mem_info(&free_b, &total);
    fraction_ = f;
    limit_ = (size_t)(f * (double)total);
  }
  double fraction() {
    std::lock_guard<std::recursive_mutex> g(mu_);
    return fraction_;
  }

  DeviceStats stats() {
    std::lock_guard<std::recursive_mutex> g(mu_);
    DeviceStats s = stats_;
    s.max_split_size = g_config.max_split_size == SIZE_MAX ? -1 : (int64_t)g_config.max_split_size;
    return s;
  }
  void reset_peak() {
    std::lock_guard<std::recursive_mutex> g(mu_);
    for (auto* arr : {&stats_.allocation, &stats_.segment, &stats_.active, &stats_.inactive_split,
                      &stats_.allocated_bytes, &stats_.reserved_bytes, &stats_.active_bytes,
                      &stats_.inactive_split_bytes, &stats_.requested_bytes})
      for (auto& st : *arr) st.reset_peak();
  }
  void reset_accumulated() {
    std::lock_guard<std::recursive_mutex> g(mu_);
    for (auto* arr : {&stats_.allocation, &stats_.segment, &stats_.active, &stats_.inactive_split,
                      &stats_.allocated_bytes, &stats_.reserved_bytes, &stats_.active_bytes,
                      &stats_.inactive_split_bytes, &stats_.requested_bytes})
      for (auto& st : *arr) st.reset_accumulated();
    stats_.num_alloc_retries = 0;
    stats_.num_ooms = 0;
  }

  // Segments in address order.  `mark`: record a SNAPSHOT history event.
  void snapshot(std::vector<SegmentInfo>& out, bool mark = false) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    std::vector<Block*> heads(segments_.begin(), segments_.end());
    std::sort(heads.begin(), heads.end(),
              [](const Block* a, const Block* b) { return (uintptr_t)a->ptr < (uintptr_t)b->ptr; });
    for (Block* head : heads) {
      SegmentInfo si;
      si.device = device_;
      si.address = (uintptr_t)head->ptr;
      si.is_large = !head->pool->is_small;
      si.stream = (uintptr_t)head->stream;
      si.context = head->seg_context;
      si.owner_pool = pool_id_of(head->pool->owner);
      for (Block* b = head; b; b = b->next) {
        BlockInfo bi;
        bi.address = (uintptr_t)b->ptr;
        bi.size = b->size;
        bi.allocated = b->allocated;
        bi.active = b->allocated || b->event_count > 0;
        bi.requested_size = bi.active ? b->requested : 0;
        bi.context = bi.active ? b->context : nullptr;
        si.total_size += b->size;
        if (b->allocated) si.allocated_size += b->size;
        if (bi.active) {
          si.active_size += b->size;
          si.requested_size += b->requested;
        }
        si.blocks.push_back(std::move(bi));
      }
      out.push_back(std::move(si));
    }
    if (mark) record(TraceAction::SNAPSHOT, nullptr, 0, nullptr, RecordContext::NEVER);
  }

  // The history, oldest entry first.
  std::vector<TraceEntry> trace() {
    std::lock_guard<std::recursive_mutex> g(mu_);
    std::vector<TraceEntry> out;
    out.reserve(trace_.size());
    for (size_t i = 0; i < trace_.size(); ++i) out.push_back(trace_[(trace_next_ + i) % trace_.size()]);
    return out;
  }

  void set_history(bool enabled, size_t max_entries) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    if (!enabled || max_entries < trace_.size()) {
      trace_.clear();
      trace_next_ = 0;
    }
    trace_max_ = std::max<size_t>(1, max_entries);
  }

  void cache_info(size_t* largest) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    if (*largest == 0) {
      size_t total = 0;
      device_mem_info(largest, &total);  // optimistic start: the device's free memory
    }
    auto scan = [&](const BlockPool& p) {
      for (const Block* b : p.blocks) *largest = std::max(*largest, b->size);
    };
    scan(large_);
    scan(small_);
    for (auto& kv : graph_pools_) {
      scan(kv.second->large);
      scan(kv.second->small);
    }
  }

  void* base_allocation(void* p, size_t* size) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    auto it = active_.find(p);
    TORCH_CHECK(it != active_.end(), "gcu allocator: invalid device pointer ", p);
    Block* b = it->second;
    while (b->prev) b = b->prev;
    if (size) {
      size_t n = 0;
      for (Block* c = b; c; c = c->next) n += c->size;
      *size = n;
    }
    return b->ptr;
  }

  bool check_pool_live(MempoolId id, const std::unordered_set<void*>& expected) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    auto it = graph_pools_.find(id);
    TORCH_CHECK(it != graph_pools_.end(), "gcu allocator: no memory pool (", id.first, ", ",
                id.second, ")");
    size_t live = 0;
    for (const auto& kv : active_) {
      if (kv.second->pool->owner != it->second.get()) continue;
      if (!expected.count(kv.first)) return false;
      ++live;
    }
    return live == expected.size();
  }

  std::shared_ptr<PoolState> checkpoint(MempoolId id) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    TORCH_CHECK(!freeable_.count(id), "gcu allocator: pool (", id.first, ", ", id.second,
                ") was released; it cannot be checkpointed");
    auto it = graph_pools_.find(id);
    TORCH_CHECK(it != graph_pools_.end(), "gcu allocator: no memory pool (", id.first, ", ",
                id.second, ")");
    auto st = std::make_shared<PoolState>();
    st->device = device_;
    st->id = id;
    for (Block* head : pool_segments(it->second.get())) {
      std::vector<BlockState> seg;
      for (Block* b = head; b; b = b->next)
        seg.push_back({(uintptr_t)b->ptr, b->size, b->allocated, (uintptr_t)b->stream});
      st->segments.push_back(std::move(seg));
    }
    return st;
  }

  // Returns the pool to a checkpointed layout: every block of the pool
  // allocated now is freed, then each checkpointed segment is cut into its
  // recorded blocks again and the blocks that were allocated are allocated.
  CheckpointDelta restore(const PoolState& st) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    OpContext oc(this, nullptr);
    TORCH_CHECK(!freeable_.count(st.id), "gcu allocator: pool (", st.id.first, ", ",
                st.id.second, ") was released; it cannot be restored");
    auto it = graph_pools_.find(st.id);
    TORCH_CHECK(it != graph_pools_.end(), "gcu allocator: no memory pool (", st.id.first, ", ",
                st.id.second, ")");
    PrivatePool* pool = it->second.get();
    CheckpointDelta delta;
    // 1. free what the pool holds now (no stream may still be using it)
    for (Block* head : pool_segments(pool)) {
      std::vector<Block*> live;
      for (Block* b = head; b; b = b->next)
        if (b->allocated) live.push_back(b);
      for (Block* b : live) {
        TORCH_CHECK(b->stream_uses.empty() && b->event_count == 0,
                    "gcu allocator: a block of the pool is still in use on another stream");
        delta.freed.push_back(b->ptr);
        free(b->ptr);
      }
    }
    // 2. every segment of the pool is now one free block
    std::unordered_map<uintptr_t, Block*> free_heads;
    for (BlockPool* bp : {&pool->small, &pool->large})
      for (Block* b : bp->blocks) free_heads[(uintptr_t)b->ptr] = b;
    // 3. cut and allocate each checkpointed segment
    for (const auto& seg : st.segments) {
      TORCH_CHECK(!seg.empty(), "gcu allocator: empty segment in a pool checkpoint");
      auto fh = free_heads.find(seg[0].ptr);
      TORCH_CHECK(fh != free_heads.end(), "gcu allocator: segment ", (void*)seg[0].ptr,
                  " of the checkpoint is not a free segment of the pool");
      Block* cur = fh->second;
      BlockPool& bp = *cur->pool;
      std::vector<Block*> blocks;
      for (size_t i = 0; i < seg.size(); ++i) {
        TORCH_CHECK(cur != nullptr && (uintptr_t)cur->ptr == seg[i].ptr && cur->size >= seg[i].size,
                    "gcu allocator: the pool's segment does not match the checkpoint");
        take_free(bp, cur);
        if (i + 1 < seg.size()) split_block(bp, cur, seg[i].size);
        TORCH_CHECK(cur->size == seg[i].size,
                    "gcu allocator: the pool's segment does not match the checkpoint");
        mark_allocated(bp, cur, seg[i].size, (hipStream_t)seg[i].stream);
        blocks.push_back(cur);
        cur = cur->next;
      }
      TORCH_CHECK(cur == nullptr, "gcu allocator: the pool's segment is longer than the checkpoint");
      // 4. free the blocks that were free in the checkpoint
      for (size_t i = 0; i < seg.size(); ++i) {
        if (seg[i].allocated) {
          delta.allocated.push_back(blocks[i]->ptr);
          continue;
        }
        free(blocks[i]->ptr);
      }
    }
    return delta;
  }

  void begin_pool(MempoolId id, std::function<bool(hipStream_t)> filter) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    auto it = graph_pools_.find(id);
    if (it == graph_pools_.end()) {
      graph_pools_[id] = std::make_unique<PrivatePool>();
    } else {
      it->second->use_count++;
      freeable_.erase(id);  // used again before its memory was returned
    }
    capturing_.push_back({id, std::move(filter)});
  }

  void end_pool(MempoolId id) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    for (auto it = capturing_.begin(); it != capturing_.end(); ++it) {
      if (it->first == id) {
        capturing_.erase(it);
        break;
      }
    }
    if (capturing_.empty()) {
      for (Block* b : deferred_) insert_events(b);
      deferred_.clear();
    }
  }

  void release_pool(MempoolId id) {
    std::lock_guard<std::recursive_mutex> g(mu_);
    auto it = graph_pools_.find(id);
    if (it == graph_pools_.end()) return;
    if (--it->second->use_count == 0) freeable_.insert(id);
    if (capturing_.empty()) release_freeable_pools();
  }

 private:
  // The stack of the public call in progress (set under the lock), for the
  // history entries of the helpers it runs.
  struct OpContext {
    OpContext(DeviceAllocator* a, Context c) : a_(a), prev_(std::move(a->op_ctx_)) {
      a_->op_ctx_ = std::move(c);
    }
    ~OpContext() { a_->op_ctx_ = std::move(prev_); }
    DeviceAllocator* a_;
    Context prev_;
  };

  void record(TraceAction action, const void* addr, int64_t size, hipStream_t stream,
              RecordContext level) {
    if (!g_hist_on.load()) return;
    TraceEntry e;
    e.action = action;
    e.device = device_;
    e.addr = (uintptr_t)addr;
    e.size = size;
    e.stream = (uintptr_t)stream;
    e.time_us = now_us();
    if (level != RecordContext::NEVER && g_hist_when.load() >= (int)level) e.context = op_ctx_;
    if (trace_.size() < trace_max_) {
      trace_.push_back(std::move(e));
    } else {
      trace_[trace_next_] = std::move(e);
      trace_next_ = (trace_next_ + 1) % trace_max_;
    }
  }

  MempoolId pool_id_of(const PrivatePool* p) const {
    if (p == nullptr) return {0, 0};
    for (const auto& kv : graph_pools_)
      if (kv.second.get() == p) return kv.first;
    return {0, 0};
  }

  // First blocks of the pool's segments, in address order.
  std::vector<Block*> pool_segments(const PrivatePool* p) const {
    std::vector<Block*> out;
    for (Block* head : segments_)
      if (head->pool->owner == p) out.push_back(head);
    std::sort(out.begin(), out.end(),
              [](const Block* a, const Block* b) { return (uintptr_t)a->ptr < (uintptr_t)b->ptr; });
    return out;
  }

  // Takes a cached free block out of its pool.
  void take_free(BlockPool& pool, Block* block) {
    pool.blocks.erase(block);
    if (block->is_split()) {  // it was counted as an inactive split
      stat_sub(stats_.inactive_split, pool.is_small, 1);
      stat_sub(stats_.inactive_split_bytes, pool.is_small, (int64_t)block->size);
    }
  }

  // Cuts `block` (out of the pool) to `size`; the rest goes back to the pool.
  void split_block(BlockPool& pool, Block* block, size_t size) {
    const size_t remaining = block->size - size;
    Block* rest = new Block();
    rest->device = block->device;
    rest->stream = block->stream;
    rest->pool = block->pool;
    rest->ptr = (char*)block->ptr + size;
    rest->size = remaining;
    rest->prev = block;
    rest->next = block->next;
    if (rest->next) rest->next->prev = rest;
    block->next = rest;
    block->size = size;
    pool.blocks.insert(rest);
    stat_add(stats_.inactive_split, pool.is_small, 1);
    stat_add(stats_.inactive_split_bytes, pool.is_small, (int64_t)remaining);
  }

  void mark_allocated(BlockPool& pool, Block* block, size_t orig, hipStream_t stream) {
    block->allocated = true;
    block->requested = orig;
    block->stream = stream;
    block->context = g_hist_when.load() >= (int)RecordContext::STATE ? op_ctx_ : nullptr;
    active_[block->ptr] = block;
    if (pool.owner) pool.owner->allocation_count++;
    stat_add(stats_.allocation, pool.is_small, 1);
    stat_add(stats_.allocated_bytes, pool.is_small, (int64_t)block->size);
    stat_add(stats_.active, pool.is_small, 1);
    stat_add(stats_.active_bytes, pool.is_small, (int64_t)block->size);
    stat_add(stats_.requested_bytes, pool.is_small, (int64_t)orig);
  }

  void stat_add(std::array<Stat, 3>& s, bool small, int64_t n) {
    s[0].inc(n);
    s[stat_index(small)].inc(n);
  }
  void stat_sub(std::array<Stat, 3>& s, bool small, int64_t n) {
    s[0].dec(n);
    s[stat_index(small)].dec(n);
  }

  static size_t round_size(size_t size) {
    if (size < kMinBlockSize) return kMinBlockSize;
    if (g_config.roundup_power2_divisions > 0 && size > kMinBlockSize)
      size = round_power2_divisions(size, g_config.roundup_power2_divisions);
    return (size + kMinBlockSize - 1) / kMinBlockSize * kMinBlockSize;
  }

  static size_t allocation_size(size_t size) {
    if (size <= kSmallSize) return kSmallBuffer;
    if (size < kMinLargeAlloc) return kLargeBuffer;
    return (size + kRoundLarge - 1) / kRoundLarge * kRoundLarge;
  }

  BlockPool& get_pool(size_t size, hipStream_t stream) {
    for (auto& c : capturing_) {
      if (c.second(stream)) {
        PrivatePool* p = graph_pools_.at(c.first).get();
        return size <= kSmallSize ? p->small : p->large;
      }
    }
    return size <= kSmallSize ? small_ : large_;
  }

  Block* find_free(BlockPool& pool, hipStream_t stream, size_t size) {
    Block key;
    key.stream = stream;
    key.size = size;
    key.ptr = nullptr;
    auto it = pool.blocks.lower_bound(&key);
    if (it == pool.blocks.end() || (*it)->stream != stream) return nullptr;
    Block* b = *it;
    // keep oversize blocks for oversize requests (max_split_size)
    if (size < g_config.max_split_size && b->size >= g_config.max_split_size) return nullptr;
    if (size >= g_config.max_split_size && b->size >= size + kLargeBuffer) return nullptr;
    return b;
  }

  void device_mem_info(size_t* free_b, size_t* total) {
    if (g_fake) {
      *total = g_fake_capacity;
      *free_b = g_fake_capacity - g_fake_used;
      return;
    }
    const auto prev = current_device();
    maybe_set_device((c10::DeviceIndex)device_);
    GCU_HIP_CHECK(hipMemGetInfo(free_b, total));
    maybe_set_device(prev);
  }

  Block* new_segment(size_t size, hipStream_t stream, BlockPool& pool) {
    if (limit_ != SIZE_MAX && reserved_total_ + size > limit_) return nullptr;
    void* p = nullptr;
    if (g_fake) {
      if (g_fake_used + size > g_fake_capacity) return nullptr;
      p = std::aligned_alloc(512, size);
      if (p == nullptr) return nullptr;
      g_fake_used += size;
    } else {
      const auto prev = current_device();
      maybe_set_device((c10::DeviceIndex)device_);
      // Allocation is legal inside a relaxed-mode capture only.
      hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
      (void)hipThreadExchangeStreamCaptureMode(&mode);
      hipError_t e = hipMalloc(&p, size);
      (void)hipThreadExchangeStreamCaptureMode(&mode);
      maybe_set_device(prev);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
      }
    }
    ++stats_.num_device_alloc;
    Block* b = new Block();
    b->device = device_;
    b->stream = stream;
    b->size = size;
    b->ptr = p;
    b->pool = &pool;
    b->seg_context = g_hist_when.load() >= (int)RecordContext::STATE ? op_ctx_ : nullptr;
    record(TraceAction::SEGMENT_ALLOC, p, (int64_t)size, stream, RecordContext::ALLOC);
    reserved_total_ += size;
    segments_.insert(b);
    stat_add(stats_.segment, pool.is_small, 1);
    stat_add(stats_.reserved_bytes, pool.is_small, (int64_t)size);
    return b;
  }

  void insert_events(Block* b) {
    if (g_fake) {  // fake events complete immediately, at the next poll
      for (size_t i = 0; i < b->stream_uses.size(); ++i) {
        b->event_count++;
        events_.push_back({nullptr, b});
      }
      b->stream_uses.clear();
      return;
    }
    const auto prev = current_device();
    maybe_set_device((c10::DeviceIndex)device_);
    for (hipStream_t s : b->stream_uses) {
      hipEvent_t e;
      GCU_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
      GCU_HIP_CHECK(hipEventRecord(e, s));
      b->event_count++;
      events_.push_back({e, b});
    }
    b->stream_uses.clear();
    maybe_set_device(prev);
  }

  void process_events() {
    for (auto it = events_.begin(); it != events_.end();) {
      if (it->first == nullptr) {
        Block* b = it->second;
        it = events_.erase(it);
        if (--b->event_count == 0) free_block(b);
        continue;
      }
      const hipError_t e = hipEventQuery(it->first);
      if (e == hipErrorNotReady) {
        (void)hipGetLastError();
        ++it;
        continue;
      }
      GCU_HIP_CHECK(e);
      GCU_HIP_CHECK(hipEventDestroy(it->first));
      Block* b = it->second;
      it = events_.erase(it);
      if (--b->event_count == 0) free_block(b);
    }
  }

  void sync_events() {
    for (auto& pe : events_) {
      if (pe.first) {
        GCU_HIP_CHECK(hipEventSynchronize(pe.first));
        GCU_HIP_CHECK(hipEventDestroy(pe.first));
      }
      if (--pe.second->event_count == 0) free_block(pe.second);
    }
    events_.clear();
  }

  void free_block(Block* b) {
    BlockPool& pool = *b->pool;
    const bool small = pool.is_small;
    const int64_t orig_size = (int64_t)b->size;
    record(TraceAction::FREE_COMPLETED, b->ptr, (int64_t)b->requested, b->stream,
           RecordContext::ALL);
    b->context.reset();
    int64_t merged_inactive = 0;
    for (Block* nb : {b->prev, b->next}) {
      if (nb == nullptr || nb->allocated || nb->event_count > 0) continue;
      // merge nb into b
      pool.blocks.erase(nb);
      merged_inactive += 1;
      stat_sub(stats_.inactive_split_bytes, small, (int64_t)nb->size);
      if (nb == b->prev) {
        b->ptr = nb->ptr;
        b->prev = nb->prev;
        if (b->prev) b->prev->next = b;
        if (segments_.erase(nb)) {
          segments_.insert(b);
          b->seg_context = std::move(nb->seg_context);
        }
      } else {
        b->next = nb->next;
        if (b->next) b->next->prev = b;
      }
      b->size += nb->size;
      delete nb;
    }
    stat_sub(stats_.inactive_split, small, merged_inactive);
    stat_sub(stats_.active, small, 1);
    stat_sub(stats_.active_bytes, small, orig_size);
    if (b->is_split()) {
      stat_add(stats_.inactive_split, small, 1);
      stat_add(stats_.inactive_split_bytes, small, (int64_t)b->size);
    }
    pool.blocks.insert(b);
    if (pool.owner && pool.owner->use_count == 0 && pool.owner->allocation_count == 0 &&
        capturing_.empty())
      release_freeable_pools();
  }

  void release_pool_blocks(BlockPool& pool) {
    for (auto it = pool.blocks.begin(); it != pool.blocks.end();) {
      Block* b = *it;
      if (b->is_split()) {
        ++it;
        continue;
      }
      it = pool.blocks.erase(it);
      release_segment(b);
    }
  }

  void release_segment(Block* b) {
    record(TraceAction::SEGMENT_FREE, b->ptr, (int64_t)b->size, b->stream, RecordContext::ALL);
    if (g_fake) {
      std::free(b->ptr);
      g_fake_used -= b->size;
    } else {
      const auto prev = current_device();
      maybe_set_device((c10::DeviceIndex)device_);
      GCU_HIP_CHECK(hipFree(b->ptr));
      maybe_set_device(prev);
    }
    ++stats_.num_device_free;
    reserved_total_ -= b->size;
    segments_.erase(b);
    stat_sub(stats_.segment, b->pool->is_small, 1);
    stat_sub(stats_.reserved_bytes, b->pool->is_small, (int64_t)b->size);
    delete b;
  }

  void release_freeable_pools() {
    for (auto it = freeable_.begin(); it != freeable_.end();) {
      auto pit = graph_pools_.find(*it);
      PrivatePool* p = pit->second.get();
      release_pool_blocks(p->small);
      release_pool_blocks(p->large);
      if (p->allocation_count == 0 && p->small.blocks.empty() && p->large.blocks.empty()) {
        graph_pools_.erase(pit);
        it = freeable_.erase(it);
      } else {
        ++it;
      }
    }
  }

  void release_cached() {
    sync_events();
    release_pool_blocks(small_);
    release_pool_blocks(large_);
    release_freeable_pools();
  }

  void maybe_collect_garbage() {
    if (g_config.garbage_collection_threshold <= 0.0 || limit_ == SIZE_MAX) return;
    if (!capturing_.empty()) return;
    if ((double)reserved_total_ > g_config.garbage_collection_threshold * (double)limit_)
      release_cached();
  }

  [[noreturn]] void raise_oom(size_t requested, size_t alloc_size);

  std::recursive_mutex mu_;
  int device_;
  BlockPool large_, small_;
  std::unordered_map<void*, Block*> active_;
  std::set<Block*> segments_;
  std::map<MempoolId, std::unique_ptr<PrivatePool>> graph_pools_;
  std::set<MempoolId> freeable_;
  std::vector<std::pair<MempoolId, std::function<bool(hipStream_t)>>> capturing_;
  std::deque<std::pair<hipEvent_t, Block*>> events_;
  std::vector<Block*> deferred_;
  DeviceStats stats_;
  Context op_ctx_;
  std::vector<TraceEntry> trace_;  // ring of at most trace_max_ entries
  size_t trace_max_;
  size_t trace_next_ = 0;          // oldest entry once the ring is full
  size_t limit_ = SIZE_MAX;
  double fraction_ = 1.0;
  size_t reserved_total_ = 0;
};

std::mutex g_devices_mu;
std::vector<std::unique_ptr<DeviceAllocator>> g_devices;
std::mutex g_obs_mu;
std::vector<OomObserver> g_observers;

DeviceAllocator& dev_alloc(int d) {
  std::lock_guard<std::mutex> g(g_devices_mu);
  if ((int)g_devices.size() <= d) g_devices.resize(d + 1);
  if (!g_devices[d]) g_devices[d] = std::make_unique<DeviceAllocator>(d);
  return *g_devices[d];
}

// pointer -> owning device, for frees that arrive without a device
std::mutex g_owner_mu;
std::unordered_map<void*, int> g_owner;

void DeviceAllocator::raise_oom(size_t requested, size_t alloc_size) {
  ++stats_.num_ooms;
  size_t free_b = 0, total = 0;
  device_mem_info(&free_b, &total);
  record(TraceAction::OOM, (const void*)(uintptr_t)free_b, (int64_t)alloc_size, nullptr,
         RecordContext::STATE);
  {
    std::lock_guard<std::mutex> g(g_obs_mu);
    for (auto& o : g_observers) o(device_, alloc_size, total, free_b);
  }
  const size_t allocated = (size_t)stats_.allocated_bytes[0].current;
  const size_t reserved = (size_t)stats_.reserved_bytes[0].current;
  std::ostringstream os;
  os << "GCU out of memory. Tried to allocate " << fmt_bytes(alloc_size) << ". GCU " << device_
     << " has a total capacity of " << fmt_bytes(total) << " of which " << fmt_bytes(free_b)
     << " is free. Of the allocated memory " << fmt_bytes(allocated)
     << " is allocated by PyTorch, and " << fmt_bytes(reserved - allocated)
     << " is reserved by PyTorch but unallocated.";
  if (limit_ != SIZE_MAX)
    os << " The per-process memory fraction " << fraction_ << " caps this process at "
       << fmt_bytes(limit_) << ".";
  (void)requested;
  TORCH_CHECK_WITH(OutOfMemoryError, false, os.str());
}

void delete_fn(void* p);

struct GCUAllocator final : public c10::Allocator {
  c10::DataPtr allocate(size_t n) override {
    const int d = current_device();
    if (n == 0) return {nullptr, nullptr, &delete_fn, c10::Device(kGCU, (c10::DeviceIndex)d)};
    void* p = raw_alloc_with_stream(n, current_hip_stream((c10::DeviceIndex)d));
    return {p, p, &delete_fn, c10::Device(kGCU, (c10::DeviceIndex)d)};
  }
  c10::DeleterFnPtr raw_deleter() const override { return &delete_fn; }
  void copy_data(void* dest, const void* src, std::size_t count) const override {
    GCU_HIP_CHECK(hipMemcpy(dest, src, count, hipMemcpyDeviceToDevice));
  }
};

void delete_fn(void* p) {
  if (p) raw_delete(p);
}

GCUAllocator g_allocator;

}  // namespace

const Config& config() {
  std::call_once(g_config_once, [] {
    const char* e = std::getenv("PYTORCH_GCU_ALLOC_CONF");
    if (e) g_config = parse_config(e);
  });
  return g_config;
}

Config parse_config(const std::string& s) {
  Config c;
  std::stringstream ss(s);
  std::string item;
  while (std::getline(ss, item, ',')) {
    const auto colon = item.find(':');
    TORCH_CHECK(colon != std::string::npos, "PYTORCH_GCU_ALLOC_CONF: expected key:value, got '",
                item, "'");
    const std::string key = item.substr(0, colon), val = item.substr(colon + 1);
    if (key == "max_split_size_mb") {
      const double mb = std::stod(val);
      TORCH_CHECK(mb > 20, "PYTORCH_GCU_ALLOC_CONF: max_split_size_mb must be > 20");
      c.max_split_size = (size_t)(mb * 1048576.0);
    } else if (key == "garbage_collection_threshold") {
      const double t = std::stod(val);
      TORCH_CHECK(t > 0.0 && t < 1.0,
                  "PYTORCH_GCU_ALLOC_CONF: garbage_collection_threshold must be in (0, 1)");
      c.garbage_collection_threshold = t;
    } else if (key == "roundup_power2_divisions") {
      const long v = std::stol(val);
      TORCH_CHECK(v > 0 && (v & (v - 1)) == 0,
                  "PYTORCH_GCU_ALLOC_CONF: roundup_power2_divisions must be a power of 2");
      c.roundup_power2_divisions = (size_t)v;
    } else if (key == "backend") {
      TORCH_CHECK(val == "native", "PYTORCH_GCU_ALLOC_CONF: only backend:native is built");
    } else if (key == "expandable_segments") {
      TORCH_CHECK(val == "False" || val == "false" || val == "0",
                  "PYTORCH_GCU_ALLOC_CONF: expandable_segments is not supported");
    } else {
      TORCH_CHECK(false, "PYTORCH_GCU_ALLOC_CONF: unknown key '", key, "'");
    }
  }
  return c;
}

c10::Allocator* get() { return &g_allocator; }

void use_host_memory_for_tests(size_t capacity) {
  std::lock_guard<std::mutex> g(g_devices_mu);
  TORCH_CHECK(g_devices.empty() || g_fake,
              "the host-memory test mode must be chosen before the first allocation");
  g_fake = true;
  g_fake_capacity = capacity;
}

bool host_memory_mode() { return g_fake; }

void* alloc_on(int device, size_t nbytes, hipStream_t stream) {
  if (nbytes == 0) return nullptr;
  config();
  Block* b = dev_alloc(device).malloc(nbytes, stream, gather_if(RecordContext::STATE));
  std::lock_guard<std::mutex> g(g_owner_mu);
  g_owner[b->ptr] = device;
  return b->ptr;
}

void record_stream_raw(void* p, hipStream_t s) {
  int d;
  {
    std::lock_guard<std::mutex> g(g_owner_mu);
    auto it = g_owner.find(p);
    if (it == g_owner.end()) return;
    d = it->second;
  }
  dev_alloc(d).record_stream(p, s);
}

void empty_cache_device(int device) { dev_alloc(device).empty_cache(); }

void init(int device_count) {
  config();
  for (int d = 0; d < device_count; ++d) dev_alloc(d);
}

void* raw_alloc_with_stream(size_t nbytes, hipStream_t stream) {
  return alloc_on(current_device(), nbytes, stream);
}

void* raw_alloc(size_t nbytes) { return raw_alloc_with_stream(nbytes, current_hip_stream()); }

void raw_delete(void* ptr) {
  if (!ptr) return;
  int d;
  {
    std::lock_guard<std::mutex> g(g_owner_mu);
    auto it = g_owner.find(ptr);
    TORCH_CHECK(it != g_owner.end(), "gcu allocator: freeing an unknown pointer ", ptr);
    d = it->second;
    g_owner.erase(it);
  }
  dev_alloc(d).free(ptr, gather_if(RecordContext::ALL));
}

void record_stream(const c10::DataPtr& ptr, c10::Stream stream) {
  void* p = ptr.get_context();
  if (!p) return;
  int d;
  {
    std::lock_guard<std::mutex> g(g_owner_mu);
    auto it = g_owner.find(p);
    if (it == g_owner.end()) return;
    d = it->second;
  }
  dev_alloc(d).record_stream(p, stream_handle(stream));
}

void empty_cache() {
  std::vector<DeviceAllocator*> devs;
  {
    std::lock_guard<std::mutex> g(g_devices_mu);
    for (auto& d : g_devices)
      if (d) devs.push_back(d.get());
  }
  for (auto* d : devs) d->empty_cache(gather_if(RecordContext::ALL));
}

void release_all_cached(int device) {
  dev_alloc(device).empty_cache();
  device_synchronize((c10::DeviceIndex)device);
}

void set_memory_fraction(double fraction, int device) {
  TORCH_CHECK(fraction >= 0.0 && fraction <= 1.0, "invalid fraction ", fraction,
              ", please set within [0, 1]");
  dev_alloc(device).set_fraction(fraction);
}

double get_memory_fraction(int device) { return dev_alloc(device).fraction(); }

DeviceStats get_stats(int device) { return dev_alloc(device).stats(); }
void reset_peak_stats(int device) { dev_alloc(device).reset_peak(); }
void reset_accumulated_stats(int device) { dev_alloc(device).reset_accumulated(); }

std::vector<SegmentInfo> snapshot() {
  std::vector<SegmentInfo> out;
  std::vector<DeviceAllocator*> devs;
  {
    std::lock_guard<std::mutex> g(g_devices_mu);
    for (auto& d : g_devices)
      if (d) devs.push_back(d.get());
  }
  for (auto* d : devs) d->snapshot(out);
  return out;
}

namespace {
std::vector<DeviceAllocator*> all_devices() {
  std::vector<DeviceAllocator*> devs;
  std::lock_guard<std::mutex> g(g_devices_mu);
  for (auto& d : g_devices)
    if (d) devs.push_back(d.get());
  return devs;
}
}  // namespace

Snapshot full_snapshot() {
  Snapshot s;
  for (auto* d : all_devices()) d->snapshot(s.segments, /*mark=*/true);
  for (auto* d : all_devices()) s.device_traces.push_back(d->trace());
  return s;
}

void record_history(bool enabled, ContextFn fn, size_t max_entries, RecordContext when) {
  TORCH_CHECK(when == RecordContext::NEVER || fn != nullptr,
              "gcu allocator: recording stacks needs a context function");
  g_hist_on.store(false);  // entries stop while the settings change
  g_hist_fn.store(enabled ? fn : nullptr);
  g_hist_when.store(enabled ? (int)when : (int)RecordContext::NEVER);
  g_hist_max.store(std::max<size_t>(1, max_entries));
  for (auto* d : all_devices()) d->set_history(enabled, std::max<size_t>(1, max_entries));
  g_hist_on.store(enabled);
}

bool history_enabled() { return g_hist_on.load(); }

void cache_info(int device, size_t* largest) { dev_alloc(device).cache_info(largest); }

void* get_base_allocation(void* ptr, size_t* size) {
  int d;
  {
    std::lock_guard<std::mutex> g(g_owner_mu);
    auto it = g_owner.find(ptr);
    TORCH_CHECK(it != g_owner.end(), "gcu allocator: invalid device pointer ", ptr);
    d = it->second;
  }
  return dev_alloc(d).base_allocation(ptr, size);
}

bool check_pool_live_allocations(int device, MempoolId id,
                                 const std::unordered_set<void*>& expected) {
  return dev_alloc(device).check_pool_live(id, expected);
}

std::shared_ptr<PoolState> get_checkpoint_state(int device, MempoolId id) {
  return dev_alloc(device).checkpoint(id);
}

CheckpointDelta set_checkpoint_pool_state(int device, const PoolState& state) {
  TORCH_CHECK(state.device == device, "gcu allocator: the checkpoint is of device ", state.device,
              ", not ", device);
  CheckpointDelta delta = dev_alloc(device).restore(state);
  std::lock_guard<std::mutex> g(g_owner_mu);
  for (void* p : delta.freed) g_owner.erase(p);
  for (void* p : delta.allocated) g_owner[p] = device;
  return delta;
}

c10::DeleterFnPtr raw_deleter() { return &delete_fn; }

MempoolId new_pool_id() {
  static std::atomic<uint64_t> next{1};
  return {0, next.fetch_add(1)};
}

void begin_allocate_to_pool(int device, MempoolId id, std::function<bool(hipStream_t)> filter) {
  dev_alloc(device).begin_pool(id, std::move(filter));
}
void end_allocate_to_pool(int device, MempoolId id) { dev_alloc(device).end_pool(id); }
void release_pool(int device, MempoolId id) { dev_alloc(device).release_pool(id); }

void attach_oom_observer(OomObserver obs) {
  std::lock_guard<std::mutex> g(g_obs_mu);
  g_observers.push_back(std::move(obs));
}

void* workspace_alloc(size_t bytes, void* stream, void*) {
  try {
    return raw_alloc_with_stream(bytes, (hipStream_t)stream);
  } catch (const c10::Error&) {
    return nullptr;  // the kernel library reports MI_ERR_WORKSPACE
  }
}

void workspace_free(void* ptr, void*, void*) {
  try {
    raw_delete(ptr);
  } catch (const c10::Error&) {
  }
}

}  // namespace allocator
}  // namespace torch_gcu
