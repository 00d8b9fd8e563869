// Caching allocator of pinned (page-locked) host memory for the "gcu" device.
//
// Interface of the reference's caching host allocator
// (torch_gcu/csrc/gcu/gcu_caching_host_allocator.h:14-30): the c10 allocator
// behind pin_memory() / torch.empty(..., pin_memory=True), the event record
// that an asynchronous copy makes so a block is not handed out again before
// the copy has read or written it, and emptyCache.  Design notes are in
// gcu_caching_host_allocator.cpp.
#pragma once

#include <c10/core/Allocator.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace torch_gcu {
namespace host_allocator {

// The c10 allocator of pinned host memory (getCachingHostAllocator,
// gcu_caching_host_allocator.h:14; also what the hooks' getPinnedMemoryAllocator
// returns, gcu_hooks.cpp:74-76).
c10::Allocator* get();

// Marks the block that holds `ptr` (or whose context is `ctx`) as used by
// work queued on `stream` of `device`: when the block is freed it goes back
// to the cache only after that work has finished.  Returns false when the
// memory is not from this allocator (CachingHostAllocator_recordEvent,
// gcu_caching_host_allocator.h:19).
bool record_event(const void* ptr, void* ctx, hipStream_t stream, int device);

// Releases every cached (free, no pending work) block with hipHostFree
// (CachingHostAllocator_emptyCache, gcu_caching_host_allocator.h:22).
void empty_cache();

// True when `ptr` lies inside a block of this allocator.
bool owns(const void* ptr);

struct Stats {
  int64_t allocated_bytes = 0;  // in blocks handed out
  int64_t reserved_bytes = 0;   // pinned by this allocator (handed out + cached)
  int64_t num_blocks = 0;       // blocks pinned
  int64_t num_host_alloc = 0;   // hipHostMalloc calls
  int64_t num_host_free = 0;    // hipHostFree calls
  int64_t num_cache_hits = 0;   // requests served from the cache
  int64_t pending_events = 0;   // recorded events not yet seen complete
};
Stats stats();

// Serves blocks from ordinary host memory, so the bookkeeping can be tested
// without a GPU.  record_event is then refused (there are no streams).  Must
// be chosen before the first allocation.
void use_plain_memory_for_tests();

}  // namespace host_allocator
}  // namespace torch_gcu
