// Stream-ordered caching allocator of the "gcu" device on hipMalloc'd
// segments.
//
// Interface of the reference's GCUCachingAllocator
// (torch_gcu/csrc/gcu/gcu_caching_allocator.h:231-425): allocate / raw_alloc /
// raw_delete, recordStream, emptyCache, memory stats, per-process memory
// fraction, and the graph private-pool calls (beginAllocateToPool,
// endAllocateToPool, releasePool) that GCUGraph uses, memory history and
// snapshots, graph-pool checkpoints, cacheInfo, getBaseAllocation and
// checkPoolLiveAllocations.  Design notes are in gcu_caching_allocator.cpp.
#pragma once

#include <c10/core/Allocator.h>
#include <c10/core/Stream.h>
#include <hip/hip_runtime_api.h>

#include <array>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

namespace torch_gcu {
namespace allocator {

// (graph id, 0) for pools made by graph capture, (0, handle id) for pools
// made by graph_pool_handle(); as c10::cuda::MempoolId_t.
using MempoolId = std::pair<uint64_t, uint64_t>;

struct Stat {
  int64_t current = 0, peak = 0, allocated = 0, freed = 0;
  void inc(int64_t n) {
    current += n;
    allocated += n;
    if (current > peak) peak = current;
  }
  void dec(int64_t n) {
    current -= n;
    freed += n;
  }
  void reset_peak() { peak = current; }
  void reset_accumulated() {
    allocated = 0;
    freed = 0;
  }
};

// Index 0: all pools, 1: small pool, 2: large pool (DeviceStats layout of
// gcu_caching_allocator.h:53-101).
struct DeviceStats {
  std::array<Stat, 3> allocation, segment, active, inactive_split;
  std::array<Stat, 3> allocated_bytes, reserved_bytes, active_bytes, inactive_split_bytes,
      requested_bytes;
  int64_t num_alloc_retries = 0;
  int64_t num_ooms = 0;
  int64_t num_sync_all_streams = 0;
  int64_t num_device_alloc = 0;
  int64_t num_device_free = 0;
  int64_t max_split_size = 0;
};

// Stack context of an allocator event (a torch::CapturedTraceback when
// recorded from Python; symbolised only when a snapshot is taken).
using Context = std::shared_ptr<c10::GatheredContext>;
using ContextFn = Context (*)();

struct BlockInfo {
  uintptr_t address = 0;
  size_t size = 0;
  size_t requested_size = 0;
  bool allocated = false;
  bool active = false;  // allocated, or freed but awaiting other streams' events
  Context context;      // where it was allocated (history with context on)
};

struct SegmentInfo {
  int device = 0;
  uintptr_t address = 0;
  size_t total_size = 0;
  size_t requested_size = 0;
  size_t allocated_size = 0;
  size_t active_size = 0;
  bool is_large = false;
  MempoolId owner_pool{0, 0};
  uintptr_t stream = 0;
  std::vector<BlockInfo> blocks;
  Context context;  // where the segment was created
};

// Memory history (gcu_caching_allocator.h:136-185): one entry per allocator
// event while recording is on, kept in a ring of at most max_entries.
enum class TraceAction { ALLOC, FREE_REQUESTED, FREE_COMPLETED, SEGMENT_ALLOC, SEGMENT_FREE,
                         SNAPSHOT, OOM };
struct TraceEntry {
  TraceAction action;
  int device = 0;
  uintptr_t addr = 0;  // for OOM: the device's free bytes
  int64_t size = 0;
  uintptr_t stream = 0;
  int64_t time_us = 0;  // wall clock, microseconds since the epoch
  Context context;
};
// Which events keep a stack: NEVER; STATE (live blocks and segments);
// ALLOC (also alloc entries of the history); ALL (also free entries).
enum class RecordContext { NEVER = 0, STATE = 1, ALLOC = 2, ALL = 3 };

struct Snapshot {
  std::vector<SegmentInfo> segments;
  std::vector<std::vector<TraceEntry>> device_traces;  // index = device
};

// A graph pool's block layout, restorable later (getCheckpointState,
// gcu_caching_allocator.cpp:1007-1222).
struct BlockState {
  uintptr_t ptr = 0;
  size_t size = 0;
  bool allocated = false;
  uintptr_t stream = 0;
};
struct PoolState {
  int device = 0;
  MempoolId id{0, 0};
  std::vector<std::vector<BlockState>> segments;  // blocks of each segment, in address order
};
// What setCheckpointPoolState changed: pointers whose blocks it freed and
// pointers of blocks it allocated (a pointer may be in both).
struct CheckpointDelta {
  std::vector<void*> freed;
  std::vector<void*> allocated;
};

// c10 allocator registered for DeviceType::PrivateUse1.
c10::Allocator* get();

void init(int device_count);
void* raw_alloc(size_t nbytes);
void* raw_alloc_with_stream(size_t nbytes, hipStream_t stream);
void raw_delete(void* ptr);
void record_stream(const c10::DataPtr& ptr, c10::Stream stream);
void empty_cache();
void set_memory_fraction(double fraction, int device);
double get_memory_fraction(int device);
DeviceStats get_stats(int device);
void reset_peak_stats(int device);
void reset_accumulated_stats(int device);
std::vector<SegmentInfo> snapshot();
// Segments plus each device's history; records a SNAPSHOT event.
Snapshot full_snapshot();
// Turns history recording on or off on every device (recordHistory,
// gcu_caching_allocator.cpp:531-546).  `fn` gathers a stack; it is called
// outside the allocator's lock.  Turning it off clears the history.
void record_history(bool enabled, ContextFn fn, size_t max_entries, RecordContext when);
bool history_enabled();
// Largest free cached block of the device (cacheInfo, :936-950); a zero
// *largest starts from the device's free memory.
void cache_info(int device, size_t* largest);
// Start and size of the segment holding an allocated pointer
// (getBaseAllocation, :861-880).
void* get_base_allocation(void* ptr, size_t* size);
// True when the allocated blocks of a graph pool are exactly `expected`
// (checkPoolLiveAllocations, :547-566).
bool check_pool_live_allocations(int device, MempoolId id,
                                 const std::unordered_set<void*>& expected);
std::shared_ptr<PoolState> get_checkpoint_state(int device, MempoolId id);
CheckpointDelta set_checkpoint_pool_state(int device, const PoolState& state);
// The deleter of every DataPtr this allocator hands out.
c10::DeleterFnPtr raw_deleter();
// Releases every cached block back to HIP and synchronises the device.
void release_all_cached(int device);

// Graph pools.
MempoolId new_pool_id();  // graph_pool_handle()
void begin_allocate_to_pool(int device, MempoolId id, std::function<bool(hipStream_t)> filter);
void end_allocate_to_pool(int device, MempoolId id);
void release_pool(int device, MempoolId id);

// Out-of-memory observers (gcu_caching_allocator.cpp:718-745 calls them
// before raising).
using OomObserver = std::function<void(int device, size_t requested, size_t device_total,
                                       size_t device_free)>;
void attach_oom_observer(OomObserver obs);

// Allocation on an explicit device and stream (no current-device query).
void* alloc_on(int device, size_t nbytes, hipStream_t stream);
void record_stream_raw(void* ptr, hipStream_t stream);
void empty_cache_device(int device);

// Serves segments from host memory with immediately-completing events, so
// the bookkeeping can be tested without a GPU.  Must be chosen before the
// first allocation.
void use_host_memory_for_tests(size_t capacity);
bool host_memory_mode();

// Workspace callbacks handed to the kernel library (mi_set_workspace_allocator).
void* workspace_alloc(size_t bytes, void* stream, void* ctx);
void workspace_free(void* ptr, void* stream, void* ctx);

// PYTORCH_GCU_ALLOC_CONF settings in effect.
struct Config {
  size_t max_split_size = SIZE_MAX;
  double garbage_collection_threshold = 0.0;
  size_t roundup_power2_divisions = 0;
};
const Config& config();
// Parses a PYTORCH_GCU_ALLOC_CONF string ("key:value,key:value").
Config parse_config(const std::string& s);

}  // namespace allocator
}  // namespace torch_gcu
