// Python bindings of the caching allocator's memory history, snapshots,
// graph-pool checkpoints and raw allocation (the reference's
// python/gcu_memory_snapshot.cpp:20-108 and python/gcu_module.cpp:254-300,
// :1094-1226, surfaced by torch_gcu/gcu/memory.py:54-100, :635-785, :856-934).
//
// Stacks are torch::CapturedTraceback objects (Python frames, plus C++ frames
// when stacks="all"), gathered by the allocator outside its lock and
// symbolised only when a snapshot is taken, so that recording costs a few
// microseconds per event.
#include <torch/csrc/profiler/combined_traceback.h>
#include <torch/extension.h>

#include <c10/core/StorageImpl.h>

#include <algorithm>
#include <thread>
#include <unordered_set>

#include "gcu_caching_allocator.h"
#include "gcu_runtime.h"

namespace torch {
// Exported by libtorch_python (torch/csrc/profiler/python/combined_traceback.h,
// whose nlohmann include is not shipped with the wheel): frames of each
// traceback as a list of {"filename", "line", "name"} dicts, and the
// registration of the Python unwinder that CapturedTraceback::gather uses.
std::vector<pybind11::object> py_symbolize(std::vector<CapturedTraceback*>& to_symbolize);
void installCapturedTracebackPython();
}  // namespace torch

namespace py = pybind11;

namespace torch_gcu {
namespace {

using allocator::Context;

Context gather_python() { return torch::CapturedTraceback::gather(true, true, false); }
Context gather_python_cpp() { return torch::CapturedTraceback::gather(true, true, true); }

void check_in(const std::string& v, std::initializer_list<const char*> ok, const char* what) {
  for (const char* o : ok)
    if (v == o) return;
  TORCH_CHECK(false, "_record_memory_history: ", what);
}

// enabled None / "state" / "all"; context None / "state" / "alloc" / "all";
// stacks "python" / "all" (torch_gcu/gcu/memory.py:635-690).
void record_memory_history(std::optional<std::string> enabled, std::optional<std::string> context,
                           const std::string& stacks, size_t max_entries) {
  if (enabled) check_in(*enabled, {"state", "all"}, "expected enabled to be 'state', 'all' or None");
  if (context)
    check_in(*context, {"state", "alloc", "all"},
             "expected context to be 'state', 'alloc', 'all' or None");
  check_in(stacks, {"python", "all"}, "expected stacks to be 'python' or 'all'");
  static bool installed = false;
  if (!installed) {
    torch::installCapturedTracebackPython();
    installed = true;
  }
  auto when = allocator::RecordContext::NEVER;
  if (context) {
    if (*context == "all") when = allocator::RecordContext::ALL;
    else if (*context == "alloc") when = allocator::RecordContext::ALLOC;
    else when = allocator::RecordContext::STATE;
  }
  // "state" keeps no event history beyond the last one
  const size_t entries = (enabled && *enabled == "all") ? max_entries : 1;
  allocator::record_history(enabled.has_value(), stacks == "all" ? &gather_python_cpp : &gather_python,
                            entries, when);
}

// The legacy boolean form (memory.py:618-632).
void record_memory_history_legacy(bool enabled, bool record_context, bool record_context_cpp,
                                  size_t trace_alloc_max_entries, bool trace_alloc_record_context) {
  static bool installed = false;
  if (!installed) {
    torch::installCapturedTracebackPython();
    installed = true;
  }
  auto when = allocator::RecordContext::NEVER;
  if (trace_alloc_record_context) when = allocator::RecordContext::ALLOC;
  else if (record_context) when = allocator::RecordContext::STATE;
  allocator::record_history(enabled, record_context_cpp ? &gather_python_cpp : &gather_python,
                            trace_alloc_max_entries, when);
}

const char* action_name(allocator::TraceAction a) {
  switch (a) {
    case allocator::TraceAction::ALLOC: return "alloc";
    case allocator::TraceAction::FREE_REQUESTED: return "free_requested";
    case allocator::TraceAction::FREE_COMPLETED: return "free_completed";
    case allocator::TraceAction::SEGMENT_ALLOC: return "segment_alloc";
    case allocator::TraceAction::SEGMENT_FREE: return "segment_free";
    case allocator::TraceAction::SNAPSHOT: return "snapshot";
    case allocator::TraceAction::OOM: return "oom";
  }
  return "unknown";
}

// Segments, blocks and history as torch.cuda.memory._snapshot() lays them
// out; every context is symbolised in one batch.
py::dict full_snapshot() {
  const allocator::Snapshot snap = allocator::full_snapshot();
  // pass 1: collect the contexts in a fixed order
  std::vector<torch::CapturedTraceback*> tbs;
  auto take = [&](const Context& c) -> long {
    auto* tb = dynamic_cast<torch::CapturedTraceback*>(c.get());
    if (!tb) return -1;
    tbs.push_back(tb);
    return (long)tbs.size() - 1;
  };
  std::vector<long> seg_ix, blk_ix, trc_ix;
  for (const auto& s : snap.segments) {
    seg_ix.push_back(take(s.context));
    for (const auto& b : s.blocks) blk_ix.push_back(take(b.context));
  }
  for (const auto& dt : snap.device_traces)
    for (const auto& e : dt) trc_ix.push_back(take(e.context));
  std::vector<py::object> frames = tbs.empty() ? std::vector<py::object>() : torch::py_symbolize(tbs);
  auto frames_of = [&](long i) -> py::object { return i < 0 ? py::object(py::list()) : frames[i]; };

  py::list segments;
  size_t bi = 0;
  for (size_t si = 0; si < snap.segments.size(); ++si) {
    const auto& s = snap.segments[si];
    py::dict d;
    d["device"] = s.device;
    d["address"] = s.address;
    d["total_size"] = s.total_size;
    d["allocated_size"] = s.allocated_size;
    d["active_size"] = s.active_size;
    d["requested_size"] = s.requested_size;
    d["stream"] = s.stream;
    d["segment_type"] = s.is_large ? "large" : "small";
    d["segment_pool_id"] = py::make_tuple(s.owner_pool.first, s.owner_pool.second);
    d["is_expandable"] = false;
    d["frames"] = frames_of(seg_ix[si]);
    py::list blocks;
    for (const auto& b : s.blocks) {
      py::dict bd;
      bd["address"] = b.address;
      bd["size"] = b.size;
      bd["requested_size"] = b.requested_size;
      bd["state"] = b.allocated ? "active_allocated" : (b.active ? "active_pending_free" : "inactive");
      bd["frames"] = frames_of(blk_ix[bi++]);
      blocks.append(bd);
    }
    d["blocks"] = blocks;
    segments.append(d);
  }
  py::list traces;
  size_t ti = 0;
  for (const auto& dt : snap.device_traces) {
    py::list l;
    for (const auto& e : dt) {
      py::dict d;
      d["action"] = action_name(e.action);
      if (e.action == allocator::TraceAction::OOM) d["device_free"] = e.addr;
      else d["addr"] = e.addr;
      d["size"] = e.size;
      d["stream"] = e.stream;
      d["time_us"] = e.time_us;
      d["frames"] = frames_of(trc_ix[ti++]);
      l.append(d);
    }
    traces.append(l);
  }
  const auto& cfg = allocator::config();
  py::dict settings;
  const char* env = std::getenv("PYTORCH_GCU_ALLOC_CONF");
  settings["PYTORCH_GCU_ALLOC_CONF"] = env ? env : "";
  settings["max_split_size"] =
      cfg.max_split_size == SIZE_MAX ? (int64_t)-1 : (int64_t)cfg.max_split_size;
  settings["garbage_collection_threshold"] = cfg.garbage_collection_threshold;
  settings["expandable_segments"] = false;
  settings["roundup_power2_divisions"] = cfg.roundup_power2_divisions;
  py::dict out;
  out["segments"] = segments;
  out["device_traces"] = traces;
  out["allocator_settings"] = settings;
  return out;
}

allocator::MempoolId pool_id(const py::tuple& t) {
  TORCH_CHECK(t.size() == 2, "a memory pool id is a tuple of two ints");
  return {t[0].cast<uint64_t>(), t[1].cast<uint64_t>()};
}

// setCheckpointPoolState with the storages of live tensors
// (gcu_module.cpp:1176-1226): storages whose blocks the restore freed lose
// their deleter (their tensors are stale, the memory now belongs to the
// checkpoint's layout), and storages created without a deleter whose
// pointers the restore allocated get the allocator's deleter.
py::tuple set_checkpoint(int device, const std::shared_ptr<allocator::PoolState>& st,
                         const std::vector<uintptr_t>& stale_storages,
                         const std::vector<uintptr_t>& storages_to_add_deleters_to) {
  TORCH_CHECK(st != nullptr, "expected a pool state from _get_checkpoint_state");
  std::vector<c10::StorageImpl*> stale;
  std::unordered_set<c10::StorageImpl*> seen;
  for (uintptr_t p : stale_storages) {
    auto* s = (c10::StorageImpl*)p;
    if (seen.insert(s).second) stale.push_back(s);
  }
  // The restore frees every block the pool holds now; those the checkpoint
  // does not allocate again belong to tensors that go stale.  Checked before
  // anything changes.
  {
    std::unordered_set<uintptr_t> target;
    for (const auto& seg : st->segments)
      for (const auto& b : seg)
        if (b.allocated) target.insert(b.ptr);
    size_t definitely_freed = 0;
    const std::shared_ptr<allocator::PoolState> now = allocator::get_checkpoint_state(device, st->id);
    for (const auto& seg : now->segments)
      for (const auto& b : seg)
        if (b.allocated && !target.count(b.ptr)) ++definitely_freed;
    TORCH_CHECK(stale.size() >= definitely_freed,
                "every stale tensor whose memory the checkpoint frees must be passed as stale");
  }
  const allocator::CheckpointDelta delta = allocator::set_checkpoint_pool_state(device, *st);
  std::unordered_set<void*> allocd(delta.allocated.begin(), delta.allocated.end());
  std::unordered_set<void*> freed(delta.freed.begin(), delta.freed.end());
  const c10::DeleterFnPtr del = allocator::raw_deleter();
  for (c10::StorageImpl* s : stale) {
    if (!s->data_ptr().get()) continue;
    TORCH_CHECK(freed.count(s->data_ptr().get()),
                "a stale storage was not freed by the checkpoint restore");
    const bool ok = s->mutable_data_ptr().compare_exchange_deleter(del, c10::detail::deleteNothing);
    TORCH_CHECK(ok, "a stale storage does not hold the allocator's deleter");
  }
  for (uintptr_t p : storages_to_add_deleters_to) {
    auto* s = (c10::StorageImpl*)p;
    void* ptr = s->data_ptr().get();
    TORCH_CHECK(allocd.count(ptr), "a storage to own its memory was not allocated by the restore");
    s->set_data_ptr_noswap(c10::DataPtr(ptr, ptr, del, c10::Device(kGCU, (c10::DeviceIndex)device)));
  }
  py::list f, a;
  for (void* p : delta.freed) f.append((uintptr_t)p);
  for (void* p : delta.allocated) a.append((uintptr_t)p);
  return py::make_tuple(f, a);
}

}  // namespace

void bind_memory(py::module& m) {
  m.def("_record_memory_history", &record_memory_history, py::arg("enabled"), py::arg("context"),
        py::arg("stacks"), py::arg("max_entries"));
  m.def("_record_memory_history_legacy", &record_memory_history_legacy);
  m.def("_is_history_enabled", &allocator::history_enabled);
  m.def("_memory_snapshot_full", &full_snapshot);
  m.def("_cache_info", [](int device) {
    size_t largest = 0;
    allocator::cache_info(device, &largest);
    return largest;
  });
  m.def("_cache_info_from", [](int device, size_t start) {
    allocator::cache_info(device, &start);
    return start;
  });
  m.def("_get_base_allocation", [](uintptr_t ptr) {
    size_t size = 0;
    void* base = allocator::get_base_allocation((void*)ptr, &size);
    return py::make_tuple((uintptr_t)base, size);
  });
  m.def("_check_pool_live_allocations", [](int device, const py::tuple& id, const py::iterable& live) {
    std::unordered_set<void*> expected;
    for (auto h : live) expected.insert((void*)h.cast<uintptr_t>());
    return allocator::check_pool_live_allocations(device, pool_id(id), expected);
  });
  py::class_<allocator::PoolState, std::shared_ptr<allocator::PoolState>>(m, "_PoolState")
      .def_property_readonly("device", [](const allocator::PoolState& s) { return s.device; })
      .def_property_readonly("pool_id", [](const allocator::PoolState& s) {
        return py::make_tuple(s.id.first, s.id.second);
      })
      .def_property_readonly("segments", [](const allocator::PoolState& s) {
        py::list out;
        for (const auto& seg : s.segments) {
          py::list l;
          for (const auto& b : seg) l.append(py::make_tuple(b.ptr, b.size, b.allocated));
          out.append(l);
        }
        return out;
      });
  m.def("_get_checkpoint_state", [](int device, const py::tuple& id) {
    return allocator::get_checkpoint_state(device, pool_id(id));
  });
  m.def("_set_checkpoint_pool_state", &set_checkpoint, py::arg("device"), py::arg("state"),
        py::arg("stale_storages") = std::vector<uintptr_t>(),
        py::arg("storages_to_add_deleters_to") = std::vector<uintptr_t>());
  // pointer-level form for raw allocations (no storages to update)
  m.def("_set_checkpoint_pool_state_raw", [](int device, const std::shared_ptr<allocator::PoolState>& st) {
    TORCH_CHECK(st != nullptr, "expected a pool state from _get_checkpoint_state");
    const allocator::CheckpointDelta delta = allocator::set_checkpoint_pool_state(device, *st);
    py::list f, a;
    for (void* p : delta.freed) f.append((uintptr_t)p);
    for (void* p : delta.allocated) a.append((uintptr_t)p);
    return py::make_tuple(f, a);
  });
  m.def("_storage_ptr", [](const at::Tensor& t) {
    return (uintptr_t)t.storage().unsafeGetStorageImpl();
  });
  m.def("_has_standard_deleter", [](uintptr_t storage) {
    return ((c10::StorageImpl*)storage)->data_ptr().get_deleter() == allocator::raw_deleter();
  });
  // raw allocation for interoperability (memory.py:54-100)
  m.def("_caching_allocator_alloc", [](int device, size_t size, uintptr_t stream) {
    return (uintptr_t)allocator::alloc_on(device, size, (hipStream_t)stream);
  });
  m.def("_caching_allocator_delete", [](uintptr_t p) { allocator::raw_delete((void*)p); });
  // routing of one thread's allocations to a pool (use_mem_pool)
  m.def("_begin_allocate_current_thread_to_pool", [](int device, const py::tuple& id) {
    const auto tid = std::this_thread::get_id();
    allocator::begin_allocate_to_pool(device, pool_id(id),
                                      [tid](hipStream_t) { return std::this_thread::get_id() == tid; });
  });
  m.def("_end_allocate_to_pool", [](int device, const py::tuple& id) {
    allocator::end_allocate_to_pool(device, pool_id(id));
  });
  m.def("_release_pool", [](int device, const py::tuple& id) {
    allocator::release_pool(device, pool_id(id));
  });
}

}  // namespace torch_gcu
