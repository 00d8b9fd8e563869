// torch_gcu._C: Python bindings of the gcu runtime (the reference's
// torch_gcu/csrc/InitGcuBindings.cpp:251-292 and python/gcu_module.cpp:
// device and stream functions :995-1080, memory APIs, graph pool APIs
// :1094-1180; python/gcu_py_graph.cpp:12-70; python/efficient_ops.cpp:12-26).
#include <torch/extension.h>

#include "efficient_ops.h"
#include "gcu_caching_allocator.h"
#include "gcu_caching_host_allocator.h"
#include "gcu_graph.h"
#include "gcu_runtime.h"
#include "op_debug.h"

namespace torch_gcu {
void ensure_initialized();
bool is_initialized();
void register_library_workspace();
void bind_memory(pybind11::module& m);  // memory_bindings.cpp
}

namespace py = pybind11;
using namespace torch_gcu;

namespace {

py::dict stats_dict(int device) {
  const auto s = allocator::get_stats(device);
  py::dict d;
  const char* pools[3] = {"all", "small_pool", "large_pool"};
  auto put = [&](const char* name, const std::array<allocator::Stat, 3>& arr) {
    for (int i = 0; i < 3; ++i) {
      const std::string base = std::string(name) + "." + pools[i] + ".";
      d[py::str(base + "current")] = arr[i].current;
      d[py::str(base + "peak")] = arr[i].peak;
      d[py::str(base + "allocated")] = arr[i].allocated;
      d[py::str(base + "freed")] = arr[i].freed;
    }
  };
  put("allocation", s.allocation);
  put("segment", s.segment);
  put("active", s.active);
  put("inactive_split", s.inactive_split);
  put("allocated_bytes", s.allocated_bytes);
  put("reserved_bytes", s.reserved_bytes);
  put("active_bytes", s.active_bytes);
  put("inactive_split_bytes", s.inactive_split_bytes);
  put("requested_bytes", s.requested_bytes);
  d["num_alloc_retries"] = s.num_alloc_retries;
  d["num_ooms"] = s.num_ooms;
  d["num_sync_all_streams"] = s.num_sync_all_streams;
  d["num_device_alloc"] = s.num_device_alloc;
  d["num_device_free"] = s.num_device_free;
  d["max_split_size"] = s.max_split_size;
  return d;
}

py::tuple stream_tuple(c10::Stream s) {
  return py::make_tuple(s.id(), (int)s.device_index(), (int)s.device_type());
}

// The calling Python stack, for op_calltrace (the reference's
// GetPythonFrame); empty when the interpreter is not running.
std::string python_stack() {
  if (!Py_IsInitialized()) return std::string();
  py::gil_scoped_acquire gil;
  try {
    std::string s;
    for (const auto& line : py::module::import("traceback").attr("format_stack")())
      s += line.cast<std::string>();
    return s;
  } catch (const std::exception& e) {
    return std::string("  <Python stack unavailable: ") + e.what() + ">\n";
  }
}

c10::Stream stream_from(int64_t id, int device) {
  return c10::Stream(c10::Stream::UNSAFE, c10::Device(kGCU, (c10::DeviceIndex)device), id);
}

}  // namespace

PYBIND11_MODULE(_C, m) {
  m.doc() = "torch_gcu MI355X runtime";

  m.def("_init", &ensure_initialized);
  m.def("_is_initialized", &is_initialized);
  // registers the caching allocator with the kernel library again (after a
  // direct C-ABI caller installed its own workspace allocator)
  m.def("_register_library_workspace", &register_library_workspace);
  m.def("_device_count", []() { return (int)device_count(); });
  m.def("_current_device", []() { return (int)current_device(); });
  m.def("_set_device", [](int d) { set_device((c10::DeviceIndex)d); });
  m.def("_synchronize", [](int d) {
    py::gil_scoped_release r;
    device_synchronize((c10::DeviceIndex)(d < 0 ? current_device() : d));
  });
  m.def("_device_properties", [](int d) {
    hipDeviceProp_t p;
    GCU_HIP_CHECK(hipGetDeviceProperties(&p, d));
    py::dict r;
    r["name"] = std::string(p.name);
    r["gcn_arch_name"] = std::string(p.gcnArchName);
    r["total_memory"] = (int64_t)p.totalGlobalMem;
    r["multi_processor_count"] = p.multiProcessorCount;
    r["clock_rate_khz"] = p.clockRate;
    r["memory_clock_rate_khz"] = p.memoryClockRate;
    r["memory_bus_width"] = p.memoryBusWidth;
    r["l2_cache_size"] = p.l2CacheSize;
    r["shared_mem_per_block"] = (int64_t)p.sharedMemPerBlock;
    r["warp_size"] = p.warpSize;
    return r;
  });
  m.def("_mem_get_info", [](int d) {
    const auto prev = current_device();
    maybe_set_device((c10::DeviceIndex)d);
    size_t f = 0, t = 0;
    GCU_HIP_CHECK(hipMemGetInfo(&f, &t));
    maybe_set_device(prev);
    return py::make_tuple((int64_t)f, (int64_t)t);
  });

  // streams: (stream_id, device_index, device_type) triples as torch.Stream uses
  m.def("_current_stream", [](int d) { return stream_tuple(current_stream((c10::DeviceIndex)d)); });
  m.def("_default_stream", [](int d) { return stream_tuple(default_stream((c10::DeviceIndex)d)); });
  m.def("_set_current_stream", [](int64_t id, int d) { set_current_stream(stream_from(id, d)); });
  m.def("_stream_handle", [](int64_t id, int d) { return (uintptr_t)stream_handle(stream_from(id, d)); });
  m.def("_wrap_external_stream", [](uintptr_t h, int d) {
    return stream_tuple(wrap_external_stream((c10::DeviceIndex)d, (hipStream_t)h));
  });
  m.def("_stream_pool_size", &stream_pool_size);

  // memory
  m.def("_memory_stats", &stats_dict);
  m.def("_reset_peak_memory_stats", &allocator::reset_peak_stats);
  m.def("_reset_accumulated_memory_stats", &allocator::reset_accumulated_stats);
  m.def("_empty_cache", []() { allocator::empty_cache(); });
  m.def("_host_empty_cache", &host_allocator::empty_cache);
  m.def("_host_memory_stats", []() {
    const host_allocator::Stats s = host_allocator::stats();
    py::dict d;
    d["allocated_bytes"] = s.allocated_bytes;
    d["reserved_bytes"] = s.reserved_bytes;
    d["num_blocks"] = s.num_blocks;
    d["num_host_alloc"] = s.num_host_alloc;
    d["num_host_free"] = s.num_host_free;
    d["num_cache_hits"] = s.num_cache_hits;
    d["pending_events"] = s.pending_events;
    return d;
  });
  m.def("_host_allocator_use_plain_memory", &host_allocator::use_plain_memory_for_tests);
  m.def("_set_memory_fraction", &allocator::set_memory_fraction);
  m.def("_get_memory_fraction", &allocator::get_memory_fraction);
  m.def("_memory_snapshot", []() {
    py::list out;
    for (const auto& s : allocator::snapshot()) {
      py::dict d;
      d["device"] = s.device;
      d["address"] = s.address;
      d["total_size"] = s.total_size;
      d["allocated_size"] = s.allocated_size;
      d["active_size"] = s.active_size;
      d["segment_type"] = s.is_large ? "large" : "small";
      d["segment_pool_id"] = py::make_tuple(s.owner_pool.first, s.owner_pool.second);
      d["stream"] = s.stream;
      d["requested_size"] = s.requested_size;
      py::list blocks;
      for (const auto& b : s.blocks) {
        py::dict bd;
        bd["address"] = b.address;
        bd["size"] = b.size;
        bd["requested_size"] = b.requested_size;
        bd["state"] = b.allocated ? "active_allocated" : (b.active ? "active_pending_free" : "inactive");
        blocks.append(bd);
      }
      d["blocks"] = blocks;
      out.append(d);
    }
    return out;
  });
  bind_memory(m);
  m.def("_parse_alloc_conf", [](const std::string& s) {
    const auto c = allocator::parse_config(s);
    py::dict d;
    d["max_split_size"] = c.max_split_size == SIZE_MAX ? (int64_t)-1 : (int64_t)c.max_split_size;
    d["garbage_collection_threshold"] = c.garbage_collection_threshold;
    d["roundup_power2_divisions"] = c.roundup_power2_divisions;
    return d;
  });
  // allocator bookkeeping on host memory (CPU tests; no GPU involved)
  m.def("_allocator_use_host_memory", &allocator::use_host_memory_for_tests);
  m.def("_allocator_host_memory_mode", &allocator::host_memory_mode);
  m.def("_allocator_alloc", [](int device, size_t n, uintptr_t stream) {
    return (uintptr_t)allocator::alloc_on(device, n, (hipStream_t)stream);
  });
  m.def("_allocator_free", [](uintptr_t p) { allocator::raw_delete((void*)p); });
  m.def("_allocator_record_stream", [](uintptr_t p, uintptr_t s) {
    allocator::record_stream_raw((void*)p, (hipStream_t)s);
  });
  m.def("_allocator_empty_cache_device", &allocator::empty_cache_device);
  m.def("_allocator_new_pool", []() {
    const auto id = allocator::new_pool_id();
    return py::make_tuple(id.first, id.second);
  });
  m.def("_allocator_begin_pool", [](int device, uint64_t a, uint64_t b, uintptr_t stream) {
    allocator::begin_allocate_to_pool(device, {a, b},
                                      [stream](hipStream_t s) { return (uintptr_t)s == stream; });
  });
  m.def("_allocator_end_pool", [](int device, uint64_t a, uint64_t b) {
    allocator::end_allocate_to_pool(device, {a, b});
  });
  m.def("_allocator_release_pool", [](int device, uint64_t a, uint64_t b) {
    allocator::release_pool(device, {a, b});
  });

  // graphs
  // graphs.py:28-34: capture state of the current stream, false (and no
  // runtime initialisation) before the device is used
  m.def("_is_current_stream_capturing", []() {
    if (!is_initialized()) return false;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    GCU_HIP_CHECK(hipStreamIsCapturing(current_hip_stream(), &st));
    return st == hipStreamCaptureStatusActive;
  });
  m.def("_graph_pool_handle", []() {
    const auto id = allocator::new_pool_id();
    return py::make_tuple(id.first, id.second);
  });
  py::class_<GCUGraph>(m, "_GCUGraph")
      .def(py::init<>())
      .def("capture_begin",
           [](GCUGraph& g, py::tuple pool, const std::string& mode) {
             allocator::MempoolId id{0, 0};
             if (pool.size() == 2) id = {pool[0].cast<uint64_t>(), pool[1].cast<uint64_t>()};
             hipStreamCaptureMode cm = hipStreamCaptureModeGlobal;
             if (mode == "thread_local") cm = hipStreamCaptureModeThreadLocal;
             else if (mode == "relaxed") cm = hipStreamCaptureModeRelaxed;
             else TORCH_CHECK(mode == "global", "unknown capture_error_mode ", mode);
             py::gil_scoped_release r;
             g.capture_begin(id, cm);
           },
           py::arg("pool") = py::make_tuple(), py::arg("capture_error_mode") = "global")
      .def("capture_end", [](GCUGraph& g) {
        py::gil_scoped_release r;
        g.capture_end();
      })
      .def("replay", [](GCUGraph& g) {
        py::gil_scoped_release r;
        g.replay();
      })
      .def("reset", [](GCUGraph& g) { g.reset(); })
      .def("pool", [](GCUGraph& g) {
        const auto id = g.pool();
        return py::make_tuple(id.first, id.second);
      })
      .def("enable_debug_mode", &GCUGraph::enable_debug_mode)
      .def("debug_dump", &GCUGraph::debug_dump)
      .def("num_nodes", &GCUGraph::num_nodes);

  // efficient ops (pybind aliases of torch.ops.torch_gcu.*)
  m.def("_rms_norm", &efficient::rms_norm, py::arg("x"), py::arg("weight"), py::arg("eps") = 1e-6);
  m.def("_rope", &efficient::rope);
  m.def("_silu_mul", &efficient::silu_mul);
  m.def("_linear_residual", &efficient::linear_residual);
  m.def("_linear_silu_mul", &efficient::linear_silu_mul);
  m.def("_int32_indices_index", [](const at::Tensor& self, std::vector<std::optional<at::Tensor>> idx) {
    c10::List<std::optional<at::Tensor>> l;
    for (auto& i : idx) l.push_back(i);
    return efficient::int32_indices_index(self, l);
  });

  // op debug (the reference's torch_gcu/csrc/InitGcuBindings.cpp:131-153)
  m.def("_set_op_debug_config", &set_op_debug_config);
  m.def("_op_debug_config", []() {
    const OpDebugConfig& c = OpDebugConfig::get();
    py::dict d;
    d["dump_path"] = c.dump_path;
    d["op_check_dump_dir"] = c.check_dump_dir;
    d["op_dump_dir"] = c.op_dump_dir;
    d["op_statistics"] = c.statistics;
    d["op_statistics_dump"] = c.statistics_dump;
    d["op_check_tol"] = py::make_tuple(py::make_tuple(c.rtol_fp32, c.atol_fp32),
                                       py::make_tuple(c.rtol_fp16, c.atol_fp16),
                                       py::make_tuple(c.rtol_bf16, c.atol_bf16));
    return d;
  });
  m.def("_op_statistics", []() {
    py::dict d;
    for (const auto& kv : op_statistics()) d[py::str(kv.first)] = py::make_tuple(kv.second.first, kv.second.second);
    return d;
  });
  m.def("_op_check_statistics", []() {
    py::dict d;
    for (const auto& kv : op_check_statistics()) {
      py::dict e;
      e["compared"] = kv.second.compared;
      e["failed"] = kv.second.failed;
      e["max_ratio"] = kv.second.max_ratio;
      e["min_ref_rms"] = kv.second.min_ref_rms;
      d[py::str(kv.first)] = e;
    }
    return d;
  });
  m.def("_clear_op_check_statistics", &clear_op_check_statistics);
  m.def("_clear_op_statistics", &clear_op_statistics);
  m.def("_clear_statistics", &clear_op_statistics);
  m.def("_get_op_statistics_info", &op_statistics_info);
  m.def("_dump_op_statistics_to_json", &dump_op_statistics_json);
  m.def("_enter_dump_op_name_scope", []() { set_scope(0, true); });
  m.def("_exit_print_cpp_name_scope", []() { set_scope(0, false); });
  m.def("_enter_fallback_cpu_scope", []() { set_scope(1, true); });
  m.def("_exit_fallback_cpu_scope", []() { set_scope(1, false); });
  m.def("_enter_op_check_scope", []() { set_scope(2, true); });
  m.def("_exit_op_check_scope", []() { set_scope(2, false); });
  m.def("_get_dump_op_name_scope_state", []() { return scope_state(0); });
  m.def("_get_fallback_cpu_scope_state", []() { return scope_state(1); });
  m.def("_get_op_check_scope_state", []() { return scope_state(2); });
  m.def("_fallback_policy", []() {
    py::dict d;
    for (const auto& kv : fallback_policy()) d[py::str(kv.first)] = kv.second;
    return d;
  });
  set_python_stack_fn(&python_stack);
}
