#include "gcu_runtime.h"
#include "mi355x_ops.h"

#include <c10/core/impl/DeviceGuardImplInterface.h>
#include <c10/core/impl/GPUTrace.h>

#include <atomic>
#include <cstdlib>
#include <deque>
#include <mutex>
#include <vector>

#include "op_debug.h"

namespace torch_gcu {

// ---- devices ------------------------------------------------------------------

c10::DeviceIndex device_count() noexcept {
  static int count = [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    return n;
  }();
  return (c10::DeviceIndex)count;
}

c10::DeviceIndex current_device() {
  int d = 0;
  GCU_HIP_CHECK(hipGetDevice(&d));
  return (c10::DeviceIndex)d;
}

void set_device(c10::DeviceIndex d) {
  TORCH_CHECK(d >= 0 && d < device_count(), "gcu: invalid device index ", (int)d,
              " (device count ", (int)device_count(), ")");
  GCU_HIP_CHECK(hipSetDevice(d));
}

void maybe_set_device(c10::DeviceIndex d) {
  if (current_device() != d) set_device(d);
}

void device_synchronize(c10::DeviceIndex d) {
  const auto prev = current_device();
  maybe_set_device(d);
  GCU_HIP_CHECK(hipDeviceSynchronize());
  maybe_set_device(prev);
  check_index_faults(d);
}

// The gather kernels record an out-of-range index instead of reading outside
// their source; once the work has been waited for, the record is raised
// here as CPU ATen raises it for the same input (IndexError), as a CUDA
// device-side assertion is reported at the next synchronisation.
void check_index_faults(c10::DeviceIndex d) {
  int64_t index = 0, size = 0;
  if (mi_index_fault_take((int32_t)d, &index, &size) != 0)
    TORCH_CHECK_INDEX(false, "index ", index, " is out of bounds for dimension with size ", size,
                      " (read by an index_select or index kernel on gcu:", (int)d,
                      "; reported at the next synchronization)");
}

// ---- streams ------------------------------------------------------------------

namespace {

struct StreamEntry {
  hipStream_t handle = nullptr;
  bool owned = false;
};

struct DeviceStreams {
  std::once_flag init;
  std::mutex mu;
  std::deque<StreamEntry> registry;  // id - 1 -> entry (deque: stable refs)
  int pool_size = 0;
  std::atomic<uint32_t> next{0};
};

constexpr int kMaxDevices = 64;
DeviceStreams g_streams[kMaxDevices];

thread_local c10::StreamId tls_current[kMaxDevices] = {};  // 0: null stream

void init_device_streams(c10::DeviceIndex d) {
  DeviceStreams& ds = g_streams[d];
  std::call_once(ds.init, [&] {
    const int n = stream_pool_size();
    const auto prev = current_device();
    maybe_set_device(d);
    std::lock_guard<std::mutex> g(ds.mu);
    for (int i = 0; i < n; ++i) {
      hipStream_t s;
      // Default priority on purpose: every stream of this library shares it.
      GCU_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
      ds.registry.push_back({s, true});
    }
    ds.pool_size = n;
    maybe_set_device(prev);
  });
}

c10::DeviceIndex resolve(c10::DeviceIndex d) { return d < 0 ? current_device() : d; }

c10::Stream make_stream(c10::DeviceIndex d, c10::StreamId id) {
  return c10::Stream(c10::Stream::UNSAFE, c10::Device(kGCU, d), id);
}

}  // namespace

int stream_pool_size() {
  static int n = [] {
    const char* e = std::getenv("ENFLAME_PT_STREAM_NUM");
    int v = e ? std::atoi(e) : 32;
    return v < 1 ? 1 : (v > 1024 ? 1024 : v);
  }();
  return n;
}

hipStream_t stream_handle(c10::Stream s) {
  TORCH_CHECK(s.device_type() == kGCU, "expected a gcu stream, got ", s);
  if (s.id() == 0) return nullptr;
  const auto d = s.device_index();
  init_device_streams(d);
  DeviceStreams& ds = g_streams[d];
  std::lock_guard<std::mutex> g(ds.mu);
  TORCH_CHECK(s.id() >= 1 && (size_t)s.id() <= ds.registry.size(), "gcu: unknown stream id ",
              s.id());
  return ds.registry[s.id() - 1].handle;
}

c10::Stream default_stream(c10::DeviceIndex d) { return make_stream(resolve(d), 0); }

c10::Stream current_stream(c10::DeviceIndex d) {
  d = resolve(d);
  TORCH_CHECK(d < kMaxDevices, "gcu: device index too large");
  return make_stream(d, tls_current[d]);
}

void set_current_stream(c10::Stream s) {
  TORCH_CHECK(s.device_type() == kGCU, "expected a gcu stream, got ", s);
  tls_current[s.device_index()] = s.id();
}

c10::Stream pool_stream(c10::DeviceIndex d) {
  d = resolve(d);
  init_device_streams(d);
  DeviceStreams& ds = g_streams[d];
  const uint32_t k = ds.next.fetch_add(1) % (uint32_t)ds.pool_size;
  return make_stream(d, (c10::StreamId)k + 1);
}

c10::Stream new_stream(c10::DeviceIndex d) {
  d = resolve(d);
  init_device_streams(d);
  const auto prev = current_device();
  maybe_set_device(d);
  hipStream_t s;
  GCU_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  maybe_set_device(prev);
  DeviceStreams& ds = g_streams[d];
  std::lock_guard<std::mutex> g(ds.mu);
  ds.registry.push_back({s, true});
  return make_stream(d, (c10::StreamId)ds.registry.size());
}

c10::Stream wrap_external_stream(c10::DeviceIndex d, hipStream_t h) {
  d = resolve(d);
  if (h == nullptr) return default_stream(d);
  init_device_streams(d);
  DeviceStreams& ds = g_streams[d];
  std::lock_guard<std::mutex> g(ds.mu);
  for (size_t i = 0; i < ds.registry.size(); ++i)
    if (ds.registry[i].handle == h) return make_stream(d, (c10::StreamId)i + 1);
  ds.registry.push_back({h, false});
  return make_stream(d, (c10::StreamId)ds.registry.size());
}

hipStream_t current_hip_stream(c10::DeviceIndex d) { return stream_handle(current_stream(d)); }

void maybe_sync_after_op(hipStream_t s) {
  if (OpDebugConfig::get().op_sync_mode && !stream_is_capturing(s)) {
    GCU_HIP_CHECK(hipStreamSynchronize(s));
    check_index_faults(current_device());
  }
}

bool stream_is_capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st == hipStreamCaptureStatusActive;
}

// ---- c10 device guard ------------------------------------------------------------

namespace {

struct GCUGuardImpl final : public c10::impl::DeviceGuardImplInterface {
  c10::DeviceType type() const override { return kGCU; }

  c10::Device exchangeDevice(c10::Device d) const override {
    TORCH_INTERNAL_ASSERT(d.type() == kGCU);
    const auto old = current_device();
    if (old != d.index()) set_device(d.index());
    return c10::Device(kGCU, old);
  }
  c10::Device getDevice() const override { return c10::Device(kGCU, current_device()); }
  void setDevice(c10::Device d) const override {
    TORCH_INTERNAL_ASSERT(d.type() == kGCU);
    maybe_set_device(d.index());
  }
  void uncheckedSetDevice(c10::Device d) const noexcept override {
    (void)hipSetDevice(d.index());
  }
  c10::Stream getStream(c10::Device d) const override { return current_stream(d.index()); }
  c10::Stream getDefaultStream(c10::Device d) const override {
    return default_stream(d.index());
  }
  c10::Stream getStreamFromGlobalPool(c10::Device d, bool) const override {
    return pool_stream(d.index());
  }
  c10::Stream getNewStream(c10::Device d, int priority) const override {
    TORCH_CHECK(priority == 0, "gcu: streams are created at the default priority only");
    return new_stream(d.index());
  }
  c10::Stream exchangeStream(c10::Stream s) const override {
    auto old = current_stream(s.device_index());
    set_current_stream(s);
    return old;
  }
  c10::DeviceIndex deviceCount() const noexcept override { return device_count(); }

  void destroyEvent(void* event, const c10::DeviceIndex device_index) const noexcept override {
    if (!event) return;
    const auto prev = current_device();
    (void)hipSetDevice(device_index);
    (void)hipEventDestroy((hipEvent_t)event);
    (void)hipSetDevice(prev);
  }

  void record(void** event, const c10::Stream& stream, const c10::DeviceIndex device_index,
              const c10::EventFlag flag) const override {
    TORCH_CHECK(device_index == -1 || device_index == stream.device_index(),
                "Event device index ", device_index, " does not match recording stream's ",
                stream.device_index());
    const auto prev = current_device();
    maybe_set_device(stream.device_index());
    hipEvent_t e = (hipEvent_t)*event;
    if (!e) {
      // torch.Event(enable_timing=True) asks for BACKEND_DEFAULT
      const unsigned flags =
          flag == c10::EventFlag::BACKEND_DEFAULT ? hipEventDefault : hipEventDisableTiming;
      GCU_HIP_CHECK(hipEventCreateWithFlags(&e, flags));
      *event = e;
    }
    GCU_HIP_CHECK(hipEventRecord(e, stream_handle(stream)));
    maybe_set_device(prev);
  }

  void block(void* event, const c10::Stream& stream) const override {
    if (!event) return;
    const auto prev = current_device();
    maybe_set_device(stream.device_index());
    GCU_HIP_CHECK(hipStreamWaitEvent(stream_handle(stream), (hipEvent_t)event, 0));
    maybe_set_device(prev);
  }

  bool queryEvent(void* event) const override {
    if (!event) return true;
    const hipError_t e = hipEventQuery((hipEvent_t)event);
    if (e == hipErrorNotReady) {
      (void)hipGetLastError();
      return false;
    }
    GCU_HIP_CHECK(e);
    return true;
  }

  bool queryStream(const c10::Stream& s) const override {
    const hipError_t e = hipStreamQuery(stream_handle(s));
    if (e == hipErrorNotReady) {
      (void)hipGetLastError();
      return false;
    }
    GCU_HIP_CHECK(e);
    return true;
  }
  void synchronizeStream(const c10::Stream& s) const override {
    GCU_HIP_CHECK(hipStreamSynchronize(stream_handle(s)));
    check_index_faults(s.device_index());
  }
  void synchronizeEvent(void* event) const override {
    if (event) GCU_HIP_CHECK(hipEventSynchronize((hipEvent_t)event));
  }
  void synchronizeDevice(const c10::DeviceIndex d) const override { device_synchronize(d); }

  void recordDataPtrOnStream(const c10::DataPtr& data_ptr,
                             const c10::Stream& stream) const override;

  double elapsedTime(void* e1, void* e2, const c10::DeviceIndex) const override {
    TORCH_CHECK(e1 && e2, "Both events must be recorded before calculating elapsed time.");
    float ms = 0.f;
    GCU_HIP_CHECK(hipEventElapsedTime(&ms, (hipEvent_t)e1, (hipEvent_t)e2));
    return ms;
  }
};

}  // namespace

}  // namespace torch_gcu

#include "gcu_caching_allocator.h"

namespace torch_gcu {
namespace {
void GCUGuardImpl::recordDataPtrOnStream(const c10::DataPtr& data_ptr,
                                         const c10::Stream& stream) const {
  allocator::record_stream(data_ptr, stream);
}
}  // namespace

C10_REGISTER_GUARD_IMPL(PrivateUse1, GCUGuardImpl);

}  // namespace torch_gcu
