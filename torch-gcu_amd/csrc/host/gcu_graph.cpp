#include "gcu_graph.h"

#include <c10/core/DeviceGuard.h>
#include <c10/util/Exception.h>

#include <atomic>

#include "gcu_runtime.h"

namespace torch_gcu {

namespace {
std::atomic<uint64_t> g_next_graph_id{1};
}

GCUGraph::GCUGraph() : id_(g_next_graph_id.fetch_add(1)) {}

GCUGraph::~GCUGraph() {
  try {
    reset();
  } catch (...) {
  }
}

void GCUGraph::capture_begin(allocator::MempoolId pool, hipStreamCaptureMode mode) {
  TORCH_CHECK(!has_exec_, "This GCUGraph instance was already used for a capture; call reset() "
              "before capturing again.");
  device_ = current_device();
  const c10::Stream stream = current_stream(device_);
  // gcu_graph.cpp:161-164: the legacy default stream cannot be captured
  TORCH_CHECK(stream.id() != 0,
              "GCU graphs must be captured on a non-default stream. "
              "(However, after capture, it's ok to replay them on the default stream.)");
  capture_stream_ = stream_handle(stream);
  if (pool.first != 0 || pool.second != 0) {
    mempool_ = pool;  // shared with another graph
  } else {
    mempool_ = {id_, 0};
  }
  const hipStream_t cs = capture_stream_;
  allocator::begin_allocate_to_pool(device_, mempool_, [cs](hipStream_t s) { return s == cs; });
  const hipError_t e = hipStreamBeginCapture(capture_stream_, mode);
  if (e != hipSuccess) {
    allocator::end_allocate_to_pool(device_, mempool_);
    GCU_HIP_CHECK(e);
  }
}

void GCUGraph::capture_end() {
  TORCH_CHECK(capture_stream_ != nullptr, "capture_end() called without capture_begin()");
  const c10::Stream stream = current_stream(device_);
  TORCH_CHECK(stream_handle(stream) == capture_stream_,
              "Capture must end on the same stream it began on.");
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(capture_stream_, &g);
  allocator::end_allocate_to_pool(device_, mempool_);
  if (e != hipSuccess || g == nullptr) {
    // nothing will replay: the pool's blocks go back to the caching allocator
    if (g != nullptr) (void)hipGraphDestroy(g);
    abandon_capture();
    TORCH_CHECK(false, "GCU graph capture failed (an operation in the captured region is not "
                "capturable, or the capture was invalidated): ", hipGetErrorString(e));
  }
  graph_ = g;
  has_graph_ = true;
  size_t n = 0;
  hipError_t ie = hipGraphGetNodes(graph_, nullptr, &n);
  if (ie == hipSuccess) ie = hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0);
  if (ie != hipSuccess) {
    (void)hipGraphDestroy(graph_);
    has_graph_ = false;
    abandon_capture();
    TORCH_CHECK(false, "GCU graph instantiation failed: ", hipGetErrorString(ie));
  }
  num_nodes_ = (int64_t)n;
  has_exec_ = true;
  if (!debug_) {
    GCU_HIP_CHECK(hipGraphDestroy(graph_));
    has_graph_ = false;
  }
}

void GCUGraph::replay() {
  TORCH_CHECK(has_exec_, "Called GCUGraph::replay without a preceding successful capture.");
  const c10::DeviceGuard guard(c10::Device(kGCU, (c10::DeviceIndex)device_));
  GCU_HIP_CHECK(hipGraphLaunch(exec_, current_hip_stream(device_)));
}

// A capture that produced no executable graph: releases the private pool
// (its blocks return to the allocator once their last uses on the device
// complete) and returns the object to its initial state.
void GCUGraph::abandon_capture() {
  allocator::release_pool(device_, mempool_);
  capture_stream_ = nullptr;
}

void GCUGraph::reset() {
  if (has_graph_) {
    (void)hipGraphDestroy(graph_);
    has_graph_ = false;
  }
  if (has_exec_) {
    (void)hipGraphExecDestroy(exec_);
    has_exec_ = false;
    allocator::release_pool(device_, mempool_);
  }
  capture_stream_ = nullptr;
}

allocator::MempoolId GCUGraph::pool() const {
  TORCH_CHECK(has_exec_ || capture_stream_ != nullptr,
              "Called GCUGraph::pool() without a preceding successful capture.");
  return mempool_;
}

void GCUGraph::enable_debug_mode() { debug_ = true; }

void GCUGraph::debug_dump(const std::string& path) {
  TORCH_CHECK(debug_ && has_graph_, "debug_dump needs enable_debug_mode() before capture");
  GCU_HIP_CHECK(hipGraphDebugDotPrint(graph_, path.c_str(), 0));
}

}  // namespace torch_gcu
