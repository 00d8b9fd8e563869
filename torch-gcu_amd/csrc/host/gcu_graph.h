// GCUGraph: stream capture into a hipGraph with a private allocator pool.
//
// Same API as the reference (torch_gcu/csrc/gcu/gcu_graph.h:24-117):
// capture_begin(pool, mode) on a non-default stream, capture_end()
// instantiates, replay() launches on the current stream, reset() frees the
// executable and releases the pool, pool() returns the mempool id so later
// captures can share it.
#pragma once

#include <hip/hip_runtime_api.h>

#include <string>

#include "gcu_caching_allocator.h"

namespace torch_gcu {

class GCUGraph {
 public:
  GCUGraph();
  ~GCUGraph();

  void capture_begin(allocator::MempoolId pool = {0, 0},
                     hipStreamCaptureMode mode = hipStreamCaptureModeGlobal);
  void capture_end();
  void replay();
  void reset();
  allocator::MempoolId pool() const;
  void enable_debug_mode();
  void debug_dump(const std::string& path);
  int64_t num_nodes() const { return num_nodes_; }

 private:
  void abandon_capture();

  hipGraph_t graph_ = nullptr;
  hipGraphExec_t exec_ = nullptr;
  bool has_graph_ = false;
  bool has_exec_ = false;
  bool debug_ = false;
  int device_ = -1;
  hipStream_t capture_stream_ = nullptr;
  allocator::MempoolId mempool_{0, 0};
  uint64_t id_ = 0;
  int64_t num_nodes_ = 0;
};

}  // namespace torch_gcu
