// Op-debug configuration and the dispatch-side helpers that use it.
//
// ENFLAME_PT_OP_DEBUG_CONFIG holds space-separated key=value pairs, as in the
// reference (torch_gcu/csrc/aten/op_debug_config.cpp:25-118):
//   fallback_cpu=<op>[,<op>...]|all_ops   run these ops on CPU ATen
//   op_check=<op>[,<op>...]|all_ops       run natively, then on CPU, compare
//   op_check_no_break=true                 warn instead of raising on mismatch
//   op_check_rtol_fp32=.. op_check_atol_fp32=..  (defaults 1e-6 / 1e-6)
//   op_check_rtol_half=.. op_check_atol_half=..  (defaults 1e-3 / 1e-3;
//                                          op_debug_config.h:144-149)
//   op_sync_mode=true                      synchronise the stream after each op
//   op_statistics=true                     count calls per op (native/fallback)
// Op names are ATen names with overload ("add.out") or without ("add").
#pragma once

#include <ATen/core/dispatch/Dispatcher.h>
#include <ATen/core/stack.h>

#include <atomic>
#include <map>
#include <mutex>
#include <set>
#include <string>

namespace torch_gcu {

struct OpDebugConfig {
  bool fallback_all = false;
  std::set<std::string> fallback_ops;
  bool check_all = false;
  std::set<std::string> check_ops;
  bool check_no_break = false;
  double rtol_fp32 = 1e-6, atol_fp32 = 1e-6;
  double rtol_half = 1e-3, atol_half = 1e-3;
  bool op_sync_mode = false;
  bool statistics = false;

  static OpDebugConfig& get();
  static OpDebugConfig parse(const std::string& s);
  bool forced_fallback(const std::string& op) const;
  bool checked(const std::string& op) const;
  bool any_debug() const {
    return fallback_all || !fallback_ops.empty() || check_all || !check_ops.empty() ||
           statistics;
  }
};

// Replaces the process configuration (used by torch_gcu._C._set_op_debug_config).
void set_op_debug_config(const std::string& s);

// Per-op call counters: name -> (native calls, CPU fallback calls).
void count_op(const std::string& op, bool fallback);
std::map<std::string, std::pair<int64_t, int64_t>> op_statistics();
void clear_op_statistics();

// Boxed CPU fallback (torch_gcu/csrc/aten/aten_cpu_fallback.cpp:342-411).
void gcu_cpu_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack);

// op_check: `stack` holds the op's arguments; runs the native kernel through
// the dispatcher, then the CPU kernel on host copies, and compares outputs
// (torch_gcu/csrc/aten/aot_ops/gcu_op_check.cpp:46-229).
void op_check_boxed(const c10::OperatorHandle& op, torch::jit::Stack* stack,
                    c10::DispatchKeySet native_ks);

}  // namespace torch_gcu
