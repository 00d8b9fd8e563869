// Op-debug configuration and the dispatch-side helpers that use it.
//
// ENFLAME_PT_OP_DEBUG_CONFIG holds space-separated key=value pairs with the
// reference's keys and defaults (torch_gcu/csrc/aten/op_debug_config.cpp:25-118,
// op_debug_config.h:144-160):
//   fallback_cpu=<ops>            run these ops on CPU ATen
//   op_check=<ops>                run natively, then on CPU ATen, and compare
//   op_input_dump=<ops>           save the inputs of every call (dump_path)
//   op_output_dump=<ops>          save the outputs of every call (dump_path)
//   deregister=<ops>              do not register these ops' native kernels
//                                 (read once, when the library loads)
//   op_check_no_break=true        log a mismatch instead of raising
//   op_check_dump=true            save inputs, gcu and CPU outputs of a mismatch
//   op_check_tol_fp32=rtol,atol   default 1e-6,1e-6; op_check_tol_fp16 and
//   op_check_tol_bf16             default 1e-3,1e-3; "rtol," or ",atol" sets one
//   dump_path=<dir>               default ./torch_gcu_dump_file
//   op_sync_mode=true             synchronise the stream after each op
//   op_statistics=true            count calls per op and argument signature
//   op_statistics_dump=true       write the statistics as JSON at exit
//   op_calltrace=true             log each op with the Python stack calling it
//   test_mode=true                dump folders without the pid/time suffix
// <ops> is a comma-separated list of op names -- the C++ name ("add_out"),
// the ATen name with or without overload ("add.out", "add") -- plus
// "all_ops" (or the older "all") for every op and "-name" to exclude one.
#pragma once

#include <ATen/core/dispatch/Dispatcher.h>
#include <ATen/core/stack.h>

#include <atomic>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

namespace torch_gcu {

// A list of ops from the configuration (op_debug_config.h:18-28).
struct OpSelection {
  bool all = false;
  std::set<std::string> include;
  std::set<std::string> exclude;
  bool any() const { return all || !include.empty(); }
  // aten_name "add.out", cpp_name "add_out"
  bool enabled(const std::string& aten_name, const std::string& cpp_name) const;
  bool excluded(const std::string& aten_name, const std::string& cpp_name) const;
};

struct OpDebugConfig {
  OpSelection fallback_cpu, op_check, input_dump, output_dump, deregister;
  bool check_no_break = false;
  bool check_dump = false;
  double rtol_fp32 = 1e-6, atol_fp32 = 1e-6;
  double rtol_fp16 = 1e-3, atol_fp16 = 1e-3;
  double rtol_bf16 = 1e-3, atol_bf16 = 1e-3;
  std::string dump_path = "./torch_gcu_dump_file";
  bool op_sync_mode = false;
  bool statistics = false;
  bool statistics_dump = false;
  bool calltrace = false;
  bool test_mode = false;
  // folders of this process's dumps (set by parse from dump_path)
  std::string check_dump_dir, op_dump_dir;

  static OpDebugConfig& get();
  static OpDebugConfig parse(const std::string& s);
  bool any_debug() const;
};

// Replaces the process configuration (torch_gcu._C._set_op_debug_config).
void set_op_debug_config(const std::string& s);

// Python-scoped switches (the reference's OpDebugCtx, torch_gcu/gcu/debug.py:
// 73-118, over op_debug_config.h:50-78): inside the fallback scope every
// native op runs on CPU ATen, inside the op-check scope every native op is
// checked, inside the op-name scope each op's names are logged.
void set_scope(int which, bool on);  // 0 op name, 1 fallback, 2 op check
bool scope_state(int which);
bool any_scope();

// The native op wrappers' decisions for one call (generated RegisterGCU.cpp).
bool forced_fallback(const std::string& aten_name, const std::string& cpp_name);
bool checked(const std::string& aten_name, const std::string& cpp_name);
bool dump_inputs(const std::string& aten_name, const std::string& cpp_name);
bool dump_outputs(const std::string& aten_name, const std::string& cpp_name);
bool deregistered(const std::string& aten_name, const std::string& cpp_name);
// op-name scope log and calltrace for one call
void trace_call(const std::string& aten_name, const std::string& cpp_name);

// Statistics: per op, native and CPU-fallback calls and the calls per
// argument signature (shapes, strides, dtypes and scalar values).
void count_op(const std::string& op, bool fallback, const torch::jit::Stack* args = nullptr,
              const c10::FunctionSchema* schema = nullptr);
std::map<std::string, std::pair<int64_t, int64_t>> op_statistics();
void clear_op_statistics();
// Human-readable table (torch.gcu.debug.get_op_statistics_info) and the JSON
// file written under dump_path (op_stat_<pid>_<time>.json); returns its path.
std::string op_statistics_info();
std::string dump_op_statistics_json();

// op_check results per op (the reference logs "<op> acc check pass" for each
// compared call, gcu_op_check.cpp:180-196): outputs compared, outputs outside
// the tolerance, the largest |gcu - cpu| / (atol + rtol |cpu|) seen (0 for an
// exact comparison that passed) and the smallest root-mean-square of a CPU
// float output (so a caller can relate a fixed atol to the outputs' scale).
struct OpCheckStat {
  int64_t compared = 0, failed = 0;
  double max_ratio = 0.0;
  double min_ref_rms = -1.0;  // -1: no float output compared
};
std::map<std::string, OpCheckStat> op_check_statistics();
void clear_op_check_statistics();

// Saves the tensor and non-tensor arguments of a call under
// <dir>/<prefix>_args<i>.pt / .txt (tensors loadable with torch.load).
void dump_ivalues(const std::string& dir, const std::string& prefix,
                  const std::vector<c10::IValue>& values);
// op_input_dump / op_output_dump of one native call
void dump_call(const std::string& cpp_name, const char* what, const std::vector<c10::IValue>& v);

// Boxed CPU fallback (torch_gcu/csrc/aten/aten_cpu_fallback.cpp:342-411),
// with the retry in float for CPU kernels that lack Half (:193-340).
void gcu_cpu_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack);

// op_check: `stack` holds the op's arguments; runs the native kernel through
// the dispatcher, then the CPU kernel on host copies, and compares outputs
// (torch_gcu/csrc/aten/aot_ops/gcu_op_check.cpp:46-229).
void op_check_boxed(const c10::OperatorHandle& op, torch::jit::Stack* stack,
                    c10::DispatchKeySet native_ks, const std::string& cpp_name);

// Set by the Python module: formats the current Python stack (calltrace).
using PyStackFn = std::string (*)();
void set_python_stack_fn(PyStackFn fn);

// ---- fallback policy (codegen/gcu_op_fallback.yaml, mi355x column) -------
// The policy of one native op: "all" or argument rules "arg::value".
void register_fallback_policy(const std::string& aten_name, const std::vector<std::string>& rules);
std::map<std::string, std::vector<std::string>> fallback_policy();

}  // namespace torch_gcu
