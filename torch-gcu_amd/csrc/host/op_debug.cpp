#include "op_debug.h"

#include <ATen/ATen.h>
#include <ATen/native/CPUFallback.h>
#include <c10/util/Exception.h>
#include <torch/library.h>

#include <cstdlib>
#include <sstream>

#include "gcu_runtime.h"

namespace torch_gcu {

namespace {
std::mutex g_cfg_mu;
OpDebugConfig* g_cfg = nullptr;

std::mutex g_stat_mu;
std::map<std::string, std::pair<int64_t, int64_t>> g_stats;

std::set<std::string> split_ops(const std::string& v) {
  std::set<std::string> out;
  std::stringstream ss(v);
  std::string item;
  while (std::getline(ss, item, ','))
    if (!item.empty()) out.insert(item);
  return out;
}

bool truthy(const std::string& v) { return v == "true" || v == "True" || v == "1"; }

bool in_set(const std::set<std::string>& s, const std::string& op) {
  if (s.count(op)) return true;
  const auto dot = op.find('.');
  return dot != std::string::npos && s.count(op.substr(0, dot));
}
}  // namespace

OpDebugConfig OpDebugConfig::parse(const std::string& s) {
  OpDebugConfig c;
  std::stringstream ss(s);
  std::string kv;
  while (ss >> kv) {
    const auto eq = kv.find('=');
    TORCH_CHECK(eq != std::string::npos, "ENFLAME_PT_OP_DEBUG_CONFIG: expected key=value, got '",
                kv, "'");
    const std::string k = kv.substr(0, eq), v = kv.substr(eq + 1);
    if (k == "fallback_cpu") {
      if (v == "all_ops") c.fallback_all = true;
      else c.fallback_ops = split_ops(v);
    } else if (k == "op_check") {
      if (v == "all_ops") c.check_all = true;
      else c.check_ops = split_ops(v);
    } else if (k == "op_check_no_break") {
      c.check_no_break = truthy(v);
    } else if (k == "op_check_rtol_fp32") {
      c.rtol_fp32 = std::stod(v);
    } else if (k == "op_check_atol_fp32") {
      c.atol_fp32 = std::stod(v);
    } else if (k == "op_check_rtol_half") {
      c.rtol_half = std::stod(v);
    } else if (k == "op_check_atol_half") {
      c.atol_half = std::stod(v);
    } else if (k == "op_sync_mode") {
      c.op_sync_mode = truthy(v);
    } else if (k == "op_statistics") {
      c.statistics = truthy(v);
    } else {
      TORCH_WARN("ENFLAME_PT_OP_DEBUG_CONFIG: ignoring unknown key '", k, "'");
    }
  }
  return c;
}

OpDebugConfig& OpDebugConfig::get() {
  std::lock_guard<std::mutex> g(g_cfg_mu);
  if (!g_cfg) {
    const char* e = std::getenv("ENFLAME_PT_OP_DEBUG_CONFIG");
    g_cfg = new OpDebugConfig(parse(e ? e : ""));
  }
  return *g_cfg;
}

void set_op_debug_config(const std::string& s) {
  OpDebugConfig next = OpDebugConfig::parse(s);
  OpDebugConfig& cur = OpDebugConfig::get();
  std::lock_guard<std::mutex> g(g_cfg_mu);
  cur = next;
}

bool OpDebugConfig::forced_fallback(const std::string& op) const {
  return fallback_all || in_set(fallback_ops, op);
}
bool OpDebugConfig::checked(const std::string& op) const {
  return check_all || in_set(check_ops, op);
}

void count_op(const std::string& op, bool fallback) {
  std::lock_guard<std::mutex> g(g_stat_mu);
  auto& e = g_stats[op];
  (fallback ? e.second : e.first)++;
}

std::map<std::string, std::pair<int64_t, int64_t>> op_statistics() {
  std::lock_guard<std::mutex> g(g_stat_mu);
  return g_stats;
}

void clear_op_statistics() {
  std::lock_guard<std::mutex> g(g_stat_mu);
  g_stats.clear();
}

// ---- boxed CPU fallback ---------------------------------------------------------

void gcu_cpu_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  const auto& name = op.operator_name();
  if (OpDebugConfig::get().statistics) {
    std::string n = name.name.substr(6);  // drop "aten::"
    if (!name.overload_name.empty()) n += "." + name.overload_name;
    count_op(n, true);
  }
  const auto s = current_hip_stream();
  TORCH_CHECK(!stream_is_capturing(s), "gcu: ", c10::toString(name),
              " has no native gcu kernel and runs on the CPU; a CPU fallback cannot be "
              "captured in a GCUGraph");
  // The generic ATen fallback moves tensor arguments to the CPU, runs the
  // CPU kernel and copies mutated / returned tensors back to the device.
  at::native::cpu_fallback(op, stack);
}

// ---- op_check ---------------------------------------------------------------------

namespace {

bool close_enough(const at::Tensor& dev, const at::Tensor& cpu, const OpDebugConfig& c,
                  std::string* why) {
  at::Tensor a = dev.cpu();
  at::Tensor b = cpu;
  if (a.sizes() != b.sizes()) {
    *why = "shape mismatch";
    return false;
  }
  if (a.scalar_type() != b.scalar_type()) b = b.to(a.scalar_type());
  if (!a.is_floating_point()) {
    const bool eq = a.equal(b);
    if (!eq) *why = "integer values differ";
    return eq;
  }
  const bool half = a.scalar_type() == at::kHalf || a.scalar_type() == at::kBFloat16;
  const double rtol = half ? c.rtol_half : c.rtol_fp32, atol = half ? c.atol_half : c.atol_fp32;
  at::Tensor af = a.to(at::kDouble), bf = b.to(at::kDouble);
  const bool ok = at::isclose(af, bf, rtol, atol, /*equal_nan=*/true).all().item<bool>();
  if (!ok) {
    const double maxd = (af - bf).abs().nan_to_num(0).max().item<double>();
    std::ostringstream os;
    os << "max |diff| " << maxd << " above rtol " << rtol << " atol " << atol;
    *why = os.str();
  }
  return ok;
}

c10::IValue to_cpu_copy(const c10::IValue& v) {
  if (v.isTensor()) {
    const at::Tensor& t = v.toTensor();
    if (!t.defined()) return v;
    return c10::IValue(t.device().is_cpu() ? t.clone() : t.cpu());
  }
  if (v.isTensorList()) {
    std::vector<at::Tensor> out;
    for (const at::Tensor& t : v.toTensorVector()) out.push_back(t.defined() ? t.cpu() : t);
    return c10::IValue(out);
  }
  if (v.isOptionalTensorList()) {
    c10::List<std::optional<at::Tensor>> out;
    for (const auto& ot : v.toOptionalTensorList()) {
      std::optional<at::Tensor> t = ot;
      out.push_back(t && t->defined() ? std::optional<at::Tensor>(t->cpu()) : t);
    }
    return c10::IValue(out);
  }
  if (v.isDevice()) {
    return c10::IValue(c10::Device(c10::kCPU));
  }
  return v;
}

void collect_tensors(const c10::IValue& v, std::vector<at::Tensor>& out) {
  if (v.isTensor()) out.push_back(v.toTensor());
  else if (v.isTensorList())
    for (const auto& t : v.toTensorVector()) out.push_back(t);
  else if (v.isTuple())
    for (const auto& e : v.toTupleRef().elements()) collect_tensors(e, out);
}

}  // namespace

void op_check_boxed(const c10::OperatorHandle& op, torch::jit::Stack* stack,
                    c10::DispatchKeySet native_ks) {
  const auto& cfg = OpDebugConfig::get();
  const auto& schema = op.schema();
  const size_t nargs = schema.arguments().size();
  // CPU copies of every argument before the native kernel mutates any
  torch::jit::Stack cpu_stack;
  for (size_t i = stack->size() - nargs; i < stack->size(); ++i)
    cpu_stack.push_back(to_cpu_copy((*stack)[i]));
  op.redispatchBoxed(native_ks, stack);
  op.redispatchBoxed(c10::DispatchKeySet(c10::DispatchKey::CPU), &cpu_stack);
  std::vector<at::Tensor> dev_out, cpu_out;
  for (size_t i = stack->size() - schema.returns().size(); i < stack->size(); ++i)
    collect_tensors((*stack)[i], dev_out);
  for (const auto& v : cpu_stack) collect_tensors(v, cpu_out);
  TORCH_CHECK(dev_out.size() == cpu_out.size(), "op_check: output count mismatch for ",
              schema.name());
  for (size_t i = 0; i < dev_out.size(); ++i) {
    if (!dev_out[i].defined()) continue;
    std::string why;
    if (!close_enough(dev_out[i], cpu_out[i], cfg, &why)) {
      std::ostringstream os;
      os << "op_check failed for " << c10::toString(op.operator_name()) << " output " << i
         << ": " << why;
      if (cfg.check_no_break) {
        TORCH_WARN(os.str());
      } else {
        TORCH_CHECK(false, os.str());
      }
    }
  }
}

}  // namespace torch_gcu

// Every aten op without a native gcu kernel runs on CPU ATen, the reference's
// fallback path (torch_gcu/csrc/aten/aten_cpu_fallback.cpp:448-451).
TORCH_LIBRARY_IMPL(_, PrivateUse1, m) {
  m.fallback(torch::CppFunction::makeFromBoxedFunction<&torch_gcu::gcu_cpu_fallback>());
}
