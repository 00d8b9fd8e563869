#include "op_debug.h"

#include <ATen/ATen.h>
#include <ATen/native/CPUFallback.h>
#include <c10/util/Exception.h>
#include <torch/csrc/jit/serialization/pickle.h>
#include <torch/library.h>
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdlib>
#include <ctime>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <sstream>

#include "gcu_runtime.h"

namespace torch_gcu {

namespace {

std::mutex g_cfg_mu;

std::atomic<bool> g_scope[3] = {false, false, false};

std::atomic<PyStackFn> g_py_stack{nullptr};

std::string time_stamp(bool millis) {
  const auto now = std::chrono::system_clock::now();
  const std::time_t t = std::chrono::system_clock::to_time_t(now);
  std::tm tm{};
  localtime_r(&t, &tm);
  std::ostringstream os;
  os << std::put_time(&tm, millis ? "%Y%m%d%H%M%S" : "%Y%m%d_%H%M%S");
  if (millis) {
    const auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(
                        now.time_since_epoch()).count() % 1000;
    os << std::setw(3) << std::setfill('0') << ms;
  }
  return os.str();
}

std::string expand_home(const std::string& p) {
  if (!p.empty() && p[0] == '~') {
    const char* h = std::getenv("HOME");
    if (h) return std::string(h) + p.substr(1);
  }
  return p;
}

void parse_ops(const std::string& v, OpSelection& sel) {
  std::stringstream ss(v);
  std::string item;
  while (std::getline(ss, item, ',')) {
    if (item.empty()) continue;
    if (item == "all_ops" || item == "all") {
      if (item == "all") TORCH_WARN("ENFLAME_PT_OP_DEBUG_CONFIG: 'all' is deprecated, use all_ops");
      sel.all = true;
    } else if (item[0] == '-') {
      sel.exclude.insert(item.substr(1));
    } else {
      sel.include.insert(item);
    }
  }
}

bool parse_bool(const std::string& v, bool cur) {
  std::string l = v;
  for (auto& c : l) c = (char)std::tolower((unsigned char)c);
  if (l == "true" || l == "1") return true;
  if (l == "false" || l == "0") return false;
  return cur;
}

// "rtol,atol", "rtol," or ",atol" (op_debug_config.cpp:260-288)
void parse_tol(const std::string& key, const std::string& v, double& rtol, double& atol) {
  const auto comma = v.find(',');
  const std::string r = v.substr(0, comma);
  const std::string a = comma == std::string::npos ? std::string() : v.substr(comma + 1);
  try {
    if (!r.empty()) rtol = std::stod(r);
    if (!a.empty()) atol = std::stod(a);
  } catch (...) {
    TORCH_WARN("ENFLAME_PT_OP_DEBUG_CONFIG: ", key, " value '", v,
               "' is not rtol,atol; keeping rtol ", rtol, " atol ", atol);
  }
}

bool names_in(const std::set<std::string>& s, const std::string& aten_name,
              const std::string& cpp_name) {
  if (s.count(aten_name) || s.count(cpp_name)) return true;
  const auto dot = aten_name.find('.');
  return dot != std::string::npos && s.count(aten_name.substr(0, dot));
}

void log_line(const std::string& s) {
  std::cerr << s << std::flush;
}

}  // namespace

bool OpSelection::enabled(const std::string& aten_name, const std::string& cpp_name) const {
  return all || names_in(include, aten_name, cpp_name);
}
bool OpSelection::excluded(const std::string& aten_name, const std::string& cpp_name) const {
  return names_in(exclude, aten_name, cpp_name);
}

OpDebugConfig OpDebugConfig::parse(const std::string& s) {
  OpDebugConfig c;
  std::stringstream ss(s);
  std::string kv;
  while (ss >> kv) {
    const auto eq = kv.find('=');
    TORCH_CHECK(eq != std::string::npos, "ENFLAME_PT_OP_DEBUG_CONFIG: expected key=value, got '",
                kv, "'");
    const std::string k = kv.substr(0, eq), v = kv.substr(eq + 1);
    if (k == "fallback_cpu") parse_ops(v, c.fallback_cpu);
    else if (k == "op_check") parse_ops(v, c.op_check);
    else if (k == "op_input_dump") parse_ops(v, c.input_dump);
    else if (k == "op_output_dump") parse_ops(v, c.output_dump);
    else if (k == "deregister") parse_ops(v, c.deregister);
    else if (k == "op_check_no_break") c.check_no_break = parse_bool(v, c.check_no_break);
    else if (k == "op_check_dump") c.check_dump = parse_bool(v, c.check_dump);
    else if (k == "op_check_tol_fp32") parse_tol(k, v, c.rtol_fp32, c.atol_fp32);
    else if (k == "op_check_tol_fp16") parse_tol(k, v, c.rtol_fp16, c.atol_fp16);
    else if (k == "op_check_tol_bf16") parse_tol(k, v, c.rtol_bf16, c.atol_bf16);
    else if (k == "dump_path") c.dump_path = expand_home(v);
    else if (k == "op_sync_mode") c.op_sync_mode = parse_bool(v, c.op_sync_mode);
    else if (k == "op_statistics") c.statistics = parse_bool(v, c.statistics);
    else if (k == "op_statistics_dump") c.statistics_dump = parse_bool(v, c.statistics_dump);
    else if (k == "op_calltrace") c.calltrace = parse_bool(v, c.calltrace);
    else if (k == "test_mode") c.test_mode = parse_bool(v, c.test_mode);
    else TORCH_WARN("ENFLAME_PT_OP_DEBUG_CONFIG: ignoring unknown key '", k, "'");
  }
  // statistics are recorded whenever they are to be dumped
  if (c.statistics_dump) c.statistics = true;
  const std::string suffix =
      c.test_mode ? std::string() : "_" + std::to_string(getpid()) + "_" + time_stamp(false);
  c.check_dump_dir = c.dump_path + "/op_check_dump" + suffix;
  c.op_dump_dir = c.dump_path + "/op_dump" + suffix;
  return c;
}

bool OpDebugConfig::any_debug() const {
  return fallback_cpu.any() || op_check.any() || input_dump.any() || output_dump.any() ||
         statistics || calltrace;
}

// Read once from the environment; no lock on the per-op path (the flags are
// replaced wholesale by set_op_debug_config, a debugging call).
OpDebugConfig& OpDebugConfig::get() {
  static OpDebugConfig* cfg = [] {
    const char* e = std::getenv("ENFLAME_PT_OP_DEBUG_CONFIG");
    return new OpDebugConfig(parse(e ? e : ""));
  }();
  return *cfg;
}

void set_op_debug_config(const std::string& s) {
  OpDebugConfig next = OpDebugConfig::parse(s);
  OpDebugConfig& cur = OpDebugConfig::get();
  std::lock_guard<std::mutex> g(g_cfg_mu);
  cur = next;
}

void set_scope(int which, bool on) {
  TORCH_CHECK(which >= 0 && which < 3, "op-debug scope ", which, " does not exist");
  g_scope[which].store(on);
}
bool scope_state(int which) { return which >= 0 && which < 3 && g_scope[which].load(); }
bool any_scope() { return g_scope[0].load() || g_scope[1].load() || g_scope[2].load(); }

bool forced_fallback(const std::string& aten_name, const std::string& cpp_name) {
  const auto& c = OpDebugConfig::get().fallback_cpu;
  return (c.enabled(aten_name, cpp_name) || g_scope[1].load()) && !c.excluded(aten_name, cpp_name);
}
bool checked(const std::string& aten_name, const std::string& cpp_name) {
  const auto& c = OpDebugConfig::get().op_check;
  return (c.enabled(aten_name, cpp_name) || g_scope[2].load()) && !c.excluded(aten_name, cpp_name);
}
bool dump_inputs(const std::string& aten_name, const std::string& cpp_name) {
  const auto& c = OpDebugConfig::get().input_dump;
  return c.enabled(aten_name, cpp_name) && !c.excluded(aten_name, cpp_name);
}
bool dump_outputs(const std::string& aten_name, const std::string& cpp_name) {
  const auto& c = OpDebugConfig::get().output_dump;
  return c.enabled(aten_name, cpp_name) && !c.excluded(aten_name, cpp_name);
}
bool deregistered(const std::string& aten_name, const std::string& cpp_name) {
  const auto& c = OpDebugConfig::get().deregister;
  return c.enabled(aten_name, cpp_name) && !c.excluded(aten_name, cpp_name);
}

void set_python_stack_fn(PyStackFn fn) { g_py_stack.store(fn); }

void trace_call(const std::string& aten_name, const std::string& cpp_name) {
  if (g_scope[0].load()) {
    log_line("torch_gcu op name \"" + cpp_name + "\" (aten::" + aten_name +
             ") for fallback_cpu and op_check\n");
  }
  if (OpDebugConfig::get().calltrace) {
    const PyStackFn fn = g_py_stack.load();
    log_line("torch_gcu op calltrace: " + cpp_name + " (aten::" + aten_name + ")\n" +
             (fn ? fn() : std::string("  <no Python stack>\n")));
  }
}

// ---- statistics ---------------------------------------------------------------------

namespace {

struct OpStat {
  int64_t native = 0, fallback = 0;
  std::string schema;
  std::map<std::string, int64_t> params;  // argument signature -> calls
};
std::mutex g_stat_mu;
std::map<std::string, OpStat> g_stats;

std::string vec_str(at::IntArrayRef v) {
  std::ostringstream os;
  os << "[";
  for (size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << v[i];
  os << "]";
  return os.str();
}

std::string tensor_sig(const at::Tensor& t) {
  if (!t.defined()) return "Undefined Tensor";
  std::ostringstream os;
  os << "Tensor(shape" << vec_str(t.sizes()) << ", strides" << vec_str(t.strides()) << ", dtype["
     << t.scalar_type() << "], " << t.device() << ")";
  return os.str();
}

std::string ivalue_sig(const c10::IValue& v) {
  if (v.isTensor()) return tensor_sig(v.toTensor());
  if (v.isTensorList()) {
    std::string s = "[";
    const auto l = v.toTensorVector();
    for (size_t i = 0; i < l.size(); ++i) s += (i ? ", " : "") + tensor_sig(l[i]);
    return s + "]";
  }
  if (v.isOptionalTensorList()) {
    std::string s = "[";
    size_t i = 0;
    for (const auto& ot : v.toOptionalTensorList()) {
      const std::optional<at::Tensor> t = ot;
      s += (i++ ? ", " : "") + (t.has_value() ? tensor_sig(*t) : std::string("None"));
    }
    return s + "]";
  }
  if (v.isNone()) return "None";
  std::ostringstream os;
  os << v;
  return os.str();
}

std::string json_escape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += c;
    } else if (c == '\n') {
      o += "\\n";
    } else if ((unsigned char)c < 0x20) {
      char b[8];
      std::snprintf(b, sizeof(b), "\\u%04x", c);
      o += b;
    } else {
      o += c;
    }
  }
  return o;
}

}  // namespace

void count_op(const std::string& op, bool fallback, const torch::jit::Stack* args,
              const c10::FunctionSchema* schema) {
  std::string sig;
  if (args != nullptr) {
    for (size_t i = 0; i < args->size(); ++i) {
      if (i) sig += ", ";
      if (schema != nullptr && i < schema->arguments().size())
        sig += schema->arguments()[i].name() + "=";
      sig += ivalue_sig((*args)[i]);
    }
  }
  std::lock_guard<std::mutex> g(g_stat_mu);
  auto& e = g_stats[op];
  (fallback ? e.fallback : e.native)++;
  if (schema != nullptr && e.schema.empty()) {
    std::ostringstream os;
    os << *schema;
    e.schema = os.str();
  }
  if (args != nullptr) e.params[sig]++;
}

std::map<std::string, std::pair<int64_t, int64_t>> op_statistics() {
  std::lock_guard<std::mutex> g(g_stat_mu);
  std::map<std::string, std::pair<int64_t, int64_t>> out;
  for (const auto& kv : g_stats) out[kv.first] = {kv.second.native, kv.second.fallback};
  return out;
}

void clear_op_statistics() {
  std::lock_guard<std::mutex> g(g_stat_mu);
  g_stats.clear();
}

std::string op_statistics_info() {
  std::lock_guard<std::mutex> g(g_stat_mu);
  std::ostringstream os;
  os << std::left << std::setw(56) << "op" << std::setw(12) << "calls" << std::setw(12)
     << "native" << std::setw(12) << "fallback" << "signatures\n";
  for (const auto& kv : g_stats) {
    const OpStat& s = kv.second;
    os << std::setw(56) << kv.first << std::setw(12) << (s.native + s.fallback) << std::setw(12)
       << s.native << std::setw(12) << s.fallback << s.params.size() << "\n";
    for (const auto& p : s.params) os << "    " << p.second << " x (" << p.first << ")\n";
  }
  return os.str();
}

std::string dump_op_statistics_json() {
  const OpDebugConfig& c = OpDebugConfig::get();
  std::filesystem::create_directories(c.dump_path);
  const std::string file = c.dump_path + "/op_stat_" + std::to_string(getpid()) + "_" +
                           time_stamp(false) + ".json";
  std::lock_guard<std::mutex> g(g_stat_mu);
  std::ofstream f(file);
  TORCH_CHECK(f.good(), "op statistics: cannot write ", file);
  f << "[\n";
  size_t i = 0;
  for (const auto& kv : g_stats) {
    const OpStat& s = kv.second;
    f << (i++ ? ",\n" : "") << "  {\"aten_op_name\": \"" << json_escape(kv.first)
      << "\", \"schema\": \"" << json_escape(s.schema) << "\", \"use_count\": "
      << (s.native + s.fallback) << ", \"native_count\": " << s.native
      << ", \"fallback_count\": " << s.fallback << ", \"params_count\": " << s.params.size()
      << ", \"params\": [";
    size_t j = 0;
    for (const auto& p : s.params)
      f << (j++ ? ", " : "") << "{\"args\": \"" << json_escape(p.first) << "\", \"count\": "
        << p.second << "}";
    f << "]}";
  }
  f << "\n]\n";
  return file;
}

// ---- dumps -----------------------------------------------------------------------------

namespace {

void save_tensor(const std::string& base, const at::Tensor& t) {
  if (!t.defined()) {
    std::ofstream(base + ".txt") << "at::Tensor: \nundefined tensor\n";
    return;
  }
  const std::vector<char> bytes = torch::jit::pickle_save(c10::IValue(t.detach().cpu().contiguous()));
  std::ofstream f(base + ".pt", std::ios::binary);
  f.write(bytes.data(), (std::streamsize)bytes.size());
}

std::atomic<int64_t> g_dump_seq{0};
std::atomic<int64_t> g_check_err_idx{0};

}  // namespace

void dump_ivalues(const std::string& dir, const std::string& prefix,
                  const std::vector<c10::IValue>& values) {
  std::filesystem::create_directories(dir);
  for (size_t i = 0; i < values.size(); ++i) {
    const std::string base = dir + "/" + prefix + "_args" + std::to_string(i);
    const c10::IValue& v = values[i];
    if (v.isTensor()) {
      save_tensor(base, v.toTensor());
    } else if (v.isTensorList()) {
      const auto l = v.toTensorVector();
      for (size_t j = 0; j < l.size(); ++j) save_tensor(base + "_" + std::to_string(j), l[j]);
    } else if (v.isOptionalTensorList()) {
      size_t j = 0;
      for (const auto& ot : v.toOptionalTensorList()) {
        const std::optional<at::Tensor> t = ot;
        if (t.has_value()) save_tensor(base + "_" + std::to_string(j), *t);
        else std::ofstream(base + "_" + std::to_string(j) + ".txt") << "std::optional<at::Tensor>: nullopt\n";
        ++j;
      }
    } else if (v.isTuple()) {
      const auto& el = v.toTupleRef().elements();
      dump_ivalues(dir, prefix + "_args" + std::to_string(i), std::vector<c10::IValue>(el.begin(), el.end()));
    } else {
      std::ofstream(base + ".txt") << v.tagKind() << ": " << ivalue_sig(v) << "\n";
    }
  }
}

void dump_call(const std::string& cpp_name, const char* what, const std::vector<c10::IValue>& v) {
  const OpDebugConfig& c = OpDebugConfig::get();
  const std::string prefix = cpp_name + "_" + time_stamp(true) + "_" +
                             std::to_string(g_dump_seq.fetch_add(1)) + "_" + what;
  dump_ivalues(c.op_dump_dir, prefix, v);
}

// ---- boxed CPU fallback, with the float retry ---------------------------------------

namespace {

// ATen's message when a CPU kernel has no instance for a 16-bit float dtype.
bool missing_low_precision(const c10::Error& e, at::ScalarType* which) {
  const std::string m = e.what_without_backtrace();
  if (m.find("not implemented for 'Half'") != std::string::npos) {
    *which = at::kHalf;
    return true;
  }
  if (m.find("not implemented for 'BFloat16'") != std::string::npos) {
    *which = at::kBFloat16;
    return true;
  }
  return false;
}

// A tensor argument (or list element) of dtype `low` replaced by its float copy.
struct Widened {
  size_t arg;
  at::Tensor original;
  at::Tensor wide;
};

at::Tensor widen_one(const at::Tensor& t, at::ScalarType low, size_t arg,
                     std::vector<Widened>& out) {
  if (!t.defined() || t.scalar_type() != low) return t;
  at::Tensor w = t.to(at::kFloat);
  out.push_back({arg, t, w});
  return w;
}

std::vector<c10::IValue> widen_args(const std::vector<c10::IValue>& args, at::ScalarType low,
                                    std::vector<Widened>& out) {
  std::vector<c10::IValue> r = args;
  for (size_t i = 0; i < r.size(); ++i) {
    const c10::IValue& v = args[i];
    if (v.isTensor()) {
      r[i] = widen_one(v.toTensor(), low, i, out);
    } else if (v.isTensorList()) {
      std::vector<at::Tensor> l = v.toTensorVector();
      for (auto& t : l) t = widen_one(t, low, i, out);
      r[i] = c10::IValue(l);
    } else if (v.isOptionalTensorList()) {
      c10::List<std::optional<at::Tensor>> l;
      for (const auto& ot : v.toOptionalTensorList()) {
        std::optional<at::Tensor> t = ot;
        l.push_back(t.has_value() ? std::optional<at::Tensor>(widen_one(*t, low, i, out)) : t);
      }
      r[i] = c10::IValue(l);
    }
  }
  return r;
}

// dtypes of the op's tensor returns from its meta kernel, or empty if the op
// has none
std::vector<at::ScalarType> meta_return_dtypes(const c10::OperatorHandle& op,
                                               const std::vector<c10::IValue>& args) {
  auto to_meta = [](const at::Tensor& t) {
    return t.defined() ? at::empty_strided(t.sizes(), t.strides(), t.options().device(at::kMeta))
                       : t;
  };
  torch::jit::Stack ms;
  for (const auto& v : args) {
    if (v.isTensor()) {
      ms.push_back(to_meta(v.toTensor()));
    } else if (v.isTensorList()) {
      std::vector<at::Tensor> l = v.toTensorVector();
      for (auto& t : l) t = to_meta(t);
      ms.push_back(l);
    } else if (v.isOptionalTensorList()) {
      c10::List<std::optional<at::Tensor>> l;
      for (const auto& ot : v.toOptionalTensorList()) {
        std::optional<at::Tensor> t = ot;
        l.push_back(t.has_value() ? std::optional<at::Tensor>(to_meta(*t)) : t);
      }
      ms.push_back(l);
    } else if (v.isDevice()) {
      ms.push_back(c10::Device(at::kMeta));
    } else {
      ms.push_back(v);
    }
  }
  std::vector<at::ScalarType> out;
  try {
    op.redispatchBoxed(c10::DispatchKeySet(c10::DispatchKey::Meta), &ms);
  } catch (const std::exception&) {
    return out;
  }
  const size_t nr = op.schema().returns().size();
  for (size_t i = ms.size() - nr; i < ms.size(); ++i) {
    if (ms[i].isTensor()) out.push_back(ms[i].toTensor().scalar_type());
    else out.push_back(at::ScalarType::Undefined);
  }
  return out;
}

bool same_alias_set(const c10::AliasInfo* a, const c10::AliasInfo* b) {
  return a != nullptr && b != nullptr && a->beforeSets() == b->beforeSets();
}

// Runs `op` on CPU ATen with every `low` tensor widened to float
// (aten_cpu_fallback.cpp:193-340): mutated arguments get the result rounded
// back into their own dtype, returns that alias them are those arguments,
// and other returns take the dtype the op's meta kernel gives for the
// original arguments (float returns go back to `low` when there is none).
void fallback_widened(const c10::OperatorHandle& op, torch::jit::Stack* stack,
                      const std::vector<c10::IValue>& args, at::ScalarType low,
                      void (*run)(const c10::OperatorHandle&, torch::jit::Stack*)) {
  const auto& schema = op.schema();
  const std::vector<at::ScalarType> want = meta_return_dtypes(op, args);
  std::vector<Widened> wid;
  const std::vector<c10::IValue> wargs = widen_args(args, low, wid);
  for (const auto& v : wargs) stack->push_back(v);
  run(op, stack);
  for (const Widened& w : wid) {
    const c10::AliasInfo* ai = schema.arguments()[w.arg].alias_info();
    if (ai == nullptr || !ai->isWrite()) continue;
    at::Tensor o = w.original;
    if (o.sizes() != w.wide.sizes()) o.resize_(w.wide.sizes());
    o.copy_(w.wide);
  }
  const size_t nr = schema.returns().size();
  for (size_t k = 0; k < nr; ++k) {
    c10::IValue& r = (*stack)[stack->size() - nr + k];
    const c10::AliasInfo* rai = schema.returns()[k].alias_info();
    bool replaced = false;
    if (rai != nullptr) {
      for (const Widened& w : wid) {
        if (same_alias_set(rai, schema.arguments()[w.arg].alias_info())) {
          r = w.original;
          replaced = true;
          break;
        }
      }
    }
    if (replaced || !r.isTensor()) continue;
    const at::Tensor t = r.toTensor();
    if (!t.defined()) continue;
    const at::ScalarType dt =
        k < want.size() && want[k] != at::ScalarType::Undefined
            ? want[k]
            : (t.scalar_type() == at::kFloat ? low : t.scalar_type());
    if (t.scalar_type() != dt) r = t.to(dt);
  }
}

void run_cpu_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  at::native::cpu_fallback(op, stack);
}

void run_cpu_kernel(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  op.redispatchBoxed(c10::DispatchKeySet(c10::DispatchKey::CPU), stack);
}

std::mutex g_warned_mu;
std::set<std::string> g_warned;

void warn_widened(const std::string& where, const std::string& op, at::ScalarType low) {
  {
    std::lock_guard<std::mutex> g(g_warned_mu);
    if (!g_warned.insert(where + op + c10::toString(low)).second) return;
  }
  TORCH_WARN(where, ": ", op, " not support ", low, ", convert ", low, " tensor to Float.");
}

// Runs `run` on the stack's arguments; a CPU kernel without the 16-bit
// dtype is retried in float.
void run_with_widening(const c10::OperatorHandle& op, torch::jit::Stack* stack, const char* where,
                       void (*run)(const c10::OperatorHandle&, torch::jit::Stack*)) {
  const size_t n = op.schema().arguments().size();
  const size_t base = stack->size() - n;
  const std::vector<c10::IValue> args(stack->begin() + base, stack->end());
  try {
    run(op, stack);
  } catch (const c10::Error& e) {
    at::ScalarType low;
    if (!missing_low_precision(e, &low)) throw;
    warn_widened(where, c10::toString(op.operator_name()), low);
    stack->resize(base);
    fallback_widened(op, stack, args, low, run);
  }
}

}  // namespace

void gcu_cpu_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  const auto& name = op.operator_name();
  if (OpDebugConfig::get().statistics) {
    std::string n = name.name.substr(name.name.find("::") == std::string::npos
                                          ? 0 : name.name.find("::") + 2);
    if (!name.overload_name.empty()) n += "." + name.overload_name;
    const size_t na = op.schema().arguments().size();
    const torch::jit::Stack args(stack->end() - na, stack->end());
    count_op(n, true, &args, &op.schema());
  }
  const auto s = current_hip_stream();
  TORCH_CHECK(!stream_is_capturing(s), "gcu: ", c10::toString(name),
              " has no native gcu kernel and runs on the CPU; a CPU fallback cannot be "
              "captured in a GCUGraph");
  // The generic ATen fallback moves tensor arguments to the CPU, runs the
  // CPU kernel and copies mutated / returned tensors back to the device.
  run_with_widening(op, stack, "cpu_fallback", &run_cpu_fallback);
}

// ---- op_check ---------------------------------------------------------------------

namespace {

// The lower of two float dtypes for the comparison (gcu_op_check.cpp:46-76).
at::ScalarType lower_float(at::ScalarType a, at::ScalarType b) {
  auto rank = [](at::ScalarType t) {
    switch (t) {
      case at::kBFloat16: return 0;
      case at::kHalf: return 1;
      case at::kFloat: return 2;
      case at::kDouble: return 3;
      default: return 4;
    }
  };
  return rank(a) <= rank(b) ? a : b;
}

std::mutex g_check_mu;
std::map<std::string, OpCheckStat> g_check_stats;

void record_check(const std::string& op, bool ok, double ratio, double ref_rms) {
  std::lock_guard<std::mutex> g(g_check_mu);
  OpCheckStat& e = g_check_stats[op];
  ++e.compared;
  if (!ok) ++e.failed;
  if (ratio > e.max_ratio) e.max_ratio = ratio;
  if (ref_rms >= 0.0 && (e.min_ref_rms < 0.0 || ref_rms < e.min_ref_rms)) e.min_ref_rms = ref_rms;
}

// *ratio: max |a - b| / (atol + rtol |b|) over elements both finite (float
// outputs), 0 or +inf for exact comparisons; *ref_rms: rms of b's finite
// elements for float outputs, -1 otherwise.
bool close_enough(const at::Tensor& dev, const at::Tensor& cpu, const OpDebugConfig& c,
                  std::string* why, double* ratio, double* ref_rms) {
  *ratio = 0.0;
  *ref_rms = -1.0;
  at::Tensor a = dev.detach().cpu();
  at::Tensor b = cpu.detach();
  if (a.sizes() != b.sizes()) {
    *why = "shape mismatch: gcu " + vec_str(a.sizes()) + " cpu " + vec_str(b.sizes());
    return false;
  }
  at::ScalarType dt = a.scalar_type();
  if (a.scalar_type() != b.scalar_type()) {
    if (a.is_floating_point() && b.is_floating_point()) dt = lower_float(a.scalar_type(), b.scalar_type());
    b = b.to(a.scalar_type());
  }
  at::Tensor ok;
  double rtol = c.rtol_fp32, atol = c.atol_fp32;
  bool equal_nan = true;
  if (!a.is_floating_point() && !a.is_complex()) {
    ok = a.eq(b);
    if (!ok.all().item<bool>()) *ratio = INFINITY;
  } else {
    if (dt == at::kHalf) {
      rtol = c.rtol_fp16;
      atol = c.atol_fp16;
    } else if (dt == at::kBFloat16) {
      rtol = c.rtol_bf16;
      atol = c.atol_bf16;
    } else if (dt != at::kFloat && dt != at::kDouble) {
      equal_nan = false;
    }
    ok = at::isclose(a.to(a.is_complex() ? a.scalar_type() : at::kDouble),
                     b.to(a.is_complex() ? a.scalar_type() : at::kDouble), rtol, atol, equal_nan);
    if (!a.is_complex() && a.numel() > 0) {
      const at::Tensor ad = a.to(at::kDouble), bd = b.to(at::kDouble);
      const at::Tensor fin = at::isfinite(ad).logical_and(at::isfinite(bd));
      if (fin.any().item<bool>()) {
        const at::Tensor af = ad.masked_select(fin), bf = bd.masked_select(fin);
        *ratio = ((af - bf).abs() / (bf.abs() * rtol + atol).clamp_min(1e-300)).max().item<double>();
        *ref_rms = bf.pow(2).mean().sqrt().item<double>();
      }
    }
  }
  if (ok.all().item<bool>()) return true;
  // the first mismatching elements, as the reference lists them
  const at::Tensor bad = ok.logical_not().reshape(-1).nonzero().reshape(-1);
  const at::Tensor af = a.reshape(-1), bf = b.reshape(-1);
  std::ostringstream os;
  os << bad.numel() << " of " << a.numel() << " elements outside rtol " << rtol << " atol "
     << atol << "; gcu(A) / cpu(B) / |A-B|:";
  const int64_t show = std::min<int64_t>(bad.numel(), 8);
  for (int64_t i = 0; i < show; ++i) {
    const int64_t j = bad[i].item<int64_t>();
    const c10::Scalar x = af[j].item(), y = bf[j].item();
    os << "\n  [" << j << "] " << x << " / " << y;
    if (!a.is_complex()) os << " / " << std::abs(x.toDouble() - y.toDouble());
  }
  *why = os.str();
  return false;
}

c10::IValue to_cpu_copy(const c10::IValue& v) {
  if (v.isTensor()) {
    const at::Tensor& t = v.toTensor();
    if (!t.defined()) return v;
    return c10::IValue(t.device().is_cpu() ? t.clone() : t.cpu());
  }
  if (v.isTensorList()) {
    std::vector<at::Tensor> out;
    for (const at::Tensor& t : v.toTensorVector()) out.push_back(t.defined() ? t.cpu().clone() : t);
    return c10::IValue(out);
  }
  if (v.isOptionalTensorList()) {
    c10::List<std::optional<at::Tensor>> out;
    for (const auto& ot : v.toOptionalTensorList()) {
      std::optional<at::Tensor> t = ot;
      out.push_back(t && t->defined() ? std::optional<at::Tensor>(t->cpu().clone()) : t);
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
                    c10::DispatchKeySet native_ks, const std::string& cpp_name) {
  const auto& cfg = OpDebugConfig::get();
  const auto& schema = op.schema();
  const size_t nargs = schema.arguments().size();
  // CPU copies of every argument before the native kernel mutates any
  torch::jit::Stack cpu_stack;
  for (size_t i = stack->size() - nargs; i < stack->size(); ++i)
    cpu_stack.push_back(to_cpu_copy((*stack)[i]));
  std::vector<c10::IValue> inputs;
  if (cfg.check_dump)
    for (const auto& v : cpu_stack) inputs.push_back(to_cpu_copy(v));
  op.redispatchBoxed(native_ks, stack);
  // the CPU kernel, retried in float where it lacks the 16-bit dtype
  // (gcu_op_check.cpp:202-229)
  run_with_widening(op, &cpu_stack, "cpu_check", &run_cpu_kernel);
  std::vector<at::Tensor> dev_out, cpu_out;
  for (size_t i = stack->size() - schema.returns().size(); i < stack->size(); ++i)
    collect_tensors((*stack)[i], dev_out);
  for (const auto& v : cpu_stack) collect_tensors(v, cpu_out);
  TORCH_CHECK(dev_out.size() == cpu_out.size(), "op_check: output count mismatch for ",
              schema.name());
  for (size_t i = 0; i < dev_out.size(); ++i) {
    if (!dev_out[i].defined() && !cpu_out[i].defined()) continue;
    std::string why;
    bool ok;
    double ratio = INFINITY, ref_rms = -1.0;
    if (!dev_out[i].defined() || !cpu_out[i].defined()) {
      ok = false;
      why = "one of the gcu and cpu outputs is undefined";
    } else {
      ok = close_enough(dev_out[i], cpu_out[i], cfg, &why, &ratio, &ref_rms);
    }
    record_check(cpp_name, ok, ratio, ref_rms);
    if (ok) continue;
    const int64_t err = g_check_err_idx.fetch_add(1);
    std::ostringstream os;
    os << "op_check failed for " << c10::toString(op.operator_name()) << " (op_id " << err
       << ") output " << i << ": " << why;
    if (cfg.check_dump) {
      const std::string prefix = cpp_name + "_" + std::to_string(err) + "_";
      dump_ivalues(cfg.check_dump_dir, prefix + "input", inputs);
      std::vector<c10::IValue> g(dev_out.begin(), dev_out.end()), c(cpu_out.begin(), cpu_out.end());
      dump_ivalues(cfg.check_dump_dir, prefix + "gcu_output", g);
      dump_ivalues(cfg.check_dump_dir, prefix + "cpu_output", c);
      os << "\n  inputs and outputs saved under " << cfg.check_dump_dir << "/" << prefix << "*";
    }
    if (cfg.check_no_break) {
      log_line(os.str() + "\n");
    } else {
      TORCH_CHECK(false, os.str());
    }
    break;
  }
}

std::map<std::string, OpCheckStat> op_check_statistics() {
  std::lock_guard<std::mutex> g(g_check_mu);
  return g_check_stats;
}

void clear_op_check_statistics() {
  std::lock_guard<std::mutex> g(g_check_mu);
  g_check_stats.clear();
}

// ---- fallback policy -----------------------------------------------------------------

namespace {
std::mutex g_policy_mu;
std::map<std::string, std::vector<std::string>>& policy_map() {
  static std::map<std::string, std::vector<std::string>> m;
  return m;
}
}  // namespace

void register_fallback_policy(const std::string& aten_name, const std::vector<std::string>& rules) {
  std::lock_guard<std::mutex> g(g_policy_mu);
  policy_map()[aten_name] = rules;
}

std::map<std::string, std::vector<std::string>> fallback_policy() {
  std::lock_guard<std::mutex> g(g_policy_mu);
  return policy_map();
}

}  // namespace torch_gcu

// Every aten op without a native gcu kernel runs on CPU ATen, the reference's
// fallback path (torch_gcu/csrc/aten/aten_cpu_fallback.cpp:448-451).
TORCH_LIBRARY_IMPL(_, PrivateUse1, m) {
  m.fallback(torch::CppFunction::makeFromBoxedFunction<&torch_gcu::gcu_cpu_fallback>());
}
