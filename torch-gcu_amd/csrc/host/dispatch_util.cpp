#include "dispatch_util.h"

#include <c10/util/Exception.h>

#include <cctype>
#include <cstdlib>
#include <string>

namespace torch_gcu {

namespace {
thread_local int tls_op_check_depth = 0;
}

bool op_debug_active() {
  static const OpDebugConfig& c = OpDebugConfig::get();
  return c.any_debug() || any_scope();
}

bool in_op_check() { return tls_op_check_depth > 0; }
OpCheckScope::OpCheckScope() { ++tls_op_check_depth; }
OpCheckScope::~OpCheckScope() { --tls_op_check_depth; }

void after_op() {
  if (C10_UNLIKELY(OpDebugConfig::get().op_sync_mode)) maybe_sync_after_op(current_hip_stream());
}

bool env_true(const char* name) {
  const char* e = std::getenv(name);
  if (e == nullptr) return false;
  std::string v(e);
  const auto b = v.find_first_not_of(' '), en = v.find_last_not_of(' ');
  v = b == std::string::npos ? std::string() : v.substr(b, en - b + 1);
  for (auto& c : v) c = (char)std::tolower((unsigned char)c);
  return v == "true";
}

mi_tensor_t desc(const at::Tensor& t) {
  mi_tensor_t d{};
  if (!t.defined()) return d;
  TORCH_CHECK(t.dim() <= MI_MAX_DIMS, "gcu kernels take at most ", MI_MAX_DIMS,
              " dims, got a tensor of rank ", t.dim());
  d.data = t.numel() > 0 ? t.data_ptr() : nullptr;
  d.dtype = (int32_t)t.scalar_type();
  d.ndim = (int32_t)t.dim();
  for (int64_t i = 0; i < t.dim(); ++i) {
    d.sizes[i] = t.size(i);
    d.strides[i] = t.stride(i);
  }
  return d;
}

mi_scalar_t scalar_of(const at::Scalar& s, bool wrapped) {
  mi_scalar_t r{};
  r.wrapped = wrapped ? 1 : 0;
  if (s.isBoolean()) {
    r.dtype = MI_BOOL;
    r.i = s.toBool() ? 1 : 0;
  } else if (s.isIntegral(false)) {
    r.dtype = MI_I64;
    r.i = s.toLong();
  } else if (s.isFloatingPoint()) {
    r.dtype = MI_F64;
    r.f = s.toDouble();
  } else {
    TORCH_CHECK(false, "gcu: complex scalars are not supported by the native kernels");
  }
  return r;
}

mi_scalar_t scalar_of_tensor(const at::Tensor& t) {
  TORCH_INTERNAL_ASSERT(t.device().is_cpu() && t.dim() == 0);
  mi_scalar_t r = scalar_of(t.item(), t.unsafeGetTensorImpl()->is_wrapped_number());
  if (!r.wrapped) r.dtype = (int32_t)t.scalar_type();  // a 0-dim tensor keeps its dtype
  if (r.dtype == MI_F32 || r.dtype == MI_F16 || r.dtype == MI_BF16) r.f = t.item<double>();
  return r;
}

void check_mi(mi_status_t st, const char* what) {
  if (st == MI_OK) return;
  TORCH_CHECK(false, "gcu kernel ", what, " failed (status ", (int)st, "): ", mi_last_error());
}

hipStream_t stream_for(const at::Tensor& t) {
  return current_hip_stream(t.device().index());
}

}  // namespace torch_gcu
