// Helpers the generated wrappers (RegisterGCU.cpp) and the native kernels
// share: device checks, the device guard target, the op-debug switch and the
// bridge from at::Tensor to the kernel library's descriptor.
#pragma once

#include <ATen/ATen.h>
#include <c10/core/Device.h>

#include <initializer_list>
#include <optional>

#include "gcu_runtime.h"
#include "mi355x_ops.h"
#include "op_debug.h"

namespace torch_gcu {

inline bool is_gcu(const at::Tensor& t) { return t.defined() && t.device().type() == kGCU; }

// CPU 0-dim tensors are scalars and may accompany gcu tensors (the
// reference's RHS/LHS_IS_SCALAR rule, codegen/gen_backend_stubs.py:1061-1078).
inline void check_device(std::optional<at::Device>& common, const at::Tensor& t, const char* op,
                         const char* arg) {
  if (!t.defined()) return;
  if (t.device().is_cpu() && t.dim() == 0) return;
  if (!common.has_value()) {
    common = t.device();
    return;
  }
  TORCH_CHECK(*common == t.device(), "Expected all tensors to be on the same device, but found "
              "at least two devices, ", *common, " and ", t.device(), "! (when checking argument ",
              arg, " in method ", op, ")");
}

inline std::optional<at::Device> gcu_device_of(const at::Tensor& t) {
  if (is_gcu(t)) return t.device();
  return std::nullopt;
}

inline std::optional<at::Device> first_gcu_device(
    std::initializer_list<std::optional<at::Device>> ds) {
  for (const auto& d : ds)
    if (d.has_value()) return d;
  return std::nullopt;
}

// True when a tensor of the list has one of the dtypes (fallback policy rules
// on tensor-list arguments).
inline bool any_dtype_in(const at::ITensorListRef& l, std::initializer_list<at::ScalarType> dts) {
  for (const at::Tensor& t : l)
    for (at::ScalarType d : dts)
      if (t.defined() && t.scalar_type() == d) return true;
  return false;
}
inline bool any_dtype_in(at::TensorList l, std::initializer_list<at::ScalarType> dts) {
  for (const at::Tensor& t : l)
    for (at::ScalarType d : dts)
      if (t.defined() && t.scalar_type() == d) return true;
  return false;
}

bool op_debug_active();
bool in_op_check();
struct OpCheckScope {
  OpCheckScope();
  ~OpCheckScope();
};

// Per-op epilogue: op_sync_mode synchronisation.
void after_op();

// True when environment variable `name` reads "true" (case-insensitive,
// surrounding spaces ignored), the way the reference reads
// ENFLAME_PT_ENABLE_LINEAR_OVERRIDE (RegisterLinearOverrideGCU.cpp:575-583).
bool env_true(const char* name);

// ---- kernel-library bridge (replaces createTopsatenTensor and
// CHECK_TOPSATEN_CALL, torch_gcu/csrc/gcu/gcu_utils.cpp:64-108) -------------

mi_tensor_t desc(const at::Tensor& t);
mi_scalar_t scalar_of(const at::Scalar& s, bool wrapped = true);
// Value of a CPU 0-dim tensor as a kernel-library scalar.
mi_scalar_t scalar_of_tensor(const at::Tensor& t);
// Throws a c10::Error with the library's message when st != MI_OK.
void check_mi(mi_status_t st, const char* what);
hipStream_t stream_for(const at::Tensor& t);
inline mi_stream_t mi_stream(const at::Tensor& t) { return (mi_stream_t)stream_for(t); }

}  // namespace torch_gcu
