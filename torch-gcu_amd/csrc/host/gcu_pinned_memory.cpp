// Pinned CPU tensors for the "gcu" device (the reference's
// torch_gcu/csrc/aten/aot_ops/gcu_pinned_memory.cpp:29-190).
//
// In a ROCm build of PyTorch, CPU factories with pin_memory=True ask the CUDA
// hooks first, which pin through PyTorch's own HIP runtime; this library runs
// on its own copy of the runtime, which does not know those pointers.  So, as
// the reference does, the CPU kernels of empty.memory_format / empty_strided
// are replaced by ones that take pinned memory from the gcu caching host
// allocator (and are ATen's own otherwise), and is_pinned / _pin_memory are
// answered at BackendSelect from the gcu hooks' allocator and pointer query.
#include <ATen/EmptyTensor.h>
#include <ATen/core/TensorBody.h>
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <ATen/native/TensorFactories.h>
#include <ATen/ops/empty_native.h>
#include <ATen/ops/empty_strided_native.h>
#include <c10/core/Storage.h>
#include <c10/util/Exception.h>
#include <torch/library.h>

#include "gcu_caching_host_allocator.h"

namespace torch_gcu {
namespace {

constexpr c10::DispatchKeySet kCPUKeys{c10::DispatchKey::CPU};

void check_strided(std::optional<at::Layout> layout) {
  TORCH_CHECK(!layout.has_value() || *layout == at::kStrided,
              "pinned memory is only supported for strided CPU tensors, got layout ", *layout);
}

at::Tensor empty_memory_format_cpu(at::IntArrayRef size, std::optional<at::ScalarType> dtype,
                                   std::optional<at::Layout> layout,
                                   std::optional<at::Device> device, std::optional<bool> pin_memory,
                                   std::optional<at::MemoryFormat> memory_format) {
  if (!pin_memory.value_or(false))
    return at::native::empty_cpu(size, dtype, layout, device, pin_memory, memory_format);
  check_strided(layout);
  const auto dt = dtype.value_or(c10::get_default_dtype_as_scalartype());
  return at::detail::empty_generic(size, host_allocator::get(), kCPUKeys, dt, memory_format);
}

at::Tensor empty_strided_cpu(at::IntArrayRef size, at::IntArrayRef stride,
                             std::optional<at::ScalarType> dtype, std::optional<at::Layout> layout,
                             std::optional<at::Device> device, std::optional<bool> pin_memory) {
  if (!pin_memory.value_or(false))
    return at::native::empty_strided_cpu(size, stride, dtype, layout, device, pin_memory);
  check_strided(layout);
  const auto dt = dtype.value_or(c10::get_default_dtype_as_scalartype());
  return at::detail::empty_strided_generic(size, stride, host_allocator::get(), kCPUKeys, dt);
}

bool is_pinned(const at::Tensor& self, std::optional<at::Device>) {
  if (!self.is_cpu() || !self.has_storage() || self.storage().data() == nullptr) return false;
  return at::detail::getPrivateUse1Hooks().isPinnedPtr(self.storage().data());
}

at::Tensor pin_memory_copy(const at::Tensor& self, std::optional<at::Device>) {
  TORCH_CHECK(self.device().is_cpu(), "cannot pin '", self.toString(),
              "' only dense CPU tensors can be pinned");
  const size_t nbytes =
      at::detail::computeStorageNbytes(self.sizes(), self.strides(), self.dtype().itemsize());
  c10::Storage storage(c10::Storage::use_byte_size_t(), nbytes, host_allocator::get(),
                       /*resizable=*/false);
  at::Tensor t = at::empty({0}, self.options()).set_(storage, 0, self.sizes(), self.strides());
  t.copy_(self);
  return t;
}

// Replacing ATen's CPU factory kernels makes the dispatcher warn once per
// kernel at load; that warning is expected here and kept off stderr.
struct Quiet final : c10::WarningHandler {
  void process(const c10::Warning&) override {}
};
Quiet g_quiet;
c10::WarningHandler* const g_prev_handler = [] {
  c10::WarningHandler* prev = c10::WarningUtils::get_warning_handler();
  c10::WarningUtils::set_warning_handler(&g_quiet);
  return prev;
}();

TORCH_LIBRARY_IMPL(aten, CPU, m) {
  m.impl("empty.memory_format", TORCH_FN(empty_memory_format_cpu));
  m.impl("empty_strided", TORCH_FN(empty_strided_cpu));
}

TORCH_LIBRARY_IMPL(aten, BackendSelect, m) {
  m.impl("is_pinned", TORCH_FN(is_pinned));
  m.impl("_pin_memory", TORCH_FN(pin_memory_copy));
}

const bool g_restored = [] {
  c10::WarningUtils::set_warning_handler(g_prev_handler);
  return true;
}();

}  // namespace
}  // namespace torch_gcu
