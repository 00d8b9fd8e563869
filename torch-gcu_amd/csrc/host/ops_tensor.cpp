// Native kernels for tensor creation, storage, views, copies and fills.
//
// The reference implements these by hand outside its op generator:
// empty/empty_strided (torch_gcu/csrc/aten/aot_ops/gcu_empty_tensor.cpp:26-229),
// copies (gcu_copy.cpp:34-460), _local_scalar_dense (gcu_scalar.cpp:22-58),
// views and resize (gcu_tensor_shape.cpp, gcu_resize.cpp).  Unlike the
// reference, 64-bit dtypes keep their full width on the device
// (gcu_empty_tensor.cpp:50-58 halves them there).
#include <ATen/EmptyTensor.h>
#include <ATen/native/Resize.h>
#include <ATen/native/TensorFactories.h>
#include <ATen/ops/as_strided_native.h>
#include <ATen/ops/unfold_native.h>
#include <ATen/ops/view_native.h>
#include <ATen/ops/_reshape_alias_native.h>
#include <c10/core/CPUAllocator.h>

#include "aotops.h"
#include "dispatch_util.h"
#include "gcu_caching_allocator.h"

namespace torch_gcu {
namespace aotops {

namespace {

constexpr c10::DispatchKeySet kGCUKeys{c10::DispatchKey::PrivateUse1};

void check_layout(std::optional<at::Layout> layout) {
  TORCH_CHECK(!layout.has_value() || *layout == at::kStrided,
              "gcu: only strided tensors are supported, got layout ", *layout);
}

void check_no_pin(std::optional<bool> pin) {
  TORCH_CHECK(!pin.has_value() || !*pin, "gcu: pin_memory applies to CPU tensors only");
}

// Grows the storage of a gcu tensor to at least `nbytes`, keeping its data.
void grow_storage(const at::Storage& storage, size_t nbytes) {
  if (nbytes <= storage.nbytes()) return;
  c10::StorageImpl* impl = storage.unsafeGetStorageImpl();
  TORCH_CHECK(impl->resizable(), "Trying to resize storage that is not resizable");
  at::DataPtr fresh = allocator::get()->allocate(nbytes);
  const size_t keep = std::min(nbytes, storage.nbytes());
  if (keep > 0 && storage.data() != nullptr)
    GCU_HIP_CHECK(hipMemcpyAsync(fresh.get(), storage.data(), keep, hipMemcpyDeviceToDevice,
                                 current_hip_stream()));
  impl->set_data_ptr_noswap(std::move(fresh));
  impl->set_nbytes(nbytes);
}

}  // namespace

at::Tensor empty_memory_format(at::IntArrayRef size, std::optional<at::ScalarType> dtype,
                               std::optional<at::Layout> layout,
                               std::optional<at::Device> device, std::optional<bool> pin_memory,
                               std::optional<at::MemoryFormat> memory_format) {
  check_layout(layout);
  check_no_pin(pin_memory);
  const auto dt = dtype.value_or(c10::get_default_dtype_as_scalartype());
  return at::detail::empty_generic(size, allocator::get(), kGCUKeys, dt, memory_format);
}

at::Tensor empty_strided(at::IntArrayRef size, at::IntArrayRef stride,
                         std::optional<at::ScalarType> dtype, std::optional<at::Layout> layout,
                         std::optional<at::Device> device, std::optional<bool> pin_memory) {
  check_layout(layout);
  check_no_pin(pin_memory);
  const auto dt = dtype.value_or(c10::get_default_dtype_as_scalartype());
  return at::detail::empty_strided_generic(size, stride, allocator::get(), kGCUKeys, dt);
}

at::Tensor as_strided(const at::Tensor& self, at::IntArrayRef size, at::IntArrayRef stride,
                      std::optional<int64_t> storage_offset) {
  return at::native::as_strided_tensorimpl(self, size, stride, storage_offset);
}

at::Tensor view(const at::Tensor& self, at::IntArrayRef size) { return at::native::view(self, size); }

at::Tensor _reshape_alias(const at::Tensor& self, at::IntArrayRef size, at::IntArrayRef stride) {
  return at::native::_reshape_alias(self, size, stride);
}

at::Tensor unfold(const at::Tensor& self, int64_t dimension, int64_t size, int64_t step) {
  return at::native::unfold(self, dimension, size, step);
}

const at::Tensor& resize_(const at::Tensor& self, at::IntArrayRef size,
                          std::optional<at::MemoryFormat> memory_format) {
  auto* impl = self.unsafeGetTensorImpl();
  if (self.sizes() == size && !memory_format.has_value()) return self;
  impl->set_sizes_contiguous(size);
  if (memory_format.has_value() && *memory_format != at::MemoryFormat::Preserve)
    impl->empty_tensor_restride(*memory_format);
  const size_t needed =
      self.numel() == 0
          ? 0
          : at::detail::computeStorageNbytes(self.sizes(), self.strides(), self.dtype().itemsize(),
                                             self.storage_offset());
  grow_storage(self.storage(), needed);
  return self;
}

at::Tensor& set__source_Storage_storage_offset(at::Tensor& self, at::Storage source,
                                               int64_t storage_offset, at::IntArrayRef size,
                                               at::IntArrayRef stride) {
  at::native::checkSetStorage(self, source, storage_offset, size, stride);
  self.unsafeGetTensorImpl()->set_storage_offset(storage_offset);
  std::optional<at::IntArrayRef> st;
  if (!stride.empty()) st = stride;
  at::native::resize_impl_cpu_(self.unsafeGetTensorImpl(), size, st, /*resize_storage=*/false);
  return self;
}

at::Tensor& set__source_Storage(at::Tensor& self, at::Storage source) {
  const int64_t n = (int64_t)(source.nbytes() / self.dtype().itemsize());
  return set__source_Storage_storage_offset(self, source, 0, {n}, {});
}

at::Tensor& set__source_Tensor(at::Tensor& self, const at::Tensor& source) {
  if (self.unsafeGetTensorImpl() == source.unsafeGetTensorImpl()) return self;
  return set__source_Storage_storage_offset(self, source.storage(), source.storage_offset(),
                                            source.sizes(), source.strides());
}

at::Tensor& set_(at::Tensor& self) {
  at::Storage empty(at::Storage::use_byte_size_t(), 0, allocator::get(), true);
  return set__source_Storage_storage_offset(self, empty, 0, {0}, {});
}

void record_stream(at::Tensor& self, at::Stream s) {
  TORCH_CHECK(s.device_type() == kGCU, "record_stream: expected a gcu stream, got ", s);
  allocator::record_stream(self.storage().data_ptr(), c10::Stream(s));
}

// ---- copies -----------------------------------------------------------------------

namespace {

void copy_d2d(const at::Tensor& dst, const at::Tensor& src) {
  const at::Tensor s = src.device() == dst.device() ? src : src.to(dst.device());
  const mi_tensor_t o = desc(dst), i = desc(s);
  check_mi(mi_copy(&o, &i, mi_stream(dst)), "copy");
}

}  // namespace

at::Tensor _copy_from(const at::Tensor& self, const at::Tensor& dst, bool non_blocking) {
  if (self.numel() == 0) return dst;
  const bool src_gcu = is_gcu(self), dst_gcu = is_gcu(dst);
  if (src_gcu && dst_gcu) {
    if (self.device() != dst.device()) {
      // cross-device: stage through a dense copy on the source device
      c10::DeviceGuard g(self.device());
      at::Tensor tmp = at::empty(dst.sizes(), self.options().dtype(dst.scalar_type()));
      copy_d2d(tmp, self.expand(dst.sizes()));
      c10::DeviceGuard g2(dst.device());
      at::Tensor landed = at::empty(dst.sizes(), dst.options());
      GCU_HIP_CHECK(hipMemcpyPeer(landed.data_ptr(), dst.device().index(), tmp.data_ptr(),
                                  self.device().index(), tmp.nbytes()));
      copy_d2d(dst, landed);
      return dst;
    }
    c10::DeviceGuard g(dst.device());
    copy_d2d(dst, self);
    return dst;
  }
  if (!src_gcu && dst_gcu) {
    // host -> device: dense host staging in dst's dtype, one H2D copy, then a
    // device-side strided copy if dst is not dense
    c10::DeviceGuard g(dst.device());
    at::Tensor host = self.to(dst.scalar_type()).expand(dst.sizes()).contiguous();
    const hipStream_t s = current_hip_stream(dst.device().index());
    if (dst.is_contiguous()) {
      GCU_HIP_CHECK(hipMemcpyAsync(dst.data_ptr(), host.data_ptr(), host.nbytes(),
                                   hipMemcpyHostToDevice, s));
    } else {
      at::Tensor staging = at::empty(dst.sizes(), dst.options().memory_format(at::MemoryFormat::Contiguous));
      GCU_HIP_CHECK(hipMemcpyAsync(staging.data_ptr(), host.data_ptr(), host.nbytes(),
                                   hipMemcpyHostToDevice, s));
      copy_d2d(dst, staging);
    }
    // a pageable host buffer may be reused as soon as this returns
    if (!(non_blocking && self.is_pinned())) GCU_HIP_CHECK(hipStreamSynchronize(s));
    return dst;
  }
  if (src_gcu && !dst_gcu) {
    TORCH_CHECK(dst.device().is_cpu(), "gcu: cannot copy to device ", dst.device());
    c10::DeviceGuard g(self.device());
    const hipStream_t s = current_hip_stream(self.device().index());
    at::Tensor dense = self;
    if (!self.is_contiguous() || self.scalar_type() != dst.scalar_type() ||
        self.sizes() != dst.sizes()) {
      dense = at::empty(dst.sizes(), self.options().dtype(dst.scalar_type()));
      copy_d2d(dense, self);
    }
    if (dst.is_contiguous()) {
      GCU_HIP_CHECK(hipMemcpyAsync(dst.data_ptr(), dense.data_ptr(), dense.nbytes(),
                                   hipMemcpyDeviceToHost, s));
      GCU_HIP_CHECK(hipStreamSynchronize(s));
    } else {
      at::Tensor host = at::empty(dst.sizes(), dst.options().memory_format(at::MemoryFormat::Contiguous));
      GCU_HIP_CHECK(hipMemcpyAsync(host.data_ptr(), dense.data_ptr(), dense.nbytes(),
                                   hipMemcpyDeviceToHost, s));
      GCU_HIP_CHECK(hipStreamSynchronize(s));
      dst.copy_(host);
    }
    return dst;
  }
  TORCH_CHECK(false, "gcu _copy_from: neither tensor is on a gcu device");
}

at::Tensor _copy_from_and_resize(const at::Tensor& self, const at::Tensor& dst) {
  if (dst.sizes() != self.sizes()) {
    at::Tensor d = dst;
    d.resize_(self.sizes());
  }
  return aotops::_copy_from(self, dst, false);
}

at::Scalar _local_scalar_dense(const at::Tensor& self) {
  TORCH_CHECK(self.numel() > 0, "_local_scalar_dense: empty tensor");
  c10::DeviceGuard g(self.device());
  const hipStream_t s = current_hip_stream(self.device().index());
  TORCH_CHECK(!stream_is_capturing(s),
              "reading a gcu tensor's value on the host is not allowed during graph capture");
  at::Tensor host = at::empty({}, self.options().device(at::kCPU));
  GCU_HIP_CHECK(hipMemcpyAsync(host.data_ptr(), self.data_ptr(), self.dtype().itemsize(),
                               hipMemcpyDeviceToHost, s));
  GCU_HIP_CHECK(hipStreamSynchronize(s));
  return host.item();
}

// ---- fills --------------------------------------------------------------------

at::Tensor& fill__Scalar(at::Tensor& self, const at::Scalar& value) {
  if (self.numel() == 0) return self;
  const mi_tensor_t o = desc(self);
  check_mi(mi_fill(&o, scalar_of(value), mi_stream(self)), "fill_");
  return self;
}

at::Tensor& fill__Tensor(at::Tensor& self, const at::Tensor& value) {
  TORCH_CHECK(value.dim() == 0, "fill_ only supports 0-dimension value tensor but got tensor with ",
              value.dim(), " dimensions.");
  if (value.device().is_cpu()) return fill__Scalar(self, value.item());
  if (self.numel() == 0) return self;
  const mi_tensor_t o = desc(self), v = desc(value);
  check_mi(mi_copy(&o, &v, mi_stream(self)), "fill_");
  return self;
}

at::Tensor& zero_(at::Tensor& self) { return fill__Scalar(self, 0); }

}  // namespace aotops
}  // namespace torch_gcu
