// Native kernels for tensor creation, storage, views, copies and fills.
//
// The reference implements these by hand outside its op generator:
// empty/empty_strided (torch_gcu/csrc/aten/aot_ops/gcu_empty_tensor.cpp:26-229),
// copies (gcu_copy.cpp:34-460), _local_scalar_dense (gcu_scalar.cpp:22-58),
// views and resize (gcu_tensor_shape.cpp, gcu_resize.cpp).  Unlike the
// reference, 64-bit dtypes keep their full width on the device
// (gcu_empty_tensor.cpp:50-58 halves them there).
#include <ATen/EmptyTensor.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/NamedTensorUtils.h>
#include <ATen/Operators.h>
#include <ATen/native/CPUFallback.h>
#include <ATen/ops/cat_meta.h>
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
#include "gcu_caching_host_allocator.h"
#include "structured_out.h"

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

namespace {

// A tensor whose elements tile [data_ptr, data_ptr + nbytes) exactly: its
// bytes move as one block and keep their meaning under the same strides.
bool dense_block(const at::Tensor& t) { return t.is_non_overlapping_and_dense(); }

// Host-device copies (gcu_copy.cpp:279-386).  The host side is one dense
// block: the tensor itself when it is dense, else a contiguous host staging
// copy.  The device side is that block's image (same sizes and strides, the
// host dtype): dst itself when its layout and dtype already match, else a
// device staging tensor that mi_copy casts, broadcasts and re-strides from or
// into.  Dtype casts thus run on the GPU, and the PCIe transfer is one
// hipMemcpyAsync on the current stream.
//
// Synchronisation: a non-blocking copy whose host block is pinned returns at
// once; the block is marked as used by the stream in the caching host
// allocator, so freeing it before the copy has run does not hand it out
// again.  Every other copy synchronises the stream before returning, since
// pageable memory may be reused by the caller as soon as the copy returns.
// Under graph capture only the first kind can be recorded.
void check_capturable(hipStream_t s, bool async_ok, const char* what) {
  TORCH_CHECK(async_ok || !stream_is_capturing(s), "gcu: ", what,
              " during graph capture needs pinned host memory, non_blocking=True and a dense "
              "host tensor");
}

// dtypes the copy kernel converts between; a cast that involves another
// dtype (complex, unsigned 16/32/64-bit, fp8) runs in CPU ATen on the host side
bool kernel_dtype(at::ScalarType t) {
  switch (t) {
    case at::kByte: case at::kChar: case at::kShort: case at::kInt: case at::kLong:
    case at::kHalf: case at::kFloat: case at::kDouble: case at::kBool: case at::kBFloat16:
      return true;
    default:
      return false;
  }
}

void mark_pinned_use(const at::Tensor& host, hipStream_t s, int device) {
  host_allocator::record_event(host.data_ptr(), host.storage().data_ptr().get_context(), s,
                               device);
}

at::Tensor copy_h2d(const at::Tensor& dst, const at::Tensor& src, bool non_blocking) {
  c10::DeviceGuard g(dst.device());
  const int dev = dst.device().index();
  const hipStream_t s = current_hip_stream(dst.device().index());
  const bool host_cast = src.scalar_type() != dst.scalar_type() &&
                         !(kernel_dtype(src.scalar_type()) && kernel_dtype(dst.scalar_type()));
  const bool dense = !host_cast && dense_block(src);
  const bool pinned = dense && src.is_pinned();
  // a non-dense (or host-cast) source is staged, in pinned memory when the
  // copy is non-blocking, so that it need not wait
  const bool async = non_blocking && (pinned || !dense);
  check_capturable(s, non_blocking && pinned, "a host-to-device copy");
  at::Tensor h = src;
  if (!dense) {
    h = at::empty(src.sizes(), src.options().dtype(host_cast ? dst.scalar_type() : src.scalar_type())
                                   .pinned_memory(async));
    h.copy_(src);
  }
  const size_t nbytes = (size_t)h.numel() * h.element_size();
  const bool direct = h.scalar_type() == dst.scalar_type() && h.sizes() == dst.sizes() &&
                      dense_block(dst) && h.strides() == dst.strides();
  if (direct) {
    GCU_HIP_CHECK(hipMemcpyAsync(dst.data_ptr(), h.data_ptr(), nbytes, hipMemcpyHostToDevice, s));
  } else {
    at::Tensor d = at::empty_strided(h.sizes(), h.strides(), dst.options().dtype(h.scalar_type()));
    GCU_HIP_CHECK(hipMemcpyAsync(d.data_ptr(), h.data_ptr(), nbytes, hipMemcpyHostToDevice, s));
    copy_d2d(dst, d.expand(dst.sizes()));
  }
  if (async)
    mark_pinned_use(h, s, dev);
  else
    GCU_HIP_CHECK(hipStreamSynchronize(s));
  return dst;
}

at::Tensor copy_d2h(const at::Tensor& dst, const at::Tensor& src, bool non_blocking) {
  c10::DeviceGuard g(src.device());
  const int dev = src.device().index();
  const hipStream_t s = current_hip_stream(src.device().index());
  const bool host_cast = src.scalar_type() != dst.scalar_type() &&
                         !(kernel_dtype(src.scalar_type()) && kernel_dtype(dst.scalar_type()));
  const bool dense = !host_cast && dense_block(dst);
  const bool async = non_blocking && dense && dst.is_pinned();
  check_capturable(s, async, "a device-to-host copy");
  // the host block the bytes land in: dst itself, or a staging copy in the
  // dtype the device holds when the cast happens on the host
  const at::Tensor h =
      dense ? dst : at::empty(dst.sizes(), dst.options().dtype(host_cast ? src.scalar_type()
                                                                           : dst.scalar_type()));
  at::Tensor d = src;
  if (!(src.scalar_type() == h.scalar_type() && src.sizes() == h.sizes() && dense_block(src) &&
        src.strides() == h.strides())) {
    d = at::empty_strided(h.sizes(), h.strides(), src.options().dtype(h.scalar_type()));
    copy_d2d(d, src.expand(h.sizes()));
  }
  GCU_HIP_CHECK(hipMemcpyAsync(h.data_ptr(), d.data_ptr(), (size_t)h.numel() * h.element_size(),
                               hipMemcpyDeviceToHost, s));
  if (async) {
    mark_pinned_use(h, s, dev);
    return dst;
  }
  GCU_HIP_CHECK(hipStreamSynchronize(s));
  check_index_faults((c10::DeviceIndex)dev);
  if (!dense) dst.copy_(h);
  return dst;
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
    // at::copy_ hands a gcu copy to _copy_from before its TensorIterator
    // would check memory overlap, so the checks are made here (CPU ATen
    // raises the same errors)
    at::assert_no_internal_overlap(dst);
    at::assert_no_partial_overlap(dst, self);
    copy_d2d(dst, self);
    return dst;
  }
  if (!src_gcu && dst_gcu) return copy_h2d(dst, self, non_blocking);
  if (src_gcu && !dst_gcu) {
    TORCH_CHECK(dst.device().is_cpu(), "gcu: cannot copy to device ", dst.device());
    return copy_d2h(dst, self, non_blocking);
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
  check_index_faults(self.device().index());
  return host.item();
}

// ---- cat ----------------------------------------------------------------------

namespace {

// cat's shape, dtype and memory-format rules are ATen's own structured meta
// function (at::meta::structured_cat: legacy 1-D empty inputs skipped, dim
// wrapped, sizes checked, result_type promotion, canCast into out, the
// memory format the inputs share); mi_cat fills the output.
using GcuCat = OneOutput<at::meta::structured_cat>;

bool kernel_dtype_all(const at::Tensor& out, const at::ITensorListRef& tensors) {
  if (!kernel_dtype(out.scalar_type())) return false;
  for (const at::Tensor& t : tensors)
    if (!kernel_dtype(t.scalar_type())) return false;
  return true;
}

void cat_fill(const at::Tensor& out, const at::ITensorListRef& tensors, int64_t dim) {
  if (out.numel() == 0) return;
  at::assert_no_internal_overlap(out);
  std::vector<mi_tensor_t> descs;
  for (const at::Tensor& t : tensors) {
    TORCH_CHECK(t.device() == out.device(), "torch.cat(): all input tensors and out must be on the "
                "same device, got ", t.device(), " and ", out.device());
    at::assert_no_overlap(out, t);
    // empty inputs add nothing (the legacy 1-D empty ones have another rank)
    if (t.numel() > 0) descs.push_back(desc(t));
  }
  std::vector<const mi_tensor_t*> ptrs;
  for (const auto& d : descs) ptrs.push_back(&d);
  const mi_tensor_t o = desc(out);
  check_mi(mi_cat(&o, ptrs.data(), (int32_t)ptrs.size(), (int32_t)dim, mi_stream(out)), "cat");
}

}  // namespace

at::Tensor cat(const at::ITensorListRef& tensors, int64_t dim) {
  GcuCat m(nullptr);
  const auto pre = m.meta(tensors, dim);
  if (!kernel_dtype_all(m.result, tensors))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(cat)>::call(tensors, dim);
  c10::DeviceGuard g(m.result.device());
  cat_fill(m.result, tensors, pre.dim);
  return m.result;
}

at::Tensor& cat_out(const at::ITensorListRef& tensors, int64_t dim, at::Tensor& out) {
  GcuCat m(&out);
  const auto pre = m.meta(tensors, dim);
  if (!kernel_dtype_all(out, tensors))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(cat, out)>::call(tensors, dim,
                                                                                     out);
  cat_fill(out, tensors, pre.dim);
  return out;
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
