// Output handling for ATen's structured meta functions on gcu tensors.
//
// A structured op's meta function (at::meta::structured_<op>::meta) checks
// the arguments and asks for its output through set_output_raw_strided; the
// in-tree backends supply the output in a small subclass, and so does this
// one: a fresh gcu tensor for the functional form, or the caller's out=
// tensor, checked for dtype and device and resized (restrided to the layout
// the meta function asks for only when it was resized), for the out form.
#pragma once

#include <ATen/ATen.h>
#include <ATen/NamedTensorUtils.h>
#include <ATen/TensorMeta.h>
#include <ATen/native/Resize.h>

namespace torch_gcu {

template <typename Meta>
struct OneOutput final : Meta {
  explicit OneOutput(const at::Tensor* out) : is_out(out != nullptr) {
    if (out != nullptr) result = *out;
  }
  const at::Tensor& maybe_get_output(int64_t) override { return result; }
  void set_output_strided(int64_t i, at::IntArrayRef sizes, at::IntArrayRef strides,
                          at::TensorOptions options, at::DimnameList names) override {
    set_output_raw_strided(i, sizes, strides, options, names);
  }
  void set_output_raw_strided(int64_t, at::IntArrayRef sizes, at::IntArrayRef strides,
                              at::TensorOptions options, at::DimnameList names) override {
    if (!is_out) {
      result = strides.empty() ? at::empty(sizes, options) : at::empty_strided(sizes, strides, options);
    } else {
      TORCH_CHECK(options.dtype() == result.dtype(), "Expected out tensor to have dtype ",
                  options.dtype(), ", but got ", result.dtype(), " instead");
      TORCH_CHECK(options.device() == result.device(), "Expected out tensor to have device ",
                  options.device(), ", but got ", result.device(), " instead");
      if (at::native::resize_output(result, sizes)) {
        if (!strides.empty())
          result.as_strided_(sizes, strides);
        else if (options.memory_format_opt().has_value())
          result.unsafeGetTensorImpl()->empty_tensor_restride(*options.memory_format_opt());
      }
    }
    if (!names.empty()) at::namedinference::propagate_names(result, names);
  }
  at::Tensor result;
  bool is_out;
};

}  // namespace torch_gcu
