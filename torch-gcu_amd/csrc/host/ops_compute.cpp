// Native kernels of the hot path: binary arithmetic, index_select,
// reductions and softmax.  Each computes the ATen output metadata (the
// structured meta / shape inference of the reference: gen_aot_ops.py:902-1063,
// torch_gcu/csrc/aten/shape_inference/*), allocates or resizes the output,
// and enqueues one kernel-library call on the current stream (the bridge of
// topsaten_bridge_define.h:323-336).  A CPU 0-dim operand is handed over by
// value (codegen/gen_backend_stubs.py:1061-1078), never copied to the device.
#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/WrapDimUtils.h>
#include <ATen/native/ReduceOpsUtils.h>
#include <ATen/native/Resize.h>

#include "aotops.h"
#include "dispatch_util.h"

namespace torch_gcu {
namespace aotops {

namespace {

bool is_cpu_scalar(const at::Tensor& t) { return t.device().is_cpu() && t.dim() == 0; }

enum class Bin { Add, Sub, Mul, Div };

at::ScalarType binary_result_type(Bin op, const at::Tensor& a, const at::Tensor& b) {
  at::ScalarType rt = at::result_type(a, b);
  if (op == Bin::Div && at::isIntegralType(rt, /*includeBool=*/true))
    rt = c10::typeMetaToScalarType(c10::get_default_dtype());
  return rt;
}

void check_alpha(Bin op, at::ScalarType common, const at::Scalar& alpha) {
  if (op == Bin::Sub) {
    TORCH_CHECK(common != at::kBool,
                "Subtraction, the `-` operator, with two bool tensors is not supported. "
                "Use the `^` or `logical_xor()` operator instead.");
  }
  if (op == Bin::Add || op == Bin::Sub) {
    TORCH_CHECK(!(at::isIntegralType(common, true) && alpha.isFloatingPoint()),
                "For integral input tensors, argument alpha must not be a floating point number.");
    TORCH_CHECK(common == at::kBool || !alpha.isBoolean(),
                "Boolean alpha only supported for Boolean results.");
  }
}

// out = op(self, other) with out already of the broadcast shape.
void run_binary(Bin op, const at::Tensor& out, const at::Tensor& self, const at::Tensor& other,
                const at::Scalar& alpha) {
  if (out.numel() == 0) return;
  const mi_tensor_t o = desc(out);
  const mi_stream_t s = mi_stream(out);
  const mi_scalar_t al = scalar_of(alpha);
  if (is_cpu_scalar(other) && is_gcu(self)) {
    const mi_tensor_t a = desc(self);
    mi_scalar_t v = scalar_of_tensor(other);
    switch (op) {
      case Bin::Add: check_mi(mi_add_scalar(&o, &a, v, al, s), "add"); return;
      case Bin::Sub: {
        mi_scalar_t neg = al;
        neg.f = -neg.f;
        neg.i = -neg.i;
        check_mi(mi_add_scalar(&o, &a, v, neg, s), "sub");
        return;
      }
      case Bin::Mul: check_mi(mi_mul_scalar(&o, &a, v, s), "mul"); return;
      case Bin::Div: check_mi(mi_div_scalar(&o, &a, v, s), "div"); return;
    }
  }
  // a CPU scalar in the first position is read as a 0-dim device tensor, so
  // it is rounded to the common dtype exactly as CPU ATen rounds it
  const at::Tensor a_t = is_cpu_scalar(self) ? self.to(out.device()) : self;
  const at::Tensor b_t = is_cpu_scalar(other) ? other.to(out.device()) : other;
  const mi_tensor_t a = desc(a_t), b = desc(b_t);
  switch (op) {
    case Bin::Add: check_mi(mi_add(&o, &a, &b, al, s), "add"); return;
    case Bin::Sub: check_mi(mi_sub(&o, &a, &b, al, s), "sub"); return;
    case Bin::Mul: check_mi(mi_mul(&o, &a, &b, s), "mul"); return;
    case Bin::Div: check_mi(mi_div(&o, &a, &b, s), "div"); return;
  }
}

// The checks TensorIterator makes before an elementwise kernel writes
// (CPU ATen raises the same errors): no element of the written tensor may
// share memory with another of its elements, and the written tensor and an
// input may share memory only element for element (in place).
void check_binary_overlap(const at::Tensor& out, const at::Tensor& self, const at::Tensor& other) {
  at::assert_no_internal_overlap(out);
  at::assert_no_partial_overlap(out, self);
  at::assert_no_partial_overlap(out, other);
}

at::Device gcu_device(const at::Tensor& a, const at::Tensor& b) {
  if (is_gcu(a)) return a.device();
  TORCH_CHECK(is_gcu(b), "gcu op called without a gcu tensor");
  return b.device();
}

at::Tensor binary_functional(Bin op, const at::Tensor& self, const at::Tensor& other,
                             const at::Scalar& alpha) {
  const at::ScalarType rt = binary_result_type(op, self, other);
  check_alpha(op, rt, alpha);
  const auto shape = at::infer_size_dimvector(self.sizes(), other.sizes());
  at::Tensor out = at::empty(shape, at::TensorOptions().dtype(rt).device(gcu_device(self, other)));
  run_binary(op, out, self, other, alpha);
  return out;
}

at::Tensor& binary_out(Bin op, const at::Tensor& self, const at::Tensor& other,
                       const at::Scalar& alpha, at::Tensor& out) {
  const at::ScalarType rt = binary_result_type(op, self, other);
  check_alpha(op, rt, alpha);
  TORCH_CHECK(at::canCast(rt, out.scalar_type()), "result type ", rt,
              " can't be cast to the desired output type ", out.scalar_type());
  const auto shape = at::infer_size_dimvector(self.sizes(), other.sizes());
  at::native::resize_output(out, shape);
  check_binary_overlap(out, self, other);
  run_binary(op, out, self, other, alpha);
  return out;
}

at::Tensor& binary_inplace(Bin op, at::Tensor& self, const at::Tensor& other,
                           const at::Scalar& alpha) {
  const at::ScalarType rt = binary_result_type(op, self, other);
  check_alpha(op, rt, alpha);
  TORCH_CHECK(at::canCast(rt, self.scalar_type()), "result type ", rt,
              " can't be cast to the desired output type ", self.scalar_type());
  const auto shape = at::infer_size_dimvector(self.sizes(), other.sizes());
  TORCH_CHECK(at::IntArrayRef(shape) == self.sizes(), "output with shape ", self.sizes(),
              " doesn't match the broadcast shape ", at::IntArrayRef(shape));
  check_binary_overlap(self, self, other);
  run_binary(op, self, self, other, alpha);
  return self;
}

}  // namespace

at::Tensor& add_out(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha,
                    at::Tensor& out) {
  return binary_out(Bin::Add, self, other, alpha, out);
}
at::Tensor add_Tensor(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha) {
  return binary_functional(Bin::Add, self, other, alpha);
}
at::Tensor& add__Tensor(at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha) {
  return binary_inplace(Bin::Add, self, other, alpha);
}
at::Tensor& sub_out(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha,
                    at::Tensor& out) {
  return binary_out(Bin::Sub, self, other, alpha, out);
}
at::Tensor sub_Tensor(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha) {
  return binary_functional(Bin::Sub, self, other, alpha);
}
at::Tensor& sub__Tensor(at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha) {
  return binary_inplace(Bin::Sub, self, other, alpha);
}
at::Tensor& mul_out(const at::Tensor& self, const at::Tensor& other, at::Tensor& out) {
  return binary_out(Bin::Mul, self, other, 1, out);
}
at::Tensor mul_Tensor(const at::Tensor& self, const at::Tensor& other) {
  return binary_functional(Bin::Mul, self, other, 1);
}
at::Tensor& mul__Tensor(at::Tensor& self, const at::Tensor& other) {
  return binary_inplace(Bin::Mul, self, other, 1);
}
at::Tensor& div_out(const at::Tensor& self, const at::Tensor& other, at::Tensor& out) {
  return binary_out(Bin::Div, self, other, 1, out);
}
at::Tensor div_Tensor(const at::Tensor& self, const at::Tensor& other) {
  return binary_functional(Bin::Div, self, other, 1);
}
at::Tensor& div__Tensor(at::Tensor& self, const at::Tensor& other) {
  return binary_inplace(Bin::Div, self, other, 1);
}

// ---- index_select ---------------------------------------------------------------

at::Tensor& index_select_out(const at::Tensor& self, int64_t dim, const at::Tensor& index,
                             at::Tensor& out) {
  // shape rules of torch_gcu/csrc/aten/shape_inference/indexing.cpp:20-69
  dim = at::maybe_wrap_dim(dim, self.dim());
  TORCH_CHECK_INDEX(index.dim() <= 1, "index_select(): Index is supposed to be a vector");
  TORCH_CHECK(index.scalar_type() == at::kLong || index.scalar_type() == at::kInt,
              "index_select(): Expected dtype int32 or int64 for index");
  TORCH_CHECK(self.scalar_type() == out.scalar_type(),
              "index_select(): self and out must have the same scalar type");
  // A device index is not range-checked on the host (that would need a
  // synchronising read); the kernel never reads outside self and writes an
  // out-of-range row as zeros.  A CPU 0-dim index (allowed as a scalar) is
  // checked here.
  at::Tensor idx = index;
  if (!is_gcu(idx)) {
    const int64_t n = self.dim() == 0 ? 1 : self.size(dim);
    const int64_t v = idx.item<int64_t>();
    TORCH_CHECK_INDEX(v >= 0 && v < n, "index out of range in self");
    idx = idx.to(self.device());
  }
  std::vector<int64_t> shape = self.sizes().vec();
  if (self.dim() > 0) shape[dim] = idx.numel();
  at::native::resize_output(out, shape);
  if (out.numel() == 0) return out;
  TORCH_CHECK_INDEX(self.dim() == 0 || self.size(dim) > 0,
                    "index_select(): self indexing axis dim should be positive");
  const mi_tensor_t o = desc(out), s = desc(self), ix = desc(idx);
  check_mi(mi_index_select(&o, &s, dim, &ix, mi_stream(out)), "index_select");
  return out;
}

at::Tensor index_select(const at::Tensor& self, int64_t dim, const at::Tensor& index) {
  at::Tensor out = at::empty({0}, self.options());
  return index_select_out(self, dim, index, out);
}

// ---- reductions ------------------------------------------------------------------

namespace {

enum class Red { Sum, Amax, Mean };

std::vector<int64_t> reduced_shape(const at::Tensor& self, at::OptionalIntArrayRef dims,
                                   bool keepdim) {
  std::vector<int64_t> out;
  const int64_t nd = self.dim();
  std::vector<bool> red(nd, false);
  if (!dims.has_value() || dims->empty()) {
    std::fill(red.begin(), red.end(), true);
  } else {
    for (int64_t d : *dims) {
      const int64_t w = at::maybe_wrap_dim(d, nd == 0 ? 1 : nd);
      if (nd > 0) {
        TORCH_CHECK(!red[w], "dim ", w, " appears multiple times in the list of dims");
        red[w] = true;
      }
    }
  }
  for (int64_t d = 0; d < nd; ++d) {
    if (!red[d]) out.push_back(self.size(d));
    else if (keepdim) out.push_back(1);
  }
  return out;
}

void run_reduce(Red op, const at::Tensor& self, at::OptionalIntArrayRef dims, bool keepdim,
                at::Tensor& out) {
  at::native::resize_output(out, reduced_shape(self, dims, keepdim));
  std::vector<int64_t> dv;
  if (dims.has_value()) dv = dims->vec();
  at::Tensor in = self;
  // an explicit dtype of another kind is applied to the input first
  if (op != Red::Amax && out.scalar_type() != self.scalar_type() &&
      !(at::isFloatingType(out.scalar_type()) && at::isFloatingType(self.scalar_type())) &&
      !(out.scalar_type() == at::kLong && at::isIntegralType(self.scalar_type(), true)))
    in = self.to(out.scalar_type());
  const mi_tensor_t o = desc(out), s = desc(in);
  const int32_t n = (int32_t)dv.size();
  const int64_t* d = dv.empty() ? nullptr : dv.data();
  switch (op) {
    case Red::Sum: check_mi(mi_sum(&o, &s, d, n, keepdim, mi_stream(out)), "sum"); break;
    case Red::Amax: check_mi(mi_amax(&o, &s, d, n, keepdim, mi_stream(out)), "amax"); break;
    case Red::Mean: check_mi(mi_mean(&o, &s, d, n, keepdim, mi_stream(out)), "mean"); break;
  }
}

at::ScalarType sum_dtype(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
  if (dtype.has_value()) return *dtype;
  return at::isIntegralType(self.scalar_type(), true) ? at::kLong : self.scalar_type();
}

}  // namespace

at::Tensor& sum_IntList_out(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                            std::optional<at::ScalarType> dtype, at::Tensor& out) {
  TORCH_CHECK(!dtype.has_value() || *dtype == out.scalar_type(),
              "Expected out tensor to have dtype ", *dtype, ", but got ", out.scalar_type());
  run_reduce(Red::Sum, self, dim, keepdim, out);
  return out;
}

at::Tensor sum_dim_IntList(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                           std::optional<at::ScalarType> dtype) {
  at::Tensor out = at::empty({0}, self.options().dtype(sum_dtype(self, dtype)));
  run_reduce(Red::Sum, self, dim, keepdim, out);
  return out;
}

at::Tensor& amax_out(const at::Tensor& self, at::IntArrayRef dim, bool keepdim, at::Tensor& out) {
  TORCH_CHECK(self.scalar_type() == out.scalar_type(), "Expected the dtype for input and out to "
              "match, but got ", self.scalar_type(), " for input's dtype and ", out.scalar_type(),
              " for out's dtype.");
  if (self.numel() == 0) {
    at::native::zero_numel_check_dims(self, dim, "amax()");
  }
  run_reduce(Red::Amax, self, dim, keepdim, out);
  return out;
}

at::Tensor amax(const at::Tensor& self, at::IntArrayRef dim, bool keepdim) {
  at::Tensor out = at::empty({0}, self.options());
  return amax_out(self, dim, keepdim, out);
}

at::Tensor& mean_out(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                     std::optional<at::ScalarType> dtype, at::Tensor& out) {
  const at::ScalarType dt = dtype.value_or(out.scalar_type());
  TORCH_CHECK(at::isFloatingType(dt) || at::isComplexType(dt),
              "mean(): could not infer output dtype. Input dtype must be either a floating point "
              "or complex dtype. Got: ", dt);
  run_reduce(Red::Mean, self, dim, keepdim, out);
  return out;
}

at::Tensor mean_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim,
                    std::optional<at::ScalarType> dtype) {
  const at::ScalarType dt = dtype.value_or(self.scalar_type());
  TORCH_CHECK(at::isFloatingType(dt) || at::isComplexType(dt),
              "mean(): could not infer output dtype. Input dtype must be either a floating point "
              "or complex dtype. Got: ", dt);
  at::Tensor out = at::empty({0}, self.options().dtype(dt));
  run_reduce(Red::Mean, self, dim, keepdim, out);
  return out;
}

// ---- softmax ------------------------------------------------------------------------

namespace {

void run_softmax(bool log, const at::Tensor& self, int64_t dim, bool half_to_float,
                 const at::Tensor& out) {
  if (half_to_float)
    TORCH_CHECK(self.scalar_type() == at::kHalf || self.scalar_type() == at::kBFloat16,
                "conversion is supported for Half and BFloat16 type only");
  dim = at::maybe_wrap_dim(dim, self.dim());
  if (self.numel() == 0) return;
  const at::Tensor in = self.contiguous();
  at::Tensor dst = out.is_contiguous() ? out : at::empty(out.sizes(), out.options());
  const mi_tensor_t o = desc(dst), s = desc(in);
  if (log) check_mi(mi_log_softmax(&o, &s, dim, mi_stream(out)), "log_softmax");
  else check_mi(mi_softmax(&o, &s, dim, mi_stream(out)), "softmax");
  if (!dst.is_same(out)) const_cast<at::Tensor&>(out).copy_(dst);
}

at::ScalarType softmax_out_type(const at::Tensor& self, bool half_to_float) {
  return half_to_float ? at::kFloat : self.scalar_type();
}

}  // namespace

at::Tensor _softmax(const at::Tensor& self, int64_t dim, bool half_to_float) {
  at::Tensor out = at::empty(self.sizes(), self.options().dtype(softmax_out_type(self, half_to_float)));
  run_softmax(false, self, dim, half_to_float, out);
  return out;
}

at::Tensor& _softmax_out(const at::Tensor& self, int64_t dim, bool half_to_float, at::Tensor& out) {
  at::native::resize_output(out, self.sizes());
  run_softmax(false, self, dim, half_to_float, out);
  return out;
}

at::Tensor _log_softmax(const at::Tensor& self, int64_t dim, bool half_to_float) {
  at::Tensor out = at::empty(self.sizes(), self.options().dtype(softmax_out_type(self, half_to_float)));
  run_softmax(true, self, dim, half_to_float, out);
  return out;
}

at::Tensor& _log_softmax_out(const at::Tensor& self, int64_t dim, bool half_to_float,
                             at::Tensor& out) {
  at::native::resize_output(out, self.sizes());
  run_softmax(true, self, dim, half_to_float, out);
  return out;
}

}  // namespace aotops
}  // namespace torch_gcu
