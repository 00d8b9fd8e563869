// The training-side backward ops the reference registers natively but sends
// to CPU on its s60 hardware (codegen/gcu_op_fallback.yaml:22-41):
// silu and silu_backward, _log_softmax_backward_data / _softmax_backward_data and
// native_layer_norm_backward, and the layer-norm forward whose statistics
// that backward takes (native_layer_norm, yaml :481).  Shape and dtype rules are ATen's (the
// structured meta functions where the op has one); the arithmetic is the
// gfx950 kernels'.  dtypes the kernels do not cover run through the CPU
// fallback, as every unregistered op does.
#include <ATen/ExpandUtils.h>
#include <ATen/Operators.h>
#include <ATen/native/CPUFallback.h>
#include <ATen/native/Resize.h>
#include <ATen/native/layer_norm.h>
#include <ATen/ops/_log_softmax_backward_data_meta.h>
#include <ATen/ops/_softmax_backward_data_meta.h>

#include "aotops.h"
#include "dispatch_util.h"
#include "structured_out.h"

namespace torch_gcu {
namespace aotops {
namespace {

bool float_kernel_dtype(at::ScalarType t) {
  return t == at::kFloat || t == at::kBFloat16 || t == at::kHalf;
}

// grad_input = silu'(self) * grad_output with TensorIterator's rules:
// broadcast shape, common dtype, result cast into out.
void silu_backward_into(const at::Tensor& grad_output, const at::Tensor& self, at::Tensor& out) {
  const at::ScalarType dt = at::result_type(grad_output, self);
  if (out.numel() == 0) return;
  const at::Tensor go = grad_output.scalar_type() == dt ? grad_output : grad_output.to(dt);
  const at::Tensor x = self.scalar_type() == dt ? self : self.to(dt);
  at::Tensor target = out.scalar_type() == dt ? out : at::empty(out.sizes(), out.options().dtype(dt));
  const mi_tensor_t o = desc(target), g = desc(go), s = desc(x);
  check_mi(mi_silu_backward(&o, &g, &s, mi_stream(out)), "silu_backward");
  if (!target.is_same(out)) out.copy_(target);
}

void softmax_bwd_into(bool log, const at::Tensor& grad, const at::Tensor& output, int64_t dim,
                      const at::Tensor& out) {
  if (out.numel() == 0) return;
  dim = at::maybe_wrap_dim(dim, grad.dim());
  const at::Tensor g = grad.contiguous(), y = output.contiguous();
  at::Tensor dst = out.is_contiguous() ? out : at::empty(out.sizes(), out.options());
  const mi_tensor_t o = desc(dst), d = desc(g), s = desc(y);
  if (log) check_mi(mi_log_softmax_backward(&o, &d, &s, dim, mi_stream(out)), "log_softmax_backward");
  else check_mi(mi_softmax_backward(&o, &d, &s, dim, mi_stream(out)), "softmax_backward");
  if (!dst.is_same(out)) const_cast<at::Tensor&>(out).copy_(dst);
}

// grad (and so output) of a dtype the kernels take, and an output of the
// grad's dtype or, for float grads, f16 / bf16
bool softmax_bwd_ok(const at::Tensor& grad, const at::Tensor& output, const at::Tensor& out) {
  if (!float_kernel_dtype(grad.scalar_type()) || output.scalar_type() != grad.scalar_type())
    return false;
  return out.scalar_type() == grad.scalar_type() ||
         (grad.scalar_type() == at::kFloat && (out.scalar_type() == at::kHalf ||
                                               out.scalar_type() == at::kBFloat16));
}

using LogSoftmaxBwdMeta = OneOutput<at::meta::structured__log_softmax_backward_data>;
using SoftmaxBwdMeta = OneOutput<at::meta::structured__softmax_backward_data>;

}  // namespace

// silu (yaml silu.out :561 of the reference's list): out = self * sigmoid(self)
// with TensorIterator's unary rules (out resized to self, result cast into out).
namespace {
void silu_into(const at::Tensor& self, at::Tensor& out) {
  if (out.numel() == 0) return;
  at::Tensor target = out.scalar_type() == self.scalar_type()
                          ? out
                          : at::empty(out.sizes(), out.options().dtype(self.scalar_type()));
  const mi_tensor_t o = desc(target), x = desc(self);
  check_mi(mi_silu(&o, &x, mi_stream(out)), "silu");
  if (!target.is_same(out)) out.copy_(target);
}
}  // namespace

at::Tensor silu(const at::Tensor& self) {
  if (!float_kernel_dtype(self.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(silu)>::call(self);
  at::Tensor out = at::empty(self.sizes(), self.options().memory_format(self.suggest_memory_format()));
  silu_into(self, out);
  return out;
}

at::Tensor& silu_(at::Tensor& self) {
  if (!float_kernel_dtype(self.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(silu_)>::call(self);
  silu_into(self, self);
  return self;
}

at::Tensor& silu_out(const at::Tensor& self, at::Tensor& out) {
  if (!float_kernel_dtype(self.scalar_type()) || !float_kernel_dtype(out.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(silu, out)>::call(self, out);
  TORCH_CHECK(at::canCast(self.scalar_type(), out.scalar_type()), "result type ",
              self.scalar_type(), " can't be cast to the desired output type ", out.scalar_type());
  at::native::resize_output(out, self.sizes());
  silu_into(self, out);
  return out;
}

at::Tensor silu_backward(const at::Tensor& grad_output, const at::Tensor& self) {
  const at::ScalarType dt = at::result_type(grad_output, self);
  if (!float_kernel_dtype(dt))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(silu_backward)>::call(grad_output,
                                                                                         self);
  at::Tensor out = at::empty(at::infer_size(grad_output.sizes(), self.sizes()),
                             grad_output.options().dtype(dt));
  silu_backward_into(grad_output, self, out);
  return out;
}

at::Tensor& silu_backward_grad_input(const at::Tensor& grad_output, const at::Tensor& self,
                                     at::Tensor& grad_input) {
  const at::ScalarType dt = at::result_type(grad_output, self);
  if (!float_kernel_dtype(dt) || !float_kernel_dtype(grad_input.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(silu_backward, grad_input)>::call(
        grad_output, self, grad_input);
  TORCH_CHECK(at::canCast(dt, grad_input.scalar_type()), "result type ", dt,
              " can't be cast to the desired output type ", grad_input.scalar_type());
  at::native::resize_output(grad_input, at::infer_size(grad_output.sizes(), self.sizes()));
  silu_backward_into(grad_output, self, grad_input);
  return grad_input;
}

at::Tensor _log_softmax_backward_data(const at::Tensor& grad_output, const at::Tensor& output,
                                      int64_t dim, at::ScalarType input_dtype) {
  LogSoftmaxBwdMeta m(nullptr);
  m.meta(grad_output, output, dim, input_dtype);
  if (!softmax_bwd_ok(grad_output, output, m.result))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(_log_softmax_backward_data)>::call(
        grad_output, output, dim, input_dtype);
  softmax_bwd_into(true, grad_output, output, dim, m.result);
  return m.result;
}

at::Tensor& _log_softmax_backward_data_out(const at::Tensor& grad_output, const at::Tensor& output,
                                           int64_t dim, at::ScalarType input_dtype,
                                           at::Tensor& out) {
  LogSoftmaxBwdMeta m(&out);
  m.meta(grad_output, output, dim, input_dtype);
  if (!softmax_bwd_ok(grad_output, output, out))
    return at::native::call_fallback_fn<&gcu_cpu_fallback,
                                        ATEN_OP2(_log_softmax_backward_data, out)>::call(
        grad_output, output, dim, input_dtype, out);
  softmax_bwd_into(true, grad_output, output, dim, out);
  return out;
}

at::Tensor _softmax_backward_data(const at::Tensor& grad_output, const at::Tensor& output,
                                  int64_t dim, at::ScalarType input_dtype) {
  SoftmaxBwdMeta m(nullptr);
  m.meta(grad_output, output, dim, input_dtype);
  if (!softmax_bwd_ok(grad_output, output, m.result))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(_softmax_backward_data)>::call(
        grad_output, output, dim, input_dtype);
  softmax_bwd_into(false, grad_output, output, dim, m.result);
  return m.result;
}

at::Tensor& _softmax_backward_data_out(const at::Tensor& grad_output, const at::Tensor& output,
                                       int64_t dim, at::ScalarType input_dtype,
                                       at::Tensor& grad_input) {
  SoftmaxBwdMeta m(&grad_input);
  m.meta(grad_output, output, dim, input_dtype);
  if (!softmax_bwd_ok(grad_output, output, grad_input))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(_softmax_backward_data, out)>::call(
        grad_output, output, dim, input_dtype, grad_input);
  softmax_bwd_into(false, grad_output, output, dim, grad_input);
  return grad_input;
}

// ATen's layer_norm_cpu contract: _check_layer_norm_inputs, mean and rstd
// fp32 when a 16-bit input meets fp32 parameters ("mixed type") and of the
// input's dtype otherwise, shaped [leading dims..., 1, ...].
std::tuple<at::Tensor, at::Tensor, at::Tensor> native_layer_norm(
    const at::Tensor& input, at::IntArrayRef normalized_shape,
    const std::optional<at::Tensor>& weight, const std::optional<at::Tensor>& bias, double eps) {
  const at::Tensor w = weight.has_value() ? *weight : at::Tensor();
  const at::Tensor b = bias.has_value() ? *bias : at::Tensor();
  const auto mn = at::native::_check_layer_norm_inputs(input, normalized_shape, w, b);
  const int64_t N = mn.second;
  const at::ScalarType dt = input.scalar_type();
  // a 16-bit input with fp32 weight / bias (ATen's is_mixed_type and
  // check_mixed_data_type)
  const bool mixed = (dt == at::kBFloat16 || dt == at::kHalf) &&
                     ((w.defined() && w.scalar_type() == at::kFloat) ||
                      (b.defined() && b.scalar_type() == at::kFloat));
  if (mixed)
    TORCH_CHECK((!w.defined() || w.scalar_type() == at::kFloat) &&
                    (!b.defined() || b.scalar_type() == at::kFloat),
                "mixed dtype (CPU): all inputs must share same datatype.");
  auto param_ok = [&](const at::Tensor& t) {
    return !t.defined() || t.scalar_type() == dt || t.scalar_type() == at::kFloat;
  };
  if (!float_kernel_dtype(dt) || !param_ok(w) || !param_ok(b))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(native_layer_norm)>::call(
        input, normalized_shape, weight, bias, eps);
  const at::Tensor x = input.contiguous();
  at::Tensor out = at::empty_like(x, at::MemoryFormat::Contiguous);
  const int64_t axis = input.dim() - (int64_t)normalized_shape.size();
  std::vector<int64_t> stat_shape;
  for (int64_t i = 0; i < input.dim(); ++i) stat_shape.push_back(i < axis ? input.size(i) : 1);
  const at::ScalarType sdt = mixed ? at::kFloat : dt;
  at::Tensor mean = at::empty(stat_shape, x.options().dtype(sdt));
  at::Tensor rstd = at::empty(stat_shape, x.options().dtype(sdt));
  const at::Tensor gamma = w.defined() ? w.contiguous() : w, beta = b.defined() ? b.contiguous() : b;
  const mi_tensor_t o = desc(out), m = desc(mean), r = desc(rstd), dx = desc(x), dw = desc(gamma),
                    db = desc(beta);
  check_mi(mi_layer_norm(&o, &m, &r, &dx, gamma.defined() ? &dw : nullptr,
                         beta.defined() ? &db : nullptr, N, eps, mi_stream(x)),
           "native_layer_norm");
  return {out, mean, rstd};
}

// ATen's layer_norm_backward_cpu contract: the checks of
// _check_layer_norm_inputs, dgamma / dbeta shaped like weight / bias (zero
// when there are no rows), outputs only where the mask asks.
std::tuple<at::Tensor, at::Tensor, at::Tensor> native_layer_norm_backward(
    const at::Tensor& grad_out, const at::Tensor& input, at::IntArrayRef normalized_shape,
    const at::Tensor& mean, const at::Tensor& rstd, const std::optional<at::Tensor>& weight,
    const std::optional<at::Tensor>& bias, std::array<bool, 3> output_mask) {
  const at::Tensor w = weight.has_value() ? *weight : at::Tensor();
  const at::Tensor b = bias.has_value() ? *bias : at::Tensor();
  const auto mn = at::native::_check_layer_norm_inputs(input, normalized_shape, w, b);
  const int64_t M = mn.first, N = mn.second;
  const at::ScalarType dt = input.scalar_type();
  const bool kernel_ok =
      float_kernel_dtype(dt) && grad_out.scalar_type() == dt &&
      (mean.scalar_type() == at::kFloat || mean.scalar_type() == dt) &&
      rstd.scalar_type() == mean.scalar_type() &&
      (!w.defined() || w.scalar_type() == dt || w.scalar_type() == at::kFloat) &&
      (!output_mask[1] || (w.defined() && float_kernel_dtype(w.scalar_type()))) &&
      (!output_mask[2] || (b.defined() && float_kernel_dtype(b.scalar_type())));
  if (!kernel_ok)
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(native_layer_norm_backward)>::call(
        grad_out, input, normalized_shape, mean, rstd, weight, bias, output_mask);
  const at::Tensor x = input.contiguous();
  const at::Tensor dy = grad_out.contiguous();
  const at::Tensor mu = mean.contiguous(), rs = rstd.contiguous();
  const at::Tensor gamma = w.defined() ? w.contiguous() : w;
  at::Tensor dx, dgamma, dbeta;
  if (output_mask[0]) dx = at::empty_like(x, at::MemoryFormat::Contiguous);
  if (output_mask[1]) dgamma = at::empty_like(gamma, at::MemoryFormat::Contiguous);
  if (output_mask[2]) dbeta = at::empty_like(b, at::MemoryFormat::Contiguous);
  if (!output_mask[0] && !output_mask[1] && !output_mask[2]) return {dx, dgamma, dbeta};
  const mi_tensor_t d_dx = desc(dx), d_dw = desc(dgamma), d_db = desc(dbeta);
  const mi_tensor_t d_dy = desc(dy), d_x = desc(x), d_mu = desc(mu), d_rs = desc(rs), d_w = desc(gamma);
  check_mi(mi_layer_norm_backward(output_mask[0] ? &d_dx : nullptr, output_mask[1] ? &d_dw : nullptr,
                                  output_mask[2] ? &d_db : nullptr, &d_dy, &d_x, &d_mu, &d_rs,
                                  gamma.defined() ? &d_w : nullptr, N, mi_stream(x)),
           "native_layer_norm_backward");
  (void)M;
  return {dx, dgamma, dbeta};
}

}  // namespace aotops
}  // namespace torch_gcu
