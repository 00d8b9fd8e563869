// torch._fused_adamw_ on gcu tensors (the reference's
// torch_gcu/csrc/aten/aot_ops/_fused_adamw_.cpp:15-52 with the checks of
// shape_inference/_fused_adamw_.cpp:12-60): the parameter lists go to
// mi_fused_adamw in one launch per 32 tensors.  A CPU lr tensor is read on
// the host (as the reference does); a gcu one, like the step counts,
// grad_scale and found_inf, is read by the kernel.
#include <ATen/native/CPUFallback.h>
#include <ATen/native/ForeachUtils.h>
#include <ATen/Operators.h>

#include <vector>

#include "aotops.h"
#include "dispatch_util.h"

namespace torch_gcu {
namespace aotops {
namespace {

bool kernel_dtype(at::ScalarType t) {
  return t == at::kFloat || t == at::kBFloat16 || t == at::kHalf || t == at::kDouble;
}

// The reference's checks: the lists agree in dtype, device, sizes and
// strides and are dense; the scalar tensors sit on the params' device.
void check_adamw(at::TensorList self, at::TensorList grads, at::TensorList exp_avgs,
                 at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs,
                 at::TensorList state_steps, bool amsgrad, const at::Tensor* lr,
                 const std::optional<at::Tensor>& grad_scale,
                 const std::optional<at::Tensor>& found_inf) {
  const size_t n = self.size();
  TORCH_CHECK(grads.size() == n && exp_avgs.size() == n && exp_avg_sqs.size() == n &&
                  state_steps.size() == n && (!amsgrad || max_exp_avg_sqs.size() == n),
              "_fused_adamw_: all tensor lists must have the same length");
  if (amsgrad) {
    TORCH_CHECK(at::native::check_fast_path_restrictions(
                    {self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs}),
                "self, grads, exp_avgs, exp_avg_sqs, and max_exp_avg_sqs must have same dtype, "
                "device, and layout");
  } else {
    TORCH_CHECK(at::native::check_fast_path_restrictions({self, grads, exp_avgs, exp_avg_sqs}),
                "self, grads, exp_avgs, and exp_avg_sqs must have same dtype, device, and layout");
  }
  const at::Device dev = self[0].device();
  if (grad_scale.has_value())
    TORCH_CHECK(grad_scale->device() == dev, "grad_scale must be on the same GCU device as the params");
  if (found_inf.has_value())
    TORCH_CHECK(found_inf->device() == dev, "found_inf must be on the same GCU device as the params");
  if (lr != nullptr && !lr->is_cpu())
    TORCH_CHECK(lr->device() == dev, "lr must be on the same GCU device as the params");
}

// Everything the kernel reads as a one-element fp32 scalar (step counts,
// grad_scale, found_inf) is fp32 on the params' device.
bool scalars_fit(at::TensorList state_steps, const std::optional<at::Tensor>& grad_scale,
                 const std::optional<at::Tensor>& found_inf, const at::Device dev) {
  auto ok = [&](const at::Tensor& t) {
    return t.device() == dev && t.scalar_type() == at::kFloat && t.numel() == 1;
  };
  for (const at::Tensor& t : state_steps)
    if (!ok(t)) return false;
  return (!grad_scale.has_value() || ok(*grad_scale)) && (!found_inf.has_value() || ok(*found_inf));
}

void run_adamw(at::TensorList self, at::TensorList grads, at::TensorList exp_avgs,
               at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs,
               at::TensorList state_steps, const at::Tensor* lr_dev, double lr, double beta1,
               double beta2, double weight_decay, double eps, bool amsgrad, bool maximize,
               const std::optional<at::Tensor>& grad_scale,
               const std::optional<at::Tensor>& found_inf) {
  c10::DeviceGuard g(self[0].device());
  const size_t n = self.size();
  std::vector<mi_tensor_t> d(n * 6);
  std::vector<const mi_tensor_t*> ptr(n * 6);
  for (size_t i = 0; i < n; ++i) {
    d[i] = desc(self[i]);
    d[n + i] = desc(grads[i]);
    d[2 * n + i] = desc(exp_avgs[i]);
    d[3 * n + i] = desc(exp_avg_sqs[i]);
    d[4 * n + i] = amsgrad ? desc(max_exp_avg_sqs[i]) : mi_tensor_t{};
    d[5 * n + i] = desc(state_steps[i]);
  }
  for (size_t i = 0; i < 6 * n; ++i) ptr[i] = &d[i];
  mi_adamw_hparams_t hp{};
  hp.lr = lr;
  hp.beta1 = beta1;
  hp.beta2 = beta2;
  hp.weight_decay = weight_decay;
  hp.eps = eps;
  hp.amsgrad = amsgrad ? 1 : 0;
  hp.maximize = maximize ? 1 : 0;
  mi_tensor_t lr_d{}, gs_d{}, fi_d{};
  if (lr_dev != nullptr) lr_d = desc(*lr_dev);
  if (grad_scale.has_value()) gs_d = desc(*grad_scale);
  if (found_inf.has_value()) fi_d = desc(*found_inf);
  check_mi(mi_fused_adamw(ptr.data(), ptr.data() + n, ptr.data() + 2 * n, ptr.data() + 3 * n,
                          amsgrad ? ptr.data() + 4 * n : nullptr, ptr.data() + 5 * n, (int32_t)n,
                          lr_dev != nullptr ? &lr_d : nullptr, &hp,
                          grad_scale.has_value() ? &gs_d : nullptr,
                          found_inf.has_value() ? &fi_d : nullptr, mi_stream(self[0])),
           "_fused_adamw_");
}

}  // namespace

void _fused_adamw_(at::TensorList self, at::TensorList grads, at::TensorList exp_avgs,
                   at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs,
                   at::TensorList state_steps, double lr, double beta1, double beta2,
                   double weight_decay, double eps, bool amsgrad, bool maximize,
                   const std::optional<at::Tensor>& grad_scale,
                   const std::optional<at::Tensor>& found_inf) {
  if (self.empty()) return;
  check_adamw(self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, amsgrad, nullptr,
              grad_scale, found_inf);
  if (!kernel_dtype(self[0].scalar_type()) ||
      !scalars_fit(state_steps, grad_scale, found_inf, self[0].device()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(_fused_adamw_)>::call(
        self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, lr, beta1, beta2,
        weight_decay, eps, amsgrad, maximize, grad_scale, found_inf);
  run_adamw(self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, nullptr, lr, beta1,
            beta2, weight_decay, eps, amsgrad, maximize, grad_scale, found_inf);
}

void _fused_adamw__tensor_lr(at::TensorList self, at::TensorList grads, at::TensorList exp_avgs,
                             at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs,
                             at::TensorList state_steps, const at::Tensor& lr, double beta1,
                             double beta2, double weight_decay, double eps, bool amsgrad,
                             bool maximize, const std::optional<at::Tensor>& grad_scale,
                             const std::optional<at::Tensor>& found_inf) {
  if (self.empty()) return;
  check_adamw(self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, amsgrad, &lr,
              grad_scale, found_inf);
  const bool lr_ok = lr.is_cpu() || ((lr.scalar_type() == at::kFloat ||
                                      lr.scalar_type() == at::kDouble) && lr.numel() == 1);
  if (!kernel_dtype(self[0].scalar_type()) || !lr_ok ||
      !scalars_fit(state_steps, grad_scale, found_inf, self[0].device()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(_fused_adamw_, tensor_lr)>::call(
        self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, lr, beta1, beta2,
        weight_decay, eps, amsgrad, maximize, grad_scale, found_inf);
  if (lr.is_cpu())
    run_adamw(self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, nullptr,
              lr.item<double>(), beta1, beta2, weight_decay, eps, amsgrad, maximize, grad_scale,
              found_inf);
  else
    run_adamw(self, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, &lr, 0.0, beta1,
              beta2, weight_decay, eps, amsgrad, maximize, grad_scale, found_inf);
}

// t += scalar for every tensor of the list (the reference's generated
// _foreach_add_.Scalar, yaml :47): one multi-tensor launch when the list is
// dense and of one float dtype with a real scalar, else ATen's per-tensor
// add_ (which runs on the native elementwise kernel).
namespace {

// One multi-tensor launch when the list is dense and of one float dtype on
// one device; false when the caller must take ATen's per-tensor path.
bool foreach_fast(at::TensorList self) {
  const at::ScalarType dt = self[0].scalar_type();
  bool fast = kernel_dtype(dt);
  for (const at::Tensor& t : self)
    fast = fast && t.scalar_type() == dt && t.device() == self[0].device() &&
           (t.numel() == 0 || t.is_non_overlapping_and_dense());
  return fast;
}

template <typename F>
void foreach_launch(at::TensorList self, const char* what, F&& call) {
  c10::DeviceGuard g(self[0].device());
  std::vector<mi_tensor_t> d;
  d.reserve(self.size());
  for (const at::Tensor& t : self) d.push_back(desc(t));
  std::vector<const mi_tensor_t*> ptr;
  for (const auto& x : d) ptr.push_back(&x);
  check_mi(call(ptr.data(), (int32_t)ptr.size(), mi_stream(self[0])), what);
}

bool real_scalar(const at::Scalar& s) { return !s.isComplex() && !s.isBoolean(); }

// The value a Python-number operand of _foreach_add_ / _foreach_mul_ takes:
// CPU ATen first rounds it to a 16-bit list's own dtype, then computes in
// float (a 0-dim tensor operand keeps its float value).
double list_scalar(const at::Scalar& s, at::ScalarType dt) {
  if (dt == at::kBFloat16) return static_cast<float>(s.to<c10::BFloat16>());
  if (dt == at::kHalf) return static_cast<float>(s.to<c10::Half>());
  return s.toDouble();
}

}  // namespace

void _foreach_add__Scalar(at::TensorList self, const at::Scalar& scalar) {
  if (self.empty()) return;
  if (!foreach_fast(self) || !real_scalar(scalar)) {
    for (const at::Tensor& t : self) const_cast<at::Tensor&>(t).add_(scalar);
    return;
  }
  foreach_launch(self, "_foreach_add_", [&](const mi_tensor_t* const* p, int32_t n, mi_stream_t s) {
    return mi_foreach_add_scalar(p, n, list_scalar(scalar, self[0].scalar_type()), s);
  });
}

// _foreach_mul_.Scalar (yaml :131): the same launch with a product.
void _foreach_mul__Scalar(at::TensorList self, const at::Scalar& scalar) {
  if (self.empty()) return;
  if (!foreach_fast(self) || !real_scalar(scalar)) {
    for (const at::Tensor& t : self) const_cast<at::Tensor&>(t).mul_(scalar);
    return;
  }
  foreach_launch(self, "_foreach_mul_", [&](const mi_tensor_t* const* p, int32_t n, mi_stream_t s) {
    return mi_foreach_mul_scalar(p, n, list_scalar(scalar, self[0].scalar_type()), nullptr, s);
  });
}

// _foreach_mul_.Tensor (yaml :133), as gradient clipping calls it: a 0-dim
// fp32 scalar on the list's device is read by the kernel (no host sync); a
// CPU scalar is read on the host; other scalars take ATen's per-tensor mul_.
void _foreach_mul__Tensor(at::TensorList self, const at::Tensor& other) {
  TORCH_CHECK(other.dim() == 0, "scalar tensor expected to be 0 dim but it has ", other.dim(),
              " dimensions and ", other.numel(), " elements.");
  if (self.empty()) return;
  const bool on_dev = other.device() == self[0].device() && other.scalar_type() == at::kFloat;
  if (!foreach_fast(self) || !(on_dev || (other.is_cpu() && !other.is_complex() &&
                                          other.scalar_type() != at::kBool))) {
    for (const at::Tensor& t : self) const_cast<at::Tensor&>(t).mul_(other);
    return;
  }
  if (on_dev) {
    const mi_tensor_t sd = desc(other);
    foreach_launch(self, "_foreach_mul_", [&](const mi_tensor_t* const* p, int32_t n, mi_stream_t s) {
      return mi_foreach_mul_scalar(p, n, 0.0, &sd, s);
    });
    return;
  }
  const double v = other.item<double>();
  foreach_launch(self, "_foreach_mul_", [&](const mi_tensor_t* const* p, int32_t n, mi_stream_t s) {
    return mi_foreach_mul_scalar(p, n, v, nullptr, s);
  });
}

// GradScaler's unscale step (the reference's generated
// _amp_foreach_non_finite_check_and_unscale_, yaml :15): one multi-tensor
// launch per list of one float dtype; other lists go to CPU ATen.
void _amp_foreach_non_finite_check_and_unscale_(at::TensorList self, at::Tensor& found_inf,
                                                const at::Tensor& inv_scale) {
  TORCH_CHECK(inv_scale.numel() == 1, "inv_scale must be a 1-element tensor.");
  TORCH_CHECK(found_inf.numel() == 1, "found_inf must be a 1-element tensor.");
  TORCH_CHECK(inv_scale.scalar_type() == at::ScalarType::Float, "inv_scale must be a float tensor.");
  TORCH_CHECK(found_inf.scalar_type() == at::ScalarType::Float, "found_inf must be a float tensor.");
  if (self.empty()) return;
  const at::ScalarType dt = self[0].scalar_type();
  bool fast = kernel_dtype(dt) && found_inf.device() == self[0].device() &&
              inv_scale.device() == self[0].device();
  for (const at::Tensor& t : self)
    fast = fast && t.scalar_type() == dt && t.device() == self[0].device() &&
           (t.numel() == 0 || t.is_non_overlapping_and_dense());
  if (!fast)
    return at::native::call_fallback_fn<&gcu_cpu_fallback,
                                        ATEN_OP(_amp_foreach_non_finite_check_and_unscale_)>::call(
        self, found_inf, inv_scale);
  c10::DeviceGuard g(self[0].device());
  std::vector<mi_tensor_t> d;
  d.reserve(self.size());
  for (const at::Tensor& t : self) d.push_back(desc(t));
  std::vector<const mi_tensor_t*> ptr;
  for (const auto& x : d) ptr.push_back(&x);
  const mi_tensor_t fi = desc(found_inf), is = desc(inv_scale);
  check_mi(mi_amp_unscale(ptr.data(), (int32_t)ptr.size(), &fi, &is, mi_stream(self[0])),
           "_amp_foreach_non_finite_check_and_unscale_");
}

// GradScaler's scale update (the reference's generated _amp_update_scale_,
// yaml :16) on the device; tensors on another device or of other dtypes go
// to CPU ATen, which raises ATen's own errors for them.
at::Tensor& _amp_update_scale_(at::Tensor& self, at::Tensor& growth_tracker,
                               const at::Tensor& found_inf, double scale_growth_factor,
                               double scale_backoff_factor, int64_t growth_interval) {
  const bool fast = self.numel() == 1 && self.scalar_type() == at::kFloat &&
                    growth_tracker.numel() == 1 && growth_tracker.scalar_type() == at::kInt &&
                    found_inf.numel() == 1 && found_inf.scalar_type() == at::kFloat &&
                    growth_tracker.device() == self.device() && found_inf.device() == self.device();
  if (!fast)
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP(_amp_update_scale_)>::call(
        self, growth_tracker, found_inf, scale_growth_factor, scale_backoff_factor,
        growth_interval);
  c10::DeviceGuard g(self.device());
  const mi_tensor_t s = desc(self), gt = desc(growth_tracker), fi = desc(found_inf);
  check_mi(mi_amp_update_scale(&s, &gt, &fi, scale_growth_factor, scale_backoff_factor,
                               growth_interval, mi_stream(self)),
           "_amp_update_scale_");
  return self;
}

}  // namespace aotops
}  // namespace torch_gcu
