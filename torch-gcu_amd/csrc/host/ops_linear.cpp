// The linear / matmul override the reference registers on PrivateUse1 only
// when ENFLAME_PT_ENABLE_LINEAR_OVERRIDE=true
// (torch_gcu/csrc/aten/RegisterLinearOverrideGCU.cpp:424-590; the
// registrations are env-gated in codegen/gcu_native_functions.yaml).
//   linear  folds a [..., K] input into one [M, K] x [K, N] product on the
//           MFMA kernel, with the bias added in the GEMM's epilogue (addmm)
//           and the result viewed back to [..., N];
//   matmul  follows ATen's operand folding (the reference restates it,
//           RegisterLinearOverrideGCU.cpp:42-103, 143-330), so a gcu matmul
//           reaches mm, bmm or addmv (mv) on the native kernels.
// Shapes these rules do not cover take ATen's own composition, which also
// raises ATen's errors.
#include <ATen/ATen.h>
#include <ATen/native/Resize.h>
#include <ATen/ops/linear_native.h>
#include <ATen/ops/matmul_native.h>

#include "aotops.h"
#include "dispatch_util.h"

namespace torch_gcu {
namespace aotops {

at::Tensor linear(const at::Tensor& input, const at::Tensor& weight,
                  const std::optional<at::Tensor>& bias) {
  const bool has_bias = bias.has_value() && bias->defined();
  if (weight.dim() != 2 || input.dim() < 2 || input.size(-1) != weight.size(1) ||
      (has_bias && bias->dim() > 1))
    return at::native::linear(input, weight, bias);
  const int64_t K = input.size(-1), N = weight.size(0);
  // a view when the leading dims fold, else a dense copy
  const at::Tensor x2 = input.dim() == 2 ? input : input.reshape({-1, K});
  at::Tensor y = has_bias ? at::addmm(*bias, x2, weight.t()) : at::mm(x2, weight.t());
  if (input.dim() == 2) return y;
  std::vector<int64_t> shape = input.sizes().vec();
  shape.back() = N;
  return y.view(shape);
}

at::Tensor& linear_out(const at::Tensor& input, const at::Tensor& weight,
                       const std::optional<at::Tensor>& bias, at::Tensor& out) {
  const at::Tensor r = aotops::linear(input, weight, bias);
  at::native::resize_output(out, r.sizes());
  out.copy_(r);
  return out;
}

at::Tensor matmul(const at::Tensor& self, const at::Tensor& other) {
  return at::native::matmul(self, other);
}

at::Tensor& matmul_out(const at::Tensor& self, const at::Tensor& other, at::Tensor& out) {
  return at::native::matmul_out(self, other, out);
}

}  // namespace aotops
}  // namespace torch_gcu
