// efficient_ops entry points (the reference's efficient_ops/ops.h:14-93 surface,
// extended with the fused ops of this build).
#pragma once

#include <ATen/ATen.h>

#include <optional>
#include <tuple>

namespace torch_gcu {
namespace efficient {

at::Tensor rms_norm(const at::Tensor& x, const std::optional<at::Tensor>& weight, double eps);
std::tuple<at::Tensor, at::Tensor> rope(const at::Tensor& q, const at::Tensor& k,
                                        const at::Tensor& positions, double theta);
void rope_(at::Tensor& q, const std::optional<at::Tensor>& k, const at::Tensor& positions,
           double theta);
at::Tensor silu_mul(const at::Tensor& gate, const at::Tensor& up);
at::Tensor int32_indices_index(const at::Tensor& self,
                               const c10::List<std::optional<at::Tensor>>& indices);
at::Tensor int8_linear(const at::Tensor& x, const at::Tensor& weight, const at::Tensor& scales,
                       const std::optional<at::Tensor>& bias);
at::Tensor linear_residual(const at::Tensor& x, const at::Tensor& weight,
                           const at::Tensor& residual);
at::Tensor linear_silu_mul(const at::Tensor& x, const at::Tensor& w_gate, const at::Tensor& w_up);

}  // namespace efficient
}  // namespace torch_gcu
