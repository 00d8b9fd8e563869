// Scaled dot-product attention on the gcu device.
//
// F.scaled_dot_product_attention asks the device's _fused_sdp_choice stub for
// a backend (the reference overrides the composite op and picks flash first,
// torch_gcu/csrc/aten/RegisterSPDA.cpp:137-273); here the stub answers
// "overrideable" whenever the flash kernel applies (bf16/fp16, head_dim 64 or
// 128, no attention mask, no dropout) and "math" otherwise, which decomposes
// into the native bmm / softmax kernels.  The overrideable op and
// _scaled_dot_product_flash_attention (torch_gcu/csrc/aten/GCUNativeFunctions.cpp:49-102,
// gcu_attention.cpp:21-79) both run mi_flash_attention_fwd.
#include <ATen/SDPBackend.h>
#include <ATen/core/grad_mode.h>
#include <ATen/native/DispatchStub.h>
#include <ATen/native/transformers/attention.h>

#include <cmath>

#include "aotops.h"
#include "dispatch_util.h"

namespace torch_gcu {
namespace aotops {

namespace {

// The shapes the flash kernel takes: 4-D bf16/fp16 q/k/v of one batch size,
// k and v of one sequence length, head_dim 64 or 128, no mask, no dropout,
// and either as many k/v heads as query heads or, with enable_gqa, a number
// that divides them (ATen's math path raises for H != Hk without it).
bool flash_applies(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                   bool has_mask, double dropout_p, bool enable_gqa) {
  if (has_mask || dropout_p > 0.0) return false;
  if (q.dim() != 4 || k.dim() != 4 || v.dim() != 4) return false;
  const auto dt = q.scalar_type();
  if ((dt != at::kBFloat16 && dt != at::kHalf) || k.scalar_type() != dt || v.scalar_type() != dt)
    return false;
  const int64_t d = q.size(3);
  if ((d != 64 && d != 128) || k.size(3) != d || v.size(3) != d) return false;
  if (q.size(0) != k.size(0) || k.size(0) != v.size(0) || k.size(2) != v.size(2)) return false;
  if (k.size(1) != v.size(1) || k.size(1) == 0 || q.size(1) % k.size(1) != 0) return false;
  if (!enable_gqa && q.size(1) != k.size(1)) return false;
  return is_gcu(q) && is_gcu(k) && is_gcu(v);
}

// The kernel is forward only: when autograd will need gradients of q, k or
// v, the math path runs instead (its bmm / softmax ops have native backward
// kernels), as the reference selects by whether the logsumexp must be kept
// for a backward pass (torch_gcu/csrc/aten/RegisterSPDA.cpp:422-428).
bool needs_grad(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  return at::GradMode::is_enabled() && (q.requires_grad() || k.requires_grad() || v.requires_grad());
}

// Makes head_dim contiguous and every row 16-byte aligned.
at::Tensor rows_aligned(const at::Tensor& t) {
  const bool ok = t.stride(3) == 1 && t.stride(2) % 8 == 0 && t.stride(1) % 8 == 0 &&
                  t.stride(0) % 8 == 0 && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
  return ok ? t : t.contiguous();
}

std::tuple<at::Tensor, at::Tensor> run_flash(const at::Tensor& q, const at::Tensor& k,
                                             const at::Tensor& v, bool is_causal,
                                             std::optional<double> scale) {
  const c10::DeviceGuard g(q.device());
  const at::Tensor qa = rows_aligned(q), ka = rows_aligned(k), va = rows_aligned(v);
  // [B, S, H, D] storage viewed as [B, H, S, D]: the usual next step,
  // out.transpose(1, 2).reshape(B, S, H * D), is then a view, not a copy
  at::Tensor out =
      at::empty({q.size(0), q.size(2), q.size(1), q.size(3)}, q.options()).transpose(1, 2);
  at::Tensor lse = at::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(at::kFloat));
  const double sc = scale.has_value() ? *scale : 1.0 / std::sqrt((double)q.size(3));
  const mi_tensor_t o = desc(out), l = desc(lse), qd = desc(qa), kd = desc(ka), vd = desc(va);
  check_mi(mi_flash_attention_fwd(&o, &l, &qd, &kd, &vd, is_causal ? 1 : 0, sc, mi_stream(out)),
           "flash_attention_fwd");
  return {out, lse};
}

int64_t gcu_fused_sdp_choice(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                             const std::optional<at::Tensor>& attn_mask, double dropout_p,
                             bool is_causal, std::optional<double> scale, bool enable_gqa) {
  (void)is_causal;
  (void)scale;
  const bool has_mask = attn_mask.has_value() && attn_mask->defined();
  if (!needs_grad(q, k, v) && flash_applies(q, k, v, has_mask, dropout_p, enable_gqa))
    return static_cast<int64_t>(at::SDPBackend::overrideable);
  return static_cast<int64_t>(at::SDPBackend::math);
}

}  // namespace

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, c10::SymInt, c10::SymInt, at::Tensor,
           at::Tensor, at::Tensor>
_scaled_dot_product_fused_attention_overrideable(const at::Tensor& query, const at::Tensor& key,
                                                 const at::Tensor& value,
                                                 const std::optional<at::Tensor>& attn_bias,
                                                 double dropout_p, bool is_causal,
                                                 bool return_debug_mask,
                                                 std::optional<double> scale) {
  const bool has_mask = attn_bias.has_value() && attn_bias->defined();
  // called directly (not through the backend choice), grouped k/v heads are
  // taken as they come, as the fused ops of ATen's other backends take them
  TORCH_CHECK(flash_applies(query, key, value, has_mask, dropout_p, /*enable_gqa=*/true),
              "gcu fused attention: needs bf16/fp16 4-D q/k/v of one batch size with head_dim "
              "64 or 128, k and v of one length, query heads a multiple of k/v heads, no "
              "attention mask and no dropout");
  TORCH_CHECK(!return_debug_mask, "gcu fused attention: return_debug_mask is not supported");
  auto [out, lse] = run_flash(query, key, value, is_causal, scale);
  const auto empty = at::empty({0}, query.options().dtype(at::kLong));
  return {out, lse, empty, empty, c10::SymInt(query.size(2)), c10::SymInt(key.size(2)), empty,
          empty, at::empty({0}, query.options())};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, c10::SymInt, c10::SymInt, at::Tensor,
           at::Tensor, at::Tensor>
_scaled_dot_product_flash_attention(const at::Tensor& query, const at::Tensor& key,
                                    const at::Tensor& value, double dropout_p, bool is_causal,
                                    bool return_debug_mask, std::optional<double> scale) {
  return aotops::_scaled_dot_product_fused_attention_overrideable(
      query, key, value, std::optional<at::Tensor>(), dropout_p, is_causal, return_debug_mask,
      scale);
}

}  // namespace aotops
}  // namespace torch_gcu

namespace at::native {
REGISTER_PRIVATEUSE1_DISPATCH(_fused_sdp_choice_stub, &torch_gcu::aotops::gcu_fused_sdp_choice)
}
