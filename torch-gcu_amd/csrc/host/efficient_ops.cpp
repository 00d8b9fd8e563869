// efficient_ops: fused entry points outside the aten namespace.
//
// The reference exposes its one efficient op through pybind only
// (torch_gcu/csrc/efficient_ops/ops.cpp:335-342, python/efficient_ops.cpp:12-26);
// here every op is also a dispatcher op in the `torch_gcu` namespace
// (torch.ops.torch_gcu.<op>) with a PrivateUse1 kernel, so it can be captured
// in a GCUGraph and shows up in profiles.  The fused ops are new (RMSNorm,
// RoPE, SiLU-mul, and the matmuls with a residual add or SiLU-mul epilogue);
// int32_indices_index keeps the reference's op.
#include <ATen/ATen.h>
#include <ATen/ExpandUtils.h>
#include <torch/library.h>

#include <sstream>

#include "dispatch_util.h"
#include "efficient_ops.h"

namespace torch_gcu {
namespace efficient {

at::Tensor rms_norm(const at::Tensor& x, const std::optional<at::Tensor>& weight, double eps) {
  TORCH_CHECK(is_gcu(x), "rms_norm: x must be a gcu tensor");
  TORCH_CHECK(x.dim() >= 1, "rms_norm: x must have at least one dim");
  const c10::DeviceGuard g(x.device());
  at::Tensor xc = x;
  if (x.stride(-1) != 1) xc = x.contiguous();
  at::Tensor out = at::empty(x.sizes(), x.options());
  const mi_tensor_t o = desc(out), xi = desc(xc);
  mi_tensor_t w{};
  at::Tensor wc;
  if (weight.has_value() && weight->defined()) {
    TORCH_CHECK(is_gcu(*weight), "rms_norm: weight must be a gcu tensor");
    TORCH_CHECK(weight->numel() == x.size(-1), "rms_norm: weight has ", weight->numel(),
                " elements, expected ", x.size(-1));
    wc = weight->contiguous();
    w = desc(wc);
  }
  mi_status_t st = mi_rms_norm(&o, &xi, wc.defined() ? &w : nullptr, eps, mi_stream(out));
  if (st == MI_ERR_UNSUPPORTED) {
    // rows without a uniform stride: make x dense and retry
    at::Tensor dense = xc.contiguous();
    const mi_tensor_t xd = desc(dense);
    st = mi_rms_norm(&o, &xd, wc.defined() ? &w : nullptr, eps, mi_stream(out));
  }
  check_mi(st, "rms_norm");
  after_op();
  return out;
}

namespace {
void check_qk(const at::Tensor& t, const char* name) {
  TORCH_CHECK(is_gcu(t), "rope: ", name, " must be a gcu tensor");
  TORCH_CHECK(t.dim() == 3, "rope: ", name, " must be [tokens, heads, head_dim]");
}
}  // namespace

void rope_(at::Tensor& q, const std::optional<at::Tensor>& k, const at::Tensor& positions,
           double theta) {
  check_qk(q, "q");
  const c10::DeviceGuard g(q.device());
  at::Tensor pos = is_gcu(positions) ? positions : positions.to(q.device());
  const mi_tensor_t qd = desc(q), pd = desc(pos);
  mi_tensor_t kd{};
  if (k.has_value() && k->defined()) {
    check_qk(*k, "k");
    kd = desc(*k);
  }
  check_mi(mi_rope(&qd, k.has_value() ? &kd : nullptr, &qd, k.has_value() ? &kd : nullptr, &pd,
                   theta, mi_stream(q)),
           "rope");
  after_op();
}

std::tuple<at::Tensor, at::Tensor> rope(const at::Tensor& q, const at::Tensor& k,
                                        const at::Tensor& positions, double theta) {
  check_qk(q, "q");
  check_qk(k, "k");
  const c10::DeviceGuard g(q.device());
  at::Tensor pos = is_gcu(positions) ? positions : positions.to(q.device());
  at::Tensor qo = at::empty(q.sizes(), q.options()), ko = at::empty(k.sizes(), k.options());
  const at::Tensor qi = q.stride(2) == 1 ? q : q.contiguous();
  const at::Tensor ki = k.stride(2) == 1 ? k : k.contiguous();
  const mi_tensor_t qod = desc(qo), kod = desc(ko), qd = desc(qi), kd = desc(ki), pd = desc(pos);
  check_mi(mi_rope(&qod, &kod, &qd, &kd, &pd, theta, mi_stream(qo)), "rope");
  after_op();
  return {qo, ko};
}

at::Tensor silu_mul(const at::Tensor& gate, const at::Tensor& up) {
  TORCH_CHECK(is_gcu(gate) && is_gcu(up), "silu_mul: gate and up must be gcu tensors");
  TORCH_CHECK(gate.scalar_type() == up.scalar_type(), "silu_mul: gate and up dtypes differ");
  const c10::DeviceGuard g(gate.device());
  const auto shape = at::infer_size_dimvector(gate.sizes(), up.sizes());
  at::Tensor out = at::empty(shape, gate.options());
  const mi_tensor_t o = desc(out), gd = desc(gate), ud = desc(up);
  check_mi(mi_silu_mul(&o, &gd, &ud, mi_stream(out)), "silu_mul");
  after_op();
  return out;
}

// Fused matmul epilogues: residual + linear(x, weight), and
// silu(linear(x, w_gate)) * linear(x, w_up), bit for bit what the unfused ops
// give (each product rounded before the add / silu_mul).  x [..., K],
// weights [N, K]; the leading dims of x are flattened into rows.
namespace {
at::Tensor rows2(const at::Tensor& x) {
  at::Tensor r = x.reshape({-1, x.size(-1)});
  return r.stride(-1) == 1 ? r : r.contiguous();
}
at::Tensor weight2(const at::Tensor& w, const char* what) {
  TORCH_CHECK(w.dim() == 2, what, ": weights must be 2-D [N, K]");
  return w.stride(1) == 1 ? w : w.contiguous();
}
}  // namespace

at::Tensor linear_residual(const at::Tensor& x, const at::Tensor& weight,
                           const at::Tensor& residual) {
  TORCH_CHECK(is_gcu(x) && is_gcu(weight) && is_gcu(residual),
              "linear_residual: x, weight and residual must be gcu tensors");
  const c10::DeviceGuard g(x.device());
  const at::Tensor x2 = rows2(x), w = weight2(weight, "linear_residual");
  std::vector<int64_t> shape = x.sizes().vec();
  shape.back() = w.size(0);
  TORCH_CHECK(residual.sizes().vec() == shape, "linear_residual: residual has shape ",
              residual.sizes(), ", expected ", at::IntArrayRef(shape));
  const at::Tensor r2 = rows2(residual);
  at::Tensor out = at::empty({x2.size(0), w.size(0)}, x.options());
  const mi_tensor_t o = desc(out), xd = desc(x2), wd = desc(w), rd = desc(r2);
  check_mi(mi_linear_residual(&o, &xd, &wd, &rd, mi_stream(out)), "linear_residual");
  after_op();
  return out.view(shape);
}

at::Tensor linear_silu_mul(const at::Tensor& x, const at::Tensor& w_gate, const at::Tensor& w_up) {
  TORCH_CHECK(is_gcu(x) && is_gcu(w_gate) && is_gcu(w_up),
              "linear_silu_mul: x, w_gate and w_up must be gcu tensors");
  TORCH_CHECK(w_gate.sizes() == w_up.sizes(), "linear_silu_mul: w_gate and w_up shapes differ");
  const c10::DeviceGuard g(x.device());
  const at::Tensor x2 = rows2(x), wg = weight2(w_gate, "linear_silu_mul"),
                   wu = weight2(w_up, "linear_silu_mul");
  // one row stride for both weights (the fused kernel reads both with it)
  const at::Tensor wu2 = wu.stride(0) == wg.stride(0) ? wu : wu.contiguous();
  const at::Tensor wg2 = wu.stride(0) == wg.stride(0) ? wg : wg.contiguous();
  at::Tensor out = at::empty({x2.size(0), wg2.size(0)}, x.options());
  const mi_tensor_t o = desc(out), xd = desc(x2), gd = desc(wg2), ud = desc(wu2);
  check_mi(mi_linear_silu_mul(&o, &xd, &gd, &ud, mi_stream(out)), "linear_silu_mul");
  after_op();
  std::vector<int64_t> shape = x.sizes().vec();
  shape.back() = wg2.size(0);
  return out.view(shape);
}

// int8 weight-only linear: y = (x @ weight^T) * scales (+ bias), x [..., K]
// bf16/fp16, weight int8 [N, K], scales fp32 [N].
at::Tensor int8_linear(const at::Tensor& x, const at::Tensor& weight, const at::Tensor& scales,
                       const std::optional<at::Tensor>& bias) {
  TORCH_CHECK(is_gcu(x) && is_gcu(weight) && is_gcu(scales),
              "int8_linear: x, weight and scales must be gcu tensors");
  TORCH_CHECK(weight.dim() == 2 && weight.scalar_type() == at::kChar,
              "int8_linear: weight must be int8 [N, K]");
  TORCH_CHECK(x.size(-1) == weight.size(1), "int8_linear: x has ", x.size(-1),
              " features, weight expects ", weight.size(1));
  const c10::DeviceGuard g(x.device());
  const at::Tensor x2 = x.reshape({-1, x.size(-1)});
  const at::Tensor w = weight.is_contiguous() ? weight : weight.contiguous();
  const at::Tensor sc = scales.to(at::kFloat).contiguous();
  at::Tensor out = at::empty({x2.size(0), w.size(0)}, x.options());
  const mi_tensor_t o = desc(out), xd = desc(x2), wd = desc(w), sd = desc(sc);
  mi_tensor_t bd{};
  if (bias.has_value() && bias->defined()) bd = desc(*bias);
  check_mi(mi_int8_linear(&o, &xd, &wd, &sd, &bd, mi_stream(out)), "int8_linear");
  after_op();
  std::vector<int64_t> shape = x.sizes().vec();
  shape.back() = w.size(0);
  return out.view(shape);
}

// Advanced index with int32 indices (torch_gcu/csrc/efficient_ops/ops.cpp:221-342):
// the reference's make_info rules -- index tensors long, int, byte or bool
// (ops.cpp:135-159), masks expanded to their nonzero positions (:101-133),
// the index tensors broadcast together (:230-240), and every one of them int32
// (:266-272), so a mask or an int64 index raises as in the reference -- then
// one mi_index gather that reads the int32 indices as they are.  Index
// tensors on the CPU are range-checked on the host and copied to the device;
// device indices are not (that would need a synchronising read), and an
// out-of-range one writes its out row as zeros.
at::Tensor int32_indices_index(const at::Tensor& self,
                               const c10::List<std::optional<at::Tensor>>& indices) {
  TORCH_CHECK(is_gcu(self), "int32_indices_index: self must be a gcu tensor");
  TORCH_CHECK_INDEX(indices.size() <= (size_t)self.dim(), "too many indices for tensor of dimension ",
                    self.dim(), " (got ", indices.size(), ")");
  const c10::DeviceGuard g(self.device());
  std::vector<at::Tensor> idx;
  for (const auto& oi : indices) {
    const std::optional<at::Tensor> i = oi;
    if (!i.has_value() || !i->defined()) {
      idx.emplace_back();
      continue;
    }
    const auto st = i->scalar_type();
    TORCH_CHECK_INDEX(st == at::kLong || st == at::kInt || st == at::kByte || st == at::kBool,
                      "tensors used as indices must be long, int, byte or bool tensors");
    TORCH_CHECK(i->is_cpu() || i->device() == self.device(),
                "indices should be either on the same device as the indexed tensor (",
                self.device(), ")");
    if (st == at::kByte || st == at::kBool) {
      // a mask: its nonzero positions, one long index per mask dim
      for (int64_t j = 0; j < i->dim(); ++j) {
        const int64_t src_dim = (int64_t)idx.size() + j;
        TORCH_CHECK_INDEX(src_dim < self.dim() && i->size(j) == self.size(src_dim),
                          "The shape of the mask ", i->sizes(), " at index ", j,
                          " does not match the shape of the indexed tensor ", self.sizes(),
                          " at index ", src_dim);
      }
      const at::Tensor nz = i->nonzero();
      for (int64_t j = 0; j < i->dim(); ++j) idx.push_back(nz.select(1, j));
    } else {
      idx.push_back(*i);
    }
  }
  TORCH_CHECK_INDEX(idx.size() <= (size_t)self.dim(), "too many indices for tensor of dimension ",
                    self.dim(), " (got ", idx.size(), ")");
  std::vector<at::Tensor> defined;
  for (const at::Tensor& t : idx)
    if (t.defined()) defined.push_back(t);
  TORCH_CHECK_INDEX(!defined.empty(), "int32_indices_index: at least one index tensor is needed");
  std::vector<at::Tensor> bcast;
  try {
    bcast = at::expand_outplace(defined);
  } catch (const std::exception&) {
    std::ostringstream os;
    for (size_t k = 0; k < defined.size(); ++k) os << (k ? ", " : "") << defined[k].sizes();
    TORCH_CHECK_INDEX(false, "shape mismatch: indexing tensors could not be broadcast together "
                      "with shapes ", os.str());
  }
  for (const at::Tensor& t : bcast)
    TORCH_CHECK_INDEX(t.scalar_type() == at::kInt, "indice error, should be int in gcu_index ",
                      "but got ", t.scalar_type());
  // the device view of each index; CPU indices range-checked here
  std::vector<at::Tensor> dev(idx.size());
  std::vector<int64_t> kdim;
  for (size_t d = 0, k = 0; d < idx.size(); ++d) {
    if (!idx[d].defined()) continue;
    at::Tensor t = bcast[k++];
    if (t.is_cpu() && t.numel() > 0) {
      const int64_t n = self.size((int64_t)d);
      const int64_t lo = t.min().item<int64_t>(), hi = t.max().item<int64_t>();
      const int64_t bad = lo < -n ? lo : hi;
      TORCH_CHECK_INDEX(lo >= -n && hi < n, "index ", bad, " is out of bounds for dimension ", d,
                        " with size ", n);
    }
    dev[d] = t.is_cpu() ? t.contiguous().to(self.device()) : t;
    kdim.push_back((int64_t)d);
  }
  // out shape: B in place of adjacent indexed dims, else in front
  bool adjacent = true;
  for (size_t k = 1; k < kdim.size(); ++k) adjacent = adjacent && kdim[k] == kdim[k - 1] + 1;
  const auto bshape = bcast[0].sizes();
  std::vector<int64_t> shape;
  if (!adjacent) shape.insert(shape.end(), bshape.begin(), bshape.end());
  for (int64_t d = 0; d < self.dim(); ++d) {
    const bool indexed = d < (int64_t)idx.size() && idx[d].defined();
    if (!indexed) {
      shape.push_back(self.size(d));
    } else if (adjacent && d == kdim[0]) {
      shape.insert(shape.end(), bshape.begin(), bshape.end());
    }
  }
  TORCH_CHECK((int64_t)shape.size() <= MI_MAX_DIMS, "int32_indices_index: result has ",
              shape.size(), " dims, at most ", MI_MAX_DIMS, " are supported");
  at::Tensor out = at::empty(shape, self.options());
  if (out.numel() == 0) {
    for (int64_t d : kdim)
      TORCH_CHECK_INDEX(self.size(d) > 0 || bcast[0].numel() == 0,
                        "index is out of bounds for dimension with size 0");
    return out;
  }
  const mi_tensor_t od = desc(out), sd = desc(self);
  std::vector<mi_tensor_t> descs(idx.size());
  std::vector<const mi_tensor_t*> ptrs(idx.size(), nullptr);
  for (size_t d = 0; d < idx.size(); ++d) {
    if (!dev[d].defined()) continue;
    descs[d] = desc(dev[d]);
    ptrs[d] = &descs[d];
  }
  check_mi(mi_index(&od, &sd, ptrs.data(), (int32_t)ptrs.size(), mi_stream(out)),
           "int32_indices_index");
  after_op();
  return out;
}

}  // namespace efficient
}  // namespace torch_gcu

TORCH_LIBRARY(torch_gcu, m) {
  m.def("rms_norm(Tensor x, Tensor? weight, float eps=1e-06) -> Tensor");
  m.def("rope(Tensor q, Tensor k, Tensor positions, float theta=10000.0) -> (Tensor, Tensor)");
  m.def("rope_(Tensor(a!) q, Tensor(b!)? k, Tensor positions, float theta=10000.0) -> ()");
  m.def("silu_mul(Tensor gate, Tensor up) -> Tensor");
  m.def("int32_indices_index(Tensor self, Tensor?[] indices) -> Tensor");
  m.def("int8_linear(Tensor x, Tensor weight, Tensor scales, Tensor? bias=None) -> Tensor");
  m.def("linear_residual(Tensor x, Tensor weight, Tensor residual) -> Tensor");
  m.def("linear_silu_mul(Tensor x, Tensor w_gate, Tensor w_up) -> Tensor");
}

TORCH_LIBRARY_IMPL(torch_gcu, PrivateUse1, m) {
  m.impl("rms_norm", TORCH_FN(torch_gcu::efficient::rms_norm));
  m.impl("rope", TORCH_FN(torch_gcu::efficient::rope));
  m.impl("rope_", TORCH_FN(torch_gcu::efficient::rope_));
  m.impl("silu_mul", TORCH_FN(torch_gcu::efficient::silu_mul));
  m.impl("int32_indices_index", TORCH_FN(torch_gcu::efficient::int32_indices_index));
  m.impl("int8_linear", TORCH_FN(torch_gcu::efficient::int8_linear));
  m.impl("linear_residual", TORCH_FN(torch_gcu::efficient::linear_residual));
  m.impl("linear_silu_mul", TORCH_FN(torch_gcu::efficient::linear_silu_mul));
}
