// Native kernels for the dense contractions: mm, addmm, bmm, baddbmm, addmv
// (codegen/gcu_native_functions.yaml mm.out :452, addmm.out :205, bmm.out
// :260, baddbmm.out :238, addmv.out :206; shape rules of
// shape_inference/blas.cpp).  bf16 /
// fp16 run on the MFMA kernel, fp32 on the VALU kernel; other dtypes take the
// CPU fallback as every unregistered op does.
#include <ATen/ExpandUtils.h>
#include <ATen/Operators.h>
#include <ATen/native/CPUFallback.h>
#include <ATen/native/Resize.h>

#include "aotops.h"
#include "dispatch_util.h"

namespace torch_gcu {
namespace aotops {

namespace {

bool native_dtype(at::ScalarType t) {
  return t == at::kBFloat16 || t == at::kHalf || t == at::kFloat;
}

void check_same_dtype(const at::Tensor& a, const at::Tensor& b, const char* what) {
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "expected ", what,
              " operands to have the same dtype, but got: ", a.scalar_type(), " != ",
              b.scalar_type());
}

void mm_check(const at::Tensor& a, const at::Tensor& b) {
  TORCH_CHECK(a.dim() == 2, "self must be a matrix");
  TORCH_CHECK(b.dim() == 2, "mat2 must be a matrix");
  TORCH_CHECK(a.size(1) == b.size(0), "mat1 and mat2 shapes cannot be multiplied (", a.size(0),
              "x", a.size(1), " and ", b.size(0), "x", b.size(1), ")");
  check_same_dtype(a, b, "mm");
}

void bmm_check(const at::Tensor& a, const at::Tensor& b) {
  TORCH_CHECK(a.dim() == 3, "batch1 must be a 3D tensor");
  TORCH_CHECK(b.dim() == 3, "batch2 must be a 3D tensor");
  TORCH_CHECK(a.size(0) == b.size(0), "batch1 and batch2 must have same number of batches, got ",
              a.size(0), " and ", b.size(0));
  TORCH_CHECK(a.size(2) == b.size(1), "Expected size for first two dimensions of batch2 tensor to be: [",
              a.size(0), ", ", a.size(2), "] but got: [", b.size(0), ", ", b.size(1), "].");
  check_same_dtype(a, b, "bmm");
}

}  // namespace

at::Tensor& mm_out(const at::Tensor& self, const at::Tensor& mat2, at::Tensor& out) {
  mm_check(self, mat2);
  if (!native_dtype(self.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(mm, out)>::call(self, mat2, out);
  at::native::resize_output(out, {self.size(0), mat2.size(1)});
  if (out.numel() == 0) return out;
  const mi_tensor_t o = desc(out), a = desc(self), b = desc(mat2);
  check_mi(mi_mm(&o, &a, &b, mi_stream(out)), "mm");
  return out;
}

at::Tensor mm(const at::Tensor& self, const at::Tensor& mat2) {
  at::Tensor out = at::empty({0}, self.options());
  return mm_out(self, mat2, out);
}

at::Tensor& addmm_out(const at::Tensor& self, const at::Tensor& mat1, const at::Tensor& mat2,
                      const at::Scalar& beta, const at::Scalar& alpha, at::Tensor& out) {
  mm_check(mat1, mat2);
  if (!native_dtype(mat1.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(addmm, out)>::call(
        self, mat1, mat2, beta, alpha, out);
  const std::vector<int64_t> shape{mat1.size(0), mat2.size(1)};
  at::native::resize_output(out, shape);
  if (out.numel() == 0) return out;
  // self broadcasts to the output; a 0-dim CPU self is a scalar
  at::Tensor bias = self;
  if (bias.device().is_cpu()) bias = bias.to(out.device());
  TORCH_CHECK(at::is_expandable_to(bias.sizes(), shape), "addmm: self of shape ", bias.sizes(),
              " cannot be broadcast to ", at::IntArrayRef(shape));
  const mi_tensor_t o = desc(out), s = desc(bias), a = desc(mat1), b = desc(mat2);
  check_mi(mi_addmm(&o, &s, &a, &b, beta.toDouble(), alpha.toDouble(), mi_stream(out)), "addmm");
  return out;
}

at::Tensor addmm(const at::Tensor& self, const at::Tensor& mat1, const at::Tensor& mat2,
                 const at::Scalar& beta, const at::Scalar& alpha) {
  at::Tensor out = at::empty({0}, mat1.options());
  return addmm_out(self, mat1, mat2, beta, alpha, out);
}

at::Tensor& addmm_(at::Tensor& self, const at::Tensor& mat1, const at::Tensor& mat2,
                   const at::Scalar& beta, const at::Scalar& alpha) {
  TORCH_CHECK(self.sizes() == at::IntArrayRef({mat1.size(0), mat2.size(1)}),
              "addmm_: self must have the output's shape");
  // self is both bias and output: compute into a temporary, then copy
  at::Tensor tmp = aotops::addmm(self, mat1, mat2, beta, alpha);
  self.copy_(tmp);
  return self;
}

at::Tensor& bmm_out(const at::Tensor& self, const at::Tensor& mat2, at::Tensor& out) {
  bmm_check(self, mat2);
  if (!native_dtype(self.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(bmm, out)>::call(self, mat2, out);
  at::native::resize_output(out, {self.size(0), self.size(1), mat2.size(2)});
  if (out.numel() == 0) return out;
  const mi_tensor_t o = desc(out), a = desc(self), b = desc(mat2);
  check_mi(mi_bmm(&o, &a, &b, mi_stream(out)), "bmm");
  return out;
}

at::Tensor bmm(const at::Tensor& self, const at::Tensor& mat2) {
  at::Tensor out = at::empty({0}, self.options());
  return bmm_out(self, mat2, out);
}

at::Tensor& baddbmm_out(const at::Tensor& self, const at::Tensor& batch1, const at::Tensor& batch2,
                        const at::Scalar& beta, const at::Scalar& alpha, at::Tensor& out) {
  bmm_check(batch1, batch2);
  if (!native_dtype(batch1.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(baddbmm, out)>::call(
        self, batch1, batch2, beta, alpha, out);
  const std::vector<int64_t> shape{batch1.size(0), batch1.size(1), batch2.size(2)};
  at::native::resize_output(out, shape);
  if (out.numel() == 0) return out;
  at::Tensor bias = self.device().is_cpu() ? self.to(out.device()) : self;
  TORCH_CHECK(at::is_expandable_to(bias.sizes(), shape), "baddbmm: self of shape ", bias.sizes(),
              " cannot be broadcast to ", at::IntArrayRef(shape));
  const mi_tensor_t o = desc(out), s = desc(bias), a = desc(batch1), b = desc(batch2);
  check_mi(mi_baddbmm(&o, &s, &a, &b, beta.toDouble(), alpha.toDouble(), mi_stream(out)),
           "baddbmm");
  return out;
}

at::Tensor baddbmm(const at::Tensor& self, const at::Tensor& batch1, const at::Tensor& batch2,
                   const at::Scalar& beta, const at::Scalar& alpha) {
  at::Tensor out = at::empty({0}, batch1.options());
  return baddbmm_out(self, batch1, batch2, beta, alpha, out);
}

// ---- addmv (addmv.out, codegen/gcu_native_functions.yaml:206); mv reaches it
// through ATen's composite mv -> addmv_ ------------------------------------------

at::Tensor& addmv_out(const at::Tensor& self, const at::Tensor& mat, const at::Tensor& vec,
                      const at::Scalar& beta, const at::Scalar& alpha, at::Tensor& out) {
  TORCH_CHECK(mat.dim() == 2 && vec.dim() == 1 && self.dim() <= 1,
              "vector + matrix @ vector expected, got ", self.dim(), ", ", mat.dim(), ", ",
              vec.dim());
  TORCH_CHECK(mat.size(1) == vec.size(0) && (mat.size(0) == self.numel() || self.numel() == 1),
              "size mismatch, got input (", self.dim() == 0 ? 1 : self.size(0), "), mat (",
              mat.size(0), "x", mat.size(1), "), vec (", vec.size(0), ")");
  check_same_dtype(mat, vec, "addmv");
  if (!native_dtype(mat.scalar_type()))
    return at::native::call_fallback_fn<&gcu_cpu_fallback, ATEN_OP2(addmv, out)>::call(
        self, mat, vec, beta, alpha, out);
  at::native::resize_output(out, {mat.size(0)});
  if (out.numel() == 0) return out;
  at::Tensor bias = self.device().is_cpu() ? self.to(out.device()) : self;
  if (bias.scalar_type() != out.scalar_type() && bias.scalar_type() != at::kFloat)
    bias = bias.to(out.scalar_type());
  const mi_tensor_t o = desc(out), s = desc(bias), a = desc(mat), v = desc(vec);
  check_mi(mi_addmv(&o, &s, &a, &v, beta.toDouble(), alpha.toDouble(), mi_stream(out)), "addmv");
  return out;
}

at::Tensor addmv(const at::Tensor& self, const at::Tensor& mat, const at::Tensor& vec,
                 const at::Scalar& beta, const at::Scalar& alpha) {
  at::Tensor out = at::empty({0}, vec.options());
  return addmv_out(self, mat, vec, beta, alpha, out);
}

at::Tensor& addmv_(at::Tensor& self, const at::Tensor& mat, const at::Tensor& vec,
                   const at::Scalar& beta, const at::Scalar& alpha) {
  TORCH_CHECK(self.dim() == 1 && self.size(0) == mat.size(0),
              "addmv_: self must have the output's shape");
  // self is both bias and output: compute into a temporary, then copy
  at::Tensor tmp = aotops::addmv(self, mat, vec, beta, alpha);
  self.copy_(tmp);
  return self;
}

}  // namespace aotops
}  // namespace torch_gcu
