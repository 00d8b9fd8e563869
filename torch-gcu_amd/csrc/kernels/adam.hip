// Fused AdamW step over lists of tensors: torch._fused_adamw_ (both the float
// and the tensor lr overloads).
//
// Per element, in fp32 for fp32/bf16/fp16 tensors and fp64 for fp64 ones
// (the AdamW of Loshchilov and Hutter with PyTorch's fused-kernel order):
//   g  = grad / grad_scale              (grad_scale given: g is written back)
//   g  = -g                             (maximize; not written back)
//   p  = p - lr * weight_decay * p
//   m  = beta1 * m + (1 - beta1) * g
//   v  = beta2 * v + (1 - beta2) * g * g
//   vm = max(vm, v)                     (amsgrad)
//   p  = p - (lr / bc1) * m / (sqrt(amsgrad ? vm : v) / sqrt(bc2) + eps)
// with bc1 = 1 - beta1^step, bc2 = 1 - beta2^step from the tensor's own
// step count (read, not advanced: the optimizer advances it).  found_inf = 1
// skips the whole step.  lr, the steps, grad_scale and found_inf are read
// on the device, so a step can be captured in a graph.
//
// HBM-bound: per element 4 (5 with amsgrad) reads and 3 (4) writes, 5 / 6 with
// the grad written back.  One launch covers up to kAdamMax tensors: every
// tensor is cut into chunks of kAdamBlock * kAdamPieces 16-byte pieces, one
// chunk per block, and a block finds its tensor by binary search in the
// table passed as kernel arguments.  A lane issues the non-temporal loads of
// all its pieces (16 x 16 B for fp32 without amsgrad) before it computes and
// stores (5.76 TB/s on one Llama-7B layer's fp32 parameters, against 5.40
// with two cached pieces).  Tensors whose buffers are not all 16-byte
// aligned, and the ragged end of each tensor, go element by element.
#include "iter.h"

namespace mi {
namespace {

constexpr int kAdamBlock = 256;
constexpr int kAdamPieces = 4;  // 16-byte pieces per lane and operand
constexpr int kAdamMax = 32;    // tensors per launch

struct AdamTensor {
  void* p;
  void* g;
  void* m;
  void* v;
  void* vm;
  const float* step;
  int64_t n;
  int64_t first_block;
  int32_t vec_ok;
};

struct AdamArgs {
  AdamTensor t[kAdamMax];
  int32_t count;
  int32_t amsgrad, maximize;
  int32_t lr_dtype;  // of *lr_ptr
  const void* lr_ptr;
  double lr, beta1, beta2, wd, eps;
  const float* grad_scale;
  const float* found_inf;
};

template <typename Acc>
struct AdamConsts {
  Acc lr_wd, b1, omb1, b2, omb2, step_size, bc2_sqrt, eps, scale;
  bool scaled, maximize, amsgrad;
};

template <typename Acc, bool AMS>
__device__ __forceinline__ void adam_elem(const AdamConsts<Acc>& c, Acc& p, Acc& g, Acc& m, Acc& v,
                                          Acc& vm) {
  if (c.scaled) g = g / c.scale;
  const Acc gd = c.maximize ? -g : g;
  p = p - c.lr_wd * p;
  m = c.b1 * m + c.omb1 * gd;
  v = c.b2 * v + c.omb2 * gd * gd;
  Acc den;
  if (AMS) {
    vm = vm > v ? vm : v;
    den = sqrt(vm) / c.bc2_sqrt + c.eps;
  } else {
    den = sqrt(v) / c.bc2_sqrt + c.eps;
  }
  p = p - c.step_size * m / den;
}

template <typename Tag, bool AMS>
__global__ __launch_bounds__(kAdamBlock) void adamw_kernel(AdamArgs a) {
  typedef typename Num<Tag>::storage St;
  typedef typename Num<Tag>::acc Acc;
  constexpr int VEC = 16 / sizeof(St);
  constexpr int64_t kChunk = (int64_t)kAdamBlock * kAdamPieces * VEC;
  if (a.found_inf != nullptr && *a.found_inf == 1.0f) return;
  int lo = 0, hi = a.count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)blockIdx.x >= a.t[mid].first_block) lo = mid;
    else hi = mid - 1;
  }
  const AdamTensor& t = a.t[lo];
  const double lr = a.lr_ptr == nullptr ? a.lr
                    : a.lr_dtype == MI_F64 ? *(const double*)a.lr_ptr
                                           : (double)*(const float*)a.lr_ptr;
  const double step = (double)*t.step;
  AdamConsts<Acc> c;
  const Acc bc1 = (Acc)(1.0 - pow(a.beta1, step));
  c.bc2_sqrt = (Acc)sqrt(1.0 - pow(a.beta2, step));
  c.step_size = (Acc)(lr / (double)bc1);
  c.lr_wd = (Acc)(lr * a.wd);
  c.b1 = (Acc)a.beta1;
  c.omb1 = (Acc)(1.0 - a.beta1);
  c.b2 = (Acc)a.beta2;
  c.omb2 = (Acc)(1.0 - a.beta2);
  c.eps = (Acc)a.eps;
  c.scaled = a.grad_scale != nullptr;
  c.scale = c.scaled ? (Acc)*a.grad_scale : (Acc)1;
  c.maximize = a.maximize != 0;
  St* P = (St*)t.p;
  St* G = (St*)t.g;
  St* M = (St*)t.m;
  St* V = (St*)t.v;
  St* VM = (St*)t.vm;
  const int64_t base = ((int64_t)blockIdx.x - t.first_block) * kChunk;
  if (t.vec_ok) {
    union U {
      uint4 u;
      St s[VEC];
    };
    // every piece's loads are issued before the first store (the compiler
    // cannot move a load of one buffer past a store to another)
    U up[kAdamPieces], ug[kAdamPieces], um[kAdamPieces], uv[kAdamPieces], uvm[kAdamPieces];
#pragma unroll
    for (int k = 0; k < kAdamPieces; ++k) {
      const int64_t e = base + ((int64_t)k * kAdamBlock + threadIdx.x) * VEC;
      if (e + VEC <= t.n) {
        up[k].u = ld_stream((const uint4*)(P + e));
        ug[k].u = ld_stream((const uint4*)(G + e));
        um[k].u = ld_stream((const uint4*)(M + e));
        uv[k].u = ld_stream((const uint4*)(V + e));
        if (AMS) uvm[k].u = ld_stream((const uint4*)(VM + e));
      }
    }
#pragma unroll
    for (int k = 0; k < kAdamPieces; ++k) {
      const int64_t e = base + ((int64_t)k * kAdamBlock + threadIdx.x) * VEC;
      if (e + VEC <= t.n) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          Acc p = Num<Tag>::load(up[k].s[q]), g = Num<Tag>::load(ug[k].s[q]);
          Acc m = Num<Tag>::load(um[k].s[q]), v = Num<Tag>::load(uv[k].s[q]);
          Acc vm = AMS ? Num<Tag>::load(uvm[k].s[q]) : (Acc)0;
          adam_elem<Acc, AMS>(c, p, g, m, v, vm);
          up[k].s[q] = Num<Tag>::store(p);
          ug[k].s[q] = Num<Tag>::store(g);
          um[k].s[q] = Num<Tag>::store(m);
          uv[k].s[q] = Num<Tag>::store(v);
          if (AMS) uvm[k].s[q] = Num<Tag>::store(vm);
        }
        st_stream((uint4*)(P + e), up[k].u);
        if (c.scaled) st_stream((uint4*)(G + e), ug[k].u);
        st_stream((uint4*)(M + e), um[k].u);
        st_stream((uint4*)(V + e), uv[k].u);
        if (AMS) st_stream((uint4*)(VM + e), uvm[k].u);
      } else {
        for (int64_t i = e; i < t.n && i < e + VEC; ++i) {
          Acc p = Num<Tag>::load(P[i]), g = Num<Tag>::load(G[i]);
          Acc m = Num<Tag>::load(M[i]), v = Num<Tag>::load(V[i]);
          Acc vm = AMS ? Num<Tag>::load(VM[i]) : (Acc)0;
          adam_elem<Acc, AMS>(c, p, g, m, v, vm);
          P[i] = Num<Tag>::store(p);
          if (c.scaled) G[i] = Num<Tag>::store(g);
          M[i] = Num<Tag>::store(m);
          V[i] = Num<Tag>::store(v);
          if (AMS) VM[i] = Num<Tag>::store(vm);
        }
      }
    }
    return;
  }
  for (int64_t k = threadIdx.x; k < kChunk; k += kAdamBlock) {
    const int64_t i = base + k;
    if (i >= t.n) break;
    Acc p = Num<Tag>::load(P[i]), g = Num<Tag>::load(G[i]);
    Acc m = Num<Tag>::load(M[i]), v = Num<Tag>::load(V[i]);
    Acc vm = AMS ? Num<Tag>::load(VM[i]) : (Acc)0;
    adam_elem<Acc, AMS>(c, p, g, m, v, vm);
    P[i] = Num<Tag>::store(p);
    if (c.scaled) G[i] = Num<Tag>::store(g);
    M[i] = Num<Tag>::store(m);
    V[i] = Num<Tag>::store(v);
    if (AMS) VM[i] = Num<Tag>::store(vm);
  }
}

// Dense in some dim order (no gaps, no overlap): the elements fill
// [data, data + numel) exactly.
bool dense_any_order(const mi_tensor_t& t) {
  int idx[MI_MAX_DIMS];
  int k = 0;
  for (int d = 0; d < t.ndim; ++d)
    if (t.sizes[d] != 1) idx[k++] = d;
  for (int a = 1; a < k; ++a)
    for (int b = a; b > 0 && t.strides[idx[b]] < t.strides[idx[b - 1]]; --b) {
      const int x = idx[b];
      idx[b] = idx[b - 1];
      idx[b - 1] = x;
    }
  int64_t expect = 1;
  for (int a = 0; a < k; ++a) {
    if (t.strides[idx[a]] != expect) return false;
    expect *= t.sizes[idx[a]];
  }
  return true;
}

bool same_layout(const mi_tensor_t& a, const mi_tensor_t& b) {
  if (a.ndim != b.ndim || a.dtype != b.dtype) return false;
  for (int d = 0; d < a.ndim; ++d)
    if (a.sizes[d] != b.sizes[d] || (a.sizes[d] != 1 && a.strides[d] != b.strides[d])) return false;
  return true;
}

mi_status_t check_scalar(const mi_tensor_t* t, const char* name, bool allow_f64) {
  MI_RETURN_IF(validate(t, name));
  MI_CHECK_ARG(numel(*t) == 1, "fused_adamw: %s must have one element, got %lld", name,
               (long long)numel(*t));
  MI_CHECK_ARG(t->dtype == MI_F32 || (allow_f64 && t->dtype == MI_F64),
               "fused_adamw: %s must be float32%s, got %s", name, allow_f64 ? " or float64" : "",
               dtype_name(t->dtype));
  return MI_OK;
}

template <typename Tag>
mi_status_t launch_adam(AdamArgs& a, bool ams, hipStream_t s, int64_t blocks) {
  if (ams)
    hipLaunchKernelGGL((adamw_kernel<Tag, true>), dim3((unsigned)blocks), dim3(kAdamBlock), 0, s, a);
  else
    hipLaunchKernelGGL((adamw_kernel<Tag, false>), dim3((unsigned)blocks), dim3(kAdamBlock), 0, s, a);
  return check_launch("fused_adamw");
}

// _foreach_add_.Scalar / _foreach_mul_.Scalar / _foreach_mul_.Tensor: every
// tensor of a list += or *= one value, in place (the optimizer's step-count
// advance, gradient clipping's scale).  One launch per kForeachMax tensors,
// the table in kernel arguments as for AdamW; the value is a host double or
// a one-element fp32 device tensor read by the kernel; the arithmetic in fp32
// (fp64 for fp64), rounded once.
constexpr int kForeachMax = 64;
constexpr int kForeachChunk = 1024;  // elements per block

struct ForeachTensor {
  void* p;
  int64_t n;
  int64_t first_block;
};

struct ForeachArgs {
  ForeachTensor t[kForeachMax];
  int32_t count;
  double value;
};

enum ForeachOp { FE_ADD = 0, FE_MUL = 1 };

template <typename Tag, int OP>
__global__ __launch_bounds__(256) void foreach_scalar_kernel(ForeachArgs a, const float* dev_value) {
  typedef typename Num<Tag>::storage St;
  typedef typename Num<Tag>::acc Acc;
  int lo = 0, hi = a.count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)blockIdx.x >= a.t[mid].first_block) lo = mid;
    else hi = mid - 1;
  }
  const ForeachTensor& t = a.t[lo];
  St* p = (St*)t.p;
  const Acc v = dev_value != nullptr ? (Acc)*dev_value : (Acc)a.value;
  const int64_t base = ((int64_t)blockIdx.x - t.first_block) * kForeachChunk;
  for (int k = threadIdx.x; k < kForeachChunk; k += 256) {
    const int64_t i = base + k;
    if (i >= t.n) break;
    const Acc x = Num<Tag>::load(p[i]);
    p[i] = Num<Tag>::store(as_rounded(OP == FE_ADD ? x + v : x * v));
  }
}

// _amp_foreach_non_finite_check_and_unscale_: every element *= inv_scale
// (left as it is when inv_scale is 1), and found_inf = 1 when any element
// was inf or NaN.  Every block that saw one stores the same 1.0, so the
// stores need no ordering.
template <typename Tag>
__global__ __launch_bounds__(256) void amp_unscale_kernel(ForeachArgs a, float* found_inf,
                                                          const float* inv_scale) {
  typedef typename Num<Tag>::storage St;
  typedef typename Num<Tag>::acc Acc;
  int lo = 0, hi = a.count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)blockIdx.x >= a.t[mid].first_block) lo = mid;
    else hi = mid - 1;
  }
  const ForeachTensor& t = a.t[lo];
  St* p = (St*)t.p;
  const float sc = *inv_scale;
  bool bad = false;
  const int64_t base = ((int64_t)blockIdx.x - t.first_block) * kForeachChunk;
  for (int k = threadIdx.x; k < kForeachChunk; k += 256) {
    const int64_t i = base + k;
    if (i >= t.n) break;
    const Acc v = Num<Tag>::load(p[i]);
    if (!isfinite(v)) bad = true;
    if (sc != 1.0f) p[i] = Num<Tag>::store(as_rounded(v * (Acc)sc));
  }
  if (bad) *found_inf = 1.0f;
}

template <typename Tag>
mi_status_t launch_foreach(ForeachArgs& a, int64_t blocks, hipStream_t s, int op,
                           const float* dev_value, float* found_inf, const float* inv_scale) {
  if (found_inf != nullptr) {
    hipLaunchKernelGGL((amp_unscale_kernel<Tag>), dim3((unsigned)blocks), dim3(256), 0, s, a,
                       found_inf, inv_scale);
    return check_launch("amp_unscale");
  }
  if (op == FE_MUL)
    hipLaunchKernelGGL((foreach_scalar_kernel<Tag, FE_MUL>), dim3((unsigned)blocks), dim3(256), 0,
                       s, a, dev_value);
  else
    hipLaunchKernelGGL((foreach_scalar_kernel<Tag, FE_ADD>), dim3((unsigned)blocks), dim3(256), 0,
                       s, a, dev_value);
  return check_launch("foreach_scalar");
}

// The multi-tensor walk shared by the list ops: found_inf == NULL means
// "add or multiply by the value", else "unscale and check".
mi_status_t foreach_run(const mi_tensor_t* const* tensors, int32_t n_tensors, double value, int op,
                        const float* dev_value, float* found_inf, const float* inv_scale,
                        const char* what, hipStream_t stream) {
  MI_CHECK_ARG(n_tensors >= 0 && (n_tensors == 0 || tensors != nullptr), "%s: bad tensor list", what);
  if (n_tensors == 0) return MI_OK;
  const int dt = tensors[0] != nullptr ? tensors[0]->dtype : -1;
  MI_CHECK_ARG(dt == MI_F32 || dt == MI_BF16 || dt == MI_F16 || dt == MI_F64,
               "%s: tensors must be float32, bfloat16, float16 or float64", what);
  ForeachArgs a{};
  a.value = value;
  int k = 0;
  int64_t blocks = 0;
  auto flush = [&]() -> mi_status_t {
    if (k == 0) return MI_OK;
    a.count = k;
    mi_status_t st;
    switch (dt) {
      case MI_F32: st = launch_foreach<float>(a, blocks, stream, op, dev_value, found_inf, inv_scale); break;
      case MI_BF16: st = launch_foreach<BF16>(a, blocks, stream, op, dev_value, found_inf, inv_scale); break;
      case MI_F16: st = launch_foreach<F16>(a, blocks, stream, op, dev_value, found_inf, inv_scale); break;
      default: st = launch_foreach<double>(a, blocks, stream, op, dev_value, found_inf, inv_scale); break;
    }
    k = 0;
    blocks = 0;
    return st;
  };
  for (int i = 0; i < n_tensors; ++i) {
    const mi_tensor_t* t = tensors[i];
    MI_RETURN_IF(validate(t, "tensor"));
    MI_CHECK_ARG(t->dtype == dt, "%s: tensor %d is %s, tensor 0 is %s", what, i,
                 dtype_name(t->dtype), dtype_name(dt));
    const int64_t n = numel(*t);
    if (n == 0) continue;
    MI_CHECK_ARG(dense_any_order(*t), "%s: tensor %d is not dense", what, i);
    a.t[k].p = t->data;
    a.t[k].n = n;
    a.t[k].first_block = blocks;
    blocks += (n + kForeachChunk - 1) / kForeachChunk;
    MI_CHECK_ARG(blocks <= 0x7fffffffLL, "%s: too many blocks", what);
    if (++k == kForeachMax) MI_RETURN_IF(flush());
  }
  return flush();
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status_t mi_foreach_add_scalar(const mi_tensor_t* const* tensors, int32_t n_tensors,
                                             double value, mi_stream_t stream_) {
  clear_error();
  return foreach_run(tensors, n_tensors, value, FE_ADD, nullptr, nullptr, nullptr,
                     "foreach_add_scalar", (hipStream_t)stream_);
}

extern "C" mi_status_t mi_foreach_mul_scalar(const mi_tensor_t* const* tensors, int32_t n_tensors,
                                             double value, const mi_tensor_t* scalar,
                                             mi_stream_t stream_) {
  clear_error();
  const float* dev = nullptr;
  if (scalar != nullptr) {
    MI_RETURN_IF(validate(scalar, "scalar"));
    MI_CHECK_ARG(numel(*scalar) == 1 && scalar->dtype == MI_F32,
                 "foreach_mul_scalar: scalar must be a one-element float32 tensor");
    dev = (const float*)scalar->data;
  }
  return foreach_run(tensors, n_tensors, value, FE_MUL, dev, nullptr, nullptr,
                     "foreach_mul_scalar", (hipStream_t)stream_);
}

extern "C" mi_status_t mi_amp_unscale(const mi_tensor_t* const* tensors, int32_t n_tensors,
                                      const mi_tensor_t* found_inf, const mi_tensor_t* inv_scale,
                                      mi_stream_t stream_) {
  clear_error();
  MI_RETURN_IF(validate(found_inf, "found_inf"));
  MI_RETURN_IF(validate(inv_scale, "inv_scale"));
  MI_CHECK_ARG(numel(*found_inf) == 1 && found_inf->dtype == MI_F32,
               "amp_unscale: found_inf must be a one-element float32 tensor");
  MI_CHECK_ARG(numel(*inv_scale) == 1 && inv_scale->dtype == MI_F32,
               "amp_unscale: inv_scale must be a one-element float32 tensor");
  return foreach_run(tensors, n_tensors, 0.0, FE_MUL, nullptr, (float*)found_inf->data,
                     (const float*)inv_scale->data, "amp_unscale", (hipStream_t)stream_);
}

// GradScaler's scale update, one lane: on inf / NaN the scale backs off and
// the growth count restarts; after growth_interval clean steps the scale
// grows (kept only when the grown value is finite).  The products are taken
// in fp64 and rounded once to fp32.
__global__ __launch_bounds__(64) void amp_update_scale_kernel(float* scale, int32_t* tracker,
                                                              const float* found_inf,
                                                              double growth, double backoff,
                                                              int64_t interval) {
  if (threadIdx.x != 0) return;
  if (*found_inf != 0.0f) {
    *scale = (float)((double)*scale * backoff);
    *tracker = 0;
    return;
  }
  const int64_t good = (int64_t)*tracker + 1;
  if (good == interval) {
    const float grown = (float)((double)*scale * growth);
    if (isfinite(grown)) *scale = grown;
    *tracker = 0;
  } else {
    *tracker = (int32_t)good;
  }
}

extern "C" mi_status_t mi_amp_update_scale(const mi_tensor_t* scale,
                                           const mi_tensor_t* growth_tracker,
                                           const mi_tensor_t* found_inf, double growth_factor,
                                           double backoff_factor, int64_t growth_interval,
                                           mi_stream_t stream_) {
  clear_error();
  MI_RETURN_IF(validate(scale, "scale"));
  MI_RETURN_IF(validate(growth_tracker, "growth_tracker"));
  MI_RETURN_IF(validate(found_inf, "found_inf"));
  MI_CHECK_ARG(numel(*scale) == 1 && scale->dtype == MI_F32,
               "amp_update_scale: current_scale must be a one-element float32 tensor");
  MI_CHECK_ARG(numel(*growth_tracker) == 1 && growth_tracker->dtype == MI_I32,
               "amp_update_scale: growth_tracker must be a one-element int32 tensor");
  MI_CHECK_ARG(numel(*found_inf) == 1 && found_inf->dtype == MI_F32,
               "amp_update_scale: found_inf must be a one-element float32 tensor");
  hipLaunchKernelGGL(amp_update_scale_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream_,
                     (float*)scale->data, (int32_t*)growth_tracker->data,
                     (const float*)found_inf->data, growth_factor, backoff_factor, growth_interval);
  return check_launch("amp_update_scale");
}

extern "C" mi_status_t mi_fused_adamw(
    const mi_tensor_t* const* params, const mi_tensor_t* const* grads,
    const mi_tensor_t* const* exp_avgs, const mi_tensor_t* const* exp_avg_sqs,
    const mi_tensor_t* const* max_exp_avg_sqs, const mi_tensor_t* const* state_steps,
    int32_t n_tensors, const mi_tensor_t* lr_tensor, const mi_adamw_hparams_t* hp,
    const mi_tensor_t* grad_scale, const mi_tensor_t* found_inf, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_CHECK_ARG(hp != nullptr, "fused_adamw: hyper-parameters are NULL");
  MI_CHECK_ARG(n_tensors >= 0, "fused_adamw: negative tensor count");
  if (n_tensors == 0) return MI_OK;
  MI_CHECK_ARG(params && grads && exp_avgs && exp_avg_sqs && state_steps,
               "fused_adamw: a tensor list is NULL");
  const bool ams = hp->amsgrad != 0;
  MI_CHECK_ARG(!ams || max_exp_avg_sqs != nullptr,
               "fused_adamw: amsgrad needs max_exp_avg_sqs");
  if (lr_tensor != nullptr) MI_RETURN_IF(check_scalar(lr_tensor, "lr", true));
  if (grad_scale != nullptr) MI_RETURN_IF(check_scalar(grad_scale, "grad_scale", false));
  if (found_inf != nullptr) MI_RETURN_IF(check_scalar(found_inf, "found_inf", false));
  const int dt = params[0] != nullptr ? params[0]->dtype : -1;
  MI_CHECK_ARG(dt == MI_F32 || dt == MI_BF16 || dt == MI_F16 || dt == MI_F64,
               "fused_adamw: params must be float32, bfloat16, float16 or float64");
  AdamArgs a{};
  a.amsgrad = ams;
  a.maximize = hp->maximize != 0;
  a.lr_ptr = lr_tensor != nullptr ? lr_tensor->data : nullptr;
  a.lr_dtype = lr_tensor != nullptr ? lr_tensor->dtype : MI_F64;
  a.lr = hp->lr;
  a.beta1 = hp->beta1;
  a.beta2 = hp->beta2;
  a.wd = hp->weight_decay;
  a.eps = hp->eps;
  a.grad_scale = grad_scale != nullptr ? (const float*)grad_scale->data : nullptr;
  a.found_inf = found_inf != nullptr ? (const float*)found_inf->data : nullptr;
  const int64_t vec = 16 / dtype_size(dt);
  const int64_t chunk = (int64_t)kAdamBlock * kAdamPieces * vec;
  int k = 0;
  int64_t blocks = 0;
  auto flush = [&]() -> mi_status_t {
    if (k == 0) return MI_OK;
    a.count = k;
    mi_status_t st;
    switch (dt) {
      case MI_F32: st = launch_adam<float>(a, ams, stream, blocks); break;
      case MI_BF16: st = launch_adam<BF16>(a, ams, stream, blocks); break;
      case MI_F16: st = launch_adam<F16>(a, ams, stream, blocks); break;
      default: st = launch_adam<double>(a, ams, stream, blocks); break;
    }
    k = 0;
    blocks = 0;
    return st;
  };
  for (int i = 0; i < n_tensors; ++i) {
    const mi_tensor_t* p = params[i];
    const mi_tensor_t* lists[4] = {grads[i], exp_avgs[i], exp_avg_sqs[i],
                                   ams ? max_exp_avg_sqs[i] : nullptr};
    static const char* names[4] = {"grad", "exp_avg", "exp_avg_sq", "max_exp_avg_sq"};
    MI_RETURN_IF(validate(p, "param"));
    MI_CHECK_ARG(p->dtype == dt, "fused_adamw: param %d is %s, param 0 is %s", i,
                 dtype_name(p->dtype), dtype_name(dt));
    for (int q = 0; q < (ams ? 4 : 3); ++q) {
      MI_RETURN_IF(validate(lists[q], names[q]));
      MI_CHECK_ARG(same_layout(*p, *lists[q]),
                   "fused_adamw: %s %d differs from its param in dtype, shape or strides",
                   names[q], i);
    }
    MI_RETURN_IF(check_scalar(state_steps[i], "state_step", false));
    const int64_t n = numel(*p);
    if (n == 0) continue;
    MI_CHECK_ARG(dense_any_order(*p), "fused_adamw: param %d is not dense", i);
    AdamTensor& t = a.t[k];
    t.p = p->data;
    t.g = lists[0]->data;
    t.m = lists[1]->data;
    t.v = lists[2]->data;
    t.vm = ams ? lists[3]->data : nullptr;
    t.step = (const float*)state_steps[i]->data;
    t.n = n;
    t.first_block = blocks;
    uintptr_t bits = (uintptr_t)t.p | (uintptr_t)t.g | (uintptr_t)t.m | (uintptr_t)t.v |
                     (uintptr_t)t.vm;
    t.vec_ok = (bits % 16) == 0;
    blocks += (n + chunk - 1) / chunk;
    MI_CHECK_ARG(blocks <= 0x7fffffffLL, "fused_adamw: too many blocks");
    if (++k == kAdamMax) MI_RETURN_IF(flush());
  }
  return flush();
}
