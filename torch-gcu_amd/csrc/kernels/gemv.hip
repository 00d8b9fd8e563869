// Matrix-vector product: out = beta * self + alpha * (mat @ vec), mat [M, K],
// vec [K], out [M] (addmv; mv is addmv with beta = 0).
//
// HBM-bound on mat (read once).  One wave owns one row of mat: its 64 lanes
// read it in 16-byte non-temporal pieces, eight in flight per lane (a whole
// 8 KiB row of K = 4096 bf16 in one round), multiply by the matching pieces
// of vec (read through the cache), accumulate in fp32, add the lanes in a
// fixed shuffle tree and round once.  (On addmv [11008, 4096] one row per
// wave and eight pieces a lane took 14.6 us against 16.7 us for two rows per
// wave with four pieces each: twice the waves in flight, each with its loads
// in one round; 16 pieces a lane, or 8 or 16 waves per block, were slower.)
// mat is used as [M, K] with K contiguous; another layout (a transposed
// view, a leading dim that breaks 16-byte alignment) is first copied densely
// into workspace, and so is a strided vec.
#include "iter.h"

namespace mi {
namespace {

constexpr int kGemvRows = 4;    // waves per 256-lane block (one row each)
constexpr int kGemvUnroll = 8;  // 16-byte pieces in flight per lane

struct GemvArgs {
  const void* mat;
  const void* vec;
  void* out;
  const void* bias;
  int bias_dtype;
  int64_t bias_s, out_s;
  int64_t M, K, lda;
  float alpha, beta;
};

template <typename Tag>
__global__ __launch_bounds__(64 * kGemvRows) void gemv_rows_kernel(GemvArgs a) {
  typedef typename Num<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  constexpr int U = kGemvUnroll;
  union V {
    uint4 u;
    St s[VEC];
  };
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kGemvRows + (threadIdx.x >> 6);
  if (row >= a.M) return;  // a whole wave
  const St* p = (const St*)a.mat + row * a.lda;
  const St* x = (const St*)a.vec;
  float acc = 0.f;
  // the host checked: mat rows and vec 16-byte aligned
  const int64_t nv = a.K / VEC;
  const V* pv = (const V*)p;
  const V* xv = (const V*)x;
  for (int64_t v0 = lane; v0 < nv; v0 += 64 * U) {
    // unconditional loads (a piece past the row end re-reads the last one and
    // is not used): under a per-piece branch each load was waited alone
    V m[U], w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = v0 + (int64_t)u * 64 < nv ? v0 + (int64_t)u * 64 : nv - 1;
      m[u] = ld_stream(pv + v);
      w[u] = xv[v];
    }
    // keep the scheduler from pulling the multiplies between the loads (each
    // use of a just-issued load costs a wait for all loads before it)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (v0 + (int64_t)u * 64 < nv) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          acc = __builtin_fmaf(Num<Tag>::load(m[u].s[e]), Num<Tag>::load(w[u].s[e]), acc);
      }
    }
  }
  for (int64_t k = nv * VEC + lane; k < a.K; k += 64)
    acc = __builtin_fmaf(Num<Tag>::load(p[k]), Num<Tag>::load(x[k]), acc);
  acc = wave_sum(acc);
  if (lane == 0) {
    // alpha == 0 leaves mat and vec out, as BLAS gemv (and CPU ATen) do
    float r = a.alpha != 0.f ? a.alpha * acc : 0.f;
    if (a.beta != 0.f) r += a.beta * load_as<float>(a.bias, row * a.bias_s, a.bias_dtype);
    ((St*)a.out)[row * a.out_s] = Num<Tag>::store(r);
  }
}

template <typename Tag>
mi_status_t launch_gemv(const GemvArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((gemv_rows_kernel<Tag>), dim3(ceil_div_u(a.M, kGemvRows)),
                     dim3(64 * kGemvRows), 0, s, a);
  return check_launch("addmv");
}

// `t` (rank 1 or 2) as a dense row-major copy in workspace when its rows are
// not K-contiguous and 16-byte aligned
mi_status_t dense_copy(const mi_tensor_t* t, Workspace& ws, mi_tensor_t* d, hipStream_t s) {
  *d = *t;
  int64_t st = 1;
  for (int i = t->ndim - 1; i >= 0; --i) {
    d->strides[i] = st;
    st *= t->sizes[i];
  }
  MI_RETURN_IF(ws.alloc((size_t)(numel(*t) * dtype_size(t->dtype)), s));
  d->data = ws.get();
  return mi_copy(d, t, (mi_stream_t)s);
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status_t mi_addmv(const mi_tensor_t* out, const mi_tensor_t* self,
                                const mi_tensor_t* mat, const mi_tensor_t* vec, double beta,
                                double alpha, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(mat, "mat"));
  MI_RETURN_IF(validate(vec, "vec"));
  MI_CHECK_ARG(mat->ndim == 2, "addmv: mat must be 2-D, got %d dims", mat->ndim);
  MI_CHECK_ARG(vec->ndim == 1, "addmv: vec must be 1-D, got %d dims", vec->ndim);
  MI_CHECK_ARG(out->ndim == 1, "addmv: out must be 1-D, got %d dims", out->ndim);
  const int64_t M = mat->sizes[0], K = mat->sizes[1];
  MI_CHECK_ARG(vec->sizes[0] == K, "addmv: size mismatch, mat [%lld, %lld], vec [%lld]",
               (long long)M, (long long)K, (long long)vec->sizes[0]);
  MI_CHECK_ARG(out->sizes[0] == M, "addmv: out has %lld elements, expected %lld",
               (long long)out->sizes[0], (long long)M);
  const int dt = mat->dtype;
  MI_CHECK_ARG(vec->dtype == dt && out->dtype == dt,
               "addmv: mat, vec and out must share a dtype (%s, %s, %s)", dtype_name(dt),
               dtype_name(vec->dtype), dtype_name(out->dtype));
  MI_CHECK_ARG(dt == MI_BF16 || dt == MI_F16 || dt == MI_F32, "addmv: dtype %s unsupported",
               dtype_name(dt));
  GemvArgs a{};
  a.bias = nullptr;
  a.bias_dtype = MI_F32;
  a.bias_s = 0;
  if (beta != 0.0) {
    MI_CHECK_ARG(self != nullptr && self->data != nullptr, "addmv: self is required when beta != 0");
    MI_RETURN_IF(validate(self, "self"));
    MI_CHECK_ARG(self->ndim <= 1, "addmv: self must be 0-D or 1-D");
    const int64_t n = self->ndim == 0 ? 1 : self->sizes[0];
    MI_CHECK_ARG(n == 1 || n == M, "addmv: self of %lld elements does not broadcast to %lld",
                 (long long)n, (long long)M);
    MI_CHECK_ARG(self->dtype == dt || self->dtype == MI_F32,
                 "addmv: self dtype %s must be the output's or fp32", dtype_name(self->dtype));
    a.bias = self->data;
    a.bias_dtype = self->dtype;
    a.bias_s = (self->ndim == 0 || n == 1) ? 0 : self->strides[0];
  }
  if (M == 0) return MI_OK;
  const int es = dtype_size(dt);
  const int64_t align_el = 16 / es;
  Workspace wm, wv;
  mi_tensor_t md = *mat, vd = *vec;
  // K == 0: the kernel reads neither mat nor vec
  const bool mat_ok = K == 0 || ((mat->strides[1] == 1 || K == 1) &&
                                 (M == 1 || mat->strides[0] % align_el == 0) &&
                                 ((uintptr_t)mat->data % 16) == 0);
  if (!mat_ok) MI_RETURN_IF(dense_copy(mat, wm, &md, stream));
  const bool vec_ok = K == 0 || ((vec->strides[0] == 1 || K == 1) && ((uintptr_t)vec->data % 16) == 0);
  if (!vec_ok) MI_RETURN_IF(dense_copy(vec, wv, &vd, stream));
  a.mat = md.data;
  a.vec = vd.data;
  a.out = out->data;
  a.out_s = out->strides[0];
  a.M = M;
  a.K = K;
  a.lda = M == 1 ? K : md.strides[0];
  a.alpha = (float)alpha;
  a.beta = (float)beta;
  switch (dt) {
    case MI_BF16: return launch_gemv<BF16>(a, stream);
    case MI_F16: return launch_gemv<F16>(a, stream);
    default: return launch_gemv<float>(a, stream);
  }
}
