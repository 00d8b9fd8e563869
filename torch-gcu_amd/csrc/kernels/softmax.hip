// softmax / log_softmax along one dim, computed in float.
//
// Rows along a dense last dim (config 2: bf16 [8192, 32000], 64,000 B per
// row) are read from HBM once: a block of up to 1024 lanes holds its row in
// registers (up to 16 x 16-byte vectors per lane), takes the row max and the sum of
// exp(x - max) with wave64 shuffles plus an LDS combine, then writes
//   log_softmax: x - max - log(sum)      softmax: exp(x - max) * (1 / sum)
// which is the same sequence of float operations ATen's CPU kernel uses
// (aten/src/ATen/native/cpu/SoftMaxKernel.cpp, _vec_log_softmax_lastdim).
// Longer or unaligned rows use a two-read block kernel with an online
// (max, sum) pair; a non-last dim uses one lane per column.
#include <cmath>

#include "iter.h"

namespace mi {
namespace {

constexpr int kBlock = 256;

template <typename Tag>
struct ST {
  typedef Tag storage;
  static __device__ __forceinline__ float load(storage v) { return (float)v; }
  static __device__ __forceinline__ storage store(float v) { return (storage)v; }
};
template <>
struct ST<BF16> {
  typedef uint16_t storage;
  static __device__ __forceinline__ float load(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_bf16(v); }
};
template <>
struct ST<F16> {
  typedef uint16_t storage;
  static __device__ __forceinline__ float load(uint16_t v) { return f16_to_f32(v); }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_f16(v); }
};

// exp used inside the kernels: hardware exp2 for 16-bit inputs (outputs are
// rounded to 8 or 11 mantissa bits), the accurate library expf for float.
template <typename Tag>
__device__ __forceinline__ float kexp(float x) {
  if constexpr (std::is_same<Tag, float>::value) return expf(x);
  else return fast_exp(x);
}

__device__ __forceinline__ float block_max_f(float v, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_nan_max(v);
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = nan_max(r, red[w]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_sum_f(float v, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r += red[w];
  __syncthreads();
  return r;
}

// Register-resident row: NTH lanes, VPT 16-byte vectors per lane.  The row
// max uses fmaxf, which skips NaN: a NaN element still makes exp(x - max)
// and therefore the row sum NaN, so every output of that row is NaN, as in
// ATen (whose max propagates the NaN).  Loads and stores are non-temporal:
// each byte is touched once.
template <int NTH>
__device__ __forceinline__ float block_fmax(float v, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_fmax(v);
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NTH / 64; ++w) r = fmaxf(r, red[w]);
  return r;
}
template <int NTH>
__device__ __forceinline__ float block_fsum(float v, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NTH / 64; ++w) r += red[w];
  return r;
}

template <typename InTag, typename OutTag, int NTH, int VPT, bool LOG>
__global__ __launch_bounds__(NTH) void softmax_reg_kernel(
    typename ST<OutTag>::storage* __restrict__ out,
    const typename ST<InTag>::storage* __restrict__ in, int64_t D, int64_t in_row_stride,
    int64_t out_row_stride) {
  typedef typename ST<InTag>::storage Si;
  typedef typename ST<OutTag>::storage So;
  constexpr int VEC = 16 / sizeof(Si);
  __shared__ float red[2][NTH / 64];
  union Vi {
    uint4 u;
    Si s[VEC];
  };
  constexpr int kWords = sizeof(So) * VEC / 16;
  union Vo {
    So s[VEC];
    uint4 u[kWords];
  };
  const int64_t row = blockIdx.x;
  const Vi* pin = (const Vi*)(in + row * in_row_stride);
  const int nv = (int)(D / VEC);
  Vi x[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = threadIdx.x + k * NTH;
    if (v < nv) x[k] = ld_stream(pin + v);
  }
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    if ((int)threadIdx.x + k * NTH < nv) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) m = fmaxf(m, ST<InTag>::load(x[k].s[e]));
    }
  }
  m = block_fmax<NTH>(m, red[0]);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    if ((int)threadIdx.x + k * NTH < nv) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += kexp<InTag>(ST<InTag>::load(x[k].s[e]) - m);
    }
  }
  s = block_fsum<NTH>(s, red[1]);
  So* po = out + row * out_row_stride;
  if constexpr (LOG) {
    const float lse = logf(s);
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = threadIdx.x + k * NTH;
      if (v < nv) {
        Vo o;
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          o.s[e] = ST<OutTag>::store((ST<InTag>::load(x[k].s[e]) - m) - lse);
#pragma unroll
        for (int w = 0; w < kWords; ++w) st_stream((uint4*)(po + (int64_t)v * VEC) + w, o.u[w]);
      }
    }
  } else {
    const float inv = 1.0f / s;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int v = threadIdx.x + k * NTH;
      if (v < nv) {
        Vo o;
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          o.s[e] = ST<OutTag>::store(kexp<InTag>(ST<InTag>::load(x[k].s[e]) - m) * inv);
#pragma unroll
        for (int w = 0; w < kWords; ++w) st_stream((uint4*)(po + (int64_t)v * VEC) + w, o.u[w]);
      }
    }
  }
}

// Any row length / alignment: online (max, sum) in one read, output in a
// second read.
template <typename InTag, typename OutTag, bool LOG>
__global__ __launch_bounds__(kBlock) void softmax_row_kernel(
    typename ST<OutTag>::storage* __restrict__ out,
    const typename ST<InTag>::storage* __restrict__ in, int64_t D, int64_t in_row_stride,
    int64_t out_row_stride) {
  __shared__ float red[16];
  __shared__ float red2[16];
  const int64_t row = blockIdx.x;
  const typename ST<InTag>::storage* p = in + row * in_row_stride;
  float m = -INFINITY, s = 0.f;
  for (int64_t j = threadIdx.x; j < D; j += kBlock) {
    const float x = ST<InTag>::load(p[j]);
    if (x != x) {
      m = x;  // NaN propagates through max and sum
    } else if (x > m) {
      s = s * kexp<InTag>(m - x) + 1.f;
      m = x;
    } else if (x > -INFINITY) {
      s += kexp<InTag>(x - m);
    }
  }
  // combine (m, s) pairs across the block
  const float gm = block_max_f(m, red);
  float ls = (m == -INFINITY) ? 0.f : s * kexp<InTag>(m - gm);
  (void)red2;
  const float gs = block_sum_f(ls, red);
  typename ST<OutTag>::storage* po = out + row * out_row_stride;
  if constexpr (LOG) {
    const float lse = logf(gs);
    for (int64_t j = threadIdx.x; j < D; j += kBlock)
      po[j] = ST<OutTag>::store((ST<InTag>::load(p[j]) - gm) - lse);
  } else {
    const float inv = 1.0f / gs;
    for (int64_t j = threadIdx.x; j < D; j += kBlock)
      po[j] = ST<OutTag>::store(kexp<InTag>(ST<InTag>::load(p[j]) - gm) * inv);
  }
}

// [outer, D, inner] with inner > 1: one lane per (outer, inner) column.
template <typename InTag, typename OutTag, bool LOG>
__global__ __launch_bounds__(kBlock) void softmax_col_kernel(
    typename ST<OutTag>::storage* __restrict__ out,
    const typename ST<InTag>::storage* __restrict__ in, int64_t outer, int64_t D,
    int64_t inner) {
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const typename ST<InTag>::storage* p = in + o * D * inner + i;
  typename ST<OutTag>::storage* q = out + o * D * inner + i;
  float m = -INFINITY;
  for (int64_t j = 0; j < D; ++j) m = nan_max(m, ST<InTag>::load(p[j * inner]));
  float s = 0.f;
  for (int64_t j = 0; j < D; ++j) s += kexp<InTag>(ST<InTag>::load(p[j * inner]) - m);
  if constexpr (LOG) {
    const float lse = logf(s);
    for (int64_t j = 0; j < D; ++j)
      q[j * inner] = ST<OutTag>::store((ST<InTag>::load(p[j * inner]) - m) - lse);
  } else {
    const float inv = 1.0f / s;
    for (int64_t j = 0; j < D; ++j)
      q[j * inner] = ST<OutTag>::store(kexp<InTag>(ST<InTag>::load(p[j * inner]) - m) * inv);
  }
}

template <typename InTag, typename OutTag, bool LOG>
mi_status_t launch_t(const mi_tensor_t* out, const mi_tensor_t* self, int dim,
                     hipStream_t stream) {
  typedef typename ST<InTag>::storage Si;
  const int nd = self->ndim;
  int64_t outer = 1, inner = 1;
  const int64_t D = nd == 0 ? 1 : self->sizes[dim];
  for (int d = 0; d < dim; ++d) outer *= self->sizes[d];
  for (int d = dim + 1; d < nd; ++d) inner *= self->sizes[d];
  if (outer * inner == 0 || D == 0) return MI_OK;
  if (inner == 1) {
    constexpr int VEC = 16 / sizeof(Si);
    const bool aligned = ((uintptr_t)self->data % 16 == 0) &&
                         ((uintptr_t)out->data % 16 == 0) && (D % VEC == 0);
    const int64_t nv = D / VEC;
    auto run_reg = [&](auto nth_c, auto vpt_c) -> mi_status_t {
      constexpr int NTH = decltype(nth_c)::value;
      constexpr int VPT = decltype(vpt_c)::value;
      hipLaunchKernelGGL((softmax_reg_kernel<InTag, OutTag, NTH, VPT, LOG>),
                         dim3((unsigned)outer), dim3(NTH), 0, stream,
                         (typename ST<OutTag>::storage*)out->data, (const Si*)self->data, D, D,
                         D);
      return check_launch("softmax_reg");
    };
    typedef std::integral_constant<int, 1> V1;
    typedef std::integral_constant<int, 1024> N1024;
    // rows of up to 256 K vectors: 1024 lanes hold up to 16 vectors each
    // (64 VGPRs of row data); short rows take one vector per lane
    if (aligned && nv <= 1024 * 16 && outer <= 0x7fffffff) {
      if (nv <= 256) return run_reg(std::integral_constant<int, 256>(), V1());
      if (nv <= 512) return run_reg(std::integral_constant<int, 512>(), V1());
      if (nv <= 1024) return run_reg(N1024(), V1());
      if (nv <= 2048) return run_reg(N1024(), std::integral_constant<int, 2>());
      if (nv <= 4096) return run_reg(N1024(), std::integral_constant<int, 4>());
      if (nv <= 8192) return run_reg(N1024(), std::integral_constant<int, 8>());
      return run_reg(N1024(), std::integral_constant<int, 16>());
    }
    hipLaunchKernelGGL((softmax_row_kernel<InTag, OutTag, LOG>), dim3((unsigned)outer),
                       dim3(kBlock), 0, stream, (typename ST<OutTag>::storage*)out->data,
                       (const Si*)self->data, D, D, D);
    return check_launch("softmax_row");
  }
  hipLaunchKernelGGL((softmax_col_kernel<InTag, OutTag, LOG>),
                     dim3(ceil_div_u(outer * inner, kBlock)), dim3(kBlock), 0, stream,
                     (typename ST<OutTag>::storage*)out->data, (const Si*)self->data, outer, D,
                     inner);
  return check_launch("softmax_col");
}

// ---- backward ---------------------------------------------------------------
//   log_softmax: gi = dy - exp(y) * sum(dy)        softmax: gi = y * (dy - sum(dy * y))
// with y the forward output, the row sums in float (ATen's
// _log_softmax_backward_data / _softmax_backward_data,
// aten/src/ATen/native/cpu/SoftMaxKernel.cpp, _vec_log_softmax_backward and
// _vec_softmax_backward).  Same layouts as the forward: a register-resident
// row for dense aligned rows, a two-read row kernel, one lane per column.
template <typename InTag, bool LOG>
__device__ __forceinline__ float bwd_term(float dy, float y) {
  return LOG ? dy : dy * y;
}
template <typename InTag, bool LOG>
__device__ __forceinline__ float bwd_out(float dy, float y, float s) {
  if constexpr (LOG) return dy - kexp<InTag>(y) * s;
  else return y * (dy - s);
}

template <typename InTag, typename OutTag, int NTH, int VPT, bool LOG>
__global__ __launch_bounds__(NTH) void softmax_bwd_reg_kernel(
    typename ST<OutTag>::storage* __restrict__ gi, const typename ST<InTag>::storage* __restrict__ dy,
    const typename ST<InTag>::storage* __restrict__ y, int64_t D) {
  typedef typename ST<InTag>::storage Si;
  typedef typename ST<OutTag>::storage So;
  constexpr int VEC = 16 / sizeof(Si);
  __shared__ float red[NTH / 64];
  union Vi {
    uint4 u;
    Si s[VEC];
  };
  // a narrower output (float grads into half) writes 8 bytes per vector
  constexpr int kBytes = sizeof(So) * VEC;
  static_assert(kBytes == 8 || kBytes % 16 == 0, "output vector of 8 or 16k bytes");
  union Vo {
    So s[VEC];
    uint2 h[kBytes / 8];
    uint4 u[(kBytes + 15) / 16];
  };
  const int64_t row = blockIdx.x;
  const Vi* pd = (const Vi*)(dy + row * D);
  const Vi* py = (const Vi*)(y + row * D);
  const int nv = (int)(D / VEC);
  Vi xd[VPT], xy[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = threadIdx.x + k * NTH;
    if (v < nv) {
      xd[k] = ld_stream(pd + v);
      xy[k] = ld_stream(py + v);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    if ((int)threadIdx.x + k * NTH < nv) {
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        s += bwd_term<InTag, LOG>(ST<InTag>::load(xd[k].s[e]), ST<InTag>::load(xy[k].s[e]));
    }
  }
  s = block_fsum<NTH>(s, red);
  So* po = gi + row * D;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    const int v = threadIdx.x + k * NTH;
    if (v < nv) {
      Vo o;
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        o.s[e] = ST<OutTag>::store(
            bwd_out<InTag, LOG>(ST<InTag>::load(xd[k].s[e]), ST<InTag>::load(xy[k].s[e]), s));
      if constexpr (kBytes == 8) {
        *(uint2*)(po + (int64_t)v * VEC) = o.h[0];
      } else {
#pragma unroll
        for (int w = 0; w < kBytes / 16; ++w) st_stream((uint4*)(po + (int64_t)v * VEC) + w, o.u[w]);
      }
    }
  }
}

template <typename InTag, typename OutTag, bool LOG>
__global__ __launch_bounds__(kBlock) void softmax_bwd_row_kernel(
    typename ST<OutTag>::storage* __restrict__ gi, const typename ST<InTag>::storage* __restrict__ dy,
    const typename ST<InTag>::storage* __restrict__ y, int64_t D) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const typename ST<InTag>::storage* pd = dy + row * D;
  const typename ST<InTag>::storage* py = y + row * D;
  float s = 0.f;
  for (int64_t j = threadIdx.x; j < D; j += kBlock)
    s += bwd_term<InTag, LOG>(ST<InTag>::load(pd[j]), ST<InTag>::load(py[j]));
  s = block_sum_f(s, red);
  typename ST<OutTag>::storage* po = gi + row * D;
  for (int64_t j = threadIdx.x; j < D; j += kBlock)
    po[j] = ST<OutTag>::store(bwd_out<InTag, LOG>(ST<InTag>::load(pd[j]), ST<InTag>::load(py[j]), s));
}

template <typename InTag, typename OutTag, bool LOG>
__global__ __launch_bounds__(kBlock) void softmax_bwd_col_kernel(
    typename ST<OutTag>::storage* __restrict__ gi, const typename ST<InTag>::storage* __restrict__ dy,
    const typename ST<InTag>::storage* __restrict__ y, int64_t outer, int64_t D, int64_t inner) {
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const int64_t base = o * D * inner + i;
  float s = 0.f;
  for (int64_t j = 0; j < D; ++j)
    s += bwd_term<InTag, LOG>(ST<InTag>::load(dy[base + j * inner]), ST<InTag>::load(y[base + j * inner]));
  for (int64_t j = 0; j < D; ++j) {
    const int64_t q = base + j * inner;
    gi[q] = ST<OutTag>::store(bwd_out<InTag, LOG>(ST<InTag>::load(dy[q]), ST<InTag>::load(y[q]), s));
  }
}

template <typename InTag, typename OutTag, bool LOG>
mi_status_t launch_bwd_t(const mi_tensor_t* gi, const mi_tensor_t* dy, const mi_tensor_t* y,
                         int dim, hipStream_t stream) {
  typedef typename ST<InTag>::storage Si;
  typedef typename ST<OutTag>::storage So;
  const int nd = y->ndim;
  int64_t outer = 1, inner = 1;
  const int64_t D = nd == 0 ? 1 : y->sizes[dim];
  for (int d = 0; d < dim; ++d) outer *= y->sizes[d];
  for (int d = dim + 1; d < nd; ++d) inner *= y->sizes[d];
  if (outer * inner == 0 || D == 0) return MI_OK;
  if (inner == 1) {
    constexpr int VEC = 16 / sizeof(Si);
    const bool aligned = (((uintptr_t)dy->data | (uintptr_t)y->data | (uintptr_t)gi->data) % 16 == 0) &&
                         (D % VEC == 0);
    const int64_t nv = D / VEC;
    auto run_reg = [&](auto nth_c, auto vpt_c) -> mi_status_t {
      constexpr int NTH = decltype(nth_c)::value;
      constexpr int VPT = decltype(vpt_c)::value;
      hipLaunchKernelGGL((softmax_bwd_reg_kernel<InTag, OutTag, NTH, VPT, LOG>),
                         dim3((unsigned)outer), dim3(NTH), 0, stream, (So*)gi->data,
                         (const Si*)dy->data, (const Si*)y->data, D);
      return check_launch("softmax_bwd_reg");
    };
    typedef std::integral_constant<int, 1> V1;
    typedef std::integral_constant<int, 1024> N1024;
    // two row operands in registers: up to 8 vectors of each per lane
    if (aligned && nv <= 1024 * 8 && outer <= 0x7fffffff) {
      if (nv <= 256) return run_reg(std::integral_constant<int, 256>(), V1());
      if (nv <= 512) return run_reg(std::integral_constant<int, 512>(), V1());
      if (nv <= 1024) return run_reg(N1024(), V1());
      if (nv <= 2048) return run_reg(N1024(), std::integral_constant<int, 2>());
      if (nv <= 4096) return run_reg(N1024(), std::integral_constant<int, 4>());
      return run_reg(N1024(), std::integral_constant<int, 8>());
    }
    hipLaunchKernelGGL((softmax_bwd_row_kernel<InTag, OutTag, LOG>), dim3((unsigned)outer),
                       dim3(kBlock), 0, stream, (So*)gi->data, (const Si*)dy->data,
                       (const Si*)y->data, D);
    return check_launch("softmax_bwd_row");
  }
  hipLaunchKernelGGL((softmax_bwd_col_kernel<InTag, OutTag, LOG>),
                     dim3(ceil_div_u(outer * inner, kBlock)), dim3(kBlock), 0, stream,
                     (So*)gi->data, (const Si*)dy->data, (const Si*)y->data, outer, D, inner);
  return check_launch("softmax_bwd_col");
}

template <bool LOG>
mi_status_t run_softmax_bwd(const mi_tensor_t* gi, const mi_tensor_t* dy, const mi_tensor_t* y,
                            int64_t dim, hipStream_t stream) {
  clear_error();
  MI_RETURN_IF(validate(gi, "grad_input"));
  MI_RETURN_IF(validate(dy, "grad_output"));
  MI_RETURN_IF(validate(y, "output"));
  const int nd = y->ndim;
  const int lim = nd == 0 ? 1 : nd;
  if (dim < 0) dim += lim;
  MI_CHECK_ARG(dim >= 0 && dim < lim, "softmax_backward: dim out of range");
  MI_CHECK_ARG(gi->ndim == nd && dy->ndim == nd, "softmax_backward: rank mismatch");
  for (int d = 0; d < nd; ++d)
    MI_CHECK_ARG(gi->sizes[d] == y->sizes[d] && dy->sizes[d] == y->sizes[d],
                 "softmax_backward: shape mismatch");
  if (numel(*y) == 0) return MI_OK;
  if (!is_contiguous(*gi) || !is_contiguous(*dy) || !is_contiguous(*y))
    MI_FAIL(MI_ERR_UNSUPPORTED, "softmax_backward: operands must be contiguous");
  MI_CHECK_ARG(dy->dtype == y->dtype, "softmax_backward: grad_output and output must share a dtype");
  const int di = y->dtype, dout = gi->dtype;
  const int d = nd == 0 ? 0 : (int)dim;
  if (di == MI_BF16 && dout == MI_BF16) return launch_bwd_t<BF16, BF16, LOG>(gi, dy, y, d, stream);
  if (di == MI_F16 && dout == MI_F16) return launch_bwd_t<F16, F16, LOG>(gi, dy, y, d, stream);
  if (di == MI_F32 && dout == MI_F32) return launch_bwd_t<float, float, LOG>(gi, dy, y, d, stream);
  if (di == MI_F32 && dout == MI_BF16) return launch_bwd_t<float, BF16, LOG>(gi, dy, y, d, stream);
  if (di == MI_F32 && dout == MI_F16) return launch_bwd_t<float, F16, LOG>(gi, dy, y, d, stream);
  MI_FAIL(MI_ERR_UNSUPPORTED, "softmax_backward: dtype %s -> %s", dtype_name(di), dtype_name(dout));
}

template <bool LOG>
mi_status_t run_softmax(const mi_tensor_t* out, const mi_tensor_t* self, int64_t dim,
                        hipStream_t stream) {
  clear_error();
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(self, "self"));
  const int nd = self->ndim;
  const int lim = nd == 0 ? 1 : nd;
  if (dim < 0) dim += lim;
  MI_CHECK_ARG(dim >= 0 && dim < lim, "softmax: dim out of range");
  MI_CHECK_ARG(out->ndim == nd, "softmax: out rank mismatch");
  for (int d = 0; d < nd; ++d)
    MI_CHECK_ARG(out->sizes[d] == self->sizes[d], "softmax: out shape mismatch");
  if (numel(*self) == 0) return MI_OK;
  // Dense operands only; the host makes other layouts dense first.
  if (!is_contiguous(*self) || !is_contiguous(*out))
    MI_FAIL(MI_ERR_UNSUPPORTED, "softmax: operands must be contiguous");
  const int di = self->dtype, dout = out->dtype;
  const int d = nd == 0 ? 0 : (int)dim;
  if (di == MI_BF16 && dout == MI_BF16) return launch_t<BF16, BF16, LOG>(out, self, d, stream);
  if (di == MI_BF16 && dout == MI_F32) return launch_t<BF16, float, LOG>(out, self, d, stream);
  if (di == MI_F16 && dout == MI_F16) return launch_t<F16, F16, LOG>(out, self, d, stream);
  if (di == MI_F16 && dout == MI_F32) return launch_t<F16, float, LOG>(out, self, d, stream);
  if (di == MI_F32 && dout == MI_F32) return launch_t<float, float, LOG>(out, self, d, stream);
  MI_FAIL(MI_ERR_UNSUPPORTED, "softmax: dtype %s -> %s", dtype_name(di), dtype_name(dout));
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

mi_status_t mi_softmax(const mi_tensor_t* out, const mi_tensor_t* self, int64_t dim,
                       mi_stream_t stream) {
  return run_softmax<false>(out, self, dim, (hipStream_t)stream);
}

mi_status_t mi_log_softmax(const mi_tensor_t* out, const mi_tensor_t* self, int64_t dim,
                           mi_stream_t stream) {
  return run_softmax<true>(out, self, dim, (hipStream_t)stream);
}

mi_status_t mi_log_softmax_backward(const mi_tensor_t* grad_input, const mi_tensor_t* grad_output,
                                    const mi_tensor_t* output, int64_t dim, mi_stream_t stream) {
  return run_softmax_bwd<true>(grad_input, grad_output, output, dim, (hipStream_t)stream);
}

mi_status_t mi_softmax_backward(const mi_tensor_t* grad_input, const mi_tensor_t* grad_output,
                                const mi_tensor_t* output, int64_t dim, mi_stream_t stream) {
  return run_softmax_bwd<false>(grad_input, grad_output, output, dim, (hipStream_t)stream);
}

}  // extern "C"
