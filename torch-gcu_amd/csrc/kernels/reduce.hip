// Reductions sum / amax / mean over arbitrary dims.
//
// The host maps self to [outer, R, inner] (R = product of the reduced dims,
// which must form one dense block; otherwise a permuted dense copy is made
// in workspace first):
//   - inner == 1 ("row" reduction, e.g. config 2's bf16 [8192, 32000] over
//     the last dim): one 256-lane block per row, 16-byte vector loads, four
//     in flight per lane, wave64 shuffle reduction then an LDS combine of the
//     four waves.  Long rows with few of them are split over several blocks
//     and finished by a second pass over the partials.
//   - inner > 1 ("column" reduction, e.g. fp32 [16384, 4096] over dim 0):
//     lanes own 16-byte column vectors so each wave reads 1 KiB contiguous
//     per row; the rows are split into chunks over blocks (partials in
//     workspace, then a second pass), which keeps more than 1000 blocks in
//     flight for a 4096-wide output.
// Floating inputs accumulate in float (double for f64), integers in int64.
#include <algorithm>
#include <cmath>
#include <vector>

#include "iter.h"

namespace mi {
namespace {

enum RedOp { R_SUM = 0, R_MAX = 1, R_MEAN = 2 };

template <typename Tag>
struct RT {  // int64/int32/int16/int8/uint8 storage
  typedef Tag storage;
  typedef int64_t acc;
  static __device__ __forceinline__ acc load(storage v) { return (acc)v; }
};
template <>
struct RT<float> {
  typedef float storage;
  typedef float acc;
  static __device__ __forceinline__ acc load(storage v) { return v; }
};
template <>
struct RT<double> {
  typedef double storage;
  typedef double acc;
  static __device__ __forceinline__ acc load(storage v) { return v; }
};
template <>
struct RT<BF16> {
  typedef uint16_t storage;
  typedef float acc;
  static __device__ __forceinline__ acc load(storage v) { return bf16_to_f32(v); }
};
template <>
struct RT<F16> {
  typedef uint16_t storage;
  typedef float acc;
  static __device__ __forceinline__ acc load(storage v) { return f16_to_f32(v); }
};
struct BoolTag {};
template <>
struct RT<BoolTag> {
  typedef uint8_t storage;
  typedef int64_t acc;
  static __device__ __forceinline__ acc load(storage v) { return v != 0; }
};

template <typename A>
__device__ __forceinline__ A red_ident(int op) {
  if (op == R_MAX) {
    if constexpr (std::is_floating_point<A>::value) return -INFINITY;
    else return (A)INT64_MIN;
  }
  return A(0);
}

template <typename A>
__device__ __forceinline__ A red_combine(int op, A a, A b) {
  return op == R_MAX ? nan_max(a, b) : a + b;
}

template <typename A>
__device__ __forceinline__ A wave_red(int op, A v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = red_combine(op, v, (A)__shfl_xor(v, off, 64));
  return v;
}

// Output descriptor: either the final tensor (dtype, mean divisor) or Acc
// partials.
struct RedOut {
  void* data;
  int dtype;       // -1: write Acc partials
  double divisor;  // mean: value / divisor
};

template <typename A>
__device__ __forceinline__ void red_store(const RedOut& o, int op, int64_t idx, A v) {
  if (o.dtype < 0) {
    ((A*)o.data)[idx] = v;
    return;
  }
  if (op == R_MEAN) {
    if constexpr (std::is_floating_point<A>::value) v = v / (A)o.divisor;
  }
  store_as<A>(o.data, idx, o.dtype, v);
}

constexpr int kRowBlock = 256;

// rows x [R] -> rows x splits partials (or final when splits == 1).
// Block (row, split) reduces elements [split*chunk, min(R, (split+1)*chunk)).
template <typename Tag>
__global__ __launch_bounds__(kRowBlock) void row_reduce_kernel(
    const typename RT<Tag>::storage* __restrict__ in, int64_t R, int64_t row_stride,
    int64_t chunk, int op, RedOut out) {
  typedef typename RT<Tag>::storage St;
  typedef typename RT<Tag>::acc A;
  constexpr int VEC = 16 / sizeof(St) > 0 ? 16 / sizeof(St) : 1;
  __shared__ A red[16];
  const int64_t row = blockIdx.x;
  const int64_t split = blockIdx.y;
  const int64_t beg = split * chunk;
  const int64_t end = beg + chunk < R ? beg + chunk : R;
  const St* p = in + row * row_stride;
  A acc = red_ident<A>(op);
  const bool vec_ok = ((((uintptr_t)(p + beg)) & 15) == 0);
  int64_t i = beg;
  if (vec_ok) {
    union V {
      uint4 u;
      St s[VEC];
    };
    const int64_t nv = (end - beg) / VEC;
    const V* pv = (const V*)(p + beg);
    int64_t v = threadIdx.x;
    for (; v + 3 * kRowBlock < nv; v += 4 * kRowBlock) {
      V x0 = pv[v], x1 = pv[v + kRowBlock], x2 = pv[v + 2 * kRowBlock], x3 = pv[v + 3 * kRowBlock];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        acc = red_combine(op, acc, RT<Tag>::load(x0.s[e]));
        acc = red_combine(op, acc, RT<Tag>::load(x1.s[e]));
        acc = red_combine(op, acc, RT<Tag>::load(x2.s[e]));
        acc = red_combine(op, acc, RT<Tag>::load(x3.s[e]));
      }
    }
    for (; v < nv; v += kRowBlock) {
      V x0 = pv[v];
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc = red_combine(op, acc, RT<Tag>::load(x0.s[e]));
    }
    i = beg + nv * VEC;
  }
  for (int64_t j = i + threadIdx.x; j < end; j += kRowBlock)
    acc = red_combine(op, acc, RT<Tag>::load(p[j]));
  // block combine
  acc = wave_red(op, acc);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    A r = red[0];
    for (int w = 1; w < kRowBlock / 64; ++w) r = red_combine(op, r, red[w]);
    red_store(out, op, row * gridDim.y + split, r);
  }
}

// Many short rows: one wave per row.
template <typename Tag>
__global__ __launch_bounds__(256) void row_reduce_wave_kernel(
    const typename RT<Tag>::storage* __restrict__ in, int64_t rows, int64_t R,
    int64_t row_stride, int op, RedOut out) {
  typedef typename RT<Tag>::acc A;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const typename RT<Tag>::storage* p = in + row * row_stride;
  A acc = red_ident<A>(op);
  for (int64_t j = lane; j < R; j += 64) acc = red_combine(op, acc, RT<Tag>::load(p[j]));
  acc = wave_red(op, acc);
  if (lane == 0) red_store(out, op, row, acc);
}

// [outer, R, inner] column reduction over R; block (64 x 4) lanes own one
// column (VEC columns when vectorised) and a quarter of the chunk's rows.
template <typename Tag, int VEC>
__global__ __launch_bounds__(256) void col_reduce_kernel(
    const typename RT<Tag>::storage* __restrict__ in, int64_t R, int64_t inner,
    int64_t chunk, int op, RedOut out) {
  typedef typename RT<Tag>::storage St;
  typedef typename RT<Tag>::acc A;
  __shared__ A part[4][64 * VEC];
  const int64_t ncv = inner / VEC;  // column vectors
  const int64_t ncb = (ncv + 63) / 64;
  const int64_t o = blockIdx.x / ncb;
  const int64_t cv = (blockIdx.x - o * ncb) * 64 + threadIdx.x;
  const int64_t split = blockIdx.y;
  const int64_t beg = split * chunk;
  const int64_t end = beg + chunk < R ? beg + chunk : R;
  A acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = red_ident<A>(op);
  if (cv < ncv) {
    const St* base = in + (o * R) * inner + cv * VEC;
    union V {
      St s[VEC];
    };
    int64_t r = beg + threadIdx.y;
    for (; r + 12 < end; r += 16) {
      V x0 = *(const V*)(base + r * inner), x1 = *(const V*)(base + (r + 4) * inner);
      V x2 = *(const V*)(base + (r + 8) * inner), x3 = *(const V*)(base + (r + 12) * inner);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        acc[e] = red_combine(op, acc[e], RT<Tag>::load(x0.s[e]));
        acc[e] = red_combine(op, acc[e], RT<Tag>::load(x1.s[e]));
        acc[e] = red_combine(op, acc[e], RT<Tag>::load(x2.s[e]));
        acc[e] = red_combine(op, acc[e], RT<Tag>::load(x3.s[e]));
      }
    }
    for (; r < end; r += 4) {
      V x0 = *(const V*)(base + r * inner);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = red_combine(op, acc[e], RT<Tag>::load(x0.s[e]));
    }
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) part[threadIdx.y][threadIdx.x * VEC + e] = acc[e];
  __syncthreads();
  if (threadIdx.y == 0 && cv < ncv) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      A v = part[0][threadIdx.x * VEC + e];
      for (int y = 1; y < 4; ++y) v = red_combine(op, v, part[y][threadIdx.x * VEC + e]);
      // output layout [outer, splits, inner]
      red_store(out, op, (o * gridDim.y + split) * inner + cv * VEC + e, v);
    }
  }
}

int acc_dtype_of(int dt) {
  if (dt == MI_F64) return MI_F64;
  if (is_floating(dt)) return MI_F32;
  return MI_I64;
}

template <typename Tag>
mi_status_t launch_row(const void* in, int64_t outer, int64_t R, int op, RedOut final_out,
                       int acc_dt, hipStream_t stream) {
  typedef typename RT<Tag>::acc A;
  const int cus = cu_count();
  if (R < 2048) {
    const unsigned grid = ceil_div_u(outer, 4);
    hipLaunchKernelGGL((row_reduce_wave_kernel<Tag>), dim3(grid), dim3(256), 0, stream,
                       (const typename RT<Tag>::storage*)in, outer, R, R, op, final_out);
    return check_launch("row_reduce_wave");
  }
  // split long rows so that at least ~4 blocks per CU are in flight
  int64_t splits = 1;
  const int64_t target = 4LL * cus;
  if (outer < target) {
    splits = (target + outer - 1) / outer;
    const int64_t max_splits = std::max<int64_t>(1, R / 16384);
    splits = std::min(splits, max_splits);
  }
  int64_t chunk = (R + splits - 1) / splits;
  // keep chunk starts 16-byte aligned
  const int64_t per16 = std::max<int64_t>(1, 16 / (int64_t)sizeof(typename RT<Tag>::storage));
  chunk = (chunk + per16 - 1) / per16 * per16;
  splits = (R + chunk - 1) / chunk;
  if (splits > 65535) splits = 65535;
  if (splits == 1) {
    hipLaunchKernelGGL((row_reduce_kernel<Tag>), dim3((unsigned)outer, 1), dim3(kRowBlock), 0,
                       stream, (const typename RT<Tag>::storage*)in, R, R, chunk, op, final_out);
    return check_launch("row_reduce");
  }
  Workspace ws;
  MI_RETURN_IF(ws.alloc((size_t)(outer * splits) * sizeof(A), stream));
  RedOut part{ws.get(), -1, 1.0};
  const int pop = op == R_MEAN ? R_SUM : op;
  hipLaunchKernelGGL((row_reduce_kernel<Tag>), dim3((unsigned)outer, (unsigned)splits),
                     dim3(kRowBlock), 0, stream, (const typename RT<Tag>::storage*)in, R, R,
                     chunk, pop, part);
  MI_RETURN_IF(check_launch("row_reduce partial"));
  // second pass over [outer, splits] partials in the accumulation type
  const unsigned grid = ceil_div_u(outer, 4);
  (void)acc_dt;
  hipLaunchKernelGGL((row_reduce_wave_kernel<typename std::conditional<
                          std::is_same<A, float>::value, float,
                          typename std::conditional<std::is_same<A, double>::value, double,
                                                    int64_t>::type>::type>),
                     dim3(grid), dim3(256), 0, stream, (const A*)ws.get(), outer, splits, splits,
                     op, final_out);
  return check_launch("row_reduce final");
}

template <typename Tag, int VEC>
mi_status_t launch_col_v(const void* in, int64_t outer, int64_t R, int64_t inner, int64_t splits,
                         int op, RedOut o, hipStream_t stream) {
  const int64_t ncv = inner / VEC;
  const int64_t chunk = (R + splits - 1) / splits;
  const int64_t s = (R + chunk - 1) / chunk;
  dim3 grid((unsigned)(ceil_div_u(ncv, 64) * outer), (unsigned)s, 1);
  hipLaunchKernelGGL((col_reduce_kernel<Tag, VEC>), grid, dim3(64, 4), 0, stream,
                     (const typename RT<Tag>::storage*)in, R, inner, chunk, op, o);
  return check_launch("col_reduce");
}

template <typename Tag>
mi_status_t launch_col_any(const void* in, int64_t outer, int64_t R, int64_t inner,
                           int64_t splits, int op, RedOut o, hipStream_t stream) {
  typedef typename RT<Tag>::storage St;
  constexpr int V = 16 / sizeof(St) >= 4 ? 4 : 16 / sizeof(St);
  if (inner % V == 0 && ((uintptr_t)in % (V * sizeof(St))) == 0)
    return launch_col_v<Tag, V>(in, outer, R, inner, splits, op, o, stream);
  return launch_col_v<Tag, 1>(in, outer, R, inner, splits, op, o, stream);
}

template <typename Tag>
mi_status_t launch_col(const void* in, int64_t outer, int64_t R, int64_t inner, int op,
                       RedOut final_out, hipStream_t stream) {
  typedef typename RT<Tag>::acc A;
  const int64_t cus = cu_count();
  const int64_t col_blocks = outer * ((inner + 255) / 256);
  int64_t splits = 1;
  if (col_blocks < 4 * cus && R >= 64) {
    splits = (4 * cus + col_blocks - 1) / col_blocks;
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, R / 32));
  }
  if (splits > 65535) splits = 65535;
  if (splits == 1) return launch_col_any<Tag>(in, outer, R, inner, 1, op, final_out, stream);
  const int64_t chunk = (R + splits - 1) / splits;
  splits = (R + chunk - 1) / chunk;
  Workspace ws;
  MI_RETURN_IF(ws.alloc((size_t)(outer * splits * inner) * sizeof(A), stream));
  RedOut part{ws.get(), -1, 1.0};
  const int pop = op == R_MEAN ? R_SUM : op;
  MI_RETURN_IF(launch_col_any<Tag>(in, outer, R, inner, splits, pop, part, stream));
  typedef typename std::conditional<
      std::is_same<A, float>::value, float,
      typename std::conditional<std::is_same<A, double>::value, double, int64_t>::type>::type
      ATag;
  return launch_col_any<ATag>(ws.get(), outer, splits, inner, 1, op, final_out, stream);
}

template <typename Tag>
mi_status_t launch_any(const void* in, int64_t outer, int64_t R, int64_t inner, int op,
                       RedOut o, int acc_dt, hipStream_t stream) {
  if (inner == 1) return launch_row<Tag>(in, outer, R, op, o, acc_dt, stream);
  return launch_col<Tag>(in, outer, R, inner, op, o, stream);
}

mi_status_t dispatch(int dt, const void* in, int64_t outer, int64_t R, int64_t inner, int op,
                     RedOut o, hipStream_t stream) {
  const int acc = acc_dtype_of(dt);
  switch (dt) {
    case MI_F32: return launch_any<float>(in, outer, R, inner, op, o, acc, stream);
    case MI_BF16: return launch_any<BF16>(in, outer, R, inner, op, o, acc, stream);
    case MI_F16: return launch_any<F16>(in, outer, R, inner, op, o, acc, stream);
    case MI_F64: return launch_any<double>(in, outer, R, inner, op, o, acc, stream);
    case MI_I64: return launch_any<int64_t>(in, outer, R, inner, op, o, acc, stream);
    case MI_I32: return launch_any<int32_t>(in, outer, R, inner, op, o, acc, stream);
    case MI_I16: return launch_any<int16_t>(in, outer, R, inner, op, o, acc, stream);
    case MI_I8: return launch_any<int8_t>(in, outer, R, inner, op, o, acc, stream);
    case MI_U8: return launch_any<uint8_t>(in, outer, R, inner, op, o, acc, stream);
    case MI_BOOL: return launch_any<BoolTag>(in, outer, R, inner, op, o, acc, stream);
    default: MI_FAIL(MI_ERR_UNSUPPORTED, "reduce: dtype %s", dtype_name(dt));
  }
}

mi_status_t run_reduce(int op, const mi_tensor_t* out, const mi_tensor_t* self,
                       const int64_t* dims, int32_t ndims, int32_t keepdim, hipStream_t stream) {
  clear_error();
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(self, "self"));
  const int nd = self->ndim;
  bool red[MI_MAX_DIMS] = {};
  if (ndims == 0) {
    for (int d = 0; d < nd; ++d) red[d] = true;
  } else {
    MI_CHECK_ARG(dims != nullptr, "reduce: dims is NULL");
    for (int k = 0; k < ndims; ++k) {
      int64_t d = dims[k];
      const int lim = nd == 0 ? 1 : nd;
      if (d < 0) d += lim;
      MI_CHECK_ARG(d >= 0 && d < lim, "reduce: dim %lld out of range", (long long)dims[k]);
      if (nd > 0) {
        MI_CHECK_ARG(!red[d], "reduce: dim %lld appears multiple times in the list of dims",
                     (long long)d);
        red[d] = true;
      }
    }
  }
  int64_t outer_n = 1, R = 1;
  for (int d = 0; d < nd; ++d) (red[d] ? R : outer_n) *= self->sizes[d];
  MI_CHECK_ARG(numel(*out) == outer_n, "reduce: out has %lld elements, expected %lld",
               (long long)numel(*out), (long long)outer_n);
  if (op == R_MEAN) {
    MI_CHECK_ARG(is_floating(out->dtype),
                 "mean(): could not infer output dtype. Input dtype must be either a floating "
                 "point or complex dtype. Got: %s", dtype_name(out->dtype));
  }
  if (outer_n == 0) return MI_OK;
  if (R == 0) {
    MI_CHECK_ARG(op != R_MAX,
                 "amax(): Expected reduction dim to have non-zero size.");
    mi_scalar_t v{};
    v.dtype = MI_F64;
    v.f = op == R_MEAN ? NAN : 0.0;
    v.wrapped = 1;
    return mi_fill(out, v, (mi_stream_t)stream);
  }
  (void)keepdim;
  // Find [outer, R, inner] over a dense self, else permute into workspace.
  int first = -1, last = -1;
  for (int d = 0; d < nd; ++d)
    if (red[d] && self->sizes[d] != 1) {
      if (first < 0) first = d;
      last = d;
    }
  bool block = true;
  for (int d = first; d >= 0 && d <= last; ++d)
    if (!red[d] && self->sizes[d] != 1) block = false;
  int64_t outer = 1, inner = 1;
  const void* src = self->data;
  Workspace perm_ws;
  if (first < 0) {  // all reduced dims have size 1: plain copy/convert
    outer = outer_n;
    R = 1;
    inner = 1;
  }
  if (!(block && is_contiguous(*self))) {
    // dense copy in order [kept dims..., reduced dims...]
    mi_tensor_t pv{}, dst{};
    pv.data = self->data;
    pv.dtype = self->dtype;
    int k = 0;
    for (int d = 0; d < nd; ++d)
      if (!red[d]) {
        pv.sizes[k] = self->sizes[d];
        pv.strides[k++] = self->strides[d];
      }
    for (int d = 0; d < nd; ++d)
      if (red[d]) {
        pv.sizes[k] = self->sizes[d];
        pv.strides[k++] = self->strides[d];
      }
    pv.ndim = nd;
    dst = pv;
    MI_RETURN_IF(perm_ws.alloc((size_t)numel(*self) * dtype_size(self->dtype), stream));
    dst.data = perm_ws.get();
    int64_t st = 1;
    for (int d = nd - 1; d >= 0; --d) {
      dst.strides[d] = st;
      st *= dst.sizes[d];
    }
    MI_RETURN_IF(mi_copy(&dst, &pv, (mi_stream_t)stream));
    src = perm_ws.get();
    outer = outer_n;
    inner = 1;
  } else if (first >= 0) {
    for (int d = 0; d < first; ++d) outer *= self->sizes[d];
    for (int d = last + 1; d < nd; ++d) inner *= self->sizes[d];
  }
  // Output: dense in kept-dim order, else compute into workspace then copy.
  Workspace out_ws;
  RedOut o{out->data, out->dtype, (double)R};
  const bool out_dense = is_contiguous(*out);
  if (!out_dense) {
    MI_RETURN_IF(out_ws.alloc((size_t)outer_n * dtype_size(out->dtype), stream));
    o.data = out_ws.get();
  }
  MI_RETURN_IF(dispatch(self->dtype, src, outer, R, inner, op, o, stream));
  if (!out_dense) {
    mi_tensor_t tmp = *out;
    tmp.data = out_ws.get();
    int64_t st = 1;
    for (int d = tmp.ndim - 1; d >= 0; --d) {
      tmp.strides[d] = st;
      st *= tmp.sizes[d];
    }
    MI_RETURN_IF(mi_copy(out, &tmp, (mi_stream_t)stream));
  }
  return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

mi_status_t mi_sum(const mi_tensor_t* out, const mi_tensor_t* self, const int64_t* dims,
                   int32_t ndims, int32_t keepdim, mi_stream_t stream) {
  return run_reduce(R_SUM, out, self, dims, ndims, keepdim, (hipStream_t)stream);
}

mi_status_t mi_amax(const mi_tensor_t* out, const mi_tensor_t* self, const int64_t* dims,
                    int32_t ndims, int32_t keepdim, mi_stream_t stream) {
  return run_reduce(R_MAX, out, self, dims, ndims, keepdim, (hipStream_t)stream);
}

mi_status_t mi_mean(const mi_tensor_t* out, const mi_tensor_t* self, const int64_t* dims,
                    int32_t ndims, int32_t keepdim, mi_stream_t stream) {
  return run_reduce(R_MEAN, out, self, dims, ndims, keepdim, (hipStream_t)stream);
}

}  // extern "C"
