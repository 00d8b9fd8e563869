// Fused efficient ops: RMSNorm, rotate-half RoPE, SiLU-mul.
//
// All three are HBM-bound (config 3 at 16384 tokens x 4096 hidden, bf16):
//   rms_norm  reads x once and writes y once: one wave per row holds the row
//             in registers (4096 bf16 = 8 x 16-byte vectors per lane), so the
//             sum of squares and the scaling share a single HBM read;
//   rope      a block computes the cos/sin tables of its few tokens once into
//             LDS (one sincosf per token and pair, shared by all 2 x 32
//             heads) while the tokens' q and k rows load, then rotates and
//             stores them;
//   silu_mul  streams gate and up with four 16-byte vectors per operand in
//             flight per lane; silu uses the hardware exp2 and reciprocal.
// Arithmetic is fp32 with one rounding to the output type, which is what
// torch.rms_norm's CPU kernel does for bf16 (upcast, x * rsqrt(mean(x^2) +
// eps) * w, one cast) and what the fp32 closed forms of RoPE and SiLU-mul do.
#include <algorithm>
#include <cmath>

#include "iter.h"

namespace mi {
namespace {

template <typename Tag>
struct FT {
  typedef Tag storage;
  static __device__ __forceinline__ float load(storage v) { return (float)v; }
  static __device__ __forceinline__ storage store(float v) { return (storage)v; }
};
template <>
struct FT<BF16> {
  typedef uint16_t storage;
  static __device__ __forceinline__ float load(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_bf16(v); }
};
template <>
struct FT<F16> {
  typedef uint16_t storage;
  static __device__ __forceinline__ float load(uint16_t v) { return f16_to_f32(v); }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_f16(v); }
};

// ---- RMSNorm ------------------------------------------------------------------

// One wave per row, VPL 16-byte vectors per lane.  The weight is copied into
// LDS once per block (dynamic, H / VEC 16-byte words) and read from there:
// read per row from L2 under the store guard, each piece's load was waited
// for in turn (the layer-norm forward's parameters measured 51.8 -> 47.5 us
// the same way).
template <typename Tag, int VPL, bool HAS_W>
__global__ __launch_bounds__(256) void rms_norm_wave_kernel(
    typename FT<Tag>::storage* __restrict__ out, const typename FT<Tag>::storage* __restrict__ x,
    const typename FT<Tag>::storage* __restrict__ w, int64_t rows, int64_t H,
    int64_t x_row_stride, int64_t out_row_stride, float eps) {
  typedef typename FT<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  union V {
    uint4 u;
    St s[VEC];
  };
  extern __shared__ uint4 wl[];
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t nv = H / VEC;
  if constexpr (HAS_W) {
    for (int64_t i = threadIdx.x; i < nv; i += 256) wl[i] = ((const uint4*)w)[i];
    __syncthreads();
  }
  if (row >= rows) return;
  const V* px = (const V*)(x + row * x_row_stride);
  // every load of the row is issued before the first sum (a sum inside the
  // guarded load loop makes each load wait for the one before it)
  V v[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int64_t i = lane + (int64_t)k * 64;
    if (i < nv) v[k] = ld_stream(px + i);
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k)
    if (lane + (int64_t)k * 64 < nv)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float f = FT<Tag>::load(v[k].s[e]);
        ss += f * f;
      }
  ss = wave_sum(ss);
  const float r = 1.0f / __builtin_sqrtf(ss / (float)H + eps);
  V* po = (V*)(out + row * out_row_stride);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int64_t i = lane + (int64_t)k * 64;
    if (i < nv) {
      V o, wv;
      if (HAS_W) wv.u = wl[i];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float y = FT<Tag>::load(v[k].s[e]) * r;
        if (HAS_W) y = y * FT<Tag>::load(wv.s[e]);
        o.s[e] = FT<Tag>::store(y);
      }
      st_stream(po + i, o);
    }
  }
}

// Any width: block per row, two reads of the row.
template <typename Tag>
__global__ __launch_bounds__(256) void rms_norm_block_kernel(
    typename FT<Tag>::storage* __restrict__ out, const typename FT<Tag>::storage* __restrict__ x,
    const void* __restrict__ w, int w_dtype, int64_t H, int64_t x_row_stride,
    int64_t out_row_stride, float eps) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const typename FT<Tag>::storage* px = x + row * x_row_stride;
  float ss = 0.f;
  for (int64_t j = threadIdx.x; j < H; j += 256) {
    const float f = FT<Tag>::load(px[j]);
    ss += f * f;
  }
  ss = block_sum(ss, red);
  const float r = 1.0f / __builtin_sqrtf(ss / (float)H + eps);
  typename FT<Tag>::storage* po = out + row * out_row_stride;
  for (int64_t j = threadIdx.x; j < H; j += 256) {
    float y = FT<Tag>::load(px[j]) * r;
    if (w) y = y * load_as<float>(w, j, w_dtype);
    po[j] = FT<Tag>::store(y);
  }
}

// Rows of a [.., H] tensor with last stride 1: returns the row count and the
// uniform row stride, or false when the leading dims do not collapse.
bool as_rows(const mi_tensor_t& t, int64_t* rows, int64_t* row_stride) {
  if (t.ndim == 0) return false;
  if (t.sizes[t.ndim - 1] > 1 && t.strides[t.ndim - 1] != 1) return false;
  const int64_t H = t.sizes[t.ndim - 1];
  int64_t r = 1, st = -1, expect = -1;
  for (int d = t.ndim - 2; d >= 0; --d) {
    if (t.sizes[d] == 1) continue;
    if (st < 0) {
      st = t.strides[d];
      expect = st * t.sizes[d];
    } else {
      if (t.strides[d] != expect) return false;
      expect *= t.sizes[d];
    }
    r *= t.sizes[d];
  }
  *rows = r;
  *row_stride = st < 0 ? H : st;
  return true;
}

template <typename Tag>
mi_status_t rms_norm_t(const mi_tensor_t* out, const mi_tensor_t* x, const mi_tensor_t* w,
                       float eps, hipStream_t stream) {
  typedef typename FT<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  const int64_t H = x->sizes[x->ndim - 1];
  int64_t rows, xs, os;
  if (!as_rows(*x, &rows, &xs) || !as_rows(*out, &rows, &os))
    MI_FAIL(MI_ERR_UNSUPPORTED, "rms_norm: rows of x/out must have a uniform stride");
  if (rows == 0 || H == 0) return MI_OK;
  const bool has_w = w != nullptr && w->data != nullptr;
  const bool w_same = !has_w || (w->dtype == x->dtype && (w->ndim == 0 || w->strides[w->ndim - 1] == 1));
  const bool aligned = (uintptr_t)x->data % 16 == 0 && (uintptr_t)out->data % 16 == 0 &&
                       (!has_w || (uintptr_t)w->data % 16 == 0) && H % VEC == 0 &&
                       xs % VEC == 0 && os % VEC == 0;
  const int64_t nv = H / VEC;
  if (aligned && w_same && nv <= 64 * 16) {
    auto go = [&](auto vpl_c) -> mi_status_t {
      constexpr int VPL = decltype(vpl_c)::value;
      const unsigned grid = ceil_div_u(rows, 4);
      if (has_w)
        hipLaunchKernelGGL((rms_norm_wave_kernel<Tag, VPL, true>), dim3(grid), dim3(256),
                           (size_t)(H / (16 / sizeof(St))) * 16, stream, (St*)out->data,
                           (const St*)x->data, (const St*)w->data, rows, H, xs, os, eps);
      else
        hipLaunchKernelGGL((rms_norm_wave_kernel<Tag, VPL, false>), dim3(grid), dim3(256), 0,
                           stream, (St*)out->data, (const St*)x->data, (const St*)nullptr, rows,
                           H, xs, os, eps);
      return check_launch("rms_norm_wave");
    };
    if (nv <= 64) return go(std::integral_constant<int, 1>());
    if (nv <= 128) return go(std::integral_constant<int, 2>());
    if (nv <= 256) return go(std::integral_constant<int, 4>());
    if (nv <= 512) return go(std::integral_constant<int, 8>());
    return go(std::integral_constant<int, 16>());
  }
  if (has_w && w->ndim > 0 && w->strides[w->ndim - 1] != 1 && w->sizes[w->ndim - 1] > 1)
    MI_FAIL(MI_ERR_UNSUPPORTED, "rms_norm: weight must be dense");
  hipLaunchKernelGGL((rms_norm_block_kernel<Tag>), dim3((unsigned)rows), dim3(256), 0, stream,
                     (St*)out->data, (const St*)x->data, has_w ? w->data : nullptr,
                     has_w ? w->dtype : MI_F32, H, xs, os, eps);
  return check_launch("rms_norm_block");
}

// ---- RoPE -----------------------------------------------------------------------

struct RopeTensor {
  void* out;
  const void* in;
  int64_t heads;
  int64_t in_tok_stride, in_head_stride;
  int64_t out_tok_stride, out_head_stride;
};

// A block owns `tpb` consecutive tokens.  A job is one (tensor, head, slice
// of P pairs) of a token and reads the two 16-byte halves x1 = x[j*P ..],
// x2 = x[half + j*P ..]; the jobs of a token are numbered head-major (q heads
// first), so a wave's loads cover 8 heads x 256 B of one token row
// contiguously.  Lane l takes jobs l, l + 256, ... (NJ of them) of every
// token, so their (tensor, head, slice) decode is done once per block and a
// token step is a stride addition.  The lanes issue their first loads, then
// build the tokens' fp32 cos/sin tables in LDS (one sincosf per token and
// pair, as the fp32 closed form does, with inv_freq computed once per
// block), then stream the tokens with eight jobs in flight per lane.
constexpr int kRopeInflight = 8;

template <typename Tag, typename PosT, int NJ>
__global__ __launch_bounds__(256) void rope_kernel(RopeTensor q, RopeTensor k, const PosT* pos,
                                                   int64_t pos_stride, int64_t tokens, int half,
                                                   int tpb, float theta_f, float dim_f) {
  typedef typename FT<Tag>::storage St;
  constexpr int P = 16 / sizeof(St);
  constexpr int TB = kRopeInflight / NJ > 0 ? kRopeInflight / NJ : 1;  // tokens per batch
  union V {
    uint4 u;
    St s[P];
  };
  extern __shared__ float rope_cs[];
  const int64_t t0 = (int64_t)blockIdx.x * tpb;
  const int nt = (int)min((int64_t)tpb, tokens - t0);
  float* cs_c = rope_cs;
  float* cs_s = rope_cs + tpb * half;
  float* inv_freq = rope_cs + 2 * tpb * half;
  const int slices = half / P;
  const int jq = q.in ? (int)q.heads * slices : 0;
  const int jpt = jq + (k.in ? (int)k.heads * slices : 0);

  // the lane's job slots, decoded once
  const St* in0[NJ];
  St* out0[NJ];
  int64_t ist[NJ], ost[NJ];
  int cso[NJ];
  bool live[NJ];
#pragma unroll
  for (int m = 0; m < NJ; ++m) {
    const int j = threadIdx.x + 256 * m;
    live[m] = j < jpt;
    int r = live[m] ? j : 0;
    const bool isk = r >= jq;
    if (isk) r -= jq;
    const RopeTensor& rt = isk ? k : q;
    const int h = r / slices, sl = r - h * slices;
    in0[m] = (const St*)rt.in + t0 * rt.in_tok_stride + h * rt.in_head_stride + sl * P;
    out0[m] = (St*)rt.out + t0 * rt.out_tok_stride + h * rt.out_head_stride + sl * P;
    ist[m] = rt.in_tok_stride;
    ost[m] = rt.out_tok_stride;
    cso[m] = sl * P;
  }
  V xa[TB][NJ], xb[TB][NJ];
  auto fetch = [&](int tt0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < TB; ++u) {
      const int tt = tt0 + u;
#pragma unroll
      for (int m = 0; m < NJ; ++m) {
        if (tt < nt && live[m]) {
          const St* in = in0[m] + tt * ist[m];
          xa[u][m] = ld_stream((const V*)in);
          xb[u][m] = ld_stream((const V*)(in + half));
        }
      }
    }
  };
  // the first batch of loads is in flight while the cos/sin tables are built
  fetch(0);
  for (int i = threadIdx.x; i < half; i += 256)
    inv_freq[i] = 1.0f / powf(theta_f, (float)(2 * i) / dim_f);  // 1 / theta^(2i/d), fp32
  __syncthreads();
  for (int idx = threadIdx.x; idx < nt * half; idx += 256) {
    const int tt = idx / half, i = idx - tt * half;
    const float p = (float)pos[(t0 + tt) * pos_stride];
    sincosf(p * inv_freq[i], &cs_s[idx], &cs_c[idx]);
  }
  __syncthreads();
  for (int tt0 = 0; tt0 < nt; tt0 += TB) {
    if (tt0 > 0) fetch(tt0);
#pragma unroll
    for (int u = 0; u < TB; ++u) {
      const int tt = tt0 + u;
#pragma unroll
      for (int m = 0; m < NJ; ++m) {
        if (tt < nt && live[m]) {
          const int ci = tt * half + cso[m];
          V oa, ob;
#pragma unroll
          for (int e = 0; e < P; ++e) {
            const float c = cs_c[ci + e], sn = cs_s[ci + e];
            const float x1 = FT<Tag>::load(xa[u][m].s[e]), x2 = FT<Tag>::load(xb[u][m].s[e]);
            oa.s[e] = FT<Tag>::store(x1 * c - x2 * sn);
            ob.s[e] = FT<Tag>::store(x2 * c + x1 * sn);
          }
          St* o = out0[m] + tt * ost[m];
          st_stream((V*)o, oa);
          st_stream((V*)(o + half), ob);
        }
      }
    }
  }
}

mi_status_t rope_view(const mi_tensor_t* o, const mi_tensor_t* in, int64_t tokens, int64_t D,
                      int esz, RopeTensor* r, const char* name) {
  if (in == nullptr || in->data == nullptr) {
    *r = RopeTensor{nullptr, nullptr, 0, 0, 0, 0, 0};
    return MI_OK;
  }
  MI_RETURN_IF(validate(in, name));
  MI_CHECK_ARG(o != nullptr && o->data != nullptr, "rope: %s output missing", name);
  MI_RETURN_IF(validate(o, name));
  MI_CHECK_ARG(in->ndim == 3 && o->ndim == 3, "rope: %s must be [tokens, heads, head_dim]", name);
  for (int d = 0; d < 3; ++d)
    MI_CHECK_ARG(o->sizes[d] == in->sizes[d], "rope: %s output shape mismatch", name);
  MI_CHECK_ARG(in->sizes[0] == tokens, "rope: %s has %lld tokens, positions has %lld", name,
               (long long)in->sizes[0], (long long)tokens);
  MI_CHECK_ARG(in->sizes[2] == D, "rope: q and k head_dim differ");
  MI_CHECK_ARG(in->strides[2] == 1 && o->strides[2] == 1, "rope: %s head_dim must be dense", name);
  MI_CHECK_ARG(in->dtype == o->dtype, "rope: %s dtype mismatch", name);
  const int P = 16 / esz;
  const bool aligned = (uintptr_t)in->data % 16 == 0 && (uintptr_t)o->data % 16 == 0 &&
                       in->strides[0] % P == 0 && in->strides[1] % P == 0 &&
                       o->strides[0] % P == 0 && o->strides[1] % P == 0;
  MI_CHECK_ARG(aligned, "rope: %s must be 16-byte aligned per head", name);
  *r = RopeTensor{o->data, in->data, in->sizes[1], in->strides[0], in->strides[1],
                  o->strides[0], o->strides[1]};
  return MI_OK;
}

// ---- SiLU-mul ---------------------------------------------------------------------

// The elementwise SiLU ops: silu(a) * b (the fused SwiGLU product), silu's
// derivative applied to a gradient, a * s * (1 + b * (1 - s)) with
// s = sigmoid(b), a = grad_output, b = the forward input (ATen's
// silu_backward formula, aten/src/ATen/native/cpu/Activation.cpp), and
// silu(a) itself (one operand: b is neither loaded nor used).
enum PairOp { P_SILU_MUL = 0, P_SILU_BWD = 1, P_SILU = 2 };

template <int OP>
__device__ __forceinline__ float pair_op(float a, float b) {
  if constexpr (OP == P_SILU_MUL) {
    return silu_mul_f32(a, b);
  } else if constexpr (OP == P_SILU) {
    return a * __builtin_amdgcn_rcpf(1.0f + fast_exp(-a));
  } else {
    const float sg = __builtin_amdgcn_rcpf(1.0f + fast_exp(-b));
    return a * sg * (1.0f + b * (1.0f - sg));
  }
}

template <typename Tag, int OP>
__global__ __launch_bounds__(256) void silu_mul_kernel(typename FT<Tag>::storage* __restrict__ out,
                                                       const typename FT<Tag>::storage* __restrict__ g,
                                                       const typename FT<Tag>::storage* __restrict__ u,
                                                       int64_t n) {
  typedef typename FT<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  constexpr int U = 4;
  union V {
    uint4 u;
    St s[VEC];
  };
  const int64_t nvec = n / VEC;
  const int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x;
  V vg[U], vu[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t i = base + k * 256;
    if (i < nvec) {
      vg[k] = ld_stream((const V*)g + i);
      if constexpr (OP != P_SILU) vu[k] = ld_stream((const V*)u + i);
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t i = base + k * 256;
    if (i < nvec) {
      V o;
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        o.s[e] = FT<Tag>::store(pair_op<OP>(
            FT<Tag>::load(vg[k].s[e]), OP == P_SILU ? 0.f : FT<Tag>::load(vu[k].s[e])));
      st_stream((V*)out + i, o);
    }
  }
  // tail elements
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rem = n - nvec * VEC;
  if (blockIdx.x == 0 && t < rem) {
    const int64_t i = nvec * VEC + t;
    out[i] = FT<Tag>::store(pair_op<OP>(FT<Tag>::load(g[i]), OP == P_SILU ? 0.f : FT<Tag>::load(u[i])));
  }
}

template <typename Tag, int OP>
__global__ __launch_bounds__(256) void silu_mul_strided_kernel(char* out, const char* g,
                                                               const char* u, OffsetCalc<3> oc,
                                                               int64_t n) {
  typedef typename FT<Tag>::storage St;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    int64_t off[3];
    oc.get(i, off);
    ((St*)out)[off[0]] = FT<Tag>::store(pair_op<OP>(
        FT<Tag>::load(((const St*)g)[off[1]]), OP == P_SILU ? 0.f : FT<Tag>::load(((const St*)u)[off[2]])));
  }
}

template <typename Tag, int OP>
mi_status_t silu_mul_t(const mi_tensor_t* out, const mi_tensor_t* g, const mi_tensor_t* u,
                       hipStream_t stream) {
  typedef typename FT<Tag>::storage St;
  const mi_tensor_t* ins[2] = {g, u};
  Iter it;
  MI_RETURN_IF(make_iter(it, *out, ins, 2));
  if (it.numel == 0) return MI_OK;
  if (it.op_contiguous(0) && it.op_contiguous(1) && it.op_contiguous(2) &&
      (((uintptr_t)it.data[0] | (uintptr_t)it.data[1] | (uintptr_t)it.data[2]) % 16) == 0) {
    constexpr int VEC = 16 / sizeof(St);
    const int64_t nvec = it.numel / VEC;
    const unsigned grid = nvec > 0 ? ceil_div_u(nvec, 256 * 4) : 1;
    hipLaunchKernelGGL((silu_mul_kernel<Tag, OP>), dim3(grid), dim3(256), 0, stream, (St*)it.data[0],
                       (const St*)it.data[1], (const St*)it.data[2], it.numel);
    return check_launch("silu_mul");
  }
  OffsetCalc<3> oc = make_offset_calc<3>(it);
  const int64_t want = (it.numel + 255) / 256;
  const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
  hipLaunchKernelGGL((silu_mul_strided_kernel<Tag, OP>), dim3(grid), dim3(256), 0, stream, it.data[0],
                     (const char*)it.data[1], (const char*)it.data[2], oc, it.numel);
  return check_launch("silu_mul_strided");
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

mi_status_t mi_rms_norm(const mi_tensor_t* out, const mi_tensor_t* x, const mi_tensor_t* weight,
                        double eps, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(x, "x"));
  MI_CHECK_ARG(x->ndim >= 1, "rms_norm: x must have at least one dim");
  MI_CHECK_ARG(out->ndim == x->ndim && out->dtype == x->dtype, "rms_norm: out must match x");
  for (int d = 0; d < x->ndim; ++d)
    MI_CHECK_ARG(out->sizes[d] == x->sizes[d], "rms_norm: out shape mismatch");
  const int64_t H = x->sizes[x->ndim - 1];
  if (weight != nullptr && weight->data != nullptr) {
    MI_RETURN_IF(validate(weight, "weight"));
    MI_CHECK_ARG(numel(*weight) == H, "rms_norm: weight has %lld elements, expected %lld",
                 (long long)numel(*weight), (long long)H);
    MI_CHECK_ARG(is_contiguous(*weight), "rms_norm: weight must be dense");
  }
  switch (x->dtype) {
    case MI_BF16: return rms_norm_t<BF16>(out, x, weight, (float)eps, stream);
    case MI_F16: return rms_norm_t<F16>(out, x, weight, (float)eps, stream);
    case MI_F32: return rms_norm_t<float>(out, x, weight, (float)eps, stream);
    default: MI_FAIL(MI_ERR_UNSUPPORTED, "rms_norm: dtype %s", dtype_name(x->dtype));
  }
}

mi_status_t mi_rope(const mi_tensor_t* q_out, const mi_tensor_t* k_out, const mi_tensor_t* q,
                    const mi_tensor_t* k, const mi_tensor_t* positions, double theta,
                    mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_CHECK_ARG(q != nullptr && q->data != nullptr, "rope: q is required");
  MI_RETURN_IF(validate(q, "q"));
  MI_RETURN_IF(validate(positions, "positions"));
  MI_CHECK_ARG(positions->ndim == 1, "rope: positions must be 1-D");
  MI_CHECK_ARG(positions->dtype == MI_I64 || positions->dtype == MI_I32,
               "rope: positions must be int32 or int64");
  MI_CHECK_ARG(theta > 0.0, "rope: theta must be positive");
  MI_CHECK_ARG(q->ndim == 3, "rope: q must be [tokens, heads, head_dim]");
  const int64_t tokens = positions->sizes[0];
  const int64_t D = q->sizes[2];
  MI_CHECK_ARG(D % 2 == 0, "rope: head_dim must be even");
  const int esz = dtype_size(q->dtype);
  MI_CHECK_ARG(q->dtype == MI_BF16 || q->dtype == MI_F16 || q->dtype == MI_F32,
               "rope: dtype %s unsupported", dtype_name(q->dtype));
  const int P = 16 / esz;
  MI_CHECK_ARG((D / 2) % P == 0, "rope: head_dim/2 must be a multiple of %d", P);
  RopeTensor rq, rk;
  MI_RETURN_IF(rope_view(q_out, q, tokens, D, esz, &rq, "q"));
  MI_RETURN_IF(rope_view(k_out, k, tokens, D, esz, &rk, "k"));
  if (k != nullptr && k->data != nullptr)
    MI_CHECK_ARG(k->dtype == q->dtype, "rope: q and k dtypes differ");
  if (tokens == 0) return MI_OK;
  const int64_t half = D / 2;
  MI_CHECK_ARG(half <= 4096, "rope: head_dim %lld too large (at most 8192)", (long long)D);
  // jobs of one token (heads x slices of q and k), spread over 256 lanes
  const int64_t jpt = (rq.heads + rk.heads) * (half / P);
  MI_CHECK_ARG(jpt <= 256 * 8, "rope: %lld (head, slice) jobs per token exceed 2048",
               (long long)jpt);
  const int nj = (int)((jpt + 255) / 256);
  // tokens per block: one batch of loads (kRopeInflight / NJ tokens), so a
  // block loads, rotates, stores and exits and the next block's loads overlap
  // its stores; fewer when the cos/sin tables (2 * tpb * half fp32) plus
  // inv_freq (half fp32) would pass 64 KiB of LDS
  const int nj_t = nj == 1 ? 1 : nj == 2 ? 2 : nj <= 4 ? 4 : 8;
  const int tpb = (int)std::max<int64_t>(
      1, std::min<int64_t>(std::max(1, kRopeInflight / nj_t), (16384 / half - 1) / 2));
  const size_t lds = (size_t)(2 * tpb + 1) * half * sizeof(float);  // cos, sin, inv_freq
  const unsigned grid = ceil_div_u(tokens, tpb);
  const float l2t = (float)theta;
  const float inv_dim = (float)D;
  const int64_t ps = positions->strides[0];
#define MI_ROPE_LAUNCH2(TAG, NJ)                                                              \
  if (positions->dtype == MI_I64)                                                             \
    hipLaunchKernelGGL((rope_kernel<TAG, int64_t, NJ>), dim3(grid), dim3(256), lds, stream, rq, \
                       rk, (const int64_t*)positions->data, ps, tokens, (int)half, tpb, l2t,   \
                       inv_dim);                                                              \
  else                                                                                        \
    hipLaunchKernelGGL((rope_kernel<TAG, int32_t, NJ>), dim3(grid), dim3(256), lds, stream, rq, \
                       rk, (const int32_t*)positions->data, ps, tokens, (int)half, tpb, l2t,   \
                       inv_dim);
#define MI_ROPE_LAUNCH(TAG)                   \
  if (nj == 1) { MI_ROPE_LAUNCH2(TAG, 1) }    \
  else if (nj == 2) { MI_ROPE_LAUNCH2(TAG, 2) } \
  else if (nj <= 4) { MI_ROPE_LAUNCH2(TAG, 4) } \
  else { MI_ROPE_LAUNCH2(TAG, 8) }
  switch (q->dtype) {
    case MI_BF16: MI_ROPE_LAUNCH(BF16) break;
    case MI_F16: MI_ROPE_LAUNCH(F16) break;
    default: MI_ROPE_LAUNCH(float) break;
  }
#undef MI_ROPE_LAUNCH
#undef MI_ROPE_LAUNCH2
  return check_launch("rope");
}

mi_status_t mi_silu_mul(const mi_tensor_t* out, const mi_tensor_t* gate, const mi_tensor_t* up,
                        mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(gate, "gate"));
  MI_RETURN_IF(validate(up, "up"));
  MI_CHECK_ARG(gate->dtype == up->dtype && out->dtype == gate->dtype,
               "silu_mul: gate, up and out must share a dtype");
  switch (out->dtype) {
    case MI_BF16: return silu_mul_t<BF16, P_SILU_MUL>(out, gate, up, stream);
    case MI_F16: return silu_mul_t<F16, P_SILU_MUL>(out, gate, up, stream);
    case MI_F32: return silu_mul_t<float, P_SILU_MUL>(out, gate, up, stream);
    default: MI_FAIL(MI_ERR_UNSUPPORTED, "silu_mul: dtype %s", dtype_name(out->dtype));
  }
}

mi_status_t mi_silu(const mi_tensor_t* out, const mi_tensor_t* self, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(self, "self"));
  MI_CHECK_ARG(out->dtype == self->dtype, "silu: self and out must share a dtype");
  // self is passed as both operands of the pair iterator; the kernels read it once
  switch (out->dtype) {
    case MI_BF16: return silu_mul_t<BF16, P_SILU>(out, self, self, stream);
    case MI_F16: return silu_mul_t<F16, P_SILU>(out, self, self, stream);
    case MI_F32: return silu_mul_t<float, P_SILU>(out, self, self, stream);
    default: MI_FAIL(MI_ERR_UNSUPPORTED, "silu: dtype %s", dtype_name(out->dtype));
  }
}

mi_status_t mi_silu_backward(const mi_tensor_t* grad_input, const mi_tensor_t* grad_output,
                             const mi_tensor_t* self, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(grad_input, "grad_input"));
  MI_RETURN_IF(validate(grad_output, "grad_output"));
  MI_RETURN_IF(validate(self, "self"));
  MI_CHECK_ARG(grad_output->dtype == self->dtype && grad_input->dtype == self->dtype,
               "silu_backward: grad_input, grad_output and self must share a dtype");
  switch (self->dtype) {
    case MI_BF16: return silu_mul_t<BF16, P_SILU_BWD>(grad_input, grad_output, self, stream);
    case MI_F16: return silu_mul_t<F16, P_SILU_BWD>(grad_input, grad_output, self, stream);
    case MI_F32: return silu_mul_t<float, P_SILU_BWD>(grad_input, grad_output, self, stream);
    default: MI_FAIL(MI_ERR_UNSUPPORTED, "silu_backward: dtype %s", dtype_name(self->dtype));
  }
}

}  // extern "C"
