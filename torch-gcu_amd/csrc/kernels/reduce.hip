// Reductions sum / amax / mean over arbitrary dims.
//
// The host maps self to [outer, R, inner] (R = product of the reduced dims,
// which must form one dense block; otherwise a permuted dense copy is made
// in workspace first):
//   - inner == 1 ("row" reduction, e.g. config 2's bf16 [8192, 32000] over
//     the last dim): one 512-lane block per row, 16-byte non-temporal loads,
//     eight in flight per lane, wave64 shuffle reduction then a combine of
//     the eight wave results.  Long rows with few of them are split over
//     several blocks and finished by a second pass over the partials.
//   - inner > 1 ("column" reduction, e.g. fp32 [16384, 4096] over dim 0):
//     lanes own 16-byte column vectors side by side, so a 256-lane block
//     reads 4 KiB contiguous per row; the rows are split into chunks over
//     blocks (partials in workspace, then a second pass), about 4 blocks per
//     CU for a 4096-wide output.
// Floating inputs accumulate in float (double for f64), integers in int64.
#include <algorithm>
#include <cmath>
#include <mutex>
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
// The same with the operation fixed at compile time (MX: max, else sum).  In
// the column kernels the run-time form became a scalar branch and a wait per
// element, so every add waited for its own load.
template <bool MX, typename A>
__device__ __forceinline__ A red_comb(A a, A b) {
  if constexpr (MX) return nan_max(a, b);
  else return a + b;
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

constexpr int kRowBlock = 512;
constexpr int kRowUnroll = 8;

// rows x [R] -> rows x splits partials (or final when splits == 1).
// Block (row, split) reduces elements [split*chunk, min(R, (split+1)*chunk)):
// 512 lanes, eight 16-byte non-temporal loads in flight per lane (a config-2
// row of 64,000 B is one batch), a wave64 shuffle reduction, then the
// per-wave results in a fixed order.  The loads are unconditional (a vector
// past the end re-reads the last one, whose values are then not added) and
// the operation is fixed at compile time (MX: max, else sum), so the eight
// loads are issued back to back and the adds wait on them in turn.
template <typename Tag, bool MX>
__global__ __launch_bounds__(kRowBlock) void row_reduce_kernel(
    const typename RT<Tag>::storage* __restrict__ in, int64_t R, int64_t row_stride,
    int64_t chunk, int op, RedOut out) {
  typedef typename RT<Tag>::storage St;
  typedef typename RT<Tag>::acc A;
  constexpr int VEC = 16 / sizeof(St) > 0 ? 16 / sizeof(St) : 1;
  __shared__ A red[kRowBlock / 64];
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
    for (int64_t v0 = threadIdx.x; v0 < nv; v0 += (int64_t)kRowBlock * kRowUnroll) {
      V x[kRowUnroll];
      bool ok[kRowUnroll];
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        const int64_t v = v0 + (int64_t)u * kRowBlock;
        ok[u] = v < nv;
        x[u] = ld_stream(pv + (ok[u] ? v : nv - 1));
      }
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        if (ok[u]) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc = red_comb<MX>(acc, RT<Tag>::load(x[u].s[e]));
        }
      }
    }
    i = beg + nv * VEC;
  }
  for (int64_t j = i + threadIdx.x; j < end; j += kRowBlock)
    acc = red_comb<MX>(acc, RT<Tag>::load(p[j]));
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

constexpr int kColUnroll = 4;  // rows a batch for narrow loads (two batches in flight)

// [outer, R, inner] column reduction over R, first pass: NTH lanes (256, 512
// or 1024) side by side along a row (a lane owns VEC adjacent columns, so a
// block reads NTH * VEC contiguous elements of each row: up to a whole
// 16 KiB row of config 2's fp32 [16384, 4096]), each walking the rows of its
// split in batches of U rows, two batches in flight (U = 2 for 16-byte
// loads, kColUnroll for narrower ones).  Output layout [outer, splits,
// inner] (Acc partials, or the final value when there is one split).
// (On config 2's mean(0), 1024-lane blocks with two 16-byte loads a batch
// ran the pass in 40.2 us, against 42.7 us for 256-lane blocks with four
// and 43.9 us for 1024 lanes with eight: whole-row blocks read each row as
// one 16 KiB run, and more loads in flight only queued.)
template <typename Tag, int VEC, int NTH, bool MX>
__global__ __launch_bounds__(NTH) void col_reduce_kernel(
    const typename RT<Tag>::storage* __restrict__ in, int64_t R, int64_t inner,
    int64_t chunk, int op, RedOut out) {
  typedef typename RT<Tag>::storage St;
  typedef typename RT<Tag>::acc A;
  const int64_t ncv = inner / VEC;  // column vectors
  const int64_t ncb = (ncv + NTH - 1) / NTH;
  const int64_t o = blockIdx.x / ncb;
  const int64_t cv = (blockIdx.x - o * ncb) * NTH + threadIdx.x;
  if (cv >= ncv) return;
  const int64_t split = blockIdx.y;
  const int64_t beg = split * chunk;
  const int64_t end = beg + chunk < R ? beg + chunk : R;
  A acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = red_ident<A>(op);
  union alignas(VEC * sizeof(St)) V {  // the host checked this alignment
    St s[VEC];
  };
  const V* base = (const V*)(in + (o * R) * inner) + cv;
  int64_t r = beg;
  // two batches of U rows: the loads of batch b + 1 are issued before batch
  // b is added, so up to 2 U loads are in flight; rows are still added in
  // ascending order
  constexpr int U = sizeof(V) == 16 ? 2 : kColUnroll;
  V xa[U], xb[U];
  auto fetch = [&](V* x, int64_t r0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (sizeof(V) == 16) x[u] = ld_stream(base + (r0 + u) * ncv);
      else x[u] = base[(r0 + u) * ncv];
    }
  };
  auto add = [&](const V* x) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = red_comb<MX>(acc[e], RT<Tag>::load(x[u].s[e]));
  };
  if (r + U <= end) {
    fetch(xa, r);
    while (true) {
      const bool nb = r + 2 * U <= end;
      if (nb) fetch(xb, r + U);
      add(xa);
      r += U;
      if (!nb) break;
      const bool na = r + 2 * U <= end;
      if (na) fetch(xa, r + U);
      add(xb);
      r += U;
      if (!na) break;
    }
  }
  for (; r < end; ++r) {
    const V x = base[r * ncv];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = red_comb<MX>(acc[e], RT<Tag>::load(x.s[e]));
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e)
    red_store(out, op, (o * gridDim.y + split) * inner + cv * VEC + e, acc[e]);
}

// Second pass over Acc partials [outer, S, inner]: a block is 16 columns x
// 16 lanes down the S partials; the 16 lane results are combined in a fixed
// order through LDS, so the result does not depend on scheduling.
// (Loads are unconditional: a lane past the last column reads the last one
// and stores nothing; loads under the guard were each waited for in turn.)
template <typename A, bool MX>
__global__ __launch_bounds__(256) void col_finish_kernel(const A* __restrict__ part, int64_t outer,
                                                         int64_t S, int64_t inner, int op,
                                                         RedOut out) {
  __shared__ A red[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t total = outer * inner;
  const int64_t cl = (int64_t)blockIdx.x * 16 + tx;  // flattened (outer, inner) column
  const bool live = cl < total;
  const int64_t c = live ? cl : total - 1;
  A acc = red_ident<A>(op);
  {
    const int64_t o = c / inner, i = c - o * inner;
    const A* p = part + o * S * inner + i;
    int64_t s = ty;
    // 16 loads in flight: 256 partials (config 2's split count) in one round
    for (; s + 240 < S; s += 256) {
      A x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = p[(s + 16 * u) * inner];
#pragma unroll
      for (int u = 0; u < 16; ++u) acc = red_comb<MX>(acc, x[u]);
    }
    for (; s < S; s += 16) acc = red_comb<MX>(acc, p[s * inner]);
  }
  red[ty][tx] = acc;
  __syncthreads();
  if (ty == 0 && live) {
    A r = red[0][tx];
#pragma unroll
    for (int y = 1; y < 16; ++y) r = red_comb<MX>(r, red[y][tx]);
    red_store(out, op, c, r);
  }
}

// The same second pass for fp32 partials with inner % 4 == 0: a block is 16
// column vectors (64 columns, 256-byte runs of each partial row) x 16 lanes
// down S, float4 loads eight at a time; each column is added in the same
// order as col_finish_kernel's (lane ty takes s = ty, ty + 16, ... in
// ascending order, then the 16 lanes in order), so the results are the same.
// (Config 2's mean(0) finish over 256 partial rows: 3.0 us against 3.2 us.)
template <bool MX>
__global__ __launch_bounds__(256) void col_finish_v4_kernel(const float* __restrict__ part,
                                                            int64_t outer, int64_t S,
                                                            int64_t inner, int op, RedOut out) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  __shared__ f4 red[16][16];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t ncv = inner / 4, total = outer * ncv;
  const int64_t cl = (int64_t)blockIdx.x * 16 + tx;  // flattened (outer, column vector)
  const bool live = cl < total;
  const int64_t cvf = live ? cl : total - 1;  // loads unconditional, as above
  const float id = red_ident<float>(op);
  f4 acc = {id, id, id, id};
  auto comb = [](f4 a, f4 b) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = red_comb<MX>(a[e], b[e]);
    return a;
  };
  {
    const int64_t o = cvf / ncv, iv = cvf - o * ncv;
    const f4* p = (const f4*)(part + o * S * inner) + iv;
    int64_t s = ty;
    for (; s + 112 < S; s += 128) {
      f4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = p[(s + 16 * u) * ncv];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = comb(acc, x[u]);
    }
    for (; s < S; s += 16) acc = comb(acc, p[s * ncv]);
  }
  red[ty][tx] = acc;
  __syncthreads();
  if (ty == 0 && live) {
    f4 r = red[0][tx];
#pragma unroll
    for (int y = 1; y < 16; ++y) r = comb(r, red[y][tx]);
#pragma unroll
    for (int e = 0; e < 4; ++e) red_store(out, op, cvf * 4 + e, r[e]);
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
    if (op == R_MAX)
      hipLaunchKernelGGL((row_reduce_kernel<Tag, true>), dim3((unsigned)outer, 1), dim3(kRowBlock),
                         0, stream, (const typename RT<Tag>::storage*)in, R, R, chunk, op,
                         final_out);
    else
      hipLaunchKernelGGL((row_reduce_kernel<Tag, false>), dim3((unsigned)outer, 1),
                         dim3(kRowBlock), 0, stream, (const typename RT<Tag>::storage*)in, R, R,
                         chunk, op, final_out);
    return check_launch("row_reduce");
  }
  Workspace ws;
  MI_RETURN_IF(ws.alloc((size_t)(outer * splits) * sizeof(A), stream));
  RedOut part{ws.get(), -1, 1.0};
  const int pop = op == R_MEAN ? R_SUM : op;
  if (pop == R_MAX)
    hipLaunchKernelGGL((row_reduce_kernel<Tag, true>), dim3((unsigned)outer, (unsigned)splits),
                       dim3(kRowBlock), 0, stream, (const typename RT<Tag>::storage*)in, R, R,
                       chunk, pop, part);
  else
    hipLaunchKernelGGL((row_reduce_kernel<Tag, false>), dim3((unsigned)outer, (unsigned)splits),
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

// Lanes of a column block: the narrowest of 256 / 512 / 1024 that covers a
// row's column vectors (1024 at most).
inline int col_block_lanes(int64_t ncv) { return ncv > 512 ? 1024 : (ncv > 256 ? 512 : 256); }

template <typename Tag, int VEC, int NTH>
mi_status_t launch_col_vn(const void* in, int64_t outer, int64_t R, int64_t inner, int64_t chunk,
                          int64_t splits, int op, RedOut o, hipStream_t stream) {
  const int64_t ncv = inner / VEC;
  dim3 grid((unsigned)(ceil_div_u(ncv, NTH) * outer), (unsigned)splits, 1);
  if (op == R_MAX)
    hipLaunchKernelGGL((col_reduce_kernel<Tag, VEC, NTH, true>), grid, dim3(NTH), 0, stream,
                       (const typename RT<Tag>::storage*)in, R, inner, chunk, op, o);
  else
    hipLaunchKernelGGL((col_reduce_kernel<Tag, VEC, NTH, false>), grid, dim3(NTH), 0, stream,
                       (const typename RT<Tag>::storage*)in, R, inner, chunk, op, o);
  return check_launch("col_reduce");
}

template <typename Tag, int VEC>
mi_status_t launch_col_v(const void* in, int64_t outer, int64_t R, int64_t inner, int64_t chunk,
                         int64_t splits, int op, RedOut o, hipStream_t stream) {
  switch (col_block_lanes(inner / VEC)) {
    case 1024: return launch_col_vn<Tag, VEC, 1024>(in, outer, R, inner, chunk, splits, op, o, stream);
    case 512: return launch_col_vn<Tag, VEC, 512>(in, outer, R, inner, chunk, splits, op, o, stream);
    default: return launch_col_vn<Tag, VEC, 256>(in, outer, R, inner, chunk, splits, op, o, stream);
  }
}

template <typename Tag>
mi_status_t launch_col_any(const void* in, int64_t outer, int64_t R, int64_t inner, int64_t chunk,
                           int64_t splits, int op, RedOut o, hipStream_t stream) {
  typedef typename RT<Tag>::storage St;
  constexpr int V = 16 / sizeof(St) >= 4 ? 4 : 16 / sizeof(St);
  if (inner % V == 0 && ((uintptr_t)in % (V * sizeof(St))) == 0)
    return launch_col_v<Tag, V>(in, outer, R, inner, chunk, splits, op, o, stream);
  return launch_col_v<Tag, 1>(in, outer, R, inner, chunk, splits, op, o, stream);
}

// Splits R so that about 16 waves per CU are in flight (config 2's fp32
// [16384, 4096] mean(0): one 1024-lane column block x 256 splits of 64 rows),
// then combines the partials in a second pass.
template <typename Tag>
mi_status_t launch_col(const void* in, int64_t outer, int64_t R, int64_t inner, int op,
                       RedOut final_out, hipStream_t stream) {
  typedef typename RT<Tag>::acc A;
  typedef typename RT<Tag>::storage St;
  constexpr int V = 16 / sizeof(St) >= 4 ? 4 : 16 / sizeof(St);
  const int64_t cus = cu_count();
  // the lane count launch_col_any picks (VEC = V on the vector path; the
  // scalar path's 256-lane blocks are only counted approximately here)
  const int nth = col_block_lanes(inner / V);
  const int64_t col_blocks = outer * ((inner / V + nth - 1) / nth);
  const int64_t target = 4 * cus * 256 / nth;  // blocks for ~16 waves per CU
  int64_t splits = 1;
  if (col_blocks < target && R >= 2 * kColUnroll) {
    splits = (target + col_blocks - 1) / col_blocks;
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, R / 32));
  }
  splits = std::min<int64_t>(splits, 1024);
  const int64_t chunk = (R + splits - 1) / splits;
  splits = (R + chunk - 1) / chunk;
  if (splits == 1) return launch_col_any<Tag>(in, outer, R, inner, chunk, 1, op, final_out, stream);
  Workspace ws;
  MI_RETURN_IF(ws.alloc((size_t)(outer * splits * inner) * sizeof(A), stream));
  RedOut part{ws.get(), -1, 1.0};
  const int pop = op == R_MEAN ? R_SUM : op;
  MI_RETURN_IF(launch_col_any<Tag>(in, outer, R, inner, chunk, splits, pop, part, stream));
  const bool mx = op == R_MAX;
  if constexpr (std::is_same<A, float>::value) {
    if (inner % 4 == 0 && ((uintptr_t)ws.get() % 16) == 0) {
      const dim3 grid(ceil_div_u(outer * inner / 4, 16));
      if (mx)
        hipLaunchKernelGGL(col_finish_v4_kernel<true>, grid, dim3(256), 0, stream,
                           (const float*)ws.get(), outer, splits, inner, op, final_out);
      else
        hipLaunchKernelGGL(col_finish_v4_kernel<false>, grid, dim3(256), 0, stream,
                           (const float*)ws.get(), outer, splits, inner, op, final_out);
      return check_launch("col_reduce finish");
    }
  }
  const dim3 grid(ceil_div_u(outer * inner, 16));
  if (mx)
    hipLaunchKernelGGL((col_finish_kernel<A, true>), grid, dim3(256), 0, stream,
                       (const A*)ws.get(), outer, splits, inner, op, final_out);
  else
    hipLaunchKernelGGL((col_finish_kernel<A, false>), grid, dim3(256), 0, stream,
                       (const A*)ws.get(), outer, splits, inner, op, final_out);
  return check_launch("col_reduce finish");
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

// ---- static scratch of mi_mean_noalloc ---------------------------------------
//
// Device memory of the reductions that take no allocation: the split-row and
// split-column partials (config 2's fp32 [16384, 4096] mean over dim 0 takes
// 256 x 4096 floats = 4 MiB), and, for inputs whose reduced dims are not one
// dense block or an output that is not dense, the staging copies.  Every
// byte a kernel reads from it was written earlier in the same call, so
// nothing is cleared between calls.  One copy per GPU, held until the
// process ends; concurrent calls on one GPU (two streams or two threads)
// share it and race.
constexpr size_t kScratchBytes = MI_MEAN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device: the address of `scratch`

// Device address of this GPU's `scratch`, looked up once per device with it
// current.  Host code never passes `scratch` itself to a kernel: on the host
// that name is a stand-in, not a device address.
mi_status_t scratch_on_current_device(char** out) {
  int dev = 0;
  const hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) MI_FAIL(MI_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(de));
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      MI_FAIL(MI_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
              hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = (char*)g_scratch_ptr[dev];
  return MI_OK;
}

// Clears the thread's arena on every return path.
struct ArenaScope {
  explicit ArenaScope(ScratchArena* a) { set_scratch_arena(a); }
  ~ArenaScope() { set_scratch_arena(nullptr); }
};

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

mi_status_t mi_mean_noalloc(const mi_tensor_t* out, const mi_tensor_t* self, const int64_t* dims,
                            int32_t ndims, int32_t keepdim, mi_stream_t stream) {
  clear_error();
  char* base = nullptr;
  MI_RETURN_IF(scratch_on_current_device(&base));
  ScratchArena arena{base, kScratchBytes, 0, 0};
  ArenaScope scope(&arena);
  return run_reduce(R_MEAN, out, self, dims, ndims, keepdim, (hipStream_t)stream);
}

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
