// Elementwise engine: binary arithmetic (add/sub/mul/div), dtype-converting
// strided copy and fill.
//
// Paths, chosen on the host after broadcasting and coalescing (iter.cpp):
//   - "2-D" path: out is dense [R, C] and every input is dense [R, C], a row
//     vector [C] broadcast over rows, a column vector [R] broadcast over
//     columns, or a single value; all of one dtype.  Each thread moves
//     UNROLL x 16-byte vectors per pass, so one wave issues 4 KiB of loads
//     per operand at once.  Config 1's a*b with b [4096] broadcast over rows
//     and +0.5 are this path.
//   - general path: any strides, any mix of dtypes (loads convert to the
//     compute type, as TensorIterator's dynamic casting does).
#include <cstring>

#include "iter.h"

namespace mi {

namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 8;

enum OpKind { OP_ADD = 0, OP_MUL = 1, OP_DIV = 2 };
enum Mode { M_FULL = 0, M_ROW = 1, M_COL = 2, M_SCALAR = 3 };

template <int OP, typename A>
__device__ __forceinline__ A apply(A a, A b, A alpha) {
  if constexpr (OP == OP_ADD) {
    if constexpr (std::is_same<A, float>::value) return __builtin_fmaf(b, alpha, a);
    else if constexpr (std::is_same<A, double>::value) return __builtin_fma(b, alpha, a);
    else return (A)((uint64_t)a + (uint64_t)alpha * (uint64_t)b);  // wraps
  } else if constexpr (OP == OP_MUL) {
    if constexpr (std::is_integral<A>::value) return (A)((uint64_t)a * (uint64_t)b);
    else return a * b;
  } else {
    return a / b;
  }
}

// Storage helpers for the typed fast path.
template <typename Tag>
struct TypeOf {
  typedef Tag storage;
  typedef Tag acc;
  static __device__ __forceinline__ acc load(storage v) { return v; }
  static __device__ __forceinline__ storage store(acc v) { return v; }
};
template <>
struct TypeOf<BF16> : Num<BF16> {};
template <>
struct TypeOf<F16> : Num<F16> {};
template <>
struct TypeOf<int32_t> {
  typedef int32_t storage;
  typedef int64_t acc;
  static __device__ __forceinline__ acc load(storage v) { return v; }
  static __device__ __forceinline__ storage store(acc v) { return (storage)v; }
};

template <typename Tag>
struct Arg2D {
  const typename TypeOf<Tag>::storage* p;
  typename TypeOf<Tag>::acc imm;  // used when mode is scalar and p == NULL
  int mode;
};

// out[R, C] = op(a, b) with each input in one of the Mode layouts.  MA / MB
// fix the layouts at compile time for the common pairs (a full operand with
// a full, row, column or scalar one); -1 reads them from the arguments.  With
// fixed layouts every load is unconditional (a vector past the end re-reads
// the last one and is not stored), so the compiler waits once for all of a
// lane's loads; a load under a branch is waited alone.
template <typename Tag, int OP, int MA, int MB>
__global__ __launch_bounds__(kBlock) void binary_2d_kernel(
    typename TypeOf<Tag>::storage* __restrict__ out, Arg2D<Tag> a, Arg2D<Tag> b,
    typename TypeOf<Tag>::acc alpha, int64_t rows, int64_t cols) {
  typedef typename TypeOf<Tag>::storage St;
  typedef typename TypeOf<Tag>::acc Acc;
  constexpr int VEC = 16 / sizeof(St);
  constexpr bool FIXED = MA >= 0 && MB >= 0;
  union V {
    uint4 u;
    St s[VEC];
  };
  const int am = MA >= 0 ? MA : a.mode, bm = MB >= 0 ? MB : b.mode;
  const int64_t vcols = cols / VEC;
  const int64_t nvec = rows * vcols;
  const int64_t base = (int64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x;

  Acc sa = a.imm, sb = b.imm;
  if (am == M_SCALAR && a.p) sa = TypeOf<Tag>::load(a.p[0]);
  if (bm == M_SCALAR && b.p) sb = TypeOf<Tag>::load(b.p[0]);

  V va[kUnroll], vb[kUnroll];
  int64_t rowv[kUnroll], colv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v0 = base + (int64_t)u * kBlock;
    if (FIXED || v0 < nvec) {
      const int64_t v = FIXED && v0 >= nvec ? nvec - 1 : v0;
      int64_t r = 0, c = v;
      if (rows > 1 && (am == M_ROW || bm == M_ROW || am == M_COL || bm == M_COL)) {
        r = v / vcols;
        c = v - r * vcols;
      }
      rowv[u] = r;
      colv[u] = c;
      // full operands are streamed (read once); a broadcast row stays cached
      if (am == M_FULL) va[u].u = ld_stream((const uint4*)a.p + v);
      else if (am == M_ROW) va[u].u = ((const uint4*)a.p)[c];
      if (bm == M_FULL) vb[u].u = ld_stream((const uint4*)b.p + v);
      else if (bm == M_ROW) vb[u].u = ((const uint4*)b.p)[c];
    }
  }
  Acc cav[kUnroll], cbv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    cav[u] = sa;
    cbv[u] = sb;
    if (FIXED || base + (int64_t)u * kBlock < nvec) {
      if (am == M_COL) cav[u] = TypeOf<Tag>::load(a.p[rowv[u]]);
      if (bm == M_COL) cbv[u] = TypeOf<Tag>::load(b.p[rowv[u]]);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t v = base + (int64_t)u * kBlock;
    if (v < nvec) {
      V o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const Acc x = (am == M_FULL || am == M_ROW) ? TypeOf<Tag>::load(va[u].s[e]) : cav[u];
        const Acc y = (bm == M_FULL || bm == M_ROW) ? TypeOf<Tag>::load(vb[u].s[e]) : cbv[u];
        o.s[e] = TypeOf<Tag>::store(apply<OP, Acc>(x, y, alpha));
      }
      st_stream((uint4*)out + v, o.u);
    }
  }
}

// General strided path with dynamic dtypes; C is the compute type.
template <typename C, int OP>
__global__ __launch_bounds__(kBlock) void binary_general_kernel(
    char* out, int dt_out, const char* a, int dt_a, const char* b, int dt_b,
    C sa, C sb, int a_imm, int b_imm, C alpha, int round_a, int round_b,
    OffsetCalc<3> oc, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    int64_t off[3];
    oc.get(i, off);
    C x = a_imm ? sa : load_as<C>(a, off[1], dt_a);
    C y = b_imm ? sb : load_as<C>(b, off[2], dt_b);
    // Inputs of another dtype are first cast to the common dtype
    // (TensorIterator's promote_inputs_to_common_dtype).
    if constexpr (std::is_same<C, float>::value) {
      if (round_a == MI_BF16) x = bf16_to_f32(f32_to_bf16(x));
      else if (round_a == MI_F16) x = f16_to_f32(f32_to_f16(x));
      if (round_b == MI_BF16) y = bf16_to_f32(f32_to_bf16(y));
      else if (round_b == MI_F16) y = f16_to_f32(f32_to_f16(y));
    }
    store_as<C>(out, off[0], dt_out, apply<OP, C>(x, y, alpha));
  }
}

// ---- copy ----------------------------------------------------------------------

template <typename V>
__device__ __forceinline__ void store_value(char* p, int64_t idx, int dt, V v) {
  store_as<V>(p, idx, dt, v);
}

// c10::convert semantics: float -> uint8 goes through int64.
__device__ __forceinline__ void convert_elem(const char* src, int64_t si, int sdt, char* dst,
                                             int64_t di, int ddt) {
  switch (sdt) {
    case MI_U8: store_value<int64_t>(dst, di, ddt, ((const uint8_t*)src)[si]); break;
    case MI_I8: store_value<int64_t>(dst, di, ddt, ((const int8_t*)src)[si]); break;
    case MI_I16: store_value<int64_t>(dst, di, ddt, ((const int16_t*)src)[si]); break;
    case MI_I32: store_value<int64_t>(dst, di, ddt, ((const int32_t*)src)[si]); break;
    case MI_I64: {
      const int64_t v = ((const int64_t*)src)[si];
      if (ddt == MI_F32) ((float*)dst)[di] = (float)v;
      else if (ddt == MI_F16) ((uint16_t*)dst)[di] = f32_to_f16((float)v);
      else if (ddt == MI_BF16) ((uint16_t*)dst)[di] = f32_to_bf16((float)v);
      else store_value<int64_t>(dst, di, ddt, v);
      break;
    }
    case MI_BOOL: store_value<int64_t>(dst, di, ddt, ((const uint8_t*)src)[si] != 0); break;
    case MI_F16: store_value<float>(dst, di, ddt, f16_to_f32(((const uint16_t*)src)[si])); break;
    case MI_BF16: store_value<float>(dst, di, ddt, bf16_to_f32(((const uint16_t*)src)[si])); break;
    case MI_F32: store_value<float>(dst, di, ddt, ((const float*)src)[si]); break;
    case MI_F64: {
      const double v = ((const double*)src)[si];
      if (ddt == MI_F16) ((uint16_t*)dst)[di] = f32_to_f16((float)v);
      else if (ddt == MI_BF16) ((uint16_t*)dst)[di] = f32_to_bf16((float)v);
      else store_value<double>(dst, di, ddt, v);
      break;
    }
    default: break;
  }
}

__global__ __launch_bounds__(kBlock) void copy_general_kernel(char* out, int dt_out,
                                                              const char* src, int dt_src,
                                                              OffsetCalc<2> oc, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    int64_t off[2];
    oc.get(i, off);
    convert_elem(src, off[1], dt_src, out, off[0], dt_out);
  }
}

// Same-dtype strided copy moving raw elements of size sizeof(T).
// out[b][r][c] = src[b][r + c * src_ld] for a dense out ([R, C] per batch,
// row stride out_ld): a transpose.  64 x 64 tiles go through LDS so that the
// reads run along src's unit-stride dim and the writes along out's.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(T* __restrict__ out, const T* __restrict__ src,
                                                        int64_t R, int64_t C, int64_t out_ld,
                                                        int64_t src_ld, int64_t out_bs,
                                                        int64_t src_bs) {
  __shared__ T tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const T* s = src + b * src_bs;
  T* o = out + b * out_bs;
  // read: lanes along r (src unit stride), rows of the tile along c
#pragma unroll 4
  for (int k = ty; k < 64; k += 4) {
    const int64_t r = r0 + tx, c = c0 + k;
    if (r < R && c < C) tile[k][tx] = s[r + c * src_ld];
  }
  __syncthreads();
  // write: lanes along c (out unit stride)
#pragma unroll 4
  for (int k = ty; k < 64; k += 4) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < R && c < C) o[r * out_ld + c] = tile[tx][k];
  }
}

// The same transpose with 16-byte accesses on both sides and no LDS.  With
// E = 16 / sizeof(T) elements per 16-byte piece, lane (a, b) of a wave
// (a = lane % 8 along r, b = lane / 8 along c) loads the E x E block at
// r0 + a*E, c0 + b*E as E column pieces (src is unit-stride along r), turns
// it around in registers (v_perm_b32 pairs for 2-byte elements, a renaming
// for 4-byte ones) and stores E row pieces (out is unit-stride along c).  Each
// load or store of a wave covers eight full 128-byte runs.  A wave owns an
// 8E x 8E tile, a block of four waves 32E rows of r.  Consecutive block ids
// go round robin to the 8 XCDs, so ids are renumbered to give each XCD one
// contiguous range of tiles (neighbouring columns share its L2); measured on
// a bf16 8192^2 transpose: 6.1 TB/s against 4.8 without the renumbering and
// with non-temporal accesses.  Lanes whose block crosses the edge copy
// element by element.  The host checks that both tensors and their leading
// dims are 16-byte aligned.
constexpr int kTrWaves = 4;

// Bijection of [0, n): the ids that land on one XCD become one range.
__device__ __forceinline__ unsigned xcd_contiguous(unsigned id, unsigned n) {
  const unsigned q = n / 8, rem = n % 8, x = id % 8, local = id / 8;
  return x < rem ? x * (q + 1) + local : rem * (q + 1) + (x - rem) * q + local;
}

template <typename T>
struct TrPiece {
  static constexpr int E = 16 / sizeof(T);
  union {
    uint4 v;
    uint32_t w[4];
    T e[E];
  };
};

template <typename T>
__global__ __launch_bounds__(64 * kTrWaves) void transpose_vec_kernel(
    T* __restrict__ out, const T* __restrict__ src, int64_t R, int64_t C, int64_t out_ld,
    int64_t src_ld, int64_t out_bs, int64_t src_bs) {
  constexpr int E = TrPiece<T>::E;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int a = lane & 7, b = lane >> 3;
  const unsigned id = xcd_contiguous(blockIdx.y * gridDim.x + blockIdx.x, gridDim.x * gridDim.y);
  const unsigned bx = id % gridDim.x, by = id / gridDim.x;
  const int64_t r = ((int64_t)by * kTrWaves + wave) * (8 * E) + a * E;
  const int64_t c = (int64_t)bx * (8 * E) + b * E;
  const T* s = src + (int64_t)blockIdx.z * src_bs;
  T* o = out + (int64_t)blockIdx.z * out_bs;
  if (r >= R || c >= C) return;
  if (r + E <= R && c + E <= C) {
    TrPiece<T> v[E], t[E];
#pragma unroll
    for (int j = 0; j < E; ++j) v[j].v = *(const uint4*)(s + (c + j) * src_ld + r);
    if constexpr (E == 8) {
      // t[i].w[m] = (v[2m].e[i], v[2m+1].e[i]): the low or high halves of
      // word i/2 of two column pieces
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int m = 0; m < 4; ++m)
          t[i].w[m] = __builtin_amdgcn_perm(v[2 * m + 1].w[i >> 1], v[2 * m].w[i >> 1],
                                            (i & 1) ? 0x07060302u : 0x05040100u);
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i)
#pragma unroll
        for (int m = 0; m < E; ++m) t[i].e[m] = v[m].e[i];
    }
#pragma unroll
    for (int i = 0; i < E; ++i) *(uint4*)(o + (r + i) * out_ld + c) = t[i].v;
    return;
  }
  for (int i = 0; i < E && r + i < R; ++i)
    for (int j = 0; j < E && c + j < C; ++j) o[(r + i) * out_ld + c + j] = s[(c + j) * src_ld + r + i];
}

template <typename T>
__global__ __launch_bounds__(kBlock) void copy_raw_kernel(T* out, const T* src,
                                                          OffsetCalc<2> oc, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    int64_t off[2];
    oc.get(i, off);
    out[off[0]] = src[off[1]];
  }
}

// Contiguous float <-> half/bfloat16 conversion, 8 elements per thread.
template <typename SrcTag, typename DstTag>
__global__ __launch_bounds__(kBlock) void convert_contig_kernel(
    typename TypeOf<DstTag>::storage* __restrict__ out,
    const typename TypeOf<SrcTag>::storage* __restrict__ src, int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * 8;
  if (i0 + 8 <= n) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      out[i0 + e] = TypeOf<DstTag>::store((typename TypeOf<DstTag>::acc)TypeOf<SrcTag>::load(src[i0 + e]));
  } else {
    for (int64_t i = i0; i < n; ++i)
      out[i] = TypeOf<DstTag>::store((typename TypeOf<DstTag>::acc)TypeOf<SrcTag>::load(src[i]));
  }
}

// ---- fill ------------------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(kBlock) void fill_contig_kernel(T* out, T v, int64_t n) {
  constexpr int VEC = 16 / sizeof(T);
  union U {
    uint4 u;
    T s[VEC];
  } pack;
#pragma unroll
  for (int e = 0; e < VEC; ++e) pack.s[e] = v;
  const int64_t nvec = n / VEC;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < nvec; i += stride)
    ((uint4*)out)[i] = pack.u;
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (t < n - nvec * VEC) out[nvec * VEC + t] = v;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void fill_strided_kernel(T* out, T v, OffsetCalc<1> oc,
                                                              int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    int64_t off[1];
    oc.get(i, off);
    out[off[0]] = v;
  }
}

unsigned grid_for(int64_t n) {
  const int64_t want = (n + kBlock - 1) / kBlock;
  const int64_t cap = (int64_t)cu_count() * 32;
  return (unsigned)(want < cap ? (want < 1 ? 1 : want) : cap);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Classifies a 2-D iterator operand.
int mode_2d(const Iter& it, int o, int64_t rows, int64_t cols) {
  const int64_t s0 = it.ndim == 2 ? it.strides[o][0] : 0;
  const int64_t s1 = it.ndim == 2 ? it.strides[o][1] : it.strides[o][0];
  if (s0 == cols && s1 == 1) return M_FULL;
  // one row (a coalesced 1-D iterator): a dense operand is the whole tensor,
  // streamed as a full one (as a broadcast row it took the kernel with
  // run-time layouts and cached loads: config 1's x + 0.5 ran 7 % slower
  // than x * row)
  if (rows == 1 && s1 == 1) return M_FULL;
  if (s0 == 0 && s1 == 1) return M_ROW;
  if (s0 == 1 && s1 == 0) return M_COL;
  if (s0 == 0 && s1 == 0) return M_SCALAR;
  return -1;
}

struct BinArgs {
  const mi_tensor_t* out;
  const mi_tensor_t* a;  // may be NULL when a_scalar is used
  const mi_tensor_t* b;
  const mi_scalar_t* a_scalar;
  const mi_scalar_t* b_scalar;
  double alpha_f;
  int64_t alpha_i;
  int common;  // common dtype
  int op;
  bool scalar_round_to_common;  // cast host scalars to the common dtype first
  // A 0-dim `other` of a reduced-float multiply/divide is read in float
  // without first rounding it to the common dtype, as CPU ATen's mul and
  // div kernels do for their second operand (original_scalar_value).
  bool b_keeps_precision;
};

template <typename Tag, int OP>
mi_status_t launch_2d(const Iter& it, int ia, int ib, const BinArgs& ba, hipStream_t stream) {
  typedef typename TypeOf<Tag>::storage St;
  typedef typename TypeOf<Tag>::acc Acc;
  constexpr int VEC = 16 / sizeof(St);
  const int64_t rows = it.ndim == 2 ? it.sizes[0] : 1;
  const int64_t cols = it.ndim == 2 ? it.sizes[1] : it.sizes[0];
  Arg2D<Tag> a{nullptr, Acc(0), M_SCALAR}, b{nullptr, Acc(0), M_SCALAR};
  auto fill = [&](Arg2D<Tag>& arg, int idx, const mi_scalar_t* s) {
    if (idx >= 0) {
      arg.p = (const St*)it.data[idx];
      arg.mode = mode_2d(it, idx, rows, cols);
    } else {
      double v = scalar_as_double(*s);
      if (std::is_integral<Acc>::value) {
        arg.imm = (Acc)scalar_as_int(*s);
      } else {
        if (ba.scalar_round_to_common) {
          if (ba.common == MI_BF16) v = host_bf16_to_f32(host_f32_to_bf16((float)v));
          else if (ba.common == MI_F16) v = host_f16_to_f32(host_f32_to_f16((float)v));
        }
        arg.imm = (Acc)v;
      }
    }
  };
  fill(a, ia, ba.a_scalar);
  fill(b, ib, ba.b_scalar);
  Acc alpha;
  if (std::is_integral<Acc>::value) alpha = (Acc)ba.alpha_i;
  else {
    double al = ba.alpha_f;
    if (ba.common == MI_BF16) al = host_bf16_to_f32(host_f32_to_bf16((float)al));
    else if (ba.common == MI_F16) al = host_f16_to_f32(host_f32_to_f16((float)al));
    alpha = (Acc)al;
  }
  const int64_t nvec = rows * (cols / VEC);
  if (nvec == 0) return MI_OK;
  const unsigned grid = ceil_div_u(nvec, (int64_t)kBlock * kUnroll);
  St* o = (St*)it.data[0];
  auto go = [&](auto ma, auto mb) -> mi_status_t {
    hipLaunchKernelGGL((binary_2d_kernel<Tag, OP, decltype(ma)::value, decltype(mb)::value>),
                       dim3(grid), dim3(kBlock), 0, stream, o, a, b, alpha, rows, cols);
    return check_launch("binary_2d");
  };
  typedef std::integral_constant<int, M_FULL> Full;
  typedef std::integral_constant<int, M_ROW> Row;
  typedef std::integral_constant<int, M_COL> Col;
  typedef std::integral_constant<int, M_SCALAR> Sc;
  typedef std::integral_constant<int, -1> Any;
  if (a.mode == M_FULL && b.mode == M_FULL) return go(Full(), Full());
  if (a.mode == M_FULL && b.mode == M_ROW) return go(Full(), Row());
  if (a.mode == M_FULL && b.mode == M_COL) return go(Full(), Col());
  if (a.mode == M_FULL && b.mode == M_SCALAR) return go(Full(), Sc());
  if (a.mode == M_ROW && b.mode == M_FULL) return go(Row(), Full());
  if (a.mode == M_SCALAR && b.mode == M_FULL) return go(Sc(), Full());
  return go(Any(), Any());
}

template <typename Tag>
mi_status_t dispatch_2d_op(const Iter& it, int ia, int ib, const BinArgs& ba, hipStream_t s) {
  switch (ba.op) {
    case OP_ADD: return launch_2d<Tag, OP_ADD>(it, ia, ib, ba, s);
    case OP_MUL: return launch_2d<Tag, OP_MUL>(it, ia, ib, ba, s);
    default: return launch_2d<Tag, OP_DIV>(it, ia, ib, ba, s);
  }
}

template <typename C, int OP>
mi_status_t launch_general_t(const Iter& it, int ia, int ib, const BinArgs& ba, C sa, C sb,
                             C alpha, hipStream_t stream) {
  OffsetCalc<3> oc;
  oc.ndim = it.ndim;
  for (int d = 0; d < MI_MAX_DIMS; ++d) {
    oc.sizes[d] = d < it.ndim ? it.sizes[d] : 1;
    oc.strides[0][d] = d < it.ndim ? it.strides[0][d] : 0;
    oc.strides[1][d] = (ia >= 0 && d < it.ndim) ? it.strides[ia][d] : 0;
    oc.strides[2][d] = (ib >= 0 && d < it.ndim) ? it.strides[ib][d] : 0;
  }
  const int dta = ia >= 0 ? it.dtype[ia] : -1, dtb = ib >= 0 ? it.dtype[ib] : -1;
  const int ra = (ia >= 0 && dta != ba.common) ? ba.common : -1;
  const int rb = (ib >= 0 && dtb != ba.common && !ba.b_keeps_precision) ? ba.common : -1;
  hipLaunchKernelGGL((binary_general_kernel<C, OP>), dim3(grid_for(it.numel)), dim3(kBlock), 0,
                     stream, it.data[0], it.dtype[0], ia >= 0 ? it.data[ia] : nullptr, dta,
                     ib >= 0 ? it.data[ib] : nullptr, dtb, sa, sb, ia < 0 ? 1 : 0,
                     ib < 0 ? 1 : 0, alpha, ra, rb, oc, it.numel);
  return check_launch("binary_general");
}

template <typename C>
mi_status_t launch_general(const Iter& it, int ia, int ib, const BinArgs& ba, hipStream_t s) {
  auto sval = [&](const mi_scalar_t* sc) -> C {
    if (sc == nullptr) return C(0);
    if (std::is_integral<C>::value) return (C)scalar_as_int(*sc);
    double v = scalar_as_double(*sc);
    if (ba.scalar_round_to_common) {
      if (ba.common == MI_BF16) v = host_bf16_to_f32(host_f32_to_bf16((float)v));
      else if (ba.common == MI_F16) v = host_f16_to_f32(host_f32_to_f16((float)v));
    }
    return (C)v;
  };
  C alpha;
  if (std::is_integral<C>::value) alpha = (C)ba.alpha_i;
  else {
    double al = ba.alpha_f;
    if (ba.common == MI_BF16) al = host_bf16_to_f32(host_f32_to_bf16((float)al));
    else if (ba.common == MI_F16) al = host_f16_to_f32(host_f32_to_f16((float)al));
    alpha = (C)al;
  }
  const C sa = sval(ba.a_scalar), sb = sval(ba.b_scalar);
  switch (ba.op) {
    case OP_ADD: return launch_general_t<C, OP_ADD>(it, ia, ib, ba, sa, sb, alpha, s);
    case OP_MUL: return launch_general_t<C, OP_MUL>(it, ia, ib, ba, sa, sb, alpha, s);
    default: return launch_general_t<C, OP_DIV>(it, ia, ib, ba, sa, sb, alpha, s);
  }
}

mi_status_t run_binary(const BinArgs& ba, hipStream_t stream) {
  MI_RETURN_IF(validate(ba.out, "out"));
  if (ba.a) MI_RETURN_IF(validate(ba.a, "self"));
  if (ba.b) MI_RETURN_IF(validate(ba.b, "other"));
  const mi_tensor_t* ins[2];
  int nin = 0, ia = -1, ib = -1;
  if (ba.a) {
    ins[nin] = ba.a;
    ia = ++nin;
  }
  if (ba.b) {
    ins[nin] = ba.b;
    ib = ++nin;
  }
  Iter it;
  MI_RETURN_IF(make_iter(it, *ba.out, ins, nin));
  if (it.numel == 0) return MI_OK;
  const int c = ba.common;
  if (ba.op == OP_DIV && !is_floating(c))
    MI_FAIL(MI_ERR_INVALID, "div: common dtype %s is not floating", dtype_name(c));

  // Typed 2-D fast path.
  bool same = it.dtype[0] == c && (ia < 0 || it.dtype[ia] == c) && (ib < 0 || it.dtype[ib] == c);
  if (same && it.ndim <= 2) {
    const int64_t cols = it.ndim == 2 ? it.sizes[1] : it.sizes[0];
    const int64_t rows = it.ndim == 2 ? it.sizes[0] : 1;
    const int esz = dtype_size(c);
    const int vec = 16 / esz;
    bool ok = it.op_contiguous(0) && cols % vec == 0 && aligned16(it.data[0]);
    for (int o : {ia, ib}) {
      if (!ok || o < 0) continue;
      const int m = mode_2d(it, o, rows, cols);
      ok = m >= 0 && ((m != M_FULL && m != M_ROW) || aligned16(it.data[o]));
    }
    if (ok) {
      switch (c) {
        case MI_F32: return dispatch_2d_op<float>(it, ia, ib, ba, stream);
        case MI_BF16: return dispatch_2d_op<BF16>(it, ia, ib, ba, stream);
        case MI_F16: return dispatch_2d_op<F16>(it, ia, ib, ba, stream);
        case MI_F64: return dispatch_2d_op<double>(it, ia, ib, ba, stream);
        case MI_I64:
          if (ba.op != OP_DIV) return dispatch_2d_op<int64_t>(it, ia, ib, ba, stream);
          break;
        case MI_I32:
          if (ba.op != OP_DIV) return dispatch_2d_op<int32_t>(it, ia, ib, ba, stream);
          break;
        default: break;
      }
    }
  }
  if (it.ndim > MI_MAX_DIMS) MI_FAIL(MI_ERR_UNSUPPORTED, "too many dims");
  if (c == MI_F64) return launch_general<double>(it, ia, ib, ba, stream);
  if (is_floating(c)) return launch_general<float>(it, ia, ib, ba, stream);
  return launch_general<int64_t>(it, ia, ib, ba, stream);
}

mi_scalar_t one_scalar() {
  mi_scalar_t s;
  s.f = 1.0;
  s.i = 1;
  s.dtype = MI_I64;
  s.wrapped = 1;
  return s;
}

mi_status_t binary_tt(int op, const mi_tensor_t* out, const mi_tensor_t* self,
                      const mi_tensor_t* other, mi_scalar_t alpha, bool negate_alpha,
                      mi_stream_t stream) {
  clear_error();
  if (!out || !self || !other) MI_FAIL(MI_ERR_INVALID, "NULL descriptor");
  ResultType rt;
  rt.add_tensor(*self);
  rt.add_tensor(*other);
  int common = rt.get();
  if (op == OP_DIV && !is_floating(common)) common = MI_F32;
  if (op == OP_ADD && negate_alpha && common == MI_BOOL)
    MI_FAIL(MI_ERR_INVALID, "sub: subtraction of bool tensors is not supported");
  BinArgs ba{};
  ba.out = out;
  ba.a = self;
  ba.b = other;
  ba.alpha_f = scalar_as_double(alpha) * (negate_alpha ? -1.0 : 1.0);
  ba.alpha_i = scalar_as_int(alpha) * (negate_alpha ? -1 : 1);
  ba.common = common;
  ba.op = op;
  ba.scalar_round_to_common = false;
  ba.b_keeps_precision = (op == OP_MUL || op == OP_DIV) && other->ndim == 0 &&
                         (common == MI_BF16 || common == MI_F16);
  return run_binary(ba, (hipStream_t)stream);
}

}  // namespace

}  // namespace mi

using namespace mi;

extern "C" {

mi_status_t mi_add(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* other,
                   mi_scalar_t alpha, mi_stream_t stream) {
  return binary_tt(OP_ADD, out, self, other, alpha, false, stream);
}

mi_status_t mi_sub(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* other,
                   mi_scalar_t alpha, mi_stream_t stream) {
  return binary_tt(OP_ADD, out, self, other, alpha, true, stream);
}

mi_status_t mi_mul(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* other,
                   mi_stream_t stream) {
  return binary_tt(OP_MUL, out, self, other, one_scalar(), false, stream);
}

mi_status_t mi_div(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* other,
                   mi_stream_t stream) {
  return binary_tt(OP_DIV, out, self, other, one_scalar(), false, stream);
}

// CPU ATen casts a wrapped scalar operand of add to the common dtype before
// the kernel runs (TensorIteratorBase::compute_types on a CPU iterator),
// so a bf16 tensor + 0.1 adds bf16(0.1).
mi_status_t mi_add_scalar(const mi_tensor_t* out, const mi_tensor_t* self, mi_scalar_t other,
                          mi_scalar_t alpha, mi_stream_t stream) {
  clear_error();
  if (!out || !self) MI_FAIL(MI_ERR_INVALID, "NULL descriptor");
  ResultType rt;
  rt.add_tensor(*self);
  rt.add_scalar(other);
  BinArgs ba{};
  ba.out = out;
  ba.a = self;
  ba.b = nullptr;
  ba.b_scalar = &other;
  ba.alpha_f = scalar_as_double(alpha);
  ba.alpha_i = scalar_as_int(alpha);
  ba.common = rt.get();
  ba.op = OP_ADD;
  ba.scalar_round_to_common = true;
  return run_binary(ba, (hipStream_t)stream);
}

// CPU ATen's mul kernel reads a scalar operand of a reduced-float multiply in
// float without first rounding it to the tensor's dtype (mul_kernel's
// original_scalar_value branch), so the scalar is kept in the compute type.
mi_status_t mi_mul_scalar(const mi_tensor_t* out, const mi_tensor_t* self, mi_scalar_t other,
                          mi_stream_t stream) {
  clear_error();
  if (!out || !self) MI_FAIL(MI_ERR_INVALID, "NULL descriptor");
  ResultType rt;
  rt.add_tensor(*self);
  rt.add_scalar(other);
  BinArgs ba{};
  ba.out = out;
  ba.a = self;
  ba.b = nullptr;
  ba.b_scalar = &other;
  ba.alpha_f = 1.0;
  ba.alpha_i = 1;
  ba.common = rt.get();
  ba.op = OP_MUL;
  ba.scalar_round_to_common = false;
  return run_binary(ba, (hipStream_t)stream);
}

// True division by a wrapped scalar, read in float like mi_mul_scalar.
mi_status_t mi_div_scalar(const mi_tensor_t* out, const mi_tensor_t* self, mi_scalar_t other,
                          mi_stream_t stream) {
  clear_error();
  if (!out || !self) MI_FAIL(MI_ERR_INVALID, "NULL descriptor");
  ResultType rt;
  rt.add_tensor(*self);
  rt.add_scalar(other);
  BinArgs ba{};
  ba.out = out;
  ba.a = self;
  ba.b = nullptr;
  ba.b_scalar = &other;
  ba.alpha_f = 1.0;
  ba.alpha_i = 1;
  ba.common = rt.get();
  if (!is_floating(ba.common)) ba.common = MI_F32;
  ba.op = OP_DIV;
  ba.scalar_round_to_common = false;
  return run_binary(ba, (hipStream_t)stream);
}

mi_status_t mi_copy(const mi_tensor_t* out, const mi_tensor_t* src, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(src, "src"));
  const mi_tensor_t* ins[1] = {src};
  Iter it;
  MI_RETURN_IF(make_iter(it, *out, ins, 1));
  if (it.numel == 0) return MI_OK;
  const int esz = dtype_size(out->dtype);
  if (out->dtype == src->dtype) {
    if (it.op_contiguous(0) && it.op_contiguous(1)) {
      if (hipMemcpyAsync(it.data[0], it.data[1], (size_t)it.numel * esz, hipMemcpyDeviceToDevice,
                         stream) != hipSuccess)
        MI_FAIL(MI_ERR_LAUNCH, "copy: hipMemcpyAsync failed: %s",
                hipGetErrorString(hipGetLastError()));
      return MI_OK;
    }
    // a transpose (out dense, src unit-stride along out's second-innermost
    // dim): tiled through LDS instead of the strided element copy
    const int nd = it.ndim;
    if ((nd == 2 || nd == 3) && it.strides[0][nd - 1] == 1 && it.strides[1][nd - 2] == 1 &&
        it.strides[1][nd - 1] != 1 && (esz == 2 || esz == 4) &&
        (nd == 2 || it.sizes[0] <= 65535)) {
      const int64_t R = it.sizes[nd - 2], C = it.sizes[nd - 1];
      const int64_t batch = nd == 3 ? it.sizes[0] : 1;
      const int64_t obs = nd == 3 ? it.strides[0][0] : 0, sbs = nd == 3 ? it.strides[1][0] : 0;
      const int64_t E = 16 / esz;
      const int64_t sld = it.strides[1][nd - 1], old_ = it.strides[0][nd - 2];
      const bool vec_ok = ((uintptr_t)it.data[0] % 16) == 0 && ((uintptr_t)it.data[1] % 16) == 0 &&
                          sld % E == 0 && old_ % E == 0 && obs % E == 0 && sbs % E == 0;
      const dim3 vgrid(ceil_div_u(C, 8 * E), ceil_div_u(R, 8 * E * kTrWaves), (unsigned)batch);
      if (vec_ok && vgrid.y <= 65535) {
        if (esz == 2)
          hipLaunchKernelGGL(transpose_vec_kernel<uint16_t>, vgrid, dim3(64 * kTrWaves), 0, stream,
                             (uint16_t*)it.data[0], (const uint16_t*)it.data[1], R, C, old_, sld,
                             obs, sbs);
        else
          hipLaunchKernelGGL(transpose_vec_kernel<uint32_t>, vgrid, dim3(64 * kTrWaves), 0, stream,
                             (uint32_t*)it.data[0], (const uint32_t*)it.data[1], R, C, old_, sld,
                             obs, sbs);
        return check_launch("transpose");
      }
      dim3 grid(ceil_div_u(C, 64), ceil_div_u(R, 64), (unsigned)batch);
      if (grid.y <= 65535) {
        if (esz == 2)
          hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(256), 0, stream,
                             (uint16_t*)it.data[0], (const uint16_t*)it.data[1], R, C,
                             it.strides[0][nd - 2], it.strides[1][nd - 1], obs, sbs);
        else
          hipLaunchKernelGGL(transpose_kernel<uint32_t>, grid, dim3(256), 0, stream,
                             (uint32_t*)it.data[0], (const uint32_t*)it.data[1], R, C,
                             it.strides[0][nd - 2], it.strides[1][nd - 1], obs, sbs);
        return check_launch("transpose");
      }
    }
    OffsetCalc<2> oc = make_offset_calc<2>(it);
    const unsigned g = grid_for(it.numel);
    switch (esz) {
      case 1: hipLaunchKernelGGL(copy_raw_kernel<uint8_t>, dim3(g), dim3(kBlock), 0, stream, (uint8_t*)it.data[0], (const uint8_t*)it.data[1], oc, it.numel); break;
      case 2: hipLaunchKernelGGL(copy_raw_kernel<uint16_t>, dim3(g), dim3(kBlock), 0, stream, (uint16_t*)it.data[0], (const uint16_t*)it.data[1], oc, it.numel); break;
      case 4: hipLaunchKernelGGL(copy_raw_kernel<uint32_t>, dim3(g), dim3(kBlock), 0, stream, (uint32_t*)it.data[0], (const uint32_t*)it.data[1], oc, it.numel); break;
      default: hipLaunchKernelGGL(copy_raw_kernel<uint64_t>, dim3(g), dim3(kBlock), 0, stream, (uint64_t*)it.data[0], (const uint64_t*)it.data[1], oc, it.numel); break;
    }
    return check_launch("copy_raw");
  }
  if (it.op_contiguous(0) && it.op_contiguous(1)) {
    const unsigned g = ceil_div_u(it.numel, (int64_t)kBlock * 8);
    const int so = src->dtype, d = out->dtype;
    bool done = true;
    if (so == MI_F32 && d == MI_BF16) hipLaunchKernelGGL((convert_contig_kernel<float, BF16>), dim3(g), dim3(kBlock), 0, stream, (uint16_t*)it.data[0], (const float*)it.data[1], it.numel);
    else if (so == MI_BF16 && d == MI_F32) hipLaunchKernelGGL((convert_contig_kernel<BF16, float>), dim3(g), dim3(kBlock), 0, stream, (float*)it.data[0], (const uint16_t*)it.data[1], it.numel);
    else if (so == MI_F32 && d == MI_F16) hipLaunchKernelGGL((convert_contig_kernel<float, F16>), dim3(g), dim3(kBlock), 0, stream, (uint16_t*)it.data[0], (const float*)it.data[1], it.numel);
    else if (so == MI_F16 && d == MI_F32) hipLaunchKernelGGL((convert_contig_kernel<F16, float>), dim3(g), dim3(kBlock), 0, stream, (float*)it.data[0], (const uint16_t*)it.data[1], it.numel);
    else done = false;
    if (done) return check_launch("convert_contig");
  }
  OffsetCalc<2> oc = make_offset_calc<2>(it);
  hipLaunchKernelGGL(copy_general_kernel, dim3(grid_for(it.numel)), dim3(kBlock), 0, stream,
                     it.data[0], out->dtype, (const char*)it.data[1], src->dtype, oc, it.numel);
  return check_launch("copy_general");
}

mi_status_t mi_fill(const mi_tensor_t* out, mi_scalar_t value, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  const int64_t n = numel(*out);
  if (n == 0) return MI_OK;
  // Bit pattern of the value converted to out's dtype (c10::convert).
  uint64_t bits = 0;
  const double v = scalar_as_double(value);
  const int64_t iv = scalar_as_int(value);
  const bool vf = is_floating(value.dtype);
  switch (out->dtype) {
    case MI_U8: bits = (uint8_t)(vf ? (int64_t)v : iv); break;
    case MI_I8: bits = (uint8_t)(int8_t)(vf ? (int64_t)v : iv); break;
    case MI_I16: bits = (uint16_t)(int16_t)(vf ? (int64_t)v : iv); break;
    case MI_I32: bits = (uint32_t)(int32_t)(vf ? (int64_t)v : iv); break;
    case MI_I64: bits = (uint64_t)(vf ? (int64_t)v : iv); break;
    case MI_BOOL: bits = (vf ? v != 0.0 : iv != 0) ? 1 : 0; break;
    case MI_F16: bits = host_f32_to_f16((float)v); break;
    case MI_BF16: bits = host_f32_to_bf16((float)v); break;
    case MI_F32: {
      float f = (float)v;
      uint32_t u;
      std::memcpy(&u, &f, 4);
      bits = u;
      break;
    }
    case MI_F64: std::memcpy(&bits, &v, 8); break;
    default: MI_FAIL(MI_ERR_UNSUPPORTED, "fill: dtype");
  }
  const int esz = dtype_size(out->dtype);
  if (is_contiguous(*out) && aligned16(out->data)) {
    const unsigned g = grid_for((n * esz + 15) / 16);
    switch (esz) {
      case 1: hipLaunchKernelGGL(fill_contig_kernel<uint8_t>, dim3(g), dim3(kBlock), 0, stream, (uint8_t*)out->data, (uint8_t)bits, n); break;
      case 2: hipLaunchKernelGGL(fill_contig_kernel<uint16_t>, dim3(g), dim3(kBlock), 0, stream, (uint16_t*)out->data, (uint16_t)bits, n); break;
      case 4: hipLaunchKernelGGL(fill_contig_kernel<uint32_t>, dim3(g), dim3(kBlock), 0, stream, (uint32_t*)out->data, (uint32_t)bits, n); break;
      default: hipLaunchKernelGGL(fill_contig_kernel<uint64_t>, dim3(g), dim3(kBlock), 0, stream, (uint64_t*)out->data, (uint64_t)bits, n); break;
    }
    return check_launch("fill_contig");
  }
  const mi_tensor_t* none[1] = {nullptr};
  Iter it;
  MI_RETURN_IF(make_iter(it, *out, none, 0));
  OffsetCalc<1> oc = make_offset_calc<1>(it);
  const unsigned g = grid_for(n);
  switch (esz) {
    case 1: hipLaunchKernelGGL(fill_strided_kernel<uint8_t>, dim3(g), dim3(kBlock), 0, stream, (uint8_t*)out->data, (uint8_t)bits, oc, n); break;
    case 2: hipLaunchKernelGGL(fill_strided_kernel<uint16_t>, dim3(g), dim3(kBlock), 0, stream, (uint16_t*)out->data, (uint16_t)bits, oc, n); break;
    case 4: hipLaunchKernelGGL(fill_strided_kernel<uint32_t>, dim3(g), dim3(kBlock), 0, stream, (uint32_t*)out->data, (uint32_t)bits, oc, n); break;
    default: hipLaunchKernelGGL(fill_strided_kernel<uint64_t>, dim3(g), dim3(kBlock), 0, stream, (uint64_t*)out->data, (uint64_t)bits, oc, n); break;
  }
  return check_launch("fill_strided");
}

}  // extern "C"
