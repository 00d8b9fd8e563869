// Shared device and host helpers of the gfx950 kernel library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "mi355x_ops.h"

namespace mi {

// ---- errors -----------------------------------------------------------------

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

struct Status {
  mi_status_t code;
};

#define MI_FAIL(code, ...)     \
  do {                         \
    ::mi::set_error(__VA_ARGS__); \
    return (code);             \
  } while (0)

#define MI_CHECK_ARG(cond, ...)                        \
  do {                                                 \
    if (!(cond)) MI_FAIL(MI_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define MI_RETURN_IF(expr)              \
  do {                                  \
    mi_status_t _st = (expr);           \
    if (_st != MI_OK) return _st;       \
  } while (0)

// Checks the launch just enqueued.
mi_status_t check_launch(const char* what);

// ---- workspace ----------------------------------------------------------------

// RAII workspace from the registered allocator, or from this thread's
// scratch arena while one is set.
class Workspace {
 public:
  Workspace() = default;
  ~Workspace();
  mi_status_t alloc(size_t bytes, hipStream_t stream);
  void* get() const { return ptr_; }
  Workspace(const Workspace&) = delete;
  Workspace& operator=(const Workspace&) = delete;

 private:
  void* ptr_ = nullptr;
  hipStream_t stream_ = nullptr;
  bool from_arena_ = false;
};

// A fixed device buffer that Workspace::alloc carves from (256-byte aligned
// bump allocation, nothing returned until the arena is cleared) while it is
// set on the calling thread.  An entry point that must not allocate sets one
// over its static scratch for the duration of the call; a request that does
// not fit fails with MI_ERR_TOO_LARGE instead of reaching the allocator.
struct ScratchArena {
  char* base;
  size_t size;
  size_t used;
  size_t peak;
};
void set_scratch_arena(ScratchArena* arena);  // nullptr clears it

int cu_count();

// Out-of-range index record of one device (index_select / index kernels):
// flag set to 1, the offending index and the size of the dimension it
// indexes (any one of them when several lanes write).  Lives in pinned,
// host-coherent memory, so recording costs nothing until an index is bad
// and the host reads it after a synchronisation without a device call.
struct IndexFault {
  int64_t flag;
  int64_t index;
  int64_t size;
};
// The current device's record (device-accessible pointer), allocated on
// first use; nullptr if pinned memory cannot be had (then nothing is
// recorded).
IndexFault* index_fault_word();
// Records a bad index (vector stores of per-lane data).
__device__ __forceinline__ void record_index_fault(IndexFault* f, int64_t index, int64_t size) {
  if (f != nullptr) {
    f->index = index;
    f->size = size;
    f->flag = 1;
  }
}

// ---- dtypes -------------------------------------------------------------------

inline int dtype_size(int dt) {
  switch (dt) {
    case MI_U8: case MI_I8: case MI_BOOL: return 1;
    case MI_I16: case MI_F16: case MI_BF16: return 2;
    case MI_I32: case MI_F32: return 4;
    case MI_I64: case MI_F64: return 8;
    default: return 0;
  }
}
inline bool dtype_valid(int dt) { return dtype_size(dt) != 0; }
inline bool is_floating(int dt) {
  return dt == MI_F16 || dt == MI_BF16 || dt == MI_F32 || dt == MI_F64;
}
inline bool is_integral(int dt, bool include_bool) {
  return dt == MI_U8 || dt == MI_I8 || dt == MI_I16 || dt == MI_I32 ||
         dt == MI_I64 || (include_bool && dt == MI_BOOL);
}
const char* dtype_name(int dt);

// ATen's promoteTypes over the dtypes above (c10/core/ScalarType.cpp).
int promote_types(int a, int b);

// ---- tensor views --------------------------------------------------------------

inline int64_t numel(const mi_tensor_t& t) {
  int64_t n = 1;
  for (int i = 0; i < t.ndim; ++i) n *= t.sizes[i];
  return n;
}
bool is_contiguous(const mi_tensor_t& t);
mi_status_t validate(const mi_tensor_t* t, const char* name);

// ---- device-side numerics ---------------------------------------------------

typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}
// Round to nearest even (hardware v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(bf16_t, b);
}
__device__ __forceinline__ float f16_to_f32(uint16_t v) {
  return (float)__builtin_bit_cast(_Float16, v);
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// The value as it stands, rounded to its own type: an empty asm the compiler
// cannot look through, so a following conversion to fp16 is not fused with
// the arithmetic that produced it into one v_fma_mixlo_f16 that rounds once.
// CPU ATen rounds the fp32 result first, then converts; ops that promise its
// bits use this before storing 16-bit results.
template <typename T>
__device__ __forceinline__ T as_rounded(T x) {
  if constexpr (sizeof(T) == 4) asm volatile("" : "+v"(x));
  return x;
}

// Storage type tags used by templated kernels.
struct BF16 {
  typedef uint16_t storage;
};
struct F16 {
  typedef uint16_t storage;
};

template <typename S>
struct Num;  // storage -> compute conversions
template <>
struct Num<float> {
  typedef float storage;
  typedef float acc;
  static __device__ __forceinline__ float load(float v) { return v; }
  static __device__ __forceinline__ float store(float v) { return v; }
};
template <>
struct Num<double> {
  typedef double storage;
  typedef double acc;
  static __device__ __forceinline__ double load(double v) { return v; }
  static __device__ __forceinline__ double store(double v) { return v; }
};
template <>
struct Num<BF16> {
  typedef uint16_t storage;
  typedef float acc;
  static __device__ __forceinline__ float load(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_bf16(v); }
};
template <>
struct Num<F16> {
  typedef uint16_t storage;
  typedef float acc;
  static __device__ __forceinline__ float load(uint16_t v) { return f16_to_f32(v); }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_f16(v); }
};

// Loads element `idx` of a buffer of runtime dtype `dt` as C.
template <typename C>
__device__ __forceinline__ C load_as(const void* p, int64_t idx, int dt) {
  switch (dt) {
    case MI_U8: return (C)((const uint8_t*)p)[idx];
    case MI_I8: return (C)((const int8_t*)p)[idx];
    case MI_I16: return (C)((const int16_t*)p)[idx];
    case MI_I32: return (C)((const int32_t*)p)[idx];
    case MI_I64: return (C)((const int64_t*)p)[idx];
    case MI_F16: return (C)f16_to_f32(((const uint16_t*)p)[idx]);
    case MI_BF16: return (C)bf16_to_f32(((const uint16_t*)p)[idx]);
    case MI_F32: return (C)((const float*)p)[idx];
    case MI_F64: return (C)((const double*)p)[idx];
    case MI_BOOL: return (C)(((const uint8_t*)p)[idx] != 0);
    default: return (C)0;
  }
}

// Stores `v` (compute type C) into element `idx` of a buffer of dtype dt,
// converting the way c10::convert does (float to f16/bf16 rounds to nearest
// even; anything to bool tests != 0).
template <typename C>
__device__ __forceinline__ void store_as(void* p, int64_t idx, int dt, C v) {
  switch (dt) {
    case MI_U8: ((uint8_t*)p)[idx] = (uint8_t)(int64_t)v; break;
    case MI_I8: ((int8_t*)p)[idx] = (int8_t)(int64_t)v; break;
    case MI_I16: ((int16_t*)p)[idx] = (int16_t)(int64_t)v; break;
    case MI_I32: ((int32_t*)p)[idx] = (int32_t)(int64_t)v; break;
    case MI_I64: ((int64_t*)p)[idx] = (int64_t)v; break;
    case MI_F16: ((uint16_t*)p)[idx] = f32_to_f16((float)v); break;
    case MI_BF16: ((uint16_t*)p)[idx] = f32_to_bf16((float)v); break;
    case MI_F32: ((float*)p)[idx] = (float)v; break;
    case MI_F64: ((double*)p)[idx] = (double)v; break;
    case MI_BOOL: ((uint8_t*)p)[idx] = (v != (C)0) ? 1 : 0; break;
    default: break;
  }
}

// ---- wavefront / block reductions (wave64) -----------------------------------

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    T o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

// NaN-propagating max, as ATen's max_impl: a NaN operand wins.
__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || a > b) ? a : b;
}

// fp32 wave64 reductions without LDS traffic: butterflies inside each row of
// 16 lanes by DPP (quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror,
// row_mirror: after them every lane holds its row's total), then the four
// row totals read into scalar registers and combined in a fixed order.
// Each DPP step is one VALU op a few cycles long, where a __shfl_xor step is
// an LDS permute waited for in turn (six of them per reduction); every lane
// gets the result.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                            0xF, 0xF, true));
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
template <typename Op>
__device__ __forceinline__ float wave_reduce_f32(float v, Op op) {
  v = op(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_f32<0x141>(v));  // row_half_mirror: quad 0 <-> quad 1 of each 8
  v = op(v, dpp_f32<0x140>(v));  // row_mirror: the two 8-lane halves of each row
  return op(op(readlane_f32(v, 0), readlane_f32(v, 16)),
            op(readlane_f32(v, 32), readlane_f32(v, 48)));
}
__device__ __forceinline__ double nan_max(double a, double b) {
  return (a != a || a > b) ? a : b;
}
template <typename T>
__device__ __forceinline__ T nan_max(T a, T b) {
  return a > b ? a : b;
}

template <typename T>
__device__ __forceinline__ T wave_nan_max(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = nan_max(v, (T)__shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce_f32(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_nan_max(float v) {
  return wave_reduce_f32(v, [](float a, float b) { return nan_max(a, b); });
}
__device__ __forceinline__ float wave_fmax(float v) {
  return wave_reduce_f32(v, [](float a, float b) { return fmaxf(a, b); });
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024); every thread gets
// the result.  `red` is LDS scratch of at least 16 entries.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  T r = lane < nw ? red[lane] : (T)0;
  return wave_sum(r);
}
template <typename T>
__device__ __forceinline__ T block_nan_max(T v, T* red, T ident) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  v = wave_nan_max(v);
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  T r = lane < nw ? red[lane] : ident;
  return wave_nan_max(r);
}

// Fast exp/log on the hardware exp2/log2 units (about 1 ulp in fp32).
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float fast_log(float x) {
  return __builtin_amdgcn_logf(x) * 0.6931471805599453f;
}
// silu(a) * b in fp32 (a / (1 + e^-a) * b on the hardware exp2 and
// reciprocal): the SwiGLU product of silu_mul and of the matmul epilogue
// that fuses it, one expression so the two round alike.  The fp32 product is
// materialised (an empty asm) before the caller converts it: with an f16
// operand the compiler otherwise folds the last multiply and the conversion
// into v_fma_mix, which rounds once where the fp32 product rounded to f16
// (CPU ATen's order) rounds twice.
__device__ __forceinline__ float silu_mul_f32(float a, float b) {
  float r = a * __builtin_amdgcn_rcpf(1.0f + fast_exp(-a)) * b;
  asm volatile("" : "+v"(r));
  return r;
}

// Global -> LDS copy of 16 bytes a lane (global_load_lds_dwordx4) from a
// wave-uniform base plus a 32-bit per-lane byte offset, to the wave's 1 KiB
// at `lds` (M0).  Written as inline assembly so that the compiler does not
// track it: it counts such a copy as a FLAT access that may touch LDS, and
// while one is in flight every wait for an LDS read it emits is lgkmcnt(0),
// so a fragment read issued ahead of the MFMA before it is waited for
// there.  Callers wait for their copies themselves (vmcnt) before the
// barrier that publishes them.  The s_nop is the wait state an LDS DMA
// needs after M0 is written.  The base must be wave-uniform; it is read
// from the first lane (free when it is already in scalar registers, which
// the "s" operand needs).
__device__ __forceinline__ void lds_copy16(const void* base, uint32_t off, void* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  // (readfirstlane returns int: each word goes through uint32_t so that the
  // low word is zero-extended, not sign-extended into the high one)
  const uint64_t b = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint64_t sb = ((uint64_t)hi << 32) | lo;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(sb), "{m0}"(m0)
               : "memory");
}

// ---- streaming 16-byte accesses ----------------------------------------------

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Non-temporal (nt bit) 16-byte load / store, for data a kernel touches once:
// the lines are not kept in L2 / MALL, which lifts a copy-shaped kernel from
// about 5.5 to about 6.1 TB/s on MI355X.  V is any 16-byte trivially
// copyable type (uint4, a union of lanes, ...).
template <typename V>
__device__ __forceinline__ V ld_stream(const V* p) {
  static_assert(sizeof(V) == 16, "16-byte type expected");
  return __builtin_bit_cast(V, __builtin_nontemporal_load((const u32x4_t*)p));
}
template <typename V>
__device__ __forceinline__ void st_stream(V* p, const V& v) {
  static_assert(sizeof(V) == 16, "16-byte type expected");
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), (u32x4_t*)p);
}

inline unsigned ceil_div_u(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace mi
