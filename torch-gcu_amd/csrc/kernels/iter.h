// Host-side TensorIterator equivalent: broadcasts operands to the output
// shape, removes size-1 dimensions and merges dimensions that are contiguous
// in every operand, so that kernels see the fewest, longest dimensions.
#pragma once

#include "common.h"

namespace mi {

constexpr int kMaxOperands = 4;

struct Iter {
  int ndim = 0;                               // after coalescing
  int nops = 0;                               // operand 0 is the output
  int64_t sizes[MI_MAX_DIMS] = {};            // outermost first
  int64_t strides[kMaxOperands][MI_MAX_DIMS] = {};  // in elements
  char* data[kMaxOperands] = {};
  int dtype[kMaxOperands] = {};
  int64_t numel = 0;

  // All operands are dense over the iteration space (stride 1 innermost, no
  // gaps) or broadcast scalars (every stride 0).
  bool op_contiguous(int i) const;
  bool op_scalar(int i) const;
};

// Builds an iterator over out's shape.  Each input must broadcast to out
// (numpy rules, right-aligned).  Returns MI_ERR_INVALID otherwise.
mi_status_t make_iter(Iter& it, const mi_tensor_t& out, const mi_tensor_t* const* ins,
                      int nin);

// Device-side offset calculator (up to MI_MAX_DIMS dims, NOPS operands).
template <int NOPS>
struct OffsetCalc {
  int ndim;
  int64_t sizes[MI_MAX_DIMS];
  int64_t strides[NOPS][MI_MAX_DIMS];

  __device__ __forceinline__ void get(int64_t linear, int64_t* offs) const {
#pragma unroll
    for (int o = 0; o < NOPS; ++o) offs[o] = 0;
    for (int d = ndim - 1; d >= 0; --d) {
      const int64_t sz = sizes[d];
      int64_t q, r;
      if (linear < 0x7fffffffLL && sz < 0x7fffffffLL) {
        const uint32_t l32 = (uint32_t)linear, s32 = (uint32_t)sz;
        q = l32 / s32;
        r = l32 - (uint32_t)q * s32;
      } else {
        q = linear / sz;
        r = linear - q * sz;
      }
#pragma unroll
      for (int o = 0; o < NOPS; ++o) offs[o] += r * strides[o][d];
      linear = q;
    }
  }
};

template <int NOPS>
OffsetCalc<NOPS> make_offset_calc(const Iter& it) {
  OffsetCalc<NOPS> oc;
  oc.ndim = it.ndim;
  for (int d = 0; d < MI_MAX_DIMS; ++d) {
    oc.sizes[d] = d < it.ndim ? it.sizes[d] : 1;
    for (int o = 0; o < NOPS; ++o) oc.strides[o][d] = d < it.ndim ? it.strides[o][d] : 0;
  }
  return oc;
}

// Host helpers for scalar conversion, with the same rounding as c10.
uint16_t host_f32_to_bf16(float f);
uint16_t host_f32_to_f16(float f);
float host_bf16_to_f32(uint16_t v);
float host_f16_to_f32(uint16_t v);

// Value of a scalar as double / int64.
inline double scalar_as_double(const mi_scalar_t& s) {
  return is_floating(s.dtype) ? s.f : (double)s.i;
}
inline int64_t scalar_as_int(const mi_scalar_t& s) {
  return is_floating(s.dtype) ? (int64_t)s.f : s.i;
}
// Effective dtype a scalar takes in type promotion (wrapped float numbers
// count as the default dtype float32, wrapped ints as int64).
inline int scalar_promo_dtype(const mi_scalar_t& s) {
  if (s.wrapped && is_floating(s.dtype)) return MI_F32;
  return s.dtype;
}

// ATen's result_type over operands in three priority classes: dimensioned
// tensors, 0-dim tensors, wrapped numbers (at::native::result_type).
struct ResultType {
  int dim_result = -1, zero_result = -1, wrapped_result = -1;
  void add_tensor(const mi_tensor_t& t);
  void add_scalar(const mi_scalar_t& s);
  int get() const;
};

}  // namespace mi
