#include "iter.h"

#include <cmath>
#include <cstring>

namespace mi {

bool Iter::op_contiguous(int i) const {
  int64_t expected = 1;
  for (int d = ndim - 1; d >= 0; --d) {
    if (strides[i][d] != expected) return false;
    expected *= sizes[d];
  }
  return true;
}

bool Iter::op_scalar(int i) const {
  for (int d = 0; d < ndim; ++d)
    if (strides[i][d] != 0) return false;
  return true;
}

mi_status_t make_iter(Iter& it, const mi_tensor_t& out, const mi_tensor_t* const* ins,
                      int nin) {
  if (nin + 1 > kMaxOperands)
    MI_FAIL(MI_ERR_INVALID, "make_iter: too many operands (%d)", nin + 1);
  it = Iter();
  it.nops = nin + 1;
  const int nd = out.ndim;
  int64_t sizes[MI_MAX_DIMS];
  int64_t strides[kMaxOperands][MI_MAX_DIMS];
  for (int d = 0; d < nd; ++d) {
    sizes[d] = out.sizes[d];
    strides[0][d] = out.strides[d];
  }
  it.data[0] = (char*)out.data;
  it.dtype[0] = out.dtype;
  for (int k = 0; k < nin; ++k) {
    const mi_tensor_t& t = *ins[k];
    if (t.ndim > nd)
      MI_FAIL(MI_ERR_INVALID, "operand %d has %d dims but the output has %d", k + 1,
              t.ndim, nd);
    const int off = nd - t.ndim;
    for (int d = 0; d < nd; ++d) {
      if (d < off) {
        strides[k + 1][d] = 0;
        continue;
      }
      const int64_t s = t.sizes[d - off];
      if (s == sizes[d]) {
        strides[k + 1][d] = s == 1 ? 0 : t.strides[d - off];
      } else if (s == 1) {
        strides[k + 1][d] = 0;
      } else {
        MI_FAIL(MI_ERR_INVALID,
                "operand %d of size %lld does not broadcast to %lld at dim %d", k + 1,
                (long long)s, (long long)sizes[d], d);
      }
    }
    it.data[k + 1] = (char*)t.data;
    it.dtype[k + 1] = t.dtype;
  }
  // Output dims of size 1 carry no iteration; zero their strides.
  it.numel = 1;
  for (int d = 0; d < nd; ++d) it.numel *= sizes[d];

  // Drop size-1 dims, then merge (outer d, inner e) when contiguous for all.
  int m = 0;
  int64_t csz[MI_MAX_DIMS];
  int64_t cst[kMaxOperands][MI_MAX_DIMS];
  for (int d = 0; d < nd; ++d) {
    if (sizes[d] == 1) continue;
    if (m > 0) {
      bool can = true;
      for (int o = 0; o < it.nops && can; ++o)
        can = cst[o][m - 1] == strides[o][d] * sizes[d];
      if (can) {
        csz[m - 1] *= sizes[d];
        for (int o = 0; o < it.nops; ++o) cst[o][m - 1] = strides[o][d];
        continue;
      }
    }
    csz[m] = sizes[d];
    for (int o = 0; o < it.nops; ++o) cst[o][m] = strides[o][d];
    ++m;
  }
  if (m == 0 && it.numel == 1) {
    // one element: iterate a single dim of size 1
    csz[0] = 1;
    for (int o = 0; o < it.nops; ++o) cst[o][0] = 1;
    m = 1;
  }
  it.ndim = m;
  for (int d = 0; d < m; ++d) {
    it.sizes[d] = csz[d];
    for (int o = 0; o < it.nops; ++o) it.strides[o][d] = cst[o][d];
  }
  return MI_OK;
}

uint16_t host_f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if (std::isnan(f)) return 0x7FC0;
  const uint32_t rounding_bias = 0x7FFF + ((u >> 16) & 1);
  return (uint16_t)((u + rounding_bias) >> 16);
}

float host_bf16_to_f32(uint16_t v) {
  uint32_t u = ((uint32_t)v) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// IEEE binary16 conversion with round to nearest even.
uint16_t host_f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000;
  uint32_t mag = x & 0x7FFFFFFF;
  if (mag >= 0x7F800000) {  // inf or nan
    return (uint16_t)(sign | 0x7C00 | (mag > 0x7F800000 ? 0x200 | ((mag >> 13) & 0x3FF) : 0));
  }
  if (mag >= 0x477FF000) return (uint16_t)(sign | 0x7C00);  // rounds to inf
  if (mag < 0x38800000) {  // result is subnormal or zero
    // value = mag as float; subnormal step is 2^-24
    float a;
    std::memcpy(&a, &mag, 4);
    const float scaled = a * 16777216.0f;  // exact: scaling by 2^24
    // round to nearest even integer
    float r = std::nearbyint(scaled);
    return (uint16_t)(sign | (uint32_t)r);
  }
  const uint32_t exp = ((mag >> 23) - 127 + 15) << 10;
  const uint32_t mant = mag & 0x7FFFFF;
  uint32_t h = exp | (mant >> 13);
  const uint32_t rem = mant & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h += 1;
  return (uint16_t)(sign | h);
}

float host_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000) << 16;
  const uint32_t exp = (h >> 10) & 0x1F;
  const uint32_t mant = h & 0x3FF;
  float r;
  if (exp == 0) {
    r = std::ldexp((float)mant, -24);
    uint32_t u;
    std::memcpy(&u, &r, 4);
    u |= sign;
    std::memcpy(&r, &u, 4);
    return r;
  }
  uint32_t u;
  if (exp == 31) {
    u = sign | 0x7F800000 | (mant << 13);
  } else {
    u = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  std::memcpy(&r, &u, 4);
  return r;
}

namespace {
int promote_skip(int a, int b) {
  if (a < 0) return b;
  if (b < 0) return a;
  return promote_types(a, b);
}
// at::native combine_categories
int combine_categories(int higher, int lower) {
  if (higher >= 0 && is_floating(higher)) return higher;
  if (higher == MI_BOOL || (lower >= 0 && is_floating(lower)))
    return promote_skip(higher, lower);
  if (higher >= 0) return higher;
  return lower;
}
}  // namespace

void ResultType::add_tensor(const mi_tensor_t& t) {
  if (t.ndim > 0)
    dim_result = promote_skip(dim_result, t.dtype);
  else
    zero_result = promote_skip(zero_result, t.dtype);
}

void ResultType::add_scalar(const mi_scalar_t& s) {
  if (s.wrapped)
    wrapped_result = promote_skip(wrapped_result, scalar_promo_dtype(s));
  else
    zero_result = promote_skip(zero_result, s.dtype);
}

int ResultType::get() const {
  return combine_categories(dim_result, combine_categories(zero_result, wrapped_result));
}

}  // namespace mi
