// cat: out = torch.cat(inputs, dim).
//
// With out and every input dense in the same dim order (row-major,
// channels-last, ...) and of out's dtype, out is
// [outer, T, inner] around `dim` and input i is [outer, L_i, inner]: each of
// its `outer` rows is one run of L_i*inner elements that lands at element
// offset (o*T + off_i)*inner of out.  So the whole cat is one launch of a
// batched row copy: input i's rows, flattened, are cut into chunks of
// kCatChunk words, one chunk per block, and the blocks of all inputs form one
// grid (HBM-bound: every byte is read once and written once).  A word is the
// widest of 16, 8, 4, 2 or 1 bytes that divides every address, row length
// and offset involved; 16-byte words move with non-temporal loads and stores.
// Any other layout or a dtype cast copies input by input into out's slices
// through mi_copy.
#include "iter.h"

namespace mi {
namespace {

constexpr int kCatBlock = 256;
constexpr int kCatUnroll = 4;
constexpr int64_t kCatChunk = (int64_t)kCatBlock * kCatUnroll;  // words per block
constexpr int kCatParts = 32;                                   // inputs per launch

struct CatPart {
  const void* src;
  int64_t row_words;    // words in one row of this input (L_i * inner)
  int64_t dst_word;     // word offset of the input's slice inside an out row
  int64_t first_block;  // first block of the grid that copies this input
  int32_t log2_row;     // log2(row_words) when a power of two, else -1
};

struct CatArgs {
  void* out;
  int64_t out_row_words;  // T * inner
  int64_t outer;
  int32_t n;
  CatPart part[kCatParts];
};

template <typename W>
__device__ __forceinline__ W cat_load(const W* p) {
  if constexpr (sizeof(W) == 16) return ld_stream(p);
  else return *p;
}
template <typename W>
__device__ __forceinline__ void cat_store(W* p, const W& v) {
  if constexpr (sizeof(W) == 16) st_stream(p, v);
  else *p = v;
}

template <typename W>
__global__ __launch_bounds__(kCatBlock) void cat_rows_kernel(CatArgs a) {
  // the input this block copies (uniform: the part table is kernel arguments)
  int p = 0;
  while (p + 1 < a.n && (int64_t)blockIdx.x >= a.part[p + 1].first_block) ++p;
  const CatPart& c = a.part[p];
  const int64_t rw = c.row_words;
  const int64_t total = a.outer * rw;
  const int64_t base = ((int64_t)blockIdx.x - c.first_block) * kCatChunk + threadIdx.x;
  const W* src = (const W*)c.src;
  W* out = (W*)a.out;
  const bool small = total < 0x7fffffffLL;
  W v[kCatUnroll];
#pragma unroll
  for (int u = 0; u < kCatUnroll; ++u) {
    const int64_t t = base + (int64_t)u * kCatBlock;
    if (t < total) v[u] = cat_load(src + t);
  }
#pragma unroll
  for (int u = 0; u < kCatUnroll; ++u) {
    const int64_t t = base + (int64_t)u * kCatBlock;
    if (t < total) {
      int64_t o, w;
      if (c.log2_row >= 0) {
        o = t >> c.log2_row;
        w = t & (rw - 1);
      } else if (small) {  // 32-bit division is several times cheaper
        const uint32_t o32 = (uint32_t)t / (uint32_t)rw;
        o = o32;
        w = (uint32_t)t - o32 * (uint32_t)rw;
      } else {
        o = t / rw;
        w = t - o * rw;
      }
      cat_store(out + o * a.out_row_words + c.dst_word + w, v[u]);
    }
  }
}

bool dense_rowmajor(const mi_tensor_t& t) {
  int64_t st = 1;
  for (int d = t.ndim - 1; d >= 0; --d) {
    if (t.sizes[d] != 1 && t.strides[d] != st) return false;
    st *= t.sizes[d];
  }
  return true;
}

// One launch over up to kCatParts non-empty dense inputs of out's dtype;
// lens / offs are their sizes and offsets along the cat dim.
mi_status_t launch_rows(void* out, int dtype, const void* const* srcs, const int64_t* lens,
                        const int64_t* offs, int n, int64_t outer, int64_t inner, int64_t T,
                        hipStream_t stream) {
  const int64_t es = dtype_size(dtype);
  uint64_t bits = (uint64_t)(uintptr_t)out | (uint64_t)(T * inner * es);
  for (int i = 0; i < n; ++i)
    bits |= (uint64_t)(uintptr_t)srcs[i] | (uint64_t)(lens[i] * inner * es) |
            (uint64_t)(offs[i] * inner * es);
  auto go = [&](auto tag) -> mi_status_t {
    using W = decltype(tag);
    constexpr int64_t ws = sizeof(W);
    CatArgs a{};
    a.out = out;
    a.out_row_words = T * inner * es / ws;
    a.outer = outer;
    a.n = n;
    int64_t blocks = 0;
    for (int i = 0; i < n; ++i) {
      CatPart& c = a.part[i];
      c.src = srcs[i];
      c.row_words = lens[i] * inner * es / ws;
      c.dst_word = offs[i] * inner * es / ws;
      c.first_block = blocks;
      c.log2_row = -1;
      if ((c.row_words & (c.row_words - 1)) == 0) {
        c.log2_row = 0;
        while ((int64_t(1) << c.log2_row) < c.row_words) ++c.log2_row;
      }
      blocks += (outer * c.row_words + kCatChunk - 1) / kCatChunk;
    }
    MI_CHECK_ARG(blocks <= 0x7fffffffLL, "cat: %lld blocks exceed the grid limit",
                 (long long)blocks);
    hipLaunchKernelGGL(cat_rows_kernel<W>, dim3((unsigned)blocks), dim3(kCatBlock), 0, stream, a);
    return check_launch("cat rows");
  };
  if (bits % 16 == 0) return go(uint4{});
  if (bits % 8 == 0) return go(uint2{});
  if (bits % 4 == 0) return go(uint32_t{});
  if (bits % 2 == 0) return go(uint16_t{});
  return go(uint8_t{});
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status_t mi_cat(const mi_tensor_t* out, const mi_tensor_t* const* inputs,
                              int32_t n_inputs, int32_t dim, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  MI_CHECK_ARG(n_inputs >= 1 && inputs != nullptr, "cat: expected at least one input, got %d",
               (int)n_inputs);
  MI_CHECK_ARG(out->ndim >= 1, "cat: out must have at least one dim");
  MI_CHECK_ARG(dim >= 0 && dim < out->ndim, "cat: dim %d out of range for %d dims", (int)dim,
               (int)out->ndim);
  // dims in out's memory order (largest stride first): a channels-last out
  // with channels-last inputs is row-major in that order
  int perm[MI_MAX_DIMS];
  for (int d = 0; d < out->ndim; ++d) perm[d] = d;
  for (int a = 1; a < out->ndim; ++a)
    for (int b = a; b > 0 && out->strides[perm[b]] > out->strides[perm[b - 1]]; --b) {
      const int x = perm[b];
      perm[b] = perm[b - 1];
      perm[b - 1] = x;
    }
  auto permuted = [&](const mi_tensor_t& t) {
    mi_tensor_t r = t;
    for (int d = 0; d < t.ndim; ++d) {
      r.sizes[d] = t.sizes[perm[d]];
      r.strides[d] = t.strides[perm[d]];
    }
    return r;
  };
  int pdim = 0;
  while (perm[pdim] != dim) ++pdim;
  const mi_tensor_t pout = permuted(*out);
  int64_t sum = 0;
  bool rows_ok = dense_rowmajor(pout);
  for (int i = 0; i < n_inputs; ++i) {
    const mi_tensor_t* t = inputs[i];
    MI_CHECK_ARG(t != nullptr, "cat: input %d is null", i);
    MI_RETURN_IF(validate(t, "input"));
    MI_CHECK_ARG(t->ndim == out->ndim, "cat: input %d has %d dims, out has %d", i, (int)t->ndim,
                 (int)out->ndim);
    for (int d = 0; d < out->ndim; ++d)
      MI_CHECK_ARG(d == dim || t->sizes[d] == out->sizes[d],
                   "cat: input %d has size %lld in dim %d, out has %lld", i,
                   (long long)t->sizes[d], d, (long long)out->sizes[d]);
    sum += t->sizes[dim];
    rows_ok = rows_ok && t->dtype == out->dtype && dense_rowmajor(permuted(*t));
  }
  MI_CHECK_ARG(sum == out->sizes[dim], "cat: input sizes along dim %d add up to %lld, out has %lld",
               (int)dim, (long long)sum, (long long)out->sizes[dim]);
  if (numel(*out) == 0) return MI_OK;
  const int es = dtype_size(out->dtype);
  if (!rows_ok) {
    // input by input into out's slice (casts and any strides)
    int64_t off = 0;
    for (int i = 0; i < n_inputs; ++i) {
      const int64_t L = inputs[i]->sizes[dim];
      if (L > 0) {
        mi_tensor_t slice = *out;
        slice.data = (char*)out->data + off * out->strides[dim] * es;
        slice.sizes[dim] = L;
        MI_RETURN_IF(mi_copy(&slice, inputs[i], stream_));
      }
      off += L;
    }
    return MI_OK;
  }
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < pdim; ++d) outer *= pout.sizes[d];
  for (int d = pdim + 1; d < out->ndim; ++d) inner *= pout.sizes[d];
  const void* srcs[kCatParts];
  int64_t lens[kCatParts], offs[kCatParts];
  int k = 0;
  int64_t off = 0;
  for (int i = 0; i < n_inputs; ++i) {
    const int64_t L = inputs[i]->sizes[dim];
    if (L > 0) {
      srcs[k] = inputs[i]->data;
      lens[k] = L;
      offs[k] = off;
      if (++k == kCatParts) {
        MI_RETURN_IF(launch_rows(out->data, out->dtype, srcs, lens, offs, k, outer, inner,
                                 out->sizes[dim], stream));
        k = 0;
      }
    }
    off += L;
  }
  if (k > 0)
    MI_RETURN_IF(launch_rows(out->data, out->dtype, srcs, lens, offs, k, outer, inner,
                             out->sizes[dim], stream));
  return MI_OK;
}
