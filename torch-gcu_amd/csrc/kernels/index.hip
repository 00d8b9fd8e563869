// index_select: out = self.index_select(dim, index).
//
// self is viewed as [outer, S, inner] around `dim`, out as [outer, N, inner].
// When self and out are dense, a selected slice is a run of inner*esize
// bytes (64 B for config 1's int64 [1048576, 8] table, 8 KiB for a bf16
// embedding row of 4096), moved in 16-byte pieces by consecutive lanes so a
// wave reads whole rows with coalesced loads.  Any other layout takes the
// general path (one element per lane, full offset arithmetic).
#include "iter.h"

namespace mi {
namespace {

constexpr int kBlock = 256;

template <typename IdxT>
__device__ __forceinline__ int64_t read_index(const IdxT* idx, int64_t i, int64_t istride) {
  return (int64_t)idx[i * istride];
}

// Dense rows, moved as 16-byte (W = uint4) or 8/4/2/1-byte words.  A lane
// takes kGatherU words a grid apart and issues their index loads, then their
// row loads, then their stores, so four index -> row chains are in flight
// per lane (the four lanes of a 64-byte row share its index load).  When the
// words per row are a power of two (LOG2 >= 0) the row and word come from a
// shift and a mask instead of a division.
constexpr int kGatherU = 4;  // words per lane: their index loads, then row loads, in flight

template <typename W, typename IdxT>
__global__ __launch_bounds__(kBlock) void gather_rows_kernel(
    W* __restrict__ out, const W* __restrict__ self, const IdxT* __restrict__ idx,
    int64_t istride, int64_t outer, int64_t n_idx, int64_t src_rows, int64_t words_per_row,
    int log2_wpr, IndexFault* fault) {
  const int64_t total = outer * n_idx * words_per_row;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  const bool small = total < 0x7fffffffLL;
  // Every load is unconditional: a word past the end decodes word total - 1
  // (not stored), and an out-of-range index reads row 0 (stored as zeros),
  // so the compiler's waits cover all kGatherU index loads at once and then
  // all row loads at once (with the loads under a branch each waited alone).
  int64_t tt[kGatherU], w[kGatherU], o[kGatherU], s[kGatherU];
#pragma unroll
  for (int u = 0; u < kGatherU; ++u) {
    const int64_t t0 = (int64_t)blockIdx.x * kBlock + threadIdx.x + u * stride;
    tt[u] = t0;
    const int64_t t = t0 < total ? t0 : total - 1;
    int64_t rr, ww, i;
    if (log2_wpr >= 0) {
      rr = t >> log2_wpr;
      ww = t & (words_per_row - 1);
    } else if (small) {  // 32-bit division is several times cheaper
      const uint32_t r32 = (uint32_t)t / (uint32_t)words_per_row;
      ww = (uint32_t)t - r32 * (uint32_t)words_per_row;
      rr = r32;
    } else {
      rr = t / words_per_row;
      ww = t - rr * words_per_row;
    }
    if (outer == 1) {
      o[u] = 0;
      i = rr;
    } else {
      o[u] = rr / n_idx;
      i = rr - o[u] * n_idx;
    }
    w[u] = ww;
    s[u] = read_index(idx, i, istride);
  }
  W v[kGatherU];
  bool ok[kGatherU];
#pragma unroll
  for (int u = 0; u < kGatherU; ++u) {
    ok[u] = s[u] >= 0 && s[u] < src_rows;
    v[u] = self[(o[u] * src_rows + (ok[u] ? s[u] : 0)) * words_per_row + w[u]];
  }
#pragma unroll
  for (int u = 0; u < kGatherU; ++u) {
    if (tt[u] < total) {
      if (!ok[u]) record_index_fault(fault, s[u], src_rows);
      const W r = ok[u] ? v[u] : W{};
      if constexpr (sizeof(W) == 16) st_stream(out + tt[u], r);
      else out[tt[u]] = r;
    }
  }
}

// General layout: iterate over out elements; coordinates decoded per element.
struct GatherGeneral {
  int ndim;
  int dim;
  int64_t sizes[MI_MAX_DIMS];  // out sizes
  int64_t ostrides[MI_MAX_DIMS];
  int64_t sstrides[MI_MAX_DIMS];
  int64_t src_dim_size;
};

template <typename T, typename IdxT>
__global__ __launch_bounds__(kBlock) void gather_general_kernel(T* out, const T* self,
                                                                const IdxT* idx,
                                                                int64_t istride,
                                                                GatherGeneral g, int64_t n,
                                                                IndexFault* fault) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < n; t += stride) {
    int64_t lin = t, oo = 0, so = 0;
    bool ok = true;
    for (int d = g.ndim - 1; d >= 0; --d) {
      const int64_t c = lin % g.sizes[d];
      lin /= g.sizes[d];
      oo += c * g.ostrides[d];
      if (d == g.dim) {
        const int64_t s = read_index(idx, c, istride);
        ok = s >= 0 && s < g.src_dim_size;
        if (!ok) record_index_fault(fault, s, g.src_dim_size);
        so += s * g.sstrides[d];
      } else {
        so += c * g.sstrides[d];
      }
    }
    out[oo] = ok ? self[so] : T{};
  }
}

unsigned grid_for(int64_t n) {
  const int64_t want = (n + kBlock - 1) / kBlock;
  const int64_t cap = (int64_t)cu_count() * 64;
  return (unsigned)(want < cap ? (want < 1 ? 1 : want) : cap);
}

template <typename IdxT>
mi_status_t launch_rows(const mi_tensor_t* out, const mi_tensor_t* self, const IdxT* idx,
                        int64_t istride, int64_t outer, int64_t n_idx, int64_t src_rows,
                        int64_t row_bytes, hipStream_t stream) {
  const uintptr_t align = (uintptr_t)out->data | (uintptr_t)self->data;
  if (outer * n_idx * row_bytes == 0) return MI_OK;
  // no source rows: every index is out of range, and the kernel's loads of
  // row 0 would have nothing to read
  if (src_rows == 0) return mi_fill(out, mi_scalar_t{0.0, 0, MI_F32, 1}, (mi_stream_t)stream);
  auto go = [&](auto word) -> mi_status_t {
    typedef decltype(word) W;
    const int64_t wpr = row_bytes / (int64_t)sizeof(W);
    const int64_t total = outer * n_idx * wpr;
    int log2_wpr = -1;
    if ((wpr & (wpr - 1)) == 0) {
      log2_wpr = 0;
      while ((int64_t(1) << log2_wpr) < wpr) ++log2_wpr;
    }
    const int64_t nb = (total + (int64_t)kBlock * kGatherU - 1) / ((int64_t)kBlock * kGatherU);
    MI_CHECK_ARG(nb <= 0x7fffffffLL, "index_select: too many rows");
    hipLaunchKernelGGL((gather_rows_kernel<W, IdxT>), dim3((unsigned)nb), dim3(kBlock), 0,
                       stream, (W*)out->data, (const W*)self->data, idx, istride, outer, n_idx,
                       src_rows, wpr, log2_wpr, index_fault_word());
    return check_launch("index_select rows");
  };
  if (row_bytes % 16 == 0 && align % 16 == 0) return go(uint4{});
  if (row_bytes % 8 == 0 && align % 8 == 0) return go(uint2{});
  if (row_bytes % 4 == 0 && align % 4 == 0) return go(uint32_t{});
  if (row_bytes % 2 == 0 && align % 2 == 0) return go(uint16_t{});
  return go(uint8_t{});
}

template <typename IdxT>
mi_status_t launch_general(const mi_tensor_t* out, const mi_tensor_t* self, int dim,
                           const IdxT* idx, int64_t istride, hipStream_t stream) {
  GatherGeneral g;
  g.ndim = out->ndim;
  g.dim = dim;
  for (int d = 0; d < MI_MAX_DIMS; ++d) {
    g.sizes[d] = d < out->ndim ? out->sizes[d] : 1;
    g.ostrides[d] = d < out->ndim ? out->strides[d] : 0;
    g.sstrides[d] = d < self->ndim ? self->strides[d] : 0;
  }
  g.src_dim_size = self->sizes[dim];
  const int64_t n = numel(*out);
  const unsigned grid = grid_for(n);
  IndexFault* fault = index_fault_word();
  switch (dtype_size(out->dtype)) {
    case 1: hipLaunchKernelGGL((gather_general_kernel<uint8_t, IdxT>), dim3(grid), dim3(kBlock), 0, stream, (uint8_t*)out->data, (const uint8_t*)self->data, idx, istride, g, n, fault); break;
    case 2: hipLaunchKernelGGL((gather_general_kernel<uint16_t, IdxT>), dim3(grid), dim3(kBlock), 0, stream, (uint16_t*)out->data, (const uint16_t*)self->data, idx, istride, g, n, fault); break;
    case 4: hipLaunchKernelGGL((gather_general_kernel<uint32_t, IdxT>), dim3(grid), dim3(kBlock), 0, stream, (uint32_t*)out->data, (const uint32_t*)self->data, idx, istride, g, n, fault); break;
    default: hipLaunchKernelGGL((gather_general_kernel<uint64_t, IdxT>), dim3(grid), dim3(kBlock), 0, stream, (uint64_t*)out->data, (const uint64_t*)self->data, idx, istride, g, n, fault); break;
  }
  return check_launch("index_select general");
}

template <typename IdxT>
mi_status_t index_select_t(const mi_tensor_t* out, const mi_tensor_t* self, int dim,
                           const mi_tensor_t* index, hipStream_t stream) {
  const IdxT* idx = (const IdxT*)index->data;
  const int64_t istride = index->ndim == 1 ? index->strides[0] : 1;
  const int64_t n_idx = index->ndim == 1 ? index->sizes[0] : 1;
  if (self->ndim == 0) {
    // 0-dim self: every index must be 0; out is 0-dim or [n_idx] of one value
    mi_tensor_t s1 = *self, o1 = *out;
    s1.ndim = 1;
    s1.sizes[0] = 1;
    s1.strides[0] = 1;
    if (o1.ndim == 0) {
      o1.ndim = 1;
      o1.sizes[0] = 1;
      o1.strides[0] = 1;
    }
    return launch_general<IdxT>(&o1, &s1, 0, idx, istride, stream);
  }
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < dim; ++d) outer *= self->sizes[d];
  for (int d = dim + 1; d < self->ndim; ++d) inner *= self->sizes[d];
  if (is_contiguous(*self) && is_contiguous(*out))
    return launch_rows<IdxT>(out, self, idx, istride, outer, n_idx, self->sizes[dim],
                             inner * dtype_size(self->dtype), stream);
  return launch_general<IdxT>(out, self, dim, idx, istride, stream);
}

// ---- advanced index (aten::index with integer index tensors) ---------------
//
// out = self[indices] with ATen's rules: the defined index tensors (already
// broadcast to one shape B by the caller, stride 0 where broadcast) select
// along their dims; out is self.shape[:first] + B + self.shape[last+1:]
// when the indexed dims are adjacent, else B + the other dims in order.
// out is dense; every out dim maps either to a self dim (a stride into
// self) or to a dim of B (a stride into each index tensor).  Trailing out
// dims that run contiguously through self are folded into a row copied in
// 16/8/4/2/1-byte words.  Negative indices count from the end; an index
// still out of range selects nothing and its row is written as zeros (the
// kernel never reads outside self).
constexpr int kMaxIdx = MI_MAX_DIMS;

struct AdvIndex {
  int nd;     // out dims decoded per row (the folded inner dims excluded)
  int n_idx;  // defined index tensors
  uint32_t idx64;  // bit k: index k is int64 (else int32)
  int64_t sizes[MI_MAX_DIMS];       // out sizes of the decoded dims
  int64_t src_bstride[MI_MAX_DIMS]; // self byte stride per decoded dim (0 for dims of B)
  int64_t idx_stride[kMaxIdx][MI_MAX_DIMS];  // element stride of index k per decoded dim
  const void* idx[kMaxIdx];
  int64_t limit[kMaxIdx];           // size of the self dim index k selects
  int64_t sel_bstride[kMaxIdx];     // byte stride of that self dim
};

// Byte offset into self of a row (out coordinates decoded from `row`), or -1
// when an index is out of range.
__device__ __forceinline__ int64_t adv_row_offset(const AdvIndex& a, int64_t row,
                                                  IndexFault* fault) {
  int64_t off = 0;
  int64_t ioff[kMaxIdx];
#pragma unroll
  for (int k = 0; k < kMaxIdx; ++k) ioff[k] = 0;
  for (int d = a.nd - 1; d >= 0; --d) {
    const int64_t sz = a.sizes[d];
    const int64_t q = row / sz;
    const int64_t c = row - q * sz;
    row = q;
    off += c * a.src_bstride[d];
#pragma unroll
    for (int k = 0; k < kMaxIdx; ++k)
      if (k < a.n_idx) ioff[k] += c * a.idx_stride[k][d];
  }
#pragma unroll
  for (int k = 0; k < kMaxIdx; ++k) {
    if (k < a.n_idx) {
      int64_t v = ((a.idx64 >> k) & 1) ? ((const int64_t*)a.idx[k])[ioff[k]]
                                       : (int64_t)((const int32_t*)a.idx[k])[ioff[k]];
      const int64_t v0 = v;
      if (v < 0) v += a.limit[k];
      if (v < 0 || v >= a.limit[k]) {
        record_index_fault(fault, v0, a.limit[k]);
        return -1;
      }
      off += v * a.sel_bstride[k];
    }
  }
  return off;
}

// Short rows: one word per lane, rows decoded per word.
template <typename W>
__global__ __launch_bounds__(kBlock) void adv_index_words_kernel(W* __restrict__ out,
                                                                 const char* __restrict__ src,
                                                                 AdvIndex a, int64_t rows,
                                                                 int64_t wpr, IndexFault* fault) {
  const int64_t total = rows * wpr;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
    const int64_t row = wpr == 1 ? t : t / wpr;
    const int64_t w = t - row * wpr;
    const int64_t off = adv_row_offset(a, row, fault);
    out[t] = off >= 0 ? ((const W*)(src + off))[w] : W{};
  }
}

// Long rows (64 words or more): a wave per row, the row decoded once and its
// words moved by the 64 lanes, four loads in flight per lane.
template <typename W>
__global__ __launch_bounds__(kBlock) void adv_index_rows_kernel(W* __restrict__ out,
                                                                const char* __restrict__ src,
                                                                AdvIndex a, int64_t rows,
                                                                int64_t wpr, IndexFault* fault) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
  const int64_t nwaves = ((int64_t)gridDim.x * kBlock) >> 6;
  for (int64_t row = wave; row < rows; row += nwaves) {
    const int64_t off = adv_row_offset(a, row, lane == 0 ? fault : nullptr);
    const W* s = (const W*)(src + (off >= 0 ? off : 0));
    W* o = out + row * wpr;
    for (int64_t w0 = lane; w0 < wpr; w0 += 4 * 64) {
      W v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t w = w0 + u * 64;
        v[u] = (off >= 0 && w < wpr) ? s[w] : W{};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t w = w0 + u * 64;
        if (w < wpr) {
          if constexpr (sizeof(W) == 16) st_stream(o + w, v[u]);
          else o[w] = v[u];
        }
      }
    }
  }
}

mi_status_t run_adv_index(const mi_tensor_t* out, const mi_tensor_t* self,
                          const mi_tensor_t* const* indices, int32_t n_indices,
                          hipStream_t stream) {
  const int snd = self->ndim;
  MI_CHECK_ARG(n_indices >= 0 && n_indices <= snd, "index: %d indices for a tensor of %d dims",
               (int)n_indices, snd);
  MI_CHECK_ARG(out->dtype == self->dtype, "index: out dtype %s != self dtype %s",
               dtype_name(out->dtype), dtype_name(self->dtype));
  // the defined indices, their dims, and the broadcast shape B
  int kdim[kMaxIdx];
  const mi_tensor_t* kt[kMaxIdx];
  int nk = 0;
  for (int d = 0; d < n_indices; ++d) {
    if (indices == nullptr || indices[d] == nullptr) continue;
    MI_RETURN_IF(validate(indices[d], "index"));
    MI_CHECK_ARG(indices[d]->dtype == MI_I32 || indices[d]->dtype == MI_I64,
                 "index: index tensors must be int32 or int64, got %s",
                 dtype_name(indices[d]->dtype));
    kdim[nk] = d;
    kt[nk++] = indices[d];
  }
  MI_CHECK_ARG(nk > 0, "index: no index tensor given");
  const mi_tensor_t& b0 = *kt[0];
  for (int k = 1; k < nk; ++k) {
    bool same = kt[k]->ndim == b0.ndim;
    for (int d = 0; same && d < b0.ndim; ++d) same = kt[k]->sizes[d] == b0.sizes[d];
    MI_CHECK_ARG(same, "index: index tensors must be broadcast to one shape by the caller");
  }
  bool adjacent = true;
  for (int k = 1; k < nk; ++k) adjacent = adjacent && kdim[k] == kdim[k - 1] + 1;
  // out dims: (self dim or -1 for a dim of B, position in B)
  int map_self[2 * MI_MAX_DIMS], map_b[2 * MI_MAX_DIMS];
  int ond = 0;
  auto push_b = [&]() {
    for (int j = 0; j < b0.ndim; ++j) {
      map_self[ond] = -1;
      map_b[ond++] = j;
    }
  };
  bool is_indexed[MI_MAX_DIMS] = {};
  for (int k = 0; k < nk; ++k) is_indexed[kdim[k]] = true;
  if (!adjacent) push_b();
  for (int d = 0; d < snd; ++d) {
    if (is_indexed[d]) {
      if (adjacent && d == kdim[0]) push_b();
      continue;
    }
    map_self[ond] = d;
    map_b[ond++] = -1;
  }
  MI_CHECK_ARG(ond == out->ndim, "index: out has %d dims, expected %d", out->ndim, ond);
  int64_t bnum = 1;
  for (int j = 0; j < b0.ndim; ++j) bnum *= b0.sizes[j];
  for (int d = 0; d < ond; ++d) {
    const int64_t want = map_self[d] >= 0 ? self->sizes[map_self[d]] : b0.sizes[map_b[d]];
    MI_CHECK_ARG(out->sizes[d] == want, "index: out size %lld at dim %d, expected %lld",
                 (long long)out->sizes[d], d, (long long)want);
  }
  if (numel(*out) == 0) return MI_OK;
  for (int k = 0; k < nk; ++k)
    MI_CHECK_ARG(self->sizes[kdim[k]] > 0 || bnum == 0,
                 "index: index is out of bounds for dimension with size 0");
  if (!is_contiguous(*out)) MI_FAIL(MI_ERR_UNSUPPORTED, "index: out must be contiguous");
  const int64_t es = dtype_size(self->dtype);
  // fold trailing out dims that run contiguously through self into the row
  int64_t row_elems = 1;
  int nd = ond;
  while (nd > 0 && map_self[nd - 1] >= 0 && self->strides[map_self[nd - 1]] == row_elems) {
    row_elems *= self->sizes[map_self[nd - 1]];
    --nd;
  }
  AdvIndex a{};
  a.nd = nd;
  a.n_idx = nk;
  uintptr_t align = (uintptr_t)out->data | (uintptr_t)self->data | (uintptr_t)(row_elems * es);
  int64_t rows = 1;
  for (int d = 0; d < nd; ++d) {
    a.sizes[d] = out->sizes[d];
    rows *= out->sizes[d];
    if (map_self[d] >= 0) {
      a.src_bstride[d] = self->strides[map_self[d]] * es;
      align |= (uintptr_t)a.src_bstride[d];
    }
    for (int k = 0; k < nk; ++k)
      a.idx_stride[k][d] = map_b[d] >= 0 ? kt[k]->strides[map_b[d]] : 0;
  }
  for (int k = 0; k < nk; ++k) {
    a.idx[k] = kt[k]->data;
    if (kt[k]->dtype == MI_I64) a.idx64 |= 1u << k;
    a.limit[k] = self->sizes[kdim[k]];
    a.sel_bstride[k] = self->strides[kdim[k]] * es;
    align |= (uintptr_t)a.sel_bstride[k];
  }
  auto go = [&](auto word) -> mi_status_t {
    typedef decltype(word) W;
    const int64_t wpr = row_elems * es / (int64_t)sizeof(W);
    const int64_t cap = (int64_t)cu_count() * 32;
    if (wpr >= 64) {
      const int64_t want = (rows + 3) / 4;  // four waves per block
      const unsigned grid = (unsigned)(want < cap ? want : cap);
      hipLaunchKernelGGL((adv_index_rows_kernel<W>), dim3(grid), dim3(kBlock), 0, stream,
                         (W*)out->data, (const char*)self->data, a, rows, wpr, index_fault_word());
    } else {
      const int64_t want = (rows * wpr + kBlock - 1) / kBlock;
      const unsigned grid = (unsigned)(want < cap ? want : cap);
      hipLaunchKernelGGL((adv_index_words_kernel<W>), dim3(grid), dim3(kBlock), 0, stream,
                         (W*)out->data, (const char*)self->data, a, rows, wpr, index_fault_word());
    }
    return check_launch("index");
  };
  if (align % 16 == 0) return go(uint4{});
  if (align % 8 == 0) return go(uint2{});
  if (align % 4 == 0) return go(uint32_t{});
  if (align % 2 == 0) return go(uint16_t{});
  return go(uint8_t{});
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status_t mi_index(const mi_tensor_t* out, const mi_tensor_t* self,
                                const mi_tensor_t* const* indices, int32_t n_indices,
                                mi_stream_t stream) {
  clear_error();
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(self, "self"));
  return run_adv_index(out, self, indices, n_indices, (hipStream_t)stream);
}

extern "C" mi_status_t mi_index_select(const mi_tensor_t* out, const mi_tensor_t* self,
                                       int64_t dim, const mi_tensor_t* index,
                                       mi_stream_t stream) {
  clear_error();
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(self, "self"));
  MI_RETURN_IF(validate(index, "index"));
  MI_CHECK_ARG(index->ndim <= 1, "index_select(): Index is supposed to be a vector");
  MI_CHECK_ARG(index->dtype == MI_I64 || index->dtype == MI_I32,
               "index_select(): Expected dtype int32 or int64 for index");
  MI_CHECK_ARG(out->dtype == self->dtype, "index_select(): out dtype %s != self dtype %s",
               dtype_name(out->dtype), dtype_name(self->dtype));
  const int nd = self->ndim == 0 ? 1 : self->ndim;
  if (dim < 0) dim += nd;
  MI_CHECK_ARG(dim >= 0 && dim < nd, "index_select(): dim out of range");
  const int64_t n_idx = index->ndim == 1 ? index->sizes[0] : 1;
  if (self->ndim > 0) {
    MI_CHECK_ARG(out->ndim == self->ndim, "index_select(): out rank mismatch");
    for (int d = 0; d < self->ndim; ++d) {
      const int64_t want = d == dim ? n_idx : self->sizes[d];
      MI_CHECK_ARG(out->sizes[d] == want, "index_select(): out size %lld at dim %d, expected %lld",
                   (long long)out->sizes[d], d, (long long)want);
    }
  }
  if (numel(*out) == 0) return MI_OK;
  MI_CHECK_ARG(self->ndim == 0 || self->sizes[dim] > 0,
               "index_select(): cannot select from an empty dimension");
  if (index->dtype == MI_I64)
    return index_select_t<int64_t>(out, self, (int)dim, index, (hipStream_t)stream);
  return index_select_t<int32_t>(out, self, (int)dim, index, (hipStream_t)stream);
}
