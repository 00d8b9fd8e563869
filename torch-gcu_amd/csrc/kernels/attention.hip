// Scaled dot-product attention forward (flash attention) on gfx950 MFMA.
//
// q [B, H, Sq, D], k/v [B, Hk, Sk, D] (Hk divides H: grouped-query heads
// share a k/v head), D = 64 or 128, bf16 or fp16; out like q; lse [B, H, Sq]
// fp32 = log(sum_j exp(scale * q.k_j)).  Causal masking is top-left aligned
// (key j is visible to query i when j <= i), as torch's is_causal.
//
// A 256-lane block owns 128 query rows (32 per wave) of one (b, h) and walks
// the keys in tiles of 64:
//   1. the tile's K rows go to LDS as [key][d] and its V rows as [d][key]
//      (transposed on the way in, so both MFMA operands are read as 16-byte
//      runs);
//   2. S = Q K^T with Q held in registers as MFMA A operands for the whole
//      block (D/16 fragments per lane), 2 x (D/16) v_mfma_f32_32x32x16;
//   3. online softmax in fp32 in the log2 domain: each lane holds 16 rows of
//      one key column, row maxima and sums are reduced across the 32 lanes of
//      its half-wave with xor shuffles, the running O rows are rescaled;
//   4. P is rounded to the input type and passed through a per-wave LDS tile
//      to become the A operand of O += P V (4 x (D/32) MFMAs).
// Key tiles entirely above the causal diagonal are never visited, and the
// query tiles are issued longest-first so the causal triangle balances.
#include <cmath>

#include "iter.h"

namespace mi {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
struct AttnOp;
template <>
struct AttnOp<BF16> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t cvt(float v) { return f32_to_bf16(v); }
};
template <>
struct AttnOp<F16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t cvt(float v) { return f32_to_f16(v); }
};

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t H, Hk, Sq, Sk;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t lse_sb, lse_sh;
  float scale_log2;  // softmax scale * log2(e)
  int causal;
  int q_tiles;
};

constexpr int QT = 128;  // query rows per block
constexpr int KT = 64;   // keys per tile
constexpr int NT = 256;

template <typename T, int D>
__global__ __launch_bounds__(NT, 2) void flash_fwd_kernel(AttnArgs p) {
  typedef typename AttnOp<T>::vec vec;
  constexpr int KP = D + 8;   // K tile pitch ([key][d])
  constexpr int VP = KT + 8;  // V^T tile pitch ([d][key])
  constexpr int PP = KT + 8;  // P tile pitch ([row][key])
  constexpr int DF = D / 16;  // k-steps of S = Q K^T
  constexpr int DT = D / 32;  // 32-column output tiles of O
  __shared__ __align__(16) uint16_t Ks[KT * KP];
  __shared__ __align__(16) uint16_t Vt[D * VP];
  __shared__ __align__(16) uint16_t Ps[4][32 * PP];

  const int qt = p.q_tiles - 1 - (int)blockIdx.x;  // longest rows first
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t hk = h * p.Hk / p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, col = lane & 31;
  const int64_t q0 = (int64_t)qt * QT;
  const int64_t wq0 = q0 + wave * 32;  // this wave's first query row

  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* V = p.v + b * p.v_sb + hk * p.v_sh;

  // Q fragments: lane holds Q[wq0 + col][16 t + 8 half .. +8], rows clamped
  vec qf[DF];
  {
    const int64_t r = min(wq0 + col, p.Sq - 1);
#pragma unroll
    for (int t = 0; t < DF; ++t) qf[t] = *(const vec*)(Q + r * p.q_ss + 16 * t + 8 * half);
  }

  f32x16 o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x16{};
  float m_run[16], l_run[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
  }

  const int64_t kv_end = p.causal ? min(p.Sk, q0 + QT) : p.Sk;
  for (int64_t kv0 = 0; kv0 < kv_end; kv0 += KT) {
    // ---- stage K as [key][d] and V as [d][key] ----
#pragma unroll
    for (int i = 0; i < KT * D / 8 / NT; ++i) {
      const int v = threadIdx.x + i * NT;
      const int key = v / (D / 8), dc = (v % (D / 8)) * 8;
      const int64_t gk = min(kv0 + key, p.Sk - 1);
      *(uint4*)(Ks + key * KP + dc) = *(const uint4*)(K + gk * p.k_ss + dc);
      union {
        uint4 u;
        uint16_t h[8];
      } vv;
      vv.u = *(const uint4*)(V + gk * p.v_ss + dc);
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[(dc + e) * VP + key] = vv.h[e];
    }
    __syncthreads();

    // ---- S = Q K^T for this wave's 32 rows x 64 keys ----
    f32x16 s[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      s[nt] = f32x16{};
      const uint16_t* kb = Ks + (nt * 32 + col) * KP + 8 * half;
#pragma unroll
      for (int t = 0; t < DF; ++t) s[nt] = AttnOp<T>::mma(qf[t], *(const vec*)(kb + 16 * t), s[nt]);
    }

    // ---- masking, online softmax (log2 domain) ----
    const bool need_mask = (kv0 + KT > p.Sk) || (p.causal && kv0 + KT - 1 > wq0);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = wq0 + 8 * (r >> 2) + 4 * half + (r & 3);
      float x0 = s[0][r] * p.scale_log2, x1 = s[1][r] * p.scale_log2;
      if (need_mask) {
        const int64_t k0 = kv0 + col, k1 = kv0 + 32 + col;
        if (k0 >= p.Sk || (p.causal && k0 > row)) x0 = -INFINITY;
        if (k1 >= p.Sk || (p.causal && k1 > row)) x1 = -INFINITY;
      }
      float mx = fmaxf(x0, x1);
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float m_new = fmaxf(m_run[r], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;  // fully masked so far
      const float p0 = __builtin_amdgcn_exp2f(x0 - m_use);
      const float p1 = __builtin_amdgcn_exp2f(x1 - m_use);
      float rs = p0 + p1;
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) rs += __shfl_xor(rs, off, 64);
      const float corr = __builtin_amdgcn_exp2f(m_run[r] - m_use);
      l_run[r] = l_run[r] * corr + rs;
      m_run[r] = m_new;
#pragma unroll
      for (int d = 0; d < DT; ++d) o[d][r] *= corr;
      const int rl = 8 * (r >> 2) + 4 * half + (r & 3);
      Ps[wave][rl * PP + col] = AttnOp<T>::cvt(p0);
      Ps[wave][rl * PP + 32 + col] = AttnOp<T>::cvt(p1);
    }
    __syncthreads();

    // ---- O += P V ----
#pragma unroll
    for (int t = 0; t < KT / 16; ++t) {
      const vec pa = *(const vec*)(&Ps[wave][col * PP + 16 * t + 8 * half]);
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const vec vb = *(const vec*)(Vt + (d * 32 + col) * VP + 16 * t + 8 * half);
        o[d] = AttnOp<T>::mma(pa, vb, o[d]);
      }
    }
    __syncthreads();
  }

  // ---- normalise and store ----
  uint16_t* O = p.o + b * p.o_sb + h * p.o_sh;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = wq0 + 8 * (r >> 2) + 4 * half + (r & 3);
    if (row >= p.Sq) continue;
    const float inv = l_run[r] > 0.f ? 1.0f / l_run[r] : 0.f;
#pragma unroll
    for (int d = 0; d < DT; ++d) O[row * p.o_ss + d * 32 + col] = AttnOp<T>::cvt(o[d][r] * inv);
    if (col == 0 && p.lse) {
      const float lse = l_run[r] > 0.f ? (m_run[r] + __builtin_amdgcn_logf(l_run[r])) * 0.6931471805599453f
                                        : INFINITY;
      p.lse[b * p.lse_sb + h * p.lse_sh + row] = lse;
    }
  }
}

mi_status_t check4(const mi_tensor_t* t, const char* name) {
  MI_RETURN_IF(validate(t, name));
  MI_CHECK_ARG(t->ndim == 4, "attention: %s must be [batch, heads, seq, head_dim]", name);
  MI_CHECK_ARG(t->strides[3] == 1, "attention: %s head_dim must be contiguous", name);
  MI_CHECK_ARG(((uintptr_t)t->data % 16) == 0 && t->strides[2] % 8 == 0 && t->strides[1] % 8 == 0 &&
                   t->strides[0] % 8 == 0,
               "attention: %s rows must be 16-byte aligned", name);
  return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status_t mi_flash_attention_fwd(const mi_tensor_t* out, const mi_tensor_t* lse,
                                              const mi_tensor_t* q, const mi_tensor_t* k,
                                              const mi_tensor_t* v, int32_t is_causal,
                                              double scale, mi_stream_t stream) {
  clear_error();
  MI_RETURN_IF(check4(q, "q"));
  MI_RETURN_IF(check4(k, "k"));
  MI_RETURN_IF(check4(v, "v"));
  MI_RETURN_IF(check4(out, "out"));
  const int64_t B = q->sizes[0], H = q->sizes[1], Sq = q->sizes[2], D = q->sizes[3];
  const int64_t Hk = k->sizes[1], Sk = k->sizes[2];
  MI_CHECK_ARG(q->dtype == k->dtype && q->dtype == v->dtype && out->dtype == q->dtype,
               "attention: q, k, v and out must share a dtype");
  MI_CHECK_ARG(q->dtype == MI_BF16 || q->dtype == MI_F16, "attention: dtype %s unsupported",
               dtype_name(q->dtype));
  MI_CHECK_ARG(D == 64 || D == 128, "attention: head_dim %lld unsupported (64 or 128)",
               (long long)D);
  MI_CHECK_ARG(k->sizes[0] == B && v->sizes[0] == B && v->sizes[1] == Hk && v->sizes[2] == Sk &&
                   k->sizes[3] == D && v->sizes[3] == D,
               "attention: k/v shapes do not match q");
  MI_CHECK_ARG(Hk > 0 && H % Hk == 0, "attention: %lld query heads are not a multiple of %lld kv heads",
               (long long)H, (long long)Hk);
  for (int d = 0; d < 4; ++d)
    MI_CHECK_ARG(out->sizes[d] == q->sizes[d], "attention: out shape mismatch");
  AttnArgs a{};
  a.q = (const uint16_t*)q->data;
  a.k = (const uint16_t*)k->data;
  a.v = (const uint16_t*)v->data;
  a.o = (uint16_t*)out->data;
  a.lse = nullptr;
  if (lse != nullptr && lse->data != nullptr) {
    MI_RETURN_IF(validate(lse, "lse"));
    MI_CHECK_ARG(lse->dtype == MI_F32 && lse->ndim == 3 && lse->sizes[0] == B &&
                     lse->sizes[1] == H && lse->sizes[2] == Sq && lse->strides[2] == 1,
                 "attention: lse must be fp32 [batch, heads, seq] with unit seq stride");
    a.lse = (float*)lse->data;
    a.lse_sb = lse->strides[0];
    a.lse_sh = lse->strides[1];
  }
  if (B == 0 || H == 0 || Sq == 0) return MI_OK;
  MI_CHECK_ARG(Sk > 0, "attention: empty key sequence");
  a.H = H;
  a.Hk = Hk;
  a.Sq = Sq;
  a.Sk = Sk;
  a.q_sb = q->strides[0];
  a.q_sh = q->strides[1];
  a.q_ss = q->strides[2];
  a.k_sb = k->strides[0];
  a.k_sh = k->strides[1];
  a.k_ss = k->strides[2];
  a.v_sb = v->strides[0];
  a.v_sh = v->strides[1];
  a.v_ss = v->strides[2];
  a.o_sb = out->strides[0];
  a.o_sh = out->strides[1];
  a.o_ss = out->strides[2];
  a.scale_log2 = (float)(scale * 1.4426950408889634);
  a.causal = is_causal ? 1 : 0;
  a.q_tiles = (int)((Sq + QT - 1) / QT);
  MI_CHECK_ARG(H <= 65535 && B <= 65535, "attention: too many heads or batches");
  dim3 grid((unsigned)a.q_tiles, (unsigned)H, (unsigned)B);
  hipStream_t s = (hipStream_t)stream;
  if (q->dtype == MI_BF16) {
    if (D == 128) hipLaunchKernelGGL((flash_fwd_kernel<BF16, 128>), grid, dim3(NT), 0, s, a);
    else hipLaunchKernelGGL((flash_fwd_kernel<BF16, 64>), grid, dim3(NT), 0, s, a);
  } else {
    if (D == 128) hipLaunchKernelGGL((flash_fwd_kernel<F16, 128>), grid, dim3(NT), 0, s, a);
    else hipLaunchKernelGGL((flash_fwd_kernel<F16, 64>), grid, dim3(NT), 0, s, a);
  }
  return check_launch("flash_attention_fwd");
}
