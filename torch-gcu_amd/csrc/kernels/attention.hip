// Scaled dot-product attention forward (flash attention) on gfx950 MFMA.
//
// q [B, H, Sq, D], k/v [B, Hk, Sk, D] (Hk divides H: grouped-query heads
// share a k/v head), D = 64 or 128, bf16 or fp16; out like q; lse [B, H, Sq]
// fp32 = log(sum_j exp(scale * q.k_j)).  Causal masking is top-left aligned
// (key j is visible to query i when j <= i), as torch's is_causal.
//
// A 256-lane block owns 128 query rows (32 per wave) of one (b, h) and walks
// the keys in tiles of 64, with two LDS stages so the copies of tile i+1
// overlap the MFMAs of tile i (one barrier per tile):
//   1. K and V rows go to LDS as [key][d] by global_load_lds (no registers,
//      no LDS stores), each row's 16-byte chunks XOR-swizzled by key so the
//      fragment reads below are free of bank conflicts;
//   2. each wave computes the transposed scores S^T = K Q^T (32 keys x its 32
//      queries per MFMA tile, v_mfma_f32_32x32x16): Q stays in registers as
//      the B operand for the whole block, so lane l owns query l % 32 and
//      holds 32 of the tile's 64 keys for it (the other 32 are in lane
//      l ^ 32);
//   3. the online softmax is therefore per lane, in fp32, in the log2
//      domain: the row max needs one exchange between the two half-waves,
//      the running sum none until the end, and the rescale factor is a
//      per-lane scalar; the scale is folded into the exp2 argument (one
//      FMA per score);
//   4. P, rounded to the input type, is already laid out as the B operand of
//      O^T += V^T P^T (keys are fed to the MFMA's k dimension in a permuted
//      order that matches the S^T accumulator layout), so P never goes
//      through LDS; the V^T operand comes from V [key][d] by
//      ds_read_b64_tr_b16, which hands each lane one d for 4 consecutive
//      keys.
// Key tiles above a wave's causal diagonal are skipped.  Blocks are ordered
// head-major with the longest query tiles first, and renumbered so each of
// the 8 XCDs (which receive workgroups round robin) walks a contiguous run of
// heads: a head's K/V is then read into one XCD's L2 while its query tiles
// run there.
#include <cmath>

#include "iter.h"

namespace mi {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
struct AttnOp;
template <>
struct AttnOp<BF16> {
  typedef bf16x8 vec;
  typedef __bf16 elem;
  static __device__ __forceinline__ f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct AttnOp<F16> {
  typedef f16x8 vec;
  typedef _Float16 elem;
  static __device__ __forceinline__ f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
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
  int n_blocks;      // q_tiles * H * B
  int xcd_remap;     // n_blocks % 8 == 0: renumber blocks per XCD
};

constexpr int QT = 128;  // query rows per block
constexpr int KT = 64;   // keys per tile
constexpr int NT = 256;

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));

// LDS stage: K tile [KT keys][D] then V tile [KT keys][D], rows unpadded,
// both filled by global_load_lds (each lane's 16-byte chunk goes to LDS at
// lane * 16 of a 1 KiB wave copy, so the chunk order inside a row is chosen
// by which global chunk a lane fetches).  Chunk c of key row r sits at
// position c ^ swz(r):
//   K (read as 16-byte MFMA fragments, 16 rows per pass): swz_k spreads one
//     chunk of 16 consecutive rows over all 64 banks;
//   V (read by ds_read_b64_tr_b16, a pass covering 4 consecutive rows x 4
//     chunks): swz_v puts those 16 chunks on distinct banks.
template <int D>
struct FlashCfg {
  static constexpr int CPR = D / 8;     // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;  // rows per 1 KiB wave copy
  static constexpr int NINS = KT / RPI; // wave copies per K (or V) tile
  static constexpr int TILE = KT * D;   // elements of one K (or V) tile
  static constexpr int STAGE = 2 * TILE;
  static __device__ __forceinline__ int swz_k(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
  static __device__ __forceinline__ int swz_v(int r) { return D == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); }
  static_assert(NINS % 4 == 0, "four waves share a tile's copies");
};

template <typename T, int D>
__global__ __launch_bounds__(NT, 2) void flash_fwd_kernel(AttnArgs p) {
  typedef typename AttnOp<T>::vec vec;
  typedef FlashCfg<D> C;
  constexpr int DF = D / 16;  // k-steps of S^T = K Q^T
  constexpr int DT = D / 32;  // 32-row d tiles of O^T
  // two stages as separate arrays: with the loop unrolled by two, each
  // half-iteration reads one and copies into the other, so the compiler can
  // tell the next tile's copies from this tile's fragment reads (through one
  // array it made every transposed read wait for the copies in flight)
  __shared__ __align__(16) uint16_t stage0[C::STAGE];
  __shared__ __align__(16) uint16_t stage1[C::STAGE];

  // block -> (b, h, query tile); head-major, longest query tile first
  int bid = (int)blockIdx.x;
  if (p.xcd_remap) bid = (bid & 7) * (p.n_blocks >> 3) + (bid >> 3);
  const int qt = p.q_tiles - 1 - bid % p.q_tiles;
  const int bh = bid / p.q_tiles;
  const int64_t h = bh % p.H, b = bh / p.H;
  const int64_t hk = h * p.Hk / p.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, col = lane & 31;
  const int64_t q0 = (int64_t)qt * QT;
  const int64_t wq0 = q0 + wave * 32;  // this wave's first query row
  const int64_t qrow = wq0 + col;      // the query this lane owns

  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* V = p.v + b * p.v_sb + hk * p.v_sh;

  // B operand of S^T: lane supplies Q[qrow][16 t + 8 half + i], rows clamped
  vec qf[DF];
  {
    const int64_t r = min(qrow, p.Sq - 1);
#pragma unroll
    for (int t = 0; t < DF; ++t) qf[t] = *(const vec*)(Q + r * p.q_ss + 16 * t + 8 * half);
  }

  // ---- K / V: global -> LDS by wave copies (no registers, no ds_write) ----
  // Per-lane element offsets are 32-bit (the host checked Sk * stride fits);
  // keys past the end of the last tile re-read the last key (masked later).
  const int k_ss = (int)p.k_ss, v_ss = (int)p.v_ss, Sk = (int)p.Sk;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  // A full tile's copies are a tile base (scalar) plus these per-lane byte
  // offsets of key row `key` of the tile, fixed for the whole loop: no
  // per-tile address arithmetic on the VALU, which the softmax saturates
  // (the clamped form cost 33 VALU per tile, 8 of them quarter-rate
  // multiplies).  Only a last tile that runs past Sk clamps per lane.
  uint32_t kob[C::NINS / 4], vob[C::NINS / 4];
#pragma unroll
  for (int i = 0; i < C::NINS / 4; ++i) {
    const int q = wv * (C::NINS / 4) + i;
    const int key = q * C::RPI + lane / C::CPR, cp = lane % C::CPR;
    kob[i] = (uint32_t)(((int64_t)key * k_ss + 8 * (cp ^ C::swz_k(key))) * 2);
    vob[i] = (uint32_t)(((int64_t)key * v_ss + 8 * (cp ^ C::swz_v(key))) * 2);
  }
  auto issue_kv = [&](int kv0, uint16_t* ks) __attribute__((always_inline)) {
    uint16_t* vs = ks + C::TILE;
    if (kv0 + KT <= Sk) {
      const char* kb = (const char*)(K + (int64_t)kv0 * k_ss);
      const char* vb = (const char*)(V + (int64_t)kv0 * v_ss);
#pragma unroll
      for (int i = 0; i < C::NINS / 4; ++i) {
        const int q = wv * (C::NINS / 4) + i;
        // the offsets enter each copy as 32-bit registers (hoisted out of the
        // loop as 64-bit values they cost a 64-bit add per copy); the copy
        // then takes the scalar base + 32-bit offset form
        uint32_t ko = kob[i], vo = vob[i];
        asm volatile("" : "+v"(ko), "+v"(vo));
        __builtin_amdgcn_global_load_lds((const void*)(kb + ko), (lds_void_t*)(ks + q * 512), 16, 0,
                                         0);
        __builtin_amdgcn_global_load_lds((const void*)(vb + vo), (lds_void_t*)(vs + q * 512), 16, 0,
                                         0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < C::NINS / 4; ++i) {
        const int q = wv * (C::NINS / 4) + i;
        const int key = q * C::RPI + lane / C::CPR, cp = lane % C::CPR;
        const int gk = min(kv0 + key, Sk - 1);
        __builtin_amdgcn_global_load_lds((const void*)(K + gk * k_ss + 8 * (cp ^ C::swz_k(key))),
                                         (lds_void_t*)(ks + q * 512), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(V + gk * v_ss + 8 * (cp ^ C::swz_v(key))),
                                         (lds_void_t*)(vs + q * 512), 16, 0, 0);
      }
    }
  };
  // K fragment k-step t of sub-tile st: key 32 st + col, chunk 2 t + half
  // (swz_k(32 + col) == swz_k(col))
  int koff[DF];
  {
    const int sk = C::swz_k(col);
#pragma unroll
    for (int t = 0; t < DF; ++t) koff[t] = col * D + 8 * ((2 * t + half) ^ sk);
  }
  // V^T fragment (k-step t, d tile dt) by two transposed reads: in each 16-lane
  // group G, lane j names row key 16 t + 4 (G / 2) + j / 4 (then + 8), columns
  // d0 = 32 dt + 16 (G % 2) + 4 (j % 4) .. + 3, and receives d = 32 dt +
  // 16 (G % 2) + j for 4 consecutive keys: the A operand of O^T += V^T P^T
  // for keys 16 t + 4 half + 0..3 and 16 t + 8 + 4 half + 0..3
  int voff[DT];
  {
    const int G = lane >> 4, j = lane & 15;
    const int key = 4 * (G >> 1) + (j >> 2);  // plus 16 t
    const int sv = C::swz_v(key) >> 2;        // swz_v(key + 16 t) == swz_v(key)
    const int low = 2 * (G & 1) + ((j & 3) >> 1), within = 4 * (j & 1);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) voff[dt] = key * D + 8 * (4 * (dt ^ sv) + low) + within;
  }

  f32x16 o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  const int kv_end = (int)(p.causal ? min(p.Sk, q0 + QT) : p.Sk);
  const int n_tiles = (kv_end + KT - 1) / KT;
  const int wq = (int)wq0, qr = (int)qrow;
  issue_kv(0, stage0);
  // the Q fragments and the first tile have landed: inside the loop the only
  // outstanding global loads are the next tile's K / V copies
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  auto tile = [&](int it, const uint16_t* ks, uint16_t* next) __attribute__((always_inline)) {
    const int kv0 = it * KT;
    const bool more = it + 1 < n_tiles;
    if (more) issue_kv(kv0 + KT, next);
    __builtin_amdgcn_sched_barrier(0);
    const uint16_t* vs = ks + C::TILE;
    if (!p.causal || kv0 <= wq + 31) {
      // ---- S^T = K Q^T: two 32-key tiles x this wave's 32 queries, the two
      // accumulator chains interleaved ----
      f32x16 s[2] = {f32x16{}, f32x16{}};
      const uint16_t* kb1 = ks + 32 * D;
      // K fragments double-buffered one k-step ahead of their MFMAs
      vec kf[2][2];
      kf[0][0] = *(const vec*)(ks + koff[0]);
      kf[0][1] = *(const vec*)(kb1 + koff[0]);
#pragma unroll
      for (int t = 0; t < DF; ++t) {
        if (t + 1 < DF) {
          kf[(t + 1) & 1][0] = *(const vec*)(ks + koff[t + 1]);
          kf[(t + 1) & 1][1] = *(const vec*)(kb1 + koff[t + 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
        s[0] = AttnOp<T>::mma(kf[t & 1][0], qf[t], s[0]);
        s[1] = AttnOp<T>::mma(kf[t & 1][1], qf[t], s[1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      // ---- mask, online softmax in the log2 domain ----
      // accumulator r of tile st holds key kv0 + 32 st + 8 (r / 4) + 4 half + r % 4.
      // The max is taken over the raw scores times the sign of the scale (a
      // free source negation) and the scale is folded into the exponent:
      // p = exp2(s * scale_log2 - m_run).  Dead keys get the raw score whose
      // scaled value is -inf.
      const bool neg = p.scale_log2 < 0.f;
      float mx = -INFINITY;
      if ((kv0 + KT > Sk) || (p.causal && kv0 + KT - 1 > wq)) {
        const float dead_s = neg ? INFINITY : -INFINITY;
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kv0 + 32 * st + 8 * (r >> 2) + 4 * half + (r & 3);
            const bool dead = key >= Sk || (p.causal && key > qr);
            const float x = dead ? dead_s : s[st][r];
            s[st][r] = x;
            mx = fmaxf(mx, neg ? -x : x);
          }
      } else if (!neg) {
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[st][r]);
      } else {
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, -s[st][r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * fabsf(p.scale_log2);
      // m_run is the exact running row max (scaled, log2 units); O and l are
      // rescaled whenever it grows.  P is rounded to the input type, and the
      // key at the running max gets p = 1 exactly: with a stale max (rescaled
      // only when a row max grew by more than 2^8) that dominant weight
      // carried the rounding too, and on keys whose scores ramp up along a
      // 1024-key sequence the output was 1.5x further from the float64
      // result than CPU ATen's (one element past the bf16 bar).
      float corr = 1.0f;
      if (mx > m_run) {
        corr = __builtin_amdgcn_exp2f(m_run - mx);  // 0 when nothing was visible yet
        m_run = mx;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;  // nothing visible yet
      const float sc = p.scale_log2;
      // P as the B operand of O^T += V^T P^T: k-step t (16 keys) takes
      // accumulators 8 (t % 2) .. 8 (t % 2) + 7 of tile t / 2
      vec pk[KT / 16];
      float rs = 0.f;
#pragma unroll
      for (int t = 0; t < KT / 16; ++t) {
        f32x8 pf;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pf[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t >> 1][8 * (t & 1) + i], sc, -m_use));
          rs += pf[i];
        }
        pk[t] = __builtin_convertvector(pf, vec);
      }
      l_run = l_run * corr + rs;
      if (__ballot(corr != 1.0f)) {
#pragma unroll
        for (int d = 0; d < DT; ++d) o[d] *= corr;
      }
      // ---- O^T += V^T P^T: the lane reads V^T[d][key] for the same keys:
      // 16 t + 4 half + 0..3 and 16 t + 8 + 4 half + 0..3; a k-step's DT
      // fragments are read before its MFMAs ----
      vec vf[2][DT];
      auto read_v = [&](int t, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
          const uint16_t* vb = vs + 16 * t * D + voff[d];
          const s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)vb);
          const s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + 8 * D));
          const s16x4 lo = a0, hi = a1;
          vf[buf][d] = __builtin_bit_cast(vec, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      };
      read_v(0, 0);
#pragma unroll
      for (int t = 0; t < KT / 16; ++t) {
        if (t + 1 < KT / 16) read_v(t + 1, (t + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < DT; ++d) o[d] = AttnOp<T>::mma(vf[t & 1][d], pk[t], o[d]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // this wave's copies of the next tile have landed; the barrier publishes
    // every wave's and retires this tile's stage for the copy after next
    if (more) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  for (int it = 0; it < n_tiles; it += 2) {
    tile(it, stage0, stage1);
    if (it + 1 < n_tiles) tile(it + 1, stage1, stage0);
  }

  // ---- normalise and store: accumulator r of d tile dt is
  // O[qrow][32 dt + 8 (r / 4) + 4 half + r % 4] ----
  const float l = l_run + __shfl_xor(l_run, 32, 64);
  if (qrow < p.Sq) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    uint16_t* O = p.o + b * p.o_sb + h * p.o_sh + qrow * p.o_ss;
#pragma unroll
    for (int d = 0; d < DT; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef typename AttnOp<T>::elem E;
        typedef E e4 __attribute__((ext_vector_type(4)));
        typedef float f4 __attribute__((ext_vector_type(4)));
        f4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = o[d][4 * g + i] * inv;
        *(e4*)(O + d * 32 + 8 * g + 4 * half) = __builtin_convertvector(v, e4);
      }
    }
    if (half == 0 && p.lse)
      p.lse[b * p.lse_sb + h * p.lse_sh + qrow] =
          l > 0.f ? (m_run + __builtin_amdgcn_logf(l)) * 0.6931471805599453f : INFINITY;
  }
}

template <typename T, int D>
mi_status_t launch_flash(const AttnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((flash_fwd_kernel<T, D>), dim3((unsigned)a.n_blocks), dim3(NT), 0, s, a);
  return check_launch("flash_attention_fwd");
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
  MI_CHECK_ARG(Sk * k->strides[2] + D < 0x7fffffffLL && Sk * v->strides[2] + D < 0x7fffffffLL &&
                   Sq + QT < 0x7fffffffLL,
               "attention: a (batch, head) of k or v spans more than 2^31 elements");
  a.scale_log2 = (float)(scale * 1.4426950408889634);
  a.causal = is_causal ? 1 : 0;
  a.q_tiles = (int)((Sq + QT - 1) / QT);
  const int64_t nb = (int64_t)a.q_tiles * H * B;
  MI_CHECK_ARG(nb <= 0x7fffffff, "attention: too many query tiles");
  a.n_blocks = (int)nb;
  a.xcd_remap = (nb % 8 == 0) ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  if (q->dtype == MI_BF16)
    return D == 128 ? launch_flash<BF16, 128>(a, s) : launch_flash<BF16, 64>(a, s);
  return D == 128 ? launch_flash<F16, 128>(a, s) : launch_flash<F16, 64>(a, s);
}
