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
  constexpr int DF = D / 16;   // k-steps of S^T = K Q^T
  constexpr int DT = D / 32;   // 32-row d tiles of O^T
  constexpr int PS = KT / 16;  // k-steps of O^T += V^T P^T
  // K and V each in a ring of two slots, as four arrays: the loop below is
  // unrolled by two so that every LDS access names its array, and the
  // compiler can tell the copies in flight from the fragment reads (through
  // one array it made every read wait for all copies)
  __shared__ __align__(16) uint16_t ks0[C::TILE];
  __shared__ __align__(16) uint16_t ks1[C::TILE];
  __shared__ __align__(16) uint16_t vs0[C::TILE];
  __shared__ __align__(16) uint16_t vs1[C::TILE];

  // block -> (b, h, query tile); head-major, longest query tile first
  int bid = (int)blockIdx.x;
  if (p.xcd_remap) bid = (bid & 7) * (p.n_blocks >> 3) + (bid >> 3);
  const int qt = p.q_tiles - 1 - bid % p.q_tiles;
  const int bh = bid / p.q_tiles;
  const int64_t h = bh % p.H, b = bh / p.H;
  const int64_t hk = h * p.Hk / p.H;
  // the wave index read as wave-uniform: the loop bounds and tile bases
  // that derive from it then stay in scalar registers
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int64_t q0 = (int64_t)qt * QT;
  const int64_t wq0 = q0 + wave * 32;  // this wave's first query row
  const int64_t qrow = wq0 + col;      // the query this lane owns
  // K and V bases are wave-uniform: pinned to scalar registers (the head
  // index's division would otherwise leave them in VGPRs, and every tile
  // copy would rebuild its scalar base from them)
  auto uniform = [](const uint16_t* ptr) __attribute__((always_inline)) {
    const uint64_t v = (uint64_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint16_t*)(((uint64_t)hi << 32) | lo);
  };
  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = uniform(p.k + b * p.k_sb + hk * p.k_sh);
  const uint16_t* V = uniform(p.v + b * p.v_sb + hk * p.v_sh);

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
  // per-tile address arithmetic on the VALU, which the softmax saturates.
  // Only a last tile that runs past Sk clamps per lane.
  // V's chunk swizzle depends only on the key's row within a wave copy, so
  // V's copies share one per-lane offset (the copy's first key goes into
  // the scalar base); K's depends on the copy too (one offset per copy).
  uint32_t kob[C::NINS / 4], vob1;
#pragma unroll
  for (int i = 0; i < C::NINS / 4; ++i) {
    const int q = wv * (C::NINS / 4) + i;
    const int key = q * C::RPI + lane / C::CPR, cp = lane % C::CPR;
    kob[i] = (uint32_t)(((int64_t)key * k_ss + 8 * (cp ^ C::swz_k(key))) * 2);
  }
  {
    const int r = lane / C::CPR, cp = lane % C::CPR;
    vob1 = (uint32_t)(((int64_t)r * v_ss + 8 * (cp ^ C::swz_v(r))) * 2);
  }
  auto copy_tile = [&](const uint16_t* G, int g_ss, bool is_v, int kv0,
                       uint16_t* dst) __attribute__((always_inline)) {
    if (kv0 + KT <= Sk) {
#pragma unroll
      for (int i = 0; i < C::NINS / 4; ++i) {
        const int q = wv * (C::NINS / 4) + i;
        // the copy takes the scalar base + 32-bit offset form
        const char* gb = (const char*)(G + (int64_t)(kv0 + (is_v ? q * C::RPI : 0)) * g_ss);
        lds_copy16(gb, is_v ? vob1 : kob[i], dst + q * 512);
      }
    } else {
      // (the lane id passes through an empty asm so that nothing of this
      // rare path is hoisted into registers held across the loop)
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int i = 0; i < C::NINS / 4; ++i) {
        const int q = wv * (C::NINS / 4) + i;
        const int key = q * C::RPI + ln / C::CPR, cp = ln % C::CPR;
        const int gk = min(kv0 + key, Sk - 1);
        const int sw = is_v ? C::swz_v(key) : C::swz_k(key);
        lds_copy16(G, (uint32_t)(gk * g_ss + 8 * (cp ^ sw)) * 2u, dst + q * 512);
      }
    }
  };
  auto copy_k = [&](int kv0, uint16_t* dst) __attribute__((always_inline)) {
    copy_tile(K, k_ss, false, kv0, dst);
  };
  auto copy_v = [&](int kv0, uint16_t* dst) __attribute__((always_inline)) {
    copy_tile(V, v_ss, true, kv0, dst);
  };
  // K fragment k-step t of sub-tile st: key 32 st + col, chunk 2 t + half
  // (swz_k(32 + col) == swz_k(col))
  // byte offset (col D + 8 ((2 t + half) ^ sk)) 2 = 2 col D + 16 (half ^ (sk & 1))
  // + 32 (t ^ (sk >> 1)); the three terms occupy disjoint bits, so it is
  // kbm ^ 32 t with kbm the t = 0 offset: one register, one XOR per read
  int kbm;
  {
    const int sk = C::swz_k(col);
    kbm = 2 * col * D + 16 * (half ^ (sk & 1)) + 32 * (sk >> 1);
  }
  // V^T fragment (k-step t, d tile dt) by two transposed reads: in each 16-lane
  // group G, lane j names row key 16 t + 4 (G / 2) + j / 4 (then + 8), columns
  // d0 = 32 dt + 16 (G % 2) + 4 (j % 4) .. + 3, and receives d = 32 dt +
  // 16 (G % 2) + j for 4 consecutive keys: the A operand of O^T += V^T P^T
  // for keys 16 t + 4 half + 0..3 and 16 t + 8 + 4 half + 0..3
  int vbm;
  {
    const int G = lane >> 4, j = lane & 15;
    const int key = 4 * (G >> 1) + (j >> 2);  // plus 16 t
    const int sv = C::swz_v(key) >> 2;        // swz_v(key + 16 t) == swz_v(key)
    const int low = 2 * (G & 1) + ((j & 3) >> 1), within = 4 * (j & 1);
    // bytes 2 key D + 64 (dt ^ sv) + 16 low + 2 within: disjoint bits again,
    // so vbm ^ 64 dt
    vbm = 2 * key * D + 64 * sv + 16 * low + 2 * within;
  }
  // Each read's offset is made by an asm XOR of the one base register: the
  // compiler then adds the array (a constant LDS address) in the read's
  // immediate offset instead of keeping array + offset for every array and
  // offset in registers across the loop (48 more VGPRs, and spills)
  auto xor_off = [](int base, int m) __attribute__((always_inline)) {
    int r;
    asm volatile("v_xor_b32 %0, %1, %2" : "=v"(r) : "i"(m), "v"(base));
    return r;
  };
  auto read_k = [&](const uint16_t* ks, int t, vec* kf) __attribute__((always_inline)) {
    const int ko = xor_off(kbm, 32 * t);
    kf[0] = *(const vec*)((const char*)ks + ko);
    kf[1] = *(const vec*)((const char*)(ks + 32 * D) + ko);
  };
  auto read_v = [&](const uint16_t* vs, int t, vec* vf, int d0, int d1) __attribute__((always_inline)) {
#pragma unroll
    for (int d = d0; d < d1; ++d) {
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const int vo = xor_off(vbm, 64 * d);
      const uint16_t* vb = (const uint16_t*)((const char*)(vs + 16 * t * D) + vo);
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)vb);
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + 8 * D));
      vf[d] = __builtin_bit_cast(vec, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };

  f32x16 o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x16{};
  // m_run: the exact running row max of the scaled scores (log2 units);
  // corr: the factor that takes O and l from the previous max to m_run
  float m_run = -INFINITY, l_run = 0.f, corr = 1.f;
  const float sc = p.scale_log2;
  const bool neg = sc < 0.f;

  const int kv_end = (int)(p.causal ? min(p.Sk, q0 + QT) : p.Sk);
  const int n_tiles = (kv_end + KT - 1) / KT;
  const int wq = (int)wq0, qr = (int)qrow;
  // the last key tile with a key this wave's queries see (tiles above the
  // diagonal are skipped; the wave still copies and meets the barriers)
  const int last = p.causal ? min(n_tiles - 1, (wq + 31) / KT) : n_tiles - 1;

  // S^T = K Q^T of one tile: two 32-key MFMA tiles x this wave's 32 queries.
  // VALU work of the previous tile is interleaved by the caller.
  // Scores: accumulator r of sub-tile st holds key kv0 + 32 st + 8 (r / 4) +
  // 4 half + r % 4.  Masked keys get the raw score whose scaled value is -inf.
  // A key is dead at or past min(Sk, qr + 1) (causal) or Sk; per element
  // the test compares a constant with one per-lane limit.  The lane id is
  // read afresh by an asm statement (mbcnt), so no per-lane value of this
  // rare path stays in a register across the loop.
  auto mask = [&](f32x16* s, int kv0) __attribute__((always_inline)) {
    if ((kv0 + KT > Sk) || (p.causal && kv0 + KT - 1 > wq)) {
      const float dead_s = neg ? INFINITY : -INFINITY;
      int ln;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
      const int key_end = p.causal ? min(Sk, wq + (ln & 31) + 1) : Sk;
      const int lim = key_end - kv0 - 4 * (ln >> 5);
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s[st][r] = 32 * st + 8 * (r >> 2) + (r & 3) >= lim ? dead_s : s[st][r];
    }
  };
  // max over sub-tile st's 16 scores (sign-adjusted: the scale's sign is a
  // free source negation, the scale itself is folded into the exponent)
  auto part_max = [&](const f32x16* s, int st, float mx) __attribute__((always_inline)) {
    if (!neg) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[st][r]);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, -s[st][r]);
    }
    return mx;
  };
  // the new running max: O and l are rescaled whenever it grows, so the key
  // at the max gets p = 1 exactly (with a stale max that dominant weight
  // carried the rounding to the input type too, and keys whose scores ramp
  // up along a 1024-key sequence missed the bf16 bar)
  auto update_max = [&](float mx) __attribute__((always_inline)) {
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * fabsf(sc);
    corr = 1.f;
    if (mx > m_run) {
      corr = __builtin_amdgcn_exp2f(m_run - mx);  // 0 when nothing was visible yet
      m_run = mx;
    }
  };
  // P as the B operand of O^T += V^T P^T: k-step t (16 keys) takes
  // accumulators 8 (t % 2) .. 8 (t % 2) + 7 of sub-tile t / 2.  Score e
  // (0..31) of the tile is accumulator e % 16 of sub-tile e / 16; p is
  // computed in place and rounded to the input type per k-step.
  vec pk[PS];
  float rs = 0.f, m_use = 0.f;
  auto exp_range = [&](f32x16* s, int e0, int e1) __attribute__((always_inline)) {
#pragma unroll
    for (int e = e0; e < e1; ++e) {
      const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e >> 4][e & 15], sc, -m_use));
      s[e >> 4][e & 15] = x;
      rs += x;
      if ((e & 7) == 7) {
        f32x8 pf;
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[i] = s[e >> 4][(e & 8) + i];
        pk[e >> 3] = __builtin_convertvector(pf, vec);
      }
    }
  };
  auto rescale_range = [&](int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
    for (int i = i0; i < i1; ++i) o[i >> 4][i & 15] *= corr;
  };

  // one key tile j, software-pipelined: its scores sc_ (masked, their max
  // already in m_run) are turned into P while the MFMAs compute the next
  // tile's scores into sn (NXT: the wave sees a key of tile j + 1), and its
  // V^T P^T MFMAs run while the next tile's max is taken.  kr / vr: the
  // slots holding K(j + 1) and V(j); kw / vw: the slots that receive
  // K(j + 2) and V(j + 1).
  constexpr int RPG = DT * 16 / DF;  // O rescales per S^T k-step
  constexpr int EPG = 16 / DF;       // exponentials per S^T k-step (first half of P)
  auto sync_and_copy = [&](int j, uint16_t* kw, uint16_t* vw) __attribute__((always_inline)) {
    // this wave's copies of K(j + 1) and V(j) have landed; the barrier
    // publishes every wave's and tells that all are done with K(j) and V(j - 1)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (j + 2 < n_tiles) copy_k((j + 2) * KT, kw);
    if (j + 1 < n_tiles) copy_v((j + 1) * KT, vw);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto iter = [&](auto nxt_c, int j, const uint16_t* kr, const uint16_t* vr, uint16_t* kw,
                  uint16_t* vw, f32x16* sc_, f32x16* sn) __attribute__((always_inline)) {
    constexpr bool NXT = decltype(nxt_c)::value;
    sync_and_copy(j, kw, vw);
    m_use = m_run == -INFINITY ? 0.f : m_run;  // nothing visible yet
    l_run *= corr;
    rs = 0.f;
    // each group: its fragment reads, then VALU work that does not need
    // them (covering part of the LDS latency), then its MFMAs
    vec kf[2][2], vf[DT];
    // ---- phase 1: S^T(j + 1) on the MFMAs; O *= corr and the first half of P(j);
    // K fragments read one k-step ahead of their MFMAs ----
    if constexpr (NXT) {
      sn[0] = f32x16{};
      sn[1] = f32x16{};
      read_k(kr, 0, kf[0]);
#pragma unroll
      for (int t = 0; t < DF; ++t) {
        if (t + 1 < DF) read_k(kr, t + 1, kf[(t + 1) & 1]);
        rescale_range(t * RPG, (t + 1) * RPG);
        exp_range(sc_, t * EPG, (t + 1) * EPG);
        sn[0] = AttnOp<T>::mma(kf[t & 1][0], qf[t], sn[0]);
        sn[1] = AttnOp<T>::mma(kf[t & 1][1], qf[t], sn[1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      rescale_range(0, DT * 16);
      exp_range(sc_, 0, 16);
      __builtin_amdgcn_sched_barrier(0);
    }
    // ---- phase 2: O^T += V^T P^T(j) on the MFMAs; the second half of P(j),
    // then the mask and max of S(j + 1) ----
    // V^T fragments of k-step t + 1 are read as soon as the MFMAs of step t
    // that use the same registers are issued (d tiles 0, 1, then 2, 3)
    float mx = -INFINITY;
    read_v(vr, 0, vf, 0, DT);
#pragma unroll
    for (int t = 0; t < PS; ++t) {
      if (t == 0) exp_range(sc_, 16, 24);
      if (t == 1) {
        exp_range(sc_, 24, 32);
        l_run += rs;
      }
      if constexpr (NXT) {
        if (t == 2) {
          mask(sn, (j + 1) * KT);
          mx = part_max(sn, 0, mx);
        }
        if (t == 3) {
          mx = part_max(sn, 1, mx);
          update_max(mx);
        }
      }
#pragma unroll
      for (int d = 0; d < DT / 2; ++d) o[d] = AttnOp<T>::mma(vf[d], pk[t], o[d]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < PS) read_v(vr, t + 1, vf, 0, DT / 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int d = DT / 2; d < DT; ++d) o[d] = AttnOp<T>::mma(vf[d], pk[t], o[d]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < PS) read_v(vr, t + 1, vf, DT / 2, DT);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  typedef std::integral_constant<bool, true> Yes;
  typedef std::integral_constant<bool, false> No;

  // prologue: K(0), V(0) landed, K(1) in flight; S(0) and its max (every
  // wave sees key 0)
  copy_k(0, ks0);
  copy_v(0, vs0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (n_tiles > 1) copy_k(KT, ks1);
  f32x16 sa[2] = {f32x16{}, f32x16{}}, sb[2];
  {
    vec kf[2];
#pragma unroll
    for (int t = 0; t < DF; ++t) {
      read_k(ks0, t, kf);
      sa[0] = AttnOp<T>::mma(kf[0], qf[t], sa[0]);
      sa[1] = AttnOp<T>::mma(kf[1], qf[t], sa[1]);
    }
    mask(sa, 0);
    update_max(part_max(sa, 1, part_max(sa, 0, -INFINITY)));
  }
  // tiles 0 .. last with compute (even tiles read K from slot 1 and V from
  // slot 0), then barriers and copies only up to the block's last tile
  int j = 0;
  for (; j + 1 < last; j += 2) {
    iter(Yes(), j, ks1, vs0, ks0, vs1, sa, sb);
    iter(Yes(), j + 1, ks0, vs1, ks1, vs0, sb, sa);
  }
  if (j < last) {
    iter(Yes(), j, ks1, vs0, ks0, vs1, sa, sb);
    iter(No(), j + 1, ks0, vs1, ks1, vs0, sb, sa);
    j += 2;
  } else {
    iter(No(), j, ks1, vs0, ks0, vs1, sa, sb);
    j += 1;
  }
  for (; j < n_tiles; ++j) sync_and_copy(j, (j & 1) ? ks1 : ks0, (j & 1) ? vs0 : vs1);

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
