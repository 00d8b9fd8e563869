// Dense contractions on gfx950 MFMA: addmm / mm / bmm / baddbmm and the int8
// weight-only linear.
//
// One kernel template, v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation:
//   - a block owns a BM x BN output tile and walks K in steps of 64;
//   - WM x WN waves each own a (BM/WM) x (BN/WN) sub-tile, i.e. a grid of
//     32 x 32 MFMA tiles (the 256 x 256 configuration gives every wave
//     16 tiles = 256 fp32 accumulators, which live in AGPRs);
//   - A rows and B rows (B is read as [N, K], K contiguous) are staged
//     through LDS with a 72-element row pitch (16 bytes of padding) so the
//     16-byte operand reads of 32 consecutive rows fall in distinct banks;
//     two LDS stages let the global loads of step k+1 overlap the MFMAs of
//     step k with one barrier per step;
//   - for the int8 weight-only linear, B tiles arrive as int8 (half the
//     bytes) and are widened to bf16 on the way into LDS (an int8 value is
//     exactly a bf16 whose low 16 fp32 bits are zero), and the epilogue
//     multiplies by the per-output-channel fp32 scale.
// MFMA operand layout (checked on the device): lane l supplies
//   A[m = l % 32][k = 8 * (l / 32) + i] and B[k = 8 * (l / 32) + i][n = l % 32],
//   i < 8, and receives D[m = 8 * (r / 4) + 4 * (l / 32) + r % 4][n = l % 32]
//   in accumulator r < 16.
// Workgroups are renumbered so that each of the 8 XCDs (which receive
// workgroups round robin) gets a contiguous run of tiles, walked in groups
// of 8 row panels, so tiles sharing A and B panels meet in one L2.
// fp32 inputs take a VALU tiled kernel.
#include <algorithm>

#include "iter.h"

namespace mi {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;
constexpr int PITCH = BK + 8;  // LDS row pitch in elements

template <typename T>
struct MfmaOp;
template <>
struct MfmaOp<BF16> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ float load(uint16_t v) { return bf16_to_f32(v); }
};
template <>
struct MfmaOp<F16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x16 mma(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_f16(v); }
  static __device__ __forceinline__ float load(uint16_t v) { return f16_to_f32(v); }
};

struct GemmArgs {
  const uint16_t* a;  // [batch][M][lda], K contiguous
  const void* b;      // [batch][N][ldb], K contiguous (16-bit or int8)
  uint16_t* c;        // [batch][M][ldc], N contiguous
  const void* bias;   // element (m, n) at bias + b*bias_sb + m*bias_sm + n*bias_sn
  const float* scale; // int8 path: per-N fp32 scale
  int bias_dtype;
  int64_t bias_sm, bias_sn, bias_sb;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sa, sb, sc;  // batch strides (elements)
  float alpha, beta;
  int tiles_m, tiles_n;
  // fused epilogues of the large-tile kernel (EPI_SILU, EPI_RESID below)
  const void* b2;       // EPI_SILU: the up weight, rows laid out like b's (the gate weight)
  const uint16_t* res;  // EPI_RESID: residual, element (m, n) at res[m * ldr + n]
  int64_t ldr;
};

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
  const int total = tiles_m * tiles_n;
  constexpr int XCD = 8;
  int id = bid;
  if (total % XCD == 0) {
    const int per = total / XCD;
    id = (bid % XCD) * per + bid / XCD;
  }
  constexpr int GROUP_M = 8;
  const int group = id / (GROUP_M * tiles_n);
  const int first_m = group * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int in_group = id - group * GROUP_M * tiles_n;
  *tm = first_m + in_group % gsize;
  *tn = in_group / gsize;
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 8 int8 (two words) -> 8 x bf16 / f16, exact. One sign-extending byte
// convert per value (v_cvt_f32_i32 with a byte select), then two values per
// word: the upper halves of the two floats for bf16 (exact, an int8 has at
// most 8 significant bits), a round-toward-zero pack for f16 (exact too).
// 12 VALU per 8 values; a (__bf16) cast of the float costs twice that.
template <typename T>
__device__ __forceinline__ typename MfmaOp<T>::vec widen8(u32x2_t w) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t d = w[p >> 1];
    const float lo = (float)(int)(int8_t)(d >> (16 * (p & 1)));
    const float hi = (float)(int)(int8_t)(d >> (16 * (p & 1) + 8));
    if constexpr (std::is_same<T, BF16>::value)
      r[p] = __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
    else
      r[p] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  }
  return __builtin_bit_cast(typename MfmaOp<T>::vec, r);
}


typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4_t __attribute__((ext_vector_type(4)));

// Four consecutive per-column values n .. n + 3 of a row vector (the int8
// scale, or a bias broadcast over rows) as floats: element k at
// base + off + k * stride, fp32 or of the output's 16-bit type T.  One
// vector load when all four columns exist, the stride is 1 and the address
// is aligned; else four loads with the column clamped to N - 1 (clamped
// columns only feed outputs that are never stored).
template <typename T>
__device__ __forceinline__ f32x4_t load_col4_t(const void* base, int dtype, int64_t n, int64_t stride,
                                               int64_t N, int64_t off) {
  f32x4_t r;
  if (dtype == MI_F32) {
    const float* b = (const float*)base + off;
    if (stride == 1 && n + 3 < N && (((uintptr_t)(b + n)) & 15) == 0) {
      r = *(const f32x4_t*)(b + n);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = b[min<int64_t>(n + e, N - 1) * stride];
    }
  } else {
    const uint16_t* b = (const uint16_t*)base + off;
    if (stride == 1 && n + 3 < N && (((uintptr_t)(b + n)) & 7) == 0) {
      const u16x4_t v = *(const u16x4_t*)(b + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = MfmaOp<T>::load(v[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = MfmaOp<T>::load(b[min<int64_t>(n + e, N - 1) * stride]);
    }
  }
  return r;
}

// Per-lane loader of a ROWS x 64 tile of a K-contiguous 16-bit matrix: V
// 16-byte vectors per lane, 8 lanes per 128-byte row segment; vector i of a
// lane covers tile row row0 + i * (NT / 8).  Rows past the end of the matrix
// are clamped to its last row: their products only reach output rows or
// columns that are never stored.  The last, partial K step (load_tail) reads
// the elements at k >= K as zero.  Addresses are formed at load time so that
// no per-vector pointer stays live across the main loop.
template <int ROWS, int NT>
struct Tile16 {
  static constexpr int V = ROWS * 8 / NT;
  static constexpr int RS = NT / 8;  // rows between a lane's vectors
  const uint16_t* base;
  int64_t ld, last, row0;
  int kc;
  uint4 r[V];
  __device__ __forceinline__ void init(const uint16_t* b, int64_t ld_, int64_t rows, int64_t r0) {
    base = b;
    ld = ld_;
    last = rows - 1;
    row0 = r0 + (threadIdx.x >> 3);
    kc = (threadIdx.x & 7) * 8;
  }
  __device__ __forceinline__ const uint16_t* at(int i, int64_t k0) const {
    const int64_t gr = min(row0 + (int64_t)i * RS, last);
    return base + gr * ld + kc + k0;
  }
  __device__ __forceinline__ void load_full(int64_t k0) {
#pragma unroll
    for (int i = 0; i < V; ++i) r[i] = *(const uint4*)at(i, k0);
  }
  __device__ __forceinline__ void load_tail(int64_t k0, int64_t K) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const uint16_t* q = at(i, k0);
      const int64_t gk = k0 + kc;
      union {
        uint4 u;
        uint16_t h[8];
      } t;
#pragma unroll
      for (int e = 0; e < 8; ++e) t.h[e] = (gk + e < K) ? q[e] : (uint16_t)0;
      r[i] = t.u;
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) const {
    uint16_t* d = lds + (threadIdx.x >> 3) * PITCH + kc;
#pragma unroll
    for (int i = 0; i < V; ++i) *(uint4*)(d + i * RS * PITCH) = r[i];
  }
};

// int8 rows: ROWS x 64 bytes = ROWS*4 vectors of 16 values per tile, widened
// to T (bf16 or f16, exact) when written to LDS (same clamping and tail rules).
template <typename T, int ROWS, int NT>
struct Tile8 {
  static constexpr int V = ROWS * 4 / NT;
  static constexpr int RS = NT / 4;
  const int8_t* base;
  int64_t ld, last, row0;
  int kc;
  uint4 r[V];
  __device__ __forceinline__ void init(const int8_t* b, int64_t ld_, int64_t rows, int64_t r0) {
    base = b;
    ld = ld_;
    last = rows - 1;
    row0 = r0 + (threadIdx.x >> 2);
    kc = (threadIdx.x & 3) * 16;
  }
  __device__ __forceinline__ const int8_t* at(int i, int64_t k0) const {
    const int64_t gr = min(row0 + (int64_t)i * RS, last);
    return base + gr * ld + kc + k0;
  }
  __device__ __forceinline__ void load_full(int64_t k0) {
#pragma unroll
    for (int i = 0; i < V; ++i) r[i] = *(const uint4*)at(i, k0);
  }
  __device__ __forceinline__ void load_tail(int64_t k0, int64_t K) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int8_t* q = at(i, k0);
      const int64_t gk = k0 + kc;
      union {
        uint4 u;
        int8_t b[16];
      } t;
#pragma unroll
      for (int e = 0; e < 16; ++e) t.b[e] = (gk + e < K) ? q[e] : (int8_t)0;
      r[i] = t.u;
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) const {
    uint16_t* d = lds + (threadIdx.x >> 2) * PITCH + kc;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      union {
        uint4 u;
        int8_t b[16];
      } in;
      in.u = r[i];
      typedef typename MfmaOp<T>::vec vec;
      *(vec*)(d + i * RS * PITCH) = widen8<T>(u32x2_t{in.u.x, in.u.y});
      *(vec*)(d + i * RS * PITCH + 8) = widen8<T>(u32x2_t{in.u.z, in.u.w});
    }
  }
};

template <typename T, int BM, int BN, int WM, int WN, bool B_INT8, bool HAS_BIAS>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_mfma_kernel(GemmArgs p) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;  // per-wave sub-tile
  constexpr int FM = TM / 32, FN = TN / 32;  // MFMA tiles per wave
  typedef typename MfmaOp<T>::vec vec;
  extern __shared__ __align__(16) uint16_t smem[];
  // stage s: A at smem + s*BM*PITCH, B at smem + 2*BM*PITCH + s*BN*PITCH
  auto As = [&](int s) { return smem + s * BM * PITCH; };
  auto Bs = [&](int s) { return smem + 2 * BM * PITCH + s * BN * PITCH; };

  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int64_t batch = blockIdx.y;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lrow = lane & 31, lk = (lane >> 5) * 8;

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

  Tile16<BM, NT> ta;
  typename std::conditional<B_INT8, Tile8<T, BN, NT>, Tile16<BN, NT>>::type tb;
  ta.init(p.a + batch * p.sa, p.lda, p.M, m0);
  if constexpr (B_INT8)
    tb.init((const int8_t*)p.b + batch * p.sb, p.ldb, p.N, n0);
  else
    tb.init((const uint16_t*)p.b + batch * p.sb, p.ldb, p.N, n0);

  // MFMAs over one LDS stage, operand fragments double-buffered across the
  // four 16-deep substeps.
  auto compute = [&](int st) {
    const uint16_t* a_s = As(st) + (wm * TM + lrow) * PITCH + lk;
    const uint16_t* b_s = Bs(st) + (wn * TN + lrow) * PITCH + lk;
    vec af[2][FM], bf[2][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[0][i] = *(const vec*)(a_s + i * 32 * PITCH);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[0][j] = *(const vec*)(b_s + j * 32 * PITCH);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int c = s & 1;
      if (s + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[c ^ 1][i] = *(const vec*)(a_s + i * 32 * PITCH + (s + 1) * 16);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bf[c ^ 1][j] = *(const vec*)(b_s + j * 32 * PITCH + (s + 1) * 16);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MfmaOp<T>::mma(af[c][i], bf[c][j], acc[i][j]);
    }
  };

  // Steps 0 .. KF-1 are full 64-deep steps, step KF (if K % 64) is partial.
  // The main loop only ever prefetches full steps, so it has no branch.
  const int KF = (int)(p.K / BK);
  const bool tail = KF * (int64_t)BK < p.K;
  if (KF > 0) {
    ta.load_full(0);
    tb.load_full(0);
  } else {
    ta.load_tail(0, p.K);
    tb.load_tail(0, p.K);
  }
  ta.store(As(0));
  tb.store(Bs(0));
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < KF; ++kt) {
    ta.load_full((int64_t)(kt + 1) * BK);
    tb.load_full((int64_t)(kt + 1) * BK);
    // keep the next step's global loads issued ahead of this step's MFMAs
    // (the scheduler would otherwise sink them next to their LDS stores and
    // expose their latency)
    __builtin_amdgcn_sched_barrier(0);
    compute(kt & 1);
    ta.store(As((kt + 1) & 1));
    tb.store(Bs((kt + 1) & 1));
    __syncthreads();
  }
  if (tail && KF > 0) {
    ta.load_tail((int64_t)KF * BK, p.K);
    tb.load_tail((int64_t)KF * BK, p.K);
    compute(kt & 1);
    ta.store(As((kt + 1) & 1));
    tb.store(Bs((kt + 1) & 1));
    __syncthreads();
    ++kt;
  }
  compute(kt & 1);

  // epilogue: out = alpha * acc (* scale[n]) + beta * bias, rounded once.  The
  // bias is fp32 or of the output's type (the host converts anything else).
  uint16_t* C = p.c + batch * p.sc;
  const bool bias_f32 = p.bias_dtype == MI_F32;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t n = n0 + wn * TN + j * 32 + lrow;
    if (n >= p.N) continue;
    const int64_t bcol = batch * p.bias_sb + n * p.bias_sn;
    const float colscale = B_INT8 ? p.alpha * p.scale[n] : p.alpha;
    // a bias broadcast over rows: one load per column
    const bool row_bias = HAS_BIAS && p.bias_sm == 0;
    float bcolv = 0.f;
    if (row_bias)
      bcolv = bias_f32 ? ((const float*)p.bias)[bcol] : MfmaOp<T>::load(((const uint16_t*)p.bias)[bcol]);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * TM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < p.M) {
          float v = colscale * acc[i][j][r];
          if (HAS_BIAS) {
            float bv = bcolv;
            if (!row_bias) {
              const int64_t bo = bcol + m * p.bias_sm;
              bv = bias_f32 ? ((const float*)p.bias)[bo] : MfmaOp<T>::load(((const uint16_t*)p.bias)[bo]);
            }
            v += p.beta * bv;
          }
          C[m * p.ldc + n] = MfmaOp<T>::store(v);
        }
      }
    }
  }
}

// ---- 16-bit operands, K % 64 == 0: direct-to-LDS pipeline --------------------------
//
// 256 x 256 output tile per 512-lane block (8 waves as 4 along M x 2 along N,
// each wave 64 x 128 = 2 x 4 MFMA tiles, so two waves share a SIMD and one
// issues MFMAs while the other waits).  K steps of 64 flow through a ring of
// two LDS stages that global_load_lds_dwordx4 fills straight from global
// memory (no VGPR staging, no ds_write): the end of step k refills the stage
// it just finished with step k + 2.  Rows are 128 B (8 chunks of 16 B) and
// chunk c of row r is stored at chunk c ^ (r & 7) ^ ((r >> 3) & 1), which
// keeps the 16-byte fragment reads of 16 consecutive rows on distinct banks
// (whether the LDS is banked 32 or 64 wide).  Each substep's fragment reads
// for the next substep, and at the step boundary the refill loads, are
// interleaved with the MFMAs.  The epilogue applies alpha / beta * bias,
// rounds once, stages each wave's 64 x 128 tile through LDS and stores whole
// 256-byte row segments.
namespace dl {
constexpr int BK = 64, STAGES = 2, WM = 4, WN = 2;
constexpr int NW = WM * WN, NT = 64 * NW;
constexpr int TM = 64, TN = 128, EP = TN + 8;          // wave tile, epilogue LDS pitch
constexpr int BM = WM * TM, BN = WN * TN;              // 256 x 256
constexpr int CH = BK / 8;                             // 16-byte chunks per row
constexpr int RPK = 512 / BK;                          // rows per 1 KiB wave load
constexpr int NQA = BM / RPK / NW, NQB = BN / RPK / NW;
constexpr int LPS = NQA + NQB;                         // wave loads per step
constexpr int TA = BM * BK, TB = BN * BK;
constexpr size_t LDS_BYTES =
    (size_t)STAGES * (TA + TB) * 2 > (size_t)NW * TM * EP * 2 ? (size_t)STAGES * (TA + TB) * 2
                                                                : (size_t)NW * TM * EP * 2;
constexpr int GROUP_M = 4;
// int8 B: 64-byte rows (4 chunks of 16 B), 16 rows per 1 KiB wave load
constexpr int CH8 = 4, RPK8 = 16, NQB8 = BN / RPK8 / NW, TB8 = BN * BK / 2;  // TB8 in 16-bit units
// int8 B adds a bf16 copy of each stage's W rows: 160 KiB in all
constexpr size_t LDS_BYTES8 = (size_t)STAGES * (TA + TB8) * 2 + (size_t)STAGES * TB * 2;
static_assert(LDS_BYTES8 <= 160 * 1024 && LDS_BYTES8 >= (size_t)NW * TM * EP * 2, "int8 LDS");
}  // namespace dl

typedef __attribute__((address_space(3))) void lds_void_t;
typedef uint16_t u16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  // s_waitcnt: vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] = 15 | vmcnt[5:4] at [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// waits until at most `later` steps' loads (LPW per step) are outstanding
template <int MAXL, int LPW>
__device__ __forceinline__ void wait_later(int later) {
  if constexpr (MAXL > 0) {
    if (later >= MAXL) {
      wait_vmcnt<MAXL * LPW>();
      return;
    }
    wait_later<MAXL - 1, LPW>(later);
  } else {
    wait_vmcnt<0>();
  }
}

// 128-byte rows (8 chunks of 16 B): chunk c of row r at c ^ f(r), with
// f(r) = (r & 3) ^ 5 (bit 2 of r) ^ 4 (bit 3 of r): bit 0 = r0 ^ r2, bit 1 =
// r1, bit 2 = r2 ^ r3.  Chosen by timing every linear map of the row's low 4
// bits to a chunk mask on this LDS (a 64-lane ds_read_b128 takes 4 cycles
// without conflicts, 5.5 with the 2-way ones): it reads without conflicts
// 16 x 16 x 32 fragments (row l % 16, chunk 4 s + l / 16), 32 x 32 x 16
// fragments (row l % 32, chunk 2 s + l / 32), and the int8 widening's
// patterns (2 lanes a row x 4 chunks, 4 lanes a row x 2 chunks).  The mask
// (r & 7) ^ (r >> 3 & 1) it replaces made every 16 x 16 x 32 fragment read
// two-way conflicted (SQ_LDS_BANK_CONFLICT half of the LDS-active cycles).
__device__ __forceinline__ int dl_swz(int r, int c) {
  return c ^ (r & 3) ^ (((r >> 2) & 1) * 5) ^ ((r >> 1) & 4);
}
// 64-byte rows: chunk c of row r at c ^ ((r >> 1) & 3) ^ ((r >> 3) & 1), conflict-free for
// 16-byte reads of 16 consecutive rows under 32- or 64-bank LDS
__device__ __forceinline__ int dl_swz64(int r, int c) { return c ^ (((r >> 1) & 3) ^ ((r >> 3) & 1)); }

// SPLIT: blockIdx.y is a K slice instead of a batch; the block multiplies
// its slice's whole 64-wide steps (slice s of S gets KT / S steps, one more
// for s < KT % S) and stores the raw fp32 sums to part[s][M][ldp] for
// splitk_combine_kernel (no scale, bias or rounding here).
// B_KN: B is a row-major [K][N] matrix (ldb = its row stride, N contiguous),
// read in place: a stage holds the step's 64 k rows of the tile's 256
// columns (512 B each, 16-byte chunk c of row k at c ^ 4 (k & 3)), and the
// B fragments are read transposed by ds_read_b64_tr_b16, which hands each
// lane one column for 4 consecutive k (two reads per 8-k fragment).  Per
// read, lanes 0..31 cover 4 rows x 128 bytes and land on 64 distinct banks.
// EPI: fused epilogues of two matmuls of a decoder layer, each reproducing
// the rounding of the unfused ops bit for bit:
//   EPI_RESID: out = residual + round(x W^T), as linear then add (the sum in
//     fp32, rounded once), the residual read in the coalesced store pass;
//   EPI_SILU:  out = silu(round(x Wg^T)) * round(x Wu^T), as two linears then
//     silu_mul: a 256-wide tile holds 128 gate columns (waves 0..3 copy their
//     B rows from Wg) and the same 128 up columns (waves 4..7 from Wu), the
//     waves of column half 0 stage gate, those of half 1 up, and after a
//     barrier each wave combines half of its row band's pairs.
constexpr int EPI_NONE = 0, EPI_RESID = 1, EPI_SILU = 2;

template <typename T, bool HAS_BIAS, bool B_INT8, bool SPLIT = false, bool B_KN = false,
          int EPI = EPI_NONE>
__global__ __launch_bounds__(dl::NT, 2) void gemm_dl_kernel(GemmArgs p, float* part, int64_t ldp) {
  static_assert(!B_KN || (!B_INT8 && !SPLIT), "row-major B: 16-bit, no split");
  static_assert(EPI == EPI_NONE || (!HAS_BIAS && !B_INT8 && !SPLIT && !B_KN),
                "fused epilogues: plain 16-bit K-contiguous matmul");
  static_assert(EPI != EPI_SILU || (dl::WN == 2 && dl::NQB * dl::RPK * dl::NW / 2 == dl::BN / 2),
                "gate rows come from waves 0..NW/2-1, up rows from the others");
  // MFMA shape: 16 x 16 x 32 (MD = 16) for K-contiguous operands, 32 x 32 x 16
  // for the transposed row-major B reads, whose lane layout is built for it
  constexpr bool M16 = !B_KN;
  constexpr int MD = M16 ? 16 : 32, KPM = 512 / MD;  // MFMA tile edge, k per MFMA
  constexpr int BK = dl::BK, STAGES = dl::STAGES, WN = dl::WN, TM = dl::TM, TN = dl::TN;
  constexpr int FM = TM / MD, FN = TN / MD, KS = BK / KPM;
  constexpr int BM = dl::BM, BN = dl::BN, CH = dl::CH, RPK = dl::RPK, NQA = dl::NQA,
                TA = dl::TA, EP = dl::EP, GROUP_M = dl::GROUP_M;
  // the B tile: 16-bit rows of 128 B, or int8 rows of 64 B (widened at fragment read)
  constexpr int NQB = B_INT8 ? dl::NQB8 : dl::NQB;
  constexpr int TB = B_INT8 ? dl::TB8 : dl::TB;
  constexpr int LPS = NQA + NQB;
  typedef typename MfmaOp<T>::vec vec;
  typedef typename std::conditional<M16, f32x4_t, f32x16>::type acc_t;
  auto mma = [](vec a, vec b, acc_t c) __attribute__((always_inline)) {
    if constexpr (!M16) return MfmaOp<T>::mma(a, b, c);
    else if constexpr (std::is_same<T, BF16>::value)
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  };
  extern __shared__ __align__(16) uint16_t smem[];
  // XCD-aware tile order (round-robin dispatch over 8 XCDs), then groups of
  // GROUP_M row panels so the tiles an XCD runs together share A and B panels
  int tm, tn;
  {
    const int total = p.tiles_m * p.tiles_n;
    int id = blockIdx.x;
    if (total % 8 == 0) {
      const int per = total / 8;
      id = (id % 8) * per + id / 8;
    }
    const int group = id / (GROUP_M * p.tiles_n);
    const int first_m = group * GROUP_M;
    const int gsize = min(p.tiles_m - first_m, GROUP_M);
    const int in_group = id - group * GROUP_M * p.tiles_n;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
  }
  const int64_t batch = SPLIT ? 0 : blockIdx.y;
  const int M = (int)p.M, N = (int)p.N, K = (int)p.K;
  const int m0 = tm * BM, n0 = tn * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int KT = K / BK, k_first = 0;
  if constexpr (SPLIT) {
    const int S = gridDim.y, sl = blockIdx.y, base = KT / S, rem = KT % S;
    k_first = sl * base + min(sl, rem);
    KT = base + (sl < rem ? 1 : 0);
  }
  const uint16_t* A = p.a + batch * p.sa + (int64_t)k_first * BK;
  // EPI_SILU: waves 0..NW/2-1 copy gate rows, the others up rows
  const void* bsrc = (EPI == EPI_SILU && wave >= dl::NW / 2) ? p.b2 : p.b;
  const char* Bbase = (const char*)bsrc + (batch * p.sb + (int64_t)k_first * BK * (B_KN ? p.ldb : 1)) *
                                              (B_INT8 ? 1 : 2);

  // per-lane byte offsets (the host checked they fit 32 bits); rows past the
  // matrix are clamped to its last row and only feed outputs never stored
  uint32_t ao[NQA], bo[NQB];
#pragma unroll
  for (int q = 0; q < NQA; ++q) {
    const int row = (wave * NQA + q) * RPK + lane / CH;
    ao[q] = (uint32_t)(((int64_t)min(m0 + row, M - 1) * p.lda + dl_swz(row, lane % CH) * 8) * 2);
  }
#pragma unroll
  for (int q = 0; q < NQB; ++q) {
    if constexpr (B_KN) {
      // wave copy q: k rows 2 (wave NQB + q) and the next, 32 chunks each;
      // columns past N re-read the last chunk (their outputs are not stored)
      const int row = 2 * (wave * NQB + q) + lane / 32, c = (lane & 31) ^ (4 * (row & 3));
      bo[q] = (uint32_t)(((int64_t)row * p.ldb + min(n0 + 8 * c, N - 8)) * 2);
    } else if constexpr (B_INT8) {
      const int row = (wave * NQB + q) * dl::RPK8 + lane / dl::CH8;
      bo[q] = (uint32_t)((int64_t)min(n0 + row, N - 1) * p.ldb + dl_swz64(row, lane % dl::CH8) * 16);
    } else {
      const int row = (wave * NQB + q) * RPK + lane / CH;
      // EPI_SILU: tile tn covers output columns 128 tn .. 128 tn + 127 (rows
      // 0..127 of the tile from the gate weight, 128..255 from the up weight)
      const int grow = EPI == EPI_SILU ? tn * (BN / 2) + (row & (BN / 2 - 1)) : n0 + row;
      bo[q] = (uint32_t)(((int64_t)min(grow, N - 1) * p.ldb + dl_swz(row, lane % CH) * 8) * 2);
    }
  }
  auto issue = [&](int st, int k0) __attribute__((always_inline)) {
    uint16_t* as = smem + st * (TA + TB);
    uint16_t* bs = as + TA;
    const char* Ab = (const char*)(A + k0);
    const char* Bb = Bbase + (int64_t)k0 * (B_KN ? p.ldb * 2 : (B_INT8 ? 1 : 2));
#pragma unroll
    for (int q = 0; q < NQA; ++q) lds_copy16(Ab, ao[q], as + (wave * NQA + q) * 512);
#pragma unroll
    for (int q = 0; q < NQB; ++q) lds_copy16(Bb, bo[q], bs + (wave * NQB + q) * 512);
  };
  // fragment read offsets: lane supplies row l % MD, 16-byte k chunk
  // (KPM / 8) s + l / MD of substep s
  int roff[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    roff[s] = (lane % MD) * BK + dl_swz(lane % MD, (KPM / 8) * s + lane / MD) * 8;
  }

  // acc[j][i] = D^T tile (n rows j, m cols i): B fragments are the MFMA's A
  // operand, so a lane ends up owning one output row m and runs of 4 n
  // (4 runs for 32 x 32 tiles, one for 16 x 16)
  acc_t acc[FN][FM];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[j][i] = acc_t{};
  vec af[2][FM], bfr[2][FN];
  // row-major B: lane (G = lane / 16, j = lane % 16) reads k row
  // 8 (G / 2) + j / 4 (+ 4 for the second half) of a substep, columns
  // wn TN + 32 jt + 16 (G % 2) + 4 (j % 4) .. + 3; the chunk swizzle makes
  // the fragment jt's offset 64 (jt ^ (j / 4)) bytes, per lane
  int kno[FN];
  if constexpr (B_KN) {
    const int G = lane >> 4, j = lane & 15;
    const int kr = 8 * (G >> 1) + (j >> 2);
    const int x = 2 * (G & 1) + ((j & 3) >> 1);
#pragma unroll
    for (int jt = 0; jt < FN; ++jt)
      kno[jt] = kr * BN + (wn * 16 + 4 * (jt ^ (j >> 2)) + x) * 8 + 4 * (j & 1);  // in elements
  }
  auto read_frags = [&](int st, int s, int buf) __attribute__((always_inline)) {
    const uint16_t* as = smem + st * (TA + TB) + wm * TM * BK + roff[s];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[buf][i] = *(const vec*)(as + i * MD * BK);
    if constexpr (B_KN) {
      typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
      const uint16_t* bs = smem + st * (TA + TB) + TA + 16 * s * BN;
#pragma unroll
      for (int jt = 0; jt < FN; ++jt) {
        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(bs + kno[jt]));
        const s16x4_t hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(bs + kno[jt] + 4 * BN));
        bfr[buf][jt] = __builtin_bit_cast(vec, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    } else if constexpr (B_INT8) {
      // the bf16 copy of the stage's W rows (converted once per block)
      const uint16_t* bs = smem + STAGES * (TA + TB) + st * dl::TB + wn * TN * BK + roff[s];
#pragma unroll
      for (int j = 0; j < FN; ++j) bfr[buf][j] = *(const vec*)(bs + j * MD * BK);
    } else {
      const uint16_t* bs = smem + st * (TA + TB) + TA + wn * TN * BK + roff[s];
#pragma unroll
      for (int j = 0; j < FN; ++j) bfr[buf][j] = *(const vec*)(bs + j * MD * BK);
    }
  };
  auto mfmas = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i) acc[j][i] = mma(bfr[buf][j], af[buf][i], acc[j][i]);
  };
  // int8 W: wave w copied rows 32 w .. 32 w + 31 of every stage itself, so
  // once its own loads have landed it widens exactly those rows into the
  // stage's bf16 copy (same chunk swizzle as a 16-bit B tile); the barrier
  // that follows publishes them.  Lane: row 32 w + l / 2, k half l % 2.
  auto convert = [&](int st) __attribute__((always_inline)) {
    if constexpr (B_INT8) {
      const char* b8 = (const char*)(smem + st * (TA + TB) + TA);
      uint16_t* bb = smem + STAGES * (TA + TB) + st * dl::TB;
      const int r = wave * 32 + (lane >> 1), h = lane & 1;
      const u32x4_t c0 = *(const u32x4_t*)(b8 + r * 64 + dl_swz64(r, 2 * h) * 16);
      const u32x4_t c1 = *(const u32x4_t*)(b8 + r * 64 + dl_swz64(r, 2 * h + 1) * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t& c = j < 2 ? c0 : c1;
        const u32x2_t w = {c[2 * (j & 1)], c[2 * (j & 1) + 1]};
        *(vec*)(bb + r * BK + dl_swz(r, 4 * h + j) * 8) = widen8<T>(w);
      }
    }
  };
  constexpr int NMF = FM * FN, NDS = FM + FN;
  // 16 x 16 x 32 schedule, in an order the compiler keeps (a scheduling fence
  // after every MFMA): A fragments double-buffered, read for the next
  // substep during the first FM MFMAs; B fragments single-buffered, fragment
  // j of the next substep read right after its last MFMA (j FM + FM - 1) of
  // this one, so each read has most of a substep to land; the refill loads
  // one per two MFMAs of the step's last substep.  Against the 32 x 32
  // tiles with grouped reads this is 4-10 % faster on the decoder-layer and
  // config-4 shapes, with bit-identical results.
  auto issue_one = [&](int st, int k0, int q) __attribute__((always_inline)) {
    uint16_t* as = smem + st * (TA + TB);
    uint16_t* bs = as + TA;
    if (q < NQA) {
      lds_copy16(A + k0, ao[q], as + (wave * NQA + q) * 512);
    } else {
      const char* Bb = Bbase + (int64_t)k0 * (B_INT8 ? 1 : 2);
      lds_copy16(Bb, bo[q - NQA], bs + (wave * NQB + q - NQA) * 512);
    }
  };
  auto read_a = [&](int st, int s, int buf, int i) __attribute__((always_inline)) {
    const uint16_t* as = smem + st * (TA + TB) + wm * TM * BK + roff[s];
    af[buf][i] = *(const vec*)(as + i * MD * BK);
  };
  auto read_b = [&](int st, int s, int j) __attribute__((always_inline)) {
    const uint16_t* bs = B_INT8 ? smem + STAGES * (TA + TB) + st * dl::TB + wn * TN * BK + roff[s]
                                : smem + st * (TA + TB) + TA + wn * TN * BK + roff[s];
    bfr[0][j] = *(const vec*)(bs + j * MD * BK);
  };
  auto mfma_one = [&](int buf, int m) __attribute__((always_inline)) {
    const int j = m / FM, i = m % FM;
    acc[j][i] = mma(bfr[0][j], af[buf][i], acc[j][i]);
  };
  // one K step over stage st.  ISSUE: refill stage st with step kt + STAGES;
  // NEXT: step kt + 1 exists and its first fragments are read here.
  auto step = [&](int st, int kt, bool ISSUE, bool NEXT) __attribute__((always_inline)) {
    if constexpr (M16) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int buf = s & 1;
        if (s + 1 < KS) {
#pragma unroll
          for (int m = 0; m < NMF; ++m) {
            mfma_one(buf, m);
            if (m < FM) read_a(st, s + 1, buf ^ 1, m);
            if (m % FM == FM - 1) read_b(st, s + 1, m / FM);
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
          const int nst = st + 1 == STAGES ? 0 : st + 1;
          if (NEXT) {
            // as below: step kt + 1 has landed and every wave is done with
            // stage st (its last fragments were read in the previous substep)
            if (ISSUE) wait_vmcnt<(STAGES - 2) * LPS>();
            else wait_vmcnt<0>();
            convert(nst);
            __syncthreads();
          }
          // one refill load per two MFMAs, from the substep's first MFMA (the
          // loads spread over all of it measured 1-3 % slower on the decoder
          // shapes, back to back 2-4 % slower)
          constexpr int MPL = 2;
          static_assert(MPL * LPS <= NMF, "every refill load is issued in the substep");
#pragma unroll
          for (int m = 0; m < NMF; ++m) {
            mfma_one(buf, m);
            if (ISSUE && m % MPL == 0 && m / MPL < LPS) issue_one(st, (kt + STAGES) * BK, m / MPL);
            if (NEXT) {
              if (m < FM) read_a(nst, 0, buf ^ 1, m);
              if (m % FM == FM - 1) read_b(nst, 0, m / FM);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      return;
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int buf = s & 1;
      if (s + 1 < KS) {
        read_frags(st, s + 1, buf ^ 1);
        mfmas(buf);
#pragma unroll
        for (int k = 0; k < NDS; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NMF - NDS, 0);
      } else {
        if (NEXT) {
          // step kt + 1 has landed once at most the newer steps' loads are
          // outstanding; the barrier also tells every wave that all waves
          // are done reading stage st
          if (ISSUE) wait_vmcnt<(STAGES - 2) * LPS>();
          else wait_vmcnt<0>();
          convert(st + 1 == STAGES ? 0 : st + 1);
          __syncthreads();
          if (ISSUE) issue(st, (kt + STAGES) * BK);
          read_frags(st + 1 == STAGES ? 0 : st + 1, 0, buf ^ 1);
        }
        mfmas(buf);
#pragma unroll
        for (int k = 0; k < NMF; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (ISSUE && k < LPS) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
          if (NEXT && k < NDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The epilogue's pointers are formed (and their scalar loads waited for)
  // before the main loop: left to the compiler, such a load (the batch
  // stride, the int8 scales) was issued just before the loop and stayed in
  // flight through it, and since scalar loads return out of order every LDS
  // wait in the loop became lgkmcnt(0), so each step's first MFMA waited for
  // reads issued after the ones it needs.
  uint16_t* Cb = p.c + batch * p.sc;
  asm volatile("" : : "s"(Cb));
  const float* scale = p.scale;
  if constexpr (B_INT8) asm volatile("" : : "s"(scale));
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
    if (s < KT) issue(s, s * BK);
  if (STAGES <= KT) wait_vmcnt<(STAGES - 1) * LPS>();
  else wait_vmcnt<0>();
  convert(0);
  __syncthreads();
  read_frags(0, 0, 0);
  int st = 0, kt = 0;
  for (; kt < KT - STAGES; ++kt) {
    step(st, kt, true, true);
    st = st + 1 == STAGES ? 0 : st + 1;
  }
  for (; kt < KT; ++kt) {
    step(st, kt, false, kt + 1 < KT);
    st = st + 1 == STAGES ? 0 : st + 1;
  }

  if constexpr (SPLIT) {
    // raw sums of this K slice: a lane's runs of 4 columns as 16-byte stores
    // (ldp is a multiple of 4, so a run that starts inside the row fits)
    float* P = part + (int64_t)blockIdx.y * p.M * ldp;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < MD * MD / 256; ++g) {
        const int64_t n = n0 + wn * TN + j * MD + (M16 ? 4 * (lane >> 4) : 8 * g + 4 * (lane >> 5));
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int64_t m = m0 + wm * TM + i * MD + (lane % MD);
          if (m < p.M && n < p.N) {
            const f32x4_t v = {acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2],
                               acc[j][i][4 * g + 3]};
            *(f32x4_t*)(P + m * ldp + n) = v;
          }
        }
      }
    return;
  }
  // epilogue: out = alpha * acc + beta * bias, one rounding, staged per wave.
  // A lane's outputs come in runs of 4 columns; the per-column factors (the
  // int8 scale, a bias broadcast over rows) are loaded once per run, four
  // at a time, and used for both row fragments (one scalar load per output
  // made the bias epilogue cost 13 % of config 4's addmm)
  __syncthreads();
  uint16_t* es = smem + wave * TM * EP;
  const float alpha = p.alpha, beta = p.beta;
  const bool row_bias = HAS_BIAS && p.bias_sm == 0;
  auto load_col4 = [&](const void* base, int dtype, int64_t n, int64_t stride, int64_t N,
                       int64_t off = 0) __attribute__((always_inline)) {
    return load_col4_t<T>(base, dtype, n, stride, N, off);
  };
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int g = 0; g < MD * MD / 256; ++g) {
      const int nl = j * MD + (M16 ? 4 * (lane >> 4) : 8 * g + 4 * (lane >> 5));
      const int64_t n = n0 + wn * TN + nl;
      f32x4_t sc4 = {1.f, 1.f, 1.f, 1.f}, bb4 = {};
      if constexpr (B_INT8) sc4 = load_col4(scale, MI_F32, n, 1, p.N);
      if (row_bias) bb4 = load_col4(p.bias, p.bias_dtype, n, p.bias_sn, p.N, batch * p.bias_sb);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int ml = i * MD + (lane % MD);
        const int64_t m = m0 + wm * TM + ml;
        u16x4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = alpha * acc[j][i][4 * g + e] * sc4[e];
          if (HAS_BIAS) {
            float bv = bb4[e];
            if (!row_bias) {
              const int64_t bo_ = batch * p.bias_sb + min<int64_t>(m, p.M - 1) * p.bias_sm +
                                  min<int64_t>(n + e, p.N - 1) * p.bias_sn;
              bv = p.bias_dtype == MI_F32 ? ((const float*)p.bias)[bo_]
                                          : MfmaOp<T>::load(((const uint16_t*)p.bias)[bo_]);
            }
            x += beta * bv;
          }
          v[e] = MfmaOp<T>::store(x);
        }
        *(u16x4_t*)(es + ml * EP + nl) = v;
      }
    }
  const int64_t rbase = m0 + wm * TM, cbase = n0 + wn * TN;
  constexpr int LPR = TN / 8, RPI = 64 / LPR;  // lanes per row, rows per pass
  const bool vec_ok = (p.ldc % 8) == 0 && (((uintptr_t)Cb) & 15) == 0;
  typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));
  if constexpr (EPI == EPI_SILU) {
    // the row band's gate values are in the staging of wave (wm, 0), its up
    // values in that of wave (wm, 1); wave (wm, wn) takes rows 32 wn .. 32 wn + 31
    __syncthreads();
    const uint16_t* eg = smem + (wm * WN) * TM * EP;
    const uint16_t* eu = eg + TM * EP;
    const int64_t cb = (int64_t)tn * (BN / 2);
#pragma unroll 4
    for (int it = 0; it < TM / 2 / RPI; ++it) {
      const int r = wn * (TM / 2) + it * RPI + lane / LPR, c = (lane % LPR) * 8;
      const u16x8_t g8 = *(const u16x8_t*)(eg + r * EP + c);
      const u16x8_t u8 = *(const u16x8_t*)(eu + r * EP + c);
      u16x8_t v;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[e] = MfmaOp<T>::store(silu_mul_f32(MfmaOp<T>::load(g8[e]), MfmaOp<T>::load(u8[e])));
      const int64_t m = rbase + r, n = cb + c;
      if (m < p.M) {
        if (vec_ok && n + 7 < p.N) {
          *(u16x8_t*)(Cb + m * p.ldc + n) = v;
        } else {
          for (int e = 0; e < 8; ++e)
            if (n + e < p.N) Cb[m * p.ldc + n + e] = v[e];
        }
      }
    }
    return;
  }
  const bool res_vec = EPI == EPI_RESID && (p.ldr % 8) == 0 && (((uintptr_t)p.res) & 15) == 0;
#pragma unroll 4
  for (int it = 0; it < TM / RPI; ++it) {
    const int r = it * RPI + lane / LPR, c = (lane % LPR) * 8;
    u16x8_t v = *(const u16x8_t*)(es + r * EP + c);
    const int64_t m = rbase + r, n = cbase + c;
    if (m < p.M) {
      if constexpr (EPI == EPI_RESID) {
        // residual + the rounded product, as the add kernel: fma(other, 1, self)
        u16x8_t rv;
        if (res_vec && n + 7 < p.N) {
          rv = *(const u16x8_t*)(p.res + m * p.ldr + n);
        } else {
          for (int e = 0; e < 8; ++e) rv[e] = n + e < p.N ? p.res[m * p.ldr + n + e] : (uint16_t)0;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[e] = MfmaOp<T>::store(
              __builtin_fmaf(MfmaOp<T>::load(v[e]), 1.0f, MfmaOp<T>::load(rv[e])));
      }
      if (vec_ok && n + 7 < p.N) {
        *(u16x8_t*)(Cb + m * p.ldc + n) = v;
      } else {
        for (int e = 0; e < 8; ++e)
          if (n + e < p.N) Cb[m * p.ldc + n + e] = v[e];
      }
    }
  }
}

// ---- int8 weight-only linear, mid-size M (64 < M <= 512): 128 x R tiles -------------
//
// (Runs where split-K over 256 x 256 tiles does not apply: a single K step,
// or enough tiles to fill the CUs; the sizes below are config 4's, which
// split-K now runs faster.)
// Config 4's M = 256 against W [11008, 4096] has 2 x 11008 / 256 = 86 W rows
// per CU: 128 x 256 tiles give 86 blocks, 128 x 64 tiles 344 (1.34 waves).
// Here a 256-lane block owns 128 rows of x (32 per wave) and R W rows, R a
// multiple of 8 up to 96 chosen so that the blocks about fill the CUs (R = 88
// for config 4: 252 blocks).  K steps of 64 flow through four LDS stages
// filled by global_load_lds (three steps in flight while one is multiplied:
// one block per CU has no other block to cover the latency): x rows as bf16
// (128-byte rows, chunk swizzle dl_swz), W rows as int8 (64-byte rows,
// dl_swz64), which waves 0..2 widen, 32 rows each, into one of two bf16
// copies (dl_swz) once their own copies of the next step have landed.
// (Measured on config 4's M = 256: 49 us, against 54-56 us for the 128 x 64
// register-staged tiles; two stages 53 us; widening spread over all four
// waves, or two steps ahead through a third copy with five stages, 53-58 us.
// The kernel stays far from its 11.7 us MFMA time: per K step its four waves
// stall on the barrier, the widening and the fragment reads in turn.)
// Each wave multiplies its 32 x rows with three 32-row W fragments
// (v_mfma_f32_32x32x16, W as the A operand, so a lane owns one output row and
// runs of 4 columns); the epilogue applies alpha, the per-column scale and
// the bias, rounds once and stores through LDS.
// cache policy operand of global_load_lds on gfx950: non-temporal (NT = bit 1)
constexpr int kCpolNT = 2;

namespace mid {
constexpr int BM = 128, BNF = 96, KB = 64, NT = 256, NW = 4;
constexpr int STAGES = 4;                     // copies in flight: steps kt + 1 .. kt + 3
constexpr int COPIES = 2;                     // bf16 W copies (steps kt, kt + 1)
constexpr int FN = BNF / 32;                  // W fragments per wave
constexpr int TA = BM * KB;                   // x tile, 16-bit elements
constexpr int TB8 = BNF * KB / 2;             // int8 W tile, in 16-bit units
constexpr int TB = BNF * KB;                  // bf16 copy of the W tile
constexpr int STAGE = TA + TB8;               // the part global_load_lds fills
constexpr int NQA = BM * KB * 2 / 1024 / NW;  // x copies per wave (4)
constexpr int NQB = 2;                        // W copies per wave 0..2 (16 rows each)
constexpr int KS = KB / 16;
constexpr int EP = BNF + 8;                   // epilogue row pitch
constexpr size_t LDS = ((size_t)STAGES * STAGE + (size_t)COPIES * TB) * 2;
static_assert(LDS >= (size_t)NW * 32 * EP * 2, "epilogue staging fits");
static_assert(LDS <= 160 * 1024, "one block's LDS");
}  // namespace mid

template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(mid::NT, 1) void int8_mid_kernel(GemmArgs p, int R) {
  using namespace mid;
  typedef typename MfmaOp<T>::vec vec;
  extern __shared__ __align__(16) uint16_t smem[];
  // XCD-aware order (round-robin dispatch over 8 XCDs): consecutive logical
  // blocks, the m tiles of one W panel first, run on one XCD and share the
  // panel through its L2
  int id = blockIdx.x;
  {
    const int total = p.tiles_m * p.tiles_n;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  }
  const int tm = id % p.tiles_m, tn = id / p.tiles_m;
  const int M = (int)p.M, N = (int)p.N, K = (int)p.K;
  const int m0 = tm * BM, n0 = tn * R;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool w_rows = wave < BNF / 32;  // waves copying and widening W rows
  const char* Bbase = (const char*)p.b;

  // per-lane byte offsets (the host checked they fit 32 bits); rows past the
  // matrix are clamped to its last row and only feed outputs never stored
  uint32_t ao[NQA], bo[NQB];
#pragma unroll
  for (int q = 0; q < NQA; ++q) {
    const int row = (wave * NQA + q) * 8 + lane / 8;
    ao[q] = (uint32_t)(((int64_t)min(m0 + row, M - 1) * p.lda + dl_swz(row, lane % 8) * 8) * 2);
  }
#pragma unroll
  for (int q = 0; q < NQB; ++q) {
    const int row = (wave * NQB + q) * 16 + lane / 4;
    bo[q] = (uint32_t)((int64_t)min(n0 + row, N - 1) * p.ldb + dl_swz64(row, lane % 4) * 16);
  }
  auto issue = [&](int st, int k0) __attribute__((always_inline)) {
    uint16_t* as = smem + st * STAGE;
    uint16_t* bs = as + TA;
    const char* Ab = (const char*)(p.a + k0);
    const char* Bb = Bbase + k0;
#pragma unroll
    for (int q = 0; q < NQA; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(Ab + ao[q]),
                                       (lds_void_t*)(as + (wave * NQA + q) * 512), 16, 0, 0);
    if (w_rows) {
      // W is streamed once (non-temporal: it should not push x out of L2)
#pragma unroll
      for (int q = 0; q < NQB; ++q)
        __builtin_amdgcn_global_load_lds((const void*)(Bb + bo[q]),
                                         (lds_void_t*)(bs + (wave * NQB + q) * 512), 16, 0, kCpolNT);
    }
  };
  // wave w < 3 copied W rows 32 w .. 32 w + 31 of every stage itself and
  // widens exactly those rows into a bf16 copy; lane: row 32 w + l / 2, k half l % 2
  auto convert = [&](int st, int cb) __attribute__((always_inline)) {
    if (w_rows) {
      const char* b8 = (const char*)(smem + st * STAGE + TA);
      uint16_t* bb = smem + STAGES * STAGE + cb * TB;
      const int r = wave * 32 + (lane >> 1), h = lane & 1;
      const u32x4_t c0 = *(const u32x4_t*)(b8 + r * 64 + dl_swz64(r, 2 * h) * 16);
      const u32x4_t c1 = *(const u32x4_t*)(b8 + r * 64 + dl_swz64(r, 2 * h + 1) * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t& c = j < 2 ? c0 : c1;
        const u32x2_t w = {c[2 * (j & 1)], c[2 * (j & 1) + 1]};
        *(vec*)(bb + r * KB + dl_swz(r, 4 * h + j) * 8) = widen8<T>(w);
      }
    }
  };
  // fragment read offsets: lane supplies row l % 32, k chunk 2 s + l / 32
  int roff[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) roff[s] = (lane & 31) * KB + dl_swz(lane & 31, 2 * s + (lane >> 5)) * 8;

  f32x16 acc[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) acc[j] = f32x16{};
  vec af[2], bfr[2][FN];
  auto read_frags = [&](int st, int cb, int s, int buf) __attribute__((always_inline)) {
    af[buf] = *(const vec*)(smem + st * STAGE + wave * 32 * KB + roff[s]);
    const uint16_t* bs = smem + STAGES * STAGE + cb * TB + roff[s];
#pragma unroll
    for (int j = 0; j < FN; ++j) bfr[buf][j] = *(const vec*)(bs + j * 32 * KB);
  };
  auto mfmas = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[j] = MfmaOp<T>::mma(bfr[buf][j], af[buf], acc[j]);
  };
  const int KT = K / KB;
  // this wave's copies of a step: the wait until step kt + 1 has landed
  // while `later` newer steps stay in flight
  auto wait_step = [&](int later) __attribute__((always_inline)) {
    if (w_rows) wait_later<STAGES - 1, NQA + NQB>(later);
    else wait_later<STAGES - 1, NQA>(later);
  };
  // One K step kt: x from stage kt % STAGES, W from bf16 copy kt % 2.  At
  // its last K substep step kt + 1 is waited for (steps kt + 2 .. kt +
  // STAGES - 1 stay in flight), widened, published by the barrier (which
  // also retires stage kt % STAGES, refilled with step kt + STAGES) and its
  // first fragments read.
  auto step = [&](int kt) __attribute__((always_inline)) {
    const int st = kt % STAGES, cb = kt & 1;
    const int st1 = (kt + 1) % STAGES, cb1 = cb ^ 1;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int buf = s & 1;
      if (s + 1 < KS) {
        read_frags(st, cb, s + 1, buf ^ 1);
        mfmas(buf);
        // MFMA, two fragment reads, then MFMA and one read each
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int k = 1; k < FN; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      } else {
        if (kt + 1 < KT) {
          wait_step(min(STAGES - 2, KT - 2 - kt));
          convert(st1, cb1);
          __syncthreads();
          if (kt + STAGES < KT) issue(st, (kt + STAGES) * KB);
          read_frags(st1, cb1, 0, buf ^ 1);
        }
        mfmas(buf);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

#pragma unroll
  for (int s = 0; s < STAGES; ++s)
    if (s < KT) issue(s, s * KB);
  // step 0 has landed once only steps 1 .. STAGES - 1 (those that exist) are in flight
  wait_step(min(STAGES, KT) - 1);
  convert(0, 0);
  __syncthreads();
  read_frags(0, 0, 0, 0);
  for (int kt = 0; kt < KT; ++kt) step(kt);

  // epilogue: out = alpha * scale[n] * acc + beta * bias, one rounding,
  // staged per wave as [32 x rows][96 W rows] and stored in 16-byte pieces
  __syncthreads();
  uint16_t* es = smem + wave * 32 * EP;
  const float alpha = p.alpha, beta = p.beta;
  const bool bias_f32 = p.bias_dtype == MI_F32;
  const int ml = lane & 31;
  const int64_t m = m0 + wave * 32 + ml;
  // the per-column scale (and a bias broadcast over rows) four columns per load
  const bool row_bias = HAS_BIAS && p.bias_sm == 0;
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = j * 32 + 8 * g + 4 * (lane >> 5);
      const f32x4_t sc4 = load_col4_t<T>(p.scale, MI_F32, n0 + nl, 1, p.N, 0);
      f32x4_t bb4 = {};
      if (row_bias) bb4 = load_col4_t<T>(p.bias, p.bias_dtype, n0 + nl, p.bias_sn, p.N, 0);
      u16x4_t v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = alpha * acc[j][4 * g + e] * sc4[e];
        if (HAS_BIAS) {
          float bv = bb4[e];
          if (!row_bias) {
            const int64_t n = min<int64_t>(n0 + nl + e, p.N - 1);
            const int64_t bo_ = min<int64_t>(m, p.M - 1) * p.bias_sm + n * p.bias_sn;
            bv = bias_f32 ? ((const float*)p.bias)[bo_]
                          : MfmaOp<T>::load(((const uint16_t*)p.bias)[bo_]);
          }
          x += beta * bv;
        }
        v[e] = MfmaOp<T>::store(x);
      }
      *(u16x4_t*)(es + ml * EP + nl) = v;
    }
  // the block's columns: n0 .. n0 + R - 1 (fewer in the last tile)
  const int ncols = min(R, N - n0);
  const bool vec_ok = (p.ldc % 8) == 0 && (((uintptr_t)p.c) & 15) == 0 && (n0 % 8) == 0;
  for (int idx = lane; idx < 32 * (BNF / 8); idx += 64) {
    const int r = idx / (BNF / 8), c = (idx % (BNF / 8)) * 8;
    const int64_t mr = m0 + wave * 32 + r;
    if (mr >= p.M || c >= ncols) continue;
    const uint4 v = *(const uint4*)(es + r * EP + c);
    uint16_t* dst = p.c + mr * p.ldc + n0 + c;
    if (vec_ok && c + 8 <= ncols) {
      *(uint4*)dst = v;
    } else {
      const uint16_t* pv = (const uint16_t*)&v;
      for (int e = 0; e < 8 && c + e < ncols; ++e) dst[e] = pv[e];
    }
  }
}

template <typename T, bool HB>
mi_status_t launch_mid(const GemmArgs& q0, hipStream_t s, const char* what) {
  static bool attr = [] {
    (void)hipFuncSetAttribute((const void*)int8_mid_kernel<T, HB>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)mid::LDS);
    return true;
  }();
  (void)attr;
  GemmArgs q = q0;
  q.tiles_m = (int)((q.M + mid::BM - 1) / mid::BM);
  // W rows per block: a multiple of 8 up to 96, so that the blocks about fill the CUs
  const int64_t want_n = std::max<int64_t>(1, cu_count() / q.tiles_m);
  int64_t R = (q.N + want_n - 1) / want_n;
  R = std::min<int64_t>(mid::BNF, std::max<int64_t>(32, (R + 7) / 8 * 8));
  q.tiles_n = (int)((q.N + R - 1) / R);
  hipLaunchKernelGGL((int8_mid_kernel<T, HB>), dim3((unsigned)(q.tiles_m * q.tiles_n)),
                     dim3(mid::NT), mid::LDS, s, q, (int)R);
  return check_launch(what);
}

// ---- int8 weight-only linear for few rows (M <= 64): HBM-bound on W -------------------
//
// A 512-lane block owns 32 output columns (two 16-row tiles of W [N, K]);
// its 8 waves split K into interleaved 128-wide chunks, so per step the block
// reads 1 KiB contiguous bytes of each of its W rows and every 128-byte line
// is read whole by one wave.  In a chunk, lane (r = l % 16, g = l / 16)
// streams W[n0 + 16 t + r][128 c + 32 g .. + 32] with two non-temporal
// 16-byte loads per tile t, widens the 32 int8 to bf16 (exact) and feeds
// v_mfma_f32_16x16x32 with the matching 32 k of each x row (x is [M, K] and
// stays in cache).  The k order inside a chunk is the same for both
// operands, so the sum is the plain dot product.  The 8 waves' partial
// 16 x 16 tiles are added in a fixed order through LDS; the epilogue applies
// the per-column scale and bias and rounds once.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int int4v_t __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma16;
template <>
struct Mfma16<BF16> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4_t mma(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec widen(int4v_t w, int half) {
    vec v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int byte = 8 * half + e;
      v[e] = (__bf16)(float)(int8_t)(w[byte >> 2] >> (8 * (byte & 3)));
    }
    return v;
  }
};
template <>
struct Mfma16<F16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4_t mma(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec widen(int4v_t w, int half) {
    vec v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int byte = 8 * half + e;
      v[e] = (_Float16)(float)(int8_t)(w[byte >> 2] >> (8 * (byte & 3)));
    }
    return v;
  }
};

constexpr int kSkN = 2;    // 16-row n-tiles per block (32 W rows)
constexpr int kSkW = 8;    // waves per block, splitting K

template <typename T, int MT, bool HAS_BIAS>
__global__ __launch_bounds__(64 * kSkW, MT == 1 ? 4 : 1) void int8_skinny_kernel(GemmArgs p) {
  typedef typename Mfma16<T>::vec vec;
  __shared__ float red[kSkW][kSkN][16][17];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16 * kSkN;
  // lane (r, g) owns bytes [32 g, 32 g + 32) of each 128-byte chunk of the W
  // rows n0 + 16 t + r, so one wave reads whole 128-byte lines
  const int8_t* wrow[kSkN];
#pragma unroll
  for (int t = 0; t < kSkN; ++t)
    wrow[t] = (const int8_t*)p.b + min<int64_t>(n0 + 16 * t + r, p.N - 1) * p.ldb + 32 * g;
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = p.a + min<int64_t>(mt * 16 + r, p.M - 1) * p.lda + 32 * g;
  f32x4_t acc[MT][kSkN];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < kSkN; ++t) acc[mt][t] = f32x4_t{};
  // one 128-wide chunk of W (kSkN tiles) and x in registers, double-buffered:
  // the loads of chunk c + kSkW are in flight while chunk c is widened and
  // multiplied
  struct Chunk {
    int4v_t w[kSkN][2];
    vec x[MT][4];
  };
  auto load = [&](Chunk& ch, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < kSkN; ++t) {
      const int8_t* wp = wrow[t] + 128 * c;
      ch.w[t][0] = __builtin_bit_cast(int4v_t, ld_stream((const uint4*)wp));
      ch.w[t][1] = __builtin_bit_cast(int4v_t, ld_stream((const uint4*)(wp + 16)));
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int h = 0; h < 4; ++h) ch.x[mt][h] = *(const vec*)(xrow[mt] + 128 * c + 8 * h);
  };
  // consecutive MFMAs go to different accumulators (n-tiles inner)
  auto compute = [&](const Chunk& ch) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int t = 0; t < kSkN; ++t) {
        // the empty asm pins the start of the byte unpacking here, so the
        // compiler cannot unpack every loaded W byte into its own register
        // right after the loads
        int4v_t wd = ch.w[t][h >> 1];
        asm volatile("" : "+v"(wd));
        const vec wk = Mfma16<T>::widen(wd, h & 1);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][t] = Mfma16<T>::mma(ch.x[mt][h], wk, acc[mt][t]);
      }
  };
  const int KC = (int)(p.K / 128);  // chunks; wave w takes chunks w, w + kSkW, ...
  // two named buffers (a runtime-indexed pair would live in scratch memory)
  Chunk b0, b1;
  if (wave < KC) load(b0, wave);
  for (int c = wave; c < KC; c += 2 * kSkW) {
    if (c + kSkW < KC) load(b1, c + kSkW);
    compute(b0);
    if (c + kSkW < KC) {
      if (c + 2 * kSkW < KC) load(b0, c + 2 * kSkW);
      compute(b1);
    }
  }
  // D[m = 4 (l / 16) + i][n = l % 16] of each 16 x 16 (m-tile, n-tile); the
  // m-tiles are reduced one at a time through LDS
  const int tn = threadIdx.x & 15, tm = (threadIdx.x >> 4) & 15, tt = threadIdx.x >> 8;
  const bool bias_f32 = p.bias_dtype == MI_F32;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (mt > 0) __syncthreads();
#pragma unroll
    for (int t = 0; t < kSkN; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][t][4 * g + i][r] = acc[mt][t][i];
    __syncthreads();
    const int64_t m = mt * 16 + tm;
    if (m >= p.M) continue;
    // 512 lanes: lane -> (n-tile tt (+2, ...), row m, column n)
#pragma unroll
    for (int t = tt; t < kSkN; t += 2) {
      const int64_t n = n0 + 16 * t + tn;
      if (n >= p.N) continue;
      float sum = red[0][t][tm][tn];
#pragma unroll
      for (int w = 1; w < kSkW; ++w) sum += red[w][t][tm][tn];
      float v = p.alpha * p.scale[n] * sum;
      if (HAS_BIAS) {
        const int64_t bo = m * p.bias_sm + n * p.bias_sn;
        v += p.beta * (bias_f32 ? ((const float*)p.bias)[bo]
                                : MfmaOp<T>::load(((const uint16_t*)p.bias)[bo]));
      }
      p.c[m * p.ldc + n] = MfmaOp<T>::store(v);
    }
  }
}

template <typename T, bool HB>
mi_status_t launch_skinny(const GemmArgs& q, hipStream_t s) {
  const dim3 grid(ceil_div_u(q.N, 16 * kSkN)), block(64 * kSkW);
  const int mt = (int)((q.M + 15) / 16);
  switch (mt) {
    case 1: hipLaunchKernelGGL((int8_skinny_kernel<T, 1, HB>), grid, block, 0, s, q); break;
    case 2: hipLaunchKernelGGL((int8_skinny_kernel<T, 2, HB>), grid, block, 0, s, q); break;
    case 3: hipLaunchKernelGGL((int8_skinny_kernel<T, 3, HB>), grid, block, 0, s, q); break;
    default: hipLaunchKernelGGL((int8_skinny_kernel<T, 4, HB>), grid, block, 0, s, q); break;
  }
  return check_launch("int8_linear skinny");
}

// ---- int8 weight-only linear for few rows, weight staged through LDS ------------------
//
// The contraction of int8_skinny_kernel for K % 1024 == 0 and 16-byte aligned
// W rows.  A 512-lane block owns R consecutive W rows, R = N / CUs rounded up
// (43 for N = 11008 on 256 CUs) and at most 48, so every CU streams the same
// share of W once (with 32-row blocks, 344 blocks on 256 CUs left 88 CUs
// streaming twice the bytes of the others).  K is walked in 1 KiB slabs of
// 48 rows (three 16-row MFMA tiles; rows past R re-read the block's last
// row, an L2 hit, and feed columns that are never stored), and wave w owns
// bytes 128 w .. 128 w + 127 of every slab row: it copies them into its own
// LDS ring by global_load_lds_dwordx4 (one copy = 8 rows x 128 bytes, whole
// cache lines) together with the matching x fragments into registers, and
// multiplies them, so the waves never wait for each other until the final
// combine.  The ring holds three slabs (two slabs of lead on the one being
// multiplied; a wave refills a slot as soon as it has multiplied it).  Lane
// (r, g) reads 16 bytes of row 16 t + r at 64 kp + 16 g (kp = 0, 1), which
// feed two v_mfma_f32_16x16x32 (8 bytes each, widened to bf16 exactly) with
// x as the 16-row operand, x's fragments taken at the same k.  Rows are 128
// bytes in LDS, chunk c of row r stored at c ^ ((r >> 1) & 7) (the copying
// lane fetches the matching global chunk), so the 16 rows of a read pass hit
// 16 distinct 16-byte bank groups.  The 8 waves' partial tiles are added in
// a fixed order through LDS; the epilogue applies the per-column scale and
// bias and rounds once.
constexpr int kStTiles = 3, kStRows = 16 * kStTiles, kStSlab = 1024, kStWaves = 8;
constexpr int kStPart = kStSlab / kStWaves;    // bytes of a slab row per wave (128)
constexpr int kStCopies = kStRows * kStPart / 1024;  // wave copies per slab (6)
constexpr int kStRing = 3;
constexpr int kStWaveLds = kStRing * kStRows * kStPart;  // one wave's ring
constexpr int kStLds = kStWaves * kStWaveLds;
static_assert(kStLds <= 160 * 1024, "slab rings fit the LDS");
static_assert(kStLds >= kStWaves * kStTiles * 16 * 17 * 4, "combine staging fits");

// SFIX > 0 fixes the slab count at compile time (K = 1024 SFIX): the loop is
// then fully unrolled and the compiler can count the loads in flight at
// every step (through the loop's back edge it waits for all of them before
// a step's first MFMA).
template <typename T, int MT, int RING, bool HAS_BIAS, int SFIX>
__global__ __launch_bounds__(64 * kStWaves, 1) void int8_stream_kernel(GemmArgs p, int R) {
  typedef typename Mfma16<T>::vec vec;
  extern __shared__ __align__(16) char st_lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * R;
  const int nrows = (int)min<int64_t>(R, p.N - n0);
  const int S = SFIX > 0 ? SFIX : (int)(p.K / kStSlab);
  char* ring = st_lds + wave * kStWaveLds;
  // copy q moves slab rows 8 q .. 8 q + 7: lane l fetches row 8 q + l / 8, the
  // global chunk that lands at chunk l % 8 of the swizzled row (source rows
  // past the block's nrows re-read its last row)
  const int8_t* wsrc[kStCopies];
#pragma unroll
  for (int q = 0; q < kStCopies; ++q) {
    const int row = 8 * q + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    wsrc[q] = (const int8_t*)p.b + (n0 + min(row, nrows - 1)) * p.ldb + kStPart * wave + 16 * c;
  }
  // x fragment j = 2 kp + h of slab s: row 16 mt + r, k = 1024 s + 128 wave + 64 kp + 16 g + 8 h
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = p.a + min<int64_t>(16 * mt + r, p.M - 1) * p.lda + kStPart * wave + 16 * g;
  // slab s: this wave's W copies into ring slot s % RING, then its x fragments
  vec xf[RING][MT][4];
  auto issue = [&](auto B, int s) __attribute__((always_inline)) {
    constexpr int buf = decltype(B)::value;
    char* dst = ring + buf * (kStRows * kStPart);
#pragma unroll
    for (int q = 0; q < kStCopies; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(wsrc[q] + (int64_t)s * kStSlab),
                                       (lds_void_t*)(dst + q * 1024), 16, 0, kCpolNT);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xf[buf][mt][j] = *(const vec*)(xrow[mt] + (int64_t)s * kStSlab + 64 * (j >> 1) + 8 * (j & 1));
  };
  f32x4_t acc[MT][kStTiles];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < kStTiles; ++t) acc[mt][t] = f32x4_t{};
  // lane (r, g) reads chunk 4 kp + g of row 16 t + r: swizzled by (r >> 1) & 7
  const int rsw = (r >> 1) & 7;
  auto compute = [&](auto B) __attribute__((always_inline)) {
    constexpr int buf = decltype(B)::value;
    const char* wb = ring + buf * (kStRows * kStPart) + r * kStPart;
#pragma unroll
    for (int kp = 0; kp < 2; ++kp)
#pragma unroll
      for (int t = 0; t < kStTiles; ++t) {
        const u32x4_t w16 = *(const u32x4_t*)(wb + t * 16 * kStPart + 16 * ((4 * kp + g) ^ rsw));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const vec wk = widen8<T>(u32x2_t{w16[2 * h], w16[2 * h + 1]});
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[mt][t] = Mfma16<T>::mma(xf[buf][mt][2 * kp + h], wk, acc[mt][t]);
        }
      }
  };
  // slab s has landed once at most the later slabs' loads (each kStCopies W
  // copies and 4 MT x loads, issued together and in slab order) are
  // outstanding; the copies are this wave's own, so no barrier is needed
  constexpr int PER = kStCopies + 4 * MT;
  auto wait_slab = [&](int later) __attribute__((always_inline)) {
    if (RING > 2 && later >= 2) wait_vmcnt<2 * PER>();
    else if (later >= 1) wait_vmcnt<PER>();
    else wait_vmcnt<0>();
  };
  // one slab step: U = s % RING picks the slot (the loop is unrolled by RING)
  auto step = [&](auto U, int s) __attribute__((always_inline)) {
    wait_slab(min(RING - 1, S - 1 - s));
    compute(U);
    if (s + RING < S) issue(U, s + RING);
  };
  static_assert(RING == 2 || RING == 3, "two or three slabs in flight");
  issue(std::integral_constant<int, 0>{}, 0);
  if (S > 1) issue(std::integral_constant<int, 1>{}, 1);
  if constexpr (RING == 3) {
    if (S > 2) issue(std::integral_constant<int, 2>{}, 2);
  }
  auto round = [&](int s) __attribute__((always_inline)) {
    step(std::integral_constant<int, 0>{}, s);
    if (s + 1 < S) step(std::integral_constant<int, 1>{}, s + 1);
    if constexpr (RING == 3) {
      if (s + 2 < S) step(std::integral_constant<int, 2>{}, s + 2);
    }
  };
  if constexpr (SFIX > 0) {
#pragma unroll
    for (int s = 0; s < SFIX; s += RING) round(s);
  } else {
    for (int s = 0; s < S; s += RING) round(s);
  }
  // fixed-order combine of the 8 waves' partial tiles (the rings are free
  // once every wave is done)
  __syncthreads();
  float(*red)[kStTiles][16][17] = (float(*)[kStTiles][16][17])st_lds;
  const bool bias_f32 = p.bias_dtype == MI_F32;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (mt > 0) __syncthreads();
#pragma unroll
    for (int t = 0; t < kStTiles; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][t][4 * g + i][r] = acc[mt][t][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < kStTiles * 256; idx += 64 * kStWaves) {
      const int tt = idx >> 8, tm = (idx >> 4) & 15, tn = idx & 15;
      const int64_t m = mt * 16 + tm;
      if (m >= p.M || 16 * tt + tn >= nrows) continue;
      const int64_t n = n0 + 16 * tt + tn;
      float sum = red[0][tt][tm][tn];
#pragma unroll
      for (int w = 1; w < kStWaves; ++w) sum += red[w][tt][tm][tn];
      float v = p.alpha * p.scale[n] * sum;
      if (HAS_BIAS) {
        const int64_t bo = m * p.bias_sm + n * p.bias_sn;
        v += p.beta * (bias_f32 ? ((const float*)p.bias)[bo]
                                : MfmaOp<T>::load(((const uint16_t*)p.bias)[bo]));
      }
      p.c[m * p.ldc + n] = MfmaOp<T>::store(v);
    }
  }
}

template <typename T, int MT, bool HB, int SFIX>
mi_status_t launch_stream_k(const GemmArgs& q, hipStream_t s, int R) {
  constexpr int RING = MT <= 2 ? 3 : 2;
  static bool attr = [] {
    (void)hipFuncSetAttribute((const void*)int8_stream_kernel<T, MT, RING, HB, SFIX>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, kStLds);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL((int8_stream_kernel<T, MT, RING, HB, SFIX>), dim3((unsigned)ceil_div_u(q.N, R)),
                     dim3(64 * kStWaves), kStLds, s, q, R);
  return check_launch("int8_linear stream");
}

template <typename T, int MT, bool HB>
mi_status_t launch_stream_mt(const GemmArgs& q, hipStream_t s) {
  // rows per block: N / CUs rounded up, at least one tile and at most a slab
  const int64_t cus = std::max(1, cu_count());
  const int R = (int)std::min<int64_t>(kStRows, std::max<int64_t>(16, (q.N + cus - 1) / cus));
  // K = 4096 (a 4096-wide hidden layer) with the slab count fixed
  if (q.K == 4 * kStSlab) return launch_stream_k<T, MT, HB, 4>(q, s, R);
  return launch_stream_k<T, MT, HB, 0>(q, s, R);
}

template <typename T, bool HB>
mi_status_t launch_stream(const GemmArgs& q, hipStream_t s) {
  switch ((int)((q.M + 15) / 16)) {
    case 1: return launch_stream_mt<T, 1, HB>(q, s);
    case 2: return launch_stream_mt<T, 2, HB>(q, s);
    case 3: return launch_stream_mt<T, 3, HB>(q, s);
    default: return launch_stream_mt<T, 4, HB>(q, s);
  }
}

// ---- fp32: VALU tiled kernel (64 x 64 tile, 4 x 4 outputs per lane) ----------------

struct GemmF32Args {
  const float* a;
  const float* b;
  float* c;
  const void* bias;
  int bias_dtype;
  int64_t bias_sm, bias_sn, bias_sb;
  int64_t M, N, K;
  int64_t a_sm, a_sk, b_sk, b_sn, ldc;
  int64_t sa, sb, sc;
  float alpha, beta;
};

template <bool HAS_BIAS>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmF32Args p) {
  __shared__ float As[16][64 + 4];
  __shared__ float Bs[16][64 + 4];
  const int64_t batch = blockIdx.z;
  const float* A = p.a + batch * p.sa;
  const float* B = p.b + batch * p.sb;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < p.K; k0 += 16) {
    for (int v = threadIdx.x; v < 16 * 64; v += 256) {
      const int kk = v / 64, mm = v % 64;
      const int64_t gm = m0 + mm, gk = k0 + kk;
      As[kk][mm] = (gm < p.M && gk < p.K) ? A[gm * p.a_sm + gk * p.a_sk] : 0.f;
      const int64_t gn = n0 + mm;
      Bs[kk][mm] = (gn < p.N && gk < p.K) ? B[gk * p.b_sk + gn * p.b_sn] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  float* C = p.c + batch * p.sc;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n >= p.N) continue;
      float v = p.alpha * acc[i][j];
      if (HAS_BIAS)
        v += p.beta * load_as<float>(p.bias, batch * p.bias_sb + m * p.bias_sm + n * p.bias_sn,
                                     p.bias_dtype);
      C[m * p.ldc + n] = v;
    }
  }
}

// ---- host side --------------------------------------------------------------------

// A batched matrix view: element (b, r, c) at data + b*sb + r*s0 + c*s1.
struct Mat {
  void* data;
  int dtype;
  int64_t batch, rows, cols;
  int64_t sb, s0, s1;
};

mi_status_t as_mat(const mi_tensor_t* t, const char* name, Mat* m) {
  MI_RETURN_IF(validate(t, name));
  if (t->ndim == 2) {
    *m = Mat{t->data, t->dtype, 1, t->sizes[0], t->sizes[1], 0, t->strides[0], t->strides[1]};
  } else if (t->ndim == 3) {
    *m = Mat{t->data, t->dtype, t->sizes[0], t->sizes[1], t->sizes[2],
             t->sizes[0] == 1 ? 0 : t->strides[0], t->strides[1], t->strides[2]};
  } else {
    MI_FAIL(MI_ERR_INVALID, "%s: expected a 2-D or 3-D tensor, got %d dims", name, t->ndim);
  }
  return MI_OK;
}

mi_tensor_t mat_desc(const Mat& m) {
  mi_tensor_t t{};
  t.data = m.data;
  t.dtype = m.dtype;
  t.ndim = 3;
  t.sizes[0] = m.batch;
  t.sizes[1] = m.rows;
  t.sizes[2] = m.cols;
  t.strides[0] = m.sb;
  t.strides[1] = m.s0;
  t.strides[2] = m.s1;
  return t;
}

// Rows of `m` must be contiguous along the columns, 16-byte aligned, with a
// leading dim that keeps every row 16-byte aligned; otherwise `m` is copied
// densely (leading dim rounded up to 16 bytes) into workspace.
mi_status_t dense_rows(Mat& m, Workspace& ws, hipStream_t stream) {
  const int es = dtype_size(m.dtype);
  const int64_t align_el = 16 / es;
  const bool unit = m.s1 == 1 || m.cols == 1;
  const bool ok = unit && (m.rows == 1 || (m.s0 % align_el == 0 && m.s0 >= m.cols)) &&
                  ((uintptr_t)m.data % 16) == 0 && (m.batch == 1 || m.sb % align_el == 0);
  if (ok) {
    if (m.rows == 1) m.s0 = (m.cols + align_el - 1) / align_el * align_el;
    m.s1 = 1;
    return MI_OK;
  }
  const int64_t ld = (m.cols + align_el - 1) / align_el * align_el;
  MI_RETURN_IF(ws.alloc((size_t)(m.batch * m.rows * ld) * es, stream));
  Mat d{ws.get(), m.dtype, m.batch, m.rows, m.cols, m.rows * ld, ld, 1};
  mi_tensor_t dt = mat_desc(d), st = mat_desc(m);
  MI_RETURN_IF(mi_copy(&dt, &st, (mi_stream_t)stream));
  m = d;
  return MI_OK;
}

Mat transposed(const Mat& m) {
  return Mat{m.data, m.dtype, m.batch, m.cols, m.rows, m.sb, m.s1, m.s0};
}

template <typename T, int BM, int BN, int WM, int WN, bool I8, bool HB>
struct Cfg {
  static void* fn() { return (void*)gemm_mfma_kernel<T, BM, BN, WM, WN, I8, HB>; }
  static size_t lds() { return (size_t)2 * (BM + BN) * PITCH * sizeof(uint16_t); }
  static mi_status_t launch(const GemmArgs& q0, int64_t batch, hipStream_t s, const char* what) {
    static bool attr = [] {
      (void)hipFuncSetAttribute(fn(), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds());
      return true;
    }();
    (void)attr;
    GemmArgs q = q0;
    q.tiles_m = (int)((q.M + BM - 1) / BM);
    q.tiles_n = (int)((q.N + BN - 1) / BN);
    dim3 grid((unsigned)(q.tiles_m * q.tiles_n), (unsigned)batch);
    hipLaunchKernelGGL((gemm_mfma_kernel<T, BM, BN, WM, WN, I8, HB>), grid, dim3(64 * WM * WN),
                       lds(), s, q);
    return check_launch(what);
  }
};

// Tile configuration by problem shape: 256 x 256 when there are enough tiles
// to fill the 256 CUs, narrower N tiles for short-M problems.
// The direct-to-LDS kernel needs K % 64 == 0, 16-byte aligned rows and
// per-batch byte offsets that fit 32 bits (lane offsets are 32-bit).
bool dl_eligible(const GemmArgs& q, bool int8) {
  const int bes = int8 ? 1 : 2;  // bytes per B element
  if (q.K % dl::BK != 0 || q.K == 0) return false;
  if (q.lda % 8 != 0 || (q.ldb * bes) % 16 != 0) return false;
  if ((((uintptr_t)q.a) | ((uintptr_t)q.b)) & 15) return false;
  if ((q.sa % 8) != 0 || (q.sb * bes) % 16 != 0) return false;
  if (q.M > 0x7fffffff || q.N > 0x7fffffff || q.K > 0x7fffffff) return false;
  const int64_t amax = (q.M - 1) * q.lda * 2 + q.K * 2,
                bmax = ((q.N - 1) * q.ldb + q.K) * bes;
  return amax < ((int64_t)1 << 32) && bmax < ((int64_t)1 << 32);
}

template <typename T, bool HB, bool I8, bool KN = false>
mi_status_t launch_dl(const GemmArgs& q0, int64_t batch, hipStream_t s, const char* what) {
  constexpr size_t lds = I8 ? dl::LDS_BYTES8 : dl::LDS_BYTES;
  static bool attr = [] {
    (void)hipFuncSetAttribute((const void*)gemm_dl_kernel<T, HB, I8, false, KN>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    return true;
  }();
  (void)attr;
  GemmArgs q = q0;
  q.tiles_m = (int)((q.M + dl::BM - 1) / dl::BM);
  q.tiles_n = (int)((q.N + dl::BN - 1) / dl::BN);
  dim3 grid((unsigned)(q.tiles_m * q.tiles_n), (unsigned)batch);
  hipLaunchKernelGGL((gemm_dl_kernel<T, HB, I8, false, KN>), grid, dim3(dl::NT), lds, s, q,
                     nullptr, (int64_t)0);
  return check_launch(what);
}

// The large-tile kernel with a fused epilogue (EPI_RESID, EPI_SILU): 256 x 256
// tiles over the output, or over 128 output columns (a gate and an up half)
// for EPI_SILU.
template <typename T, int EPI>
mi_status_t launch_dl_epi(const GemmArgs& q0, hipStream_t s, const char* what) {
  constexpr size_t lds = dl::LDS_BYTES;
  static bool attr = [] {
    (void)hipFuncSetAttribute((const void*)gemm_dl_kernel<T, false, false, false, false, EPI>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    return true;
  }();
  (void)attr;
  GemmArgs q = q0;
  const int64_t bn = EPI == EPI_SILU ? dl::BN / 2 : dl::BN;
  q.tiles_m = (int)((q.M + dl::BM - 1) / dl::BM);
  q.tiles_n = (int)((q.N + bn - 1) / bn);
  hipLaunchKernelGGL((gemm_dl_kernel<T, false, false, false, false, EPI>),
                     dim3((unsigned)(q.tiles_m * q.tiles_n)), dim3(dl::NT), lds, s, q, nullptr,
                     (int64_t)0);
  return check_launch(what);
}

// Row-major [K][N] B read in place by the large-tile kernel: enough tiles to
// fill the CUs, K % 64 == 0, 16-byte aligned rows of both operands, N a
// multiple of 8 (whole 16-byte column chunks) and 32-bit lane offsets.
// The transposed fragment reads make the main loop about 9 % slower than
// with K-contiguous B (M8192 N4096 K4096: 0.257 against 0.236 ms), while a
// K-contiguous copy of B costs a fixed 2 K N x 2 bytes at about 6 TB/s
// (16 us there, 0.247 ms in all): in place wins while M x batch <= 4096.
bool dl_kn_eligible(const GemmArgs& q, int64_t batch) {
  if (q.M * batch > 4096) return false;
  const int64_t tiles = ((q.M + dl::BM - 1) / dl::BM) * ((q.N + dl::BN - 1) / dl::BN) * batch;
  if (tiles < cu_count()) return false;
  if (q.K % dl::BK != 0 || q.K == 0 || q.N % 8 != 0 || q.N < 8) return false;
  if (q.lda % 8 != 0 || q.ldb % 8 != 0 || q.ldb < q.N) return false;
  if ((((uintptr_t)q.a) | ((uintptr_t)q.b)) & 15) return false;
  if ((q.sa % 8) != 0 || (q.sb % 8) != 0) return false;
  if (q.M > 0x7fffffff || q.N > 0x7fffffff || q.K > 0x7fffffff) return false;
  const int64_t amax = (q.M - 1) * q.lda * 2 + q.K * 2, bmax = (dl::BK * q.ldb + q.N) * 2;
  return amax < ((int64_t)1 << 32) && bmax < ((int64_t)1 << 32);
}

// ---- split-K over 256 x 256 tiles, for too few tiles to fill the CUs ----------------
//
// The int8 linear at M = 256 has 43 tiles of 256 x 256 for 256 CUs.  With S
// K slices per tile (one block per CU, S = 5 there) each block keeps the
// large tile's low LDS traffic per MFMA, which 128-row tiles over the whole
// K cannot (every CU would copy all of x into LDS); the price is the fp32
// partial sums, written once and read once by the combine (M = 256: 34.5 us
// for the slices, 10.5 us for the combine of 56 MB).
//
// out = alpha * scale[n] * sum_s part[s] + beta * bias, the slices added in
// order s = 0 .. S - 1 (deterministic) and rounded once.  One lane per run
// of 4 columns of a row.
template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(256) void splitk_combine_kernel(GemmArgs p, const float* part, int S,
                                                             int64_t ldp) {
  const int64_t runs = ldp / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t m = idx / runs, n = (idx - m * runs) * 4;
  if (m >= p.M || n >= p.N) return;
  const float* src = part + m * ldp + n;
  const int64_t slice = p.M * ldp;
  f32x4_t acc = *(const f32x4_t*)src;
#pragma unroll 4
  for (int s = 1; s < S; ++s) acc += *(const f32x4_t*)(src + s * slice);
  f32x4_t sc4 = {1.f, 1.f, 1.f, 1.f}, bb4 = {};
  if (p.scale != nullptr) sc4 = load_col4_t<T>(p.scale, MI_F32, n, 1, p.N, 0);
  const bool row_bias = HAS_BIAS && p.bias_sm == 0;
  if (row_bias) bb4 = load_col4_t<T>(p.bias, p.bias_dtype, n, p.bias_sn, p.N, 0);
  u16x4_t v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float x = p.alpha * acc[e] * sc4[e];
    if (HAS_BIAS) {
      float bv = bb4[e];
      if (!row_bias) {
        const int64_t bo = m * p.bias_sm + min<int64_t>(n + e, p.N - 1) * p.bias_sn;
        bv = p.bias_dtype == MI_F32 ? ((const float*)p.bias)[bo]
                                    : MfmaOp<T>::load(((const uint16_t*)p.bias)[bo]);
      }
      x += p.beta * bv;
    }
    v[e] = MfmaOp<T>::store(x);
  }
  uint16_t* dst = p.c + m * p.ldc + n;
  if (n + 3 < p.N && (p.ldc % 4) == 0 && (((uintptr_t)p.c) & 7) == 0) {
    *(u16x4_t*)dst = v;
  } else {
    for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = v[e];
  }
}

// Slices for split-K over 256 x 256 tiles: as many as fill the CUs with one
// block each (at least 2, at most one 64-wide K step per slice); 1 = no split.
int splitk_slices(const GemmArgs& q) {
  const int64_t tiles = ((q.M + dl::BM - 1) / dl::BM) * ((q.N + dl::BN - 1) / dl::BN);
  const int64_t s = std::min<int64_t>(cu_count() / std::max<int64_t>(tiles, 1), q.K / dl::BK);
  return s >= 2 ? (int)std::min<int64_t>(s, 16) : 1;
}

template <typename T, bool HB, bool I8>
mi_status_t launch_splitk(const GemmArgs& q0, int S, hipStream_t s, const char* what) {
  constexpr size_t lds = I8 ? dl::LDS_BYTES8 : dl::LDS_BYTES;
  static bool attr = [] {
    (void)hipFuncSetAttribute((const void*)gemm_dl_kernel<T, false, I8, true>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    return true;
  }();
  (void)attr;
  GemmArgs q = q0;
  q.tiles_m = (int)((q.M + dl::BM - 1) / dl::BM);
  q.tiles_n = (int)((q.N + dl::BN - 1) / dl::BN);
  const int64_t ldp = (q.N + 3) / 4 * 4;
  Workspace wp;
  MI_RETURN_IF(wp.alloc((size_t)S * (size_t)q.M * (size_t)ldp * sizeof(float), s));
  float* part = (float*)wp.get();
  hipLaunchKernelGGL((gemm_dl_kernel<T, false, I8, true>),
                     dim3((unsigned)(q.tiles_m * q.tiles_n), (unsigned)S), dim3(dl::NT), lds, s, q,
                     part, ldp);
  MI_RETURN_IF(check_launch(what));
  const int64_t lanes = q.M * (ldp / 4);
  hipLaunchKernelGGL((splitk_combine_kernel<T, HB>), dim3((unsigned)((lanes + 255) / 256)),
                     dim3(256), 0, s, q, (const float*)part, S, ldp);
  return check_launch(what);
}

template <typename T, bool I8, bool HB>
mi_status_t launch_mfma(const GemmArgs& q, int64_t batch, hipStream_t s, const char* what) {
  const int64_t cus = cu_count();
  // int8 W and 64 < M <= 512 (config 4's M = 256): split-K over 256 x 256
  // tiles when they are too few to fill the CUs (M = 256: 43 tiles x 5 K
  // slices, 43.6 us against 49.9 us for 128-row tiles over the whole K; M =
  // 96 .. 512 all faster), else 128-row tiles sized to the CUs
  if (I8 && batch == 1 && q.M > 64 && q.M <= 4 * mid::BM && dl_eligible(q, true)) {
    const int S = splitk_slices(q);
    if (S > 1) return launch_splitk<T, HB, true>(q, S, s, what);
    return launch_mid<T, HB>(q, s, what);
  }
  const int64_t big = ((q.M + 255) / 256) * ((q.N + 255) / 256) * batch;
  if (big >= cus && dl_eligible(q, I8)) return launch_dl<T, HB, I8>(q, batch, s, what);
  if (big >= cus) return Cfg<T, 256, 256, 2, 4, I8, HB>::launch(q, batch, s, what);
  if (q.M <= 32) return Cfg<T, 32, 64, 1, 2, I8, HB>::launch(q, batch, s, what);
  const int64_t mid = ((q.M + 127) / 128) * ((q.N + 127) / 128) * batch;
  // int8 B (config 4's M = 256: 172 tiles of 128 x 128) runs 128 x 64 tiles:
  // twice the blocks, so CUs hold two and overlap one's loads with the
  // other's MFMAs (about 15 % faster)
  if (mid >= cus / 2 && I8) return Cfg<T, 128, 64, 2, 2, I8, HB>::launch(q, batch, s, what);
  if (mid >= cus / 2) return Cfg<T, 128, 128, 2, 2, I8, HB>::launch(q, batch, s, what);
  return Cfg<T, 128, 64, 2, 2, I8, HB>::launch(q, batch, s, what);
}

template <typename T>
mi_status_t dispatch_mfma(const GemmArgs& q, bool int8, bool has_bias, int64_t batch,
                          hipStream_t s, const char* what) {
  if (int8) {
    if (has_bias) return launch_mfma<T, true, true>(q, batch, s, what);
    return launch_mfma<T, true, false>(q, batch, s, what);
  }
  if (has_bias) return launch_mfma<T, false, true>(q, batch, s, what);
  return launch_mfma<T, false, false>(q, batch, s, what);
}

struct BiasView {
  const void* data = nullptr;
  int dtype = MI_F32;
  int64_t sb = 0, sm = 0, sn = 0;
};

mi_status_t bias_view(const mi_tensor_t* bias, int64_t batch, int64_t M, int64_t N,
                      const char* what, BiasView* bv) {
  MI_RETURN_IF(validate(bias, "bias"));
  MI_CHECK_ARG(bias->ndim <= 3, "%s: bias has too many dims", what);
  int64_t sz[3] = {1, 1, 1}, st[3] = {0, 0, 0};
  const int off = 3 - bias->ndim;
  for (int d = 0; d < bias->ndim; ++d) {
    sz[off + d] = bias->sizes[d];
    st[off + d] = bias->sizes[d] == 1 ? 0 : bias->strides[d];
  }
  MI_CHECK_ARG((sz[0] == 1 || sz[0] == batch) && (sz[1] == 1 || sz[1] == M) &&
                   (sz[2] == 1 || sz[2] == N),
               "%s: bias does not broadcast to the output", what);
  bv->data = bias->data;
  bv->dtype = bias->dtype;
  bv->sb = st[0];
  bv->sm = st[1];
  bv->sn = st[2];
  return MI_OK;
}

// Converts a bias of a dtype the epilogue does not read into a dense fp32
// copy in workspace (same shape, so the broadcast view is unchanged).
mi_status_t bias_to_f32(const mi_tensor_t* bias, Workspace& ws, hipStream_t stream,
                        BiasView* bv) {
  mi_tensor_t dst = *bias;
  MI_RETURN_IF(ws.alloc((size_t)numel(*bias) * 4, stream));
  dst.data = ws.get();
  dst.dtype = MI_F32;
  int64_t s = 1;
  for (int d = dst.ndim - 1; d >= 0; --d) {
    dst.strides[d] = s;
    s *= dst.sizes[d];
  }
  MI_RETURN_IF(mi_copy(&dst, bias, (mi_stream_t)stream));
  int64_t st[3] = {0, 0, 0};
  const int off = 3 - dst.ndim;
  for (int d = 0; d < dst.ndim; ++d) st[off + d] = dst.sizes[d] == 1 ? 0 : dst.strides[d];
  bv->data = ws.get();
  bv->dtype = MI_F32;
  bv->sb = st[0];
  bv->sm = st[1];
  bv->sn = st[2];
  return MI_OK;
}

// out[b] = beta * bias[b] + alpha * a[b] @ b[b]; `wt` (when not NULL) is an
// int8 weight [N, K] with per-N fp32 `scale`, used instead of `b`.
mi_status_t run_gemm(const mi_tensor_t* out, const mi_tensor_t* a, const mi_tensor_t* b,
                     const mi_tensor_t* wt, const mi_tensor_t* scale, const mi_tensor_t* bias,
                     double alpha, double beta, hipStream_t stream, const char* what) {
  clear_error();
  Mat A, B, C;
  const bool int8 = wt != nullptr;
  MI_RETURN_IF(as_mat(a, "mat1", &A));
  if (int8) {
    MI_RETURN_IF(as_mat(wt, "weight", &B));
    MI_CHECK_ARG(B.batch == 1 && wt->ndim == 2, "%s: weight must be 2-D [N, K]", what);
    MI_CHECK_ARG(B.dtype == MI_I8, "%s: weight must be int8", what);
    B = transposed(B);  // [K, N] view of the weight
  } else {
    MI_RETURN_IF(as_mat(b, "mat2", &B));
  }
  MI_RETURN_IF(as_mat(out, "out", &C));
  MI_CHECK_ARG(A.dtype == C.dtype && (int8 || B.dtype == A.dtype),
               "%s: expected operands and out of one dtype, got %s, %s, %s", what,
               dtype_name(A.dtype), dtype_name(B.dtype), dtype_name(C.dtype));
  MI_CHECK_ARG(A.dtype == MI_BF16 || A.dtype == MI_F16 || (A.dtype == MI_F32 && !int8),
               "%s: dtype %s is not supported", what, dtype_name(A.dtype));
  MI_CHECK_ARG(A.cols == B.rows,
               "%s: mat1 and mat2 shapes cannot be multiplied (%lldx%lld and %lldx%lld)", what,
               (long long)A.rows, (long long)A.cols, (long long)B.rows, (long long)B.cols);
  const int64_t batch = std::max(A.batch, std::max(B.batch, C.batch));
  MI_CHECK_ARG((A.batch == batch || A.batch == 1) && (B.batch == batch || B.batch == 1) &&
                   C.batch == batch,
               "%s: batch sizes differ", what);
  MI_CHECK_ARG(C.rows == A.rows && C.cols == B.cols,
               "%s: out has shape %lldx%lld, expected %lldx%lld", what, (long long)C.rows,
               (long long)C.cols, (long long)A.rows, (long long)B.cols);
  MI_CHECK_ARG(batch <= 65535, "%s: batch too large", what);
  if (A.batch == 1) A.sb = 0;
  if (B.batch == 1) B.sb = 0;
  A.batch = B.batch = batch;
  const int64_t M = A.rows, N = B.cols, K = A.cols;
  if (int8) {
    MI_RETURN_IF(validate(scale, "scales"));
    MI_CHECK_ARG(scale->dtype == MI_F32 && numel(*scale) == N && is_contiguous(*scale),
                 "%s: scales must be a dense fp32 vector of %lld elements", what, (long long)N);
  }
  if (M == 0 || N == 0 || batch == 0) return MI_OK;
  const bool has_bias = bias != nullptr && bias->data != nullptr && beta != 0.0;
  BiasView bv;
  Workspace wbias;
  if (has_bias) {
    MI_RETURN_IF(bias_view(bias, batch, M, N, what, &bv));
    if (A.dtype != MI_F32 && bv.dtype != MI_F32 && bv.dtype != A.dtype)
      MI_RETURN_IF(bias_to_f32(bias, wbias, stream, &bv));
  }
  if (K == 0) {
    mi_tensor_t ct = mat_desc(C);
    mi_scalar_t z{};
    z.dtype = MI_F64;
    z.wrapped = 1;
    if (!has_bias) return mi_fill(&ct, z, (mi_stream_t)stream);
    mi_tensor_t bt{};
    bt.data = (void*)bv.data;
    bt.dtype = bv.dtype;
    bt.ndim = 3;
    bt.sizes[0] = batch;
    bt.sizes[1] = M;
    bt.sizes[2] = N;
    bt.strides[0] = bv.sb;
    bt.strides[1] = bv.sm;
    bt.strides[2] = bv.sn;
    mi_scalar_t bs = z;
    bs.f = beta;
    return mi_mul_scalar(&ct, &bt, bs, (mi_stream_t)stream);
  }

  if (A.dtype == MI_F32) {
    MI_CHECK_ARG(C.s1 == 1 || N == 1, "%s: out must have unit column stride", what);
    GemmF32Args q{};
    q.a = (const float*)A.data;
    q.b = (const float*)B.data;
    q.c = (float*)C.data;
    q.bias = bv.data;
    q.bias_dtype = bv.dtype;
    q.bias_sm = bv.sm;
    q.bias_sn = bv.sn;
    q.bias_sb = bv.sb;
    q.M = M;
    q.N = N;
    q.K = K;
    q.a_sm = A.s0;
    q.a_sk = A.s1;
    q.b_sk = B.s0;
    q.b_sn = B.s1;
    q.ldc = C.s0;
    q.sa = A.sb;
    q.sb = B.sb;
    q.sc = C.sb;
    q.alpha = (float)alpha;
    q.beta = (float)beta;
    dim3 grid(ceil_div_u(N, 64), ceil_div_u(M, 64), (unsigned)batch);
    if (has_bias) hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(256), 0, stream, q);
    else hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(256), 0, stream, q);
    return check_launch(what);
  }

  // MFMA path: A as [M, K] rows, B as [N, K] rows (B^T with K contiguous),
  // or B as row-major [K, N] rows read in place by the large-tile kernel
  Workspace wa, wb, wc;
  Mat Bt = transposed(B);
  MI_RETURN_IF(dense_rows(A, wa, stream));
  bool b_kn = false;
  if (!int8 && B.s1 == 1 && N > 1 && Bt.s1 != 1) {
    GemmArgs kq{};
    kq.a = (const uint16_t*)A.data;
    kq.b = B.data;
    kq.M = M;
    kq.N = N;
    kq.K = K;
    kq.lda = A.s0;
    kq.ldb = B.s0;
    kq.sa = A.sb;
    kq.sb = B.sb;
    b_kn = dl_kn_eligible(kq, batch);
  }
  if (!b_kn) MI_RETURN_IF(dense_rows(Bt, wb, stream));
  Mat Cw = C;
  const bool c_ok = (C.s1 == 1 || N == 1) && (C.batch == 1 || C.sb != 0);
  if (!c_ok) {
    MI_RETURN_IF(wc.alloc((size_t)(batch * M * N) * 2, stream));
    Cw = Mat{wc.get(), C.dtype, batch, M, N, M * N, N, 1};
  }
  GemmArgs q{};
  q.a = (const uint16_t*)A.data;
  q.b = Bt.data;
  q.c = (uint16_t*)Cw.data;
  q.bias = bv.data;
  q.scale = int8 ? (const float*)scale->data : nullptr;
  q.bias_dtype = bv.dtype;
  q.bias_sm = bv.sm;
  q.bias_sn = bv.sn;
  q.bias_sb = bv.sb;
  q.M = M;
  q.N = N;
  q.K = K;
  q.lda = A.s0;
  q.ldb = Bt.s0;
  q.ldc = Cw.s0;
  q.sa = A.sb;
  q.sb = Bt.sb;
  q.sc = Cw.sb;
  q.alpha = (float)alpha;
  q.beta = (float)beta;
  if (b_kn) {
    q.b = B.data;
    q.ldb = B.s0;
    q.sb = B.sb;
    mi_status_t st;
    if (A.dtype == MI_BF16)
      st = has_bias ? launch_dl<BF16, true, false, true>(q, batch, stream, what)
                    : launch_dl<BF16, false, false, true>(q, batch, stream, what);
    else
      st = has_bias ? launch_dl<F16, true, false, true>(q, batch, stream, what)
                    : launch_dl<F16, false, false, true>(q, batch, stream, what);
    MI_RETURN_IF(st);
    if (!c_ok) {
      mi_tensor_t dst = mat_desc(C), src = mat_desc(Cw);
      MI_RETURN_IF(mi_copy(&dst, &src, (mi_stream_t)stream));
    }
    return MI_OK;
  }
  // int8 weight with few rows of x: the weight stream dominates
  const bool skinny = int8 && batch == 1 && M <= 64 && K % 128 == 0 && (q.lda % 8) == 0 &&
                      (q.ldb % 16) == 0 && ((((uintptr_t)q.a) | ((uintptr_t)q.b)) & 15) == 0 &&
                      (N == 1 || Cw.s1 == 1);
  // K in whole 1 KiB slabs: the LDS-staged weight stream; else the register one
  const bool stream_ok = skinny && K % kStSlab == 0;
  if (stream_ok) {
    mi_status_t st;
    if (A.dtype == MI_BF16)
      st = has_bias ? launch_stream<BF16, true>(q, stream) : launch_stream<BF16, false>(q, stream);
    else
      st = has_bias ? launch_stream<F16, true>(q, stream) : launch_stream<F16, false>(q, stream);
    MI_RETURN_IF(st);
  } else if (skinny) {
    mi_status_t st;
    if (A.dtype == MI_BF16)
      st = has_bias ? launch_skinny<BF16, true>(q, stream) : launch_skinny<BF16, false>(q, stream);
    else
      st = has_bias ? launch_skinny<F16, true>(q, stream) : launch_skinny<F16, false>(q, stream);
    MI_RETURN_IF(st);
  } else if (A.dtype == MI_BF16) {
    MI_RETURN_IF(dispatch_mfma<BF16>(q, int8, has_bias, batch, stream, what));
  } else {
    MI_RETURN_IF(dispatch_mfma<F16>(q, int8, has_bias, batch, stream, what));
  }
  if (!c_ok) {
    mi_tensor_t dst = mat_desc(C), src = mat_desc(Cw);
    MI_RETURN_IF(mi_copy(&dst, &src, (mi_stream_t)stream));
  }
  return MI_OK;
}

// x [M, K] @ W^T with W [N, K] (a linear layer's weight) and a fused
// epilogue: EPI_RESID adds `aux` (residual [M, N]) to the rounded product,
// EPI_SILU multiplies silu(x Wg^T) by x Wu^T (W = Wg, aux = Wu), each product
// rounded first, as the unfused ops do.  The large-tile kernel takes the whole
// op when it applies (tiles enough to fill the CUs and its alignment and
// 32-bit offset rules); otherwise the products go to workspace through the
// regular matmul and the elementwise op follows, with the same results.
mi_status_t run_linear_epi(int epi, const mi_tensor_t* out, const mi_tensor_t* x,
                           const mi_tensor_t* w, const mi_tensor_t* aux, hipStream_t stream,
                           const char* what) {
  clear_error();
  MI_CHECK_ARG(out && x && w && aux, "%s: NULL descriptor", what);
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(x, "x"));
  MI_RETURN_IF(validate(w, "weight"));
  MI_RETURN_IF(validate(aux, epi == EPI_SILU ? "w_up" : "residual"));
  MI_CHECK_ARG(x->ndim == 2 && w->ndim == 2 && out->ndim == 2 && aux->ndim == 2,
               "%s: x, weights, residual and out must be 2-D", what);
  const int dt = x->dtype;
  MI_CHECK_ARG(dt == MI_BF16 || dt == MI_F16, "%s: dtype %s is not supported", what,
               dtype_name(dt));
  MI_CHECK_ARG(w->dtype == dt && out->dtype == dt && aux->dtype == dt,
               "%s: x, weights, residual and out must share a dtype", what);
  const int64_t M = x->sizes[0], K = x->sizes[1], N = w->sizes[0];
  MI_CHECK_ARG(w->sizes[1] == K, "%s: x has %lld features, the weight expects %lld", what,
               (long long)K, (long long)w->sizes[1]);
  MI_CHECK_ARG(out->sizes[0] == M && out->sizes[1] == N, "%s: out must be [%lld, %lld]", what,
               (long long)M, (long long)N);
  MI_CHECK_ARG(aux->sizes[0] == (epi == EPI_SILU ? N : M) && aux->sizes[1] == (epi == EPI_SILU ? K : N),
               "%s: %s has the wrong shape", what, epi == EPI_SILU ? "w_up" : "residual");
  if (M == 0 || N == 0) return MI_OK;
  // the fused kernel: unit column strides, enough tiles, the dl kernel's rules
  GemmArgs q{};
  q.a = (const uint16_t*)x->data;
  q.b = w->data;
  q.c = (uint16_t*)out->data;
  q.M = M;
  q.N = N;
  q.K = K;
  q.lda = x->strides[0];
  q.ldb = w->strides[0];
  q.ldc = out->strides[0];
  q.alpha = 1.f;
  q.beta = 0.f;
  bool fused = x->strides[1] == 1 && w->strides[1] == 1 && out->strides[1] == 1 &&
               aux->strides[1] == 1 && K > 0 && dl_eligible(q, false);
  if (epi == EPI_SILU) {
    q.b2 = aux->data;
    fused = fused && aux->strides[0] == q.ldb && ((uintptr_t)aux->data & 15) == 0 &&
            ((N - 1) * q.ldb + K) * 2 < ((int64_t)1 << 32);
  } else {
    q.res = (const uint16_t*)aux->data;
    q.ldr = aux->strides[0];
  }
  const int64_t bn = epi == EPI_SILU ? dl::BN / 2 : dl::BN;
  fused = fused && ((M + dl::BM - 1) / dl::BM) * ((N + bn - 1) / bn) >= cu_count();
  if (fused) {
    if (dt == MI_BF16)
      return epi == EPI_SILU ? launch_dl_epi<BF16, EPI_SILU>(q, stream, what)
                             : launch_dl_epi<BF16, EPI_RESID>(q, stream, what);
    return epi == EPI_SILU ? launch_dl_epi<F16, EPI_SILU>(q, stream, what)
                           : launch_dl_epi<F16, EPI_RESID>(q, stream, what);
  }
  // unfused: the product(s) into workspace, then the elementwise op
  auto wt = [](const mi_tensor_t* t) {  // [K, N] view of a [N, K] weight
    mi_tensor_t v = *t;
    v.sizes[0] = t->sizes[1];
    v.sizes[1] = t->sizes[0];
    v.strides[0] = t->strides[1];
    v.strides[1] = t->strides[0];
    return v;
  };
  mi_tensor_t tmp{};
  tmp.dtype = dt;
  tmp.ndim = 2;
  tmp.sizes[0] = M;
  tmp.sizes[1] = N;
  tmp.strides[0] = N;
  tmp.strides[1] = 1;
  Workspace w1, w2;
  MI_RETURN_IF(w1.alloc((size_t)(M * N) * 2, stream));
  tmp.data = w1.get();
  const mi_tensor_t wv = wt(w);
  MI_RETURN_IF(run_gemm(&tmp, x, &wv, nullptr, nullptr, nullptr, 1.0, 0.0, stream, what));
  if (epi == EPI_RESID) {
    mi_scalar_t one{};
    one.dtype = MI_F64;
    one.f = 1.0;
    one.i = 1;
    one.wrapped = 1;
    return mi_add(out, aux, &tmp, one, (mi_stream_t)stream);
  }
  mi_tensor_t tmp2 = tmp;
  MI_RETURN_IF(w2.alloc((size_t)(M * N) * 2, stream));
  tmp2.data = w2.get();
  const mi_tensor_t uv = wt(aux);
  MI_RETURN_IF(run_gemm(&tmp2, x, &uv, nullptr, nullptr, nullptr, 1.0, 0.0, stream, what));
  return mi_silu_mul(out, &tmp, &tmp2, (mi_stream_t)stream);
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

mi_status_t mi_addmm(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* mat1,
                     const mi_tensor_t* mat2, double beta, double alpha, mi_stream_t stream) {
  return run_gemm(out, mat1, mat2, nullptr, nullptr, self, alpha, beta, (hipStream_t)stream,
                  "addmm");
}

mi_status_t mi_mm(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* mat2,
                  mi_stream_t stream) {
  return run_gemm(out, self, mat2, nullptr, nullptr, nullptr, 1.0, 0.0, (hipStream_t)stream, "mm");
}

mi_status_t mi_bmm(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* mat2,
                   mi_stream_t stream) {
  clear_error();
  MI_CHECK_ARG(self && mat2 && out, "bmm: NULL descriptor");
  MI_CHECK_ARG(self->ndim == 3 && mat2->ndim == 3 && out->ndim == 3, "bmm: expected 3-D tensors");
  MI_CHECK_ARG(self->sizes[0] == mat2->sizes[0], "bmm: batch sizes differ");
  return run_gemm(out, self, mat2, nullptr, nullptr, nullptr, 1.0, 0.0, (hipStream_t)stream, "bmm");
}

mi_status_t mi_baddbmm(const mi_tensor_t* out, const mi_tensor_t* self, const mi_tensor_t* batch1,
                       const mi_tensor_t* batch2, double beta, double alpha, mi_stream_t stream) {
  return run_gemm(out, batch1, batch2, nullptr, nullptr, self, alpha, beta, (hipStream_t)stream,
                  "baddbmm");
}

mi_status_t mi_linear_residual(const mi_tensor_t* out, const mi_tensor_t* x,
                               const mi_tensor_t* weight, const mi_tensor_t* residual,
                               mi_stream_t stream) {
  return run_linear_epi(EPI_RESID, out, x, weight, residual, (hipStream_t)stream,
                        "linear_residual");
}

mi_status_t mi_linear_silu_mul(const mi_tensor_t* out, const mi_tensor_t* x,
                               const mi_tensor_t* w_gate, const mi_tensor_t* w_up,
                               mi_stream_t stream) {
  return run_linear_epi(EPI_SILU, out, x, w_gate, w_up, (hipStream_t)stream, "linear_silu_mul");
}

mi_status_t mi_int8_linear(const mi_tensor_t* out, const mi_tensor_t* x, const mi_tensor_t* weight,
                           const mi_tensor_t* scales, const mi_tensor_t* bias, mi_stream_t stream) {
  clear_error();
  MI_CHECK_ARG(out && x && weight && scales, "int8_linear: NULL descriptor");
  MI_CHECK_ARG(x->ndim == 2 && out->ndim == 2, "int8_linear: x and out must be 2-D");
  return run_gemm(out, x, nullptr, weight, scales, bias, 1.0, 1.0, (hipStream_t)stream,
                  "int8_linear");
}

}  // extern "C"
