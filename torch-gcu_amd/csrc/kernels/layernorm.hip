// native_layer_norm (forward, at the end of this file) and
// native_layer_norm_backward over the last N elements (normalized_shape
// flattened): with xh = (x - mean) * rstd and gw = dy * gamma (dy without a
// weight), per row
//   dx = rstd * (gw - sum(gw) / N - xh * sum(gw * xh) / N)
// and per column, over all M rows,
//   dgamma = sum(dy * xh)      dbeta = sum(dy)
// all in fp32 (ATen's LayerNormBackwardKernelImpl,
// aten/src/ATen/native/cpu/layer_norm_kernel.cpp, is the same arithmetic in
// the form a*dy*gamma + b*x + c).  mean and rstd may be fp32 or the input's
// dtype, gamma fp32 or the input's dtype.
//
// HBM-bound.  Fused path (dense rows, N <= 2048 16-byte vectors, aligned):
// a block walks up to kLnRows rows, every G-th one of G blocks (fewer rows
// on short inputs, so that every CU gets a block; more if there would be
// over kLnMaxParts blocks), RS at a time with the next step's loads in flight while it reduces
// the current one, and one block reduction per step; each lane owns the same
// column vectors in every row, so gamma stays in registers and the dgamma /
// dbeta column sums over the block's rows accumulate in registers.  Per row:
// one read of dy and x, two block sums, one write of dx.  The block's column
// partials go to workspace (one row of 2N floats per block) and a finish pass
// adds them in a fixed order.  Other shapes: one block per row for dx (two
// reads of the row) and a column-partial pass for dgamma / dbeta.
#include "iter.h"

namespace mi {
namespace {

constexpr int kLnBlock = 256;
constexpr int kLnRows = 64;       // rows per block (at most, unless over kLnMaxParts), fused path
constexpr int kLnMinRows = 16;    // rows per block (at least), fused path
constexpr int kLnMaxVpl = 4;      // 16-byte vectors per lane and row (512 lanes), fused path
constexpr int kLnColRows = 64;    // rows per partial (at least), column pass
constexpr int64_t kLnMaxParts = 2048;  // partial rows: at most 2048 x 2N floats
constexpr int kLnFwdRows = 16;         // rows per block, forward

struct LnArgs {
  void* dx;
  const void* dy;
  const void* x;
  const void* mean;
  const void* rstd;
  const void* gamma;
  float* part;  // [nparts, 2, N]: dgamma partials, then dbeta partials
  int64_t M, N;
  int64_t rows_per_part;  // rows summed into one partial row
  int mean_dt, gamma_dt;
  int need_dx, need_dw, need_db;
};

__device__ __forceinline__ float2 block_sum2(float a, float b, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  a = wave_sum(a);
  b = wave_sum(b);
  if (lane == 0) {
    red[2 * wid] = a;
    red[2 * wid + 1] = b;
  }
  __syncthreads();
  float ra = red[0], rb = red[1];
#pragma unroll
  for (int w = 1; w < kLnBlock / 64; ++w) {
    ra += red[2 * w];
    rb += red[2 * w + 1];
  }
  __syncthreads();
  return make_float2(ra, rb);
}

// The sums of RS rows at once: one pair of barriers for all of them.
template <int RS, int NT>
__device__ __forceinline__ void block_sums(float (&s1)[RS], float (&s2)[RS], float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < RS; ++q) {
    s1[q] = wave_sum(s1[q]);
    s2[q] = wave_sum(s2[q]);
  }
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < RS; ++q) {
      red[(2 * q) * (NT / 64) + wid] = s1[q];
      red[(2 * q + 1) * (NT / 64) + wid] = s2[q];
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < RS; ++q) {
    float a = red[(2 * q) * (NT / 64)], b = red[(2 * q + 1) * (NT / 64)];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) {
      a += red[(2 * q) * (NT / 64) + w];
      b += red[(2 * q + 1) * (NT / 64) + w];
    }
    s1[q] = a;
    s2[q] = b;
  }
  __syncthreads();
}

// The same with one barrier: the caller alternates between two halves of
// `red` (2 * RS * NT / 64 floats each) on consecutive steps, so a half is
// written again only after the next step's barrier, which every wave reaches
// after it has read this step's sums.
template <int RS, int NT>
__device__ __forceinline__ void block_sums1(float (&s1)[RS], float (&s2)[RS], float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < RS; ++q) {
    s1[q] = wave_sum(s1[q]);
    s2[q] = wave_sum(s2[q]);
  }
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < RS; ++q) {
      red[(2 * q) * (NT / 64) + wid] = s1[q];
      red[(2 * q + 1) * (NT / 64) + wid] = s2[q];
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < RS; ++q) {
    float a = red[(2 * q) * (NT / 64)], b = red[(2 * q + 1) * (NT / 64)];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) {
      a += red[(2 * q) * (NT / 64) + w];
      b += red[(2 * q + 1) * (NT / 64) + w];
    }
    s1[q] = a;
    s2[q] = b;
  }
}

// RS rows per step: their loads are all in flight together (RS * 2 * VPL
// 16-byte loads per lane) and their sums share one block reduction.  The
// next step's rows are loaded before this step is reduced (two register
// buffers; past the block's last row the prefetch re-reads that row, which
// is never used).  Every load is unconditional (row and column indices
// clamped, guards only on the arithmetic and the stores), so the compiler's
// waits count only the loads of the step being consumed.  MF32: mean and
// rstd are fp32, else the input's dtype.
template <typename Tag, int VPL, int RS, int NT, bool MF32>
__global__ __launch_bounds__(NT) void ln_bwd_fused_kernel(LnArgs a) {
  typedef typename Num<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  union V {
    uint4 u;
    St s[VEC];
  };
  union P {  // VEC fp32 values
    uint4 u[VEC / 4];
    float f[VEC];
  };
  struct Rows {
    V vd[RS][VPL], vx[RS][VPL];
    float mu[RS], rs[RS];
  };
  constexpr int RED = 2 * RS * NT / 64;  // one half of the sums' LDS (block_sums1)
  __shared__ float red[2 * RED];
  const int64_t nv = a.N / VEC;
  const float invN = 1.0f / (float)a.N;
  float gam[VPL][VEC], pw[VPL][VEC], pb[VPL][VEC];
  {
    // gamma pieces: one 16-byte load per vector (input dtype) or VEC / 4 (fp32)
    const bool g32 = a.gamma != nullptr && a.gamma_dt == MI_F32;
    const bool g16 = a.gamma != nullptr && a.gamma_dt != MI_F32;
    V gv[VPL];
    P gf[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int64_t v = min<int64_t>(threadIdx.x + (int64_t)k * NT, nv - 1);
      if (g32) {
#pragma unroll
        for (int w = 0; w < VEC / 4; ++w) gf[k].u[w] = ((const uint4*)((const float*)a.gamma + v * VEC))[w];
      } else if (g16) {
        gv[k] = ((const V*)a.gamma)[v];
      }
    }
#pragma unroll
    for (int k = 0; k < VPL; ++k)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        gam[k][e] = g32 ? gf[k].f[e] : (g16 ? Num<Tag>::load(gv[k].s[e]) : 1.0f);
        pw[k][e] = 0.f;
        pb[k][e] = 0.f;
      }
  }
  // block b takes rows b, b + G, b + 2 G, ... (G blocks; step i of r1): at
  // any moment the blocks stream G consecutive rows, where contiguous
  // 64-row bands per block kept G separate DRAM streams 512 KiB apart open
  // per tensor (81.5 -> 77.4 us on bf16 [16384, 4096])
  const int64_t r0 = 0, r1 = (a.M - (int64_t)blockIdx.x + gridDim.x - 1) / gridDim.x;
  auto row_of = [&](int64_t i) { return (int64_t)blockIdx.x + i * (int64_t)gridDim.x; };
  auto issue = [&](Rows& b, int64_t rb) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < RS; ++q) {
      const int64_t r = row_of(min<int64_t>(rb + q, r1 - 1));
      const V* pdy = (const V*)((const St*)a.dy + r * a.N);
      const V* px = (const V*)((const St*)a.x + r * a.N);
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const int64_t v = min<int64_t>(threadIdx.x + (int64_t)k * NT, nv - 1);
        b.vd[q][k] = ld_stream(pdy + v);
        b.vx[q][k] = ld_stream(px + v);
      }
      if constexpr (MF32) {
        b.mu[q] = ((const float*)a.mean)[r];
        b.rs[q] = ((const float*)a.rstd)[r];
      } else {
        b.mu[q] = Num<Tag>::load(((const St*)a.mean)[r]);
        b.rs[q] = Num<Tag>::load(((const St*)a.rstd)[r]);
      }
    }
  };
  auto consume = [&](const Rows& b, int64_t rb, int half) __attribute__((always_inline)) {
    float s1[RS], s2[RS];
    // x-hat (one FMA: x rstd - mean rstd) and dy * gamma of every element,
    // kept in registers for dx (computing them again there, and dx as
    // rstd (g - m1 - x m2), took 185 VALU a row against 140: 83.6 -> 81.4 us
    // on bf16 [16384, 4096])
    float xh[RS][VPL][VEC], gw[RS][VPL][VEC];
#pragma unroll
    for (int q = 0; q < RS; ++q) {
      s1[q] = 0.f;
      s2[q] = 0.f;
      const float nmr = -b.mu[q] * b.rs[q];
      const bool live = rb + q < r1;
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const bool on = live && threadIdx.x + (int64_t)k * NT < nv;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float dy = Num<Tag>::load(b.vd[q][k].s[e]);
          const float x = __builtin_fmaf(Num<Tag>::load(b.vx[q][k].s[e]), b.rs[q], nmr);
          const float g = dy * gam[k][e];
          xh[q][k][e] = x;
          gw[q][k][e] = g;
          if (on) {
            s1[q] += g;
            s2[q] = __builtin_fmaf(g, x, s2[q]);
            pw[k][e] = __builtin_fmaf(dy, x, pw[k][e]);
            pb[k][e] += dy;
          }
        }
      }
    }
    if (a.need_dx) {
      block_sums1<RS, NT>(s1, s2, red + half * RED);
#pragma unroll
      for (int q = 0; q < RS; ++q) {
        const int64_t r = row_of(rb + q);
        if (rb + q < r1) {
          // dx = rstd (g - m1 - x m2) = g rstd + c0 + x c1
          const float rsq = b.rs[q];
          const float c0 = -s1[q] * invN * rsq, c1 = -s2[q] * invN * rsq;
          V* pdx = (V*)((St*)a.dx + r * a.N);
#pragma unroll
          for (int k = 0; k < VPL; ++k) {
            const int64_t v = threadIdx.x + (int64_t)k * NT;
            if (v < nv) {
              V o;
#pragma unroll
              for (int e = 0; e < VEC; ++e)
                o.s[e] = Num<Tag>::store(__builtin_fmaf(xh[q][k][e], c1, __builtin_fmaf(gw[q][k][e], rsq, c0)));
              st_stream(pdx + v, o);
            }
          }
        }
      }
    }
  };
  Rows A, B;
  issue(A, r0);
  for (int64_t rb = r0;;) {
    issue(B, rb + RS);
    consume(A, rb, 0);
    rb += RS;
    if (rb >= r1) break;
    issue(A, rb + RS);
    consume(B, rb, 1);
    rb += RS;
    if (rb >= r1) break;
  }
  if (a.need_dw || a.need_db) {
    float* pwr = a.part + (int64_t)blockIdx.x * 2 * a.N;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int64_t v = threadIdx.x + (int64_t)k * NT;
      if (v < nv) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          pwr[v * VEC + e] = pw[k][e];
          pwr[a.N + v * VEC + e] = pb[k][e];
        }
      }
    }
  }
}

// dx of one row per block, any N (the row is read twice).
template <typename Tag>
__global__ __launch_bounds__(kLnBlock) void ln_bwd_row_kernel(LnArgs a) {
  typedef typename Num<Tag>::storage St;
  __shared__ float red[2 * kLnBlock / 64];
  const int64_t r = blockIdx.x;
  const St* dy = (const St*)a.dy + r * a.N;
  const St* x = (const St*)a.x + r * a.N;
  const float mu = load_as<float>(a.mean, r, a.mean_dt);
  const float rs = load_as<float>(a.rstd, r, a.mean_dt);
  float s1 = 0.f, s2 = 0.f;
  for (int64_t j = threadIdx.x; j < a.N; j += kLnBlock) {
    const float g = a.gamma != nullptr ? load_as<float>(a.gamma, j, a.gamma_dt) : 1.0f;
    const float gw = Num<Tag>::load(dy[j]) * g;
    s1 += gw;
    s2 += gw * (Num<Tag>::load(x[j]) - mu) * rs;
  }
  const float2 s = block_sum2(s1, s2, red);
  const float m1 = s.x / (float)a.N, m2 = s.y / (float)a.N;
  St* dx = (St*)a.dx + r * a.N;
  for (int64_t j = threadIdx.x; j < a.N; j += kLnBlock) {
    const float g = a.gamma != nullptr ? load_as<float>(a.gamma, j, a.gamma_dt) : 1.0f;
    const float xh = (Num<Tag>::load(x[j]) - mu) * rs;
    dx[j] = Num<Tag>::store(rs * (Num<Tag>::load(dy[j]) * g - m1 - xh * m2));
  }
}

// Column partials for dgamma / dbeta: block (cx, p) sums rows_per_part rows
// starting at p * rows_per_part for 256 columns.
template <typename Tag>
__global__ __launch_bounds__(kLnBlock) void ln_bwd_col_kernel(LnArgs a) {
  typedef typename Num<Tag>::storage St;
  const int64_t j = (int64_t)blockIdx.x * kLnBlock + threadIdx.x;
  const int64_t p = blockIdx.y;
  if (j >= a.N) return;
  const int64_t r0 = p * a.rows_per_part;
  const int64_t r1 = r0 + a.rows_per_part < a.M ? r0 + a.rows_per_part : a.M;
  float sw = 0.f, sb = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float dy = Num<Tag>::load(((const St*)a.dy)[r * a.N + j]);
    const float xh = (Num<Tag>::load(((const St*)a.x)[r * a.N + j]) -
                      load_as<float>(a.mean, r, a.mean_dt)) *
                     load_as<float>(a.rstd, r, a.mean_dt);
    sw += dy * xh;
    sb += dy;
  }
  a.part[p * 2 * a.N + j] = sw;
  a.part[p * 2 * a.N + a.N + j] = sb;
}

// dgamma / dbeta from the partial rows (2N floats each: dgamma columns, then
// dbeta columns), in a fixed order.  A block owns 32 columns (8 lanes x 4)
// and 32 groups of consecutive partial rows, one 8-lane group each; a group
// loads its rows kFinBatch at a time (clamped, unconditional: all in flight)
// and adds them in row order, and the groups' sums are added in group order
// through LDS.  The 2N / 32 blocks spread the partials over every CU (on
// [16384, 4096], 256 blocks for 256 partial rows: 3.7 us, against 4.7 us for
// 32 blocks of 256 columns with 16 waves down the rows).
constexpr int kFinGroups = 32, kFinBatch = 8;

__global__ __launch_bounds__(256) void ln_bwd_finish_kernel(const float* __restrict__ part,
                                                            int64_t nparts, int64_t N, void* dw,
                                                            int dw_dt, void* db, int db_dt) {
  __shared__ float red[kFinGroups][4][8];
  const int l = threadIdx.x & 7, g = threadIdx.x >> 3;
  const int64_t W = 2 * N;
  const int64_t c = (int64_t)blockIdx.x * 32 + l * 4;
  const int64_t per = (nparts + kFinGroups - 1) / kFinGroups;
  const int64_t p0 = g * per, p1 = p0 + per < nparts ? p0 + per : nparts;
  float sum[4] = {0.f, 0.f, 0.f, 0.f};
  if (c < W && p0 < p1) {
    if (W % 4 == 0) {
      // c is a multiple of 4 below W: the 4 columns are in the row, 16-byte aligned
      for (int64_t q0 = p0; q0 < p1; q0 += kFinBatch) {
        float4 v[kFinBatch];
#pragma unroll
        for (int i = 0; i < kFinBatch; ++i) {
          const int64_t p = q0 + i < p1 ? q0 + i : p1 - 1;
          v[i] = *(const float4*)(part + p * W + c);
        }
#pragma unroll
        for (int i = 0; i < kFinBatch; ++i)
          if (q0 + i < p1) {
            sum[0] += v[i].x;
            sum[1] += v[i].y;
            sum[2] += v[i].z;
            sum[3] += v[i].w;
          }
      }
    } else {
      for (int e = 0; e < 4 && c + e < W; ++e)
        for (int64_t p = p0; p < p1; ++p) sum[e] += part[p * W + c + e];
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) red[g][e][l] = sum[e];
  __syncthreads();
  if (g == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t j = c + e;
      if (j >= W) break;
      float t = red[0][e][l];
#pragma unroll
      for (int k = 1; k < kFinGroups; ++k) t += red[k][e][l];
      if (j < N) {
        if (dw != nullptr) store_as<float>(dw, j, dw_dt, t);
      } else if (db != nullptr) {
        store_as<float>(db, j - N, db_dt, t);
      }
    }
  }
}

template <typename Tag>
mi_status_t launch_ln_bwd(LnArgs& a, void* dw, int dw_dt, void* db, int db_dt,
                          hipStream_t stream) {
  typedef typename Num<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  const bool cols = a.need_dw || a.need_db;
  const uintptr_t bits = (uintptr_t)a.dy | (uintptr_t)a.x | (uintptr_t)a.dx | (uintptr_t)a.gamma;
  const int64_t nv = a.N / VEC;
  const bool fused = a.N % VEC == 0 && bits % 16 == 0 && nv <= (int64_t)512 * kLnMaxVpl;
  const bool mf32 = a.mean_dt == MI_F32;
  Workspace ws;
  int64_t nparts = 0;
  if (fused) {
    // one block per CU while there are rows enough (kLnRows rows a block),
    // fewer rows a block (at least kLnMinRows) to reach every CU on short inputs
    const int64_t cus = cu_count();
    a.rows_per_part = std::max<int64_t>(kLnMinRows, std::min<int64_t>(kLnRows, (a.M + cus - 1) / cus));
    if ((a.M + a.rows_per_part - 1) / a.rows_per_part > kLnMaxParts)
      a.rows_per_part = (a.M + kLnMaxParts - 1) / kLnMaxParts;
    const int64_t blocks = (a.M + a.rows_per_part - 1) / a.rows_per_part;
    if (cols) {
      nparts = blocks;
      MI_RETURN_IF(ws.alloc((size_t)(nparts * 2 * a.N) * sizeof(float), stream));
      a.part = (float*)ws.get();
    }
    auto go = [&](auto vpl_c, auto rs_c, auto nt_c) -> mi_status_t {
      constexpr int VPL = decltype(vpl_c)::value;
      constexpr int RS = decltype(rs_c)::value;
      constexpr int NT = decltype(nt_c)::value;
      if (mf32)
        hipLaunchKernelGGL((ln_bwd_fused_kernel<Tag, VPL, RS, NT, true>), dim3((unsigned)blocks),
                           dim3(NT), 0, stream, a);
      else
        hipLaunchKernelGGL((ln_bwd_fused_kernel<Tag, VPL, RS, NT, false>), dim3((unsigned)blocks),
                           dim3(NT), 0, stream, a);
      return check_launch("layer_norm_backward");
    };
    // measured on bf16 [16384, 4096] with the prefetching kernel: 64 rows a
    // block (one block per CU), one row a step: 78 us + 5.6 us finish
    // (86 us in all, 4.7 TB/s); two rows a step 89 us, 32 rows a block 95 us,
    // 48 or 96 rows a block (blocks not a multiple of the CUs) 110 us
    typedef std::integral_constant<int, 1> I1;
    typedef std::integral_constant<int, 2> I2;
    typedef std::integral_constant<int, 4> I4;
    typedef std::integral_constant<int, 256> T256;
    typedef std::integral_constant<int, 512> T512;
    if (nv <= 256) MI_RETURN_IF(go(I1(), I2(), T256()));
    else if (nv <= 512) MI_RETURN_IF(go(I1(), I1(), T512()));
    else if (nv <= 1024) MI_RETURN_IF(go(I2(), I2(), T512()));
    else MI_RETURN_IF(go(I4(), I1(), T512()));
  } else {
    if (a.need_dx) {
      MI_CHECK_ARG(a.M <= 0x7fffffffLL, "layer_norm_backward: too many rows");
      hipLaunchKernelGGL((ln_bwd_row_kernel<Tag>), dim3((unsigned)a.M), dim3(kLnBlock), 0, stream,
                         a);
      MI_RETURN_IF(check_launch("layer_norm_backward rows"));
    }
    if (cols) {
      a.rows_per_part = kLnColRows;
      if ((a.M + kLnColRows - 1) / kLnColRows > kLnMaxParts)
        a.rows_per_part = (a.M + kLnMaxParts - 1) / kLnMaxParts;
      nparts = (a.M + a.rows_per_part - 1) / a.rows_per_part;
      MI_RETURN_IF(ws.alloc((size_t)(nparts * 2 * a.N) * sizeof(float), stream));
      a.part = (float*)ws.get();
      hipLaunchKernelGGL((ln_bwd_col_kernel<Tag>), dim3(ceil_div_u(a.N, kLnBlock), (unsigned)nparts),
                         dim3(kLnBlock), 0, stream, a);
      MI_RETURN_IF(check_launch("layer_norm_backward columns"));
    }
  }
  if (cols) {
    hipLaunchKernelGGL(ln_bwd_finish_kernel, dim3(ceil_div_u(2 * a.N, 32)), dim3(256), 0, stream,
                       (const float*)a.part, nparts, a.N, dw, dw_dt, db, db_dt);
    MI_RETURN_IF(check_launch("layer_norm_backward finish"));
  }
  return MI_OK;
}

// ---- forward -------------------------------------------------------------------
// out = (x - mean) * rstd * gamma + beta over rows of N, mean and
// rstd = 1 / sqrt(var + eps) (biased variance, two passes over the row held
// in registers) in fp32, stored in mean_dt; out uses the unrounded fp32 values
// (ATen's LayerNormKernelImpl does the same with y = x * scale + shift,
// aten/src/ATen/native/cpu/layer_norm_kernel.cpp).  Rows of up to 1024
// 16-byte vectors: one wave per row; up to 2048: kLnFwdRows rows per 512-lane
// block; longer or unaligned rows take one block each and are read three
// times.
struct LnFwdArgs {
  void* out;
  void* mean;
  void* rstd;
  const void* x;
  const void* gamma;
  const void* beta;
  int64_t M, N;
  float eps;
  int mean_dt, gamma_dt, beta_dt;
};

// NT lanes own fixed 16-byte column pieces of every row: gamma and beta are
// read once per block into registers; rows go RS at a time (their loads in
// flight together, their sums in one block reduction, two per step: the
// mean, then the squared deviations).
template <typename Tag, int VPL, int RS, int NT>
__global__ __launch_bounds__(NT) void ln_fwd_reg_kernel(LnFwdArgs a) {
  typedef typename Num<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  union V {
    uint4 u;
    St s[VEC];
  };
  __shared__ float red[2 * RS * NT / 64];
  const int64_t nv = a.N / VEC;
  const float invN = 1.0f / (float)a.N;
  float gam[VPL][VEC], bet[VPL][VEC];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int64_t v = threadIdx.x + (int64_t)k * NT;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      gam[k][e] = (a.gamma != nullptr && v < nv) ? load_as<float>(a.gamma, v * VEC + e, a.gamma_dt) : 1.0f;
      bet[k][e] = (a.beta != nullptr && v < nv) ? load_as<float>(a.beta, v * VEC + e, a.beta_dt) : 0.0f;
    }
  }
  const int64_t r0 = (int64_t)blockIdx.x * kLnFwdRows;
  const int64_t r1 = r0 + kLnFwdRows < a.M ? r0 + kLnFwdRows : a.M;
  for (int64_t rb = r0; rb < r1; rb += RS) {
    V vx[RS][VPL];
    float s1[RS], s2[RS];
#pragma unroll
    for (int q = 0; q < RS; ++q) {
      s1[q] = 0.f;
      s2[q] = 0.f;
      if (rb + q < r1) {
        const V* px = (const V*)((const St*)a.x + (rb + q) * a.N);
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
          const int64_t v = threadIdx.x + (int64_t)k * NT;
          if (v < nv) vx[q][k] = ld_stream(px + v);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < RS; ++q)
      if (rb + q < r1)
#pragma unroll
        for (int k = 0; k < VPL; ++k)
          if (threadIdx.x + (int64_t)k * NT < nv)
#pragma unroll
            for (int e = 0; e < VEC; ++e) s1[q] += Num<Tag>::load(vx[q][k].s[e]);
    block_sums<RS, NT>(s1, s2, red);
    float mu[RS];
#pragma unroll
    for (int q = 0; q < RS; ++q) {
      mu[q] = s1[q] * invN;
      s1[q] = 0.f;
      s2[q] = 0.f;
      if (rb + q < r1)
#pragma unroll
        for (int k = 0; k < VPL; ++k)
          if (threadIdx.x + (int64_t)k * NT < nv)
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              const float d = Num<Tag>::load(vx[q][k].s[e]) - mu[q];
              s1[q] += d * d;
            }
    }
    block_sums<RS, NT>(s1, s2, red);
#pragma unroll
    for (int q = 0; q < RS; ++q) {
      const int64_t r = rb + q;
      if (r < r1) {
        const float rs = 1.0f / sqrtf(s1[q] * invN + a.eps);
        V* po = (V*)((St*)a.out + r * a.N);
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
          const int64_t v = threadIdx.x + (int64_t)k * NT;
          if (v < nv) {
            V o;
#pragma unroll
            for (int e = 0; e < VEC; ++e)
              o.s[e] = Num<Tag>::store((Num<Tag>::load(vx[q][k].s[e]) - mu[q]) * rs * gam[k][e] +
                                       bet[k][e]);
            st_stream(po + v, o);
          }
        }
        if (threadIdx.x == 0) {
          store_as<float>(a.mean, r, a.mean_dt, mu[q]);
          store_as<float>(a.rstd, r, a.mean_dt, rs);
        }
      }
    }
  }
}

template <typename Tag>
__global__ __launch_bounds__(kLnBlock) void ln_fwd_row_kernel(LnFwdArgs a) {
  typedef typename Num<Tag>::storage St;
  __shared__ float red[2 * kLnBlock / 64];
  const int64_t r = blockIdx.x;
  const St* x = (const St*)a.x + r * a.N;
  float s = 0.f;
  for (int64_t j = threadIdx.x; j < a.N; j += kLnBlock) s += Num<Tag>::load(x[j]);
  const float mu = block_sum2(s, 0.f, red).x / (float)a.N;
  float q = 0.f;
  for (int64_t j = threadIdx.x; j < a.N; j += kLnBlock) {
    const float d = Num<Tag>::load(x[j]) - mu;
    q += d * d;
  }
  const float rs = 1.0f / sqrtf(block_sum2(q, 0.f, red).x / (float)a.N + a.eps);
  St* o = (St*)a.out + r * a.N;
  for (int64_t j = threadIdx.x; j < a.N; j += kLnBlock) {
    float y = (Num<Tag>::load(x[j]) - mu) * rs;
    if (a.gamma != nullptr) y *= load_as<float>(a.gamma, j, a.gamma_dt);
    if (a.beta != nullptr) y += load_as<float>(a.beta, j, a.beta_dt);
    o[j] = Num<Tag>::store(y);
  }
  if (threadIdx.x == 0) {
    store_as<float>(a.mean, r, a.mean_dt, mu);
    store_as<float>(a.rstd, r, a.mean_dt, rs);
  }
}

// One wave per row (four rows per 256-lane block): the row in registers,
// both sums by wave shuffles, no block barrier; gamma / beta pieces read per
// row (they stay in L2).  WF32: the parameters are fp32 (mixed type).
// Every load of the row is issued before the first sum: with the sum inside
// the guarded load loop each load waited for the one before it (a quarter
// slower on [16384, 4096] bf16).  A wave that keeps the parameters in
// registers and walks 2 or 4 rows, loading the next row before reducing the
// current one, measured 40-65 % slower, and 8 rows no faster than one.
// LDSP: the block first copies gamma and beta into LDS (dynamic, 2 nv PW
// 16-byte words) and the waves read their pieces from there: read per row
// from L2, each piece's loads were waited for in turn (bf16 [16384, 4096]:
// 51.8 -> 47.5 us in a harness; walking 2-8 rows a wave over the staged copy
// was no faster than one).
template <typename Tag, int VPL, bool WF32, bool LDSP>
__global__ __launch_bounds__(256) void ln_fwd_wave_kernel(LnFwdArgs a) {
  typedef typename Num<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  union V {
    uint4 u;
    St s[VEC];
  };
  union P {  // VEC fp32 parameters
    uint4 u[VEC / 4];
    float f[VEC];
  };
  constexpr int PW = WF32 ? VEC / 4 : 1;  // 16-byte words per piece per parameter
  extern __shared__ uint4 prm[];            // LDSP: gamma's words, then beta's
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t nv = a.N / VEC;
  const bool has_g = a.gamma != nullptr, has_b = a.beta != nullptr;
  if constexpr (LDSP) {
    for (int64_t i = threadIdx.x; i < nv * PW; i += 256) {
      prm[i] = has_g ? ((const uint4*)a.gamma)[i] : uint4{0, 0, 0, 0};
      prm[nv * PW + i] = has_b ? ((const uint4*)a.beta)[i] : uint4{0, 0, 0, 0};
    }
    __syncthreads();
  }
  if (row >= a.M) return;
  const V* px = (const V*)((const St*)a.x + row * a.N);
  V v[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int64_t i = lane + (int64_t)k * 64;
    if (i < nv) v[k] = ld_stream(px + i);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k)
    if (lane + (int64_t)k * 64 < nv)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += Num<Tag>::load(v[k].s[e]);
  const float mu = wave_sum(s) / (float)a.N;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k)
    if (lane + (int64_t)k * 64 < nv)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = Num<Tag>::load(v[k].s[e]) - mu;
        q += d * d;
      }
  const float rs = 1.0f / sqrtf(wave_sum(q) / (float)a.N + a.eps);
  V* po = (V*)((St*)a.out + row * a.N);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int64_t i = lane + (int64_t)k * 64;
    if (i < nv) {
      float g[VEC], b[VEC];
      if constexpr (LDSP) {
        P pg, pb;
#pragma unroll
        for (int w = 0; w < PW; ++w) {
          pg.u[w] = prm[i * PW + w];
          pb.u[w] = prm[nv * PW + i * PW + w];
        }
        if constexpr (WF32) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            g[e] = has_g ? pg.f[e] : 1.0f;
            b[e] = pb.f[e];
          }
        } else {
          V vg, vb;
          vg.u = pg.u[0];
          vb.u = pb.u[0];
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            g[e] = has_g ? Num<Tag>::load(vg.s[e]) : 1.0f;
            b[e] = Num<Tag>::load(vb.s[e]);
          }
        }
      } else if (has_g) {
        if constexpr (WF32) {
          P pg;
#pragma unroll
          for (int w = 0; w < VEC / 4; ++w) pg.u[w] = ((const uint4*)((const float*)a.gamma + i * VEC))[w];
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] = pg.f[e];
        } else {
          const V pg = ((const V*)a.gamma)[i];
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] = Num<Tag>::load(pg.s[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = 1.0f;
      }
      if constexpr (!LDSP) {
        if (has_b) {
          if constexpr (WF32) {
            P pb;
#pragma unroll
            for (int w = 0; w < VEC / 4; ++w) pb.u[w] = ((const uint4*)((const float*)a.beta + i * VEC))[w];
#pragma unroll
            for (int e = 0; e < VEC; ++e) b[e] = pb.f[e];
          } else {
            const V pb = ((const V*)a.beta)[i];
#pragma unroll
            for (int e = 0; e < VEC; ++e) b[e] = Num<Tag>::load(pb.s[e]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) b[e] = 0.0f;
        }
      }
      V o;
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        o.s[e] = Num<Tag>::store((Num<Tag>::load(v[k].s[e]) - mu) * rs * g[e] + b[e]);
      st_stream(po + i, o);
    }
  }
  if (lane == 0) {
    store_as<float>(a.mean, row, a.mean_dt, mu);
    store_as<float>(a.rstd, row, a.mean_dt, rs);
  }
}

template <typename Tag>
mi_status_t launch_ln_fwd(const LnFwdArgs& a, hipStream_t stream) {
  typedef typename Num<Tag>::storage St;
  constexpr int VEC = 16 / sizeof(St);
  const int64_t nv = a.N / VEC;
  MI_CHECK_ARG(a.M <= 0x7fffffffLL, "layer_norm: too many rows");
  const bool reg = a.N % VEC == 0 && (((uintptr_t)a.x | (uintptr_t)a.out) % 16) == 0 &&
                   nv <= (int64_t)512 * 4;
  // parameters of one dtype (both fp32, or both the input's) for the wave kernel
  const int pdt = a.gamma != nullptr ? a.gamma_dt : (a.beta != nullptr ? a.beta_dt : -1);
  const bool params_ok = (a.gamma == nullptr || a.gamma_dt == pdt) &&
                          (a.beta == nullptr || a.beta_dt == pdt) &&
                          ((((uintptr_t)a.gamma | (uintptr_t)a.beta) % 16) == 0);
  if (reg && params_ok && nv <= 64 * 16 && (a.M + 3) / 4 <= 0x7fffffffLL) {
    const bool wf32 = pdt == MI_F32 && !std::is_same<Tag, float>::value;
    const unsigned grid = (unsigned)((a.M + 3) / 4);
    // parameters staged in LDS up to 32 KiB a block (more would cost occupancy)
    const size_t lds = (size_t)2 * nv * (wf32 ? VEC / 4 : 1) * 16;
    const bool ldsp = lds <= 32 * 1024;
    auto go = [&](auto vpl_c) -> mi_status_t {
      constexpr int VPL = decltype(vpl_c)::value;
      if (ldsp) {
        if (wf32)
          hipLaunchKernelGGL((ln_fwd_wave_kernel<Tag, VPL, true, true>), dim3(grid), dim3(256), lds,
                             stream, a);
        else
          hipLaunchKernelGGL((ln_fwd_wave_kernel<Tag, VPL, false, true>), dim3(grid), dim3(256),
                             lds, stream, a);
      } else if (wf32) {
        hipLaunchKernelGGL((ln_fwd_wave_kernel<Tag, VPL, true, false>), dim3(grid), dim3(256), 0,
                           stream, a);
      } else {
        hipLaunchKernelGGL((ln_fwd_wave_kernel<Tag, VPL, false, false>), dim3(grid), dim3(256), 0,
                           stream, a);
      }
      return check_launch("layer_norm");
    };
    if (nv <= 64) return go(std::integral_constant<int, 1>());
    if (nv <= 128) return go(std::integral_constant<int, 2>());
    if (nv <= 256) return go(std::integral_constant<int, 4>());
    if (nv <= 512) return go(std::integral_constant<int, 8>());
    return go(std::integral_constant<int, 16>());
  }
  if (reg) {
    const unsigned blocks = (unsigned)((a.M + kLnFwdRows - 1) / kLnFwdRows);
    if (nv <= 256)
      hipLaunchKernelGGL((ln_fwd_reg_kernel<Tag, 1, 2, 256>), dim3(blocks), dim3(256), 0, stream, a);
    else if (nv <= 512)
      hipLaunchKernelGGL((ln_fwd_reg_kernel<Tag, 1, 2, 512>), dim3(blocks), dim3(512), 0, stream, a);
    else if (nv <= 1024)
      hipLaunchKernelGGL((ln_fwd_reg_kernel<Tag, 2, 2, 512>), dim3(blocks), dim3(512), 0, stream, a);
    else
      hipLaunchKernelGGL((ln_fwd_reg_kernel<Tag, 4, 1, 512>), dim3(blocks), dim3(512), 0, stream, a);
    return check_launch("layer_norm");
  }
  hipLaunchKernelGGL((ln_fwd_row_kernel<Tag>), dim3((unsigned)a.M), dim3(kLnBlock), 0, stream, a);
  return check_launch("layer_norm rows");
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" mi_status_t mi_layer_norm(const mi_tensor_t* out, const mi_tensor_t* mean,
                                     const mi_tensor_t* rstd, const mi_tensor_t* input,
                                     const mi_tensor_t* weight, const mi_tensor_t* bias,
                                     int64_t normalized_numel, double eps, mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(out, "out"));
  MI_RETURN_IF(validate(mean, "mean"));
  MI_RETURN_IF(validate(rstd, "rstd"));
  MI_RETURN_IF(validate(input, "input"));
  const int dt = input->dtype;
  MI_CHECK_ARG(dt == MI_F32 || dt == MI_BF16 || dt == MI_F16, "layer_norm: input dtype %s unsupported",
               dtype_name(dt));
  MI_CHECK_ARG(out->dtype == dt && is_contiguous(*out) && is_contiguous(*input) &&
                   numel(*out) == numel(*input),
               "layer_norm: input and out must be contiguous, of one dtype and size");
  const int64_t total = numel(*input), N = normalized_numel;
  MI_CHECK_ARG(N >= 1 && total % N == 0, "layer_norm: %lld elements do not form rows of %lld",
               (long long)total, (long long)N);
  const int64_t M = total / N;
  MI_CHECK_ARG(numel(*mean) == M && numel(*rstd) == M && is_contiguous(*mean) &&
                   is_contiguous(*rstd) && mean->dtype == rstd->dtype &&
                   (mean->dtype == dt || mean->dtype == MI_F32),
               "layer_norm: mean and rstd must be contiguous with %lld elements, fp32 or the input's "
               "dtype", (long long)M);
  LnFwdArgs a{};
  for (int i = 0; i < 2; ++i) {
    const mi_tensor_t* p = i == 0 ? weight : bias;
    if (p != nullptr && p->data != nullptr) {
      MI_RETURN_IF(validate(p, i == 0 ? "weight" : "bias"));
      MI_CHECK_ARG(numel(*p) == N && is_contiguous(*p) && (p->dtype == dt || p->dtype == MI_F32),
                   "layer_norm: weight and bias must be contiguous with %lld elements of the input's "
                   "dtype or fp32", (long long)N);
      if (i == 0) {
        a.gamma = p->data;
        a.gamma_dt = p->dtype;
      } else {
        a.beta = p->data;
        a.beta_dt = p->dtype;
      }
    }
  }
  if (total == 0) return MI_OK;
  a.out = out->data;
  a.mean = mean->data;
  a.rstd = rstd->data;
  a.x = input->data;
  a.M = M;
  a.N = N;
  a.eps = (float)eps;
  a.mean_dt = mean->dtype;
  switch (dt) {
    case MI_BF16: return launch_ln_fwd<BF16>(a, stream);
    case MI_F16: return launch_ln_fwd<F16>(a, stream);
    default: return launch_ln_fwd<float>(a, stream);
  }
}

extern "C" mi_status_t mi_layer_norm_backward(
    const mi_tensor_t* grad_input, const mi_tensor_t* grad_weight, const mi_tensor_t* grad_bias,
    const mi_tensor_t* grad_out, const mi_tensor_t* input, const mi_tensor_t* mean,
    const mi_tensor_t* rstd, const mi_tensor_t* weight, int64_t normalized_numel,
    mi_stream_t stream_) {
  clear_error();
  hipStream_t stream = (hipStream_t)stream_;
  MI_RETURN_IF(validate(grad_out, "grad_out"));
  MI_RETURN_IF(validate(input, "input"));
  MI_RETURN_IF(validate(mean, "mean"));
  MI_RETURN_IF(validate(rstd, "rstd"));
  const int dt = input->dtype;
  MI_CHECK_ARG(dt == MI_F32 || dt == MI_BF16 || dt == MI_F16,
               "layer_norm_backward: input dtype %s unsupported", dtype_name(dt));
  MI_CHECK_ARG(grad_out->dtype == dt, "layer_norm_backward: grad_out must have input's dtype");
  MI_CHECK_ARG(is_contiguous(*input) && is_contiguous(*grad_out),
               "layer_norm_backward: input and grad_out must be contiguous");
  const int64_t total = numel(*input);
  MI_CHECK_ARG(numel(*grad_out) == total, "layer_norm_backward: grad_out size mismatch");
  const int64_t N = normalized_numel;
  MI_CHECK_ARG(N >= 1 && total % N == 0, "layer_norm_backward: %lld elements do not form rows of %lld",
               (long long)total, (long long)N);
  const int64_t M = total / N;
  MI_CHECK_ARG(numel(*mean) == M && numel(*rstd) == M && is_contiguous(*mean) && is_contiguous(*rstd),
               "layer_norm_backward: mean and rstd must be contiguous with %lld elements", (long long)M);
  MI_CHECK_ARG(mean->dtype == rstd->dtype && (mean->dtype == MI_F32 || mean->dtype == dt),
               "layer_norm_backward: mean and rstd must be fp32 or the input's dtype");
  const bool has_w = weight != nullptr && weight->data != nullptr;
  if (has_w) {
    MI_RETURN_IF(validate(weight, "weight"));
    MI_CHECK_ARG(numel(*weight) == N && is_contiguous(*weight) &&
                     (weight->dtype == dt || weight->dtype == MI_F32),
                 "layer_norm_backward: weight must be contiguous with %lld elements of the input's "
                 "dtype or fp32", (long long)N);
  }
  const bool need_dx = grad_input != nullptr && grad_input->data != nullptr;
  const bool need_dw = grad_weight != nullptr && grad_weight->data != nullptr;
  const bool need_db = grad_bias != nullptr && grad_bias->data != nullptr;
  if (need_dx) {
    MI_RETURN_IF(validate(grad_input, "grad_input"));
    MI_CHECK_ARG(grad_input->dtype == dt && numel(*grad_input) == total && is_contiguous(*grad_input),
                 "layer_norm_backward: grad_input must be contiguous like input");
  }
  if (need_dw) {
    MI_RETURN_IF(validate(grad_weight, "grad_weight"));
    MI_CHECK_ARG(numel(*grad_weight) == N && is_contiguous(*grad_weight) &&
                     (grad_weight->dtype == MI_F32 || grad_weight->dtype == MI_BF16 ||
                      grad_weight->dtype == MI_F16),
                 "layer_norm_backward: grad_weight must be contiguous with %lld elements", (long long)N);
  }
  if (need_db) {
    MI_RETURN_IF(validate(grad_bias, "grad_bias"));
    MI_CHECK_ARG(numel(*grad_bias) == N && is_contiguous(*grad_bias) &&
                     (grad_bias->dtype == MI_F32 || grad_bias->dtype == MI_BF16 ||
                      grad_bias->dtype == MI_F16),
                 "layer_norm_backward: grad_bias must be contiguous with %lld elements", (long long)N);
  }
  if (total == 0) {
    // no rows: dgamma and dbeta are zero
    if (need_dw && N > 0) MI_RETURN_IF(mi_fill(grad_weight, mi_scalar_t{0.0, 0, MI_F32, 1}, stream_));
    if (need_db && N > 0) MI_RETURN_IF(mi_fill(grad_bias, mi_scalar_t{0.0, 0, MI_F32, 1}, stream_));
    return MI_OK;
  }
  if (!need_dx && !need_dw && !need_db) return MI_OK;
  LnArgs a{};
  a.dx = need_dx ? grad_input->data : nullptr;
  a.dy = grad_out->data;
  a.x = input->data;
  a.mean = mean->data;
  a.rstd = rstd->data;
  a.gamma = has_w ? weight->data : nullptr;
  a.M = M;
  a.N = N;
  a.mean_dt = mean->dtype;
  a.gamma_dt = has_w ? weight->dtype : MI_F32;
  a.need_dx = need_dx;
  a.need_dw = need_dw;
  a.need_db = need_db;
  void* dw = need_dw ? grad_weight->data : nullptr;
  void* db = need_db ? grad_bias->data : nullptr;
  const int dw_dt = need_dw ? grad_weight->dtype : MI_F32;
  const int db_dt = need_db ? grad_bias->dtype : MI_F32;
  switch (dt) {
    case MI_BF16: return launch_ln_bwd<BF16>(a, dw, dw_dt, db, db_dt, stream);
    case MI_F16: return launch_ln_bwd<F16>(a, dw, dw_dt, db, db_dt, stream);
    default: return launch_ln_bwd<float>(a, dw, dw_dt, db, db_dt, stream);
  }
}
