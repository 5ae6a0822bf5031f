// Fused causal depthwise convolution + SiLU (the Mamba conv section), forward and backward:
//
//   p_t  = bias + sum_{k<K} w_k xbuf_{t-(K-1)+k},   xbuf_s = x_s (s >= 0), tail_{K-1+s} (s < 0)
//   out_t = p_t sigmoid(p_t)
//
// per channel d, over x [B, L, D] read through arbitrary element strides (the reference passes
// the strided in_proj chunk view), tail [B, D, K-1] the carried causal left context.
// Reference semantics: tsfast/models/architectures/mamba/conv_triton.py:59-263 (kernels and
// ops, tail gradient at :241-250) and the eager path mamba/core.py:38-58.
//
// No recurrence, so the layout is chosen for memory-level parallelism, per I/O type:
//  * fp32: a thread owns 4 channels (one 16-byte vector per row) and a run of steps, and keeps
//    the whole run plus its K-1 step halo in registers, loaded before the arithmetic.
//  * bf16: a 16-byte vector holds 8 channels, too many for register tiles, so a workgroup owns
//    256 consecutive channels (one per thread) of one batch row over a segment of kSeg steps.
//    Row tiles are moved into LDS with 16-byte vector loads (element loads for layouts without
//    aligned rows), and the next tile's loads are in flight while the current tile is computed.
//    Each thread walks its channel's column with K-step rolling windows in registers (tile rows
//    are a multiple of K, so ring slots are compile-time), so its registers hold only the windows,
//    taps and partial sums and many waves stay resident.
// fwd reads x and writes out; bwd reads x and gy and writes gx, recomputing p (cheaper than
// storing it), forming gx from the K-step window of pre-activation gradients, and accumulating
// grad-w / grad-bias per 128 steps, summed over (batch, segment) by a second kernel in a fixed
// order (deterministic).
#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

#ifndef TSF_CONV_SEG
#define TSF_CONV_SEG 128
#endif
#ifndef TSF_CONV_FWD_TM
#define TSF_CONV_FWD_TM 2
#endif
#ifndef TSF_CONV_BWD_TM
#define TSF_CONV_BWD_TM 1
#endif
constexpr int kCh = 256;           // channels per workgroup, one per thread
constexpr int kSeg = TSF_CONV_SEG;  // steps per workgroup segment (one grad-w / grad-bias partial each)

template <typename TIO>
TSF_DEV TIO zero_io();
template <>
TSF_DEV float zero_io<float>() {
  return 0.0f;
}
template <>
TSF_DEV bf16 zero_io<bf16>() {
  bf16 r;
  r.bits = 0;
  return r;
}

// Rows per LDS tile: a multiple of K near 16, so that a step's ring slot (stream row mod K) is
// the same compile-time value in every tile.
template <int K>
struct Tile {
  static constexpr int TR = K * ((16 + K - 1) / K);
};

// One 16-byte piece of a tile row (VE elements).
template <typename TIO>
struct alignas(16) Piece {
  static constexpr int VE = 16 / sizeof(TIO);
  TIO v[VE];
};

// A tile of TR rows x kCh channels of one tensor, staged through registers: thread t handles
// pieces e = t + q * kCh (row e / PPR, piece e % PPR). Rows outside [0, L) and channels past D
// read as zero. VECL: rows are 16-byte aligned runs (channel stride 1, D a multiple of VE), so a
// piece is one vector load; otherwise its elements are loaded one by one.
template <typename TIO, int TR>
struct TileRegs2 {
  static constexpr int VE = Piece<TIO>::VE;
  static constexpr int PPR = kCh / VE;  // pieces per row
  static constexpr int NQ = (TR * PPR + kCh - 1) / kCh;
  Piece<TIO> r[NQ];
};

// Issue the loads of stream rows [s0, s0 + TR) (sequence rows; row s at base + s * sl + c * sc for
// channel c) into the staging registers.
template <typename TIO, int TR, bool VECL>
TSF_DEV void tile_issue(TileRegs2<TIO, TR>& rg, const TIO* __restrict__ base, int64_t s0, int64_t L, int64_t c0,
                        int64_t D, int64_t sl, int64_t sc) {
  using R = TileRegs2<TIO, TR>;
#pragma unroll
  for (int q = 0; q < R::NQ; ++q) {
    const int e = threadIdx.x + q * kCh;
    const int row = e / R::PPR, pc = e % R::PPR;
    const int64_t srow = s0 + row, c = c0 + (int64_t)pc * R::VE;
    const bool rok = e < TR * R::PPR && srow >= 0 && srow < L;
    if (VECL) {
      if (rok && c < D) {
        rg.r[q] = ld32(reinterpret_cast<const Piece<TIO>*>(base), (uint32_t)((srow * sl + c) / R::VE));
      } else {
#pragma unroll
        for (int v = 0; v < R::VE; ++v) rg.r[q].v[v] = zero_io<TIO>();
      }
    } else {
#pragma unroll
      for (int v = 0; v < R::VE; ++v)
        rg.r[q].v[v] = (rok && c + v < D) ? ld32(base, (uint32_t)(srow * sl + (c + v) * sc)) : zero_io<TIO>();
    }
  }
}

template <typename TIO, int TR>
TSF_DEV void tile_commit(const TileRegs2<TIO, TR>& rg, TIO (*tile)[kCh]) {
  using R = TileRegs2<TIO, TR>;
#pragma unroll
  for (int q = 0; q < R::NQ; ++q) {
    const int e = threadIdx.x + q * kCh;
    if (e < TR * R::PPR) *reinterpret_cast<Piece<TIO>*>(&tile[e / R::PPR][(e % R::PPR) * R::VE]) = rg.r[q];
  }
}

// Store tile rows r (r0 <= r < r1) as sequence rows s0 + r of a contiguous [*, L, D] row source
// (dst = its batch row), channels past D skipped; the same piece mapping as tile_issue.
template <typename TIO, int TR, bool VECL>
TSF_DEV void tile_store(TIO (*tile)[kCh], TIO* __restrict__ dst, int64_t s0, int r0, int r1, int64_t c0, int64_t D) {
  using R = TileRegs2<TIO, TR>;
#pragma unroll
  for (int q = 0; q < R::NQ; ++q) {
    const int e = threadIdx.x + q * kCh;
    const int row = e / R::PPR, pc = e % R::PPR;
    const int64_t c = c0 + (int64_t)pc * R::VE;
    if (e < TR * R::PPR && row >= r0 && row < r1) {
      const Piece<TIO> v = *reinterpret_cast<const Piece<TIO>*>(&tile[row][pc * R::VE]);
      const int64_t o = (s0 + row) * D + c;
      if (VECL) {
        if (c < D) st32(reinterpret_cast<Piece<TIO>*>(dst), (uint32_t)(o / R::VE), v);
      } else {
#pragma unroll
        for (int u = 0; u < R::VE; ++u)
          if (c + u < D) st32(dst, (uint32_t)(o + u), v.v[u]);
      }
    }
  }
}

TSF_DEV float silu_f(float p) { return p * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-p * kLog2e)); }

// xbuf_s of channel d for s < 0 (the carried tail, zero without one) or s >= 0 (x).
template <typename TIO, int K>
TSF_DEV float xbuf_at(const TIO* __restrict__ xrow, const TIO* __restrict__ tail, int64_t b, int64_t s, int64_t d,
                      int64_t L, int64_t D, int64_t sxl, int64_t sxd) {
  if (s >= 0) return s < L ? to_f32(ld32(xrow, (uint32_t)(s * sxl + d * sxd))) : 0.0f;
  return tail ? to_f32(tail[(b * D + d) * (K - 1) + (K - 1 + s)]) : 0.0f;
}

// Workgroup coordinates from a one-dimensional grid of nx * ny * B workgroups (x fastest, then
// y, then the batch row, the order a three-dimensional grid dispatches in), so that neither the
// batch nor the segment count is bounded by a grid dimension's 65535 limit.
struct Wg3 {
  int64_t x, y, z;
};
TSF_DEV Wg3 wg3(uint32_t nx, uint32_t ny) {
  const uint32_t lin = blockIdx.x;
  const uint32_t r = lin / nx;
  return {(int64_t)(lin - r * nx), (int64_t)(r % ny), (int64_t)(r / ny)};
}

// ------------------------------------------------------------------------------------ forward
template <typename TIO, int K, bool VECL>
__global__ void __launch_bounds__(kCh) conv_silu_fwd_kernel(const TIO* __restrict__ x, const TIO* __restrict__ tail,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ bias, TIO* __restrict__ out,
                                                            int64_t L, int64_t D, int64_t sxb, int64_t sxl,
                                                            int64_t sxd, uint32_t nx, uint32_t ny) {
  constexpr int TR = TSF_CONV_FWD_TM * Tile<K>::TR;  // one input tile only: more rows between barriers
  __shared__ __align__(16) TIO s_x[TR][kCh];
  const int tid = threadIdx.x;
  const Wg3 wg = wg3(nx, ny);
  const int64_t c0 = wg.x * kCh, d = c0 + tid, b = wg.z;
  const int64_t t0 = wg.y * kSeg;
  const bool live = d < D;
  const int64_t nrow = (L - t0) < kSeg ? (L - t0) : kSeg;  // stream rows: the segment's steps
  const TIO* xrow = x + b * sxb;
  float wk[K], xr[K], bv = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    wk[k] = live ? w[d * K + k] : 0.0f;
    xr[k] = 0.0f;
  }
  if (live && bias) bv = bias[d];
  // ring slot of stream row j is j mod K; rows -(K-1) .. -1 take slots 1 .. K-1
#pragma unroll
  for (int k = 1; k < K; ++k)
    if (live) xr[k] = xbuf_at<TIO, K>(xrow, tail, b, t0 - K + k, d, L, D, sxl, sxd);
  TIO* orow = out + b * L * D;
  TileRegs2<TIO, TR> rg;
  tile_issue<TIO, TR, VECL>(rg, xrow, t0, L, c0, D, sxl, sxd);
  const bool all_live = c0 + kCh <= D;  // uniform over the workgroup
  for (int64_t jb = 0; jb < nrow; jb += TR) {
    __syncthreads();
    tile_commit<TIO, TR>(rg, s_x);
    __syncthreads();
    if (jb + TR < nrow) tile_issue<TIO, TR, VECL>(rg, xrow, t0 + jb + TR, L, c0, D, sxl, sxd);
    if (all_live && jb + TR <= nrow) {
      // a whole tile of a fully live workgroup: no per-step exit or store mask. Groups of K steps
      // (TR is a multiple of K, so a step's ring slot is its place in the group) in a loop that is
      // not unrolled: unrolled over the whole tile, the compiler hoisted the later steps' reads
      // and offsets (130 VGPRs against 51)
      const uint32_t o0 = (uint32_t)((t0 + jb) * D + d);
#pragma unroll 1
      for (int i0 = 0; i0 < TR; i0 += K) {
#pragma unroll
        for (int r = 0; r < K; ++r) {
          xr[r] = to_f32(s_x[i0 + r][tid]);
          float p = bv;
#pragma unroll
          for (int k = 0; k < K; ++k) p = fmaf(wk[k], xr[(r + 1 + k) % K], p);
          st32(orow, o0 + (uint32_t)((i0 + r) * D), from_f32<TIO>(silu_f(p)));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TR; ++i) {
        if (jb + i >= nrow) break;  // uniform over the workgroup
        xr[i % K] = to_f32(s_x[i][tid]);
        float p = bv;
#pragma unroll
        for (int k = 0; k < K; ++k) p = fmaf(wk[k], xr[(i + 1 + k) % K], p);
        if (live) st32(orow, (uint32_t)((t0 + jb + i) * D + d), from_f32<TIO>(silu_f(p)));
      }
    }
  }
}

// ----------------------------------------------------------------------------------- backward
// gpre_t = gy_t silu'(p_t); gx_t = sum_k w_k gpre_{t+K-1-k}; grad w_k = sum_t gpre_t
// xbuf_{t-(K-1)+k}; grad bias = sum_t gpre_t; grad tail_j = sum_{t<=j} gpre_t w_{j-t}.
// A segment streams rows t0 .. t0+kSeg+K-2 (the last K-1 give the gpre that its own last gx
// rows need); gx of row j - (K-1) is formed once gpre_j is known. One partial row per (batch,
// segment): part [B, nseg, D, K+1] (K taps, then the bias term).
template <typename TIO, int K, bool VECL>
__global__ void __launch_bounds__(kCh) conv_silu_bwd_kernel(
    const TIO* __restrict__ x, const TIO* __restrict__ tail, const float* __restrict__ w,
    const float* __restrict__ bias, const TIO* __restrict__ gy, TIO* __restrict__ gx, TIO* __restrict__ gtail,
    float* __restrict__ part, int64_t L, int64_t D, int64_t sxb, int64_t sxl, int64_t sxd, uint32_t nx,
    uint32_t ny) {
  constexpr int TR = TSF_CONV_BWD_TM * Tile<K>::TR;
  constexpr int KP = K + 1;
  __shared__ __align__(16) TIO s_x[TR][kCh];
  __shared__ __align__(16) TIO s_g[TR][kCh];
  const int tid = threadIdx.x;
  const Wg3 wg = wg3(nx, ny);
  const int64_t c0 = wg.x * kCh, d = c0 + tid, b = wg.z;
  const int64_t t0 = wg.y * kSeg;
  const bool live = d < D;
  const int64_t own = (L - t0) < kSeg ? (L - t0) : kSeg;  // the segment's own steps
  const int64_t nrow = own + K - 1;                        // stream rows, with the right halo
  const TIO* xrow = x + b * sxb;
  const TIO* gyrow = gy + b * L * D;
  TIO* gxrow = gx + b * L * D;
  float wk[K], xr[K], gr[K], acc[KP], bv = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    wk[k] = live ? w[d * K + k] : 0.0f;
    xr[k] = 0.0f;
    gr[k] = 0.0f;
  }
#pragma unroll
  for (int k = 0; k < KP; ++k) acc[k] = 0.0f;
  if (live && bias) bv = bias[d];
#pragma unroll
  for (int k = 1; k < K; ++k)
    if (live) xr[k] = xbuf_at<TIO, K>(xrow, tail, b, t0 - K + k, d, L, D, sxl, sxd);
  TileRegs2<TIO, TR> rx, rgy;
  tile_issue<TIO, TR, VECL>(rx, xrow, t0, L, c0, D, sxl, sxd);
  tile_issue<TIO, TR, VECL>(rgy, gyrow, t0, L, c0, D, D, 1);
  for (int64_t jb = 0; jb < nrow; jb += TR) {
    __syncthreads();
    tile_commit<TIO, TR>(rx, s_x);
    tile_commit<TIO, TR>(rgy, s_g);
    __syncthreads();
    if (jb + TR < nrow) {
      tile_issue<TIO, TR, VECL>(rx, xrow, t0 + jb + TR, L, c0, D, sxl, sxd);
      tile_issue<TIO, TR, VECL>(rgy, gyrow, t0 + jb + TR, L, c0, D, D, 1);
    }
#pragma unroll
    for (int i = 0; i < TR; ++i) {
      const int64_t j = jb + i;  // stream row; sequence row t0 + j
      if (j >= nrow) break;      // uniform over the workgroup
      xr[i % K] = to_f32(s_x[i][tid]);
      float p = bv;
#pragma unroll
      for (int k = 0; k < K; ++k) p = fmaf(wk[k], xr[(i + 1 + k) % K], p);
      const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-p * kLog2e));
      const float gp = to_f32(s_g[i][tid]) * (sg * fmaf(p, 1.0f - sg, 1.0f));  // zero past L (gy = 0)
      gr[i % K] = gp;
      if (j < own) {
#pragma unroll
        for (int k = 0; k < K; ++k) acc[k] = fmaf(gp, xr[(i + 1 + k) % K], acc[k]);
        acc[K] += gp;
      }
      {
        // gx of sequence row t0 + j - (K-1) replaces gy in tile row i (stored below)
        float g = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) g = fmaf(wk[k], gr[(i - k + K) % K], g);
        s_g[i][tid] = from_f32<TIO>(g);
      }
      // the carried tail feeds the first K-1 outputs: once gpre_0 .. gpre_{K-2} are known
      if (t0 == 0 && j == K - 2 && gtail && live) {
#pragma unroll
        for (int jj = 0; jj < K - 1; ++jj) {
          float g = 0.0f;
#pragma unroll
          for (int t = 0; t <= jj; ++t) g = fmaf(gr[t], wk[jj - t], g);  // gpre_t in slot t (t < K)
          gtail[(b * D + d) * (K - 1) + jj] = from_f32<TIO>(g);
        }
      }
    }
    // tile row i holds gx of sequence row t0 + jb + i - (K-1): store those in [t0, t0 + own)
    __syncthreads();
    {
      const int64_t lo = (K - 1) - jb, hi = own + (K - 1) - jb;
      const int r0 = lo > 0 ? (int)lo : 0, r1 = hi < TR ? (int)(hi > 0 ? hi : 0) : TR;
      tile_store<TIO, TR, VECL>(s_g, gxrow, t0 + jb - (K - 1), r0, r1, c0, D);
    }
  }
  if (live) {
    float* pr = part + ((b * ny + wg.y) * D + d) * KP;
#pragma unroll
    for (int k = 0; k < KP; ++k) pr[k] = acc[k];
  }
}

// ------------------------------------------------------------------ float I/O: register tiles
// With fp32 rows a 16-byte vector holds 4 channels, so a thread owns 4 channels and a run of
// steps and keeps the whole run (plus the K-1 step halo) in registers, loaded with one vector per
// row before the arithmetic; consecutive threads own consecutive channel groups. This measures
// faster for fp32 than staging through LDS; bf16 (8 channels per vector) uses the LDS tiles below.
constexpr int kRun = 16;   // forward steps per thread
constexpr int kCgWg = 64;  // channel groups per workgroup (one wave wide)
constexpr int kRunsWg = 4; // runs per workgroup (one per wave)

// VEC consecutive channels of one row: one vector access when the row is contiguous.
template <typename TIO, int VEC>
struct alignas(sizeof(TIO) * VEC) Vec {
  TIO v[VEC];
};

// VEC channels at element offset o of a row base (32-bit byte offsets from a workgroup-uniform
// base: the SGPR-base + VGPR-offset address form, no 64-bit arithmetic per access).
template <typename TIO, int VEC>
TSF_DEV void load_vec(float (&dst)[VEC], const TIO* base, uint32_t o) {
  if (VEC > 1) {
    const Vec<TIO, VEC> r = ld32(reinterpret_cast<const Vec<TIO, VEC>*>(base), o / VEC);
#pragma unroll
    for (int c = 0; c < VEC; ++c) dst[c] = to_f32(r.v[c]);
  } else {
    dst[0] = to_f32(ld32(base, o));
  }
}

template <typename TIO, int VEC>
TSF_DEV void store_vec(TIO* base, uint32_t o, const float (&src)[VEC]) {
  if (VEC > 1) {
    Vec<TIO, VEC> r;
#pragma unroll
    for (int c = 0; c < VEC; ++c) r.v[c] = from_f32<TIO>(src[c]);
    st32(reinterpret_cast<Vec<TIO, VEC>*>(base), o / VEC, r);
  } else {
    st32(base, o, from_f32<TIO>(src[0]));
  }
}


// Thread coordinates: channel group cg (VEC channels from d0 = cg * VEC), run r, batch row b.
struct Coord {
  int64_t b, run, d0;
  bool live;
};
template <int VEC>
TSF_DEV Coord coord(int64_t D, int64_t runs, uint32_t nx, uint32_t ny) {
  const Wg3 wg = wg3(nx, ny);
  const int64_t cgs = (D + VEC - 1) / VEC;
  const int64_t cg = wg.x * kCgWg + (threadIdx.x % kCgWg);
  const int64_t run = wg.y * kRunsWg + threadIdx.x / kCgWg;
  Coord c;
  c.b = wg.z;
  c.run = run;
  c.d0 = cg * VEC;
  c.live = cg < cgs && run < runs;
  return c;
}

// xbuf_s for VEC channels (s may be negative: the carried tail); zero outside [-(K-1), L).
// xrow = x + b * sxb (uniform per workgroup); the vector path has sxd == 1.
template <typename TIO, int VEC, int K>
TSF_DEV void load_xbuf(float (&dst)[VEC], const TIO* __restrict__ xrow, const TIO* __restrict__ tail, int64_t b,
                       int64_t s, int64_t d0, int64_t L, int64_t D, int64_t sxl, int64_t sxd) {
  if (s >= 0 && s < L) {
    load_vec<TIO, VEC>(dst, xrow, (uint32_t)(s * sxl + d0 * sxd));
  } else if (s < 0 && s >= -(K - 1)) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) dst[c] = tail ? to_f32(tail[(b * D + d0 + c) * (K - 1) + (K - 1 + s)]) : 0.0f;
  } else {
#pragma unroll
    for (int c = 0; c < VEC; ++c) dst[c] = 0.0f;
  }
}

// ------------------------------------------------------------------ register-tiled forward (fp32)
template <typename TIO, int K, int VEC>
__global__ void __launch_bounds__(kCgWg* kRunsWg) conv_silu_fwd_reg(
    const TIO* __restrict__ x, const TIO* __restrict__ tail, const float* __restrict__ w,
    const float* __restrict__ bias, TIO* __restrict__ out, int64_t L, int64_t D, int64_t sxb, int64_t sxl,
    int64_t sxd, int64_t runs, uint32_t nx, uint32_t ny) {
  const Coord c = coord<VEC>(D, runs, nx, ny);
  if (!c.live) return;
  float wk[K][VEC], bv[VEC];
#pragma unroll
  for (int ch = 0; ch < VEC; ++ch) {
#pragma unroll
    for (int k = 0; k < K; ++k) wk[k][ch] = w[(c.d0 + ch) * K + k];
    bv[ch] = bias ? bias[c.d0 + ch] : 0.0f;
  }
  const int64_t t0 = c.run * kRun;
  // the run's inputs with its K-1 step causal halo, all loads issued before the arithmetic
  const TIO* xrow = x + c.b * sxb;
  float xb[kRun + K - 1][VEC];
#pragma unroll
  for (int i = 0; i < kRun + K - 1; ++i)
    load_xbuf<TIO, VEC, K>(xb[i], xrow, tail, c.b, t0 - (K - 1) + i, c.d0, L, D, sxl, sxd);
  TIO* orow = out + c.b * L * D;
#pragma unroll
  for (int i = 0; i < kRun; ++i) {
    if (t0 + i >= L) break;
    float o[VEC];
#pragma unroll
    for (int ch = 0; ch < VEC; ++ch) {
      float p = bv[ch];
#pragma unroll
      for (int k = 0; k < K; ++k) p = fmaf(wk[k][ch], xb[i + k][ch], p);
      o[ch] = silu_f(p);
    }
    store_vec<TIO, VEC>(orow, (uint32_t)((t0 + i) * D + c.d0), o);
  }
}

// ----------------------------------------------------------------- register-tiled backward (fp32)
// gpre_t = gy_t silu'(p_t); gx_t = sum_k w_k gpre_{t+K-1-k}; grad w_k = sum_t gpre_t
// xbuf_{t-(K-1)+k}; grad bias = sum_t gpre_t; grad tail_j = sum_{t<=j} gpre_t w_{j-t}.
// A backward thread walks kRpt consecutive runs, accumulating its parameter partials in
// registers; the workgroup's kRunsWg threads per channel group meet in LDS, and the result is
// one partial row per (batch, run block): part [B, G, D, K+1] (K taps, then the bias term).
constexpr int kRpt = 4;
constexpr int kRunB = 8;  // backward steps per run: its register tiles hold x and gy with halos
static_assert(kRunsWg * kRpt * kRunB == kSeg, "both backward paths write one partial per kSeg steps");

template <typename TIO, int K, int VEC>
__global__ void __launch_bounds__(kCgWg* kRunsWg) conv_silu_bwd_reg(
    const TIO* __restrict__ x, const TIO* __restrict__ tail, const float* __restrict__ w,
    const float* __restrict__ bias, const TIO* __restrict__ gy, TIO* __restrict__ gx, TIO* __restrict__ gtail,
    float* __restrict__ part, int64_t L, int64_t D, int64_t sxb, int64_t sxl, int64_t sxd, int64_t runs,
    uint32_t nx, uint32_t ny) {
  constexpr int KP = K + 1;
  constexpr int NP = kRunB + K - 1;  // steps whose gpre a run needs: t0 .. t0+kRunB+K-2
  __shared__ float s_part[kRunsWg][KP][kCgWg * VEC];
  const int wv = threadIdx.x / kCgWg, ln = threadIdx.x % kCgWg;
  const Wg3 wg = wg3(nx, ny);
  const int64_t cg = wg.x * kCgWg + ln;
  const int64_t b = wg.z;
  const int64_t d0 = cg * VEC;
  const int64_t run0 = (wg.y * kRunsWg + wv) * kRpt;
  const TIO* xrow = x + b * sxb;
  const TIO* gyrow = gy + b * L * D;
  TIO* gxrow = gx + b * L * D;
  float acc[KP][VEC];
#pragma unroll
  for (int k = 0; k < KP; ++k)
#pragma unroll
    for (int ch = 0; ch < VEC; ++ch) acc[k][ch] = 0.0f;

  if (cg < (D + VEC - 1) / VEC) {
    float wk[K][VEC], bv[VEC];
#pragma unroll
    for (int ch = 0; ch < VEC; ++ch) {
#pragma unroll
      for (int k = 0; k < K; ++k) wk[k][ch] = w[(d0 + ch) * K + k];
      bv[ch] = bias ? bias[d0 + ch] : 0.0f;
    }
#pragma unroll 1
    for (int r = 0; r < kRpt; ++r) {
      const int64_t t0 = (run0 + r) * kRunB;
      if (t0 >= L) break;
      // xbuf from t0-(K-1) to t0+kRunB+K-2 and gy from t0 to t0+kRunB+K-2, loads issued first
      float xb[NP + K - 1][VEC], gp[NP][VEC];
#pragma unroll
      for (int i = 0; i < NP + K - 1; ++i)
        load_xbuf<TIO, VEC, K>(xb[i], xrow, tail, b, t0 - (K - 1) + i, d0, L, D, sxl, sxd);
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        if (t0 + i < L) {
          load_vec<TIO, VEC>(gp[i], gyrow, (uint32_t)((t0 + i) * D + d0));
        } else {
#pragma unroll
          for (int ch = 0; ch < VEC; ++ch) gp[i][ch] = 0.0f;  // rows past the end carry no gradient
        }
      }
      // gpre in place of gy
#pragma unroll
      for (int i = 0; i < NP; ++i)
#pragma unroll
        for (int ch = 0; ch < VEC; ++ch) {
          float p = bv[ch];
#pragma unroll
          for (int k = 0; k < K; ++k) p = fmaf(wk[k][ch], xb[i + k][ch], p);
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-p * kLog2e));
          gp[i][ch] *= sg * fmaf(p, 1.0f - sg, 1.0f);
        }
#pragma unroll
      for (int i = 0; i < kRunB; ++i) {
        if (t0 + i >= L) break;
        float g[VEC];
#pragma unroll
        for (int ch = 0; ch < VEC; ++ch) {
          float s = 0.0f;
#pragma unroll
          for (int k = 0; k < K; ++k) s = fmaf(wk[k][ch], gp[i + K - 1 - k][ch], s);
          g[ch] = s;
          // parameter partials over this run's own steps
#pragma unroll
          for (int k = 0; k < K; ++k) acc[k][ch] = fmaf(gp[i][ch], xb[i + k][ch], acc[k][ch]);
          acc[K][ch] += gp[i][ch];
        }
        store_vec<TIO, VEC>(gxrow, (uint32_t)((t0 + i) * D + d0), g);
      }
      // the carried tail feeds the first K-1 outputs
      if (t0 == 0 && gtail) {
#pragma unroll
        for (int ch = 0; ch < VEC; ++ch)
#pragma unroll
          for (int j = 0; j < K - 1; ++j) {
            float s = 0.0f;
#pragma unroll
            for (int t = 0; t <= j; ++t) s = fmaf(gp[t][ch], wk[j - t][ch], s);  // gp = 0 past L
            gtail[(b * D + d0 + ch) * (K - 1) + j] = from_f32<TIO>(s);
          }
      }
    }
  }
  // reduce the workgroup's threads of each channel group in LDS (fixed order)
#pragma unroll
  for (int k = 0; k < KP; ++k)
#pragma unroll
    for (int ch = 0; ch < VEC; ++ch) s_part[wv][k][ln * VEC + ch] = acc[k][ch];
  __syncthreads();
  const int64_t groups = ny;
  for (int idx = threadIdx.x; idx < KP * kCgWg * VEC; idx += kCgWg * kRunsWg) {
    const int k = idx / (kCgWg * VEC), dd = idx % (kCgWg * VEC);
    const int64_t d = wg.x * kCgWg * VEC + dd;
    if (d < D) {
      float s = 0.0f;
#pragma unroll
      for (int r = 0; r < kRunsWg; ++r) s += s_part[r][k][dd];
      part[(wg.z * groups + wg.y) * D * KP + d * KP + k] = s;
    }
  }
}

// grad w [D, K] and grad bias [D]: sum the partials [P, D, K+1] over P in a fixed order. A
// workgroup owns 64 consecutive outputs; its kRedWaves waves sum contiguous segments of the
// P rows (independent loads in flight), and wave 0 adds the segment sums in order.
constexpr int kRedWaves = 16;
__global__ void __launch_bounds__(64 * kRedWaves) conv_reduce_params(const float* __restrict__ part,
                                                                    float* __restrict__ gw, float* __restrict__ gb,
                                                                    int64_t P, int64_t D, int K) {
  __shared__ float s_seg[kRedWaves][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t n = D * (K + 1);
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  const int64_t seg = (P + kRedWaves - 1) / kRedWaves;
  const int64_t p0 = wv * seg, p1 = (p0 + seg < P) ? p0 + seg : P;
  float s = 0.0f;
  if (i < n) {
#pragma unroll 8
    for (int64_t p = p0; p < p1; ++p) s += part[p * n + i];
  }
  s_seg[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && i < n) {
    float t = s_seg[0][lane];
    for (int j = 1; j < kRedWaves; ++j) t += s_seg[j][lane];
    const int64_t d = i / (K + 1);
    const int k = (int)(i % (K + 1));
    if (k < K)
      gw[d * K + k] = t;
    else if (gb)
      gb[d] = t;
  }
}

__global__ void __launch_bounds__(256) conv_zero_f32(float* __restrict__ p, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// Grid: (channel blocks of kCh, segments of kSeg steps, batch rows).
struct ConvPlan {
  int64_t cblocks, nseg;
};
ConvPlan conv_plan(int64_t L, int64_t D) {
  ConvPlan p;
  p.cblocks = (D + kCh - 1) / kCh;
  p.nseg = (L + kSeg - 1) / kSeg;
  return p;
}

// Whole 16-byte pieces per tile row: channel stride 1, D and the row strides multiples of the
// piece, 16-byte aligned bases (y, z: the contiguous [B, L, D] tensors read or written the same
// way, or NULL).
template <typename TIO>
bool vec_rows(const void* x, int64_t D, int64_t sxb, int64_t sxl, int64_t sxd, const void* y, const void* z) {
  constexpr int64_t VE = 16 / sizeof(TIO);
  const uintptr_t a = (uintptr_t)x | (uintptr_t)y | (uintptr_t)z;
  return sxd == 1 && D % VE == 0 && sxl % VE == 0 && sxb % VE == 0 && a % 16 == 0;
}

template <typename TIO, int K>
void fwd_k(bool vec, int64_t B, int64_t L, int64_t D, const void* x, int64_t sxb, int64_t sxl, int64_t sxd,
           const void* tail, const float* w, const float* bias, void* out, hipStream_t s) {
  const ConvPlan p = conv_plan(L, D);
  const dim3 grid((unsigned)(p.cblocks * p.nseg * B));
  const uint32_t nx = (uint32_t)p.cblocks, ny = (uint32_t)p.nseg;
  if (vec)
    hipLaunchKernelGGL((conv_silu_fwd_kernel<TIO, K, true>), grid, dim3(kCh), 0, s, (const TIO*)x, (const TIO*)tail, w,
                       bias, (TIO*)out, L, D, sxb, sxl, sxd, nx, ny);
  else
    hipLaunchKernelGGL((conv_silu_fwd_kernel<TIO, K, false>), grid, dim3(kCh), 0, s, (const TIO*)x, (const TIO*)tail,
                       w, bias, (TIO*)out, L, D, sxb, sxl, sxd, nx, ny);
}

template <typename TIO, int K>
void bwd_k(bool vec, int64_t B, int64_t L, int64_t D, const void* x, int64_t sxb, int64_t sxl, int64_t sxd,
           const void* tail, const float* w, const float* bias, const void* gy, void* gx, void* gtail, float* gw,
           float* gb, float* part, hipStream_t s) {
  const ConvPlan p = conv_plan(L, D);
  const dim3 grid((unsigned)(p.cblocks * p.nseg * B));
  const uint32_t nx = (uint32_t)p.cblocks, ny = (uint32_t)p.nseg;
  if (vec)
    hipLaunchKernelGGL((conv_silu_bwd_kernel<TIO, K, true>), grid, dim3(kCh), 0, s, (const TIO*)x, (const TIO*)tail, w,
                       bias, (const TIO*)gy, (TIO*)gx, (TIO*)gtail, part, L, D, sxb, sxl, sxd, nx, ny);
  else
    hipLaunchKernelGGL((conv_silu_bwd_kernel<TIO, K, false>), grid, dim3(kCh), 0, s, (const TIO*)x, (const TIO*)tail,
                       w, bias, (const TIO*)gy, (TIO*)gx, (TIO*)gtail, part, L, D, sxb, sxl, sxd, nx, ny);
  const int64_t n = D * (K + 1);
  hipLaunchKernelGGL(conv_reduce_params, dim3((unsigned)((n + 63) / 64)), dim3(64 * kRedWaves), 0, s,
                     (const float*)part, gw, gb, B * p.nseg, D, K);
}

struct RegPlan {
  int64_t runs, cg_blocks, run_groups;
};
// run_groups: runs per workgroup row of the grid (kRunsWg for the forward, kRunsWg * kRpt for
// the backward, whose threads walk kRpt runs each)
RegPlan reg_plan(int64_t L, int64_t D, int vec, int run_len, int runs_per_group) {
  RegPlan p;
  p.runs = (L + run_len - 1) / run_len;
  p.cg_blocks = ((D + vec - 1) / vec + kCgWg - 1) / kCgWg;
  p.run_groups = (p.runs + runs_per_group - 1) / runs_per_group;
  return p;
}

// Vector width 4 (both passes) when every row of x and of the contiguous outputs is a 16-byte-aligned run of
// whole channel groups; the tail, weights and bias are read per channel either way.
template <typename TIO>
int vec_for(const void* x, int64_t D, int64_t sxb, int64_t sxl, int64_t sxd, const void* y) {
  const uintptr_t a = (uintptr_t)x | (uintptr_t)y;
  const bool ok = sxd == 1 && D % 4 == 0 && sxl % 4 == 0 && sxb % 4 == 0 && a % (4 * sizeof(TIO)) == 0;
  return ok ? 4 : 1;
}

template <typename TIO, int K, int VEC>
void launch_fwd(int64_t B, int64_t L, int64_t D, const void* x, int64_t sxb, int64_t sxl, int64_t sxd,
                const void* tail, const float* w, const float* bias, void* out, hipStream_t s) {
  const RegPlan p = reg_plan(L, D, VEC, kRun, kRunsWg);
  const dim3 grid((unsigned)(p.cg_blocks * p.run_groups * B));
  hipLaunchKernelGGL((conv_silu_fwd_reg<TIO, K, VEC>), grid, dim3(kCgWg * kRunsWg), 0, s, (const TIO*)x,
                     (const TIO*)tail, w, bias, (TIO*)out, L, D, sxb, sxl, sxd, p.runs, (uint32_t)p.cg_blocks,
                     (uint32_t)p.run_groups);
}

template <typename TIO, int K, int VEC>
void launch_bwd(int64_t B, int64_t L, int64_t D, const void* x, int64_t sxb, int64_t sxl, int64_t sxd,
                const void* tail, const float* w, const float* bias, const void* gy, void* gx, void* gtail,
                float* gw, float* gb, float* part, hipStream_t s) {
  const RegPlan p = reg_plan(L, D, VEC, kRunB, kRunsWg * kRpt);
  const dim3 grid((unsigned)(p.cg_blocks * p.run_groups * B));
  hipLaunchKernelGGL((conv_silu_bwd_reg<TIO, K, VEC>), grid, dim3(kCgWg * kRunsWg), 0, s, (const TIO*)x,
                     (const TIO*)tail, w, bias, (const TIO*)gy, (TIO*)gx, (TIO*)gtail, part, L, D, sxb, sxl, sxd,
                     p.runs, (uint32_t)p.cg_blocks, (uint32_t)p.run_groups);
  const int64_t n = D * (K + 1);
  hipLaunchKernelGGL(conv_reduce_params, dim3((unsigned)((n + 63) / 64)), dim3(64 * kRedWaves), 0, s,
                     (const float*)part, gw, gb, B * p.run_groups, D, K);
}

template <typename TIO, int K>
void fwd_reg(int vec, int64_t B, int64_t L, int64_t D, const void* x, int64_t sxb, int64_t sxl, int64_t sxd,
           const void* tail, const float* w, const float* bias, void* out, hipStream_t s) {
  if (vec == 4)
    launch_fwd<TIO, K, 4>(B, L, D, x, sxb, sxl, sxd, tail, w, bias, out, s);
  else
    launch_fwd<TIO, K, 1>(B, L, D, x, sxb, sxl, sxd, tail, w, bias, out, s);
}

template <typename TIO, int K>
void bwd_reg(int vec, int64_t B, int64_t L, int64_t D, const void* x, int64_t sxb, int64_t sxl, int64_t sxd,
           const void* tail, const float* w, const float* bias, const void* gy, void* gx, void* gtail, float* gw,
           float* gb, float* part, hipStream_t s) {
  if (vec == 4)
    launch_bwd<TIO, K, 4>(B, L, D, x, sxb, sxl, sxd, tail, w, bias, gy, gx, gtail, gw, gb, part, s);
  else
    launch_bwd<TIO, K, 1>(B, L, D, x, sxb, sxl, sxd, tail, w, bias, gy, gx, gtail, gw, gb, part, s);
}

// fp32 I/O from this many taps takes the LDS-tiled backward (the bf16 kernels' family) instead of
// the register-tile one, whose 6- to 8-tap instances run one wave per SIMD: at B 16, L 4096,
// D 1536 the tiled backward measured 264 / 272 / 285 us at K 5 / 6 / 8 against 287 / 364 /
// 430 us, and 262 / 273 us against 250 / 264 us at K 3 / 4.
#ifndef TSF_CONV_F32_TILED_K
#define TSF_CONV_F32_TILED_K 5
#endif
#define TSF_CONV_K_SWITCH(K, CALL) \
  switch (K) {                     \
    case 2: CALL(2); break;        \
    case 3: CALL(3); break;        \
    case 4: CALL(4); break;        \
    case 5: CALL(5); break;        \
    case 6: CALL(6); break;        \
    case 7: CALL(7); break;        \
    case 8: CALL(8); break;        \
    default: return TSF_ERR_UNSUPPORTED; \
  }

// TSF_OK when the sizes are valid and supported, else the status to return
// The grids are one-dimensional with 256-thread workgroups (kernels index it in 32 bits): at most
// 2^24 - 1 workgroups. The register-tile forward with one channel per thread has the most,
// ceil(D / 64) * ceil(ceil(L / 16) / 4) per batch row.
constexpr int64_t kMaxWgs = (1 << 24) - 1;
int conv_args_status(int64_t B, int64_t L, int64_t D, int64_t K) {
  if (B < 0 || L < 0 || D < 0 || K < 2) return TSF_ERR_ARG;
  if (K > 8) return TSF_ERR_UNSUPPORTED;
  const int64_t per_row = ((D + kCgWg - 1) / kCgWg) * ((((L + kRun - 1) / kRun) + kRunsWg - 1) / kRunsWg);
  if (per_row > 0 && B > kMaxWgs / per_row) return TSF_ERR_UNSUPPORTED;
  return TSF_OK;
}

// The kernels address one batch row of x and of the [B, L, D] outputs with 32-bit byte offsets.
int conv_layout_status(int64_t L, int64_t D, int64_t sxl, int64_t sxd, int64_t esz) {
  if (sxl < 0 || sxd < 0) return TSF_ERR_ARG;
  const int64_t lim = (int64_t)1 << 32;
  const bool ok = ((L + 8) * sxl + (D + 8) * sxd) * esz < lim && (L + 8) * D * esz < lim;
  return ok ? TSF_OK : TSF_ERR_UNSUPPORTED;
}

}  // namespace

extern "C" {

int64_t tsfast_hip_conv_silu_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t K) {
  if (conv_args_status(B, L, D, K) != TSF_OK) return -1;
  return B * conv_plan(L, D).nseg * D * (K + 1) * 4;
}

int tsfast_hip_conv_silu_fwd(int64_t B, int64_t L, int64_t D, int64_t K, int io_dtype, const void* x, int64_t sxb,
                             int64_t sxl, int64_t sxd, const void* tail, const float* weight, const float* bias,
                             void* out, void* stream) {
  if (const int st = conv_args_status(B, L, D, K)) return st;
  if (B == 0 || L == 0 || D == 0) return TSF_OK;
  if (!x || !weight || !out) return TSF_ERR_ARG;
  if (const int st = conv_layout_status(L, D, sxl, sxd, io_dtype == TSF_DTYPE_BF16 ? 2 : 4)) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (io_dtype == TSF_DTYPE_F32) {
    const int vec = vec_for<float>(x, D, sxb, sxl, sxd, out);
#define CALL(KK) fwd_reg<float, KK>(vec, B, L, D, x, sxb, sxl, sxd, tail, weight, bias, out, s)
    TSF_CONV_K_SWITCH(K, CALL)
#undef CALL
  } else if (io_dtype == TSF_DTYPE_BF16) {
    const bool vec = vec_rows<bf16>(x, D, sxb, sxl, sxd, out, nullptr);
#define CALL(KK) fwd_k<bf16, KK>(vec, B, L, D, x, sxb, sxl, sxd, tail, weight, bias, out, s)
    TSF_CONV_K_SWITCH(K, CALL)
#undef CALL
  } else {
    return TSF_ERR_ARG;
  }
  return tsf_launch_status();
}

int tsfast_hip_conv_silu_bwd(int64_t B, int64_t L, int64_t D, int64_t K, int io_dtype, const void* x, int64_t sxb,
                             int64_t sxl, int64_t sxd, const void* tail, const float* weight, const float* bias,
                             const void* gy, void* gx, void* gtail, float* gw, float* gb, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  if (const int st = conv_args_status(B, L, D, K)) return st;
  if (D == 0) return TSF_OK;
  if (!weight || !gw || (bias && !gb)) return TSF_ERR_ARG;
  if (B > 0 && L > 0 && (!x || !gy || !gx)) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_conv_silu_workspace_bytes(B, L, D, K) || (!workspace && B * L > 0))
    return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || L == 0) {
    // empty sequence: parameter gradients are zero, the tail receives no gradient
    const int64_t n = D * K;
    hipLaunchKernelGGL(conv_zero_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gw, n);
    if (gb) hipLaunchKernelGGL(conv_zero_f32, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, s, gb, D);
    return tsf_launch_status();
  }
  if (const int st = conv_layout_status(L, D, sxl, sxd, io_dtype == TSF_DTYPE_BF16 ? 2 : 4)) return st;
  float* part = static_cast<float*>(workspace);
  if (io_dtype == TSF_DTYPE_F32 && K >= TSF_CONV_F32_TILED_K) {
    const bool vec = vec_rows<float>(x, D, sxb, sxl, sxd, gy, gx);
#define CALL(KK) bwd_k<float, KK>(vec, B, L, D, x, sxb, sxl, sxd, tail, weight, bias, gy, gx, gtail, gw, gb, part, s)
    TSF_CONV_K_SWITCH(K, CALL)
#undef CALL
  } else if (io_dtype == TSF_DTYPE_F32) {
    const int vec = vec_for<float>(x, D, sxb, sxl, sxd, gy) == 4 && ((uintptr_t)gx % 16 == 0) ? 4 : 1;
#define CALL(KK) bwd_reg<float, KK>(vec, B, L, D, x, sxb, sxl, sxd, tail, weight, bias, gy, gx, gtail, gw, gb, part, s)
    TSF_CONV_K_SWITCH(K, CALL)
#undef CALL
  } else if (io_dtype == TSF_DTYPE_BF16) {
    const bool vec = vec_rows<bf16>(x, D, sxb, sxl, sxd, gy, gx);
#define CALL(KK) bwd_k<bf16, KK>(vec, B, L, D, x, sxb, sxl, sxd, tail, weight, bias, gy, gx, gtail, gw, gb, part, s)
    TSF_CONV_K_SWITCH(K, CALL)
#undef CALL
  } else {
    return TSF_ERR_ARG;
  }
  return tsf_launch_status();
}

}  // extern "C"
