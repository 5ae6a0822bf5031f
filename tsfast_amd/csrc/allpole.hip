// dynoNet all-pole IIR scan  y_t = w_t - sum_{i=1..na} a_i y_{t-i}  and its adjoint, float32.
//
// Reference semantics: tsfast/models/architectures/dynonet/allpole_triton.py:59-123 (kernels),
// :174-233 (ops, y0 head taps :202-213); the companion-matrix form is
// tsfast/models/architectures/dynonet/core.py:23-135.
//
// Layout: lanes [lanes, L] with time contiguous; a [lanes, na]; y0 [lanes, na] newest first
// (y0[j] = y_{-1-j}). The recurrence order NA is a template parameter (1..16), so the delay
// line s_0..s_{NA-1} (s_k = y_{t-1-k}) lives in registers and a step is NA FMAs.
//
// Arithmetic: fp32 in and out, fp64 inside (delay line, transfer matrices, carries, grad
// accumulators). High-order direct-form filters amplify fp32 rounding badly (order 16 with
// poles near 0.98 loses ~3 digits), and the scan is HBM-bound, so the wider state is free.
//
// Parallel structure. A chunk of steps maps its entering state s (the last NA outputs before it)
// to M s + e, with M a power of the companion matrix C and e the chunk's zero-state end. Orders
// NA <= 4 run single-pass kernels with a decoupled look-back between workgroups (every input
// element read once; described at allpole_fwd_lb). Higher orders, whose NA x NA matrices do not
// fit in registers, run a two-pass scan with chunks of T_c steps (at most 256 when the sequence
// takes more than one chunk), one thread per (lane, chunk) in the streaming passes:
//   1. transfer   per (lane, column): M = C^{T_c}, C applied T_c times to a unit vector;
//   2. chunk_end  per (lane, chunk): e_c from a zero entering state;
//   3. carry      per lane (16 threads, one state component each): entering states
//                 S_c = M S_{c-1} + e_{c-1}, sequential over chunks;
//   4. apply      per (lane, chunk): run the chunk from S_c and write y.
// The adjoint G_t = g_t - sum_i a_i G_{t+i} is the same filter run backwards, so the backward
// reuses the matrices with the chunk order reversed and accumulates grad_a partials per chunk;
// a final cooperative kernel sums them in a fixed order and adds the y0 head taps and grad_y0.
#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

#include "allpole_core.h"


// M = C^{T_c} for chunks of at most kColsT steps, one thread per (lane, column): column col is C
// applied T_c times to the unit vector e_col, step by step in fp64 (see companion_powers_col for
// why not by squaring), in unrolled 32-step blocks.
constexpr int64_t kColsT = 256;
template <int NA>
__global__ void __launch_bounds__(64) allpole_transfer_cols(const float* __restrict__ a, double* __restrict__ M,
                                                            int64_t lanes, int T_c) {
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= lanes * NA) return;
  const int64_t lane = idx / NA;
  const int col = (int)(idx - lane * NA);
  double ac[NA], x[NA];
#pragma unroll
  for (int c = 0; c < NA; ++c) {
    ac[c] = (double)a[lane * NA + c];
    x[c] = c == col ? 1.0 : 0.0;
  }
  int t = 0;
  for (; t + 32 <= T_c; t += 32)
#pragma unroll
    for (int step = 0; step < 32; ++step) companion_apply<NA>(x, ac);
  for (; t < T_c; ++t) companion_apply<NA>(x, ac);
#pragma unroll
  for (int r = 0; r < NA; ++r) M[(lane * NA + r) * NA + col] = x[r];
}

// M = C^{T_c} per lane for chunks longer than kColsT (only sequences of more than 65535 x 256
// steps). Powers up to C^256 are built step by step from the unit vectors; a longer chunk takes
// (C^256)^q C^r, squaring only C^256, whose transient growth has decayed for the stable filters
// this scan serves.
template <int NA>
__global__ void __launch_bounds__(256) allpole_transfer(const float* __restrict__ a, double* __restrict__ Mout,
                                                        int64_t lanes, int64_t T_c) {
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  constexpr int64_t kStep = 256;
  double ac[NA];
#pragma unroll
  for (int c = 0; c < NA; ++c) ac[c] = (double)a[lane * NA + c];
  const int64_t base = T_c < kStep ? T_c : kStep;
  const int64_t q = T_c / base, rem = T_c - q * base;
  double Q[NA][NA], R[NA][NA], T[NA][NA];  // Q = C^base, R = C^rem
  for (int col = 0; col < NA; ++col) {
    double x[NA];
#pragma unroll
    for (int r = 0; r < NA; ++r) x[r] = r == col ? 1.0 : 0.0;
    for (int64_t step = 1; step <= base; ++step) {
      companion_apply<NA>(x, ac);
      if (step == rem)
#pragma unroll
        for (int r = 0; r < NA; ++r) R[r][col] = x[r];
    }
#pragma unroll
    for (int r = 0; r < NA; ++r) Q[r][col] = x[r];
    if (rem == 0)
#pragma unroll
      for (int r = 0; r < NA; ++r) R[r][col] = r == col ? 1.0 : 0.0;
  }
  auto mul = [&](double (&dst)[NA][NA], const double (&x)[NA][NA], const double (&y)[NA][NA]) {
    for (int r = 0; r < NA; ++r)
      for (int c = 0; c < NA; ++c) {
        double s = 0.0;
        for (int j = 0; j < NA; ++j) s = fma(x[r][j], y[j][c], s);
        T[r][c] = s;
      }
    for (int r = 0; r < NA; ++r)
      for (int c = 0; c < NA; ++c) dst[r][c] = T[r][c];
  };
  for (int64_t k = q; k > 0; k >>= 1) {  // R <- R Q^q
    if (k & 1) mul(R, R, Q);
    if (k > 1) mul(Q, Q, Q);
  }
  for (int r = 0; r < NA; ++r)
    for (int c = 0; c < NA; ++c) Mout[lane * NA * NA + r * NA + c] = R[r][c];
}

// 2. forward chunk ends from a zero entering state, chunks 0 .. nchunk-2.
template <int NA>
__global__ void __launch_bounds__(kTile) allpole_fwd_chunk_end(const float* __restrict__ a,
                                                               const float* __restrict__ w, double* __restrict__ e,
                                                               int64_t lanes, int64_t L, int64_t T_c,
                                                               int64_t nchunk) {
  __shared__ float tile[kTile][kTileT + 1];
  const int tid = threadIdx.x;
  const int64_t l0 = (int64_t)blockIdx.x * kTile, c = blockIdx.y;
  const int64_t lane = l0 + tid;
  const bool act = lane < lanes;
  double av[NA], s[NA];
#pragma unroll
  for (int k = 0; k < NA; ++k) {
    av[k] = act ? (double)a[lane * NA + k] : 0.0;
    s[k] = 0.0;
  }
  const int64_t t0 = c * T_c;
  TileRegs rg;
  tile_fetch(rg, w, lanes, L, l0, t0, (int)(T_c < kTileT ? T_c : kTileT), tid);
  for (int64_t tt = 0; tt < T_c; tt += kTileT) {
    const int n = (int)((T_c - tt) < kTileT ? (T_c - tt) : kTileT);
    tile_put(rg, tile, tid);
    __syncthreads();
    if (tt + kTileT < T_c)
      tile_fetch(rg, w, lanes, L, l0, t0 + tt + kTileT, (int)((T_c - tt - kTileT) < kTileT ? (T_c - tt - kTileT) : kTileT), tid);
    if (n == kTileT) {
#pragma unroll
      for (int k = 0; k < kTileT; ++k) step<NA>(av, s, (double)tile[tid][k]);
    } else {
      for (int k = 0; k < n; ++k) step<NA>(av, s, (double)tile[tid][k]);
    }
    __syncthreads();
  }
  if (act) {
#pragma unroll
    for (int k = 0; k < NA; ++k) e[(c * lanes + lane) * NA + k] = s[k];
  }
}

// 3. forward carries: the entering state of every chunk, sequential over chunks per lane. Sixteen
// threads per lane (one 16-lane DPP row): thread r holds state component r and row r of M, and
// reads the other components by row broadcast. The chunk ends e_c do not depend on the carry and
// are loaded kCarryPf chunks ahead.
constexpr int kCarryPf = 8;
template <int NA>
__global__ void __launch_bounds__(256) allpole_fwd_carry(const double* __restrict__ M, const double* __restrict__ e,
                                                         const float* __restrict__ y0, double* __restrict__ S,
                                                         int64_t lanes, int64_t nchunk) {
  const int r = threadIdx.x & 15;
  const int64_t lane = blockIdx.x * (int64_t)16 + (threadIdx.x >> 4);
  const bool ld = lane < lanes && r < NA;
  double m[NA];
#pragma unroll
  for (int c = 0; c < NA; ++c) m[c] = ld ? M[(lane * NA + r) * NA + c] : 0.0;
  double s = (ld && y0) ? (double)y0[lane * NA + r] : 0.0;
  double ev[kCarryPf];  // ev[k] = e of chunk cb + k (chunks 0 .. nchunk-2 have one)
#pragma unroll
  for (int k = 0; k < kCarryPf; ++k) ev[k] = (ld && k + 1 < nchunk) ? e[(k * lanes + lane) * NA + r] : 0.0;
  for (int64_t cb = 0; cb < nchunk; cb += kCarryPf) {
#pragma unroll
    for (int k = 0; k < kCarryPf; ++k) {
      const int64_t c = cb + k;
      if (c < nchunk) {  // uniform over the workgroup
        if (ld) S[(c * lanes + lane) * NA + r] = s;
        if (c + 1 < nchunk) {
          double a0 = ev[k], a1 = 0.0;
          row_dot2<NA>(m, s, a0, a1);
          s = a0 + a1;
        }
        const int64_t cn = c + kCarryPf;
        ev[k] = (ld && cn + 1 < nchunk) ? e[(cn * lanes + lane) * NA + r] : 0.0;
      }
    }
  }
}

// 4. forward apply.
template <int NA>
__global__ void __launch_bounds__(kTile) allpole_fwd_apply(const float* __restrict__ a, const float* __restrict__ w,
                                                           const double* __restrict__ S, float* __restrict__ y,
                                                           int64_t lanes, int64_t L, int64_t T_c, int64_t nchunk) {
  __shared__ float tile[kTile][kTileT + 1];
  const int tid = threadIdx.x;
  const int64_t l0 = (int64_t)blockIdx.x * kTile, c = blockIdx.y;
  const int64_t lane = l0 + tid;
  const bool act = lane < lanes;
  double av[NA], s[NA];
#pragma unroll
  for (int k = 0; k < NA; ++k) {
    av[k] = act ? (double)a[lane * NA + k] : 0.0;
    s[k] = act ? S[(c * lanes + lane) * NA + k] : 0.0;
  }
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  TileRegs rg;
  tile_fetch(rg, w, lanes, L, l0, t0, (int)(len < kTileT ? len : kTileT), tid);
  for (int64_t tt = 0; tt < len; tt += kTileT) {
    const int n = (int)((len - tt) < kTileT ? (len - tt) : kTileT);
    tile_put(rg, tile, tid);
    __syncthreads();
    if (tt + kTileT < len)
      tile_fetch(rg, w, lanes, L, l0, t0 + tt + kTileT, (int)((len - tt - kTileT) < kTileT ? (len - tt - kTileT) : kTileT), tid);
    if (n == kTileT) {
#pragma unroll
      for (int k = 0; k < kTileT; ++k) tile[tid][k] = (float)step<NA>(av, s, (double)tile[tid][k]);
    } else {
      for (int k = 0; k < n; ++k) tile[tid][k] = (float)step<NA>(av, s, (double)tile[tid][k]);
    }
    __syncthreads();
    tile_store(tile, y, lanes, L, l0, t0 + tt, n, tid);
    __syncthreads();
  }
}

// Backward 2. reverse chunk exits (G_{t0}, G_{t0+1}, ...) with zero entering state, chunks >= 1.
template <int NA>
__global__ void __launch_bounds__(kTile) allpole_bwd_chunk_start(const float* __restrict__ a,
                                                                 const float* __restrict__ g, double* __restrict__ f,
                                                                 int64_t lanes, int64_t L, int64_t T_c,
                                                                 int64_t nchunk) {
  __shared__ float tile[kTile][kTileT + 1];
  const int tid = threadIdx.x;
  const int64_t l0 = (int64_t)blockIdx.x * kTile, c = (int64_t)blockIdx.y + 1;
  const int64_t lane = l0 + tid;
  const bool act = lane < lanes;
  double av[NA], s[NA];
#pragma unroll
  for (int k = 0; k < NA; ++k) {
    av[k] = act ? (double)a[lane * NA + k] : 0.0;
    s[k] = 0.0;
  }
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const int64_t last = ((len - 1) / kTileT) * kTileT;
  TileRegs rg;
  tile_fetch(rg, g, lanes, L, l0, t0 + last, (int)((len - last) < kTileT ? (len - last) : kTileT), tid);
  for (int64_t tt = last; tt >= 0; tt -= kTileT) {
    const int n = (int)((len - tt) < kTileT ? (len - tt) : kTileT);
    tile_put(rg, tile, tid);
    __syncthreads();
    if (tt > 0) tile_fetch(rg, g, lanes, L, l0, t0 + tt - kTileT, kTileT, tid);
    if (n == kTileT) {
#pragma unroll
      for (int k = kTileT - 1; k >= 0; --k) step<NA>(av, s, (double)tile[tid][k]);
    } else {
      for (int k = n - 1; k >= 0; --k) step<NA>(av, s, (double)tile[tid][k]);
    }
    __syncthreads();
  }
  if (act) {
#pragma unroll
    for (int k = 0; k < NA; ++k) f[(c * lanes + lane) * NA + k] = s[k];
  }
}

// Backward 3. entering (from the right) states of every chunk: R_last = 0, R_{last-1} = f_last,
// R_c = M R_{c+1} + f_{c+1}; the thread layout and prefetch of the forward carry.
template <int NA>
__global__ void __launch_bounds__(256) allpole_bwd_carry(const double* __restrict__ M, const double* __restrict__ f,
                                                         double* __restrict__ R, int64_t lanes, int64_t nchunk) {
  const int r = threadIdx.x & 15;
  const int64_t lane = blockIdx.x * (int64_t)16 + (threadIdx.x >> 4);
  const bool ld = lane < lanes && r < NA;
  double m[NA];
#pragma unroll
  for (int c = 0; c < NA; ++c) m[c] = ld ? M[(lane * NA + r) * NA + c] : 0.0;
  double s = 0.0;
  double fv[kCarryPf];  // fv[k] = f of chunk nchunk-1 - (cb + k) (chunks 1 .. nchunk-1 have one)
#pragma unroll
  for (int k = 0; k < kCarryPf; ++k) {
    const int64_t c = nchunk - 1 - k;
    fv[k] = (ld && c >= 1) ? f[(c * lanes + lane) * NA + r] : 0.0;
  }
  for (int64_t cb = 0; cb < nchunk; cb += kCarryPf) {
#pragma unroll
    for (int k = 0; k < kCarryPf; ++k) {
      const int64_t c = nchunk - 1 - (cb + k);
      if (c >= 0) {  // uniform over the workgroup
        if (ld) R[(c * lanes + lane) * NA + r] = s;
        if (c > 0) {
          if (c == nchunk - 1) {
            s = fv[k];  // the last chunk enters from a zero state: its exit is f alone
          } else {
            double a0 = fv[k], a1 = 0.0;
            row_dot2<NA>(m, s, a0, a1);
            s = a0 + a1;
          }
        }
        const int64_t cn = c - kCarryPf;
        fv[k] = (ld && cn >= 1) ? f[(cn * lanes + lane) * NA + r] : 0.0;
      }
    }
  }
}

// Backward 4. reverse apply: G_t, gw = G, and grad_a partials sum_u G_{u+1+k} y_u per chunk.
template <int NA>
__global__ void __launch_bounds__(kTile) allpole_bwd_apply(const float* __restrict__ a, const float* __restrict__ g,
                                                           const float* __restrict__ y, const double* __restrict__ R,
                                                           float* __restrict__ gw, double* __restrict__ ga_part,
                                                           int64_t lanes, int64_t L, int64_t T_c, int64_t nchunk) {
  __shared__ float tg[kTile][kTileT + 1];
  __shared__ float ty[kTile][kTileT + 1];
  const int tid = threadIdx.x;
  const int64_t l0 = (int64_t)blockIdx.x * kTile, c = blockIdx.y;
  const int64_t lane = l0 + tid;
  const bool act = lane < lanes;
  double av[NA], s[NA], ga[NA];
#pragma unroll
  for (int k = 0; k < NA; ++k) {
    av[k] = act ? (double)a[lane * NA + k] : 0.0;
    s[k] = act ? R[(c * lanes + lane) * NA + k] : 0.0;
    ga[k] = 0.0;
  }
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const int64_t last = ((len - 1) / kTileT) * kTileT;
  // Above order 8 the next tile is not prefetched during the recurrence: its 64 registers would
  // take the kernel to one wave per SIMD.
  constexpr bool kPf = NA <= 8;
  TileRegs rgg, rgy;
  if (kPf) {
    const int n0 = (int)((len - last) < kTileT ? (len - last) : kTileT);
    tile_fetch(rgg, g, lanes, L, l0, t0 + last, n0, tid);
    tile_fetch(rgy, y, lanes, L, l0, t0 + last, n0, tid);
  }
  for (int64_t tt = last; tt >= 0; tt -= kTileT) {
    const int n = (int)((len - tt) < kTileT ? (len - tt) : kTileT);
    if (!kPf) {
      tile_fetch(rgg, g, lanes, L, l0, t0 + tt, n, tid);
      tile_fetch(rgy, y, lanes, L, l0, t0 + tt, n, tid);
    }
    tile_put(rgg, tg, tid);
    tile_put(rgy, ty, tid);
    __syncthreads();
    if (kPf && tt > 0) {
      tile_fetch(rgg, g, lanes, L, l0, t0 + tt - kTileT, kTileT, tid);
      tile_fetch(rgy, y, lanes, L, l0, t0 + tt - kTileT, kTileT, tid);
    }
    auto bstep = [&](int k) __attribute__((always_inline)) {
      const double yu = ty[tid][k];
#pragma unroll
      for (int q = 0; q < NA; ++q) ga[q] = fma(s[q], yu, ga[q]);  // s_q = G_{u+1+q} before the step
      tg[tid][k] = (float)step<NA>(av, s, (double)tg[tid][k]);
    };
    if (n == kTileT) {
#pragma unroll
      for (int k = kTileT - 1; k >= 0; --k) bstep(k);
    } else {
      for (int k = n - 1; k >= 0; --k) bstep(k);
    }
    __syncthreads();
    tile_store(tg, gw, lanes, L, l0, t0 + tt, n, tid);
    __syncthreads();
  }
  if (act) {
#pragma unroll
    for (int k = 0; k < NA; ++k) ga_part[(c * lanes + lane) * NA + k] = ga[k];
  }
}

template <int NA>
__global__ void __launch_bounds__(64 * kLbWaves) __attribute__((amdgpu_waves_per_eu(4))) allpole_fwd_lb(
    const float* __restrict__ a, const float* __restrict__ w, const float* __restrict__ y0, float* __restrict__ y,
    const double* __restrict__ Mc, const double* __restrict__ Ms, double* __restrict__ agg, double* __restrict__ inc,
    unsigned* __restrict__ counter, int64_t lanes, int64_t L, int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  constexpr int NN = NA * NA;
  __shared__ LdsTile s_lds[kLbWaves];
  __shared__ int s_flag[kLbWaves][64];
  __shared__ int s_pend[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  __shared__ double s_mat[MatStage<NA>::kDoubles];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * kTileT;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t sc = tile / groups, l0 = (tile - sc * groups) * kTile, lane = l0 + lid;
    const bool live = lane < lanes;
    const int64_t t0 = sc * SL + (int64_t)k * kTileT;
    const int n = (L - t0) >= kTileT ? kTileT : (L - t0) > 0 ? (int)(L - t0) : 0;
    double av[NA], s[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      av[q] = live ? (double)a[lane * NA + q] : 0.0;
      s[q] = 0.0;
    }
    float xb[kTileT];
    if (n > 0) chunk_to_regs(xb, w, lanes, L, l0, t0, n, s_lds[k], lid);
    if constexpr (MatStage<NA>::kLds) stage_mats<NA>(s_mat, Mc, Ms, l0, lanes);
    if (n == kTileT) {
#pragma unroll
      for (int i = 0; i < kTileT; ++i) step<NA>(av, s, (double)xb[i]);
    } else {
#pragma unroll
      for (int i = 0; i < kTileT; ++i)
        if (i < n) step<NA>(av, s, (double)xb[i]);
    }
    double* vk = vec_area<NA>(s_lds, k) + lid * NA;
#pragma unroll
    for (int q = 0; q < NA; ++q) vk[q] = s[q];
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    // wave 0: the super-chunk's zero-state end (chunks before a non-empty one are full, so Mc is
    // every fold's matrix; the map is published only for full super-chunks)
    double sup[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) sup[q] = 0.0;
    if (k == 0 && live) {
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = 0; j < K; ++j) {
        double ej[NA];
        const double* vj = vec_area<NA>(s_lds, j) + lid * NA;
#pragma unroll
        for (int q = 0; q < NA; ++q) ej[q] = vj[q];
        matvec_add<NA>(sup, mc, sup, ej);
      }
      if (lb_pub_agg(sc, lb_spacing) && sc + 1 < nsuper) put_vec<NA>(agg + (sc * lanes + lane) * NA, sup);
    }
    double S[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) S[q] = (sc == 0 && y0 && live && k == 0) ? (double)y0[lane * NA + q] : 0.0;
    if (sc > 0)  // uniform over the workgroup
      ap_look_back<NA>(S, agg, inc, MatStage<NA>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN, k == 0 && live, sc - 1, (int64_t)-1, nsuper, lanes, lane, K,
                       k, lid, s_lds, s_flag, s_pend, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(sc, lb_spacing) && sc + 1 < nsuper) {
        double ms[NA][NA], o[NA];
        load_mat<NA>(ms, MatStage<NA>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN);
        matvec_add<NA>(o, ms, S, sup);
        put_vec<NA>(inc + (sc * lanes + lane) * NA, o);
      }
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = 0; j < K; ++j) {  // entering state of every chunk, in place of its summary
        double ej[NA];
        double* vj = vec_area<NA>(s_lds, j) + lid * NA;
#pragma unroll
        for (int q = 0; q < NA; ++q) {
          ej[q] = vj[q];
          vj[q] = S[q];
        }
        matvec_add<NA>(S, mc, S, ej);
      }
    }
    __syncthreads();
    if (n > 0) {
#pragma unroll
      for (int q = 0; q < NA; ++q) s[q] = vk[q];
      if (n == kTileT) {
#pragma unroll
        for (int i = 0; i < kTileT; ++i) xb[i] = (float)step<NA>(av, s, (double)xb[i]);
      } else {
#pragma unroll
        for (int i = 0; i < kTileT; ++i)
          if (i < n) xb[i] = (float)step<NA>(av, s, (double)xb[i]);
      }
      __builtin_amdgcn_wave_barrier();
      regs_to_chunk(xb, y, lanes, L, l0, t0, n, s_lds[k], lid);
    }
  }
}

// Backward: the adjoint G_t = g_t - sum_i a_i G_{t+i} is the same filter run from the right
// end, so the chunk and super-chunk maps are the same matrices with the scan order reversed.
// y enters only the grad_a sums, so it is loaded after the look-back (it does not stay in
// registers across it). grad_a partials (sum_u G_{u+1+q} y_u) are summed over the K chunks in
// LDS and written per super-chunk; allpole_finish adds them up in a fixed order.
template <int NA>
__global__ void __launch_bounds__(64 * kLbWaves) __attribute__((amdgpu_waves_per_eu(4))) allpole_bwd_lb(
    const float* __restrict__ a, const float* __restrict__ g, const float* __restrict__ y,
    const double* __restrict__ Mc, const double* __restrict__ Ms, double* __restrict__ agg, double* __restrict__ inc,
    unsigned* __restrict__ counter, float* __restrict__ gw, double* __restrict__ part, int64_t lanes, int64_t L,
    int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  constexpr int NN = NA * NA;
  __shared__ LdsTile s_lds[kLbWaves];
  __shared__ int s_flag[kLbWaves][64];
  __shared__ int s_pend[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  __shared__ double s_mat[MatStage<NA>::kDoubles];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * kTileT;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t r = tile / groups, sc = nsuper - 1 - r, l0 = (tile - r * groups) * kTile, lane = l0 + lid;
    const bool live = lane < lanes;
    const int64_t t0 = sc * SL + (int64_t)k * kTileT;
    const int n = (L - t0) >= kTileT ? kTileT : (L - t0) > 0 ? (int)(L - t0) : 0;
    double av[NA], s[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      av[q] = live ? (double)a[lane * NA + q] : 0.0;
      s[q] = 0.0;
    }
    float gb[kTileT];
    if (n > 0) chunk_to_regs(gb, g, lanes, L, l0, t0, n, s_lds[k], lid);
    if constexpr (MatStage<NA>::kLds) stage_mats<NA>(s_mat, Mc, Ms, l0, lanes);
    if (n == kTileT) {
#pragma unroll
      for (int i = kTileT - 1; i >= 0; --i) step<NA>(av, s, (double)gb[i]);
    } else {
#pragma unroll
      for (int i = kTileT - 1; i >= 0; --i)
        if (i < n) step<NA>(av, s, (double)gb[i]);
    }
    double* vk = vec_area<NA>(s_lds, k) + lid * NA;
#pragma unroll
    for (int q = 0; q < NA; ++q) vk[q] = s[q];
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    // wave 0: the super-chunk's exit to the left from a zero entering state, folded from its
    // rightmost chunk (chunks past the end of the sequence are empty and contribute zero)
    double sup[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) sup[q] = 0.0;
    if (k == 0 && live) {
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = K - 1; j >= 0; --j) {
        double fj[NA];
        const double* vj = vec_area<NA>(s_lds, j) + lid * NA;
#pragma unroll
        for (int q = 0; q < NA; ++q) fj[q] = vj[q];
        matvec_add<NA>(sup, mc, sup, fj);
      }
      if (lb_pub_agg(nsuper - 1 - sc, lb_spacing) && sc > 0) put_vec<NA>(agg + (sc * lanes + lane) * NA, sup);
    }
    double R[NA];  // state entering the super-chunk from the right
#pragma unroll
    for (int q = 0; q < NA; ++q) R[q] = 0.0;
    if (sc + 1 < nsuper)  // uniform over the workgroup
      ap_look_back<NA>(R, agg, inc, MatStage<NA>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN, k == 0 && live, sc + 1, (int64_t)1, nsuper, lanes, lane, K,
                       k, lid, s_lds, s_flag, s_pend, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(nsuper - 1 - sc, lb_spacing) && sc > 0) {
        double ms[NA][NA], o[NA];
        load_mat<NA>(ms, MatStage<NA>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN);
        matvec_add<NA>(o, ms, R, sup);
        put_vec<NA>(inc + (sc * lanes + lane) * NA, o);
      }
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = K - 1; j >= 0; --j) {  // state entering every chunk from the right
        double fj[NA];
        double* vj = vec_area<NA>(s_lds, j) + lid * NA;
#pragma unroll
        for (int q = 0; q < NA; ++q) {
          fj[q] = vj[q];
          vj[q] = R[q];
        }
        matvec_add<NA>(R, mc, R, fj);
      }
    }
    __syncthreads();
    double ga[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) ga[q] = 0.0;
    if (n > 0) {
#pragma unroll
      for (int q = 0; q < NA; ++q) s[q] = vk[q];
      __builtin_amdgcn_wave_barrier();
      float yb[kTileT];
      chunk_to_regs(yb, y, lanes, L, l0, t0, n, s_lds[k], lid);
      auto bstep = [&](int i) __attribute__((always_inline)) {
        const double yu = yb[i];
#pragma unroll
        for (int q = 0; q < NA; ++q) ga[q] = fma(s[q], yu, ga[q]);  // s_q = G_{u+1+q} before the step
        gb[i] = (float)step<NA>(av, s, (double)gb[i]);
      };
      if (n == kTileT) {
#pragma unroll
        for (int i = kTileT - 1; i >= 0; --i) bstep(i);
      } else {
#pragma unroll
        for (int i = kTileT - 1; i >= 0; --i)
          if (i < n) bstep(i);
      }
      regs_to_chunk(gb, gw, lanes, L, l0, t0, n, s_lds[k], lid);
    }
#pragma unroll
    for (int q = 0; q < NA; ++q) vk[q] = ga[q];
    __syncthreads();
    if (k == 0 && live) {
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        double t = 0.0;
        for (int j = 0; j < K; ++j) t += (vec_area<NA>(s_lds, j) + lid * NA)[q];
        part[(sc * lanes + lane) * NA + q] = t;
      }
    }
    __syncthreads();  // wave 0's reads of every vec area precede the next tile's loads into them
  }
}

// grad_a = -(sum over the n partials [n][lanes][NA] + y0 head taps) and grad_y0, per lane. One
// workgroup of 16 waves per 64 lanes: wave k sums the k-th of 16 contiguous segments of the
// partials, and wave 0 adds the 16 segment sums in order (fixed order, deterministic).
template <int NA>
__global__ void __launch_bounds__(1024) allpole_finish(const float* __restrict__ a, const float* __restrict__ gw,
                                                       const float* __restrict__ y0, const double* __restrict__ part,
                                                       float* __restrict__ ga, float* __restrict__ gy0, int64_t lanes,
                                                       int64_t L, int64_t n) {
  __shared__ double s_p[16][64];
  __shared__ double s_tot[NA][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t lane = blockIdx.x * 64 + lid;
  const bool live = lane < lanes;
  const int64_t seg = (n + 15) / 16;
  const int64_t r0 = k * seg, r1 = (r0 + seg < n) ? r0 + seg : n;
  for (int q = 0; q < NA; ++q) {
    double acc = 0.0;
    if (live)
      for (int64_t r = r0; r < r1; ++r) acc += part[(r * lanes + lane) * NA + q];
    s_p[k][lid] = acc;
    __syncthreads();
    if (k == 0) {
      double t = s_p[0][lid];
      for (int j = 1; j < 16; ++j) t += s_p[j][lid];
      s_tot[q][lid] = t;
    }
    __syncthreads();
  }
  if (k != 0 || !live) return;  // no barrier follows
  double Gh[NA];  // G_0 .. G_{NA-1}, zero past the end of the sequence
#pragma unroll
  for (int q = 0; q < NA; ++q) Gh[q] = (q < L) ? (double)gw[lane * L + q] : 0.0;
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    double t = s_tot[q][lid];
    if (y0) {
      // a_i (i = q + 1) also multiplied y_{t-i} = y0[i-t-1] for t < i
#pragma unroll
      for (int j = 1; j <= q + 1; ++j) t = fma(Gh[q + 1 - j], (double)y0[lane * NA + j - 1], t);
    }
    ga[lane * NA + q] = (float)(-t);
  }
  if (y0 && gy0) {
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      double t = 0.0;
#pragma unroll
      for (int i = j + 1; i <= NA; ++i) t = fma((double)a[lane * NA + i - 1], Gh[i - 1 - j], t);
      gy0[lane * NA + j] = (float)(-t);
    }
  }
}

struct Plan {
  int64_t T_c, nchunk;
  size_t off_M, off_e, off_S, off_part, bytes;
};

Plan plan(int64_t lanes, int64_t L, int64_t na) {
  Plan p;
  p.T_c = allpole_chunk(lanes, L, na);
  // a chunked sequence takes chunks of at most kColsT steps, whose transfer matrix is stepped
  // column by column, unless that needs more than 65535 chunks (one grid row each)
  if (p.T_c < L && p.T_c > kColsT && (L + kColsT - 1) / kColsT <= 65535) p.T_c = kColsT;
  p.nchunk = (L + p.T_c - 1) / p.T_c;
  const size_t f = 8;  // fp64 transfer matrices, carries and partials
  p.off_M = 0;
  p.off_e = p.off_M + f * lanes * na * na;
  p.off_S = p.off_e + f * p.nchunk * lanes * na;
  p.off_part = p.off_S + f * p.nchunk * lanes * na;
  p.bytes = p.off_part + f * p.nchunk * lanes * na;
  return p;
}

template <int NA>
void fwd_lb(int64_t lanes, int64_t L, const float* a, const float* w, const float* y0, float* y, char* ws,
            hipStream_t s) {
  static int occ[kMaxNA + 1];
  const LbPlan p = lb_plan(lanes, L, NA);
  double* Mc = reinterpret_cast<double*>(ws + p.off_Mc);
  double* Ms = reinterpret_cast<double*>(ws + p.off_Ms);
  const ResetJob rj = reset_job(ws, 2 * p.nsuper * lanes * NA, 64);
  hipLaunchKernelGGL((allpole_transfer2<NA>), dim3(transfer_grid(lanes, NA).x + rj.blocks), dim3(64), 0, s, a, Mc, Ms,
                     lanes, p.K, rj);
  const int64_t tiles = p.groups * p.nsuper, cap = resident_wgs(allpole_fwd_lb<NA>, 64 * p.K, occ);
  hipLaunchKernelGGL((allpole_fwd_lb<NA>), dim3((unsigned)(tiles < cap ? tiles : cap)), dim3(64 * p.K), 0, s, a, w,
                     y0, y, (const double*)Mc, (const double*)Ms, reinterpret_cast<double*>(ws + p.off_agg),
                     reinterpret_cast<double*>(ws + p.off_inc), reinterpret_cast<unsigned*>(ws), lanes, L, p.groups,
                     p.K, p.nsuper, lb_spacing_for(p.K));
}

template <int NA>
void bwd_lb(int64_t lanes, int64_t L, const float* g, const float* a, const float* y, const float* y0, float* gw,
            float* ga, float* gy0, char* ws, hipStream_t s) {
  static int occ[kMaxNA + 1];
  const LbPlan p = lb_plan(lanes, L, NA);
  double* part = reinterpret_cast<double*>(ws + p.off_part);
  if (L > 0) {
    double* Mc = reinterpret_cast<double*>(ws + p.off_Mc);
    double* Ms = reinterpret_cast<double*>(ws + p.off_Ms);
    const ResetJob rj = reset_job(ws, 2 * p.nsuper * lanes * NA, 64);
    hipLaunchKernelGGL((allpole_transfer2<NA>), dim3(transfer_grid(lanes, NA).x + rj.blocks), dim3(64), 0, s, a, Mc,
                       Ms, lanes, p.K, rj);
    const int64_t tiles = p.groups * p.nsuper, cap = resident_wgs(allpole_bwd_lb<NA>, 64 * p.K, occ);
    hipLaunchKernelGGL((allpole_bwd_lb<NA>), dim3((unsigned)(tiles < cap ? tiles : cap)), dim3(64 * p.K), 0, s, a, g,
                       y, (const double*)Mc, (const double*)Ms, reinterpret_cast<double*>(ws + p.off_agg),
                       reinterpret_cast<double*>(ws + p.off_inc), reinterpret_cast<unsigned*>(ws), gw, part, lanes, L,
                       p.groups, p.K, p.nsuper, lb_spacing_for(p.K));
  }
  hipLaunchKernelGGL((allpole_finish<NA>), dim3((unsigned)p.groups), dim3(1024), 0, s, a, gw, y0, (const double*)part,
                     ga, gy0, lanes, L, p.nsuper);
}

// M = C^{T_c} (needed only when the sequence takes more than one chunk; a single chunk enters
// from y0 directly)
template <int NA>
void transfer_launch(const Plan& p, const float* a, double* M, int64_t lanes, hipStream_t s) {
  if (p.T_c <= kColsT)
    hipLaunchKernelGGL((allpole_transfer_cols<NA>), dim3((unsigned)((lanes * NA + 63) / 64)), dim3(64), 0, s, a, M,
                       lanes, (int)p.T_c);
  else
    hipLaunchKernelGGL((allpole_transfer<NA>), grid_for(lanes), dim3(256), 0, s, a, M, lanes, p.T_c);
}

size_t workspace_bytes_for(int64_t lanes, int64_t L, int64_t na) {
  return na <= kLbNA ? lb_plan(lanes, L, na).bytes : plan(lanes, L, na).bytes;
}

template <int NA>
int fwd_impl(int64_t lanes, int64_t L, const float* a, const float* w, const float* y0, float* y, char* ws,
             hipStream_t s) {
  if constexpr (NA <= kLbNA) {
    fwd_lb<NA>(lanes, L, a, w, y0, y, ws, s);
    return tsf_launch_status();
  }
  const Plan p = plan(lanes, L, NA);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  double* e = reinterpret_cast<double*>(ws + p.off_e);
  double* S = reinterpret_cast<double*>(ws + p.off_S);
  const unsigned groups = (unsigned)((lanes + kTile - 1) / kTile);
  if (p.nchunk > 1) {
    transfer_launch<NA>(p, a, M, lanes, s);
    hipLaunchKernelGGL((allpole_fwd_chunk_end<NA>), dim3(groups, (unsigned)(p.nchunk - 1)), dim3(kTile), 0, s, a, w, e,
                       lanes, L, p.T_c, p.nchunk);
  }
  hipLaunchKernelGGL((allpole_fwd_carry<NA>), dim3((unsigned)((lanes + 15) / 16)), dim3(256), 0, s, M, e, y0, S,
                     lanes, p.nchunk);
  hipLaunchKernelGGL((allpole_fwd_apply<NA>), dim3(groups, (unsigned)p.nchunk), dim3(kTile), 0, s, a, w, S, y, lanes,
                     L, p.T_c, p.nchunk);
  return tsf_launch_status();
}

template <int NA>
int bwd_impl(int64_t lanes, int64_t L, const float* g, const float* a, const float* y, const float* y0, float* gw,
             float* ga, float* gy0, char* ws, hipStream_t s) {
  if constexpr (NA <= kLbNA) {
    bwd_lb<NA>(lanes, L, g, a, y, y0, gw, ga, gy0, ws, s);
    return tsf_launch_status();
  }
  const Plan p = plan(lanes, L, NA);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  double* f = reinterpret_cast<double*>(ws + p.off_e);
  double* R = reinterpret_cast<double*>(ws + p.off_S);
  double* part = reinterpret_cast<double*>(ws + p.off_part);
  if (L > 0) {
    const unsigned groups = (unsigned)((lanes + kTile - 1) / kTile);
    if (p.nchunk > 1) {
      transfer_launch<NA>(p, a, M, lanes, s);
      hipLaunchKernelGGL((allpole_bwd_chunk_start<NA>), dim3(groups, (unsigned)(p.nchunk - 1)), dim3(kTile), 0, s, a,
                         g, f, lanes, L, p.T_c, p.nchunk);
    }
    hipLaunchKernelGGL((allpole_bwd_carry<NA>), dim3((unsigned)((lanes + 15) / 16)), dim3(256), 0, s, M, f, R, lanes,
                       p.nchunk);
    hipLaunchKernelGGL((allpole_bwd_apply<NA>), dim3(groups, (unsigned)p.nchunk), dim3(kTile), 0, s, a, g, y, R, gw,
                       part, lanes, L, p.T_c, p.nchunk);
  }
  hipLaunchKernelGGL((allpole_finish<NA>), dim3((unsigned)((lanes + kTile - 1) / kTile)), dim3(1024), 0, s, a, gw, y0,
                     (const double*)part, ga, gy0, lanes, L, L > 0 ? p.nchunk : (int64_t)0);
  return tsf_launch_status();
}

#define TSF_NA_CASES(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15) X(16)

}  // namespace

extern "C" {

int64_t tsfast_hip_allpole_workspace_bytes(int64_t lanes, int64_t L, int64_t na) {
  if (lanes < 0 || L < 0 || na < 1 || na > kMaxNA) return -1;
  return (int64_t)workspace_bytes_for(lanes, L, na);
}

int tsfast_hip_allpole_fwd(int64_t lanes, int64_t L, int64_t na, const float* a, const float* w, const float* y0,
                           float* y, void* workspace, int64_t workspace_bytes, void* stream) {
  if (lanes < 0 || L < 0) return TSF_ERR_ARG;
  if (na < 1 || na > kMaxNA) return TSF_ERR_UNSUPPORTED;
  if (lanes == 0 || L == 0) return TSF_OK;
  if (!a || !w || !y) return TSF_ERR_ARG;
  if (!workspace || workspace_bytes < tsfast_hip_allpole_workspace_bytes(lanes, L, na)) return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  switch (na) {
#define X(K) \
  case K:    \
    return fwd_impl<K>(lanes, L, a, w, y0, y, ws, s);
    TSF_NA_CASES(X)
#undef X
  }
  return TSF_ERR_UNSUPPORTED;
}

int tsfast_hip_allpole_bwd(int64_t lanes, int64_t L, int64_t na, const float* g, const float* a, const float* y,
                           const float* y0, float* gw, float* ga, float* gy0, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  if (lanes < 0 || L < 0) return TSF_ERR_ARG;
  if (na < 1 || na > kMaxNA) return TSF_ERR_UNSUPPORTED;
  if (lanes == 0) return TSF_OK;
  if (!a || !ga || (L > 0 && (!g || !y || !gw))) return TSF_ERR_ARG;
  if (y0 && !gy0) return TSF_ERR_ARG;
  if (!workspace || workspace_bytes < tsfast_hip_allpole_workspace_bytes(lanes, L, na)) return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  switch (na) {
#define X(K) \
  case K:    \
    return bwd_impl<K>(lanes, L, g, a, y, y0, gw, ga, gy0, ws, s);
    TSF_NA_CASES(X)
#undef X
  }
  return TSF_ERR_UNSUPPORTED;
}

}  // extern "C"
