// Constant-matrix linear recurrence  x_t = A x_{t-1} + v_t  and its adjoint, float32 I/O.
//
// Reference semantics: tsfast/models/architectures/dynonet/core.py:23-52 (the log-doubling scan
// and the tsfast::linear_recurrence op, x0 folded into the first step), :60-73 (the analytic
// adjoint: G_t = A^T G_{t+1} + g_t, grad_v = G, grad_A = sum_t G_t x_{t-1}^T, grad_x0 = A^T G_1)
// and :103-127 (linear_recurrence, which broadcasts A, v and x0 to common leading dims).
//
// Layout: lanes are the flattened leading dims. A [lanes, n, n] row-major, v, x and g
// [lanes, L, n] (per lane the n state components of a step are contiguous, steps follow each
// other), x0 [lanes, n]. The state size n (1..8) is a template parameter, so a step is n x n
// fp64 FMAs on registers. n = 1..4 take the single-pass look-back scan described next; n = 5..8,
// whose n x n matrices and n-vectors do not fit that scan's registers and look-back areas, take
// the two-pass path at the end of the file.
//
// A lane's sequence is one row of L * n floats, so a chunk of S = floor(32 / n) steps is a row
// segment of S * n <= 32 floats, and the [64 x 33] LDS tiles of the all-pole scan move the
// segments of 64 lanes with coalesced 128-byte row accesses. The parallel structure is the
// single-pass look-back scan of allpole_core.h with a dense step: a chunk maps its entering state
// s to Mc s + e (Mc = A^S), a super-chunk of K chunks to Ms s + e (Ms = A^(S K)), and only the
// e vectors are published between workgroups. The adjoint runs the same machinery from the right
// end with A^T; its grad_A partials are summed over the K chunks of a tile in LDS, written per
// super-chunk, and added up in a fixed order by linrec_finish. (With the look-back in its
// deterministic mode, lookback.h, every output is then bitwise reproducible run to run.)
//
// Arithmetic: fp32 in and out, fp64 state, transfer matrices, published words and grad_A sums.

#include <initializer_list>

#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

#include "allpole_core.h"

constexpr int kMaxNS = 4;  // state sizes on the single-pass path (an n x n fp64 matrix per thread)
static_assert(kMaxNS <= kLbNA, "the look-back areas hold kLbNA doubles per lane");
constexpr int kMaxWideNS = 8;  // state sizes 5..8 take the two-pass path below

template <int NS>
constexpr int steps_per_chunk() {
  return kTileT / NS;
}

// Transfer matrices per lane: Mc = P^S and Ms = P^(S K) with P = A (forward) or A^T (adjoint),
// one thread per (lane, column c): column c is P applied S K times to the unit vector e_c, in
// fp64. (Repeated squaring would compound rounding errors through the transient growth of
// non-normal powers, which for companion matrices with poles near the unit circle reach 1e5
// before they decay; step-by-step application keeps them at the level of the recurrence itself.)
// The last rj.blocks workgroups run the scan's look-back reset instead.
template <int NS>
__global__ void __launch_bounds__(256) linrec_transfer(const float* __restrict__ A, double* __restrict__ Mc,
                                                       double* __restrict__ Ms, int64_t lanes, int K, int transpose,
                                                       ResetJob rj) {
  const unsigned tb = gridDim.x - rj.blocks;
  if (blockIdx.x >= tb) {
    run_reset(rj, blockIdx.x - tb);
    return;
  }
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= lanes * NS) return;
  const int64_t lane = idx / NS;
  const int col = (int)(idx - lane * NS);
  constexpr int S = steps_per_chunk<NS>();
  double P[NS][NS], x[NS];
  const float* a = A + lane * NS * NS;
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    x[r] = r == col ? 1.0 : 0.0;
#pragma unroll
    for (int c = 0; c < NS; ++c) P[r][c] = (double)(transpose ? a[c * NS + r] : a[r * NS + c]);
  }
  double* mc = Mc + lane * NS * NS + col;
  double* ms = Ms + lane * NS * NS + col;
  // blocks of S steps, unrolled (no per-step branch; independent work scheduled around the chain)
  for (int blk = 0; blk < K; ++blk) {
#pragma unroll
    for (int step = 0; step < S; ++step) {
      double y[NS];
#pragma unroll
      for (int r = 0; r < NS; ++r) {
        double acc = 0.0;
#pragma unroll
        for (int c = 0; c < NS; ++c) acc = fma(P[r][c], x[c], acc);
        y[r] = acc;
      }
#pragma unroll
      for (int r = 0; r < NS; ++r) x[r] = y[r];
    }
    if (blk == 0)
#pragma unroll
      for (int r = 0; r < NS; ++r) mc[r * NS] = x[r];
  }
#pragma unroll
  for (int r = 0; r < NS; ++r) ms[r * NS] = x[r];
}

// The lane's matrix (or its transpose) in fp64. The kernels load it once before the look-back
// and again after it, through a pointer the compiler cannot see through, so that the n x n
// doubles are not held in registers across the look-back (an L2 hit instead of a spill).
template <int NS>
TSF_DEV void load_lane_matrix(double (&m)[NS][NS], const float* A, int64_t lane, bool live, bool transpose) {
  asm volatile("" : "+v"(A));
  const float* a = A + lane * NS * NS;
#pragma unroll
  for (int r = 0; r < NS; ++r)
#pragma unroll
    for (int c = 0; c < NS; ++c) m[r][c] = live ? (double)a[transpose ? c * NS + r : r * NS + c] : 0.0;
}

// One step s <- m s + x (x the NS floats of the step).
template <int NS>
TSF_DEV void dense_step(const double (&m)[NS][NS], double (&s)[NS], const float* x) {
  double t[NS];
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    double acc = (double)x[r];
#pragma unroll
    for (int c = 0; c < NS; ++c) acc = fma(m[r][c], s[c], acc);
    t[r] = acc;
  }
#pragma unroll
  for (int r = 0; r < NS; ++r) s[r] = t[r];
}

// Forward. A tile is 64 lanes x one super-chunk of K chunks; wave k owns chunk k. The wave moves
// its chunk's row segments through its LDS tile into registers, summarises the chunk from a zero
// state, and after the look-back re-runs it from its entering state, writing x in place of v.
template <int NS>
__global__ void __launch_bounds__(64 * kLbWaves) __attribute__((amdgpu_waves_per_eu(4))) linrec_fwd_lb(
    const float* __restrict__ A, const float* __restrict__ v, const float* __restrict__ x0, float* __restrict__ x,
    const double* __restrict__ Mc, const double* __restrict__ Ms, double* __restrict__ agg, double* __restrict__ inc,
    unsigned* __restrict__ counter, int64_t lanes, int64_t L, int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  constexpr int S = steps_per_chunk<NS>(), NN = NS * NS;
  __shared__ LdsTile s_lds[kLbWaves];
  __shared__ int s_flag[kLbWaves][64];
  __shared__ int s_pend[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  __shared__ double s_mat[MatStage<NS>::kDoubles];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * S, row = L * NS;
  // This wave's chunk of a tile: first lane, first step and length.
  auto chunk_of = [&](int64_t tile, int64_t& sc, int64_t& l0, int64_t& t0) __attribute__((always_inline)) {
    sc = tile / groups;
    l0 = (tile - sc * groups) * kTile;
    t0 = sc * SL + (int64_t)k * S;
    return (L - t0) >= S ? S : (L - t0) > 0 ? (int)(L - t0) : 0;
  };
  // For small states the next tile's chunk is fetched into rg while the current tile finishes
  // (after its look-back), so its load latency overlaps the re-run and the stores; larger states
  // have no registers to spare and load each chunk when its tile starts.
  constexpr bool kPrefetch = NS <= 2;
  TileRegs rg;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  if (kPrefetch && (int64_t)s_tile[0] < tiles) {
    int64_t sc0, l00, t00;
    const int n0 = chunk_of(s_tile[0], sc0, l00, t00);
    if (n0 > 0) tile_fetch(rg, v, lanes, row, l00, t00 * NS, n0 * NS, lid);
  }
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    int64_t sc, l0, t0;
    const int n = chunk_of(tile, sc, l0, t0);
    const int64_t lane = l0 + lid;
    const bool live = lane < lanes;
    double s[NS];
#pragma unroll
    for (int r = 0; r < NS; ++r) s[r] = 0.0;
    float xb[kTileT];
    if (n > 0 && !kPrefetch) tile_fetch(rg, v, lanes, row, l0, t0 * NS, n * NS, lid);
    if (n > 0) {
      tile_put(rg, s_lds[k], lid);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < kTileT; ++i) xb[i] = s_lds[k][lid][i];
      __builtin_amdgcn_wave_barrier();
    }
    if constexpr (MatStage<NS>::kLds) stage_mats<NS>(s_mat, Mc, Ms, l0, lanes);
    {
      double am[NS][NS];
      load_lane_matrix<NS>(am, A, lane, live, false);
      if (n == S) {
#pragma unroll
        for (int i = 0; i < S; ++i) dense_step<NS>(am, s, &xb[i * NS]);
      } else {
#pragma unroll
        for (int i = 0; i < S; ++i)
          if (i < n) dense_step<NS>(am, s, &xb[i * NS]);
      }
    }
    double* vk = vec_area<NS>(s_lds, k) + lid * NS;
#pragma unroll
    for (int q = 0; q < NS; ++q) vk[q] = s[q];
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    // wave 0: the super-chunk's zero-state end (chunks before a non-empty one are full, so Mc is
    // every fold's matrix; the map is published only for full super-chunks)
    double sup[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) sup[q] = 0.0;
    if (k == 0 && live) {
      double mc[NS][NS];
      load_mat<NS>(mc, MatStage<NS>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = 0; j < K; ++j) {
        double ej[NS];
        const double* vj = vec_area<NS>(s_lds, j) + lid * NS;
#pragma unroll
        for (int q = 0; q < NS; ++q) ej[q] = vj[q];
        matvec_add<NS>(sup, mc, sup, ej);
      }
      if (lb_pub_agg(sc, lb_spacing) && sc + 1 < nsuper) put_vec<NS>(agg + (sc * lanes + lane) * NS, sup);
    }
    double St[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) St[q] = (sc == 0 && x0 && live && k == 0) ? (double)x0[lane * NS + q] : 0.0;
    if (sc > 0)  // uniform over the workgroup
      ap_look_back<NS>(St, agg, inc, MatStage<NS>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN, k == 0 && live, sc - 1, (int64_t)-1, nsuper, lanes, lane, K,
                       k, lid, s_lds, s_flag, s_pend, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(sc, lb_spacing) && sc + 1 < nsuper) {
        double ms[NS][NS], o[NS];
        load_mat<NS>(ms, MatStage<NS>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN);
        matvec_add<NS>(o, ms, St, sup);
        put_vec<NS>(inc + (sc * lanes + lane) * NS, o);
      }
      double mc[NS][NS];
      load_mat<NS>(mc, MatStage<NS>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = 0; j < K; ++j) {  // entering state of every chunk, in place of its summary
        double ej[NS];
        double* vj = vec_area<NS>(s_lds, j) + lid * NS;
#pragma unroll
        for (int q = 0; q < NS; ++q) {
          ej[q] = vj[q];
          vj[q] = St[q];
        }
        matvec_add<NS>(St, mc, St, ej);
      }
    }
    if (kPrefetch && (int64_t)s_tile[buf ^ 1] < tiles) {  // prefetch the next tile's chunk
      int64_t sc1, l01, t01;
      const int n1 = chunk_of(s_tile[buf ^ 1], sc1, l01, t01);
      if (n1 > 0) tile_fetch(rg, v, lanes, row, l01, t01 * NS, n1 * NS, lid);
    }
    __syncthreads();
    if (n > 0) {
#pragma unroll
      for (int q = 0; q < NS; ++q) s[q] = vk[q];
      double am[NS][NS];
      load_lane_matrix<NS>(am, A, lane, live, false);
      auto fstep = [&](int i) __attribute__((always_inline)) {
        dense_step<NS>(am, s, &xb[i * NS]);
#pragma unroll
        for (int r = 0; r < NS; ++r) xb[i * NS + r] = (float)s[r];
      };
      if (n == S) {
#pragma unroll
        for (int i = 0; i < S; ++i) fstep(i);
      } else {
#pragma unroll
        for (int i = 0; i < S; ++i)
          if (i < n) fstep(i);
      }
      __builtin_amdgcn_wave_barrier();
      regs_to_chunk(xb, x, lanes, row, l0, t0 * NS, n * NS, s_lds[k], lid);
    }
  }
}

// Backward: G_t = A^T G_{t+1} + g_t is the same scan from the right end with A^T (Mc and Ms are
// the powers of A^T here). After the look-back each wave re-runs its chunk from the right, writes
// grad_v = G, and accumulates grad_A += G_t x_{t-1}^T in fp64, with x_{t-1} from the forward
// output (loaded after the look-back, so it does not stay in registers across it) or x0. The
// tile's K per-chunk sums are added in LDS and written per super-chunk.
template <int NS>
__global__ void __launch_bounds__(64 * kLbWaves) __attribute__((amdgpu_waves_per_eu(4))) linrec_bwd_lb(
    const float* __restrict__ A, const float* __restrict__ g, const float* __restrict__ out,
    const float* __restrict__ x0, float* __restrict__ gv, float* __restrict__ gx0, const double* __restrict__ Mc,
    const double* __restrict__ Ms, double* __restrict__ agg, double* __restrict__ inc, double* __restrict__ part,
    unsigned* __restrict__ counter, int64_t lanes, int64_t L, int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  constexpr int S = steps_per_chunk<NS>(), NN = NS * NS;
  static_assert(64 * NN * sizeof(double) <= sizeof(LdsTile), "a wave's grad_A sums fit in its tile");
  __shared__ LdsTile s_lds[kLbWaves];
  __shared__ int s_flag[kLbWaves][64];
  __shared__ int s_pend[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  __shared__ double s_mat[MatStage<NS>::kDoubles];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * S, row = L * NS;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t r = tile / groups, sc = nsuper - 1 - r, l0 = (tile - r * groups) * kTile, lane = l0 + lid;
    const bool live = lane < lanes;
    const int64_t t0 = sc * SL + (int64_t)k * S;
    const int n = (L - t0) >= S ? S : (L - t0) > 0 ? (int)(L - t0) : 0;
    double s[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) s[i] = 0.0;
    float gb[kTileT];
    if constexpr (MatStage<NS>::kLds) stage_mats<NS>(s_mat, Mc, Ms, l0, lanes);
    if (n > 0) chunk_to_regs(gb, g, lanes, row, l0, t0 * NS, n * NS, s_lds[k], lid);
    {
      double at[NS][NS];  // A^T
      load_lane_matrix<NS>(at, A, lane, live, true);
      if (n == S) {
#pragma unroll
        for (int i = S - 1; i >= 0; --i) dense_step<NS>(at, s, &gb[i * NS]);
      } else {
#pragma unroll
        for (int i = S - 1; i >= 0; --i)
          if (i < n) dense_step<NS>(at, s, &gb[i * NS]);
      }
    }
    double* vk = vec_area<NS>(s_lds, k) + lid * NS;
#pragma unroll
    for (int q = 0; q < NS; ++q) vk[q] = s[q];
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    // wave 0: the super-chunk's exit to the left from a zero entering state, folded from its
    // rightmost chunk (chunks past the end of the sequence are empty and contribute zero)
    double sup[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) sup[q] = 0.0;
    if (k == 0 && live) {
      double mc[NS][NS];
      load_mat<NS>(mc, MatStage<NS>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = K - 1; j >= 0; --j) {
        double fj[NS];
        const double* vj = vec_area<NS>(s_lds, j) + lid * NS;
#pragma unroll
        for (int q = 0; q < NS; ++q) fj[q] = vj[q];
        matvec_add<NS>(sup, mc, sup, fj);
      }
      if (lb_pub_agg(nsuper - 1 - sc, lb_spacing) && sc > 0) put_vec<NS>(agg + (sc * lanes + lane) * NS, sup);
    }
    double R[NS];  // adjoint state entering the super-chunk from the right
#pragma unroll
    for (int q = 0; q < NS; ++q) R[q] = 0.0;
    if (sc + 1 < nsuper)  // uniform over the workgroup
      ap_look_back<NS>(R, agg, inc, MatStage<NS>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN, k == 0 && live, sc + 1, (int64_t)1, nsuper, lanes, lane, K, k, lid,
                       s_lds, s_flag, s_pend, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(nsuper - 1 - sc, lb_spacing) && sc > 0) {
        double ms[NS][NS], o[NS];
        load_mat<NS>(ms, MatStage<NS>::kLds ? &s_mat[64 * NN + lid * NN] : Ms + lane * NN);
        matvec_add<NS>(o, ms, R, sup);
        put_vec<NS>(inc + (sc * lanes + lane) * NS, o);
      }
      double mc[NS][NS];
      load_mat<NS>(mc, MatStage<NS>::kLds ? &s_mat[lid * NN] : Mc + lane * NN);
      for (int j = K - 1; j >= 0; --j) {  // state entering every chunk from the right
        double fj[NS];
        double* vj = vec_area<NS>(s_lds, j) + lid * NS;
#pragma unroll
        for (int q = 0; q < NS; ++q) {
          fj[q] = vj[q];
          vj[q] = R[q];
        }
        matvec_add<NS>(R, mc, R, fj);
      }
    }
    __syncthreads();
    double acc[NN];
#pragma unroll
    for (int q = 0; q < NN; ++q) acc[q] = 0.0;
    if (n > 0) {
#pragma unroll
      for (int q = 0; q < NS; ++q) s[q] = vk[q];
      double at[NS][NS];
      load_lane_matrix<NS>(at, A, lane, live, true);
      auto bstep = [&](int i) __attribute__((always_inline)) {
        dense_step<NS>(at, s, &gb[i * NS]);
#pragma unroll
        for (int q = 0; q < NS; ++q) gb[i * NS + q] = (float)s[q];
      };
      if (n == S) {
#pragma unroll
        for (int i = S - 1; i >= 0; --i) bstep(i);
      } else {
#pragma unroll
        for (int i = S - 1; i >= 0; --i)
          if (i < n) bstep(i);
      }
      // grad_x0 = A^T G at the first step, from the chunk that holds it
      if (t0 == 0 && gx0 && live) {
#pragma unroll
        for (int q = 0; q < NS; ++q) {
          double t = 0.0;
#pragma unroll
          for (int c = 0; c < NS; ++c) t = fma(at[q][c], s[c], t);
          gx0[lane * NS + q] = (float)t;
        }
      }
      __builtin_amdgcn_wave_barrier();
      regs_to_chunk(gb, gv, lanes, row, l0, t0 * NS, n * NS, s_lds[k], lid);
      // x_{t-1} for the chunk's steps: x at t0 - 1 (or x0), then the chunk's own outputs but the last
      float pv[NS];
#pragma unroll
      for (int q = 0; q < NS; ++q)
        pv[q] = !live ? 0.0f : t0 > 0 ? out[lane * row + (t0 - 1) * NS + q] : (x0 ? x0[lane * NS + q] : 0.0f);
      float xc[kTileT];
      chunk_to_regs(xc, out, lanes, row, l0, t0 * NS, n * NS, s_lds[k], lid);
      auto gstep = [&](int i) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < NS; ++p)
#pragma unroll
          for (int c = 0; c < NS; ++c)
            acc[p * NS + c] = fma((double)gb[i * NS + p], (double)(i == 0 ? pv[c] : xc[(i - 1) * NS + c]),
                                  acc[p * NS + c]);
      };
      if (n == S) {
#pragma unroll
        for (int i = 0; i < S; ++i) gstep(i);
      } else {
#pragma unroll
        for (int i = 0; i < S; ++i)
          if (i < n) gstep(i);
      }
    }
    // the K chunks' grad_A sums, added in LDS in chunk order, one partial per super-chunk
    double* ak = reinterpret_cast<double*>(&s_lds[k][0][0]) + lid * NN;
#pragma unroll
    for (int q = 0; q < NN; ++q) ak[q] = acc[q];
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * NN; e += blockDim.x) {
      const int el = e / NN, q = e - el * NN;
      if (l0 + el < lanes) {
        double t = 0.0;
        for (int j = 0; j < K; ++j) t += reinterpret_cast<const double*>(&s_lds[j][0][0])[el * NN + q];
        part[(sc * lanes + l0 + el) * NN + q] = t;
      }
    }
    __syncthreads();  // every read of the tiles precedes the next tile's loads into them
  }
}

// grad_A = the sum of the super-chunks' partials [nsuper][lanes * n * n]. A workgroup of 16 waves
// owns 64 consecutive entries: wave k sums the k-th of 16 contiguous runs of super-chunks (64
// consecutive doubles per read), and the 16 run sums are added in order (deterministic).
__global__ void __launch_bounds__(1024) linrec_finish(const double* __restrict__ part, float* __restrict__ gA,
                                                      int64_t entries, int64_t nsuper) {
  __shared__ double s_p[16][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t e = blockIdx.x * 64 + lid;
  const int64_t seg = (nsuper + 15) / 16;
  const int64_t r0 = k * seg, r1 = (r0 + seg < nsuper) ? r0 + seg : nsuper;
  double acc = 0.0;
  if (e < entries)
    for (int64_t r = r0; r < r1; ++r) acc += part[r * entries + e];
  s_p[k][lid] = acc;
  __syncthreads();
  if (k == 0 && e < entries) {
    double t = s_p[0][lid];
    for (int j = 1; j < 16; ++j) t += s_p[j][lid];
    gA[e] = (float)t;
  }
}

__global__ void __launch_bounds__(256) linrec_zero(float* __restrict__ p, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// Plan: K (chunks per tile) starts at kLbWaves and halves down to 2 while there are fewer than
// kApTileTarget tiles. Workspace: the tile counter, agg and inc [nsuper][lanes][n] (reset
// before each scan), the grad_A partials [nsuper][lanes][n][n], and Mc, Ms [lanes][n][n].
struct LrPlan {
  int64_t groups = 0, nsuper = 0;
  int K = 1;
  size_t off_agg = 0, off_inc = 0, off_part = 0, off_Mc = 0, off_Ms = 0, bytes = 0;
};

LrPlan lr_plan(int64_t lanes, int64_t L, int64_t ns) {
  LrPlan p;
  const int64_t S = kTileT / ns;
  p.groups = (lanes + kTile - 1) / kTile;
  if (L > 0) {
    p.K = kLbWaves;
    auto tiles = [&](int K) { return p.groups * ((L + S * K - 1) / (S * K)); };
    while (p.K > 2 && tiles(p.K) < kApTileTarget) p.K /= 2;
    const int64_t chunks = (L + S - 1) / S;
    if (p.K > chunks) p.K = (int)chunks;
    p.nsuper = (L + S * p.K - 1) / (S * p.K);
  }
  const size_t f = 8, vecs = f * p.nsuper * lanes * ns;
  p.off_agg = kCounterBytes;
  p.off_inc = p.off_agg + vecs;
  p.off_part = p.off_inc + vecs;
  p.off_Mc = p.off_part + vecs * ns;
  p.off_Ms = p.off_Mc + f * lanes * ns * ns;
  p.bytes = p.off_Ms + f * lanes * ns * ns;
  return p;
}

inline unsigned blocks_for(int64_t threads) { return (unsigned)((threads + 255) / 256); }

template <int NS>
int fwd_impl(int64_t lanes, int64_t L, const float* A, const float* v, const float* x0, float* x, char* ws,
             hipStream_t s) {
  static int occ[kLbWaves + 1];
  const LrPlan p = lr_plan(lanes, L, NS);
  double* Mc = reinterpret_cast<double*>(ws + p.off_Mc);
  double* Ms = reinterpret_cast<double*>(ws + p.off_Ms);
  const ResetJob rj = reset_job(ws, 2 * p.nsuper * lanes * NS, 256);
  hipLaunchKernelGGL((linrec_transfer<NS>), dim3(blocks_for(lanes * NS) + rj.blocks), dim3(256), 0, s, A, Mc, Ms, lanes,
                     p.K, 0, rj);
  const int64_t tiles = p.groups * p.nsuper, cap = resident_wgs(linrec_fwd_lb<NS>, 64 * p.K, occ);
  hipLaunchKernelGGL((linrec_fwd_lb<NS>), dim3((unsigned)(tiles < cap ? tiles : cap)), dim3(64 * p.K), 0, s, A, v, x0,
                     x, (const double*)Mc, (const double*)Ms, reinterpret_cast<double*>(ws + p.off_agg),
                     reinterpret_cast<double*>(ws + p.off_inc), reinterpret_cast<unsigned*>(ws), lanes, L, p.groups,
                     p.K, p.nsuper, lb_spacing_for(p.K));
  return tsf_launch_status();
}

template <int NS>
int bwd_impl(int64_t lanes, int64_t L, const float* g, const float* A, const float* out, const float* x0, float* gA,
             float* gv, float* gx0, char* ws, hipStream_t s) {
  static int occ[kLbWaves + 1];
  if (L == 0) {  // no steps: grad_A = 0, grad_x0 = A^T G_1 with G empty = 0
    hipLaunchKernelGGL(linrec_zero, dim3(blocks_for(lanes * NS * NS)), dim3(256), 0, s, gA, lanes * NS * NS);
    if (gx0) hipLaunchKernelGGL(linrec_zero, dim3(blocks_for(lanes * NS)), dim3(256), 0, s, gx0, lanes * NS);
    return tsf_launch_status();
  }
  const LrPlan p = lr_plan(lanes, L, NS);
  double* Mc = reinterpret_cast<double*>(ws + p.off_Mc);
  double* Ms = reinterpret_cast<double*>(ws + p.off_Ms);
  double* part = reinterpret_cast<double*>(ws + p.off_part);
  const ResetJob rj = reset_job(ws, 2 * p.nsuper * lanes * NS, 256);
  hipLaunchKernelGGL((linrec_transfer<NS>), dim3(blocks_for(lanes * NS) + rj.blocks), dim3(256), 0, s, A, Mc, Ms, lanes,
                     p.K, 1, rj);
  const int64_t tiles = p.groups * p.nsuper, cap = resident_wgs(linrec_bwd_lb<NS>, 64 * p.K, occ);
  hipLaunchKernelGGL((linrec_bwd_lb<NS>), dim3((unsigned)(tiles < cap ? tiles : cap)), dim3(64 * p.K), 0, s, A, g, out,
                     x0, gv, gx0, (const double*)Mc, (const double*)Ms, reinterpret_cast<double*>(ws + p.off_agg),
                     reinterpret_cast<double*>(ws + p.off_inc), part, reinterpret_cast<unsigned*>(ws), lanes, L,
                     p.groups, p.K, p.nsuper, lb_spacing_for(p.K));
  hipLaunchKernelGGL(linrec_finish, dim3((unsigned)((lanes * NS * NS + 63) / 64)), dim3(1024), 0, s,
                     (const double*)part, gA, lanes * NS * NS, p.nsuper);
  return tsf_launch_status();
}

#define TSF_NS_CASES(X) X(1) X(2) X(3) X(4)

// ------------------------------------------------------------------------------ n = 5..8
// Two-pass path for state sizes above the single-pass kernels' look-back areas. Two threads per
// lane and chunk of kWideT steps (each owning half the state rows), no waiting between workgroups:
//   forward:  chunk ends from a zero state (e) -> per lane, the entering state of every chunk by a
//             sequential carry over the chunks with M = A^kWideT -> every chunk re-run from its
//             entering state, writing x;
//   backward: chunk starts of the adjoint from a zero right-end state (f) -> per lane, the adjoint
//             entering every chunk from the right with M = (A^T)^kWideT, and grad_x0 -> every
//             chunk re-run backwards, writing grad_v and its grad_A partial; linrec_finish adds the
//             partials up in chunk order.
// A stays fp32 in registers (exact in fp64 on use); state, carries and partials are fp64.
constexpr int kWideT = 256;
constexpr int kWidePf = 4;  // steps fetched ahead by the chunk kernels
constexpr int kWideThreads = 256;

// One step's NS floats of a lane's row, VEC floats per access (VEC divides NS; the host picks
// VEC = 4 or 2 only when every row pointer is aligned to it).
template <int NS, int VEC>
TSF_DEV void ld_step(float (&d)[NS], const float* __restrict__ p) {
  if constexpr (VEC == 4) {
#pragma unroll
    for (int i = 0; i < NS; i += 4) {
      const float4 q = *reinterpret_cast<const float4*>(p + i);
      d[i] = q.x; d[i + 1] = q.y; d[i + 2] = q.z; d[i + 3] = q.w;
    }
  } else if constexpr (VEC == 2) {
#pragma unroll
    for (int i = 0; i < NS; i += 2) {
      const float2 q = *reinterpret_cast<const float2*>(p + i);
      d[i] = q.x; d[i + 1] = q.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NS; ++i) d[i] = p[i];
  }
}

// M = P^e per lane, P = A or A^T, one thread per (lane, column c): column c is P applied e times
// to the unit vector e_c in fp64 (step-by-step, as linrec_transfer, for the same accuracy reason).
template <int NS>
__global__ void __launch_bounds__(64) lw_power(const float* __restrict__ A, double* __restrict__ M, int64_t lanes,
                                                int e, int transpose) {
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= lanes * NS) return;
  const int64_t lane = idx / NS;
  const int col = (int)(idx - lane * NS);
  double P[NS][NS], x[NS];
  const float* a = A + lane * NS * NS;
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    x[r] = r == col ? 1.0 : 0.0;
#pragma unroll
    for (int c = 0; c < NS; ++c) P[r][c] = (double)(transpose ? a[c * NS + r] : a[r * NS + c]);
  }
#pragma unroll 8
  for (int step = 0; step < e; ++step) {
    double y[NS];
#pragma unroll
    for (int r = 0; r < NS; ++r) {
      double acc = 0.0;
#pragma unroll
      for (int c = 0; c < NS; ++c) acc = fma(P[r][c], x[c], acc);
      y[r] = acc;
    }
#pragma unroll
    for (int r = 0; r < NS; ++r) x[r] = y[r];
  }
#pragma unroll
  for (int r = 0; r < NS; ++r) M[lane * NS * NS + r * NS + col] = x[r];
}

// The chunk kernels run two threads per lane (adjacent threads): thread h = threadIdx.x & 1 owns
// state rows h * NH .. h * NH + NH - 1 (NH = ceil(n / 2); rows past n are zero padding), the
// same rows of the step matrix P (A forward, A^T adjoint) split into the owned and the partner's
// columns, and, in the adjoint re-run, the same rows of grad_A. A step reads the partner's
// components by a DPP lane swap and sums the owned components' terms first. One thread per lane
// held 228 VGPRs (the adjoint re-run 360, with the n x n fp64 grad_A accumulators): one or two
// waves per SIMD, latency-bound.
constexpr int half_rows(int ns) { return (ns + 1) / 2; }
constexpr int kWideLanes = kWideThreads / 2;  // lanes per workgroup

template <int NS, bool TR>
TSF_DEV void half_matrix(float (&mo)[half_rows(NS)][half_rows(NS)], float (&mp)[half_rows(NS)][half_rows(NS)],
                         const float* __restrict__ a, int own0, int par0) {
  constexpr int NH = half_rows(NS);
#pragma unroll
  for (int i = 0; i < NH; ++i)
#pragma unroll
    for (int j = 0; j < NH; ++j) {
      const int oi = own0 + i, oj = own0 + j, pi = par0 + i;
      // P[r][c] = TR ? A[c][r] : A[r][c]; mo[i][j] = P[oj][oi], mp[i][j] = P[oj][pi]
      mo[i][j] = (oi < NS && oj < NS) ? (TR ? a[oi * NS + oj] : a[oj * NS + oi]) : 0.0f;
      mp[i][j] = (pi < NS && oj < NS) ? (TR ? a[pi * NS + oj] : a[oj * NS + pi]) : 0.0f;
    }
}
// the partner's (lane ^ 1) values of s
template <int NH>
TSF_DEV void half_swap(double (&sp)[NH], const double (&s)[NH]) {
#pragma unroll
  for (int i = 0; i < NH; ++i) {
    const uint64_t b = (uint64_t)__double_as_longlong(s[i]);
    // quad_perm [1,0,3,2] reads a lane of every pair, so no lane keeps its old value: mov_dpp
    // (no old operand) spares the zeroing move update_dpp(0, ...) would need per word
    const uint64_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, 0xB1, 0xF, 0xF, false);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), 0xB1, 0xF, 0xF, false);
    sp[i] = __longlong_as_double((long long)((hi << 32) | lo));
  }
}
// owned rows of s <- P s + x; called by both threads of every pair together
template <int NH>
TSF_DEV void half_step(const float (&mo)[NH][NH], const float (&mp)[NH][NH], double (&s)[NH], const float (&x)[NH]) {
  double sp[NH], t[NH];
  half_swap<NH>(sp, s);
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    double acc = (double)x[j];
#pragma unroll
    for (int i = 0; i < NH; ++i) acc = fma((double)mo[i][j], s[i], acc);
#pragma unroll
    for (int i = 0; i < NH; ++i) acc = fma((double)mp[i][j], sp[i], acc);
    t[j] = acc;
  }
#pragma unroll
  for (int j = 0; j < NH; ++j) s[j] = t[j];
}
// access width of a thread's half of a step (its rows start own0 floats into the step)
template <int NS, int VEC>
constexpr int half_vec() {
  return (VEC == 4 && half_rows(NS) % 4 == 0) ? 4 : (VEC >= 2 && half_rows(NS) % 2 == 0) ? 2 : 1;
}
// the owned rows of one step: p points at the step's row own0 (padding rows read as zero). A
// padding row (odd NS, second thread) reads the step's last row and keeps zero, so every load is
// unconditional; with MASKED it is a masked load instead. Measured per kernel at n 5 and 7: the
// unconditional form made the chunk sums 8-19% faster and n 5's adjoint re-run 4%, and n 7's
// adjoint re-run 8% slower, which therefore keeps the masked form.
template <int NS, int VH, bool MASKED = false>
TSF_DEV void ld_half(float (&d)[half_rows(NS)], const float* __restrict__ p, int own0) {
  constexpr int NH = half_rows(NS);
  if constexpr (VH > 1) {
    ld_step<NH, VH>(d, p);  // NS even: no padding rows
  } else if constexpr (MASKED) {
#pragma unroll
    for (int i = 0; i < NH; ++i) d[i] = (own0 + i < NS) ? p[i] : 0.0f;
  } else {
#pragma unroll
    for (int i = 0; i < NH; ++i) {
      const float v = p[own0 + i < NS ? i : NS - 1 - own0];
      d[i] = own0 + i < NS ? v : 0.0f;
    }
  }
}
struct HalfIdx {
  int h, ll, own0, par0;
  int64_t lane, c, t0, t1;
  bool live;
};
TSF_DEV HalfIdx half_idx(int64_t lanes, int64_t L, int NH) {
  HalfIdx q;
  q.h = threadIdx.x & 1;
  q.ll = threadIdx.x >> 1;
  q.own0 = q.h * NH;
  q.par0 = (1 - q.h) * NH;
  q.lane = blockIdx.x * (int64_t)kWideLanes + q.ll;
  q.live = q.lane < lanes;
  q.c = blockIdx.y;
  q.t0 = q.c * kWideT;
  q.t1 = (q.t0 + kWideT < L) ? q.t0 + kWideT : L;
  return q;
}

// Forward chunk ends from a zero state: e [nchunks][lanes][NS]
template <int NS, int VEC>
__global__ void __launch_bounds__(kWideThreads) lw_sum_fwd(const float* __restrict__ A, const float* __restrict__ v,
                                                           double* __restrict__ e, int64_t lanes, int64_t L) {
  constexpr int NH = half_rows(NS), VH = half_vec<NS, VEC>();
  const HalfIdx q = half_idx(lanes, L, NH);
  if (!q.live) return;  // both threads of a pair
  float mo[NH][NH], mp[NH][NH];
  half_matrix<NS, false>(mo, mp, A + q.lane * NS * NS, q.own0, q.par0);
  double s[NH];
#pragma unroll
  for (int i = 0; i < NH; ++i) s[i] = 0.0;
  const float* row = v + q.lane * L * NS + q.own0;
  // kWidePf steps' loads in flight: step t + kWidePf is fetched while step t computes. The whole
  // blocks run without per-step branches: a fetch past the chunk's end re-reads its last step
  // (never used), and the remaining n % kWidePf steps follow the loop.
  const int64_t t0 = q.t0, tl = q.t1 - 1, n = q.t1 - q.t0, nfull = n - n % kWidePf;
  float d[kWidePf][NH];
#pragma unroll
  for (int k = 0; k < kWidePf; ++k) ld_half<NS, VH>(d[k], row + (t0 + k < tl ? t0 + k : tl) * NS, q.own0);
  for (int64_t tb = t0; tb < t0 + nfull; tb += kWidePf) {
#pragma unroll
    for (int k = 0; k < kWidePf; ++k) {
      half_step<NH>(mo, mp, s, d[k]);
      const int64_t tn = tb + k + kWidePf;
      ld_half<NS, VH>(d[k], row + (tn < tl ? tn : tl) * NS, q.own0);
    }
  }
#pragma unroll
  for (int k = 0; k < kWidePf - 1; ++k)
    if (k < n - nfull) half_step<NH>(mo, mp, s, d[k]);
#pragma unroll
  for (int i = 0; i < NH; ++i)
    if (q.own0 + i < NS) e[(q.c * lanes + q.lane) * NS + q.own0 + i] = s[i];
}

// Steps per output sub-block of the re-run kernels: a multiple of kWidePf whose NS-float steps fill
// at most 64 floats, so one lane's sub-block is one contiguous row segment of <= 256 bytes.
template <int NS>
constexpr int wide_out_sb() {
  return kWidePf * (64 / (kWidePf * NS));
}

// A re-run's outputs of sub-block tb (cnt steps) leave through LDS: each thread left its rows of
// every step in its lane's LDS row, and each wave now writes its 32 lanes' row segments with
// whole-segment (coalesced) stores, one lane at a time, so HBM sees full lines.
template <int NS, int SB>
TSF_DEV void half_write_segments(float* __restrict__ dst, const float (*s_o)[SB * NS + 1], int64_t lanes, int64_t L,
                                 int64_t tb, int cnt) {
  const int wl = threadIdx.x & 63, wlane0 = (threadIdx.x & ~63) >> 1;
  const int64_t l0 = blockIdx.x * (int64_t)kWideLanes;
  const int wseg = cnt * NS;
#pragma unroll 8
  for (int l = 0; l < 32; ++l) {
    const int64_t ln = l0 + wlane0 + l;
    if (ln < lanes && wl < wseg) dst[(ln * L + tb) * NS + wl] = s_o[wlane0 + l][wl];
  }
}

// Every chunk re-run from its entering state, writing x.
template <int NS, int VEC>
__global__ void __launch_bounds__(kWideThreads) lw_apply_fwd(const float* __restrict__ A, const float* __restrict__ v,
                                                             const double* __restrict__ carry, float* __restrict__ x,
                                                             int64_t lanes, int64_t L) {
  constexpr int NH = half_rows(NS), VH = half_vec<NS, VEC>();
  constexpr int SB = wide_out_sb<NS>();
  __shared__ float s_o[kWideLanes][SB * NS + 1];
  const HalfIdx q = half_idx(lanes, L, NH);
  float mo[NH][NH], mp[NH][NH];
  double s[NH];
  float d[kWidePf][NH];
  const float* row = v + (q.live ? q.lane : 0) * L * NS + q.own0;
  if (q.live) {
    half_matrix<NS, false>(mo, mp, A + q.lane * NS * NS, q.own0, q.par0);
#pragma unroll
    for (int i = 0; i < NH; ++i) s[i] = (q.own0 + i < NS) ? carry[(q.c * lanes + q.lane) * NS + q.own0 + i] : 0.0;
#pragma unroll
    for (int k = 0; k < kWidePf; ++k)
      if (q.t0 + k < q.t1) ld_half<NS, VH>(d[k], row + (q.t0 + k) * NS, q.own0);
  }
  const int64_t tl = q.t1 - 1;
  for (int64_t tb = q.t0; tb < q.t1; tb += SB) {
    const int cnt = (int)((q.t1 - tb) < SB ? (q.t1 - tb) : SB);
    if (q.live && cnt == SB) {
      // a whole sub-block without per-step branches (which made the compiler copy the prefetch
      // ring between register sets every step): a fetch past the chunk's end re-reads its last step
#pragma unroll
      for (int kk = 0; kk < SB; kk += kWidePf) {
#pragma unroll
        for (int k = 0; k < kWidePf; ++k) {
          half_step<NH>(mo, mp, s, d[k]);
#pragma unroll
          for (int i = 0; i < NH; ++i)
            if (q.own0 + i < NS) s_o[q.ll][(kk + k) * NS + q.own0 + i] = (float)s[i];
          const int64_t tn = tb + kk + k + kWidePf;
          ld_half<NS, VH>(d[k], row + (tn < tl ? tn : tl) * NS, q.own0);
        }
      }
    } else if (q.live) {
      for (int kk = 0; kk < SB; kk += kWidePf) {
#pragma unroll
        for (int k = 0; k < kWidePf; ++k) {
          const int64_t t = tb + kk + k;
          if (t < q.t1) {
            half_step<NH>(mo, mp, s, d[k]);
#pragma unroll
            for (int i = 0; i < NH; ++i)
              if (q.own0 + i < NS) s_o[q.ll][(kk + k) * NS + q.own0 + i] = (float)s[i];
            if (t + kWidePf < q.t1) ld_half<NS, VH>(d[k], row + (t + kWidePf) * NS, q.own0);
          }
        }
      }
    }
    __syncthreads();
    half_write_segments<NS, SB>(x, s_o, lanes, L, tb, cnt);
    __syncthreads();
  }
}

// Adjoint chunk starts from a zero right-end state: f [nchunks][lanes][NS]
template <int NS, int VEC>
__global__ void __launch_bounds__(kWideThreads) lw_sum_bwd(const float* __restrict__ A, const float* __restrict__ g,
                                                           double* __restrict__ f, int64_t lanes, int64_t L) {
  constexpr int NH = half_rows(NS), VH = half_vec<NS, VEC>();
  const HalfIdx q = half_idx(lanes, L, NH);
  if (!q.live) return;  // both threads of a pair
  float mo[NH][NH], mp[NH][NH];
  half_matrix<NS, true>(mo, mp, A + q.lane * NS * NS, q.own0, q.par0);
  double G[NH];
#pragma unroll
  for (int i = 0; i < NH; ++i) G[i] = 0.0;
  const float* row = g + q.lane * L * NS + q.own0;
  // as lw_sum_fwd, from the chunk's last step down: whole blocks without per-step branches (a
  // fetch before the chunk's start re-reads its first step), then the remaining steps
  const int64_t t0 = q.t0, tl = q.t1 - 1, n = q.t1 - q.t0, nblk = (n - n % kWidePf) / kWidePf;
  float d[kWidePf][NH];
#pragma unroll
  for (int k = 0; k < kWidePf; ++k) ld_half<NS, VH>(d[k], row + (tl - k > t0 ? tl - k : t0) * NS, q.own0);
  for (int64_t it = 0; it < nblk; ++it) {
    const int64_t tb = tl - it * kWidePf;
#pragma unroll
    for (int k = 0; k < kWidePf; ++k) {
      half_step<NH>(mo, mp, G, d[k]);
      const int64_t tn = tb - k - kWidePf;
      ld_half<NS, VH>(d[k], row + (tn > t0 ? tn : t0) * NS, q.own0);
    }
  }
#pragma unroll
  for (int k = 0; k < kWidePf - 1; ++k)
    if (k < n - nblk * kWidePf) half_step<NH>(mo, mp, G, d[k]);
#pragma unroll
  for (int i = 0; i < NH; ++i)
    if (q.own0 + i < NS) f[(q.c * lanes + q.lane) * NS + q.own0 + i] = G[i];
}

// Entering state of every chunk: carry[c] = M carry[c-1] + e[c-1], carry[0] = x0 (or 0)
template <int NS>
__global__ void __launch_bounds__(64) lw_carry_fwd(const double* __restrict__ M, const float* __restrict__ x0,
                                                    const double* __restrict__ e, double* __restrict__ carry,
                                                    int64_t lanes, int64_t nchunks) {
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  double m[NS][NS], s[NS];
  for (int r = 0; r < NS; ++r) {
    for (int c = 0; c < NS; ++c) m[r][c] = M[lane * NS * NS + r * NS + c];
    s[r] = x0 ? (double)x0[lane * NS + r] : 0.0;
  }
  for (int64_t c = 0; c < nchunks; ++c) {
    double t[NS];
    for (int r = 0; r < NS; ++r) {
      carry[(c * lanes + lane) * NS + r] = s[r];
      double acc = e[(c * lanes + lane) * NS + r];
      for (int j = 0; j < NS; ++j) acc = fma(m[r][j], s[j], acc);
      t[r] = acc;
    }
    for (int r = 0; r < NS; ++r) s[r] = t[r];
  }
}


// Adjoint entering every chunk from the right: rc[c] = G at the first step of chunk c + 1 (zero
// for the last chunk), rc[c-1] = f[c] + M rc[c]; then grad_x0 = A^T G_0 with G_0 = f[0] + M rc[0].
template <int NS>
__global__ void __launch_bounds__(64) lw_carry_bwd(const float* __restrict__ A, const double* __restrict__ M,
                                                    const double* __restrict__ f, double* __restrict__ rc,
                                                    float* __restrict__ gx0, int64_t lanes, int64_t nchunks) {
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  double m[NS][NS], R[NS];
  for (int r = 0; r < NS; ++r) {
    for (int c = 0; c < NS; ++c) m[r][c] = M[lane * NS * NS + r * NS + c];
    R[r] = 0.0;
  }
  for (int64_t c = nchunks - 1; c >= 0; --c) {
    double t[NS];
    for (int r = 0; r < NS; ++r) {
      rc[(c * lanes + lane) * NS + r] = R[r];
      double acc = f[(c * lanes + lane) * NS + r];
      for (int j = 0; j < NS; ++j) acc = fma(m[r][j], R[j], acc);
      t[r] = acc;
    }
    for (int r = 0; r < NS; ++r) R[r] = t[r];
  }
  if (gx0) {  // R now holds G_0; grad_x0 = A^T G_0
    const float* a = A + lane * NS * NS;
    for (int r = 0; r < NS; ++r) {
      double acc = 0.0;
      for (int j = 0; j < NS; ++j) acc = fma((double)a[j * NS + r], R[j], acc);
      gx0[lane * NS + r] = (float)acc;
    }
  }
}

// Every chunk re-run backwards from its right-end adjoint, writing grad_v and the chunk's grad_A
// partial sum_t G_t x_{t-1}^T (x_{-1} = x0 or 0) into part [nchunks][lanes][NS * NS]: each thread
// its rows of grad_A, with the columns of its own half of x_{t-1} first and the partner's half
// (by DPP lane swap) second, so each thread loads half a row of x per step.
template <int NS, int VEC>
__global__ void __launch_bounds__(kWideThreads) lw_apply_bwd(const float* __restrict__ A, const float* __restrict__ g,
                                                             const float* __restrict__ out, const float* __restrict__ x0,
                                                             const double* __restrict__ rc, float* __restrict__ gv,
                                                             double* __restrict__ part, int64_t lanes, int64_t L) {
  constexpr int NH = half_rows(NS), VH = half_vec<NS, VEC>();
  constexpr int SB = wide_out_sb<NS>();
  constexpr int kPfB = 2;  // steps fetched ahead; SB is a multiple of it (4 and 8 measured no faster)
  constexpr bool kMaskPad = NS == 7;  // ld_half's load form (measured, see there)
  static_assert(SB % kPfB == 0, "sub-blocks hold whole prefetch pairs");
  __shared__ float s_o[kWideLanes][SB * NS + 1];
  const HalfIdx q = half_idx(lanes, L, NH);
  float mo[NH][NH], mp[NH][NH];
  double G[NH], acc[NH][2 * NH];  // acc[i][j]: column own0 + j (j < NH), par0 + j - NH (j >= NH)
#pragma unroll
  for (int i = 0; i < NH; ++i) {
    G[i] = (q.live && q.own0 + i < NS) ? rc[(q.c * lanes + q.lane) * NS + q.own0 + i] : 0.0;
#pragma unroll
    for (int j = 0; j < 2 * NH; ++j) acc[i][j] = 0.0;
  }
  const int64_t lrow = (q.live ? q.lane : 0) * L * NS + q.own0;
  const float* grow = g + lrow;
  const float* xrow = out + lrow;
  // slot k of the ring holds the owned rows of g_t and of x_{t-1} of a step t with (t - t0) % kPfB == k
  float dg[kPfB][NH], dx[kPfB][NH];
  auto fetch = [&](int k, int64_t t) __attribute__((always_inline)) {
    ld_half<NS, VH, kMaskPad>(dg[k], grow + t * NS, q.own0);
    if (t > 0) {
      ld_half<NS, VH, kMaskPad>(dx[k], xrow + (t - 1) * NS, q.own0);
    } else {
#pragma unroll
      for (int i = 0; i < NH; ++i) dx[k][i] = (x0 && q.own0 + i < NS) ? x0[q.lane * NS + q.own0 + i] : 0.0f;
    }
  };
  const int64_t t0 = q.t0, t1 = q.t1;
  if (q.live) {
    half_matrix<NS, true>(mo, mp, A + q.lane * NS * NS, q.own0, q.par0);
#pragma unroll
    for (int i = 0; i < kPfB; ++i) {
      const int64_t t = t1 - 1 - i;
      if (t >= t0) fetch((int)((t - t0) % kPfB), t);
    }
  }
  const int64_t nsb = (t1 - t0 + SB - 1) / SB;
  for (int64_t j = nsb - 1; j >= 0; --j) {
    const int64_t tb = t0 + j * SB;
    const int cnt = (int)((t1 - tb) < SB ? (t1 - tb) : SB);
    // one step of the re-run: G, its store to the tile, grad_A += G_t x_{t-1}^T (x_{t-1}: the
    // owned rows and, by a DPP swap, the partner's)
    auto step = [&](int k, int slot) __attribute__((always_inline)) {
      half_step<NH>(mo, mp, G, dg[k]);
      float xo[NH], xq[NH];
#pragma unroll
      for (int i = 0; i < NH; ++i) {
        xo[i] = dx[k][i];
        xq[i] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(xo[i]), 0xB1, 0xF, 0xF, false));
      }
#pragma unroll
      for (int i = 0; i < NH; ++i)
        if (q.own0 + i < NS) s_o[q.ll][slot * NS + q.own0 + i] = (float)G[i];
      return [&, xo, xq]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NH; ++i) {
#pragma unroll
          for (int jj = 0; jj < NH; ++jj) acc[i][jj] = fma(G[i], (double)xo[jj], acc[i][jj]);
#pragma unroll
          for (int jj = 0; jj < NH; ++jj) acc[i][NH + jj] = fma(G[i], (double)xq[jj], acc[i][NH + jj]);
        }
      };
    };
    // (odd n keeps the guarded loop: its padded half rows took the branch-free form past 256 VGPRs)
    if (NS % 2 == 0 && q.live && cnt == SB && tb > 0) {
      // a whole sub-block without per-step branches: a fetch before the chunk's start re-reads its
      // first step (never used); every fetched step is >= 1 here (t0 > 0, or tb >= SB > kPfB), so
      // x_{t-1} is a row of out
      for (int kk = SB - kPfB; kk >= 0; kk -= kPfB) {
#pragma unroll
        for (int k = kPfB - 1; k >= 0; --k) {
          auto grad_a = step(k, kk + k);
          const int64_t tn = tb + kk + k - kPfB, tc = tn > t0 ? tn : t0;
          ld_half<NS, VH, kMaskPad>(dg[k], grow + tc * NS, q.own0);
          ld_half<NS, VH, kMaskPad>(dx[k], xrow + (tc - 1) * NS, q.own0);
          grad_a();
        }
      }
    } else if (q.live) {
      for (int kk = SB - kPfB; kk >= 0; kk -= kPfB) {
#pragma unroll
        for (int k = kPfB - 1; k >= 0; --k) {
          const int64_t t = tb + kk + k;
          if (t < t1) {  // uniform over the workgroup (one chunk)
            auto grad_a = step(k, kk + k);
            if (t - kPfB >= t0) fetch(k, t - kPfB);
            grad_a();
          }
        }
      }
    }
    __syncthreads();
    half_write_segments<NS, SB>(gv, s_o, lanes, L, tb, cnt);
    __syncthreads();
  }
  if (q.live) {
    double* prow = part + (q.c * lanes + q.lane) * NS * NS;
#pragma unroll
    for (int i = 0; i < NH; ++i)
      if (q.own0 + i < NS) {
#pragma unroll
        for (int jj = 0; jj < NH; ++jj) {
          if (q.own0 + jj < NS) prow[(q.own0 + i) * NS + q.own0 + jj] = acc[i][jj];
          if (q.par0 + jj < NS) prow[(q.own0 + i) * NS + q.par0 + jj] = acc[i][NH + jj];
        }
      }
  }
}

// Workspace of the two-pass path: e/f and the carries [nchunks][lanes][n], M [lanes][n][n], and
// the grad_A partials [nchunks][lanes][n][n] (fp64).
struct LwPlan {
  int64_t nchunks = 0;
  size_t off_e = 0, off_carry = 0, off_M = 0, off_part = 0, bytes = 0;
};

LwPlan lw_plan(int64_t lanes, int64_t L, int64_t ns) {
  LwPlan p;
  p.nchunks = (L + kWideT - 1) / kWideT;
  const size_t f = 8, vecs = f * p.nchunks * lanes * ns;
  p.off_e = 0;
  p.off_carry = vecs;
  p.off_M = 2 * vecs;
  p.off_part = p.off_M + f * lanes * ns * ns;
  p.bytes = p.off_part + vecs * ns;
  return p;
}

inline bool lw_grid_fits(int64_t lanes, int64_t L) {
  // one grid row per chunk; two threads per lane, at most 2^32 - 1 threads per grid row
  return (L + kWideT - 1) / kWideT <= 65535 && (lanes + kWideLanes - 1) / kWideLanes <= UINT32_MAX / kWideThreads;
}

template <int NS, int VEC>
int wide_fwd_impl(int64_t lanes, int64_t L, const float* A, const float* v, const float* x0, float* x, char* ws,
                  hipStream_t s) {
  const LwPlan p = lw_plan(lanes, L, NS);
  double* e = reinterpret_cast<double*>(ws + p.off_e);
  double* carry = reinterpret_cast<double*>(ws + p.off_carry);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  const dim3 grid((unsigned)((lanes + kWideLanes - 1) / kWideLanes), (unsigned)p.nchunks);
  const unsigned lb = (unsigned)((lanes + 63) / 64);
  hipLaunchKernelGGL((lw_power<NS>), dim3((unsigned)((lanes * NS + 63) / 64)), dim3(64), 0, s, A, M, lanes, kWideT, 0);
  hipLaunchKernelGGL((lw_sum_fwd<NS, VEC>), grid, dim3(kWideThreads), 0, s, A, v, e, lanes, L);
  hipLaunchKernelGGL((lw_carry_fwd<NS>), dim3(lb), dim3(64), 0, s, (const double*)M, x0, (const double*)e, carry,
                     lanes, p.nchunks);
  hipLaunchKernelGGL((lw_apply_fwd<NS, VEC>), grid, dim3(kWideThreads), 0, s, A, v, (const double*)carry, x, lanes, L);
  return tsf_launch_status();
}

template <int NS, int VEC>
int wide_bwd_impl(int64_t lanes, int64_t L, const float* g, const float* A, const float* out, const float* x0,
                  float* gA, float* gv, float* gx0, char* ws, hipStream_t s) {
  if (L == 0) {
    hipLaunchKernelGGL(linrec_zero, dim3(blocks_for(lanes * NS * NS)), dim3(256), 0, s, gA, lanes * NS * NS);
    if (gx0) hipLaunchKernelGGL(linrec_zero, dim3(blocks_for(lanes * NS)), dim3(256), 0, s, gx0, lanes * NS);
    return tsf_launch_status();
  }
  const LwPlan p = lw_plan(lanes, L, NS);
  double* f = reinterpret_cast<double*>(ws + p.off_e);
  double* rc = reinterpret_cast<double*>(ws + p.off_carry);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  double* part = reinterpret_cast<double*>(ws + p.off_part);
  const dim3 grid((unsigned)((lanes + kWideLanes - 1) / kWideLanes), (unsigned)p.nchunks);
  const unsigned lb = (unsigned)((lanes + 63) / 64);
  hipLaunchKernelGGL((lw_power<NS>), dim3((unsigned)((lanes * NS + 63) / 64)), dim3(64), 0, s, A, M, lanes, kWideT, 1);
  hipLaunchKernelGGL((lw_sum_bwd<NS, VEC>), grid, dim3(kWideThreads), 0, s, A, g, f, lanes, L);
  hipLaunchKernelGGL((lw_carry_bwd<NS>), dim3(lb), dim3(64), 0, s, A, (const double*)M, (const double*)f, rc, gx0,
                     lanes, p.nchunks);
  hipLaunchKernelGGL((lw_apply_bwd<NS, VEC>), grid, dim3(kWideThreads), 0, s, A, g, out, x0, (const double*)rc, gv, part,
                     lanes, L);
  hipLaunchKernelGGL(linrec_finish, dim3((unsigned)((lanes * NS * NS + 63) / 64)), dim3(1024), 0, s,
                     (const double*)part, gA, lanes * NS * NS, p.nchunks);
  return tsf_launch_status();
}

// Widest access every row pointer allows: rows start at multiples of NS floats.
template <int NS>
int wide_vec(std::initializer_list<const void*> ptrs) {
  auto aligned = [&](uintptr_t a) {
    for (const void* p : ptrs)
      if (p && (reinterpret_cast<uintptr_t>(p) % a) != 0) return false;
    return true;
  };
  if (NS % 4 == 0 && aligned(16)) return 4;
  if (NS % 2 == 0 && aligned(8)) return 2;
  return 1;
}
template <int NS>
int wide_fwd(int64_t lanes, int64_t L, const float* A, const float* v, const float* x0, float* x, char* ws,
             hipStream_t s) {
  switch (wide_vec<NS>({v, x})) {
    case 4: return wide_fwd_impl<NS, (NS % 4 == 0 ? 4 : 1)>(lanes, L, A, v, x0, x, ws, s);
    case 2: return wide_fwd_impl<NS, (NS % 2 == 0 ? 2 : 1)>(lanes, L, A, v, x0, x, ws, s);
    default: return wide_fwd_impl<NS, 1>(lanes, L, A, v, x0, x, ws, s);
  }
}
template <int NS>
int wide_bwd(int64_t lanes, int64_t L, const float* g, const float* A, const float* out, const float* x0, float* gA,
             float* gv, float* gx0, char* ws, hipStream_t s) {
  switch (wide_vec<NS>({g, out, gv})) {
    case 4: return wide_bwd_impl<NS, (NS % 4 == 0 ? 4 : 1)>(lanes, L, g, A, out, x0, gA, gv, gx0, ws, s);
    case 2: return wide_bwd_impl<NS, (NS % 2 == 0 ? 2 : 1)>(lanes, L, g, A, out, x0, gA, gv, gx0, ws, s);
    default: return wide_bwd_impl<NS, 1>(lanes, L, g, A, out, x0, gA, gv, gx0, ws, s);
  }
}

#define TSF_WIDE_CASES(X) X(5) X(6) X(7) X(8)

// ------------------------------------------------------------------------------ n = 9..16
// Spread two-pass path: the phases of the n = 5..8 path (chunk summaries from a zero state, a
// sequential carry over the chunks with M = P^kWideT, every chunk re-run from its entering state),
// with one (lane, chunk) per group of 16 threads, a DPP row. Thread r of a group holds component r
// of the state (fp64) and row r of the step matrix (fp64, zero beyond n), and a step
//     s_r <- sum_c P[r][c] s_c + x_r
// takes the other components s_c by row broadcasts (two 32-bit row_newbcast moves per fp64
// value), in the n = 5..8 path's summation order (c = 0 .. n-1 onto x_r). Per step a group reads
// or writes one contiguous segment of n floats (coalesced), and the adjoint's grad_A partial
// sum_t G_t x_{t-1}^T is accumulated row by row, thread r holding row r. Components r >= n stay
// zero: their matrix rows and inputs are zero, and nothing is stored for them.
constexpr int kSpread = 16;     // threads per group = the padded state size
constexpr int kMaxSpreadNS = 16;
constexpr int kSpreadPf = 8;    // steps fetched ahead by the chunk kernels

// acc + sum_c p[c] * (s of lane c), c = 0 .. 15 in order
template <int C = 0>
TSF_DEV double spread_dot(const double (&p)[kSpread], double s, double acc) {
  if constexpr (C == kSpread) {
    return acc;
  } else {
    return spread_dot<C + 1>(p, s, fma(p[C], row_lane<C>(s), acc));
  }
}
// acc[c] += g * (x of lane c), c = 0 .. 15
template <int C = 0>
TSF_DEV void spread_outer(double (&acc)[kSpread], double g, float x) {
  if constexpr (C < kSpread) {
    acc[C] = fma(g, (double)row_lane<C>(x), acc[C]);
    spread_outer<C + 1>(acc, g, x);
  }
}

// Row r of P = A (forward) or A^T (adjoint) of one lane, fp64, zero beyond n.
TSF_DEV void spread_row(double (&p)[kSpread], const float* __restrict__ A, int64_t lane, int n, int r, bool live,
                        bool transpose) {
  const float* a = A + lane * n * n;
#pragma unroll
  for (int c = 0; c < kSpread; ++c)
    p[c] = (live && r < n && c < n) ? (double)a[transpose ? c * n + r : r * n + c] : 0.0;
}

// M = P^e per lane, fp64 [lanes][n][n]: a workgroup per lane, group c runs column c (P applied e
// times to the unit vector e_c, step by step as lw_power).
__global__ void __launch_bounds__(256) lsp_power(const float* __restrict__ A, double* __restrict__ M, int64_t lanes,
                                                 int n, int e, int transpose) {
  const int64_t lane = blockIdx.x;
  const int r = threadIdx.x & 15, col = threadIdx.x >> 4;
  double p[kSpread];
  spread_row(p, A, lane, n, r, true, transpose != 0);
  double x = r == col ? 1.0 : 0.0;
  for (int step = 0; step < e; ++step) x = spread_dot(p, x, 0.0);
  if (r < n && col < n) M[(lane * n + r) * n + col] = x;
}

// One (lane, chunk) per group: group g of workgroup (bx, chunk) is lane bx * 16 + g.
struct SpreadIdx {
  int64_t lane, c, t0, t1;
  int r;
  bool live;
};
TSF_DEV SpreadIdx spread_idx(int64_t lanes, int64_t L) {
  SpreadIdx q;
  q.r = threadIdx.x & 15;
  q.lane = blockIdx.x * (int64_t)16 + (threadIdx.x >> 4);
  q.live = q.lane < lanes;
  q.c = blockIdx.y;
  q.t0 = q.c * kWideT;
  q.t1 = (q.t0 + kWideT < L) ? q.t0 + kWideT : L;
  return q;
}

// Forward chunk ends from a zero state: e [nchunks][lanes][n]
__global__ void __launch_bounds__(256) lsp_sum_fwd(const float* __restrict__ A, const float* __restrict__ v,
                                                   double* __restrict__ e, int64_t lanes, int64_t L, int n) {
  const SpreadIdx q = spread_idx(lanes, L);
  const bool ld = q.live && q.r < n;
  double p[kSpread];
  spread_row(p, A, q.lane, n, q.r, q.live, false);
  // whole blocks of kSpreadPf steps without per-step branches (which made the compiler copy the
  // prefetch ring between register sets every step): every load is unconditional, a fetch past
  // the chunk's end re-reads its last step (never used) and threads r >= n read component n - 1
  // (their inputs are taken as zero); the remaining steps follow the loop
  const float* row = v + (q.live ? q.lane : 0) * L * n + (q.r < n ? q.r : n - 1);
  const int64_t t0 = q.t0, tl = q.t1 - 1, cnt = q.t1 - q.t0, nfull = cnt - cnt % kSpreadPf;
  float d[kSpreadPf];
#pragma unroll
  for (int k = 0; k < kSpreadPf; ++k) d[k] = row[(t0 + k < tl ? t0 + k : tl) * n];
  double s = 0.0;
  for (int64_t tb = t0; tb < t0 + nfull; tb += kSpreadPf) {
#pragma unroll
    for (int k = 0; k < kSpreadPf; ++k) {
      s = spread_dot(p, s, ld ? (double)d[k] : 0.0);
      const int64_t tn = tb + k + kSpreadPf;
      d[k] = row[(tn < tl ? tn : tl) * n];
    }
  }
#pragma unroll
  for (int k = 0; k < kSpreadPf - 1; ++k)
    if (k < cnt - nfull) s = spread_dot(p, s, ld ? (double)d[k] : 0.0);
  if (ld) e[(q.c * lanes + q.lane) * n + q.r] = s;
}

// Entering state of every chunk: carry[c] = M carry[c-1] + e[c-1], carry[0] = x0 (or 0); a group
// per lane.
__global__ void __launch_bounds__(256) lsp_carry_fwd(const double* __restrict__ M, const float* __restrict__ x0,
                                                     const double* __restrict__ e, double* __restrict__ carry,
                                                     int64_t lanes, int64_t nchunks, int n) {
  const int r = threadIdx.x & 15;
  const int64_t lane = blockIdx.x * (int64_t)16 + (threadIdx.x >> 4);
  const bool live = lane < lanes, ld = live && r < n;
  double m[kSpread];
#pragma unroll
  for (int c = 0; c < kSpread; ++c) m[c] = (ld && c < n) ? M[(lane * n + r) * n + c] : 0.0;
  double s = (ld && x0) ? (double)x0[lane * n + r] : 0.0;
  for (int64_t c = 0; c < nchunks; ++c) {
    if (ld) carry[(c * lanes + lane) * n + r] = s;
    s = spread_dot(m, s, ld ? e[(c * lanes + lane) * n + r] : 0.0);
  }
}

// Every chunk re-run from its entering state, writing x.
__global__ void __launch_bounds__(256) lsp_apply_fwd(const float* __restrict__ A, const float* __restrict__ v,
                                                     const double* __restrict__ carry, float* __restrict__ x,
                                                     int64_t lanes, int64_t L, int n) {
  const SpreadIdx q = spread_idx(lanes, L);
  const bool ld = q.live && q.r < n;
  double p[kSpread];
  spread_row(p, A, q.lane, n, q.r, q.live, false);
  const int64_t off = (q.live ? q.lane : 0) * L * n + (q.r < n ? q.r : n - 1);
  const float* row = v + off;
  float* orow = x + off;
  // as lsp_sum_fwd: whole blocks without per-step branches, then the remaining steps
  const int64_t t0 = q.t0, tl = q.t1 - 1, cnt = q.t1 - q.t0, nfull = cnt - cnt % kSpreadPf;
  float d[kSpreadPf];
#pragma unroll
  for (int k = 0; k < kSpreadPf; ++k) d[k] = row[(t0 + k < tl ? t0 + k : tl) * n];
  double s = ld ? carry[(q.c * lanes + q.lane) * n + q.r] : 0.0;
  for (int64_t tb = t0; tb < t0 + nfull; tb += kSpreadPf) {
#pragma unroll
    for (int k = 0; k < kSpreadPf; ++k) {
      s = spread_dot(p, s, ld ? (double)d[k] : 0.0);
      if (ld) orow[(tb + k) * n] = (float)s;
      const int64_t tn = tb + k + kSpreadPf;
      d[k] = row[(tn < tl ? tn : tl) * n];
    }
  }
#pragma unroll
  for (int k = 0; k < kSpreadPf - 1; ++k)
    if (k < cnt - nfull) {
      s = spread_dot(p, s, ld ? (double)d[k] : 0.0);
      if (ld) orow[(t0 + nfull + k) * n] = (float)s;
    }
}

// Adjoint chunk starts from a zero right-end state: f [nchunks][lanes][n]
__global__ void __launch_bounds__(256) lsp_sum_bwd(const float* __restrict__ A, const float* __restrict__ g,
                                                   double* __restrict__ f, int64_t lanes, int64_t L, int n) {
  const SpreadIdx q = spread_idx(lanes, L);
  const bool ld = q.live && q.r < n;
  double p[kSpread];
  spread_row(p, A, q.lane, n, q.r, q.live, true);
  // as lsp_sum_fwd from the chunk's last step down (a fetch before its start re-reads its first)
  const float* row = g + (q.live ? q.lane : 0) * L * n + (q.r < n ? q.r : n - 1);
  const int64_t t0 = q.t0, tl = q.t1 - 1, cnt = q.t1 - q.t0, nblk = (cnt - cnt % kSpreadPf) / kSpreadPf;
  float d[kSpreadPf];
#pragma unroll
  for (int k = 0; k < kSpreadPf; ++k) d[k] = row[(tl - k > t0 ? tl - k : t0) * n];
  double G = 0.0;
  for (int64_t it = 0; it < nblk; ++it) {
    const int64_t tb = tl - it * kSpreadPf;
#pragma unroll
    for (int k = 0; k < kSpreadPf; ++k) {
      G = spread_dot(p, G, ld ? (double)d[k] : 0.0);
      const int64_t tn = tb - k - kSpreadPf;
      d[k] = row[(tn > t0 ? tn : t0) * n];
    }
  }
#pragma unroll
  for (int k = 0; k < kSpreadPf - 1; ++k)
    if (k < cnt - nblk * kSpreadPf) G = spread_dot(p, G, ld ? (double)d[k] : 0.0);
  if (ld) f[(q.c * lanes + q.lane) * n + q.r] = G;
}

// Adjoint entering every chunk from the right: rc[c] = G at the first step of chunk c + 1 (zero
// for the last chunk), rc[c-1] = f[c] + M rc[c]; then grad_x0 = A^T G_0 with G_0 = f[0] + M rc[0].
__global__ void __launch_bounds__(256) lsp_carry_bwd(const float* __restrict__ A, const double* __restrict__ M,
                                                     const double* __restrict__ f, double* __restrict__ rc,
                                                     float* __restrict__ gx0, int64_t lanes, int64_t nchunks, int n) {
  const int r = threadIdx.x & 15;
  const int64_t lane = blockIdx.x * (int64_t)16 + (threadIdx.x >> 4);
  const bool live = lane < lanes, ld = live && r < n;
  double m[kSpread];
#pragma unroll
  for (int c = 0; c < kSpread; ++c) m[c] = (ld && c < n) ? M[(lane * n + r) * n + c] : 0.0;
  double R = 0.0;
  for (int64_t c = nchunks - 1; c >= 0; --c) {
    if (ld) rc[(c * lanes + lane) * n + r] = R;
    R = spread_dot(m, R, ld ? f[(c * lanes + lane) * n + r] : 0.0);
  }
  if (gx0) {  // R now holds G_0; grad_x0 = A^T G_0
    double p[kSpread];
    spread_row(p, A, lane, n, r, live, true);
    const double gx = spread_dot(p, R, 0.0);
    if (ld) gx0[lane * n + r] = (float)gx;
  }
}

// Every chunk re-run backwards from its right-end adjoint, writing grad_v and the chunk's grad_A
// partial sum_t G_t x_{t-1}^T (x_{-1} = x0 or 0) into part [nchunks][lanes][n][n].
__global__ void __launch_bounds__(256) lsp_apply_bwd(const float* __restrict__ A, const float* __restrict__ g,
                                                     const float* __restrict__ out, const float* __restrict__ x0,
                                                     const double* __restrict__ rc, float* __restrict__ gv,
                                                     double* __restrict__ part, int64_t lanes, int64_t L, int n) {
  const SpreadIdx q = spread_idx(lanes, L);
  const bool ld = q.live && q.r < n;
  double p[kSpread], acc[kSpread];
  spread_row(p, A, q.lane, n, q.r, q.live, true);
#pragma unroll
  for (int c = 0; c < kSpread; ++c) acc[c] = 0.0;
  const int64_t off = (q.live ? q.lane : 0) * L * n + (q.r < n ? q.r : n - 1);
  const float* grow = g + off;
  const float* xrow = out + off;
  float* orow = gv + off;
  const float x_init = (ld && x0) ? x0[q.lane * n + q.r] : 0.0f;  // x_{-1}
  // slot k holds g_t and x_{t-1} of a step t with (t1 - 1 - t) % kSpreadPf == k. Every load is
  // unconditional (as lsp_sum_bwd: fetches before the chunk's start re-read its first step, threads
  // r >= n read component n - 1, masked on use); x_{t-1} of step 0 is x_init.
  float dg[kSpreadPf], dx[kSpreadPf];
  const int64_t t0 = q.t0, tl = q.t1 - 1, cnt = q.t1 - q.t0, nblk = (cnt - cnt % kSpreadPf) / kSpreadPf;
  auto fetch = [&](int k, int64_t t) __attribute__((always_inline)) {
    const int64_t tc = t > t0 ? t : t0;
    dg[k] = grow[tc * n];
    const float xv = xrow[(tc > 0 ? tc - 1 : 0) * n];
    dx[k] = tc > 0 ? xv : x_init;
  };
  double G = ld ? rc[(q.c * lanes + q.lane) * n + q.r] : 0.0;
  auto step = [&](int k, int64_t t) __attribute__((always_inline)) {
    G = spread_dot(p, G, ld ? (double)dg[k] : 0.0);
    if (ld) orow[t * n] = (float)G;
    spread_outer(acc, G, ld ? dx[k] : 0.0f);
  };
#pragma unroll
  for (int k = 0; k < kSpreadPf; ++k) fetch(k, tl - k);
  for (int64_t it = 0; it < nblk; ++it) {
    const int64_t tb = tl - it * kSpreadPf;
#pragma unroll
    for (int k = 0; k < kSpreadPf; ++k) {
      step(k, tb - k);
      fetch(k, tb - k - kSpreadPf);
    }
  }
#pragma unroll
  for (int k = 0; k < kSpreadPf - 1; ++k)
    if (k < cnt - nblk * kSpreadPf) step(k, tl - nblk * kSpreadPf - k);
  if (ld) {
    double* pr = part + ((q.c * lanes + q.lane) * n + q.r) * n;
#pragma unroll
    for (int c = 0; c < kSpread; ++c)
      if (c < n) pr[c] = acc[c];
  }
}

int spread_fwd(int64_t lanes, int64_t L, int n, const float* A, const float* v, const float* x0, float* x, char* ws,
               hipStream_t s) {
  const LwPlan p = lw_plan(lanes, L, n);
  double* e = reinterpret_cast<double*>(ws + p.off_e);
  double* carry = reinterpret_cast<double*>(ws + p.off_carry);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  const unsigned lg = (unsigned)((lanes + 15) / 16);
  const dim3 grid(lg, (unsigned)p.nchunks);
  hipLaunchKernelGGL(lsp_power, dim3((unsigned)lanes), dim3(256), 0, s, A, M, lanes, n, kWideT, 0);
  hipLaunchKernelGGL(lsp_sum_fwd, grid, dim3(256), 0, s, A, v, e, lanes, L, n);
  hipLaunchKernelGGL(lsp_carry_fwd, dim3(lg), dim3(256), 0, s, (const double*)M, x0, (const double*)e, carry, lanes,
                     p.nchunks, n);
  hipLaunchKernelGGL(lsp_apply_fwd, grid, dim3(256), 0, s, A, v, (const double*)carry, x, lanes, L, n);
  return tsf_launch_status();
}

int spread_bwd(int64_t lanes, int64_t L, int n, const float* g, const float* A, const float* out, const float* x0,
               float* gA, float* gv, float* gx0, char* ws, hipStream_t s) {
  if (L == 0) {
    hipLaunchKernelGGL(linrec_zero, dim3(blocks_for(lanes * n * n)), dim3(256), 0, s, gA, lanes * n * n);
    if (gx0) hipLaunchKernelGGL(linrec_zero, dim3(blocks_for(lanes * n)), dim3(256), 0, s, gx0, lanes * n);
    return tsf_launch_status();
  }
  const LwPlan p = lw_plan(lanes, L, n);
  double* f = reinterpret_cast<double*>(ws + p.off_e);
  double* rc = reinterpret_cast<double*>(ws + p.off_carry);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  double* part = reinterpret_cast<double*>(ws + p.off_part);
  const unsigned lg = (unsigned)((lanes + 15) / 16);
  const dim3 grid(lg, (unsigned)p.nchunks);
  hipLaunchKernelGGL(lsp_power, dim3((unsigned)lanes), dim3(256), 0, s, A, M, lanes, n, kWideT, 1);
  hipLaunchKernelGGL(lsp_sum_bwd, grid, dim3(256), 0, s, A, g, f, lanes, L, n);
  hipLaunchKernelGGL(lsp_carry_bwd, dim3(lg), dim3(256), 0, s, A, (const double*)M, (const double*)f, rc, gx0, lanes,
                     p.nchunks, n);
  hipLaunchKernelGGL(lsp_apply_bwd, grid, dim3(256), 0, s, A, g, out, x0, (const double*)rc, gv, part, lanes, L, n);
  hipLaunchKernelGGL(linrec_finish, dim3((unsigned)((lanes * n * n + 63) / 64)), dim3(1024), 0, s,
                     (const double*)part, gA, lanes * n * n, p.nchunks);
  return tsf_launch_status();
}

}  // namespace

extern "C" {

int64_t tsfast_hip_linrec_workspace_bytes(int64_t lanes, int64_t L, int64_t n) {
  if (lanes < 0 || L < 0 || n < 1 || n > kMaxSpreadNS) return -1;
  if (n > kMaxNS) return (int64_t)lw_plan(lanes, L, n).bytes;
  return (int64_t)lr_plan(lanes, L, n).bytes;
}

int tsfast_hip_linrec_fwd(int64_t lanes, int64_t L, int64_t n, const float* A, const float* v, const float* x0,
                          float* x, void* workspace, int64_t workspace_bytes, void* stream) {
  if (lanes < 0 || L < 0) return TSF_ERR_ARG;
  if (n < 1 || n > kMaxSpreadNS) return TSF_ERR_UNSUPPORTED;
  if (lanes == 0 || L == 0) return TSF_OK;
  if (n > kMaxWideNS && lanes > (int64_t)UINT32_MAX) return TSF_ERR_UNSUPPORTED;
  if (n > kMaxNS && !lw_grid_fits(lanes, L)) return TSF_ERR_UNSUPPORTED;
  if (!A || !v || !x) return TSF_ERR_ARG;
  if (!workspace || workspace_bytes < tsfast_hip_linrec_workspace_bytes(lanes, L, n)) return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  switch (n) {
#define X(K) \
  case K:    \
    return fwd_impl<K>(lanes, L, A, v, x0, x, ws, s);
    TSF_NS_CASES(X)
#undef X
#define X(K) \
  case K:    \
    return wide_fwd<K>(lanes, L, A, v, x0, x, ws, s);
    TSF_WIDE_CASES(X)
#undef X
    default:
      return spread_fwd(lanes, L, (int)n, A, v, x0, x, ws, s);
  }
}

int tsfast_hip_linrec_bwd(int64_t lanes, int64_t L, int64_t n, const float* g, const float* A, const float* out,
                          const float* x0, float* gA, float* gv, float* gx0, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  if (lanes < 0 || L < 0) return TSF_ERR_ARG;
  if (n < 1 || n > kMaxSpreadNS) return TSF_ERR_UNSUPPORTED;
  if (lanes == 0) return TSF_OK;
  if (n > kMaxWideNS && lanes > (int64_t)UINT32_MAX) return TSF_ERR_UNSUPPORTED;
  if (n > kMaxNS && !lw_grid_fits(lanes, L)) return TSF_ERR_UNSUPPORTED;
  if (!A || !gA || (L > 0 && (!g || !out || !gv))) return TSF_ERR_ARG;
  if (x0 && !gx0) return TSF_ERR_ARG;
  if (!workspace || workspace_bytes < tsfast_hip_linrec_workspace_bytes(lanes, L, n)) return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  switch (n) {
#define X(K) \
  case K:    \
    return bwd_impl<K>(lanes, L, g, A, out, x0, gA, gv, gx0, ws, s);
    TSF_NS_CASES(X)
#undef X
#define X(K) \
  case K:    \
    return wide_bwd<K>(lanes, L, g, A, out, x0, gA, gv, gx0, ws, s);
    TSF_WIDE_CASES(X)
#undef X
    default:
      return spread_bwd(lanes, L, (int)n, g, A, out, x0, gA, gv, gx0, ws, s);
  }
}

}  // extern "C"
