// Fused dynoNet G-block: LinearDynamicalOperator.forward with an all-pole denominator,
//
//   w_p[t] = sum_k b[o, j, k] u[t - k, j]                      (FIR per pair, u_{-m} from u_tail)
//   y_p[t] = w_p[t] - sum_{i=1..na} a[o, j, i] y_p[t - i]       (all-pole per pair, y_{-m} from x0)
//   y[t, o] = sum_j y_p[t]                                      (sum over inputs)
//
// for pairs p = j * O + o (the reference's input-major order), u [B, L, I] and y [B, L, O]
// channel-last, fp32 in and out, fp64 recurrence state. Reference semantics:
// tsfast/models/architectures/dynonet/core.py:196-258 (FIR conv1d :219-222, all-pole :225-235,
// input sum :250, returned state :239-245, 254-257).
//
// Neither the FIR output w nor the per-pair outputs y_p (each [B, P, L], P times the size of u)
// ever reach HBM: the forward reads u and writes y; the backward reads u and gy and writes gu.
// Both run the single-pass look-back scheme of the all-pole kernels (allpole_core.h) over lanes
// lane = b * Pp + p, where Pp is P rounded up to a power of two (a batch row's lanes p >= P are
// idle: zero inputs, nothing stored), 64 lanes (64 / Pp whole batch rows) to a tile:
//   forward   each wave loads its lanes' u window (its 32-step chunk plus the nb - 1 step FIR
//             halo, straight from u: the lanes of one batch row read a few contiguous bytes per
//             step), forms w, runs the all-pole scan with look-back, saves each super-chunk's
//             entering state for the backward (nsuper x lanes x na doubles), and sums the pairs
//             of each output channel through its LDS tile.
//   backward  recomputes y_p per chunk from the saved entering state, then runs two adjoint
//             recurrences of the same dynamics with one look-back: G (the all-pole adjoint of the
//             pair's upstream gradient g = gy[., o] + the x_last gradient) and c = A^-T (B^T g).
//             FIR and all-pole commute, so c is the FIR adjoint of G, i.e. the pair's input
//             gradient; forming it from B^T g needs only the gy halo to the right, not another
//             tile's G. grad a = -sum G_t y_{t-i} and grad b = sum G_t u_{t-k} are reduced per
//             tile; gu (sum of c over o) and the tail gradient go through LDS.
// Orders na <= 4, nb <= 16 (taps padded to NBT in {2, 4, 8, 16} with zeros), I * O <= 64.
#include <type_traits>

#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

#include "allpole_core.h"

// Deterministic-mode anchor spacing: every tile an anchor (a chained look-back), measured the
// cheapest at config 4's channels (4.5% over the default mode, against 12% at spacing K).
constexpr int kGbAnchorSpacing = 1;

constexpr int kGbMaxNB = 16;

// lane = b * Pp + p in the padded lane space; rl = b * P + p indexes the caller's per-pair state
// tensors (x0, x_last and their gradients, [B, P, na]).
struct GbLane {
  int64_t b, rl;
  int p, j, o;
  bool live;
};
TSF_DEV GbLane gb_lane(int64_t lane, int64_t lanes, int P, int Pp, int O) {
  GbLane g;
  const int64_t l = lane < lanes ? lane : 0;
  g.b = l / Pp;
  g.p = (int)(l - g.b * Pp);
  g.live = lane < lanes && g.p < P;
  if (!g.live) g.p = 0;
  g.j = g.p / O;
  g.o = g.p - g.j * O;
  g.rl = g.b * P + g.p;
  return g;
}

// P pairs per batch row rounded up to a power of two (P <= 64), so 64 / Pp batch rows fill a tile.
TSF_HOST_DEV int padded_pairs(int P) {
  int pp = 1;
  while (pp < P) pp *= 2;
  return pp;
}

// The lane's FIR input u_s for s in [t0 - (NBT - 1), t0 + kTileT): u [B, L, I] for s in [0, L),
// u_tail [B, nb - 1, I] for s in [-(nb - 1), 0) (zero when u_tail is NULL), zero elsewhere.
template <int NBT>
TSF_DEV void load_u_window(float (&uw)[kTileT + NBT - 1], const float* __restrict__ u,
                           const float* __restrict__ u_tail, const GbLane& g, int64_t t0, int64_t L, int I, int nb) {
  const float* __restrict__ urow = u + g.b * L * I + g.j;
  if (t0 - (NBT - 1) >= 0 && t0 + kTileT <= L) {  // the whole window inside the sequence
#pragma unroll
    for (int i = 0; i < kTileT + NBT - 1; ++i) uw[i] = g.live ? urow[(t0 - (NBT - 1) + i) * I] : 0.0f;
  } else {
#pragma unroll
    for (int i = 0; i < kTileT + NBT - 1; ++i) {
      const int64_t s = t0 - (NBT - 1) + i;
      float v = 0.0f;
      if (g.live) {
        if (s >= 0 && s < L)
          v = urow[s * I];
        else if (s < 0 && s >= -(nb - 1) && u_tail)
          v = u_tail[(g.b * (nb - 1) + (s + nb - 1)) * I + g.j];
      }
      uw[i] = v;
    }
  }
}

// w_{t0+i} = sum_k b_k u_{t0+i-k} for the chunk's 32 steps.
template <int NBT>
TSF_DEV void fir(float (&w)[kTileT], const float (&uw)[kTileT + NBT - 1], const float (&bk)[NBT]) {
#pragma unroll
  for (int i = 0; i < kTileT; ++i) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NBT; ++k) s = fmaf(bk[k], uw[i + NBT - 1 - k], s);
    w[i] = s;
  }
}

// The coefficients of pair lid % Pp, the pair that lane l0 + lid holds in every tile (l0 a multiple
// of 64 and Pp dividing 64): loaded once per workgroup. Idle lanes (padding or beyond the tensor)
// see zero inputs and store nothing; they take pair 0's coefficients.
template <int NA, int NBT>
TSF_DEV void load_pair_coeffs(double (&av)[NA], float (&bk)[NBT], const float* __restrict__ bcoef,
                              const float* __restrict__ acoef, int lid, int I, int O, int nb, int Pp) {
  int p = lid % Pp;
  if (p >= I * O) p = 0;
  const int pair = (p % O) * I + p / O;  // [O, I, .] parameter layout
#pragma unroll
  for (int q = 0; q < NA; ++q) av[q] = (double)acoef[pair * NA + q];
#pragma unroll
  for (int k = 0; k < NBT; ++k) bk[k] = k < nb ? bcoef[pair * nb + k] : 0.0f;
}

// Transfer matrices per lane from its pair's coefficients a [O, I, NA] (lane = b * Pp + j * O + o;
// padding lanes take pair 0's). One thread per (lane, column); the last rj.blocks workgroups run
// the scan's look-back reset.
template <int NA>
__global__ void __launch_bounds__(64) gblock_transfer(const float* __restrict__ acoef, double* __restrict__ Mc,
                                                      double* __restrict__ Ms, int64_t lanes, int I, int O, int Pp,
                                                      int K, ResetJob rj) {
  const unsigned tb = gridDim.x - rj.blocks;
  if (blockIdx.x >= tb) {
    run_reset(rj, blockIdx.x - tb);
    return;
  }
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= lanes * NA) return;
  const int64_t lane = idx / NA;
  int p = (int)(lane % Pp);
  if (p >= I * O) p = 0;
  const int j = p / O, o = p % O;
  companion_powers_col<NA>(acoef + (o * I + j) * NA, Mc + lane * NA * NA, Ms + lane * NA * NA, K,
                           (int)(idx - lane * NA));
}

// ---------------------------------------------------------------------------------- forward
template <int NA, int NBT>
__global__ void __launch_bounds__(64 * kLbWaves) gblock_fwd_lb(
    const float* __restrict__ u, const float* __restrict__ bcoef, const float* __restrict__ acoef,
    const float* __restrict__ u_tail, const float* __restrict__ x0, float* __restrict__ y, float* __restrict__ x_last,
    double* __restrict__ saved, const double* __restrict__ Mc, const double* __restrict__ Ms, double* __restrict__ agg,
    double* __restrict__ inc, unsigned* __restrict__ counter, int64_t B, int64_t L, int I, int O, int Pp, int nb,
    int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  __shared__ LdsTile s_lds[kLbWaves];
  __shared__ int s_flag[kLbWaves][64];
  __shared__ int s_pend[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  __shared__ double s_mat[MatStage<NA>::kDoubles];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int P = I * O, R = kTile / Pp;
  const int64_t lanes = B * Pp;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * kTileT;
  // the pair's coefficients and transfer matrices are the same in every tile (load_pair_coeffs)
  double av[NA];
  float bk[NBT];
  load_pair_coeffs<NA, NBT>(av, bk, bcoef, acoef, lid, I, O, nb, Pp);
  if constexpr (MatStage<NA>::kLds) stage_mats<NA>(s_mat, Mc, Ms, 0, lanes);
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t sc = tile / groups, l0 = (tile - sc * groups) * kTile, lane = l0 + lid;
    const GbLane g = gb_lane(lane, lanes, P, Pp, O);
    const bool live = g.live;
    const int64_t t0 = sc * SL + (int64_t)k * kTileT;
    const int n = (L - t0) >= kTileT ? kTileT : (L - t0) > 0 ? (int)(L - t0) : 0;
    double s[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) s[q] = 0.0;
    float xb[kTileT];
    if (n > 0) {
      float uw[kTileT + NBT - 1];
      load_u_window<NBT>(uw, u, u_tail, g, t0, L, I, nb);
      fir<NBT>(xb, uw, bk);
      if (n == kTileT) {
#pragma unroll
        for (int i = 0; i < kTileT; ++i) step<NA>(av, s, (double)xb[i]);
      } else {
#pragma unroll
        for (int i = 0; i < kTileT; ++i)
          if (i < n) step<NA>(av, s, (double)xb[i]);
      }
    }
    double* vk = vec_area<NA>(s_lds, k) + lid * NA;
#pragma unroll
    for (int q = 0; q < NA; ++q) vk[q] = s[q];
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    double sup[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) sup[q] = 0.0;
    if (k == 0 && live) {
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NA * NA] : Mc + lane * NA * NA);
      for (int jj = 0; jj < K; ++jj) {
        double ej[NA];
        const double* vj = vec_area<NA>(s_lds, jj) + lid * NA;
#pragma unroll
        for (int q = 0; q < NA; ++q) ej[q] = vj[q];
        matvec_add<NA>(sup, mc, sup, ej);
      }
      if (lb_pub_agg(sc, lb_spacing) && sc + 1 < nsuper) put_vec<NA>(agg + (sc * lanes + lane) * NA, sup);
    }
    double S[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) S[q] = (sc == 0 && x0 && live && k == 0) ? (double)x0[g.rl * NA + q] : 0.0;
    if (sc > 0)  // uniform over the workgroup
      ap_look_back<NA>(S, agg, inc, MatStage<NA>::kLds ? &s_mat[64 * NA * NA + lid * NA * NA] : Ms + lane * NA * NA, k == 0 && live, sc - 1, (int64_t)-1, nsuper, lanes, lane, K,
                       k, lid, s_lds, s_flag, s_pend, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (saved) {
#pragma unroll
        for (int q = 0; q < NA; ++q) saved[(sc * lanes + lane) * NA + q] = S[q];
      }
      if (lb_pub_inc(sc, lb_spacing) && sc + 1 < nsuper) {
        double ms[NA][NA], o[NA];
        load_mat<NA>(ms, MatStage<NA>::kLds ? &s_mat[64 * NA * NA + lid * NA * NA] : Ms + lane * NA * NA);
        matvec_add<NA>(o, ms, S, sup);
        put_vec<NA>(inc + (sc * lanes + lane) * NA, o);
      }
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NA * NA] : Mc + lane * NA * NA);
      for (int jj = 0; jj < K; ++jj) {
        double ej[NA];
        double* vj = vec_area<NA>(s_lds, jj) + lid * NA;
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
      // the delay line after the sequence's last step is the returned state (newest first)
      if (x_last && live && t0 + n == L) {
#pragma unroll
        for (int q = 0; q < NA; ++q) x_last[g.rl * NA + q] = (float)s[q];
      }
      // y[b, t, o] = sum_j y_{j*O+o}[t]: the pairs' rows meet in the wave's LDS tile
      float(*tl)[kTileT + 1] = s_lds[k];
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < kTileT; ++i) tl[lid][i] = xb[i];
      __builtin_amdgcn_wave_barrier();
      const int64_t b0 = l0 / Pp;
      for (int qi = lid; qi < R * kTileT * O; qi += kTile) {
        const int o = qi % O, i = (qi / O) % kTileT, rb = qi / (O * kTileT);
        const int64_t bb = b0 + rb;
        if (i < n && bb < B) {
          float acc = 0.0f;
#pragma unroll 8
          for (int jj = 0; jj < I; ++jj) acc += tl[rb * Pp + jj * O + o][i];  // reads go out together
          y[(bb * L + t0 + i) * O + o] = acc;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// --------------------------------------------------------------------------------- backward
// Per-lane partials of one tile: grad a (NA doubles) then grad b (NBT floats) in a wave's LDS tile.
template <int NA, int NBT>
TSF_DEV double* part_a_area(LdsTile* lds, int wv) {
  return reinterpret_cast<double*>(&lds[wv][0][0]);
}
template <int NA, int NBT>
TSF_DEV float* part_b_area(LdsTile* lds, int wv) {
  return reinterpret_cast<float*>(reinterpret_cast<double*>(&lds[wv][0][0]) + 64 * NA);
}

// Runs body(whole) with whole a compile-time true for a whole tile (n == kTileT steps, every
// chunk but the sequence's last) and false otherwise. A loop whose steps are each guarded by
// `i < n` makes the compiler merge the recurrence state at every step (register copies on every
// step); the whole-tile instance has no guards.
template <typename F>
TSF_DEV void whole_or_part(int n, F&& body) {
  if (n == kTileT)
    body(std::true_type{});
  else
    body(std::false_type{});
}

template <int NA, int NBT>
__global__ void __launch_bounds__(64 * kLbWaves) gblock_bwd_lb(
    const float* __restrict__ gy, const float* __restrict__ g_xlast, const float* __restrict__ u,
    const float* __restrict__ bcoef, const float* __restrict__ acoef, const float* __restrict__ u_tail,
    const float* __restrict__ x0, const double* __restrict__ saved, const double* __restrict__ Mc,
    const double* __restrict__ Ms, double* __restrict__ agg, double* __restrict__ inc, unsigned* __restrict__ counter,
    float* __restrict__ gu, float* __restrict__ gu_tail, double* __restrict__ part_ga, double* __restrict__ part_gb,
    double* __restrict__ gh, int64_t B, int64_t L, int I, int O, int Pp, int nb, int64_t groups, int K, int64_t nsuper,
    LbCfg lb_spacing) {
  static_assert(64 * (NA * sizeof(double) + NBT * sizeof(float)) <= sizeof(LdsTile), "partials fit in a tile");
  constexpr int V = 2 * NA;  // adjoint state: G then c
  __shared__ LdsTile s_lds[kLbWaves];
  __shared__ int s_flag[kLbWaves][64];
  __shared__ int s_pend[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  __shared__ double s_mat[MatStage<NA>::kDoubles];
  // each wave's u window, kept from the forward recompute for the sweep's grad b (NBT <= 8: 80 KB)
  constexpr int kUW = kTileT + NBT - 1;
  constexpr bool kStashU = NBT <= 8;
  __shared__ float s_uw[kStashU ? kLbWaves : 1][kStashU ? 64 : 1][kStashU ? kUW : 1];
  __shared__ double s_st[64][NA];  // the super-chunk's saved entering state, prefetched by wave 0
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int P = I * O, R = kTile / Pp;
  const int64_t lanes = B * Pp;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * kTileT;
  // the pair's coefficients and transfer matrices are the same in every tile (load_pair_coeffs)
  double av[NA];
  float bk[NBT];
  load_pair_coeffs<NA, NBT>(av, bk, bcoef, acoef, lid, I, O, nb, Pp);
  if constexpr (MatStage<NA>::kLds) stage_mats<NA>(s_mat, Mc, Ms, 0, lanes);
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t r = tile / groups, sc = nsuper - 1 - r, l0 = (tile - r * groups) * kTile, lane = l0 + lid;
    const GbLane g = gb_lane(lane, lanes, P, Pp, O);
    const bool live = g.live;
    const int64_t t0 = sc * SL + (int64_t)k * kTileT;
    const int n = (L - t0) >= kTileT ? kTileT : (L - t0) > 0 ? (int)(L - t0) : 0;
    double s[NA];
    // The phases are ordered so that no 32-step window is live across the look-back: the adjoint
    // summaries and look-back first (g window dropped after the summaries), then the forward
    // recompute of y_p, then the sweep over a reloaded g window.
    auto load_g_window = [&](float (&gw_)[kTileT + NBT - 1]) __attribute__((always_inline)) {
      const float* __restrict__ grow = gy + g.b * L * O + g.o;
#pragma unroll
      for (int i = 0; i < kTileT + NBT - 1; ++i) {
        const int64_t s2 = t0 + i;
        float v = (live && s2 < L) ? grow[s2 * O] : 0.0f;
        if (g_xlast && live && s2 < L && s2 >= L - NA) v += g_xlast[g.rl * NA + (L - 1 - s2)];
        gw_[i] = v;
      }
    };
    double* vk = vec_area<NA>(s_lds, k) + lid * V;
    double sG[NA], sC[NA];
    // wave 0 issues the load of the super-chunk's saved entering state with its g window, so that
    // its latency overlaps theirs; parked in LDS for the state composition below
    double st_pre[NA];
    if (k == 0) {
#pragma unroll
      for (int q = 0; q < NA; ++q)
        st_pre[q] = !live ? 0.0 : sc == 0 ? (x0 ? (double)x0[g.rl * NA + q] : 0.0) : saved[(sc * lanes + lane) * NA + q];
    }
    {
      // --- zero-state summaries of both adjoint recurrences over the chunk, right to left
      float gw[kTileT + NBT - 1];
      load_g_window(gw);
#pragma unroll
      for (int q = 0; q < NA; ++q) sG[q] = sC[q] = 0.0;
      whole_or_part(n, [&](auto whole) __attribute__((always_inline)) {
#pragma unroll
        for (int i = kTileT - 1; i >= 0; --i)
          if (decltype(whole)::value || i < n) {
            float h = 0.0f;
#pragma unroll
            for (int kk = 0; kk < NBT; ++kk) h = fmaf(bk[kk], gw[i + kk], h);
            step<NA>(av, sG, (double)gw[i]);
            step<NA>(av, sC, (double)h);
          }
      });
    }
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      vk[q] = sG[q];
      vk[NA + q] = sC[q];
    }
    if (k == 0) {
#pragma unroll
      for (int q = 0; q < NA; ++q) s_st[lid][q] = st_pre[q];
    }
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    double sup[V];
#pragma unroll
    for (int q = 0; q < V; ++q) sup[q] = 0.0;
    if (k == 0 && live) {
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NA * NA] : Mc + lane * NA * NA);
      for (int jj = K - 1; jj >= 0; --jj) {
        double fj[V];
        const double* vj = vec_area<NA>(s_lds, jj) + lid * V;
#pragma unroll
        for (int q = 0; q < V; ++q) fj[q] = vj[q];
        block_matvec_add<NA, 2>(sup, mc, sup, fj);
      }
      if (lb_pub_agg(nsuper - 1 - sc, lb_spacing) && sc > 0) put_vec<V>(agg + (sc * lanes + lane) * V, sup);
    }
    double Rv[V];  // adjoint state entering the super-chunk from the right
#pragma unroll
    for (int q = 0; q < V; ++q) Rv[q] = 0.0;
    if (sc + 1 < nsuper)  // uniform over the workgroup
      ap_look_back<NA, 2>(Rv, agg, inc, MatStage<NA>::kLds ? &s_mat[64 * NA * NA + lid * NA * NA] : Ms + lane * NA * NA, k == 0 && live, sc + 1, (int64_t)1, nsuper, lanes, lane,
                          K, k, lid, s_lds, s_flag, s_pend, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(nsuper - 1 - sc, lb_spacing) && sc > 0) {
        double ms[NA][NA], o[V];
        load_mat<NA>(ms, MatStage<NA>::kLds ? &s_mat[64 * NA * NA + lid * NA * NA] : Ms + lane * NA * NA);
        block_matvec_add<NA, 2>(o, ms, Rv, sup);
        put_vec<V>(inc + (sc * lanes + lane) * V, o);
      }
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NA * NA] : Mc + lane * NA * NA);
      for (int jj = K - 1; jj >= 0; --jj) {
        double fj[V];
        double* vj = vec_area<NA>(s_lds, jj) + lid * V;
#pragma unroll
        for (int q = 0; q < V; ++q) {
          fj[q] = vj[q];
          vj[q] = Rv[q];
        }
        block_matvec_add<NA, 2>(Rv, mc, Rv, fj);
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NA; ++q) {  // this chunk's adjoint entering state, kept for the sweep
      sG[q] = vk[q];
      sC[q] = vk[NA + q];
    }
    // --- forward recompute of the chunk's pair outputs y_p (into xb) from the saved state
    float xb[kTileT];
#pragma unroll
    for (int q = 0; q < NA; ++q) s[q] = 0.0;
    if (n > 0) {
      float uw[kTileT + NBT - 1];
      load_u_window<NBT>(uw, u, u_tail, g, t0, L, I, nb);
      if constexpr (kStashU) {
#pragma unroll
        for (int i = 0; i < kUW; ++i) s_uw[k][lid][i] = uw[i];
      }
      fir<NBT>(xb, uw, bk);
      whole_or_part(n, [&](auto whole) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kTileT; ++i)
          if (decltype(whole)::value || i < n) step<NA>(av, s, (double)xb[i]);
      });
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int q = 0; q < NA; ++q) vk[q] = s[q];
    __syncthreads();
    if (k == 0 && live) {
      double st[NA];
#pragma unroll
      for (int q = 0; q < NA; ++q) st[q] = s_st[lid][q];
      double mc[NA][NA];
      load_mat<NA>(mc, MatStage<NA>::kLds ? &s_mat[lid * NA * NA] : Mc + lane * NA * NA);
      for (int jj = 0; jj < K; ++jj) {
        double ej[NA];
        double* vj = vec_area<NA>(s_lds, jj) + lid * V;
#pragma unroll
        for (int q = 0; q < NA; ++q) {
          ej[q] = vj[q];
          vj[q] = st[q];
        }
        matvec_add<NA>(st, mc, st, ej);
      }
    }
    __syncthreads();
    if (n > 0) {
#pragma unroll
      for (int q = 0; q < NA; ++q) s[q] = vk[q];
      whole_or_part(n, [&](auto whole) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kTileT; ++i)
          if (decltype(whole)::value || i < n) xb[i] = (float)step<NA>(av, s, (double)xb[i]);
      });
    }
    // --- adjoint sweep: G, c, grad a, grad b, head taps and the tail gradient
    double ga[NA];
    float gbk[NBT];
#pragma unroll
    for (int q = 0; q < NA; ++q) ga[q] = 0.0;
#pragma unroll
    for (int kk = 0; kk < NBT; ++kk) gbk[kk] = 0.0f;
    float(*tl)[kTileT + 1] = s_lds[k];
    if (n > 0) {
      float gw[kTileT + NBT - 1];
      load_g_window(gw);
      // pass 1, right to left: G, c (into xb) and grad a; G_t then goes into gw[i + NBT - 1],
      // the window slot no later step reads (step i' < i reads gw[i' .. i' + NBT - 1])
      whole_or_part(n, [&](auto whole) __attribute__((always_inline)) {
#pragma unroll
        for (int i = kTileT - 1; i >= 0; --i)
          if (decltype(whole)::value || i < n) {
            const double yu = xb[i];
#pragma unroll
            for (int q = 0; q < NA; ++q) ga[q] = fma(sG[q], yu, ga[q]);  // sG_q = G_{t+1+q} before the step
            float h = 0.0f;
#pragma unroll
            for (int kk = 0; kk < NBT; ++kk) h = fmaf(bk[kk], gw[i + kk], h);
            const float G = (float)step<NA>(av, sG, (double)gw[i]);
            xb[i] = (float)step<NA>(av, sC, (double)h);  // c_t, the pair's input gradient at t
            gw[i + NBT - 1] = G;
          }
      });
      // gu[b, t, j] = sum_o c_{j*O+o}[t] through the wave's LDS tile
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < kTileT; ++i) tl[lid][i] = xb[i];
      __builtin_amdgcn_wave_barrier();
      const int64_t b0 = l0 / Pp;
      for (int qi = lid; qi < R * kTileT * I; qi += kTile) {
        const int jj = qi % I, i = (qi / I) % kTileT, rb = qi / (I * kTileT);
        const int64_t bb = b0 + rb;
        if (i < n && bb < B) {
          float acc = 0.0f;
#pragma unroll 8
          for (int o = 0; o < O; ++o) acc += tl[rb * Pp + jj * O + o][i];  // reads go out together
          gu[(bb * L + t0 + i) * I + jj] = acc;
        }
      }
      // pass 2: grad b = sum_t G_t u_{t-k} (u window reloaded), head taps, tail gradient
      float gt[NBT > 1 ? NBT - 1 : 1];  // tail gradient of this lane, t0 == 0 only
#pragma unroll
      for (int m = 0; m < (NBT > 1 ? NBT - 1 : 1); ++m) gt[m] = 0.0f;
      {
        float uw[kTileT + NBT - 1];
        if constexpr (kStashU) {
#pragma unroll
          for (int i = 0; i < kUW; ++i) uw[i] = s_uw[k][lid][i];  // this wave's own, same lane
        } else {
          load_u_window<NBT>(uw, u, u_tail, g, t0, L, I, nb);
        }
        whole_or_part(n, [&](auto whole) __attribute__((always_inline)) {
#pragma unroll
          for (int i = 0; i < kTileT; ++i)
            if (decltype(whole)::value || i < n) {
              const float G = gw[i + NBT - 1];
#pragma unroll
              for (int kk = 0; kk < NBT; ++kk) gbk[kk] = fmaf(G, uw[i + NBT - 1 - kk], gbk[kk]);
              if (t0 == 0) {
                // u_tail[m] (time m - (nb - 1)) met b_kk at steps i = m - (nb - 1) + kk >= 0
#pragma unroll
                for (int kk = 1; kk < NBT; ++kk)
                  if (i < kk && i - kk + NBT - 1 >= 0) gt[i - kk + NBT - 1] = fmaf(bk[kk], G, gt[i - kk + NBT - 1]);
                if (i < NA && live) gh[lane * NA + i] = G;  // G_0 .. G_{NA-1} for the x0 head taps
              }
            }
        });
      }
      if (t0 == 0 && gu_tail && nb > 1) {
        // gt[m'] holds tail position m' - (NBT - 1) + (nb - 1) = m; only m' >= NBT - nb are real
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int m = 0; m < (NBT > 1 ? NBT - 1 : 1); ++m) tl[lid][m] = gt[m];
        __builtin_amdgcn_wave_barrier();
        for (int qi = lid; qi < R * (nb - 1) * I; qi += kTile) {
          const int jj = qi % I, m = (qi / I) % (nb - 1), rb = qi / (I * (nb - 1));
          const int64_t bb = b0 + rb;
          if (bb < B) {
            float acc = 0.0f;
#pragma unroll 8
            for (int o = 0; o < O; ++o) acc += tl[rb * Pp + jj * O + o][m + NBT - nb];
            gu_tail[(bb * (nb - 1) + m) * I + jj] = acc;
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    // grad a / grad b partials: summed over the K chunks in LDS, one row per (super-chunk, lane)
    {
      double* pa = part_a_area<NA, NBT>(s_lds, k) + lid * NA;
      float* pb = part_b_area<NA, NBT>(s_lds, k) + lid * NBT;
#pragma unroll
      for (int q = 0; q < NA; ++q) pa[q] = ga[q];
#pragma unroll
      for (int kk = 0; kk < NBT; ++kk) pb[kk] = gbk[kk];
    }
    __syncthreads();
    // wave w of the K sums partial values w, w + K, ... of its lane over the K chunks, in chunk
    // order (the chunks' reads issued together)
    if (live) {
      for (int v = k; v < NA + NBT; v += K) {
        double pv[kLbWaves];
#pragma unroll
        for (int jj = 0; jj < kLbWaves; ++jj)
          pv[jj] = jj >= K   ? 0.0
                   : v < NA ? (part_a_area<NA, NBT>(s_lds, jj) + lid * NA)[v]
                            : (double)(part_b_area<NA, NBT>(s_lds, jj) + lid * NBT)[v - NA];
        double t = 0.0;
#pragma unroll
        for (int jj = 0; jj < kLbWaves; ++jj)
          if (jj < K) t += pv[jj];
        if (v < NA)
          part_ga[(sc * lanes + lane) * NA + v] = t;
        else
          part_gb[(sc * lanes + lane) * NBT + (v - NA)] = t;
      }
    }
    __syncthreads();  // every wave's reads of the tile precede the next tile's writes into them
  }
}

// Per lane: grad a = -(sum over super-chunks + x0 head taps), grad x0 (head taps plus the x_last
// gradient that lands on x0 when L < na), grad b = sum over super-chunks; the super-chunk sums
// run in a fixed order (16 waves per 64 lanes, contiguous segments, then in order).
template <int NA, int NBT>
__global__ void __launch_bounds__(1024) gblock_finish_lane(
    const float* __restrict__ acoef, const float* __restrict__ x0, const float* __restrict__ g_xlast,
    const double* __restrict__ gh, const double* __restrict__ part_ga, const double* __restrict__ part_gb,
    double* __restrict__ ga_lane, double* __restrict__ gb_lane, float* __restrict__ gx0, int64_t lanes, int I, int O,
    int Pp, int64_t L, int64_t n) {
  __shared__ double s_p[16][64];
  __shared__ double s_tot[NA + NBT][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t lane = blockIdx.x * 64 + lid;
  const int P = I * O;
  const int p = (int)(lane % Pp);
  const bool live = lane < lanes && p < P;
  const int64_t rl = lane / Pp * P + p;  // the caller's [B, P, na] row
  const int64_t seg = (n + 15) / 16;
  const int64_t r0 = k * seg, r1 = (r0 + seg < n) ? r0 + seg : n;
  for (int q = 0; q < NA + NBT; ++q) {
    double acc = 0.0;
    if (live)
      for (int64_t r = r0; r < r1; ++r)
        acc += q < NA ? part_ga[(r * lanes + lane) * NA + q] : part_gb[(r * lanes + lane) * NBT + (q - NA)];
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
  const int j = p / O, o = p % O;
  const int pair = o * I + j;
  double Gh[NA];  // G_0 .. G_{NA-1}, zero past the end of the sequence
#pragma unroll
  for (int q = 0; q < NA; ++q) Gh[q] = (q < L) ? gh[lane * NA + q] : 0.0;
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    double t = s_tot[q][lid];
    if (x0) {
#pragma unroll
      for (int jj = 1; jj <= q + 1; ++jj) t = fma(Gh[q + 1 - jj], (double)x0[rl * NA + jj - 1], t);
    }
    ga_lane[lane * NA + q] = -t;
  }
#pragma unroll
  for (int kk = 0; kk < NBT; ++kk) gb_lane[lane * NBT + kk] = s_tot[NA + kk][lid];
  if (gx0) {
#pragma unroll
    for (int jj = 0; jj < NA; ++jj) {
      double t = 0.0;
#pragma unroll
      for (int i = jj + 1; i <= NA; ++i) t = fma((double)acoef[pair * NA + i - 1], Gh[i - 1 - jj], t);
      t = -t;
      // x_last[q] = x0[q - L] for q >= L: that part of the x_last gradient reaches x0 directly
      if (g_xlast && jj + L < NA) t += (double)g_xlast[rl * NA + jj + L];
      gx0[rl * NA + jj] = (float)t;
    }
  }
}

// grad a [O, I, NA] and grad b [O, I, nb]: per pair, the sum over batch rows in order.
template <int NA, int NBT>
__global__ void __launch_bounds__(256) gblock_finish_pairs(const double* __restrict__ ga_lane,
                                                            const double* __restrict__ gb_lane, float* __restrict__ ga,
                                                            float* __restrict__ gb, int64_t B, int I, int O, int Pp,
                                                            int nb) {
  const int P = I * O;
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= (int64_t)P * (NA + nb)) return;
  const int p = (int)(idx / (NA + nb)), q = (int)(idx % (NA + nb));
  const int j = p / O, o = p % O, pair = o * I + j;
  double t = 0.0;
#pragma unroll 8
  for (int64_t b = 0; b < B; ++b)
    t += q < NA ? ga_lane[(b * Pp + p) * NA + q] : gb_lane[(b * Pp + p) * NBT + (q - NA)];
  if (q < NA)
    ga[pair * NA + q] = (float)t;
  else
    gb[pair * nb + (q - NA)] = (float)t;
}

// L == 0: the returned state is x0 (zero without it).
__global__ void __launch_bounds__(256) gblock_copy_state(const float* __restrict__ x0, float* __restrict__ x_last,
                                                          int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) x_last[i] = x0 ? x0[i] : 0.0f;
}

__global__ void __launch_bounds__(256) gblock_zero(float* __restrict__ p, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// ------------------------------------------------------------------------------------- host
int nbt_for(int64_t nb) { return nb <= 2 ? 2 : nb <= 4 ? 4 : nb <= 8 ? 8 : 16; }

// Workspace (both directions): the tile counter, agg and inc [nsuper][lanes][2 na] (reset before
// each scan), grad-a and grad-b partials [nsuper][lanes][na | NBT], the head taps G_0.. [lanes][na],
// per-lane grad a / grad b [lanes][na | NBT], and the transfer matrices Mc, Ms [lanes][na][na].
struct GbPlan {
  LbPlan lb;
  int64_t lanes = 0;  // B * Pp: batch rows padded to a power-of-two pair count
  int pp = 1;
  int nbt = 2;
  size_t off_agg = 0, off_inc = 0, off_pa = 0, off_pb = 0, off_gh = 0, off_gal = 0, off_gbl = 0, off_Mc = 0,
         off_Ms = 0, bytes = 0;
};

GbPlan gb_plan(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na) {
  GbPlan p;
  p.pp = padded_pairs((int)(I * O));
  p.lanes = B * p.pp;
  p.nbt = nbt_for(nb);
  p.lb = lb_plan(p.lanes, L, na);
  const size_t f = 8, rows = (size_t)p.lb.nsuper * p.lanes;
  p.off_agg = kCounterBytes;
  p.off_inc = p.off_agg + f * rows * 2 * na;
  p.off_pa = p.off_inc + f * rows * 2 * na;
  p.off_pb = p.off_pa + f * rows * na;
  p.off_gh = p.off_pb + f * rows * p.nbt;
  p.off_gal = p.off_gh + f * p.lanes * na;
  p.off_gbl = p.off_gal + f * p.lanes * na;
  p.off_Mc = p.off_gbl + f * p.lanes * p.nbt;
  p.off_Ms = p.off_Mc + f * p.lanes * na * na;
  p.bytes = p.off_Ms + f * p.lanes * na * na;
  return p;
}

int gb_args_status(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na) {
  if (B < 0 || L < 0 || I < 1 || O < 1 || nb < 1 || na < 1) return TSF_ERR_ARG;
  if (na > kLbNA || nb > kGbMaxNB || I * O > kTile) return TSF_ERR_UNSUPPORTED;
  if (B * I * O * (L > 0 ? L : 1) >= ((int64_t)1 << 40)) return TSF_ERR_UNSUPPORTED;
  return TSF_OK;
}

template <int NA, int NBT>
void fwd_impl(const GbPlan& p, int64_t B, int64_t L, int I, int O, int nb, const float* u, const float* bcoef,
              const float* acoef, const float* u_tail, const float* x0, float* y, float* x_last, double* saved,
              char* ws, hipStream_t s) {
  static int occ[kMaxNA + 1];
  double* Mc = reinterpret_cast<double*>(ws + p.off_Mc);
  double* Ms = reinterpret_cast<double*>(ws + p.off_Ms);
  const ResetJob rj = reset_job(ws, p.lb.nsuper * p.lanes * 2 * NA * 2, 64);
  hipLaunchKernelGGL((gblock_transfer<NA>), dim3(transfer_grid(p.lanes, NA).x + rj.blocks), dim3(64), 0, s, acoef, Mc,
                     Ms, p.lanes, I, O, p.pp, p.lb.K, rj);
  const int64_t tiles = p.lb.groups * p.lb.nsuper, cap = resident_wgs(gblock_fwd_lb<NA, NBT>, 64 * p.lb.K, occ);
  hipLaunchKernelGGL((gblock_fwd_lb<NA, NBT>), dim3((unsigned)(tiles < cap ? tiles : cap)), dim3(64 * p.lb.K), 0, s, u,
                     bcoef, acoef, u_tail, x0, y, x_last, saved, (const double*)Mc, (const double*)Ms,
                     reinterpret_cast<double*>(ws + p.off_agg), reinterpret_cast<double*>(ws + p.off_inc),
                     reinterpret_cast<unsigned*>(ws), B, L, I, O, p.pp, nb, p.lb.groups, p.lb.K, p.lb.nsuper,
                     lb_spacing_for(kGbAnchorSpacing));
}

template <int NA, int NBT>
void bwd_impl(const GbPlan& p, int64_t B, int64_t L, int I, int O, int nb, const float* gy, const float* g_xlast,
              const float* u, const float* bcoef, const float* acoef, const float* u_tail, const float* x0,
              const double* saved, float* gu, float* gu_tail, float* gb, float* ga, float* gx0, char* ws,
              hipStream_t s) {
  static int occ[kMaxNA + 1];
  double* gh = reinterpret_cast<double*>(ws + p.off_gh);
  double* pa = reinterpret_cast<double*>(ws + p.off_pa);
  double* pb = reinterpret_cast<double*>(ws + p.off_pb);
  if (L > 0) {
    double* Mc = reinterpret_cast<double*>(ws + p.off_Mc);
    double* Ms = reinterpret_cast<double*>(ws + p.off_Ms);
    const ResetJob rj = reset_job(ws, p.lb.nsuper * p.lanes * 2 * NA * 2, 64);
    hipLaunchKernelGGL((gblock_transfer<NA>), dim3(transfer_grid(p.lanes, NA).x + rj.blocks), dim3(64), 0, s, acoef, Mc,
                       Ms, p.lanes, I, O, p.pp, p.lb.K, rj);
    const int64_t tiles = p.lb.groups * p.lb.nsuper, cap = resident_wgs(gblock_bwd_lb<NA, NBT>, 64 * p.lb.K, occ);
    hipLaunchKernelGGL((gblock_bwd_lb<NA, NBT>), dim3((unsigned)(tiles < cap ? tiles : cap)), dim3(64 * p.lb.K), 0, s,
                       gy, g_xlast, u, bcoef, acoef, u_tail, x0, saved, (const double*)Mc, (const double*)Ms,
                       reinterpret_cast<double*>(ws + p.off_agg), reinterpret_cast<double*>(ws + p.off_inc),
                       reinterpret_cast<unsigned*>(ws), gu, gu_tail, pa, pb, gh, B, L, I, O, p.pp, nb, p.lb.groups,
                       p.lb.K, p.lb.nsuper, lb_spacing_for(kGbAnchorSpacing));
  } else if (gu_tail && nb > 1) {
    const int64_t nt = B * (nb - 1) * I;
    hipLaunchKernelGGL(gblock_zero, grid_for(nt), dim3(256), 0, s, gu_tail, nt);
  }
  double* gal = reinterpret_cast<double*>(ws + p.off_gal);
  double* gbl = reinterpret_cast<double*>(ws + p.off_gbl);
  hipLaunchKernelGGL((gblock_finish_lane<NA, NBT>), dim3((unsigned)p.lb.groups > 0 ? (unsigned)p.lb.groups : 1u),
                     dim3(1024), 0, s, acoef, x0, g_xlast, (const double*)gh, (const double*)pa, (const double*)pb, gal,
                     gbl, gx0, p.lanes, I, O, p.pp, L, L > 0 ? p.lb.nsuper : (int64_t)0);
  const int64_t np = (int64_t)I * O * (NA + nb);
  hipLaunchKernelGGL((gblock_finish_pairs<NA, NBT>), grid_for(np), dim3(256), 0, s, (const double*)gal,
                     (const double*)gbl, ga, gb, B, I, O, p.pp, nb);
}

// ------------------------------------------------------------------------------- FIR stage
// The G-block's FIR stage on its own, for denominators above the fused kernels' orders (the
// all-pole stage then runs as tsfast_hip::dynonet_allpole on the pair lanes, and the pairs are
// summed over inputs): the grouped causal convolution of dynonet/core.py:219-222,
//   w[b, j*O + o, t] = sum_{k < nb} b[o, j, k] u[b, t - k, j]     (u[b, -m, j] = u_tail[b, nb-1-m, j])
// with w in the all-pole lane layout [B, I*O, L] (time contiguous). A workgroup takes one batch
// row, one input channel and kFirT steps, a thread kFirS consecutive steps: the steps' u values
// and their halo go through LDS once (u is channel-last, so a row of steps is strided), each
// thread keeps its window of them in registers and forms its steps for every output channel
// from it. The tap count is padded to NBT (4, 8, 16, 32 or 64; the padding taps are zero), so
// the inner loops are fixed; a block of kFirOB output channels' taps sits in LDS, read by every
// thread at the same address.
constexpr int kFirS = 4;                // steps per thread: one 16-byte row segment of w
constexpr int kFirW = 256;              // threads per workgroup
constexpr int kFirT = kFirS * kFirW;    // steps per workgroup
constexpr int kFirMaxNB = 64;
constexpr int kFirOB = 8;               // output channels per LDS round

inline int fir_nbt(int64_t nb) { return nb <= 4 ? 4 : nb <= 8 ? 8 : nb <= 16 ? 16 : nb <= 32 ? 32 : 64; }

struct FirTile {
  int64_t b, t0;
  int j;
};
// workgroup -> (batch row, input channel, tile); the grid has at most INT32_MAX workgroups
TSF_DEV FirTile fir_tile(unsigned tiles_t, unsigned I) {
  FirTile f;
  const unsigned g = blockIdx.x, rest = g / tiles_t;
  f.t0 = (int64_t)(g - rest * tiles_t) * kFirT;
  f.j = (int)(rest % I);
  f.b = rest / I;
  return f;
}
// u_ext[b, t, j] for t in [-(nb - 1), L): u, then the carried tail (zero without it, and zero
// outside both)
TSF_DEV float fir_u(const float* __restrict__ u, const float* __restrict__ u_tail, int64_t b, int64_t t, int j,
                    int64_t L, int I, int nb) {
  if (t >= 0) return t < L ? u[(b * L + t) * I + j] : 0.0f;
  if (!u_tail || t < -(int64_t)(nb - 1)) return 0.0f;
  return u_tail[(b * (nb - 1) + (nb - 1 + t)) * I + j];
}
// s_u[i] = u_ext[t0 - (NBT - 1) + i], i < kFirT + NBT: every load issued before the first LDS
// store, so the thread waits on them together rather than one round trip at a time
template <int NBT>
TSF_DEV void fir_stage_u(float* s_u, const float* __restrict__ u, const float* __restrict__ u_tail, const FirTile& f,
                         int64_t L, int I, int nb) {
  constexpr int NU = (kFirT + NBT + kFirW - 1) / kFirW;
  float v[NU];
#pragma unroll
  for (int c = 0; c < NU; ++c) {
    const int i = threadIdx.x + c * kFirW;
    v[c] = i < kFirT + NBT ? fir_u(u, u_tail, f.b, f.t0 - (NBT - 1) + i, f.j, L, I, nb) : 0.0f;
  }
#pragma unroll
  for (int c = 0; c < NU; ++c) {
    const int i = threadIdx.x + c * kFirW;
    if (i < kFirT + NBT) s_u[i] = v[c];
  }
}
// taps of output channels o0 .. o0 + kFirOB - 1 for input j, zero past nb and past O
template <int NBT>
TSF_DEV void fir_stage_b(float (*s_b)[NBT], const float* __restrict__ bcoef, int o0, int O, int I, int j, int nb) {
  for (int e = threadIdx.x; e < kFirOB * NBT; e += kFirW) {
    const int r = e / NBT, k = e - r * NBT;
    s_b[r][k] = (o0 + r < O && k < nb) ? bcoef[((int64_t)(o0 + r) * I + j) * nb + k] : 0.0f;
  }
}
// x[m] = s[4 * threadIdx.x + m], m < N (16-byte LDS reads; s is 16-byte aligned)
template <int N>
TSF_DEV void fir_window(float (&x)[N], const float* s) {
  const float4* p = reinterpret_cast<const float4*>(s) + threadIdx.x;
#pragma unroll
  for (int c = 0; c < (N + 3) / 4; ++c) {
    const float4 q = p[c];
    if (4 * c + 0 < N) x[4 * c + 0] = q.x;
    if (4 * c + 1 < N) x[4 * c + 1] = q.y;
    if (4 * c + 2 < N) x[4 * c + 2] = q.z;
    if (4 * c + 3 < N) x[4 * c + 3] = q.w;
  }
}
// whether rows of length L starting at p are 16-byte aligned (then every kFirS-step segment is)
TSF_DEV bool fir_vec(const float* p, int64_t L) { return (L & 3) == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// the kFirS steps t .. t + 3 of one row (one 16-byte store when the rows are aligned)
TSF_DEV void fir_store(float* __restrict__ row, int64_t t, int64_t L, bool vec, const float (&v)[kFirS]) {
  if (vec && t + kFirS <= L) {
    *reinterpret_cast<float4*>(row + t) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int i = 0; i < kFirS; ++i)
      if (t + i < L) row[t + i] = v[i];
  }
}

template <int NBT>
__global__ void __launch_bounds__(kFirW) gb_fir_fwd(const float* __restrict__ u, const float* __restrict__ bcoef,
                                                    const float* __restrict__ u_tail, float* __restrict__ w,
                                                    int64_t L, int I, int O, int nb, unsigned tiles_t) {
  __shared__ __align__(16) float s_u[kFirT + NBT];
  __shared__ __align__(16) float s_b[kFirOB][NBT];
  const FirTile f = fir_tile(tiles_t, (unsigned)I);
  fir_stage_u<NBT>(s_u, u, u_tail, f, L, I, nb);
  __syncthreads();
  constexpr int NW = NBT + kFirS - 1;
  float uw[NW];  // uw[m] = u_ext[t - (NBT - 1) + m]
  fir_window<NW>(uw, s_u);
  const int64_t t = f.t0 + kFirS * threadIdx.x;
  const int64_t P = (int64_t)I * O;
  const bool vec = fir_vec(w, L);
  for (int o0 = 0; o0 < O; o0 += kFirOB) {
    __syncthreads();  // the previous block's taps are read
    fir_stage_b<NBT>(s_b, bcoef, o0, O, I, f.j, nb);
    __syncthreads();
    const int ob = (O - o0) < kFirOB ? (O - o0) : kFirOB;
    for (int r = 0; r < ob; ++r) {
      float acc[kFirS] = {};
#pragma unroll
      for (int k0 = 0; k0 < NBT; k0 += 4) {
        const float4 bq = *reinterpret_cast<const float4*>(&s_b[r][k0]);
        const float bk[4] = {bq.x, bq.y, bq.z, bq.w};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int i = 0; i < kFirS; ++i) acc[i] = fmaf(bk[kk], uw[i + NBT - 1 - (k0 + kk)], acc[i]);
      }
      fir_store(w + (f.b * P + (int64_t)f.j * O + o0 + r) * L, t, L, vec, acc);
    }
  }
}

// The sum over a wave's 64 lanes, left in lane 63 (DPP: within quads, across the 16-lane rows by
// rotation, then row to row by broadcast).
TSF_DEV float wave_sum_last(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // lane ^ 1
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // lane ^ 2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row rotate 4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row rotate 8
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));  // row bcast 15
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));  // row bcast 31
  return v;
}

// FIR adjoint, one workgroup per (batch row, input channel, kFirT steps) as the forward:
//   gu[b, t, j]      = sum_o sum_k b[o, j, k] gw[b, j*O + o, t + k]      (gw zero from L on)
//   gu_tail[b, m, j] = the same sum at t = m - (nb - 1) < 0
//   part[., o, k]    = sum over the tile's steps of gw[b, j*O + o, t] u_ext[b, t - k, j]
// A block of kFirOB rows of gw (with the NBT - 1 step halo on the right) goes through LDS; each
// thread forms its kFirS steps of gu and its share of every (o, k) partial from register windows,
// the partials are summed over each wave (DPP) and then over the waves in a fixed order into fp64
// part [B * tiles][I][O][nb], which gb_fir_reduce sums over batch rows and tiles.
template <int NBT>
__global__ void __launch_bounds__(kFirW) gb_fir_bwd(const float* __restrict__ gw, const float* __restrict__ u,
                                                    const float* __restrict__ bcoef, const float* __restrict__ u_tail,
                                                    float* __restrict__ gu, float* __restrict__ gu_tail,
                                                    double* __restrict__ part, int64_t L, int I, int O, int nb,
                                                    unsigned tiles_t) {
  constexpr int NS = kFirT + NBT;  // staged steps per row (the halo, rounded up)
  __shared__ __align__(16) float s_u[NS];
  __shared__ __align__(16) float s_g[kFirOB][NS];
  __shared__ __align__(16) float s_b[kFirOB][NBT];
  __shared__ float s_red[kFirW / 64][kFirOB][NBT];
  const FirTile f = fir_tile(tiles_t, (unsigned)I);
  const int tid = threadIdx.x, wave = tid >> 6;
  fir_stage_u<NBT>(s_u, u, u_tail, f, L, I, nb);
  const int64_t P = (int64_t)I * O;
  const int64_t t = f.t0 + kFirS * tid;
  const bool tail = f.t0 == 0 && gu_tail && nb > 1 && tid < nb - 1;
  const bool vec = fir_vec(gw, L);
  float gacc[kFirS] = {};
  float acc_tail = 0.0f;
  constexpr int NW = NBT + kFirS - 1;
  float uw[NW];  // uw[m] = u_ext[t - (NBT - 1) + m]
  double* pw = part + (((f.b * tiles_t + f.t0 / kFirT) * I + f.j) * O) * nb;
  for (int o0 = 0; o0 < O; o0 += kFirOB) {
    const int ob = (O - o0) < kFirOB ? (O - o0) : kFirOB;
    __syncthreads();  // the previous block's rows, taps and wave sums are read
    // the block's gw rows: every load issued before the first LDS store
    if (vec) {
      constexpr int NQ = (NS / 4 + kFirW - 1) / kFirW;  // 16-byte pieces per thread and row
      float4 x[kFirOB][NQ];
#pragma unroll
      for (int r = 0; r < kFirOB; ++r) {
        const float* grow = gw + (f.b * P + (int64_t)f.j * O + o0 + r) * L;
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
          const int q = tid + c * kFirW;
          const int64_t tq = f.t0 + 4 * q;
          x[r][c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          if (r < ob && q < NS / 4 && tq < L) x[r][c] = *reinterpret_cast<const float4*>(grow + tq);  // L % 4 == 0
        }
      }
#pragma unroll
      for (int r = 0; r < kFirOB; ++r)
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
          const int q = tid + c * kFirW;
          if (q < NS / 4) reinterpret_cast<float4*>(&s_g[r][0])[q] = x[r][c];
        }
    } else {
      constexpr int NE = (NS + kFirW - 1) / kFirW;
      float x[kFirOB][NE];
#pragma unroll
      for (int r = 0; r < kFirOB; ++r) {
        const float* grow = gw + (f.b * P + (int64_t)f.j * O + o0 + r) * L;
#pragma unroll
        for (int c = 0; c < NE; ++c) {
          const int i = tid + c * kFirW;
          x[r][c] = (r < ob && i < NS && f.t0 + i < L) ? grow[f.t0 + i] : 0.0f;
        }
      }
#pragma unroll
      for (int r = 0; r < kFirOB; ++r)
#pragma unroll
        for (int c = 0; c < NE; ++c) {
          const int i = tid + c * kFirW;
          if (i < NS) s_g[r][i] = x[r][c];
        }
    }
    fir_stage_b<NBT>(s_b, bcoef, o0, O, I, f.j, nb);
    __syncthreads();
    if (o0 == 0) fir_window<NW>(uw, s_u);
    for (int r = 0; r < ob; ++r) {
      float gv[NW];  // gv[m] = gw[t + m]
      fir_window<NW>(gv, &s_g[r][0]);
      float p[NBT];
#pragma unroll
      for (int k0 = 0; k0 < NBT; k0 += 4) {
        const float4 bq = *reinterpret_cast<const float4*>(&s_b[r][k0]);
        const float bk[4] = {bq.x, bq.y, bq.z, bq.w};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int k = k0 + kk;
          float pk = 0.0f;
#pragma unroll
          for (int i = 0; i < kFirS; ++i) {
            gacc[i] = fmaf(bk[kk], gv[i + k], gacc[i]);
            pk = fmaf(gv[i], uw[i + NBT - 1 - k], pk);
          }
          p[k] = pk;
        }
      }
#pragma unroll
      for (int k = 0; k < NBT; ++k) {
        const float v = wave_sum_last(p[k]);
        if ((tid & 63) == 63) s_red[wave][r][k] = v;
      }
      if (tail) {
        // gu_tail[m] with m = tid: t = m - (nb - 1), so gw index t + k >= 0 means k >= nb - 1 - m
        for (int k = nb - 1 - tid; k < nb; ++k) acc_tail = fmaf(s_b[r][k], s_g[r][tid - (nb - 1) + k], acc_tail);
      }
    }
    __syncthreads();
    for (int e = tid; e < ob * nb; e += kFirW) {
      const int r = e / nb, k = e - r * nb;
      double d = 0.0;
#pragma unroll
      for (int wv = 0; wv < kFirW / 64; ++wv) d += (double)s_red[wv][r][k];
      pw[(o0 + r) * nb + k] = d;
    }
  }
#pragma unroll
  for (int i = 0; i < kFirS; ++i)
    if (t + i < L) gu[(f.b * L + t + i) * I + f.j] = gacc[i];
  if (tail) gu_tail[(f.b * (nb - 1) + tid) * I + f.j] = acc_tail;
}

// grad b [O, I, nb]: per entry, the sum of the partials over batch rows and tiles in a fixed
// order (a workgroup per entry: strided partial sums, then a tree in LDS).
__global__ void __launch_bounds__(256) gb_fir_reduce(const double* __restrict__ part, float* __restrict__ gb,
                                                     int64_t rows, int I, int O, int nb) {
  __shared__ double s_r[256];
  const int64_t e = blockIdx.x;  // (o, j, k) with the [O, I, nb] layout of b
  const int k = (int)(e % nb), j = (int)((e / nb) % I), o = (int)(e / ((int64_t)nb * I));
  double acc = 0.0;
  for (int64_t r = threadIdx.x; r < rows; r += 256) acc += part[((r * I + j) * O + o) * nb + k];
  s_r[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) s_r[threadIdx.x] += s_r[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) gb[e] = (float)s_r[0];
}

int fir_args_status(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb) {
  if (B < 0 || L < 0 || I < 1 || O < 1 || nb < 1) return TSF_ERR_ARG;
  if (nb > kFirMaxNB) return TSF_ERR_UNSUPPORTED;
  const int64_t tiles = B * I * ((L + kFirT - 1) / kFirT);
  if (tiles > INT32_MAX || I * O > INT32_MAX / 2) return TSF_ERR_UNSUPPORTED;
  return TSF_OK;
}

#define TSF_FIR_NBT(X) X(4) X(8) X(16) X(32) X(64)

#define TSF_GB_CASES(X) \
  X(1, 2) X(1, 4) X(1, 8) X(1, 16) X(2, 2) X(2, 4) X(2, 8) X(2, 16) X(3, 2) X(3, 4) X(3, 8) X(3, 16) X(4, 2) X(4, 4) X(4, 8) X(4, 16)

}  // namespace

extern "C" {

int64_t tsfast_hip_gblock_workspace_bytes(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na) {
  if (gb_args_status(B, L, I, O, nb, na) != TSF_OK) return -1;
  return (int64_t)gb_plan(B, L, I, O, nb, na).bytes;
}

int64_t tsfast_hip_gblock_saved_doubles(int64_t B, int64_t L, int64_t I, int64_t O, int64_t na) {
  if (gb_args_status(B, L, I, O, 1, na) != TSF_OK) return -1;
  const GbPlan p = gb_plan(B, L, I, O, 1, na);
  return p.lb.nsuper * p.lanes * na;
}

int tsfast_hip_gblock_fwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na, const float* u,
                          const float* b, const float* a, const float* u_tail, const float* x0, float* y,
                          float* x_last, double* saved, void* workspace, int64_t workspace_bytes, void* stream) {
  const int st = gb_args_status(B, L, I, O, nb, na);
  if (st != TSF_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0) return TSF_OK;
  if (L == 0) {
    if (x_last) hipLaunchKernelGGL(gblock_copy_state, grid_for(B * I * O * na), dim3(256), 0, s, x0, x_last, B * I * O * na);
    return tsf_launch_status();
  }
  if (!u || !b || !a || !y) return TSF_ERR_ARG;
  if (!workspace || workspace_bytes < tsfast_hip_gblock_workspace_bytes(B, L, I, O, nb, na)) return TSF_ERR_WORKSPACE;
  const GbPlan p = gb_plan(B, L, I, O, nb, na);
  char* ws = static_cast<char*>(workspace);
  switch (na * 100 + p.nbt) {
#define X(NA_, NB_)                                                                                                  \
  case NA_ * 100 + NB_:                                                                                              \
    fwd_impl<NA_, NB_>(p, B, L, (int)I, (int)O, (int)nb, u, b, a, u_tail, x0, y, x_last, saved, ws, s); \
    break;
    TSF_GB_CASES(X)
#undef X
    default:
      return TSF_ERR_UNSUPPORTED;
  }
  return tsf_launch_status();
}

int tsfast_hip_gblock_bwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na, const float* gy,
                          const float* g_xlast, const float* u, const float* b, const float* a, const float* u_tail,
                          const float* x0, const double* saved, float* gu, float* gu_tail, float* gb, float* ga,
                          float* gx0, void* workspace, int64_t workspace_bytes, void* stream) {
  const int st = gb_args_status(B, L, I, O, nb, na);
  if (st != TSF_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!b || !a || !gb || !ga) return TSF_ERR_ARG;
  if (L > 0 && (!gy || !u || !gu)) return TSF_ERR_ARG;
  if (L > 0 && !saved && gb_plan(B, L, I, O, nb, na).lb.nsuper > 1) return TSF_ERR_ARG;
  if (!workspace || workspace_bytes < tsfast_hip_gblock_workspace_bytes(B, L, I, O, nb, na)) return TSF_ERR_WORKSPACE;
  const GbPlan p = gb_plan(B, L, I, O, nb, na);
  char* ws = static_cast<char*>(workspace);
  switch (na * 100 + p.nbt) {
#define X(NA_, NB_)                                                                                                  \
  case NA_ * 100 + NB_:                                                                                              \
    bwd_impl<NA_, NB_>(p, B, L, (int)I, (int)O, (int)nb, gy, g_xlast, u, b, a, u_tail, x0, saved, gu, gu_tail, gb, ga, \
                       gx0, ws, s);                                                                                  \
    break;
    TSF_GB_CASES(X)
#undef X
    default:
      return TSF_ERR_UNSUPPORTED;
  }
  return tsf_launch_status();
}

int64_t tsfast_hip_gblock_fir_workspace_bytes(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb) {
  if (fir_args_status(B, L, I, O, nb) != TSF_OK) return -1;
  return 8 * B * ((L + kFirT - 1) / kFirT) * I * O * nb;
}

int tsfast_hip_gblock_fir_fwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, const float* u, const float* b,
                              const float* u_tail, float* w, void* stream) {
  const int st = fir_args_status(B, L, I, O, nb);
  if (st != TSF_OK) return st;
  if (B == 0 || L == 0) return TSF_OK;
  if (!u || !b || !w) return TSF_ERR_ARG;
  const int64_t tiles_t = (L + kFirT - 1) / kFirT;
  const dim3 grid((unsigned)(B * I * tiles_t));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (fir_nbt(nb)) {
#define X(NBT_)                                                                                                    \
  case NBT_:                                                                                                       \
    hipLaunchKernelGGL((gb_fir_fwd<NBT_>), grid, dim3(kFirW), 0, s, u, b, u_tail, w, L, (int)I, (int)O, (int)nb, \
                       (unsigned)tiles_t);                                                                         \
    break;
    TSF_FIR_NBT(X)
#undef X
  }
  return tsf_launch_status();
}

int tsfast_hip_gblock_fir_bwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, const float* gw,
                              const float* u, const float* b, const float* u_tail, float* gu, float* gu_tail,
                              float* gb, void* workspace, int64_t workspace_bytes, void* stream) {
  const int st = fir_args_status(B, L, I, O, nb);
  if (st != TSF_OK) return st;
  if (!b || !gb || (L > 0 && B > 0 && (!gw || !u || !gu))) return TSF_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tiles_t = (L + kFirT - 1) / kFirT, rows = B * tiles_t;
  if (rows == 0) {  // no steps: grad b and the tail gradient are zero
    hipLaunchKernelGGL(gblock_zero, grid_for(O * I * nb), dim3(256), 0, s, gb, O * I * nb);
    if (gu_tail && nb > 1 && B > 0)
      hipLaunchKernelGGL(gblock_zero, grid_for(B * (nb - 1) * I), dim3(256), 0, s, gu_tail, B * (nb - 1) * I);
    return tsf_launch_status();
  }
  if (!workspace || workspace_bytes < tsfast_hip_gblock_fir_workspace_bytes(B, L, I, O, nb)) return TSF_ERR_WORKSPACE;
  double* part = static_cast<double*>(workspace);
  const dim3 grid((unsigned)(B * I * tiles_t));
  switch (fir_nbt(nb)) {
#define X(NBT_)                                                                                                 \
  case NBT_:                                                                                                    \
    hipLaunchKernelGGL((gb_fir_bwd<NBT_>), grid, dim3(kFirW), 0, s, gw, u, b, u_tail, gu, gu_tail, part, L,     \
                       (int)I, (int)O, (int)nb, (unsigned)tiles_t);                                             \
    break;
    TSF_FIR_NBT(X)
#undef X
  }
  hipLaunchKernelGGL(gb_fir_reduce, dim3((unsigned)(O * I * nb)), dim3(256), 0, s, (const double*)part, gb, rows,
                     (int)I, (int)O, (int)nb);
  return tsf_launch_status();
}

}  // extern "C"
