// Projected complex diagonal scan: the core of tsfast's LRU and S5 layers in one pass.
//   v_t = W u_t                  W = W_re + i W_im  [N, H], u real [B, L, H]
//   x_t = lam * x_{t-1} + v_t    lam [N] complex, shared by every row; x_{-1} = x0 (or 0)
//   y_t = Re(C x_t)              C = C_re + i C_im  [O, N], y real [B, L, O]
// Reference: the composition complex_in_proj -> diagonal_recurrence -> real_out_proj
// (tsfast/models/_core/scan.py:221-243, 272-313) that LRU.forward (architectures/lru.py:100-110)
// and S5.forward (architectures/s5.py:180-198) run. The reference materialises v and x
// ([B, L, N] complex each); this pass reads u and writes y, and neither v nor x touches HBM.
//
// Work layout. A tile is one row b by a chunk of kChunk = 32 steps (2 blocks of 16) by all N
// states; a workgroup has one wave per 32 states (N <= 256: at most 8 waves, two per SIMD, so
// each wave has 256 registers) and takes tiles in scan order (chunk-major) from a counter. Both
// projections run on the fp32 matrix cores (v_mfma_f32_16x16x4f32) with time as the row index of
// a 16 x 16 block:
//   in-proj   V[t][s] = sum_h u[t][h] W[s][h]     A = the u block, B = W^T held in registers;
//   read-out  Y[t][o] = sum_rho X[t][rho] Ct[rho][o] over the wave's 64 interleaved real state
//             rows rho (re, im; the im rows carry -C_im), A = the X block re-read through LDS in
//             operand layout, B = Ct held in registers; the waves' partial Y are added in LDS.
// An MFMA result holds steps 4g .. 4g+3 of column j in lane (g, j) (g = lane / 16, j = lane % 16),
// so the recurrence runs serially over a lane's 4 steps, then across the 4 lane groups (two
// shift-and-combine stages through ds_bpermute), then from block to block.
// Chunks are chained by decoupled look-back (lookback.h): every chunk publishes its end state from
// a zero start (agg) and the state leaving it (inc), and a tile walks back over the aggs to the
// nearest published inc. In deterministic mode (tsfast_hip_set_deterministic) only every eighth
// chunk of a row in scan order publishes an inc (anchored publication), so the state entering
// each chunk is composed the same way on every run. Carries are fp64; the chunk-entering states
// are saved for the backward pass.
#include <algorithm>

#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

#include "lookback.h"

using f4 = __attribute__((__vector_size__(4 * sizeof(float)))) float;

constexpr int kBlk = 16;                  // steps per MFMA block
constexpr int kBlocks = 2;                // blocks per chunk
constexpr int kChunk = kBlk * kBlocks;    // steps per forward tile
constexpr int kBwdBlocks = 2;             // blocks per backward tile
constexpr int kSub = kBlk * kBwdBlocks;   // steps per backward tile (the saved-state interval)
static_assert(kChunk % kSub == 0, "forward tiles cover whole saved-state intervals");
constexpr int kSlots = 2;                 // 16-state column blocks per wave
constexpr int kWaveStates = 16 * kSlots;  // states per wave
constexpr int kRho = 2 * kWaveStates;     // interleaved real rows (re, im) of a wave's states
constexpr int kMaxWaves = 8;              // N <= 256
constexpr int kXtStride = kRho + 4;       // floats per row of a wave's transposed block in LDS
constexpr uint32_t kOob = 0xFFFFFFF0u;    // buffer offset past every resource: loads return 0
constexpr int kProjAnchorSpacing = 2;     // deterministic-mode anchor spacing (measured: 1-2 cost nothing, 8 cost 10%)

TSF_DEV f4 mfma(float a, float b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
TSF_DEV f4 f4_zero() { return f4{0.0f, 0.0f, 0.0f, 0.0f}; }

TSF_DEV float2 from_lane(float2 v, int src) {
  return make_float2(__int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v.x))),
                     __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v.y))));
}
// the value of lane - 16 d (the same column, d lane groups lower); zero in the first d groups
TSF_DEV float2 from_group_below(float2 v, int lane, int d) {
  const float2 r = from_lane(v, lane - 16 * d);
  return lane >= 16 * d ? r : make_float2(0.0f, 0.0f);
}
template <int K>
TSF_DEV float2 pick(const float2 (&v)[K], int i) {
  float2 r = v[0];
#pragma unroll
  for (int k = 1; k < K; ++k) r = i == k ? v[k] : r;
  return r;
}
TSF_DEV double2 up2(float2 v) { return make_double2((double)v.x, (double)v.y); }
TSF_DEV float2 down2(double2 v) { return make_float2((float)v.x, (float)v.y); }

// In-block scan of one 16-state column block from a zero state at the block start: x[r] holds
// v at step 4g + r of column j on entry, the states on return. lm = lam, lm4 = lam^4, lm8 = lam^8.
TSF_DEV void block_scan(float2 (&x)[4], float2 lm, float2 lm4, float2 lm8, int lane) {
  x[1] = cfma(lm, x[0], x[1]);
  x[2] = cfma(lm, x[1], x[2]);
  x[3] = cfma(lm, x[2], x[3]);
  // inclusive scan of the group ends over the 4 lane groups: E_g = sum_{g' <= g} lam^(4(g-g')) e_g'
  float2 e = x[3];
  e = cfma(lm4, from_group_below(e, lane, 1), e);
  e = cfma(lm8, from_group_below(e, lane, 2), e);
  // the state after group g-1 enters group g
  float2 p = cmul(lm, from_group_below(e, lane, 1));
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    x[r] = cadd(x[r], p);
    p = cmul(lm, p);
  }
}

// Carry of chunk c for this lane's state, looked up over the chunks before it in scan order
// (c - 1, c - 2, ... for dir = -1; c + 1, c + 2, ... for dir = +1; nc chunks), W at a time. A
// published inc (the carry leaving that chunk) ends the walk; a published agg (that chunk's carry
// from a zero start; every such chunk has the multiplier P) is composed and the walk moves on; an
// unpublished word ends the round. The walk ends: the first chunk in scan order publishes its inc
// without waiting, and every chunk waited on belongs to a tile taken earlier by a running
// workgroup; a lane that makes no progress for spin_max rounds gives up with NaN.
template <int W>
TSF_DEV double2 walk(const double2* __restrict__ agg, const double2* __restrict__ inc, int64_t cstride, int64_t widx,
                     int c, int dir, int nc, double2 P, unsigned* __restrict__ lb_counter, uint32_t spin_max) {
  double2 accP = Num<double2>::one(), acce = Num<double2>::zero();
  int r = c + dir;
  uint32_t spins = 0;
  for (;;) {
    double2 vi[W], va[W];
    bool hi[W], ha[W];
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const int rr = r + dir * i;
      hi[i] = ha[i] = false;
      if (rr >= 0 && rr < nc) {
        hi[i] = get(inc + (int64_t)rr * cstride + widx, vi[i]);
        ha[i] = get(agg + (int64_t)rr * cstride + widx, va[i]);
      }
    }
    int i = 0;
    for (; i < W; ++i) {
      const int rr = r + dir * i;
      if (rr < 0 || rr >= nc) break;
      if (hi[i]) return Num<double2>::fma(accP, vi[i], acce);
      if (!ha[i]) break;
      acce = Num<double2>::fma(accP, va[i], acce);
      accP = Num<double2>::mul(accP, P);
    }
    if (i == 0 && ++spins > spin_max) {
      lb_gave_up(lb_counter);
      return quiet_nan<double2>();
    }
    r += dir * i;
  }
}

// Dynamic LDS of the forward: per wave a transposed X block [kBlk][kXtStride], then the waves'
// partial Y blocks, double-buffered [2][NW][kBlk][16 OB].
template <int OB>
constexpr size_t fwd_lds_bytes(int nw) {
  return sizeof(float) * ((size_t)nw * kBlk * kXtStride + 2 * (size_t)nw * kBlk * 16 * OB);
}

template <int KS, int OB>
__global__ void __launch_bounds__(64 * kMaxWaves) __attribute__((amdgpu_waves_per_eu(2)))
    projscan_fwd(const float* __restrict__ u, const float* __restrict__ w_re, const float* __restrict__ w_im,
                 const float2* __restrict__ lam, const float* __restrict__ c_re, const float* __restrict__ c_im,
                 const float2* __restrict__ x0, float* __restrict__ y, float2* __restrict__ x_last,
                 float2* __restrict__ saved, double2* __restrict__ agg, double2* __restrict__ inc,
                 unsigned* __restrict__ counter, int B, int L, int H, int N, int O, int nchunks, int nsub, LbCfg lb_spacing) {
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  __shared__ unsigned s_tile[2];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, NW = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  float* const s_xt = s_dyn + (size_t)w * kBlk * kXtStride;  // this wave's [kBlk][kXtStride]
  float* const s_y = s_dyn + (size_t)NW * kBlk * kXtStride;  // [2][NW][kBlk][16 OB]
  const int64_t NS = (int64_t)NW * kWaveStates, cstride = (int64_t)B * NS, tiles = (int64_t)nchunks * B;
  const Rsrc ru = make_rsrc(u, (uint32_t)((int64_t)B * L * H * 4));

  // in-proj B operands: W_p[s][h] for s = 64w + 16q + j, h = g KS + kk (p = 0 re, 1 im)
  float wB[kSlots][2][KS];
#pragma unroll
  for (int q = 0; q < kSlots; ++q) {
    const int s = kWaveStates * w + 16 * q + j;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int h = g * KS + kk;
      const bool ok = s < N && h < H;
      wB[q][0][kk] = ok ? w_re[(int64_t)s * H + h] : 0.0f;
      wB[q][1][kk] = ok ? w_im[(int64_t)s * H + h] : 0.0f;
    }
  }
  // read-out B operands: row rho = (kRho / 4) g + m is state kWaveStates w + rho/2, re (C_re) for
  // even rho, im (-C_im) for odd
  constexpr int kM = kRho / 4;  // MFMAs per 16-output block
  float cB[OB][kM];
#pragma unroll
  for (int ob = 0; ob < OB; ++ob) {
    const int o = 16 * ob + j;
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      const int rho = kM * g + m, s = kWaveStates * w + (rho >> 1);
      const bool ok = o < O && s < N;
      cB[ob][m] = !ok ? 0.0f : (rho & 1) ? -c_im[(int64_t)o * N + s] : c_re[(int64_t)o * N + s];
    }
  }
  // scan constants of the lane's slots (state 64w + 16q + j): lam, lam^4, lam^8, lam^(4g+1), lam^16
  float2 lm[kSlots], lm4[kSlots], lm8[kSlots], lmg[kSlots], lm16[kSlots];
#pragma unroll
  for (int q = 0; q < kSlots; ++q) {
    const int s = kWaveStates * w + 16 * q + j;
    const float2 a = s < N ? lam[s] : make_float2(0.0f, 0.0f);
    lm[q] = a;
    lm4[q] = ipow(a, 4);
    lm8[q] = ipow(a, 8);
    lmg[q] = ipow(a, 4 * g + 1);
    lm16[q] = ipow(a, 16);
  }
  // the lane's look-back state kWaveStates w + lane (slot g of column j); lanes past the wave's
  // states take no part in the look-back
  const bool lb_lane = lane < kWaveStates;
  const int s_lb = kWaveStates * w + lane;
  const double2 a_lb = lb_lane && s_lb < N ? up2(lam[s_lb]) : Num<double2>::zero();
  const double2 P16 = ipow(a_lb, 16), Pc = ipow(a_lb, kChunk);

  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    if (threadIdx.x == 0) s_tile[buf ^ 1] = take_tile(counter);
    const int c = (int)(tile / B), b = (int)(tile - (int64_t)c * B);
    const int t0 = c * kChunk;

    // phase A: both projections' first half -- V by MFMA, the block scans from zero
    float2 x[kBlocks][kSlots][4];
    float2 e[kBlocks][kSlots];  // block end states from a zero block start, every lane of the column
#pragma unroll
    for (int k = 0; k < kBlocks; ++k) {
      const int t = t0 + kBlk * k + j;
      float ua[KS];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int h = g * KS + kk;
        const uint32_t off = (t < L && h < H) ? (uint32_t)((((int64_t)b * L + t) * H + h) * 4) : kOob;
        ua[kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ru, off, 0, 0));
      }
      f4 acc[kSlots][2];
#pragma unroll
      for (int q = 0; q < kSlots; ++q) acc[q][0] = acc[q][1] = f4_zero();
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
#pragma unroll
        for (int q = 0; q < kSlots; ++q) {
          acc[q][0] = mfma(ua[kk], wB[q][0][kk], acc[q][0]);
          acc[q][1] = mfma(ua[kk], wB[q][1][kk], acc[q][1]);
        }
#pragma unroll
      for (int q = 0; q < kSlots; ++q) {
#pragma unroll
        for (int r = 0; r < 4; ++r) x[k][q][r] = make_float2(acc[q][0][r], acc[q][1][r]);
        block_scan(x[k][q], lm[q], lm4[q], lm8[q], lane);
        e[k][q] = from_lane(x[k][q][3], 48 + j);
      }
    }

    // look-back on lane (g, j) for state kWaveStates w + lane (slot g)
    double2 agg_v = Num<double2>::zero();
#pragma unroll
    for (int k = 0; k < kBlocks; ++k) agg_v = Num<double2>::fma(P16, agg_v, up2(pick(e[k], g)));
    const int64_t widx = (int64_t)b * NS + s_lb;
    double2 cin = Num<double2>::zero();
    if (lb_lane) {
      if (c == 0) {
        if (x0 != nullptr && s_lb < N) cin = up2(x0[(int64_t)b * N + s_lb]);
      } else {
        if (lb_pub_agg(c, lb_spacing) && c + 1 < nchunks) put(agg + (int64_t)c * cstride + widx, agg_v);
        cin = walk<2>(agg, inc, cstride, widx, c, -1, nchunks, Pc, counter, lb_spacing.spin_max);
      }
      if (lb_pub_inc(c, lb_spacing) && c + 1 < nchunks)
        put(inc + (int64_t)c * cstride + widx, Num<double2>::fma(Pc, cin, agg_v));
    }
    float2 carry[kSlots];
    {
      const float2 cf = down2(cin);
#pragma unroll
      for (int q = 0; q < kSlots; ++q) carry[q] = from_lane(cf, 16 * q + j);
    }

    // phase B: fix up each block with its entering state, read out through the matrix cores
#pragma unroll
    for (int k = 0; k < kBlocks; ++k) {
      // the state entering every half chunk is saved for the backward pass (its tiles are 32 steps)
      const int tk = t0 + kBlk * k, sub = tk / kSub;
      if (saved != nullptr && tk % kSub == 0 && sub < nsub && lb_lane && s_lb < N)
        saved[((int64_t)b * nsub + sub) * N + s_lb] = pick(carry, g);
#pragma unroll
      for (int q = 0; q < kSlots; ++q) {
        float2 p = cmul(lmg[q], carry[q]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[k][q][r] = cadd(x[k][q][r], p);
          p = cmul(lm[q], p);
        }
        carry[q] = cfma(lm16[q], carry[q], e[k][q]);
      }
      const int tl = L - 1 - t0 - kBlk * k;  // block-relative step of the sequence's last step
      if (x_last != nullptr && tl >= 0 && tl < kBlk && g == (tl >> 2)) {
#pragma unroll
        for (int q = 0; q < kSlots; ++q) {
          const int s = kWaveStates * w + 16 * q + j;
          if (s < N) x_last[(int64_t)b * N + s] = pick(x[k][q], tl & 3);
        }
      }
      // transpose through LDS: row t, column 2 s_local + p
#pragma unroll
      for (int q = 0; q < kSlots; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<float2*>(&s_xt[(4 * g + r) * kXtStride + 2 * (16 * q + j)]) = x[k][q][r];
      float xa[kM];
#pragma unroll
      for (int v = 0; v < kM / 4; ++v) {
        const f4 q4 = *reinterpret_cast<const f4*>(&s_xt[j * kXtStride + kM * g + 4 * v]);
        xa[4 * v] = q4[0];
        xa[4 * v + 1] = q4[1];
        xa[4 * v + 2] = q4[2];
        xa[4 * v + 3] = q4[3];
      }
      f4 yacc[OB];
#pragma unroll
      for (int ob = 0; ob < OB; ++ob) yacc[ob] = f4_zero();
#pragma unroll
      for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int ob = 0; ob < OB; ++ob) yacc[ob] = mfma(xa[m], cB[ob][m], yacc[ob]);
      constexpr int kYw = kBlk * 16 * OB;  // floats of one wave's Y block
      float* const sy = s_y + (size_t)(k & 1) * NW * kYw;
#pragma unroll
      for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < 4; ++r) sy[w * kYw + (4 * g + r) * 16 * OB + 16 * ob + j] = yacc[ob][r];
      __syncthreads();
      for (int idx = threadIdx.x; idx < kBlk * O; idx += blockDim.x) {
        const int tt = idx / O, o = idx - tt * O;
        float sum = sy[tt * 16 * OB + o];
        for (int ww = 1; ww < NW; ++ww) sum += sy[ww * kYw + tt * 16 * OB + o];
        const int t = t0 + kBlk * k + tt;
        if (t < L) y[((int64_t)b * L + t) * O + o] = sum;
      }
    }
  }
}

__global__ void __launch_bounds__(256) projscan_copy_state(const float2* __restrict__ x0, float2* __restrict__ x_last,
                                                           int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) x_last[i] = x0 != nullptr ? x0[i] : make_float2(0.0f, 0.0f);
}

// ---------------------------------------------------------------- backward
// Adjoint, with the upstream gradients gy [B, L, O] and g_xlast [B, N] (of the returned state):
//   g_x_t = gy_t conj(C) (+ g_xlast at the last step),  G_t = g_x_t + conj(lam) G_{t+1},
//   g_u_t = Re(G_t conj(W)),  grad W_re/W_im = sum_t Re/Im(G_t) u_t^T,
//   grad C_re = sum_t gy_t Re(x_t)^T,  grad C_im = -sum_t gy_t Im(x_t)^T,
//   grad lam = sum_{b,t} G_t conj(x_{t-1}),  g_x0 = conj(lam) G_0.
// A backward tile is one row by kSub = 32 steps (2 blocks) by all states, taken from the right
// end (one wave per 32 states, as in the forward). Phase A: g_x by MFMA (A = the gy block, B =
// conj(C)^T reloaded from L2 each tile), the reverse in-block scans from zero, the tile's
// aggregate, a look-back over the later chunks of the row, the fix-up of both G blocks. Phase B,
// block by block from the left: x recomputed (in-proj MFMA with B = W^T read from the wave's W
// rows in LDS at each use, and the scan from the saved state entering the tile), grad lam on the
// VALU, grad C (A = gy^T loaded in operand layout, B = x) and grad W (A = u^T, B = G) accumulated
// on the matrix cores over every tile the workgroup takes, and g_u (A = G transposed through LDS,
// B = W rows in LDS), whose per-wave partial sums are added in LDS. Each workgroup finally writes
// its grad W / C / lam sums to its slot of the partial buffer, which projscan_bwd_reduce adds in a
// fixed order.
constexpr int kWuStride = kRho + 4;      // floats per h row of a wave's W rows in LDS

// conj(a) * x and conj(a) * x + b
TSF_DEV float2 cmul_c(float2 a, float2 x) { return make_float2(fmaf(a.x, x.x, a.y * x.y), fmaf(a.x, x.y, -(a.y * x.x))); }
TSF_DEV float2 cfma_c(float2 a, float2 x, float2 b) {
  return make_float2(fmaf(a.x, x.x, fmaf(a.y, x.y, b.x)), fmaf(a.x, x.y, fmaf(-a.y, x.x, b.y)));
}
TSF_DEV double2 conj2(double2 a) { return make_double2(a.x, -a.y); }
// the value of lane + 16 d (the same column, d lane groups higher); zero in the last d groups
TSF_DEV float2 from_group_above(float2 v, int lane, int d) {
  const float2 r = from_lane(v, lane + 16 * d);
  return lane + 16 * d < 64 ? r : make_float2(0.0f, 0.0f);
}

// Reverse in-block scan G_t = x_t + conj(lam) G_{t+1} from zero after the block's last step.
TSF_DEV void block_scan_rev(float2 (&x)[4], float2 lm, float2 lm4, float2 lm8, int lane) {
  x[2] = cfma_c(lm, x[3], x[2]);
  x[1] = cfma_c(lm, x[2], x[1]);
  x[0] = cfma_c(lm, x[1], x[0]);
  // inclusive scan of the group starts from the right: E_g = sum_{g' >= g} conj(lam)^(4(g'-g)) e_g'
  float2 e = x[0];
  e = cfma_c(lm4, from_group_above(e, lane, 1), e);
  e = cfma_c(lm8, from_group_above(e, lane, 2), e);
  float2 p = cmul_c(lm, from_group_above(e, lane, 1));
#pragma unroll
  for (int r = 3; r >= 0; --r) {
    x[r] = cadd(x[r], p);
    p = cmul_c(lm, p);
  }
}

// The g_x product's B operands, read from the weights (L2-resident) when the phase starts, so that
// they hold registers only while it runs.
// g_x: conj(C)_p[o][s], o = g OKS + kk (p = 0: C_re, 1: -C_im).
// Read through buffer resources (o >= O falls past the end and reads 0) with 32-bit offsets from a
// per-lane base that passes through an empty asm, so that neither the values nor their addresses
// stay live across the tile loop.
template <int OKS>
TSF_DEV void load_c_operands(float (&cG)[kSlots][2][OKS], const Rsrc& rre, const Rsrc& rim, int w, int g, int j,
                             int N) {
  int base = g * OKS * N + kWaveStates * w + j;
  asm volatile("" : "+v"(base));
#pragma unroll
  for (int q = 0; q < kSlots; ++q) {
    const bool live = kWaveStates * w + 16 * q + j < N;
#pragma unroll
    for (int kk = 0; kk < OKS; ++kk) {
      const uint32_t off = live ? (uint32_t)(base + kk * N + 16 * q) * 4u : kOob;
      cG[q][0][kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rre, off, 0, 0));
      cG[q][1][kk] = -__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rim, off, 0, 0));
    }
  }
}

// Per-wave table of the powers of lam the backward's scans use, in LDS, read at each use rather
// than held in registers across the tile loop: lam, lam^4, lam^8, lam^16 per (slot, column) and
// lam^(4g+1), lam^(13-4g) per (slot, lane), float2 each.
constexpr int kPwFloats = 2 * (4 * kSlots * 16 + 2 * kSlots * 64);
// Dynamic LDS of the backward: per wave its W rows [16 HB][kWuStride] and a transposed G block
// [kBlk][kXtStride], then the waves' partial g_u blocks, double-buffered [2][NW][kBlk][16 HB],
// then the waves' power tables [NW][kPwFloats].
template <int HB>
constexpr size_t bwd_lds_bytes(int nw) {
  return sizeof(float) * ((size_t)nw * 16 * HB * kWuStride + (size_t)nw * kBlk * kXtStride +
                          2 * (size_t)nw * kBlk * 16 * HB + (size_t)nw * kPwFloats);
}
struct Pows {
  float2 lm, lm4, lm8, lm16, lmx;  // lmx = lam^(4g+1) (forward-time fix-up) or lam^(13-4g) (reverse)
};
// Table layout in float2: [4][kSlots][16] (lam, lam^4, lam^8, lam^16 per column j), then
// [2][kSlots][64] (lam^(4g+1), lam^(13-4g) per lane).
TSF_DEV int pow_col(int kind, int q, int j) { return (kind * kSlots + q) * 16 + j; }
TSF_DEV int pow_lane(int kind, int q, int lane) { return 4 * kSlots * 16 + (kind * kSlots + q) * 64 + lane; }
// The powers of slot q for this lane. `zero` is 0 passed through an empty asm at the call site, so
// the LDS reads stay where they are used instead of being hoisted out of the tile loop.
TSF_DEV Pows read_pows(const float2* t, int zero, int q, int j, int lane, bool reverse) {
  Pows p;
  p.lm = t[zero + pow_col(0, q, j)];
  p.lm4 = t[zero + pow_col(1, q, j)];
  p.lm8 = t[zero + pow_col(2, q, j)];
  p.lm16 = t[zero + pow_col(3, q, j)];
  p.lmx = t[zero + pow_lane(reverse ? 1 : 0, q, lane)];
  return p;
}
TSF_DEV int opaque_zero() {
  int z = 0;
  asm volatile("" : "+v"(z));
  return z;
}

template <int KS>
constexpr int hb_for_ks() { return KS == 8 ? 2 : 1; }

template <int KS, int OB>
__global__ void __launch_bounds__(64 * kMaxWaves) __attribute__((amdgpu_waves_per_eu(2)))
    projscan_bwd(const float* __restrict__ gy, const float2* __restrict__ g_xlast, const float2* __restrict__ saved,
                 const float* __restrict__ u, const float* __restrict__ w_re, const float* __restrict__ w_im,
                 const float2* __restrict__ lam, const float* __restrict__ c_re, const float* __restrict__ c_im,
                 float* __restrict__ g_u, float2* __restrict__ g_x0, float* __restrict__ part, int64_t part_stride,
                 double2* __restrict__ agg, double2* __restrict__ inc, unsigned* __restrict__ counter, int B, int L,
                 int H, int N, int O, int nsub, LbCfg lb_spacing) {
  constexpr int HB = hb_for_ks<KS>();  // 16-wide h blocks of g_u and grad W (H <= 16 HB)
  constexpr int OKS = 4 * OB;          // o per lane group in the g_x product (O <= 16 OB)
  constexpr int kM = kRho / 4;         // MFMAs per 16-wide h block of g_u
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  __shared__ unsigned s_tile[2];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, NW = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  float* const s_wu = s_dyn + (size_t)w * 16 * HB * kWuStride;  // this wave's [16 HB][kWuStride]
  float* const s_xt = s_dyn + (size_t)NW * 16 * HB * kWuStride + (size_t)w * kBlk * kXtStride;
  float* const s_gu = s_dyn + (size_t)NW * (16 * HB * kWuStride + kBlk * kXtStride);  // [2][NW][kBlk][16 HB]
  float2* const s_pw = reinterpret_cast<float2*>(s_gu + (size_t)2 * NW * kBlk * 16 * HB) + (size_t)w * kPwFloats / 2;
  const int64_t NS = (int64_t)NW * kWaveStates, cstride = (int64_t)B * NS, tiles = (int64_t)nsub * B;
  const Rsrc ru = make_rsrc(u, (uint32_t)((int64_t)B * L * H * 4));
  const Rsrc rg = make_rsrc(gy, (uint32_t)((int64_t)B * L * O * 4));
  const Rsrc rcre = make_rsrc(c_re, (uint32_t)(O * N * 4)), rcim = make_rsrc(c_im, (uint32_t)(O * N * 4));

  // the wave's W rows in LDS, zero outside [N, H]: s_wu[h][rho] = W_p[kWaveStates w + rho/2][h],
  // p = rho & 1 (the B operands of both the in-proj recompute and g_u)
  for (int idx = lane; idx < 16 * HB * kRho; idx += 64) {
    const int h = idx / kRho, rho = idx - h * kRho, s = kWaveStates * w + (rho >> 1);
    const bool ok = s < N && h < H;
    s_wu[h * kWuStride + rho] = !ok ? 0.0f : (rho & 1) ? w_im[(int64_t)s * H + h] : w_re[(int64_t)s * H + h];
  }
  // the wave's power table (read back by read_pows at each use)
#pragma unroll
  for (int q = 0; q < kSlots; ++q) {
    const int s = kWaveStates * w + 16 * q + j;
    const float2 a = s < N ? lam[s] : make_float2(0.0f, 0.0f);
    if (g == 0) {
      s_pw[pow_col(0, q, j)] = a;
      s_pw[pow_col(1, q, j)] = ipow(a, 4);
      s_pw[pow_col(2, q, j)] = ipow(a, 8);
      s_pw[pow_col(3, q, j)] = ipow(a, 16);
    }
    s_pw[pow_lane(0, q, lane)] = ipow(a, 4 * g + 1);
    s_pw[pow_lane(1, q, lane)] = ipow(a, 13 - 4 * g);
  }
  const bool lb_lane = lane < kWaveStates;
  const int s_lb = kWaveStates * w + lane;

  f4 accC[OB][kSlots][2], accW[HB][kSlots][2];
#pragma unroll
  for (int q = 0; q < kSlots; ++q) {
#pragma unroll
    for (int ob = 0; ob < OB; ++ob) accC[ob][q][0] = accC[ob][q][1] = f4_zero();
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) accW[hb][q][0] = accW[hb][q][1] = f4_zero();
  }
  float2 gl[kSlots];
#pragma unroll
  for (int q = 0; q < kSlots; ++q) gl[q] = make_float2(0.0f, 0.0f);

  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    if (threadIdx.x == 0) s_tile[buf ^ 1] = take_tile(counter);
    const int cr = (int)(tile / B), b = (int)(tile - (int64_t)cr * B);
    const int c = nsub - 1 - cr, t0 = c * kSub;

    // phase A: g_x by MFMA, reverse scans from zero at each block's end
    float cG[kSlots][2][OKS];
    // reloaded per tile (L2 hits), so that they do not stay live across phase B
    load_c_operands<OKS>(cG, rcre, rcim, w, g, j, N);
    float2 G[kBwdBlocks][kSlots][4];
    float2 eg[kBwdBlocks][kSlots];  // G at each block's first step from zero after its end
#pragma unroll
    for (int k = 0; k < kBwdBlocks; ++k) {
      const int t = t0 + kBlk * k + j;
      float ga[OKS];
#pragma unroll
      for (int kk = 0; kk < OKS; ++kk) {
        const int o = g * OKS + kk;
        const uint32_t off = (t < L && o < O) ? (uint32_t)((((int64_t)b * L + t) * O + o) * 4) : kOob;
        ga[kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rg, off, 0, 0));
      }
      f4 acc[kSlots][2];
#pragma unroll
      for (int q = 0; q < kSlots; ++q) acc[q][0] = acc[q][1] = f4_zero();
#pragma unroll
      for (int kk = 0; kk < OKS; ++kk)
#pragma unroll
        for (int q = 0; q < kSlots; ++q) {
          acc[q][0] = mfma(ga[kk], cG[q][0][kk], acc[q][0]);
          acc[q][1] = mfma(ga[kk], cG[q][1][kk], acc[q][1]);
        }
      const int tl = L - 1 - t0 - kBlk * k;  // block-relative step of the sequence's last step
      const bool last_here = g_xlast != nullptr && tl >= 0 && tl < kBlk && g == (tl >> 2);
#pragma unroll
      for (int q = 0; q < kSlots; ++q) {
#pragma unroll
        for (int r = 0; r < 4; ++r) G[k][q][r] = make_float2(acc[q][0][r], acc[q][1][r]);
        if (last_here) {
          const int s = kWaveStates * w + 16 * q + j;
          const float2 gl_in = s < N ? g_xlast[(int64_t)b * N + s] : make_float2(0.0f, 0.0f);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r == (tl & 3)) G[k][q][r] = cadd(G[k][q][r], gl_in);
        }
        const Pows pw = read_pows(s_pw, opaque_zero(), q, j, lane, true);
        block_scan_rev(G[k][q], pw.lm, pw.lm4, pw.lm8, lane);
        eg[k][q] = from_lane(G[k][q][0], j);
      }
    }

    // look-back on lane (g, j) for state kWaveStates w + lane over the later chunks of the row; the
    // multipliers come from lam per tile (an L2 hit) instead of living across the tile loop
    const float2* lam_t = lam;
    asm volatile("" : "+s"(lam_t));
    const double2 a_lb = lb_lane && s_lb < N ? up2(lam_t[s_lb]) : Num<double2>::zero();
    const double2 cP16 = conj2(ipow(a_lb, 16)), cP32 = conj2(ipow(a_lb, kSub));
    double2 agg_v = Num<double2>::zero();
#pragma unroll
    for (int k = kBwdBlocks - 1; k >= 0; --k) agg_v = Num<double2>::fma(cP16, agg_v, up2(pick(eg[k], g)));
    const int64_t widx = (int64_t)b * NS + s_lb;
    double2 R = Num<double2>::zero();  // G at the first step of the next chunk
    if (lb_lane) {
      if (c + 1 < nsub) {
        if (lb_pub_agg(cr, lb_spacing) && c > 0) put(agg + (int64_t)c * cstride + widx, agg_v);
        R = walk<4>(agg, inc, cstride, widx, c, +1, nsub, cP32, counter, lb_spacing.spin_max);
      }
      const double2 first = Num<double2>::fma(cP32, R, agg_v);  // G at this chunk's first step
      if (lb_pub_inc(cr, lb_spacing) && c > 0) put(inc + (int64_t)c * cstride + widx, first);
      if (c == 0 && g_x0 != nullptr && s_lb < N)
        g_x0[(int64_t)b * N + s_lb] = down2(Num<double2>::mul(conj2(a_lb), first));
    }
    float2 Rq[kSlots];
    {
      const float2 rf = down2(R);
#pragma unroll
      for (int q = 0; q < kSlots; ++q) Rq[q] = from_lane(rf, 16 * q + j);
    }
#pragma unroll
    for (int k = kBwdBlocks - 1; k >= 0; --k)
#pragma unroll
      for (int q = 0; q < kSlots; ++q) {
        const Pows pw = read_pows(s_pw, opaque_zero(), q, j, lane, true);
        float2 p = cmul_c(pw.lmx, Rq[q]);
#pragma unroll
        for (int r = 3; r >= 0; --r) {
          G[k][q][r] = cadd(G[k][q][r], p);
          p = cmul_c(pw.lm, p);
        }
        Rq[q] = cfma_c(pw.lm16, Rq[q], eg[k][q]);
      }

    // phase B: x recomputed block by block; the parameter gradients and g_u
    float2 xc[kSlots];  // state entering the current block
    {
      const float2 sv = lb_lane && s_lb < N ? saved[((int64_t)b * nsub + c) * N + s_lb] : make_float2(0.0f, 0.0f);
#pragma unroll
      for (int q = 0; q < kSlots; ++q) xc[q] = from_lane(sv, 16 * q + j);
    }
#pragma unroll
    for (int k = 0; k < kBwdBlocks; ++k) {
      const int tb = t0 + kBlk * k;
      float2 X[kSlots][4];
      {
        const int t = tb + j;
        float ua[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const int h = g * KS + kk;
          const uint32_t off = (t < L && h < H) ? (uint32_t)((((int64_t)b * L + t) * H + h) * 4) : kOob;
          ua[kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ru, off, 0, 0));
        }
        // in-proj B operands W_p[s][h] (s = kWaveStates w + 16 q + j, h = g KS + kk) read from LDS
        // at each use: the offset passes through an empty asm so the reads are not hoisted out of
        // the loops and the 2 kSlots KS values do not stay live across the tile
        int wofs = (g * KS) * kWuStride + 2 * j;
        asm volatile("" : "+v"(wofs));
        f4 acc[kSlots][2];
#pragma unroll
        for (int q = 0; q < kSlots; ++q) acc[q][0] = acc[q][1] = f4_zero();
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
          for (int q = 0; q < kSlots; ++q) {
            const float2 wv = *reinterpret_cast<const float2*>(&s_wu[wofs + kk * kWuStride + 32 * q]);
            acc[q][0] = mfma(ua[kk], wv.x, acc[q][0]);
            acc[q][1] = mfma(ua[kk], wv.y, acc[q][1]);
          }
#pragma unroll
        for (int q = 0; q < kSlots; ++q) {
#pragma unroll
          for (int r = 0; r < 4; ++r) X[q][r] = make_float2(acc[q][0][r], acc[q][1][r]);
          const Pows pw = read_pows(s_pw, opaque_zero(), q, j, lane, false);
          block_scan(X[q], pw.lm, pw.lm4, pw.lm8, lane);
          const float2 ex = from_lane(X[q][3], 48 + j);
          float2 p = cmul(pw.lmx, xc[q]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            X[q][r] = cadd(X[q][r], p);
            p = cmul(pw.lm, p);
          }
          // grad lam: G_t conj(x_{t-1}); x_{t-1} of a group's first step is the group below's last
          const float2 below = from_lane(X[q][3], lane - 16);
          const float2 xp = lane >= 16 ? below : xc[q];
          float2 acc_l = cmul_conj(G[k][q][0], xp);
#pragma unroll
          for (int r = 1; r < 4; ++r) acc_l = cadd(acc_l, cmul_conj(G[k][q][r], X[q][r - 1]));
          gl[q] = cadd(gl[q], acc_l);
          xc[q] = cfma(pw.lm16, xc[q], ex);
        }
      }
      // grad C (A = gy^T: lane j -> o = 16 ob + j, group g -> step 4g + r; B = x)
#pragma unroll
      for (int ob = 0; ob < OB; ++ob) {
        float gt[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = tb + 4 * g + r, o = 16 * ob + j;
          const uint32_t off = (t < L && o < O) ? (uint32_t)((((int64_t)b * L + t) * O + o) * 4) : kOob;
          gt[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rg, off, 0, 0));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int q = 0; q < kSlots; ++q) {
            accC[ob][q][0] = mfma(gt[r], X[q][r].x, accC[ob][q][0]);
            accC[ob][q][1] = mfma(gt[r], X[q][r].y, accC[ob][q][1]);
          }
      }
      // grad W (A = u^T: lane j -> h = 16 hb + j, group g -> step 4g + r; B = G)
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        float ut[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = tb + 4 * g + r, h = 16 * hb + j;
          const uint32_t off = (t < L && h < H) ? (uint32_t)((((int64_t)b * L + t) * H + h) * 4) : kOob;
          ut[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ru, off, 0, 0));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int q = 0; q < kSlots; ++q) {
            accW[hb][q][0] = mfma(ut[r], G[k][q][r].x, accW[hb][q][0]);
            accW[hb][q][1] = mfma(ut[r], G[k][q][r].y, accW[hb][q][1]);
          }
      }
      // g_u: G transposed through LDS (row t, column 2 s_local + p), W rows from LDS
#pragma unroll
      for (int q = 0; q < kSlots; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<float2*>(&s_xt[(4 * g + r) * kXtStride + 2 * (16 * q + j)]) = G[k][q][r];
      float xa[kM];
#pragma unroll
      for (int v = 0; v < kM / 4; ++v) {
        const f4 q4 = *reinterpret_cast<const f4*>(&s_xt[j * kXtStride + kM * g + 4 * v]);
        xa[4 * v] = q4[0];
        xa[4 * v + 1] = q4[1];
        xa[4 * v + 2] = q4[2];
        xa[4 * v + 3] = q4[3];
      }
      constexpr int kGw = kBlk * 16 * HB;  // floats of one wave's g_u block
      float* const sg = s_gu + (size_t)(k & 1) * NW * kGw;
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        f4 gacc = f4_zero();
#pragma unroll
        for (int v = 0; v < kM / 4; ++v) {
          const f4 wv = *reinterpret_cast<const f4*>(&s_wu[(16 * hb + j) * kWuStride + kM * g + 4 * v]);
          gacc = mfma(xa[4 * v], wv[0], gacc);
          gacc = mfma(xa[4 * v + 1], wv[1], gacc);
          gacc = mfma(xa[4 * v + 2], wv[2], gacc);
          gacc = mfma(xa[4 * v + 3], wv[3], gacc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sg[w * kGw + (4 * g + r) * 16 * HB + 16 * hb + j] = gacc[r];
      }
      __syncthreads();
      for (int idx = threadIdx.x; idx < kBlk * H; idx += blockDim.x) {
        const int tt = idx / H, h = idx - tt * H;
        float sum = sg[tt * 16 * HB + h];
        for (int ww = 1; ww < NW; ++ww) sum += sg[ww * kGw + tt * 16 * HB + h];
        const int t = tb + tt;
        if (t < L) g_u[((int64_t)b * L + t) * H + h] = sum;
      }
    }
  }

  // this workgroup's sums: [grad W: p, s, h (16 HB)] [grad C: p, s, o (16 OB)] [grad lam: s, re/im]
  constexpr int Hp = 16 * HB, Op = 16 * OB;
  float* pw = part + (int64_t)blockIdx.x * part_stride;
  float* pc = pw + 2 * NS * Hp;
  float* pl = pc + 2 * NS * Op;
#pragma unroll
  for (int q = 0; q < kSlots; ++q) {
    const int64_t s = kWaveStates * w + 16 * q + j;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) *reinterpret_cast<f4*>(&pw[(p * NS + s) * Hp + 16 * hb + 4 * g]) = accW[hb][q][p];
#pragma unroll
      for (int ob = 0; ob < OB; ++ob) *reinterpret_cast<f4*>(&pc[(p * NS + s) * Op + 16 * ob + 4 * g]) = accC[ob][q][p];
    }
    float2 v = gl[q];
    v = cadd(v, from_lane(v, lane ^ 16));
    v = cadd(v, from_lane(v, lane ^ 32));
    if (g == 0) *reinterpret_cast<float2*>(&pl[2 * s]) = v;
  }
}

// Adds the workgroups' partial sums: grad W_re / W_im [N, H], grad C_re / C_im [O, N] (C_im's
// sums negated), grad lam [N] complex. A block of 256 threads takes 64 outputs, consecutive in the
// partial buffer's layout (so every load of a wave is one contiguous row segment); thread slice k
// (of 4) adds the workgroups k, k + 4, ... in order, and the four slice sums are added in slice
// order, so the result does not depend on timing.
__global__ void __launch_bounds__(256) projscan_bwd_reduce(const float* __restrict__ part, int64_t part_stride,
                                                           int groups, int N, int NS, int H, int Hp, int O, int Op,
                                                           float* __restrict__ g_w_re, float* __restrict__ g_w_im,
                                                           float* __restrict__ g_c_re, float* __restrict__ g_c_im,
                                                           float* __restrict__ g_lam) {
  __shared__ float s_sum[4][64];
  const int lo = threadIdx.x & 63, slice = threadIdx.x >> 6;
  const int64_t i = blockIdx.x * (int64_t)64 + lo;
  const int64_t nW = 2 * (int64_t)N * H, nC = 2 * (int64_t)O * N, nL = 2 * (int64_t)N;
  int64_t off = 0;
  float* dst = nullptr;
  float sign = 1.0f;
  if (i < nW) {
    const int64_t p = i / ((int64_t)N * H), rem = i - p * N * H, s = rem / H, h = rem - s * H;
    off = (p * NS + s) * Hp + h;
    dst = (p ? g_w_im : g_w_re) + s * H + h;
  } else if (i < nW + nC) {
    const int64_t k = i - nW, p = k / ((int64_t)O * N), rem = k - p * O * N, s = rem / O, o = rem - s * O;
    off = 2 * (int64_t)NS * Hp + (p * NS + s) * Op + o;
    dst = (p ? g_c_im : g_c_re) + o * N + s;
    sign = p ? -1.0f : 1.0f;
  } else if (i < nW + nC + nL) {
    const int64_t k = i - nW - nC;
    off = 2 * (int64_t)NS * Hp + 2 * (int64_t)NS * Op + k;
    dst = g_lam + k;
  }
  float sum = 0.0f;
  if (dst != nullptr) {
#pragma unroll 4
    for (int grp = slice; grp < groups; grp += 4) sum += part[(int64_t)grp * part_stride + off];
  }
  s_sum[slice][lo] = sum;
  __syncthreads();
  if (slice == 0 && dst != nullptr) *dst = sign * (((s_sum[0][lo] + s_sum[1][lo]) + s_sum[2][lo]) + s_sum[3][lo]);
}

// Gradients of an empty sequence (L = 0): the parameters get zeros, g_x0 = g_xlast (x_last = x0).
__global__ void __launch_bounds__(256) projscan_bwd_empty(const float2* __restrict__ g_xlast, float2* __restrict__ g_x0,
                                                          int64_t nx, float* __restrict__ g_w_re,
                                                          float* __restrict__ g_w_im, int64_t nw,
                                                          float* __restrict__ g_c_re, float* __restrict__ g_c_im,
                                                          int64_t nc, float* __restrict__ g_lam, int64_t nl) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (g_x0 != nullptr && i < nx) g_x0[i] = g_xlast != nullptr ? g_xlast[i] : make_float2(0.0f, 0.0f);
  if (i < nw) g_w_re[i] = g_w_im[i] = 0.0f;
  if (i < nc) g_c_re[i] = g_c_im[i] = 0.0f;
  if (i < nl) g_lam[i] = 0.0f;
}

// ---------------------------------------------------------------- host side
constexpr int64_t kMaxH = 32, kMaxN = 256, kMaxO = 32;

struct PsPlan {
  int nw = 1;
  int64_t nchunks = 0, nsub = 0, tiles = 0, words = 0;  // words: double2 look-back slots per array
  size_t off_agg = 0, off_inc = 0, bytes = 0;
};

PsPlan ps_plan(int64_t B, int64_t L, int64_t N) {
  PsPlan p;
  p.nw = (int)((N + kWaveStates - 1) / kWaveStates);
  p.nchunks = (L + kChunk - 1) / kChunk;
  p.nsub = (L + kSub - 1) / kSub;
  p.tiles = p.nchunks * B;
  p.words = p.nchunks * B * p.nw * kWaveStates;
  p.off_agg = kCounterBytes;
  p.off_inc = p.off_agg + sizeof(double2) * (size_t)p.words;
  p.bytes = p.off_inc + sizeof(double2) * (size_t)p.words;
  return p;
}

int ks_for(int64_t H) { return H <= 4 ? 1 : H <= 8 ? 2 : H <= 16 ? 4 : 8; }
int ob_for(int64_t O) { return O <= 16 ? 1 : 2; }

// Backward: 32-step tiles, look-back words per half chunk, and one partial-sum slot per
// workgroup (a compute unit holds at most kMaxWaves / nw of them: two waves per SIMD).
struct PbPlan {
  int nw = 1, groups = 1;
  int64_t nsub = 0, tiles = 0, words = 0, part_stride = 0;
  size_t off_agg = 0, off_inc = 0, off_part = 0, bytes = 0;
};

PbPlan pb_plan(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O) {
  PbPlan p;
  p.nw = (int)((N + kWaveStates - 1) / kWaveStates);
  p.nsub = (L + kSub - 1) / kSub;
  p.tiles = p.nsub * B;
  p.words = p.nsub * B * p.nw * kWaveStates;
  const int64_t NS = p.nw * kWaveStates, Hp = ks_for(H) == 8 ? 32 : 16, Op = 16 * ob_for(O);
  p.part_stride = ((2 * NS * Hp + 2 * NS * Op + 2 * NS) + 63) / 64 * 64;
  const int64_t cap = (int64_t)device_cus() * (kMaxWaves / p.nw > 0 ? kMaxWaves / p.nw : 1);
  p.groups = (int)(p.tiles < cap ? (p.tiles > 0 ? p.tiles : 1) : cap);
  p.off_agg = kCounterBytes;
  p.off_inc = p.off_agg + sizeof(double2) * (size_t)p.words;
  p.off_part = (p.off_inc + sizeof(double2) * (size_t)p.words + 255) / 256 * 256;
  p.bytes = p.off_part + sizeof(float) * (size_t)p.part_stride * p.groups;
  return p;
}

int ps_args_status(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O) {
  if (B < 0 || L < 0 || H < 1 || N < 1 || O < 1) return TSF_ERR_ARG;
  if (H > kMaxH || N > kMaxN || O > kMaxO) return TSF_ERR_UNSUPPORTED;
  // u and gy are read through buffer resources with 32-bit byte offsets; chunk and row indices are int
  if (B * L * H * 4 >= ((int64_t)1 << 31) || B * L * O * 4 >= ((int64_t)1 << 31) || B > INT32_MAX / 2 ||
      L > INT32_MAX / 2)
    return TSF_ERR_UNSUPPORTED;
  return TSF_OK;
}

#define TSF_PS_CASES(X) X(1, 1) X(1, 2) X(2, 1) X(2, 2) X(4, 1) X(4, 2) X(8, 1) X(8, 2)

// Persistent grid size for a kernel with dynamic LDS (per device, cached by wave count); raises the
// kernel's dynamic-LDS limit first when it needs more than the default 64 KiB.
template <typename F>
int resident_wgs_lds(F kern, int threads, size_t lds, int (&cache)[64][kMaxWaves + 1], int64_t& out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return tsf_record_hip_error(e);
  if (dev < 0 || dev >= 64) return TSF_ERR_UNSUPPORTED;
  int& c = cache[dev][threads / 64];
  if (c == 0) {
    if (lds > 65536) {
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return tsf_record_hip_error(e);
    }
    int n = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds);
    if (e != hipSuccess) return tsf_record_hip_error(e);
    if (n < 1) return TSF_ERR_UNSUPPORTED;
    c = n;
  }
  out = (int64_t)c * device_cus();
  return TSF_OK;
}

template <int KS, int OB>
int fwd_launch(const PsPlan& p, int64_t B, int64_t L, int64_t H, int64_t N, int64_t O, const float* u,
               const float* w_re, const float* w_im, const float2* lam, const float* c_re, const float* c_im,
               const float2* x0, float* y, float2* x_last, float2* saved, char* ws, hipStream_t s) {
  static int occ[64][kMaxWaves + 1];
  const int threads = 64 * p.nw;
  const size_t lds = fwd_lds_bytes<OB>(p.nw);
  int64_t cap = 0;
  const int st = resident_wgs_lds(projscan_fwd<KS, OB>, threads, lds, occ, cap);
  if (st != TSF_OK) return st;
  lookback_reset_launch(ws, 4 * p.words, s);
  hipLaunchKernelGGL((projscan_fwd<KS, OB>), dim3((unsigned)(p.tiles < cap ? p.tiles : cap)), dim3(threads), lds, s, u,
                     w_re, w_im, lam, c_re, c_im, x0, y, x_last, saved, reinterpret_cast<double2*>(ws + p.off_agg),
                     reinterpret_cast<double2*>(ws + p.off_inc), reinterpret_cast<unsigned*>(ws), (int)B, (int)L,
                     (int)H, (int)N, (int)O, (int)p.nchunks, (int)p.nsub, lb_spacing_for(kProjAnchorSpacing));
  return TSF_OK;
}

template <int KS, int OB>
int bwd_launch(const PbPlan& p, int64_t B, int64_t L, int64_t H, int64_t N, int64_t O, const float* gy,
                const float2* g_xlast, const float2* saved, const float* u, const float* w_re, const float* w_im,
                const float2* lam, const float* c_re, const float* c_im, float* g_u, float* g_w_re, float* g_w_im,
                float* g_lam, float* g_c_re, float* g_c_im, float2* g_x0, char* ws, hipStream_t s) {
  static int occ[64][kMaxWaves + 1];
  const int threads = 64 * p.nw;
  const size_t lds = bwd_lds_bytes<hb_for_ks<KS>()>(p.nw);
  int64_t cap = 0;
  const int st = resident_wgs_lds(projscan_bwd<KS, OB>, threads, lds, occ, cap);
  if (st != TSF_OK) return st;
  lookback_reset_launch(ws, 4 * p.words, s);
  const int grid = (int)(p.groups < cap ? p.groups : cap);
  float* part = reinterpret_cast<float*>(ws + p.off_part);
  hipLaunchKernelGGL((projscan_bwd<KS, OB>), dim3((unsigned)grid), dim3(threads), lds, s, gy, g_xlast, saved, u, w_re,
                     w_im, lam, c_re, c_im, g_u, g_x0, part, p.part_stride,
                     reinterpret_cast<double2*>(ws + p.off_agg), reinterpret_cast<double2*>(ws + p.off_inc),
                     reinterpret_cast<unsigned*>(ws), (int)B, (int)L, (int)H, (int)N, (int)O, (int)p.nsub, lb_spacing_for(kProjAnchorSpacing));
  const int64_t outs = 2 * N * H + 2 * O * N + 2 * N;
  hipLaunchKernelGGL(projscan_bwd_reduce, dim3((unsigned)((outs + 63) / 64)), dim3(256), 0, s, part, p.part_stride,
                     grid, (int)N, p.nw * kWaveStates, (int)H, KS == 8 ? 32 : 16, (int)O, 16 * OB, g_w_re, g_w_im, g_c_re,
                     g_c_im, g_lam);
  return TSF_OK;
}

}  // namespace

extern "C" {

int64_t tsfast_hip_projscan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O) {
  if (ps_args_status(B, L, H, N, O) != TSF_OK) return -1;
  return (int64_t)ps_plan(B, L, N).bytes;
}

int64_t tsfast_hip_projscan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O) {
  if (ps_args_status(B, L, H, N, O) != TSF_OK) return -1;
  return (int64_t)pb_plan(B, L, H, N, O).bytes;
}

int64_t tsfast_hip_projscan_saved_floats(int64_t B, int64_t L, int64_t N) {
  if (B < 0 || L < 0 || N < 1) return -1;
  return 2 * B * ps_plan(B, L, N).nsub * N;
}

int tsfast_hip_projscan_fwd(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O, const float* u, const float* w_re,
                            const float* w_im, const void* lam, const float* c_re, const float* c_im, const void* x0,
                            float* y, void* x_last, float* saved, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  const int st = ps_args_status(B, L, H, N, O);
  if (st != TSF_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0) return TSF_OK;
  const float2* x0c = static_cast<const float2*>(x0);
  float2* xl = static_cast<float2*>(x_last);
  if (L == 0) {
    if (xl) hipLaunchKernelGGL(projscan_copy_state, dim3((unsigned)((B * N + 255) / 256)), dim3(256), 0, s, x0c, xl, B * N);
    return tsf_launch_status();
  }
  if (!u || !w_re || !w_im || !lam || !c_re || !c_im || !y) return TSF_ERR_ARG;
  const PsPlan p = ps_plan(B, L, N);
  if (!workspace || workspace_bytes < (int64_t)p.bytes) return TSF_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  const float2* lamc = static_cast<const float2*>(lam);
  float2* sv = reinterpret_cast<float2*>(saved);
  switch (ks_for(H) * 10 + ob_for(O)) {
#define X(KS_, OB_)                                                                                            \
  case KS_ * 10 + OB_: {                                                                                       \
    const int rc = fwd_launch<KS_, OB_>(p, B, L, H, N, O, u, w_re, w_im, lamc, c_re, c_im, x0c, y, xl, sv, ws, s); \
    if (rc != TSF_OK) return rc;                                                                               \
    break;                                                                                                     \
  }
    TSF_PS_CASES(X)
#undef X
    default:
      return TSF_ERR_UNSUPPORTED;
  }
  return tsf_launch_status();
}

int tsfast_hip_projscan_bwd(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O, const float* gy,
                            const void* g_xlast, const float* saved, const float* u, const float* w_re,
                            const float* w_im, const void* lam, const float* c_re, const float* c_im, float* g_u,
                            float* g_w_re, float* g_w_im, void* g_lam, float* g_c_re, float* g_c_im, void* g_x0,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  const int st = ps_args_status(B, L, H, N, O);
  if (st != TSF_OK) return st;
  if (!g_w_re || !g_w_im || !g_lam || !g_c_re || !g_c_im) return TSF_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float2* gxl = static_cast<const float2*>(g_xlast);
  float2* gx0 = static_cast<float2*>(g_x0);
  float* gl = static_cast<float*>(g_lam);
  if (B == 0 || L == 0) {
    const int64_t n = std::max({B * N, N * H, O * N, 2 * N, (int64_t)1});
    hipLaunchKernelGGL(projscan_bwd_empty, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gxl, gx0, B * N, g_w_re,
                       g_w_im, N * H, g_c_re, g_c_im, O * N, gl, 2 * N);
    return tsf_launch_status();
  }
  if (!gy || !saved || !u || !w_re || !w_im || !lam || !c_re || !c_im || !g_u) return TSF_ERR_ARG;
  const PbPlan p = pb_plan(B, L, H, N, O);
  if (!workspace || workspace_bytes < (int64_t)p.bytes) return TSF_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  const float2* lamc = static_cast<const float2*>(lam);
  const float2* sv = reinterpret_cast<const float2*>(saved);
  switch (ks_for(H) * 10 + ob_for(O)) {
#define X(KS_, OB_)                                                                                                 \
  case KS_ * 10 + OB_: {                                                                                            \
    const int rc = bwd_launch<KS_, OB_>(p, B, L, H, N, O, gy, gxl, sv, u, w_re, w_im, lamc, c_re, c_im, g_u, g_w_re, \
                                        g_w_im, gl, g_c_re, g_c_im, gx0, ws, s);                                    \
    if (rc != TSF_OK) return rc;                                                                                    \
    break;                                                                                                          \
  }
    TSF_PS_CASES(X)
#undef X
    default:
      return TSF_ERR_UNSUPPORTED;
  }
  return tsf_launch_status();
}

}  // extern "C"
