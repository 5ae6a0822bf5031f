// Fused Mamba selective SSM, forward and backward, bf16 or fp32 I/O with fp32 state.
//
//   delta_t = softplus(draw_t)                        (threshold 20, as F.softplus)
//   h_t     = exp(delta_t A) * h_{t-1} + delta_t u_t B_t
//   out_t   = (sum_n h_t C_t + Dp u_t) * z_t * sigmoid(z_t)
//
// Reference semantics: tsfast/models/architectures/mamba/mamba_triton.py:85-286 (kernels) and
// :286-489 (ops), mamba/backend_c.py:105-245 (CPU kernels, same algebra).
//
// The scan is VALU-bound on gfx950 (one exp and ~4 (fwd) / ~13 (bwd) fp32 ops per state element
// against 2-5 bytes of HBM traffic per element), so the layout minimises per-element VALU work
// and LDS traffic and keeps every SIMD busy:
//
//  * Workgroup = one batch row b x a tile of DT=32 channels, all N states, walking the whole
//    sequence. NG lanes share a channel, each holding NPT = NS/NG states in VGPRs (NG = 8 for
//    N >= 8), so the grid B * D/32 (768 workgroups of 4 waves at config 3) puts three
//    workgroups on every CU with no tail; workgroups are renumbered so that each XCD works on a
//    contiguous range of tiles (neighbouring tiles share L2 lines).
//  * Time advances in chunks. Per-(t, d) scalar work (softplus, sigmoid, gates, the D skip) is
//    done once per (t, d) by an "owner" thread and staged through LDS, with coalesced 32-channel
//    row loads/stores; each lane then runs only the per-state recurrence.
//  * Forward: every lane stores its partial sum over its states (y = h.C) to LDS and the owner
//    thread adds the NG partials of its (t, d).
//  * Backward: each 16-lane DPP row holds one state group; the chunk's B_t/C_t values live in
//    VGPRs spread over the row and reach the lanes through DPP row broadcasts. It recomputes
//    each chunk's states from the forward's fp32 checkpoint into registers (lam_t, lam_t h_{t-1}
//    and h_t for the chunk), then runs the adjoint
//        G_t = gy_t C_t + lam_{t+1} G_{t+1}
//    backwards through the chunk, so exp is evaluated once per element per pass; the gate
//    gradient reads the forward's saved pre-gate output y instead of recomputing sum_n h C.
//  * grad B_t / grad C_t (sums over channels) are reduced over the channels of the tile (32; 16
//    in the backward from N = 32, see bwd_dt) in LDS and written as partials [D/DT, B, L, 2*NS]
//    in the I/O type (the reference keeps its
//    per-block partials in the I/O dtype too); a second kernel sums the partials in fp32 in a
//    fixed order (no atomics: deterministic run to run).
// The next chunk's inputs are loaded into registers while the current chunk computes.
#include <type_traits>

#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

int ns_for(int64_t N) {
  if (N <= 4) return 4;
  if (N <= 8) return 8;
  if (N <= 16) return 16;
  if (N <= 32) return 32;
  if (N <= 64) return 64;
  return 0;
}

// Forward steps whose LDS operands are read in one batch, ahead of their use (NPT <= 2).
#ifndef TSF_MAMBA_FWD_RD
#define TSF_MAMBA_FWD_RD 4
#endif
// Channels per workgroup of the forward and of the backward (16 or 32).
#ifndef TSF_MAMBA_FWD_DT
#define TSF_MAMBA_FWD_DT 32
#endif
#ifndef TSF_MAMBA_BWD_DT
#define TSF_MAMBA_BWD_DT 32
#endif
#ifndef TSF_MAMBA_BWD_HG
#define TSF_MAMBA_BWD_HG 0
#endif

// Lanes per channel of the forward (8 or 16) and its steps per LDS round (0: the default).
#ifndef TSF_MAMBA_FWD_NG
#define TSF_MAMBA_FWD_NG 8
#endif
#ifndef TSF_MAMBA_FWD_TF
#define TSF_MAMBA_FWD_TF 0
#endif

// Backward lane split and the checkpoint interval shared by both directions.
template <int NS>
struct MCfg {
  static constexpr int NG = NS >= 8 ? 8 : NS;  // lanes per channel
  static constexpr int NPT = NS / NG;          // states per lane
  // checkpoint interval = backward recompute chunk (lam_t and h_t of a chunk live in VGPRs)
  static constexpr int CHK = NPT <= 2 ? 8 : (NPT == 4 ? 8 : 4);
};

// Forward tiling: DT channels per workgroup, NG lanes per channel with NPT states each.
template <int NS>
struct FCfg {
  static constexpr int NG = NS >= TSF_MAMBA_FWD_NG ? TSF_MAMBA_FWD_NG : NS;
  static constexpr int NPT = NS / NG;
  static constexpr int DT = TSF_MAMBA_FWD_DT;
  static constexpr int TH = DT * NG;
  static constexpr int CHK = MCfg<NS>::CHK;
  static constexpr int TF = TSF_MAMBA_FWD_TF > 0 ? TSF_MAMBA_FWD_TF : (NPT <= 2 ? 32 : 2 * CHK);
  static constexpr int IT_F = (TF * DT + TH - 1) / TH;  // owned (t, d) items per thread
  static constexpr int BC_F = (TF * NS + TH - 1) / TH;  // B/C tile elements per thread
  static constexpr int WAVES = TH / 64;
  static constexpr int OCC = (12 / WAVES) > 1 ? (12 / WAVES) : 1;  // workgroups per CU aimed at
};

template <typename TIO>
TSF_DEV TIO io_zero();
template <>
TSF_DEV float io_zero<float>() {
  return 0.0f;
}
template <>
TSF_DEV bf16 io_zero<bf16>() {
  bf16 zr;
  zr.bits = 0;
  return zr;
}

template <bool V>
using Bool = std::integral_constant<bool, V>;

// Wave issue priority (s_setprio takes an immediate, 0..3).
TSF_DEV void set_wave_priority(unsigned p) {
  switch (p) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
  }
}


// Streaming store for the training forward's saved state, which is read back only by the
// backward (non-temporal: it is not kept in the caches on the way out).
TSF_DEV void nt_store(float* p, float v) { __builtin_nontemporal_store(v, p); }
TSF_DEV void nt_store(bf16* p, bf16 v) { __builtin_nontemporal_store(v.bits, &p->bits); }
// The same at a 32-bit element index from a workgroup-uniform base (SGPR base + VGPR offset).
template <typename T>
TSF_DEV void nt_st32(T* __restrict__ base, uint32_t idx, T v) {
  nt_store(reinterpret_cast<T*>(reinterpret_cast<char*>(base) + idx * (uint32_t)sizeof(T)), v);
}

// Pairwise sum of K values (K a power of two), in a fixed order.
template <int K>
TSF_DEV float tree_sum(const float* v) {
  if constexpr (K == 1) {
    return v[0];
  } else {
    return tree_sum<K / 2>(v) + tree_sum<K / 2>(v + K / 2);
  }
}

// Floats of training-forward saved state per batch row: fp32 checkpoints [NC, N, D], then the
// pre-gate output y [L, D] in the I/O type (padded to whole floats).
template <typename TIO>
TSF_HOST_DEV int64_t saved_row_floats(int64_t L, int64_t D, int64_t N, int64_t NC) {
  return NC * N * D + (L * D * (int64_t)sizeof(TIO) + 3) / 4;
}

// Workgroups go to the 8 XCDs (each with its own L2) round-robin by linear id. Renumber them so
// that every XCD receives a contiguous range of (channel tile, batch row) pairs: neighbouring
// channel tiles share the 128-byte lines of each bf16 [B, L, D] row (one tile's row segment is
// 64 bytes), and on one XCD the second read of a line hits that XCD's L2 instead of HBM.
// The grid is one-dimensional (nT channel tiles x B batch rows, tile-major), so the batch size
// is not bounded by the 65535 limit of a grid's y dimension.
constexpr unsigned kXcds = 8;
TSF_DEV void xcd_remap(int64_t nT, int64_t& tile, int64_t& row) {
  const unsigned total = gridDim.x;
  unsigned lin = blockIdx.x;
  if (total % kXcds == 0) lin = (lin % kXcds) * (total / kXcds) + lin / kXcds;
  tile = lin % nT;
  row = lin / nT;
}

// ------------------------------------------------------------------------------------ DPP rows
// Lane layout shared by both directions: the workgroup's TH = DT * NG threads form rows of 16
// lanes (a DPP row); row r holds state group ng = r / (DT / 16) for channels
// dl = 16 * (r % (DT / 16)) + (lane in row), and a lane's NPT states are n = j * NG + ng. B_t and
// C_t of a row's states are the same for its 16 lanes, so a tile of B/C values sits in VGPRs
// spread over the row (slot s = i * NPT + j in lane s % 16 of register s / 16) and reaches every
// lane through a DPP row broadcast (row_newbcast) folded into the consuming multiply; no LDS
// round trip. Consecutive state groups sit in adjacent rows of the per-state-group scratch, so
// every per-step LDS store of a wave is 64 consecutive floats.
template <int K>
TSF_DEV float row_bcast_k(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + K, 0xF, 0xF, true));
}
// lane k (0..15) of this lane's DPP row; k must fold to a constant at compile time
TSF_DEV float row_bcast(float x, int k) {
  switch (k) {
    case 0: return row_bcast_k<0>(x);
    case 1: return row_bcast_k<1>(x);
    case 2: return row_bcast_k<2>(x);
    case 3: return row_bcast_k<3>(x);
    case 4: return row_bcast_k<4>(x);
    case 5: return row_bcast_k<5>(x);
    case 6: return row_bcast_k<6>(x);
    case 7: return row_bcast_k<7>(x);
    case 8: return row_bcast_k<8>(x);
    case 9: return row_bcast_k<9>(x);
    case 10: return row_bcast_k<10>(x);
    case 11: return row_bcast_k<11>(x);
    case 12: return row_bcast_k<12>(x);
    case 13: return row_bcast_k<13>(x);
    case 14: return row_bcast_k<14>(x);
    default: return row_bcast_k<15>(x);
  }
}

// ------------------------------------------------------------------------------------ forward
// SAVE: training forward (writes the checkpoints and y to chk); chk is unused otherwise.
template <typename TIO, int NS, bool SAVE>
__global__ void __launch_bounds__(FCfg<NS>::TH, FCfg<NS>::WAVES >= 8 ? 3 : 1) mamba_fwd_kernel(
    const TIO* __restrict__ draw, const float* __restrict__ A, const TIO* __restrict__ Bt,
    const TIO* __restrict__ Ct, const TIO* __restrict__ u, const TIO* __restrict__ z, const float* __restrict__ Dp,
    const float* __restrict__ h0, TIO* __restrict__ out, float* __restrict__ h_last, float* __restrict__ chk,
    int64_t L, int64_t D, int N, int64_t NC, unsigned cus) {
  using C = FCfg<NS>;
  constexpr int NPT = C::NPT, NG = C::NG, DT = C::DT, TH = C::TH, CHK = C::CHK, TF = C::TF;
  constexpr int IT = C::IT_F, BCI = C::BC_F;
  __shared__ float2 s_sc[TF][DT];       // (delta, delta * u)
  __shared__ float2 s_bc[TF][NS];       // (B, C)
  // y partial per lane (state group); odd groups store channel dl at column dl ^ 16, so the two
  // lanes of a state pair (same channel, rows 32 floats apart) write to different banks
  __shared__ float s_y[TF][NG][DT];
  // with 32-channel tiles the two lanes of a state pair sit in one half-wave, 32 floats apart
  constexpr int kSwz = DT >= 32 ? 16 : 0;

  const int tid = threadIdx.x;
  int64_t tile, b;
  xcd_remap((D + DT - 1) / DT, tile, b);
  const int64_t d0 = tile * DT;
  // recurrence mapping: adjacent lanes hold the two halves of a state pair
  const int pr = tid & 1;
  const int dl = (tid >> 1) & (DT - 1);
  const int ng = 2 * (tid / (2 * DT)) + pr;
  const int n0 = ng * NPT;
  const int64_t d = d0 + dl;
  const bool act = d < D;
  // owner mapping: item k of this thread is (t = tid / DT + k * NG, channel d0 + tid % DT)
  const int od = tid % DT;
  const bool oact = d0 + od < D;
  // workgroup-uniform bases and 32-bit per-thread offsets (the host bounds L*D and L*N)
  const int64_t rowD = b * L * D + d0, rowN = b * L * N;
  const uint32_t Du = (uint32_t)D, Nu = (uint32_t)N;

  float A2[NPT], h[NPT];
  uint32_t co[NPT];  // offset of state n0 + j of this channel within one checkpoint slot [N, D]
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int n = n0 + j;
    A2[j] = (act && n < N) ? A[d * N + n] * kLog2e : 0.0f;
    h[j] = (act && h0 && n < N) ? h0[(b * D + d) * N + n] : 0.0f;
    co[j] = (uint32_t)n * Du + (uint32_t)dl;
  }
  const uint32_t slot_floats = Nu * Du;
  const float dp_o = oact ? Dp[d0 + od] : 0.0f;

  // workgroup-uniform row bases: loads use SGPR base + 32-bit VGPR offset addressing
  const TIO* __restrict__ drw = draw + rowD;
  const TIO* __restrict__ urw = u + rowD;
  const TIO* __restrict__ zrw = z + rowD;
  TIO* __restrict__ orw = out + rowD;
  const TIO* __restrict__ brw = Bt + rowN;
  const TIO* __restrict__ crw = Ct + rowN;
  // saved state of this batch row (training only): checkpoints [NC, N, D], then y [L, D]
  float* __restrict__ svb = SAVE ? chk + b * saved_row_floats<TIO>(L, D, N, NC) : nullptr;
  float* __restrict__ chkb = SAVE ? svb + d0 : nullptr;
  TIO* __restrict__ yrw = SAVE ? reinterpret_cast<TIO*>(svb + NC * N * D) + d0 : nullptr;

  TIO r_dr[IT], r_u[IT], r_z[IT], r_b[BCI], r_c[BCI];
  auto load_chunk = [&](uint32_t t0, auto full) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full)::value;
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      const int idx = tid + k * TH;
      const uint32_t t = (uint32_t)(idx / DT);
      bool v = idx < TF * DT;
      if (!FULL) v = v && oact && (int64_t)(t0 + t) < L;
      const uint32_t o = (t0 + t) * Du + (uint32_t)od;
      r_dr[k] = v ? ld32(drw, o) : io_zero<TIO>();
      r_u[k] = v ? ld32(urw, o) : io_zero<TIO>();
      r_z[k] = v ? ld32(zrw, o) : io_zero<TIO>();
    }
#pragma unroll
    for (int k = 0; k < BCI; ++k) {
      const int idx = tid + k * TH;
      const uint32_t t = (uint32_t)(idx / NS), n = (uint32_t)(idx % NS);
      bool v = idx < TF * NS;
      if (!FULL) v = v && (int)n < N && (int64_t)(t0 + t) < L;
      const uint32_t o = (t0 + t) * Nu + n;
      r_b[k] = v ? ld32(brw, o) : io_zero<TIO>();
      r_c[k] = v ? ld32(crw, o) : io_zero<TIO>();
    }
  };
  // FULL loads (no per-element guard): all TF steps in the sequence, all DT channels in range
  // and N == NS; workgroup-uniform
  const bool wg_full = d0 + DT <= D && N == NS;
  if (L > 0) {
    if (TF <= L && wg_full)
      load_chunk(0u, Bool<true>());
    else
      load_chunk(0u, Bool<false>());
  }

  float o_u[IT], o_z[IT];
  // Steps past the end of the sequence run as identity steps (delta = 0: lam = 1, no input),
  // so the recurrence needs no per-step guard; only stores check the length.
  auto chunk = [&](uint32_t t0, int len) __attribute__((always_inline)) {
    // phase 1: owner scalars and the B/C tile into LDS
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      const int idx = tid + k * TH;
      if ((TF * DT) % TH == 0 || idx < TF * DT) {
        o_u[k] = to_f32(r_u[k]);
        o_z[k] = to_f32(r_z[k]);
        const bool live = oact && idx / DT < len;
        const float delta = live ? softplus_ref(to_f32(r_dr[k])) : 0.0f;
        s_sc[idx / DT][idx % DT] = make_float2(delta, delta * o_u[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < BCI; ++k) {
      const int idx = tid + k * TH;
      if (idx < TF * NS) s_bc[idx / NS][idx % NS] = make_float2(to_f32(r_b[k]), to_f32(r_c[k]));
    }
    // prefetch the next round while this one computes
    const uint32_t t1 = t0 + TF;
    if ((int64_t)t1 < L) {
      if ((int64_t)t1 + TF <= L && wg_full)
        load_chunk(t1, Bool<true>());
      else
        load_chunk(t1, Bool<false>());
    }
    __syncthreads();
    // phase 2: the recurrence, NPT states per lane, in batches of kRd steps. The LDS operands
    // of the next batch are read while the current batch computes (two register buffers), and
    // the step body has no branch (every lane stores its own y partial).
    constexpr int kRd = NPT <= 2 ? TSF_MAMBA_FWD_RD : 2;
    static_assert(TF % kRd == 0 && CHK % kRd == 0, "read batches must not straddle checkpoints");
    float2 sv[2][kRd], bcv[2][kRd][NPT];
    auto read_batch = [&](int buf, int i0) __attribute__((always_inline)) {
#pragma unroll
      for (int r = 0; r < kRd; ++r) {
        sv[buf][r] = s_sc[i0 + r][dl];
#pragma unroll
        for (int j = 0; j < NPT; ++j) bcv[buf][r][j] = s_bc[i0 + r][n0 + j];
      }
    };
    read_batch(0, 0);
#pragma unroll
    for (int i0 = 0; i0 < TF; i0 += kRd) {
      const int cur = (i0 / kRd) & 1;
      if (i0 + kRd < TF) read_batch(cur ^ 1, i0 + kRd);
#pragma unroll
      for (int r = 0; r < kRd; ++r) {
        const int i = i0 + r;
        float y = 0.0f;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
          const float lam = fast_exp2(sv[cur][r].x * A2[j]);
          h[j] = fmaf(lam, h[j], sv[cur][r].y * bcv[cur][r][j].x);
          y = fmaf(h[j], bcv[cur][r][j].y, y);
        }
        s_y[i][ng][dl ^ ((ng & 1) * kSwz)] = y;
      }
      // checkpoint slot k holds the state after step (k + 1) * CHK - 1 (layout [B, NC, N, D])
      const int ie = i0 + kRd - 1;
      if (SAVE && (ie % CHK) == CHK - 1 && act && ie < len) {
        const uint32_t slot = (t0 + (uint32_t)ie) / CHK;
#pragma unroll
        for (int j = 0; j < NPT; ++j)
          if (n0 + j < N) nt_st32(chkb, slot * slot_floats + co[j], h[j]);
      }
    }
    __syncthreads();
    // phase 3: owners finish y, apply the D skip and the SiLU gate, store the output row
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      const int idx = tid + k * TH;
      const int t = idx / DT;
      if (((TF * DT) % TH == 0 || idx < TF * DT) && t < len && oact) {
        float yp[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) yp[g] = s_y[t][g][od ^ ((g & 1) * kSwz)];
        const float y = tree_sum<NG>(yp);
        const float zz = o_z[k];
        const uint32_t o = (t0 + (uint32_t)t) * Du + (uint32_t)od;
        const float yv = fmaf(dp_o, o_u[k], y);
        st32(orw, o, from_f32<TIO>(yv * zz * sigmoid_fast(zz)));
        if (SAVE) nt_st32(yrw, o, from_f32<TIO>(yv));  // the backward's gate gradient needs y before the gate
      }
    }
  };
  // Workgroups sharing a CU (slot = dispatch round) are issued oldest-first, so the first one
  // races ahead and the last ones finish alone; rotating the issue priority among the slots
  // every four rounds evens their progress and shortens the tail.
  const unsigned slot = blockIdx.x / cus;
  for (int64_t t0 = 0; t0 < L; t0 += TF) {
    if (((t0 / TF) & 3) == 0) set_wave_priority((slot + (unsigned)(t0 / TF / 4)) % 3);
    chunk((uint32_t)t0, (int)((L - t0) < TF ? (L - t0) : TF));
  }
  (void)NG;
  if (act) {
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if (n0 + j < N) h_last[(b * D + d) * N + n0 + j] = h[j];
  }
}

// ------------------------------------------------------------------------------------ backward
// Tiling: a workgroup covers one batch row x DT = 32 channels (config 3: 768 workgroups of 4
// waves, three per CU, so a workgroup waiting at a barrier leaves the CU to the other two), in
// the DPP-row lane layout above; each chunk's B/C tile is broadcast from registers.
template <int NS, int DT_>
struct BCfg {
  static constexpr int NG = MCfg<NS>::NG, NPT = MCfg<NS>::NPT;
  static constexpr int DT = DT_;
  static constexpr int TH = DT * NG;
  static constexpr int RPG = DT / 16;                    // DPP rows per state group
  static constexpr int CHK = MCfg<NS>::CHK;              // the forward's checkpoint interval
  static constexpr int IT = (CHK * DT + TH - 1) / TH;    // owned (t, d) items per thread
  static constexpr int W2 = 2 * NS;                      // grad B / grad C columns
  static constexpr int NSL = CHK * NPT;                  // B/C broadcast slots per chunk and row
  static constexpr int NBV = (NSL + 15) / 16;            // VGPRs per B (and per C) tile
  static constexpr int WAVES = TH / 64;
  static constexpr int OCC = (12 / WAVES) > 1 ? (12 / WAVES) : 1;  // workgroups per CU aimed at
  static_assert(DT % 16 == 0, "channel tile must be whole DPP rows");
};

// Per chunk of CHK steps (walking from the end of the sequence), between two barriers:
//   A  recompute the chunk's states from its checkpoint into registers (lam_t, lam_t h_{t-1}, h_t)
//   B  adjoint G_t = gy_t C_t + lam_{t+1} G_{t+1} backwards through the chunk; per-lane partial
//      sums over states (sum_n A Q, sum_n G B) and the channel terms of grad B / grad C to LDS
//   -- barrier --
//   C  owners finish the chunk's per-(t, d) gradients; the channel sums of grad B / grad C
//      are written as this tile's partials
//   D  owners prepare the previous chunk's per-(t, d) scalars in LDS (its inputs were loaded
//      at the top of this iteration) and store grad z, which needs no recurrence
//   -- barrier --
template <typename TIO, int NS, int DT_>
__global__ void __launch_bounds__((BCfg<NS, DT_>::TH), (BCfg<NS, DT_>::OCC)) mamba_bwd_kernel(
    const TIO* __restrict__ draw, const float* __restrict__ A, const TIO* __restrict__ Bt,
    const TIO* __restrict__ Ct, const TIO* __restrict__ u, const TIO* __restrict__ z, const float* __restrict__ Dp,
    const float* __restrict__ h0, const float* __restrict__ saved, const TIO* __restrict__ gout,
    const float* __restrict__ ghlast, TIO* __restrict__ gdraw, TIO* __restrict__ gu, TIO* __restrict__ gz,
    float* __restrict__ gA_part, float* __restrict__ gDp_part, TIO* __restrict__ gBC_part, float* __restrict__ gh0,
    int64_t B, int64_t L, int64_t D, int N, int64_t NC, unsigned cus) {
  using C = BCfg<NS, DT_>;
  constexpr int NPT = C::NPT, NG = C::NG, DT = C::DT, TH = C::TH, CHK = C::CHK, IT = C::IT;
  constexpr int W2 = C::W2, NBV = C::NBV, NSL = C::NSL, RPG = C::RPG;
  // per (t, d): (delta, delta u) as an aligned pair, and gy in its own array. gy also weights
  // the channel sums of grad C, which read it after the chunk's adjoint while the next chunk's
  // values are being written: two copies by chunk parity. 52 KB in all at DT = 32, so that three
  // workgroups share a CU.
  __shared__ float2 s_dx[CHK][DT];
  __shared__ __align__(16) float s_gw[2][CHK][DT];
  __shared__ float s_np[CHK][2][NG][DT];             // (sum_n A Q, sum_n G B) per state group
  __shared__ __align__(16) float s_dp[CHK][W2][DT];  // per (step, column): the channels' (G du | h)

  const int tid = threadIdx.x;
  int64_t tile, b;
  xcd_remap((D + DT - 1) / DT, tile, b);
  const int64_t d0 = tile * DT;
  const int rw = tid >> 4, lk = tid & 15;
  const int ng = rw / RPG;
  const int dl = lk + 16 * (rw % RPG);
  const int64_t d = d0 + dl;
  const bool act = d < D;
  const int64_t rowD = b * L * D + d0, rowN = b * L * N;
  const uint32_t Du = (uint32_t)D, Nu = (uint32_t)N;

  float A2[NPT], Av[NPT], G[NPT], gA[NPT], lam_next[NPT];
  uint32_t co[NPT];  // offset of state j * NG + ng of this channel within one checkpoint slot [N, D]
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int n = j * NG + ng;
    const bool v = act && n < N;
    co[j] = (uint32_t)n * Du + (uint32_t)dl;
    Av[j] = v ? A[d * N + n] : 0.0f;
    A2[j] = Av[j] * kLog2e;
    G[j] = (v && ghlast) ? ghlast[(b * D + d) * N + n] : 0.0f;
    gA[j] = 0.0f;
    lam_next[j] = 1.0f;  // no step after the last one
  }
  float gdp = 0.0f;

  // Row streams through buffer resources (see make_rsrc): a per-lane byte offset fixed for the
  // whole walk plus a per-chunk SGPR offset. An inactive lane (channel or state beyond the tensor,
  // a padding slot) gets the resource's size as its offset, and steps past the end of the sequence
  // fall beyond it too, so their loads read 0 and their stores are dropped: no guarded copy of the
  // load code for partial tiles or the last chunk.
  constexpr uint32_t esz = sizeof(TIO);
  const uint32_t rowD_bytes = (uint32_t)((L * D - d0) * esz);  // [L, D] rows seen from channel d0
  const uint32_t rowN_bytes = (uint32_t)(L * N * esz);
  // saved state of this batch row: checkpoints [NC, N, D] then pre-gate outputs y [L, D]
  const float* __restrict__ svb = saved + b * saved_row_floats<TIO>(L, D, N, NC);
  const uint32_t chk_bytes = (uint32_t)((NC * N * D - d0) * 4);
  const Rsrc rs_dr = make_rsrc(draw + rowD, rowD_bytes), rs_u = make_rsrc(u + rowD, rowD_bytes);
  const Rsrc rs_z = make_rsrc(z + rowD, rowD_bytes), rs_go = make_rsrc(gout + rowD, rowD_bytes);
  const Rsrc rs_y = make_rsrc(reinterpret_cast<const TIO*>(svb + NC * N * D) + d0, rowD_bytes);
  const Rsrc rs_gd = make_rsrc(gdraw + rowD, rowD_bytes), rs_gu = make_rsrc(gu + rowD, rowD_bytes);
  const Rsrc rs_gz = make_rsrc(gz + rowD, rowD_bytes);
  const Rsrc rs_b = make_rsrc(Bt + rowN, rowN_bytes), rs_c = make_rsrc(Ct + rowN, rowN_bytes);
  const Rsrc rs_ck = make_rsrc(svb + d0, chk_bytes);
  const Rsrc rs_pt = make_rsrc(gBC_part + (tile * B + b) * L * W2, (uint32_t)(L * W2 * esz));  // [L, 2*NS] partials

  // owner items: item k of this thread is (t = idx / DT, channel d0 + idx % DT), idx = tid + k * TH
  float dp_o[IT];
  uint32_t ov[IT];  // byte offset of the item within a chunk of a [L, D] row
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int idx = tid + k * TH;
    const int od = idx % DT, t = idx / DT;
    const bool ok = d0 + od < D && ((CHK * DT) % TH == 0 || idx < CHK * DT);
    dp_o[k] = d0 + od < D ? Dp[d0 + od] : 0.0f;
    ov[k] = ok ? ((uint32_t)t * Du + (uint32_t)od) * esz : rowD_bytes;
  }
  // B/C broadcast slots of this lane: slot s = i * NPT + j -> (step i of the chunk, state j * NG + ng)
  uint32_t bco[NBV];
#pragma unroll
  for (int q = 0; q < NBV; ++q) {
    const int s = q * 16 + lk;
    const int n = (s % NPT) * NG + ng;
    const bool ok = n < N && (NSL % 16 == 0 || s < NSL);
    bco[q] = ok ? ((uint32_t)(s / NPT) * Nu + (uint32_t)n) * esz : rowN_bytes;
  }
  uint32_t cko[NPT];  // byte offset of this lane's states within a checkpoint slot
#pragma unroll
  for (int j = 0; j < NPT; ++j) cko[j] = (act && j * NG + ng < N) ? co[j] * 4u : chk_bytes;

  // inputs of one chunk, loaded at the top of the iteration that consumes them
  TIO r_dr[IT], r_u[IT], r_z[IT], r_go[IT], r_y[IT], r_bv[NBV], r_cv[NBV];
  float r_hs[NPT];
  auto load_chunk = [&](int64_t c) __attribute__((always_inline)) {
    const uint32_t t0 = (uint32_t)(c * CHK);
    const uint32_t sD = t0 * Du * esz, sN = t0 * Nu * esz;
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      r_dr[k] = buf_load<TIO>(rs_dr, ov[k], sD);
      r_u[k] = buf_load<TIO>(rs_u, ov[k], sD);
      r_z[k] = buf_load<TIO>(rs_z, ov[k], sD);
      r_go[k] = buf_load<TIO>(rs_go, ov[k], sD);
      r_y[k] = buf_load<TIO>(rs_y, ov[k], sD);
    }
#pragma unroll
    for (int q = 0; q < NBV; ++q) {
      r_bv[q] = buf_load<TIO>(rs_b, bco[q], sN);
      r_cv[q] = buf_load<TIO>(rs_c, bco[q], sN);
    }
    // state entering the chunk: checkpoint slot c-1, or h0 for the first chunk
    if (c > 0) {
      const uint32_t sC = (uint32_t)(c - 1) * (Nu * Du) * 4u;
#pragma unroll
      for (int j = 0; j < NPT; ++j) r_hs[j] = buf_load<float>(rs_ck, cko[j], sC);
    } else {
#pragma unroll
      for (int j = 0; j < NPT; ++j) {
        const int n = j * NG + ng;
        r_hs[j] = (h0 && act && n < N) ? h0[(b * D + d) * N + n] : 0.0f;
      }
    }
  };

  // per-(t, d) values the owner keeps from D to C: u, sigmoid(draw), delta, gy
  float o_u[IT], o_sd[IT], o_dl[IT], o_gy[IT];
  float bv[NBV], cv[NBV], hst[NPT];
  // D: the loaded chunk c's per-(t, d) scalars into LDS, grad z out, B/C and entering state into
  // their registers. Steps past the end of the sequence get delta = 0 and gy = 0 (identity steps
  // with no injected gradient), so the sweeps need no per-step guard; only stores check the length.
  auto prepare = [&](int64_t c) __attribute__((always_inline)) {
    const uint32_t t0 = (uint32_t)(c * CHK);
    const int wb = (int)(c & 1);
    const int64_t len = (L - (int64_t)t0) < CHK ? (L - (int64_t)t0) : CHK;
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      const int idx = tid + k * TH;
      if ((CHK * DT) % TH == 0 || idx < CHK * DT) {
        const int t = idx / DT, od = idx % DT;
        const bool live = d0 + od < D && t < len;
        const float xd = to_f32(r_dr[k]), uu = to_f32(r_u[k]), zz = to_f32(r_z[k]), go = to_f32(r_go[k]);
        // softplus as the reference writes it (mamba_triton.py:75-78): log(1 + e^x), x above 20
        // passed through; d softplus / d draw = e^x / (1 + e^x)
        const float e = fast_exp2(fminf(xd, 20.0f) * kLog2e);
        const float up = 1.0f + e;
        const float delta = live ? (xd > 20.0f ? xd : __builtin_amdgcn_logf(up) * kLn2) : 0.0f;
        const float sg = sigmoid_fast(zz);
        const float gyv = live ? go * zz * sg : 0.0f;
        o_u[k] = uu;
        o_sd[k] = e * __builtin_amdgcn_rcpf(up);
        o_dl[k] = delta;
        o_gy[k] = gyv;
        gdp = fmaf(gyv, uu, gdp);
        s_dx[t][od] = make_float2(delta, delta * uu);
        s_gw[wb][t][od] = gyv;
        buf_store(from_f32<TIO>(go * to_f32(r_y[k]) * sg * fmaf(zz, 1.0f - sg, 1.0f)), rs_gz, ov[k], t0 * Du * esz);
      }
    }
#pragma unroll
    for (int q = 0; q < NBV; ++q) {
      bv[q] = to_f32(r_bv[q]);
      cv[q] = to_f32(r_cv[q]);
    }
#pragma unroll
    for (int j = 0; j < NPT; ++j) hst[j] = r_hs[j];
  };

  if (NC > 0) {
    load_chunk(NC - 1);
    prepare(NC - 1);
  }
  __syncthreads();

  float lamb[CHK][NPT], lhb[CHK][NPT], hb[CHK][NPT];
  // The forward's issue-priority rotation among the workgroups sharing a CU (every 16 chunks =
  // 128 steps): without it the oldest workgroup races ahead and the last one finishes alone.
  const unsigned slot = blockIdx.x / cus;
  for (int64_t c = NC - 1; c >= 0; --c) {
    const int64_t r = NC - 1 - c;
    if (C::OCC > 1 && (r & 15) == 0) set_wave_priority((slot + (unsigned)(r / 16)) % C::OCC);
    const uint32_t t0 = (uint32_t)(c * CHK);
    const int wb = (int)(c & 1);
    // the previous chunk's inputs, consumed at the end of this iteration (D): loads issued and
    // used within one iteration, so no pending load is carried around the loop
    if (c > 0) load_chunk(c - 1);

    // A: recompute this chunk's states into registers: lam_t, lam_t h_{t-1} and h_t (the chunk's
    // (delta, delta u) stay in registers for B: one LDS read per step instead of two)
    float2 scb[CHK];
    {
      float hs[NPT];
#pragma unroll
      for (int j = 0; j < NPT; ++j) hs[j] = hst[j];
#pragma unroll
      for (int i = 0; i < CHK; ++i) {
        const float2 sc = s_dx[i][dl];
        scb[i] = sc;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
          const int s = i * NPT + j;
          const float lam = fast_exp2(sc.x * A2[j]);
          lamb[i][j] = lam;
          lhb[i][j] = lam * hs[j];
          hs[j] = fmaf(row_bcast(bv[s / 16], s % 16), sc.y, lhb[i][j]);
          hb[i][j] = hs[j];
        }
      }
    }
    // B: adjoint sweep backwards through the chunk
#pragma unroll
    for (int i = CHK - 1; i >= 0; --i) {
      const float2 sc = scb[i];  // (delta, delta * u), kept from A
      const float gyv = s_gw[wb][i][dl];
      float aq = 0.0f, gb = 0.0f;
#pragma unroll
      for (int j = 0; j < NPT; ++j) {
        const int s = i * NPT + j;
        const float an = (i + 1 < CHK) ? lamb[(i + 1) % CHK][j] : lam_next[j];
        G[j] = fmaf(an, G[j], row_bcast(cv[s / 16], s % 16) * gyv);
        const float Q = G[j] * lhb[i][j];  // G_t * lam_t h_{t-1}
        gA[j] = fmaf(sc.x, Q, gA[j]);
        aq = fmaf(Av[j], Q, aq);
        gb = fmaf(row_bcast(bv[s / 16], s % 16), G[j], gb);
        s_dp[i][j * NG + ng][dl] = G[j] * sc.y;
        s_dp[i][NS + j * NG + ng][dl] = TSF_MAMBA_BWD_HG ? hb[i][j] * gyv : hb[i][j];
      }
      s_np[i][0][ng][dl] = aq;
      s_np[i][1][ng][dl] = gb;
    }
#pragma unroll
    for (int j = 0; j < NPT; ++j) lam_next[j] = lamb[0][j];
    __syncthreads();

    // C: owners finish this chunk's per-(t, d) gradients
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      const int idx = tid + k * TH;
      const int t = idx / DT, od = idx % DT;
      if ((CHK * DT) % TH == 0 || idx < CHK * DT) {  // stores of steps past L or inactive channels drop
        float aqp[NG], gbp[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          aqp[g] = s_np[t][0][g][od];
          gbp[g] = s_np[t][1][g][od];
        }
        const float aq = tree_sum<NG>(aqp), gb = tree_sum<NG>(gbp);
        buf_store(from_f32<TIO>(fmaf(o_u[k], gb, aq) * o_sd[k]), rs_gd, ov[k], t0 * Du * esz);
        buf_store(from_f32<TIO>(fmaf(o_dl[k], gb, o_gy[k] * dp_o[k])), rs_gu, ov[k], t0 * Du * esz);
      }
    }
    // grad B_t / grad C_t: the tile's DT channels of each (t, column) summed, grad C's weighted
    // by the channel's gy (grad B's terms carry delta u already). Items are ordered grad B first,
    // so for NS >= 8 every wave takes one kind (no divergence). Each thread reads its row as DT/4
    // float4s starting at a column-dependent offset, so that the lanes of one b128 pass
    // (consecutive columns, rows a multiple of 128 B apart) hit distinct banks.
    for (int idx = tid; idx < CHK * W2; idx += TH) {
      const int half = idx / (CHK * NS), r = idx % (CHK * NS);
      const int ii = r / NS, c = r % NS, col = half * NS + c;
      const float4* row = reinterpret_cast<const float4*>(&s_dp[ii][col][0]);
      constexpr int NQ = DT / 4;
      float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (half == 0 || TSF_MAMBA_BWD_HG) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const float4 v = row[(q + (c >> 1)) % NQ];
          part[q & 3] += (v.x + v.y) + (v.z + v.w);
        }
      } else {
        const float4* wrow = reinterpret_cast<const float4*>(&s_gw[wb][ii][0]);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const int f = (q + (c >> 1)) % NQ;
          const float4 v = row[f], w = wrow[f];
          part[q & 3] = fmaf(v.x, w.x, fmaf(v.y, w.y, fmaf(v.z, w.z, fmaf(v.w, w.w, part[q & 3]))));
        }
      }
      // rows past the end of the sequence fall beyond the partials' resource
      buf_store(from_f32<TIO>((part[0] + part[1]) + (part[2] + part[3])), rs_pt,
                ((uint32_t)ii * W2 + (uint32_t)col) * esz, t0 * (uint32_t)W2 * esz);
    }
    // D: the previous chunk's inputs (loaded during this one) into place
    if (c > 0) prepare(c - 1);
    __syncthreads();
  }

  if (act) {
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if (j * NG + ng < N) gA_part[(b * D + d) * N + j * NG + ng] = gA[j];
  }
  // gh0 = lam_0 G_0 (lam_next now holds lam_0; an empty sequence passes the state through)
  if (gh0 && act) {
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if (j * NG + ng < N) gh0[(b * D + d) * N + j * NG + ng] = lam_next[j] * G[j];
  }
  // gDp: every owner thread of channel od holds a partial; sum them through LDS (in a fixed order)
  float* red = &s_dp[0][0][0];
  static_assert(CHK * W2 * DT >= TH, "reduction scratch too small");
  red[tid] = gdp;
  __syncthreads();
  if (tid < DT && d0 + tid < D) {
    float s = 0.0f;
    for (int k = tid; k < TH; k += DT) s += red[k];
    gDp_part[b * D + d0 + tid] = s;
  }
}

// gBt/gCt: sum the per-tile partials [nT, B, L, 2*NS] over the channel tiles, in order, in fp32.
template <typename TIO>
__global__ void __launch_bounds__(256) mamba_reduce_bc(const TIO* __restrict__ part, TIO* __restrict__ gBt,
                                                       TIO* __restrict__ gCt, int64_t nT, int64_t BL, int N,
                                                       int NS) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;  // over BL * N
  if (i >= BL * N) return;
  const int64_t row = i / N;
  const int n = (int)(i % N);
  float sb = 0.0f, sc = 0.0f;
  for (int64_t k = 0; k < nT; ++k) {
    const TIO* p = part + (k * BL + row) * (2 * NS);
    sb += to_f32(p[n]);
    sc += to_f32(p[NS + n]);
  }
  gBt[i] = from_f32<TIO>(sb);
  gCt[i] = from_f32<TIO>(sc);
}

// The same sum with 16-byte accesses when N == NS and a 16-byte vector holds whole columns of
// one kind (NS a multiple of V = 16 / sizeof(TIO)): thread (row, q) adds columns V q .. V q + V - 1
// of every tile's [2*NS] row, in tile order, and writes them to gBt (V q < NS) or gCt.
template <typename TIO>
TSF_DEV void reduce_bc_vec(const TIO* __restrict__ part, TIO* __restrict__ gBt, TIO* __restrict__ gCt, int64_t nT,
                           int64_t BL, int NS, unsigned block) {
  constexpr int V = 16 / sizeof(TIO);
  const int QR = 2 * NS / V;  // vectors per row
  const int64_t i = block * (int64_t)blockDim.x + threadIdx.x;  // over BL * QR
  if (i >= BL * QR) return;
  const int64_t row = i / QR;
  const int q = (int)(i % QR);
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  const uint4* src = reinterpret_cast<const uint4*>(part + row * 2 * NS) + q;
  const int64_t tstride = BL * 2 * NS / V;  // uint4 per tile
  for (int64_t k = 0; k < nT; ++k) {
    const uint4 w = src[k * tstride];
    const TIO* e = reinterpret_cast<const TIO*>(&w);
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] += to_f32(e[v]);
  }
  uint4 o;
  TIO* oe = reinterpret_cast<TIO*>(&o);
#pragma unroll
  for (int v = 0; v < V; ++v) oe[v] = from_f32<TIO>(acc[v]);
  const int c0 = q * V;
  TIO* dst = c0 < NS ? gBt + row * NS + c0 : gCt + row * NS + (c0 - NS);
  *reinterpret_cast<uint4*>(dst) = o;
}

// Sum [B, X] partials over the batch into [X] (gA with X = D*N, gDp with X = D), in batch order.
TSF_DEV void reduce_batch(const float* __restrict__ part, float* __restrict__ dst, int64_t B, int64_t X,
                          unsigned block) {
  const int64_t i = block * (int64_t)blockDim.x + threadIdx.x;
  if (i >= X) return;
  float s = 0.0f;
  for (int64_t b = 0; b < B; ++b) s += part[b * X + i];
  dst[i] = s;
}
__global__ void __launch_bounds__(256) mamba_reduce_batch(const float* __restrict__ part, float* __restrict__ dst,
                                                          int64_t B, int64_t X) {
  reduce_batch(part, dst, B, X, blockIdx.x);
}

// The backward's three sums in one launch (each a few microseconds of work, so the launches
// themselves were most of their time): blocks [0, nb_bc) the grad B_t / grad C_t sum over channel
// tiles (reduce_bc_vec), the next nb_a blocks grad A over the batch, the rest grad Dp.
template <typename TIO>
__global__ void __launch_bounds__(256) mamba_reduce_all(const TIO* __restrict__ part, TIO* __restrict__ gBt,
                                                        TIO* __restrict__ gCt, int64_t nT, int64_t BL, int NS,
                                                        unsigned nb_bc, const float* __restrict__ gA_part,
                                                        float* __restrict__ gA, const float* __restrict__ gDp_part,
                                                        float* __restrict__ gDp, int64_t B, int64_t XA, int64_t XD,
                                                        unsigned nb_a) {
  if (blockIdx.x < nb_bc) {
    reduce_bc_vec<TIO>(part, gBt, gCt, nT, BL, NS, blockIdx.x);
  } else if (blockIdx.x - nb_bc < nb_a) {
    reduce_batch(gA_part, gA, B, XA, blockIdx.x - nb_bc);
  } else {
    reduce_batch(gDp_part, gDp, B, XD, blockIdx.x - nb_bc - nb_a);
  }
}

template <typename TIO, int NS>
int launch_fwd(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
               const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, void* out,
               float* h_last, float* chk, hipStream_t s) {
  using C = FCfg<NS>;
  const int64_t NC = (L + C::CHK - 1) / C::CHK;
  dim3 grid((unsigned)((D + C::DT - 1) / C::DT * B));
  if (chk)
    hipLaunchKernelGGL((mamba_fwd_kernel<TIO, NS, true>), grid, dim3(C::TH), 0, s, (const TIO*)draw, A,
                       (const TIO*)Bt, (const TIO*)Ct, (const TIO*)u, (const TIO*)z, Dp, h0, (TIO*)out, h_last, chk, L,
                       D, (int)N, NC, device_cus());
  else
    hipLaunchKernelGGL((mamba_fwd_kernel<TIO, NS, false>), grid, dim3(C::TH), 0, s, (const TIO*)draw, A,
                       (const TIO*)Bt, (const TIO*)Ct, (const TIO*)u, (const TIO*)z, Dp, h0, (TIO*)out, h_last, chk, L,
                       D, (int)N, NC, device_cus());
  return tsf_launch_status();
}

// Channel tile of the backward. (A 96-channel tile, one 12-wave workgroup per CU with a third of
// the grad-B/C partials, measured 16% slower at config 3: with one workgroup per CU nothing runs
// while its waves wait at the chunk barriers.)
constexpr int kBwdDT = TSF_MAMBA_BWD_DT;
// From 32 states a launch takes 16-channel tiles: at 32 channels their per-chunk LDS (86 KB at
// N = 32) fits one workgroup per CU, one wave per SIMD; at 16 channels two (backward -13% at
// N = 32, -12% at N = 64 on config 3's B, L, D). At N = 16 the 32-channel tile stays faster
// (the narrower tile doubles the grad-B/C partials; +10%).
template <int NS>
constexpr int bwd_dt() {
  return NS >= 32 ? 16 : kBwdDT;
}

// Backward workspace: grad-B/C partials [nT, B, L, 2*NS] in the I/O type (padded to 256 bytes),
// then the fp32 per-row partials of gA [B, D, N] and gDp [B, D].
template <int NS>
int64_t bwd_partial_bytes(int64_t B, int64_t L, int64_t D, int64_t esz) {
  const int64_t nT = (D + bwd_dt<NS>() - 1) / bwd_dt<NS>();
  return (nT * B * L * 2 * NS * esz + 255) / 256 * 256;
}
template <int NS>
int64_t bwd_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t N, int64_t esz) {
  return bwd_partial_bytes<NS>(B, L, D, esz) + 4 * (B * D * N + B * D);
}

template <typename TIO, int NS, int DT>
void launch_bwd_tile(int64_t B, int64_t L, int64_t D, int64_t N, int64_t NC, const void* draw, const float* A,
                     const void* Bt, const void* Ct, const void* u, const void* z, const float* Dp, const float* h0,
                     const float* chk, const void* gout, const float* ghlast, void* gdraw, void* gu, void* gz,
                     float* gA_part, float* gDp_part, TIO* gBC_part, float* gh0, hipStream_t s) {
  using C = BCfg<NS, DT>;
  const int64_t nT = (D + DT - 1) / DT;
  hipLaunchKernelGGL((mamba_bwd_kernel<TIO, NS, DT>), dim3((unsigned)(nT * B)), dim3(C::TH), 0, s,
                     (const TIO*)draw, A, (const TIO*)Bt, (const TIO*)Ct, (const TIO*)u, (const TIO*)z, Dp, h0, chk,
                     (const TIO*)gout, ghlast, (TIO*)gdraw, (TIO*)gu, (TIO*)gz, gA_part, gDp_part, gBC_part, gh0, B,
                     L, D, (int)N, NC, device_cus());
}

template <typename TIO, int NS>
int launch_bwd(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
               const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, const float* chk,
               const void* gout, const float* ghlast, void* gdraw, float* gA, void* gBt, void* gCt, void* gu, void* gz,
               float* gDp, float* gh0, void* workspace, hipStream_t s) {
  using C = MCfg<NS>;
  const int64_t NC = (L + C::CHK - 1) / C::CHK;
  const int64_t nT = (D + bwd_dt<NS>() - 1) / bwd_dt<NS>();
  TIO* gBC_part = static_cast<TIO*>(workspace);
  float* gA_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + bwd_partial_bytes<NS>(B, L, D, sizeof(TIO)));
  float* gDp_part = gA_part + B * D * N;
  if (B > 0 && D > 0)
    launch_bwd_tile<TIO, NS, bwd_dt<NS>()>(B, L, D, N, NC, draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gu, gz,
                                     gA_part, gDp_part, gBC_part, gh0, s);
  const int64_t BLN = B * L * N;
  constexpr int V = 16 / sizeof(TIO);
  if (BLN > 0 && N == NS && NS % V == 0) {
    const int64_t items = B * L * (2 * NS / V);
    const unsigned nb_bc = (unsigned)((items + 255) / 256), nb_a = (unsigned)((D * N + 255) / 256),
                   nb_d = (unsigned)((D + 255) / 256);
    hipLaunchKernelGGL((mamba_reduce_all<TIO>), dim3(nb_bc + nb_a + nb_d), dim3(256), 0, s, gBC_part, (TIO*)gBt,
                       (TIO*)gCt, nT, B * L, NS, nb_bc, gA_part, gA, gDp_part, gDp, B, D * N, D, nb_a);
    return tsf_launch_status();
  }
  if (BLN > 0) {
    hipLaunchKernelGGL((mamba_reduce_bc<TIO>), dim3((unsigned)((BLN + 255) / 256)), dim3(256), 0, s, gBC_part,
                       (TIO*)gBt, (TIO*)gCt, nT, B * L, (int)N, NS);
  }
  if (D > 0) {
    hipLaunchKernelGGL(mamba_reduce_batch, dim3((unsigned)((D * N + 255) / 256)), dim3(256), 0, s, gA_part, gA, B,
                       D * N);
    hipLaunchKernelGGL(mamba_reduce_batch, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, s, gDp_part, gDp, B, D);
  }
  return tsf_launch_status();
}

#define TSF_DISPATCH_NS(NSV, FN, ...) \
  switch (NSV) {                      \
    case 4:                           \
      return FN<4>(__VA_ARGS__);      \
    case 8:                           \
      return FN<8>(__VA_ARGS__);      \
    case 16:                          \
      return FN<16>(__VA_ARGS__);     \
    case 32:                          \
      return FN<32>(__VA_ARGS__);     \
    case 64:                          \
      return FN<64>(__VA_ARGS__);     \
    default:                          \
      return TSF_ERR_UNSUPPORTED;     \
  }

template <int NS>
int fwd_f32(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
            const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, void* out, float* h_last,
            float* chk, hipStream_t s) {
  return launch_fwd<float, NS>(B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, out, h_last, chk, s);
}
template <int NS>
int fwd_bf16(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
             const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, void* out, float* h_last,
             float* chk, hipStream_t s) {
  return launch_fwd<bf16, NS>(B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, out, h_last, chk, s);
}
template <int NS>
int bwd_f32(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
            const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, const float* chk,
            const void* gout, const float* ghlast, void* gdraw, float* gA, void* gBt, void* gCt, void* gu, void* gz,
            float* gDp, float* gh0, void* ws, hipStream_t s) {
  return launch_bwd<float, NS>(B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gA, gBt, gCt, gu,
                               gz, gDp, gh0, ws, s);
}
template <int NS>
int bwd_bf16(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
             const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, const float* chk,
             const void* gout, const float* ghlast, void* gdraw, float* gA, void* gBt, void* gCt, void* gu, void* gz,
             float* gDp, float* gh0, void* ws, hipStream_t s) {
  return launch_bwd<bf16, NS>(B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gA, gBt, gCt, gu,
                              gz, gDp, gh0, ws, s);
}

// The kernels index one batch row with 32-bit byte offsets from a per-workgroup base, and the
// backward streams rows through buffer resources whose size is a signed 32-bit byte count: one
// batch row of every [B, L, *] tensor (fp32 at most, the last chunk's identity steps included),
// one batch row of the saved state (checkpoints [NC, N, D] and y [L, D]) and of the grad-B/C
// partials [L, 2*NS] must stay below 2 GiB. (mamba_hip.supports repeats this test.)
bool offsets_fit(int64_t L, int64_t D, int64_t N, int64_t chk_interval) {
  const int64_t lim = ((int64_t)1 << 31) / 4;  // fp32 elements
  const int64_t nc = (L + chk_interval - 1) / chk_interval;
  return (L + 64) * D < lim && (L + 64) * 2 * ns_for(N) < lim && nc * N * D + L * D < lim;
}

int chk_interval_for(int ns) {
  switch (ns) {
    case 4:
      return MCfg<4>::CHK;
    case 8:
      return MCfg<8>::CHK;
    case 16:
      return MCfg<16>::CHK;
    case 32:
      return MCfg<32>::CHK;
    case 64:
      return MCfg<64>::CHK;
    default:
      return 0;
  }
}

// The workspace for fp32 I/O, which also covers bf16 I/O (half-size partials).
int64_t workspace_bytes(int ns, int64_t B, int64_t L, int64_t D, int64_t N) {
  switch (ns) {
    case 4:
      return bwd_workspace_bytes<4>(B, L, D, N, 4);
    case 8:
      return bwd_workspace_bytes<8>(B, L, D, N, 4);
    case 16:
      return bwd_workspace_bytes<16>(B, L, D, N, 4);
    case 32:
      return bwd_workspace_bytes<32>(B, L, D, N, 4);
    case 64:
      return bwd_workspace_bytes<64>(B, L, D, N, 4);
    default:
      return -1;
  }
}

}  // namespace

extern "C" {

int64_t tsfast_hip_mamba_chk_interval(int64_t N) { return chk_interval_for(ns_for(N)); }

int64_t tsfast_hip_mamba_saved_floats(int64_t L, int64_t D, int64_t N, int io_dtype) {
  const int ns = ns_for(N);
  if (ns == 0 || N < 1 || L < 0 || D < 0) return -1;
  if (!offsets_fit(L, D, N, chk_interval_for(ns))) return -1;
  const int64_t nc = (L + chk_interval_for(ns) - 1) / chk_interval_for(ns);
  if (io_dtype == TSF_DTYPE_F32) return saved_row_floats<float>(L, D, N, nc);
  if (io_dtype == TSF_DTYPE_BF16) return saved_row_floats<bf16>(L, D, N, nc);
  return -1;
}

int64_t tsfast_hip_mamba_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t N) {
  const int ns = ns_for(N);
  if (ns == 0 || N < 1) return -1;
  return workspace_bytes(ns, B, L, D, N);
}

int tsfast_hip_mamba_fwd(int64_t B, int64_t L, int64_t D, int64_t N, int io_dtype, const void* draw, const float* A,
                         const void* Bt, const void* Ct, const void* u, const void* z, const float* Dp,
                         const float* h0, void* out, float* h_last, float* chk, void* stream) {
  if (B < 0 || L < 0 || D < 0 || N < 1) return TSF_ERR_ARG;
  if ((D + 31) / 32 * B > INT32_MAX) return TSF_ERR_UNSUPPORTED;  // one-dimensional grid
  const int ns = ns_for(N);
  if (ns == 0) return TSF_ERR_UNSUPPORTED;
  if (B == 0 || D == 0) return TSF_OK;
  if (!A || !Dp || !h_last) return TSF_ERR_ARG;
  if (L > 0 && (!draw || !Bt || !Ct || !u || !z || !out)) return TSF_ERR_ARG;
  if (!offsets_fit(L, D, N, chk_interval_for(ns))) return TSF_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (io_dtype == TSF_DTYPE_F32) {
    TSF_DISPATCH_NS(ns, fwd_f32, B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, out, h_last, chk, s)
  } else if (io_dtype == TSF_DTYPE_BF16) {
    TSF_DISPATCH_NS(ns, fwd_bf16, B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, out, h_last, chk, s)
  }
  return TSF_ERR_ARG;
}

int tsfast_hip_mamba_bwd(int64_t B, int64_t L, int64_t D, int64_t N, int io_dtype, const void* draw, const float* A,
                         const void* Bt, const void* Ct, const void* u, const void* z, const float* Dp,
                         const float* h0, const float* chk, const void* gout, const float* ghlast, void* gdraw,
                         float* gA, void* gBt, void* gCt, void* gu, void* gz, float* gDp, float* gh0, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  if (B < 0 || L < 0 || D < 0 || N < 1) return TSF_ERR_ARG;
  const int ns = ns_for(N);
  if (ns == 0) return TSF_ERR_UNSUPPORTED;
  const int64_t dt = ns >= 32 ? bwd_dt<32>() : kBwdDT;  // the backward's channel tile
  if ((D + dt - 1) / dt * B > INT32_MAX) return TSF_ERR_UNSUPPORTED;  // one-dimensional grid
  if (!A || !Dp || !gA || !gDp) return TSF_ERR_ARG;
  if (L > 0 && (!draw || !Bt || !Ct || !u || !z || !gout || !gdraw || !gBt || !gCt || !gu || !gz)) return TSF_ERR_ARG;
  if (h0 && !gh0) return TSF_ERR_ARG;
  if (L > 0 && !chk) return TSF_ERR_ARG;  // the saved state holds y as well as checkpoints
  if (workspace_bytes < tsfast_hip_mamba_workspace_bytes(B, L, D, N) || !workspace) return TSF_ERR_WORKSPACE;
  if (!offsets_fit(L, D, N, chk_interval_for(ns))) return TSF_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (io_dtype == TSF_DTYPE_F32) {
    TSF_DISPATCH_NS(ns, bwd_f32, B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gA, gBt, gCt,
                    gu, gz, gDp, gh0, workspace, s)
  } else if (io_dtype == TSF_DTYPE_BF16) {
    TSF_DISPATCH_NS(ns, bwd_bf16, B, L, D, N, draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gA, gBt, gCt,
                    gu, gz, gDp, gh0, workspace, s)
  }
  return TSF_ERR_ARG;
}

}  // extern "C"
