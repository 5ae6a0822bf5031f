// Shared building blocks of the all-pole scans (allpole.hip) and the fused dynoNet G-block
// (gblock.hip): the fp64 delay-line step, the [64 x 33] LDS transposition tiles for
// time-contiguous lanes, and the single-pass look-back machinery (transfer matrices, chunk and
// super-chunk maps, windowed look-back) with its tile plan.
// Included inside each file's anonymous namespace (after common.h and `using namespace tsf`).
#pragma once

constexpr int kMaxNA = 16;

#include "lookback.h"

// 1. M = C^{T_c} for the companion matrix C of lane `lane`: row 0 is (-a_1 .. -a_NA), row k is
//    the unit shift e_{k-1}. Stored row-major per lane.
inline dim3 grid_for(int64_t threads) { return dim3((unsigned)((threads + 255) / 256)); }

int64_t allpole_chunk(int64_t lanes, int64_t L, int64_t na) {
  if (L < 1) return 1;
  // one wave per (64-lane group, chunk): aim for ~4096 waves, chunks of at least 64 steps
  const int64_t groups = (lanes + 63) / 64;
  const int64_t target_waves = 4096;
  int64_t T_c = L;
  const int64_t min_len = na > 64 ? na : 64;
  while (T_c / 2 >= min_len && groups * ((L + T_c - 1) / T_c) < target_waves) T_c = (T_c + 1) / 2;
  return T_c;
}

// Streaming kernels: one wave owns 64 consecutive lanes x one time chunk. Time-contiguous rows
// are moved through a [64 x 33] LDS tile: the wave loads/stores 32-step row segments with
// coalesced 128-byte accesses, and each lane then walks its own row from LDS (the padding keeps
// the column walk conflict-free). The recurrence itself runs in fp64 registers.
constexpr int kTile = 64;   // lanes per wave (tile rows)
constexpr int kTileT = 32;  // time steps per tile (tile columns)

// rows [l0, l0+64) x columns [c0, c0+ncol) of a [lanes, L] matrix <-> tile (zero outside).
// Each access instruction moves two rows: lanes 0-31 one row, lanes 32-63 the next, 128-byte
// contiguous segments. Loads go to registers first (tile_fetch: all 32 issued back to back, so
// a whole tile is in flight at once) and into LDS afterwards (tile_put), which lets the next
// tile's loads overlap the current tile's recurrence.
struct TileRegs {
  float v[kTile / 2];
};
// `lid` is the thread's lane within its wave (the tile belongs to one wave).
// The row pointer starts from a per-thread base that passes through an empty asm and steps by two
// rows per access, so the compiler cannot hoist the 32 row addresses (64 VGPRs per matrix) out of
// a kernel's tile loop.
TSF_DEV void tile_fetch(TileRegs& rg, const float* __restrict__ src, int64_t lanes, int64_t L, int64_t l0, int64_t c0,
                        int ncol, int lid) {
  const int col = lid & (kTileT - 1), half = lid >> 5;
  const float* p = src + ((l0 + half) * L + c0 + col);
  asm volatile("" : "+v"(p));
  const bool cok = col < ncol;
#pragma unroll
  for (int r2 = 0; r2 < kTile / 2; ++r2) {
    const int64_t lane = l0 + 2 * r2 + half;
    rg.v[r2] = (lane < lanes && cok) ? *p : 0.0f;
    p += 2 * L;
  }
}
TSF_DEV void tile_put(const TileRegs& rg, float (*tile)[kTileT + 1], int lid) {
  const int col = lid & (kTileT - 1), half = lid >> 5;
#pragma unroll
  for (int r2 = 0; r2 < kTile / 2; ++r2) tile[2 * r2 + half][col] = rg.v[r2];
}
TSF_DEV void tile_store(float (*tile)[kTileT + 1], float* __restrict__ dst, int64_t lanes, int64_t L, int64_t l0,
                        int64_t c0, int ncol, int lid) {
  const int col = lid & (kTileT - 1), half = lid >> 5;
  float* p = dst + ((l0 + half) * L + c0 + col);
  asm volatile("" : "+v"(p));
#pragma unroll 8
  for (int r2 = 0; r2 < kTile / 2; ++r2) {
    const int r = 2 * r2 + half;
    const int64_t lane = l0 + r;
    if (lane < lanes && col < ncol) *p = tile[r][col];
    p += 2 * L;
  }
}

// One filter step on the register delay line: returns the new output and shifts it in.
// The oldest taps are accumulated first so that only the last FMA (with y_{t-1}) sits on the
// step-to-step dependency chain.
template <int NA>
TSF_DEV double step(const double (&av)[NA], double (&s)[NA], double x) {
  double acc = x;
#pragma unroll
  for (int k = NA - 1; k >= 0; --k) acc = fma(-av[k], s[k], acc);
#pragma unroll
  for (int k = NA - 1; k > 0; --k) s[k] = s[k - 1];
  s[0] = acc;
  return acc;
}

// ---------------------------------------------------------------- single-pass path, NA <= kLbNA
// For low orders the forward and backward are single-pass kernels with a decoupled look-back
// between workgroups (the protocol of lookback.h), so every input element is read once from HBM.
// A tile is 64 lanes x one super-chunk of K x 32 steps; wave k of the workgroup owns the k-th
// 32-step chunk: it moves the chunk through its own [64 x 33] LDS tile into registers (each
// thread then holds 32 values of its lane's row), summarises it from a zero state, and re-runs
// it from its true entering state once that is known. A chunk maps its entering state s to
// Mc s + e (Mc = C^32), a super-chunk to Ms s + e (Ms = C^(32 K)); both matrices come from
// allpole_transfer2. Only the e vectors are published: agg = a super-chunk's e from a zero
// state, inc = the state leaving it. A published vector may hold NV independent states of the
// same dynamics (NV blocks of NA, each mapped by the same matrices). Between the tile's barriers
// a wave's LDS tile is reused as two fp64 areas of up to 2 kLbNA values per lane: vec (chunk
// summary -> entering state -> partial sums) and slot (its look-back window entry).
constexpr int kLbNA = 4;     // highest order on the single-pass path (matrices stay in registers)
#ifndef TSF_AP_KMAX
#define TSF_AP_KMAX 8
#endif
constexpr int kLbWaves = TSF_AP_KMAX;  // chunks per tile at most (sizes the LDS of a workgroup)

using LdsTile = float[kTile][kTileT + 1];

template <int NA>
TSF_DEV double* vec_area(LdsTile* lds, int wv) {
  return reinterpret_cast<double*>(&lds[wv][0][0]);
}
template <int NA>
TSF_DEV double* slot_area(LdsTile* lds, int wv) {
  return reinterpret_cast<double*>(&lds[wv][0][0]) + 64 * 2 * kLbNA;
}
static_assert(64 * 4 * kLbNA * sizeof(double) <= sizeof(LdsTile), "vec and slot areas fit in a wave's tile");

template <int NA>
TSF_DEV void load_mat(double (&m)[NA][NA], const double* __restrict__ src) {
#pragma unroll
  for (int r = 0; r < NA; ++r)
#pragma unroll
    for (int c = 0; c < NA; ++c) m[r][c] = src[r * NA + c];
}
template <int NA>
TSF_DEV void matvec_add(double (&out)[NA], const double (&m)[NA][NA], const double (&x)[NA], const double (&b)[NA]) {
  double t[NA];
#pragma unroll
  for (int r = 0; r < NA; ++r) {
    double acc = b[r];
#pragma unroll
    for (int c = 0; c < NA; ++c) acc = fma(m[r][c], x[c], acc);
    t[r] = acc;
  }
#pragma unroll
  for (int r = 0; r < NA; ++r) out[r] = t[r];
}

// y = C x for the companion matrix C of a (row 0 = -a, ones on the subdiagonal), in fp64. The sum
// starts from the oldest entry, so only its last FMA waits on the previous step's new entry x[0]:
// a chain of steps costs one FMA latency per step.
template <int NA>
TSF_DEV void companion_apply(double (&x)[NA], const double (&a)[NA]) {
  double y0 = 0.0;
#pragma unroll
  for (int c = NA - 1; c >= 0; --c) y0 = fma(-a[c], x[c], y0);
#pragma unroll
  for (int r = NA - 1; r > 0; --r) x[r] = x[r - 1];
  x[0] = y0;
}

// The value x holds in lane K (0..15) of this thread's 16-lane DPP row (row_newbcast: every lane
// of the row reads lane K; an fp64 value moves as two 32-bit halves).
template <int K>
TSF_DEV uint32_t row_lane_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x150 + K, 0xF, 0xF, true);
}
template <int K>
TSF_DEV double row_lane(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint64_t lo = row_lane_u32<K>((uint32_t)b), hi = row_lane_u32<K>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)((hi << 32) | lo));
}
template <int K>
TSF_DEV float row_lane(float x) {
  return __uint_as_float(row_lane_u32<K>(__float_as_uint(x)));
}

// a0 + a1 + sum_{c < N} m[c] * (s of row lane c): one matrix row times a state vector spread over
// a 16-lane DPP row (component c in lane c), in two interleaved partial sums so that consecutive
// FMAs do not wait on each other. Called by all 16 lanes of the row together.
template <int N, int C = 0>
TSF_DEV void row_dot2(const double (&m)[N], double s, double& a0, double& a1) {
  if constexpr (C < N) {
    if constexpr (C % 2 == 0) {
      a0 = fma(m[C], row_lane<C>(s), a0);
    } else {
      a1 = fma(m[C], row_lane<C>(s), a1);
    }
    row_dot2<N, C + 1>(m, s, a0, a1);
  }
}

// Column `col` of both transfer matrices of one companion matrix (row 0 = -arow): Mc = C^32 and
// Ms = C^(32 K), row-major NA x NA each. The column is C applied step by step to the unit vector
// e_col in fp64: repeated squaring would compound rounding errors through the transient growth of
// the powers of a non-normal C (poles near the unit circle), step-by-step application keeps them
// at the level of the recurrence itself. One thread per column keeps the dependent chain short.
template <int NA>
TSF_DEV void companion_powers_col(const float* __restrict__ arow, double* __restrict__ Mc_out,
                                  double* __restrict__ Ms_out, int K, int col) {
  double a[NA], x[NA];
#pragma unroll
  for (int c = 0; c < NA; ++c) {
    a[c] = (double)arow[c];
    x[c] = c == col ? 1.0 : 0.0;
  }
  // 32-step blocks, unrolled: each step waits on one FMA (the newest state's term), and the
  // others are scheduled around it
  for (int blk = 0; blk < K; ++blk) {
#pragma unroll
    for (int step = 0; step < 32; ++step) companion_apply<NA>(x, a);
    if (blk == 0)
#pragma unroll
      for (int r = 0; r < NA; ++r) Mc_out[r * NA + col] = x[r];
  }
#pragma unroll
  for (int r = 0; r < NA; ++r) Ms_out[r * NA + col] = x[r];
}

// Both transfer matrices per lane ([lanes][NA][NA] each), a [lanes, NA].
// One thread per (lane, column); the last rj.blocks workgroups run the scan's look-back reset.
template <int NA>
__global__ void __launch_bounds__(64) allpole_transfer2(const float* __restrict__ a, double* __restrict__ Mc,
                                                        double* __restrict__ Ms, int64_t lanes, int K, ResetJob rj) {
  const unsigned tb = gridDim.x - rj.blocks;
  if (blockIdx.x >= tb) {
    run_reset(rj, blockIdx.x - tb);
    return;
  }
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (idx >= lanes * NA) return;
  const int64_t lane = idx / NA;
  companion_powers_col<NA>(a + lane * NA, Mc + lane * NA * NA, Ms + lane * NA * NA, K, (int)(idx - lane * NA));
}
inline dim3 transfer_grid(int64_t lanes, int na) { return dim3((unsigned)((lanes * na + 63) / 64)); }

template <int NA>
TSF_DEV bool get_vec(const double* __restrict__ p, double (&x)[NA]) {
  bool ok = true;
#pragma unroll
  for (int q = 0; q < NA; ++q) ok = get_word(p + q, x[q]) && ok;
  return ok;
}
template <int NA>
TSF_DEV void put_vec(double* p, const double (&x)[NA]) {
#pragma unroll
  for (int q = 0; q < NA; ++q) put_word(p + q, x[q]);
}

// State entering a super-chunk (result in wave 0's lanes), by looking back over the super-chunks
// before it in scan order: pos0 is the nearest, dj the step away from it; the words of slot r of
// a lane are at (r * lanes + lane) * NA. Called by every thread of the workgroup (it holds
// barriers). Wave 0 first probes the nearest inc. Pending lanes then go through rounds in which
// wave w reads slot pos0 + w dj (its inc, else its agg) into its slot area, and wave 0 looks for
// an inc at some slot w* with published aggs at every slot before it: the entering state is then
// Horner's rule back from that inc (s <- Ms s + agg). Otherwise the round is repeated. Every
// wait ends: the nearest super-chunk publishes its inc once its own look-back ends, and the first
// one in scan order publishes its inc without looking back (the window never has to move); a
// lane without progress for spin_max rounds gives up with NaN.
// out = m x + b applied to each of the NV blocks of NA values.
template <int NA, int NV>
TSF_DEV void block_matvec_add(double (&out)[NA * NV], const double (&m)[NA][NA], const double (&x)[NA * NV],
                              const double (&b)[NA * NV]) {
  double t[NA * NV];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int r = 0; r < NA; ++r) {
      double acc = b[v * NA + r];
#pragma unroll
      for (int c = 0; c < NA; ++c) acc = fma(m[r][c], x[v * NA + c], acc);
      t[v * NA + r] = acc;
    }
#pragma unroll
  for (int r = 0; r < NA * NV; ++r) out[r] = t[r];
}

template <int NA, int NV = 1>
TSF_DEV void ap_look_back(double (&S)[NA * NV], const double* __restrict__ agg, const double* __restrict__ inc,
                          const double* __restrict__ MsLane, bool need, int64_t pos0, int64_t dj, int64_t nsuper,
                          int64_t lanes, int64_t lane, int K, int k, int lid, LdsTile* lds, int (*flag)[64],
                          int* pend_s, int* any_s, unsigned* __restrict__ lb_counter, uint32_t spin_max) {
  constexpr int V = NA * NV;
  uint32_t spins = 0;
  if (k == 0) {
    int p = 0;
    if (need) {
      double x[V];
      if (get_vec<V>(inc + (pos0 * lanes + lane) * V, x)) {
#pragma unroll
        for (int q = 0; q < V; ++q) S[q] = x[q];
      } else {
        p = 1;
      }
    }
    pend_s[lid] = p;
    const bool any = __any(p != 0);
    if (lid == 0) *any_s = any ? 1 : 0;
  }
  __syncthreads();
  while (*any_s) {
    if (pend_s[lid]) {
      const int64_t r = pos0 + dj * k;
      int f = 0;
      double* sl = slot_area<NA>(lds, k) + lid * V;
      if (r >= 0 && r < nsuper) {
        double xi[V], xa[V];
        const bool hi = get_vec<V>(inc + (r * lanes + lane) * V, xi);
        const bool ha = get_vec<V>(agg + (r * lanes + lane) * V, xa);
        if (hi || ha) {
          f = hi ? 2 : 1;
#pragma unroll
          for (int q = 0; q < V; ++q) sl[q] = hi ? xi[q] : xa[q];
        }
      }
      flag[k][lid] = f;
    }
    __syncthreads();
    if (k == 0) {
      bool pending = false;
      if (pend_s[lid]) {
        int w = 0;
        for (; w < K; ++w)
          if (flag[w][lid] != 1) break;
        if (w < K && flag[w][lid] == 2) {
          double ms[NA][NA];
          load_mat<NA>(ms, MsLane);
          const double* sw = slot_area<NA>(lds, w) + lid * V;
#pragma unroll
          for (int q = 0; q < V; ++q) S[q] = sw[q];
          for (int v = w - 1; v >= 0; --v) {
            double ag[V];
            const double* sv = slot_area<NA>(lds, v) + lid * V;
#pragma unroll
            for (int q = 0; q < V; ++q) ag[q] = sv[q];
            block_matvec_add<NA, NV>(S, ms, S, ag);
          }
        } else if (++spins > spin_max) {
#pragma unroll
          for (int q = 0; q < V; ++q) S[q] = quiet_nan<double>();
          lb_gave_up(lb_counter);
        } else {
          pending = true;
        }
        pend_s[lid] = pending ? 1 : 0;
      }
      const bool any = __any(pending);
      if (lid == 0) *any_s = any ? 1 : 0;
    }
    __syncthreads();
  }
}

// Transfer matrices of a tile's 64 lanes, staged in LDS by the whole workgroup when the tile
// starts (the loads overlap the chunk loads): wave 0's folds, its look-back and the inclusive
// map then read them from LDS instead of waiting on global memory three times in a row. Mc and
// Ms of 64 consecutive lanes are contiguous blocks of [lanes][n][n]. States up to 3 fit next to
// the tiles with two workgroups per CU; n = 4 reads them from global memory. (n is the order,
// or the state size of a dense recurrence.)
template <int NS>
struct MatStage {
  static constexpr bool kLds = NS <= 3;
  static constexpr int kDoubles = kLds ? 2 * 64 * NS * NS : 1;
};
template <int NS>
TSF_DEV void stage_mats(double* s_mat, const double* __restrict__ Mc, const double* __restrict__ Ms, int64_t l0,
                        int64_t lanes) {
  constexpr int NN = NS * NS;
  const int64_t valid = ((lanes - l0) < 64 ? (lanes - l0) : 64) * NN;
  for (int e = threadIdx.x; e < 2 * 64 * NN; e += blockDim.x) {
    const int h = e >= 64 * NN, q = e - h * 64 * NN;
    s_mat[e] = q < valid ? (h ? Ms : Mc)[l0 * NN + q] : 0.0;
  }
}

// Loads the chunk [t0, t0 + n) of the wave's 64 rows through its LDS tile into xb (this
// thread's row). Cooperative over the wave.
TSF_DEV void chunk_to_regs(float (&xb)[kTileT], const float* __restrict__ src, int64_t lanes, int64_t L, int64_t l0,
                           int64_t t0, int n, float (*tile)[kTileT + 1], int lid) {
  TileRegs rg;
  tile_fetch(rg, src, lanes, L, l0, t0, n, lid);
  tile_put(rg, tile, lid);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < kTileT; ++i) xb[i] = tile[lid][i];
  __builtin_amdgcn_wave_barrier();
}

// Stores xb (this thread's row) as the chunk [t0, t0 + n) of the wave's 64 rows, through its LDS
// tile. Cooperative over the wave.
TSF_DEV void regs_to_chunk(const float (&xb)[kTileT], float* __restrict__ dst, int64_t lanes, int64_t L, int64_t l0,
                           int64_t t0, int n, float (*tile)[kTileT + 1], int lid) {
#pragma unroll
  for (int i = 0; i < kTileT; ++i) tile[lid][i] = xb[i];
  __builtin_amdgcn_wave_barrier();
  tile_store(tile, dst, lanes, L, l0, t0, n, lid);
  __builtin_amdgcn_wave_barrier();
}

// Tile plan of the single-pass path: K (chunks per tile) starts at kLbWaves and halves down to 2
// while there are fewer than kApTileTarget tiles. Workspace: the tile counter, agg and inc
// [nsuper][lanes][NA] (reset before each scan), the grad_a partials [nsuper][lanes][NA], and
// the transfer matrices Mc, Ms [lanes][NA][NA].
#ifndef TSF_AP_TILE_TARGET
#define TSF_AP_TILE_TARGET 256
#endif
constexpr int64_t kApTileTarget = TSF_AP_TILE_TARGET;

struct LbPlan {
  int64_t groups = 0, nsuper = 0;
  int K = 1;
  size_t off_agg = 0, off_inc = 0, off_part = 0, off_Mc = 0, off_Ms = 0, bytes = 0;
};

LbPlan lb_plan(int64_t lanes, int64_t L, int64_t na) {
  LbPlan p;
  p.groups = (lanes + kTile - 1) / kTile;
  if (L > 0) {
    p.K = kLbWaves;
    auto tiles = [&](int K) { return p.groups * ((L + (int64_t)kTileT * K - 1) / ((int64_t)kTileT * K)); };
    while (p.K > 2 && tiles(p.K) < kApTileTarget) p.K /= 2;
    const int64_t chunks = (L + kTileT - 1) / kTileT;
    if (p.K > chunks) p.K = (int)chunks;
    p.nsuper = (L + (int64_t)kTileT * p.K - 1) / ((int64_t)kTileT * p.K);
  }
  const size_t f = 8, vecs = f * p.nsuper * lanes * na;
  p.off_agg = kCounterBytes;
  p.off_inc = p.off_agg + vecs;
  p.off_part = p.off_inc + vecs;
  p.off_Mc = p.off_part + vecs;
  p.off_Ms = p.off_Mc + f * lanes * na * na;
  p.bytes = p.off_Ms + f * lanes * na * na;
  return p;
}

