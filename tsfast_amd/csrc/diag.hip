// Diagonal linear-recurrence scans on the lane layout [M, L, N] (N contiguous):
//   constant coefficient  x_t = lam * x_{t-1} + v_t            (lam [M, N], real or complex)
//   time-varying          x_t = a_t * x_{t-1} + v_t            (a   [M, L, N], real)
// and their adjoints G_t = g_t + conj(c_{t+1}) G_{t+1}.
//
// Reference semantics: tsfast/models/_core/scan.py:100-215 (ops), :52-80 (doubling scans),
// scan_backends/diagonal_triton.py:82-228 and selective_triton.py:48-109 (kernels).
//
// Both are single-pass scans with decoupled look-back: every input element is read once and every
// output element written once. A tile (one workgroup of K waves) covers 64 consecutive lanes by
// one super-chunk of K * TC consecutive steps; consecutive threads own consecutive lanes, so
// every per-step load/store of a wave is one coalesced row segment along N, and each wave keeps
// its TC-step chunk in registers. A tile summarises its chunks from a zero state, composes the
// summaries in LDS into its super-chunk's affine map, publishes that map, obtains the state
// entering the super-chunk from the tiles before it (look-back), publishes the state leaving
// it, and re-runs its chunks from registers. Carries are fp64 (complex128). Workgroups are
// persistent and take tiles in scan order from a counter.
#include <atomic>
#include <mutex>

#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

// All kernels load fp32 (or complex64) and carry the recurrence in fp64 (complex128): W below.
constexpr int kMaxWaves = 16;
constexpr unsigned kXcds = 8;  // XCDs of an MI355X, each with its own L2

// ---------------------------------------------------------------- affine maps and look-back
template <typename W>
struct Map {  // x -> P x + e
  W P, e;
};
template <typename W>
TSF_DEV Map<W> then(Map<W> first, Map<W> second) {  // apply `first`, then `second`
  return {Num<W>::mul(second.P, first.P), Num<W>::fma(second.P, first.e, second.e)};
}
template <typename W>
TSF_DEV W apply(Map<W> m, W x) {
  return Num<W>::fma(m.P, x, m.e);
}

#include "lookback.h"

template <typename W>
TSF_DEV void put(Map<W>* p, Map<W> m) {
  put(&p->P, m.P);
  put(&p->e, m.e);
}
template <typename W>
TSF_DEV bool get(const Map<W>* p, Map<W>& m) {
  const bool a = get(&p->P, m.P);
  const bool b = get(&p->e, m.e);
  return a && b;
}

constexpr int kWindow = kMaxWaves;  // look-back slots examined per round


// State entering a tile, found by looking back over the tiles before it in scan order. Called
// by every thread of the workgroup (it holds barriers) with a workgroup-uniform decision to call
// it; `need` marks the lanes (of wave 0) that look back, starting at super-chunk `pos0` and
// stepping by dj; slot r of a lane is at r * lanes + lane. Wave 0 first probes slot pos0 alone.
// Lanes that are still pending then go through rounds: the K waves read the kWindow slots pos,
// pos + dj, ... of every pending lane (inc and agg words together; slot w by wave w mod K) into
// LDS, and wave 0 walks the window in order. A published inc (state leaving that tile) ends the
// lane's walk, a published agg (that tile's map from a zero start) is composed and the walk
// moves on, an unpublished slot ends the round (the next round starts there). The walk always
// ends: the first tile in scan order publishes its inc without looking back, and every tile
// waited on was taken from the counter earlier by a workgroup that is running; a lane that
// makes no progress for spin_max rounds gives up with NaN. Returns the entering state in wave
// 0's lanes. LDS: win/flag [kWindow][64], pos [64] and one flag word, owned by the caller.
template <typename W>
TSF_DEV W look_back(const Map<W>* __restrict__ agg, const W* __restrict__ inc, bool need, int64_t pos0, int64_t dj,
                    int64_t nsuper, int64_t lanes, int64_t lane, int K, int k, int lid, Map<W> (*win)[64],
                    int (*flag)[64], int64_t* pos_s, int* any_s, unsigned* __restrict__ lb_counter,
                    uint32_t spin_max) {
  Map<W> acc = {Num<W>::one(), Num<W>::zero()};  // composition of the aggregates walked over
  W result = Num<W>::zero();
  uint32_t spins = 0;
  if (k == 0) {
    // direct probe of the nearest tile by wave 0: in the steady state of a long scan its inc is
    // already published, and the window rounds below are skipped
    int64_t p = -1;
    if (need) {
      W x;
      Map<W> m;
      const bool have_inc = get(inc + pos0 * lanes + lane, x);
      const bool have_agg = get(agg + pos0 * lanes + lane, m);
      if (have_inc) {
        result = x;
      } else if (have_agg) {  // never the first tile in scan order, which publishes no agg
        acc = m;
        p = pos0 + dj;
      } else {
        p = pos0;
      }
    }
    pos_s[lid] = p;
    const bool any = __any(p >= 0);
    if (lid == 0) *any_s = any ? 1 : 0;
  }
  __syncthreads();
  while (*any_s) {
    const int64_t pos = pos_s[lid];
    if (pos >= 0) {
      for (int w = k; w < kWindow; w += K) {
        const int64_t r = pos + dj * w;
        int f = 0;
        Map<W> m = {Num<W>::zero(), Num<W>::zero()};
        if (r >= 0 && r < nsuper) {
          W x;
          const bool have_inc = get(inc + r * lanes + lane, x);
          const bool have_agg = get(agg + r * lanes + lane, m);
          if (have_inc) {
            f = 2;
            m.e = x;
          } else if (have_agg) {
            f = 1;
          }
        }
        flag[w][lid] = f;
        win[w][lid] = m;
      }
    }
    __syncthreads();
    if (k == 0) {
      bool pending = false;
      if (pos >= 0) {
        int64_t p = pos;
        int w = 0;
        for (; w < kWindow; ++w) {
          const int f = flag[w][lid];
          if (f == 2) {
            result = apply(acc, win[w][lid].e);
            p = -1;
            break;
          }
          if (f != 1) break;
          acc = then(win[w][lid], acc);
          p += dj;
        }
        if (p >= 0 && w == 0 && ++spins > spin_max) {
          result = quiet_nan<W>();
          lb_gave_up(lb_counter);
          p = -1;
        }
        pending = p >= 0;
        pos_s[lid] = p;
      }
      const bool any = __any(pending);
      if (lid == 0) *any_s = any ? 1 : 0;
    }
    __syncthreads();
  }
  return result;
}


// ---------------------------------------------------------------- constant coefficient
// One tile = 64 lanes x one super-chunk of K * TC steps (K waves of TC-step chunks). Tile index
// `tile` is super-chunk tile / groups (forward from the left, backward from the right) of lane
// group tile % groups. Per tile: every wave loads its chunk (all loads issued at once) and
// summarises it from a zero state; wave 0 composes the K summaries into the super-chunk's map,
// publishes it, looks back for the state entering the super-chunk, publishes the state leaving
// it and writes the state entering each chunk to LDS; every wave then re-runs its chunk from
// registers. Each wave reads only its own slot of s_start after the second barrier, so the next
// tile's first writes (before its first barrier) cannot race with a slower wave's reads.
template <typename T, int TC>
__global__ void __launch_bounds__(1024) diag_fwd(const T* __restrict__ lam, const T* __restrict__ v,
                                                 const T* __restrict__ x0, T* __restrict__ out,
                                                 Map<typename Wide<T>::type>* __restrict__ agg,
                                                 typename Wide<T>::type* __restrict__ inc, unsigned* __restrict__ counter,
                                                 int64_t lanes, int64_t L, int64_t N, int64_t groups, int K,
                                                 int64_t nsuper, LbCfg lb_spacing) {
  using W = typename Wide<T>::type;
  __shared__ W s_e[kMaxWaves][64];
  // the look-back window, then (once the look-back is done) the state entering each chunk
  __shared__ Map<W> s_win[kMaxWaves][64];
  __shared__ int s_flag[kMaxWaves][64];
  __shared__ int64_t s_pos[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  W(*s_start)[64] = reinterpret_cast<W(*)[64]>(&s_win[0][0]);
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * TC;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t sc = tile / groups, lane = (tile - sc * groups) * 64 + lid;
    const bool live = lane < lanes;
    const int64_t t0 = sc * SL + (int64_t)k * TC;
    const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
    W a = Num<W>::zero(), e = Num<W>::zero();
    T vb[TC];
    int64_t base = 0;
    if (live) {
      a = Wide<T>::up(lam[lane]);
      const int64_t m = lane / N, n = lane - m * N;
      base = (m * L + t0) * N + n;
      const T* vp = v + base;
      if (len == TC) {
#pragma unroll
        for (int i = 0; i < TC; ++i) vb[i] = vp[i * N];
#pragma unroll
        for (int i = 0; i < TC; ++i) e = Num<W>::fma(a, e, Wide<T>::up(vb[i]));
      } else {
#pragma unroll
        for (int i = 0; i < TC; ++i)
          if (i < len) vb[i] = vp[i * N];
#pragma unroll
        for (int i = 0; i < TC; ++i)
          if (i < len) e = Num<W>::fma(a, e, Wide<T>::up(vb[i]));
      }
    }
    s_e[k][lid] = e;
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    // chunks before a non-empty one are full, so lam^TC is every fold's multiplier; the
    // super-chunk map is published only for full super-chunks (all but the last)
    const W Pc = ipow(a, TC);
    Map<W> sup = {ipow(Pc, K), Num<W>::zero()};
    if (k == 0 && live) {
      sup.e = s_e[0][lid];
      for (int j = 1; j < K; ++j) sup.e = Num<W>::fma(Pc, sup.e, s_e[j][lid]);
      if (lb_pub_agg(sc, lb_spacing) && sc + 1 < nsuper) put(agg + sc * lanes + lane, sup);
    }
    W s = x0 && live && k == 0 ? Wide<T>::up(x0[lane]) : Num<W>::zero();
    if (sc > 0)  // uniform over the workgroup
      s = look_back(agg, inc, k == 0 && live, sc - 1, (int64_t)-1, nsuper, lanes, lane, K, k, lid, s_win, s_flag,
                    s_pos, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(sc, lb_spacing) && sc + 1 < nsuper) put(inc + sc * lanes + lane, apply(sup, s));
      for (int j = 0; j < K; ++j) {
        s_start[j][lid] = s;
        s = Num<W>::fma(Pc, s, s_e[j][lid]);
      }
    }
    __syncthreads();
    if (live && len > 0) {
      W s = s_start[k][lid];
      T* op = out + base;
      if (len == TC) {
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          s = Num<W>::fma(a, s, Wide<T>::up(vb[i]));
          op[i * N] = Wide<T>::down(s);
        }
      } else {
#pragma unroll
        for (int i = 0; i < TC; ++i)
          if (i < len) {
            s = Num<W>::fma(a, s, Wide<T>::up(vb[i]));
            op[i * N] = Wide<T>::down(s);
          }
      }
    }
  }
}

// Backward: G_t = g_t + conj(lam) G_{t+1} from the right end; gv = G, gx0 = conj(lam) G_0, and
// glam = sum_t G_t conj(x_{t-1}) reduced over the K chunks in LDS and over super-chunks by
// diag_sum_parts (fixed order, deterministic). Chunks past the end of the sequence are empty and
// contribute zero, so conj(lam)^TC is the right multiplier for every fold.
template <typename T, int TC>
__global__ void __launch_bounds__(1024) diag_bwd(const T* __restrict__ lam, const T* __restrict__ g,
                                                 const T* __restrict__ out, const T* __restrict__ x0,
                                                 Map<typename Wide<T>::type>* __restrict__ agg,
                                                 typename Wide<T>::type* __restrict__ inc, unsigned* __restrict__ counter,
                                                 T* __restrict__ gv, typename Wide<T>::type* __restrict__ part,
                                                 T* __restrict__ glam, T* __restrict__ gx0, int64_t lanes, int64_t L,
                                                 int64_t N, int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  using W = typename Wide<T>::type;
  __shared__ W s_f[kMaxWaves][64];
  // the look-back window, then G entering each chunk from the right (s_start) and the glam
  // partials of the chunks (s_acc)
  __shared__ Map<W> s_win[kMaxWaves][64];
  __shared__ int s_flag[kMaxWaves][64];
  __shared__ int64_t s_pos[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  W(*s_start)[64] = reinterpret_cast<W(*)[64]>(&s_win[0][0]);
  W(*s_acc)[64] = s_start + kMaxWaves;
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * TC;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t r = tile / groups, sc = nsuper - 1 - r, lane = (tile - r * groups) * 64 + lid;
    const bool live = lane < lanes;
    const int64_t t0 = sc * SL + (int64_t)k * TC;
    const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
    // With R the G entering the chunk from the right, G_t = G0_t + c^(t_end - t) R (c = conj(lam),
    // G0 the chunk's scan from zero), so the chunk's glam partial is A + R B with
    // A = sum_t G0_t conj(x_{t-1}) = sum_s g_s H_s, H_s = c H_{s-1} + conj(x_{s-1}) (H before the
    // chunk = 0), and B = sum_t c^(t_end - t) conj(x_{t-1}) = c H_last. Everything runs forward
    // through the chunk, and x_{t-1} is not kept in registers across the look-back.
    W ac = Num<W>::zero(), f = Num<W>::zero(), A = Num<W>::zero(), B = Num<W>::zero();
    T gb[TC];  // g_t of the chunk's steps
    int64_t base = 0;
    if (live) {
      ac = Num<W>::conj(Wide<T>::up(lam[lane]));
      const int64_t m = lane / N, n = lane - m * N;
      base = (m * L + t0) * N + n;
      const T* gp = g + base;
      const T* xp = out + base;
      T xb[TC];  // x_{t-1}
      W H = Num<W>::zero(), pw = Num<W>::one();
      if (len == TC && t0 > 0) {
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          gb[i] = gp[i * N];
          xb[i] = xp[(i - 1) * N];
        }
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          const W gi = Wide<T>::up(gb[i]);
          H = Num<W>::fma(ac, H, Num<W>::conj(Wide<T>::up(xb[i])));
          A = Num<W>::fma(gi, H, A);
          f = Num<W>::fma(pw, gi, f);
          pw = Num<W>::mul(pw, ac);
        }
      } else if (len > 0) {
        // partial or first chunk: loads clamped into the chunk (branch-free), steps guarded
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          const int ii = i < len ? i : len - 1;
          gb[i] = gp[ii * N];
          xb[i] = xp[(t0 + ii > 0 ? ii - 1 : 0) * N];
        }
        if (t0 == 0) xb[0] = x0 ? x0[lane] : T{};  // x_{-1}: the initial state (zero without x0)
#pragma unroll
        for (int i = 0; i < TC; ++i)
          if (i < len) {
            const W gi = Wide<T>::up(gb[i]);
            H = Num<W>::fma(ac, H, Num<W>::conj(Wide<T>::up(xb[i])));
            A = Num<W>::fma(gi, H, A);
            f = Num<W>::fma(pw, gi, f);
            pw = Num<W>::mul(pw, ac);
          }
      }
      B = Num<W>::mul(ac, H);
    }
    s_f[k][lid] = f;
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    const W Pc = ipow(ac, TC);
    Map<W> sup = {ipow(Pc, K), Num<W>::zero()};
    if (k == 0 && live) {
      sup.e = s_f[K - 1][lid];
      for (int j = K - 2; j >= 0; --j) sup.e = Num<W>::fma(Pc, sup.e, s_f[j][lid]);
      if (lb_pub_agg(nsuper - 1 - sc, lb_spacing) && sc > 0) put(agg + sc * lanes + lane, sup);
    }
    W R = Num<W>::zero();  // G entering the super-chunk from the right
    if (sc + 1 < nsuper)   // uniform over the workgroup
      R = look_back(agg, inc, k == 0 && live, sc + 1, (int64_t)1, nsuper, lanes, lane, K, k, lid, s_win, s_flag, s_pos,
                    &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(nsuper - 1 - sc, lb_spacing) && sc > 0) put(inc + sc * lanes + lane, apply(sup, R));
      for (int j = K - 1; j >= 0; --j) {
        s_start[j][lid] = R;
        R = Num<W>::fma(Pc, R, s_f[j][lid]);
      }
    }
    __syncthreads();
    W acc = Num<W>::zero();
    if (live && len > 0) {
      W G = s_start[k][lid];
      acc = Num<W>::fma(G, B, A);
      T* gvp = gv + base;
      if (len == TC) {
#pragma unroll
        for (int i = TC - 1; i >= 0; --i) {
          G = Num<W>::fma(ac, G, Wide<T>::up(gb[i]));
          gvp[i * N] = Wide<T>::down(G);
        }
      } else {
#pragma unroll
        for (int i = TC - 1; i >= 0; --i)
          if (i < len) {
            G = Num<W>::fma(ac, G, Wide<T>::up(gb[i]));
            gvp[i * N] = Wide<T>::down(G);
          }
      }
      if (t0 == 0 && gx0) gx0[lane] = Wide<T>::down(Num<W>::mul(ac, G));
    }
    s_acc[k][lid] = acc;
    __syncthreads();
    if (k == 0 && live) {
      W s = s_acc[0][lid];
      for (int j = 1; j < K; ++j) s = Num<W>::add(s, s_acc[j][lid]);
      if (nsuper == 1)
        glam[lane] = Wide<T>::down(s);
      else
        part[sc * lanes + lane] = s;
    }
  }
}

// ---------------------------------------------------------------- whole-sequence tiles
// When K <= KMAX chunks of TC steps cover the sequence, one workgroup of K x LG threads takes an
// LG-lane group's whole sequence (threads k*LG .. k*LG + LG-1 the k-th chunk): no look-back, no
// workspace words and no reset launch, so each direction is a single kernel. After one barrier
// every chunk composes the summaries of the chunks before it (forward) or after it (backward)
// from LDS into its entering state, at most K - 1 fp64 folds. Narrow groups (LG = 16, or 8 in the
// forward) give a small scan more workgroups than there are lane groups of 64; whole_group()
// hands each XCD a contiguous range of groups, so the groups whose rows share a 128-byte line
// share an L2.
TSF_DEV int64_t whole_group() {
  const unsigned total = gridDim.x;
  unsigned lin = blockIdx.x;
  if (total % kXcds == 0) lin = (lin % kXcds) * (total / kXcds) + lin / kXcds;
  return lin;
}

template <typename T, int TC, int LG, int KMAX>
__global__ void __launch_bounds__(LG * KMAX) diag_whole_fwd(const T* __restrict__ lam, const T* __restrict__ v,
                                                                 const T* __restrict__ x0, T* __restrict__ out,
                                                                 unsigned* __restrict__ ws_head, int64_t lanes,
                                                                 int64_t L, int64_t N) {
  using W = typename Wide<T>::type;
  __shared__ W s_e[KMAX][LG];
  const int lid = threadIdx.x % LG, k = threadIdx.x / LG;
  const int64_t lane = whole_group() * LG + lid;
  const bool live = lane < lanes;
  const int64_t t0 = (int64_t)k * TC;
  const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) ws_head[kErrWord] = 0;  // no look-back: nothing can give up
  W a = Num<W>::zero(), e = Num<W>::zero();
  T vb[TC];
  int64_t base = 0;
  if (live) {
    a = Wide<T>::up(lam[lane]);
    const int64_t m = lane / N, n = lane - m * N;
    base = (m * L + t0) * N + n;
    const T* vp = v + base;
    if (len == TC) {
#pragma unroll
      for (int i = 0; i < TC; ++i) vb[i] = vp[i * N];
#pragma unroll
      for (int i = 0; i < TC; ++i) e = Num<W>::fma(a, e, Wide<T>::up(vb[i]));
    } else {
#pragma unroll
      for (int i = 0; i < TC; ++i)
        if (i < len) vb[i] = vp[i * N];
#pragma unroll
      for (int i = 0; i < TC; ++i)
        if (i < len) e = Num<W>::fma(a, e, Wide<T>::up(vb[i]));
    }
  }
  s_e[k][lid] = e;
  __syncthreads();
  if (!live || len == 0) return;
  const W Pc = ipow(a, TC);  // every chunk before a non-empty one is full
  W x = x0 ? Wide<T>::up(x0[lane]) : Num<W>::zero();
  for (int j = 0; j < k; ++j) x = Num<W>::fma(Pc, x, s_e[j][lid]);
  T* op = out + base;
  if (len == TC) {
#pragma unroll
    for (int i = 0; i < TC; ++i) {
      x = Num<W>::fma(a, x, Wide<T>::up(vb[i]));
      op[i * N] = Wide<T>::down(x);
    }
  } else {
#pragma unroll
    for (int i = 0; i < TC; ++i)
      if (i < len) {
        x = Num<W>::fma(a, x, Wide<T>::up(vb[i]));
        op[i * N] = Wide<T>::down(x);
      }
  }
}

// Backward of the whole-sequence tile: each chunk summarises its adjoint from a zero state
// (f = G at the chunk's first step), then re-runs it from the G entering from the right, writing
// gv and accumulating glam = sum_t G_t conj(x_{t-1}). With 64-lane groups (16 waves, 128 VGPRs)
// the re-run goes half a chunk at a time and reloads its g values (L2 hits) together with x,
// through a pointer the compiler cannot see through, so at most one chunk of values is live at
// a time; narrower groups have the registers to load the chunk's g and x values together before
// the barrier (one round trip to memory). The K per-chunk glam sums are added in order.
template <typename T, int TC, int LG, int KMAX>
__global__ void __launch_bounds__(LG * KMAX) diag_whole_bwd(const T* __restrict__ lam, const T* __restrict__ g,
                                                                 const T* __restrict__ out, const T* __restrict__ x0,
                                                                 T* __restrict__ gv, T* __restrict__ glam,
                                                                 T* __restrict__ gx0, unsigned* __restrict__ ws_head,
                                                                 int64_t lanes, int64_t L, int64_t N) {
  using W = typename Wide<T>::type;
  constexpr int H2 = TC / 2;
  constexpr bool kKeep = LG * KMAX <= 256;
  __shared__ W s_f[KMAX][LG];
  __shared__ W s_acc[KMAX][LG];
  const int lid = threadIdx.x % LG, k = threadIdx.x / LG, K = blockDim.x / LG;
  const int64_t lane = whole_group() * LG + lid;
  const bool live = lane < lanes;
  const int64_t t0 = (int64_t)k * TC;
  const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) ws_head[kErrWord] = 0;  // no look-back: nothing can give up
  W ac = Num<W>::zero(), f = Num<W>::zero();
  int64_t base = 0;
  T gb[TC];
  T xb[kKeep ? TC : 1];  // narrow groups: x_{t-1} of the whole chunk, loaded with g
  if (live) {
    ac = Num<W>::conj(Wide<T>::up(lam[lane]));
    const int64_t m = lane / N, n = lane - m * N;
    base = (m * L + t0) * N + n;
    const T* gp = g + base;
    if (kKeep) {
      const T* xp = out + base;
      if (len == TC && t0 > 0) {
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          gb[i] = gp[i * N];
          xb[i] = xp[(i - 1) * N];
        }
      } else {
#pragma unroll
        for (int i = 0; i < TC; ++i) {  // clamped into the chunk, branch-free
          const int ii = i < len ? i : len - 1;
          gb[i] = gp[ii * N];
          xb[i] = xp[(t0 + ii > 0 ? ii - 1 : 0) * N];
        }
        if (t0 == 0) xb[0] = x0 ? x0[lane] : T{};
      }
#pragma unroll
      for (int i = TC - 1; i >= 0; --i)
        if (len == TC || i < len) f = Num<W>::fma(ac, f, Wide<T>::up(gb[i]));
    } else if (len == TC) {
#pragma unroll
      for (int i = 0; i < TC; ++i) gb[i] = gp[i * N];
#pragma unroll
      for (int i = TC - 1; i >= 0; --i) f = Num<W>::fma(ac, f, Wide<T>::up(gb[i]));
    } else {
#pragma unroll
      for (int i = 0; i < TC; ++i) gb[i] = gp[(i < len ? i : len - 1) * N];  // clamped, branch-free
#pragma unroll
      for (int i = TC - 1; i >= 0; --i)
        if (i < len) f = Num<W>::fma(ac, f, Wide<T>::up(gb[i]));
    }
  }
  s_f[k][lid] = f;
  __syncthreads();
  W acc = Num<W>::zero();
  if (live && len > 0) {
    const W Pc = ipow(ac, TC);  // every chunk before a non-empty one is full
    W G = Num<W>::zero();       // G entering the chunk from the right
    for (int j = K - 1; j > k; --j) G = Num<W>::fma(Pc, G, s_f[j][lid]);
    T* gvp = gv + base;
    if (kKeep) {
#pragma unroll
      for (int i = TC - 1; i >= 0; --i)
        if (i < len) {
          G = Num<W>::fma(ac, G, Wide<T>::up(gb[i]));
          gvp[i * N] = Wide<T>::down(G);
          acc = Num<W>::fma(G, Num<W>::conj(Wide<T>::up(xb[i])), acc);
        }
    } else {
#pragma unroll
      for (int h = 1; h >= 0; --h) {
        const T* gp = g + base;
        const T* xp = out + base;
        asm volatile("" : "+v"(gp), "+v"(xp));
        T gh[H2], xh[H2];  // g_t and x_{t-1} (x0, or zero without it, before the first step)
        if (len == TC && t0 > 0) {
#pragma unroll
          for (int i = 0; i < H2; ++i) {
            gh[i] = gp[(h * H2 + i) * N];
            xh[i] = xp[(h * H2 + i - 1) * N];
          }
        } else {
#pragma unroll
          for (int i = 0; i < H2; ++i) {  // clamped into the chunk, branch-free
            const int ii = h * H2 + i < len ? h * H2 + i : len - 1;
            gh[i] = gp[ii * N];
            xh[i] = xp[(t0 + ii > 0 ? ii - 1 : 0) * N];
          }
          if (t0 == 0 && h == 0) xh[0] = x0 ? x0[lane] : T{};
        }
#pragma unroll
        for (int i = H2 - 1; i >= 0; --i) {
          const int ii = h * H2 + i;
          if (ii < len) {
            G = Num<W>::fma(ac, G, Wide<T>::up(gh[i]));
            gvp[ii * N] = Wide<T>::down(G);
            acc = Num<W>::fma(G, Num<W>::conj(Wide<T>::up(xh[i])), acc);
          }
        }
      }
    }
    if (k == 0 && gx0) gx0[lane] = Wide<T>::down(Num<W>::mul(ac, G));
  }
  s_acc[k][lid] = acc;
  __syncthreads();
  if (k == 0 && live) {
    W sum = s_acc[0][lid];
    for (int j = 1; j < K; ++j) sum = Num<W>::add(sum, s_acc[j][lid]);
    glam[lane] = Wide<T>::down(sum);
  }
}

// glam = sum over super-chunks of the partials, in a fixed order (deterministic run to run):
// wave k adds the k-th of 16 contiguous segments, wave 0 adds the 16 segment sums in order.
template <typename T>
__global__ void __launch_bounds__(1024) diag_sum_parts(const typename Wide<T>::type* __restrict__ part,
                                                       T* __restrict__ dst, int64_t lanes, int64_t n) {
  using W = typename Wide<T>::type;
  __shared__ W s_p[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t lane = blockIdx.x * 64 + lid;
  const bool live = lane < lanes;
  const int64_t seg = (n + kMaxWaves - 1) / kMaxWaves;
  const int64_t r0 = k * seg, r1 = (r0 + seg < n) ? r0 + seg : n;
  W s = Num<W>::zero();
  if (live) {
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) s = Num<W>::add(s, part[r * lanes + lane]);
  }
  s_p[k][lid] = s;
  __syncthreads();
  if (k == 0 && live) {
    W t = s_p[0][lid];
    for (int j = 1; j < kMaxWaves; ++j) t = Num<W>::add(t, s_p[j][lid]);
    dst[lane] = Wide<T>::down(t);
  }
}

// Zero fill (gradients of an empty sequence); a kernel rather than a memset node, so that a
// captured graph replays it reliably.
__global__ void __launch_bounds__(256) zero_fill(float* __restrict__ p, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// ---------------------------------------------------------------- time-varying coefficient (real)
// Same tiles and look-back; a chunk's summary is the affine map x -> P x + e with P the product
// of its coefficients, and the chunk maps (P, e) meet in LDS.
template <int TC>
__global__ void __launch_bounds__(1024) sel_fwd(const float* __restrict__ a, const float* __restrict__ v,
                                                const float* __restrict__ x0, float* __restrict__ out,
                                                Map<double>* __restrict__ agg, double* __restrict__ inc,
                                                unsigned* __restrict__ counter, int64_t lanes, int64_t L, int64_t N,
                                                int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  __shared__ double2 s_m[kMaxWaves][64];  // chunk maps (P, e)
  // the look-back window, then the state entering each chunk
  __shared__ Map<double> s_win[kMaxWaves][64];
  __shared__ int s_flag[kMaxWaves][64];
  __shared__ int64_t s_pos[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  double(*s_start)[64] = reinterpret_cast<double(*)[64]>(&s_win[0][0]);
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * TC;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t sc = tile / groups, lane = (tile - sc * groups) * 64 + lid;
    const bool live = lane < lanes;
    const int64_t t0 = sc * SL + (int64_t)k * TC;
    const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
    double P = 1.0, e = 0.0;
    float ab[TC], vb[TC];
    int64_t base = 0;
    if (live) {
      const int64_t m = lane / N, n = lane - m * N;
      base = (m * L + t0) * N + n;
      if (len == TC) {  // full chunk: every load issued before the arithmetic, no per-step guard
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          ab[i] = a[base + i * N];
          vb[i] = v[base + i * N];
        }
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          e = fma((double)ab[i], e, (double)vb[i]);
          P *= (double)ab[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          ab[i] = i < len ? a[base + i * N] : 1.0f;
          vb[i] = i < len ? v[base + i * N] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < TC; ++i)
          if (i < len) {
            e = fma((double)ab[i], e, (double)vb[i]);
            P *= (double)ab[i];
          }
      }
    }
    s_m[k][lid] = make_double2(P, e);
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    Map<double> sup = {1.0, 0.0};
    if (k == 0 && live) {
      for (int j = 0; j < K; ++j) sup = then(sup, Map<double>{s_m[j][lid].x, s_m[j][lid].y});
      if (lb_pub_agg(sc, lb_spacing) && sc + 1 < nsuper) put(agg + sc * lanes + lane, sup);
    }
    double s = x0 && live && k == 0 ? (double)x0[lane] : 0.0;
    if (sc > 0)  // uniform over the workgroup
      s = look_back(agg, inc, k == 0 && live, sc - 1, (int64_t)-1, nsuper, lanes, lane, K, k, lid, s_win, s_flag,
                    s_pos, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(sc, lb_spacing) && sc + 1 < nsuper) put(inc + sc * lanes + lane, apply(sup, s));
      for (int j = 0; j < K; ++j) {
        s_start[j][lid] = s;
        s = fma(s_m[j][lid].x, s, s_m[j][lid].y);
      }
    }
    __syncthreads();
    if (live && len > 0) {
      double s = s_start[k][lid];
      if (len == TC) {
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          s = fma((double)ab[i], s, (double)vb[i]);
          out[base + i * N] = (float)s;
        }
      } else {
#pragma unroll
        for (int i = 0; i < TC; ++i)
          if (i < len) {
            s = fma((double)ab[i], s, (double)vb[i]);
            out[base + i * N] = (float)s;
          }
      }
    }
  }
}

// Backward: G_t = g_t + a_{t+1} G_{t+1} from the right end (a_L taken as 0: nothing enters),
// gv = G, glam_t = G_t x_{t-1} (x_{-1} the initial state), gx0 = a_0 G_0. A chunk's map takes
// G at the first step after it to G at its first step: (product of its a_{t+1}, value from zero).
template <int TC>
__global__ void __launch_bounds__(1024) sel_bwd(const float* __restrict__ a, const float* __restrict__ g,
                                                const float* __restrict__ out, const float* __restrict__ x0,
                                                Map<double>* __restrict__ agg, double* __restrict__ inc,
                                                unsigned* __restrict__ counter, float* __restrict__ glam,
                                                float* __restrict__ gv, float* __restrict__ gx0, int64_t lanes,
                                                int64_t L, int64_t N, int64_t groups, int K, int64_t nsuper, LbCfg lb_spacing) {
  __shared__ double2 s_m[kMaxWaves][64];
  // the look-back window, then G entering each chunk from the right
  __shared__ Map<double> s_win[kMaxWaves][64];
  __shared__ int s_flag[kMaxWaves][64];
  __shared__ int64_t s_pos[64];
  __shared__ int s_any;
  __shared__ unsigned s_tile[2];
  double(*s_start)[64] = reinterpret_cast<double(*)[64]>(&s_win[0][0]);
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t tiles = groups * nsuper, SL = (int64_t)K * TC;
  if (threadIdx.x == 0) s_tile[0] = take_tile(counter);
  __syncthreads();
  for (int buf = 0;; buf ^= 1) {
    const int64_t tile = s_tile[buf];
    if (tile >= tiles) break;
    unsigned next = 0;
    if (threadIdx.x == 0) next = take_tile(counter);
    const int64_t r = tile / groups, sc = nsuper - 1 - r, lane = (tile - r * groups) * 64 + lid;
    const bool live = lane < lanes;
    const int64_t t0 = sc * SL + (int64_t)k * TC;
    const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
    double M = 1.0, f = 0.0;
    float gb[TC], an[TC], xb[TC];  // g_t, a_{t+1}, x_{t-1}
    int64_t base = 0;
    if (live && len > 0) {
      const int64_t m = lane / N, n = lane - m * N;
      base = (m * L + t0) * N + n;
      if (len == TC && t0 > 0 && t0 + TC < L) {  // interior full chunk: no per-step guard
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          gb[i] = g[base + i * N];
          an[i] = a[base + (i + 1) * N];
          xb[i] = out[base + (i - 1) * N];
        }
#pragma unroll
        for (int i = TC - 1; i >= 0; --i) {
          f = fma((double)an[i], f, (double)gb[i]);
          M *= (double)an[i];
        }
      } else {
        const float xinit = x0 ? x0[lane] : 0.0f;  // x_{-1}
#pragma unroll
        for (int i = 0; i < TC; ++i) {
          gb[i] = i < len ? g[base + i * N] : 0.0f;
          an[i] = (i < len && t0 + i + 1 < L) ? a[base + (i + 1) * N] : 0.0f;
          xb[i] = i >= len ? 0.0f : (t0 + i > 0) ? out[base + (i - 1) * N] : xinit;
        }
#pragma unroll
        for (int i = TC - 1; i >= 0; --i)
          if (i < len) {
            f = fma((double)an[i], f, (double)gb[i]);
            M *= (double)an[i];
          }
      }
    }
    s_m[k][lid] = make_double2(M, f);
    if (threadIdx.x == 0) s_tile[buf ^ 1] = next;
    __syncthreads();
    Map<double> sup = {1.0, 0.0};
    if (k == 0 && live) {
      sup = Map<double>{s_m[K - 1][lid].x, s_m[K - 1][lid].y};
      for (int j = K - 2; j >= 0; --j) sup = then(sup, Map<double>{s_m[j][lid].x, s_m[j][lid].y});
      if (lb_pub_agg(nsuper - 1 - sc, lb_spacing) && sc > 0) put(agg + sc * lanes + lane, sup);
    }
    double R = 0.0;
    if (sc + 1 < nsuper)  // uniform over the workgroup
      R = look_back(agg, inc, k == 0 && live, sc + 1, (int64_t)1, nsuper, lanes, lane, K, k, lid, s_win, s_flag,
                    s_pos, &s_any, counter, lb_spacing.spin_max);
    if (k == 0 && live) {
      if (lb_pub_inc(nsuper - 1 - sc, lb_spacing) && sc > 0) put(inc + sc * lanes + lane, apply(sup, R));
      for (int j = K - 1; j >= 0; --j) {
        s_start[j][lid] = R;
        R = fma(s_m[j][lid].x, R, s_m[j][lid].y);
      }
    }
    __syncthreads();
    if (live && len > 0) {
      double G = s_start[k][lid];
      if (len == TC) {
#pragma unroll
        for (int i = TC - 1; i >= 0; --i) {
          G = fma((double)an[i], G, (double)gb[i]);
          gv[base + i * N] = (float)G;
          glam[base + i * N] = (float)(G * (double)xb[i]);
        }
      } else {
#pragma unroll
        for (int i = TC - 1; i >= 0; --i)
          if (i < len) {
            G = fma((double)an[i], G, (double)gb[i]);
            gv[base + i * N] = (float)G;
            glam[base + i * N] = (float)(G * (double)xb[i]);
          }
      }
      if (t0 == 0 && gx0) gx0[lane] = (float)((double)a[base] * G);
    }
  }
}

inline dim3 grid_for(int64_t threads) { return dim3((unsigned)((threads + 255) / 256)); }

// Tile shape for one call. TC (steps per chunk) is a template parameter, at most tc_max: 32 for
// real lanes, 16 for complex ones and for the time-varying backward (a thread keeps its chunk's
// inputs in registers across the look-back: TC complex values, or three TC-step arrays, within
// the 128 VGPRs a 1024-thread workgroup allows). Every
// thread issues all TC loads of its chunk at once, so the bytes in flight do not depend on TC;
// the wave count (lanes / 64 x L / TC) does, and TC drops to 16 when 32 would leave fewer than
// kDiagWaveTarget waves. K (chunks per tile) starts at TSF_DIAG_KMAX and halves down to 4 while
// there are fewer than kDiagTileTarget tiles.
#ifndef TSF_DIAG_TILE_TARGET
#define TSF_DIAG_TILE_TARGET 256
#endif
#ifndef TSF_DIAG_WAVE_TARGET
#define TSF_DIAG_WAVE_TARGET 4096
#endif
#ifndef TSF_DIAG_KMAX
#define TSF_DIAG_KMAX 16
#endif
constexpr int64_t kDiagTileTarget = TSF_DIAG_TILE_TARGET;
constexpr int64_t kDiagWaveTarget = TSF_DIAG_WAVE_TARGET;
static_assert(TSF_DIAG_KMAX >= 4 && TSF_DIAG_KMAX <= kMaxWaves, "K range");

struct DiagTile {
  int64_t lanes = 0, groups = 0, nsuper = 0, SL = 0;
  int TC = 0, K = 0;
};

DiagTile diag_tile(int64_t lanes, int64_t L, int tc_max) {
  DiagTile t;
  t.lanes = lanes;
  if (lanes < 1 || L < 1) return t;
  t.groups = (lanes + 63) / 64;
  t.TC = (t.groups * ((L + 31) / 32) < kDiagWaveTarget) ? 16 : 32;
  if (t.TC > tc_max) t.TC = tc_max;
  t.K = TSF_DIAG_KMAX;
  auto tiles = [&](int K) { return t.groups * ((L + (int64_t)t.TC * K - 1) / ((int64_t)t.TC * K)); };
  while (t.K > 4 && tiles(t.K) < kDiagTileTarget) t.K /= 2;
  const int64_t chunks = (L + t.TC - 1) / t.TC;
  if (t.K > chunks) t.K = (int)chunks;  // no waves past the end of a short sequence
  t.SL = (int64_t)t.TC * t.K;
  t.nsuper = (L + t.SL - 1) / t.SL;
  return t;
}

DiagTile const_tile(int64_t lanes, int64_t L, bool cplx, bool bwd) {
  (void)bwd;
  return diag_tile(lanes, L, cplx ? 16 : 32);
}
DiagTile sel_tile(int64_t lanes, int64_t L, bool bwd) { return diag_tile(lanes, L, bwd ? 16 : 32); }

inline bool grid_fits(const DiagTile& t) { return t.groups * t.nsuper <= INT32_MAX; }

// Workspace of one scan: the tile counter (first 256 bytes), then agg [nsuper, lanes] maps and
// inc [nsuper, lanes] states of the look-back, then (constant-coefficient backward) the glam
// partials [nsuper, lanes].
inline int64_t lookback_bytes(const DiagTile& t, int64_t wbytes) { return t.nsuper * t.lanes * 3 * wbytes; }

template <typename F>
unsigned persistent_grid(const DiagTile& t, F kern, int* cache) {
  const int64_t tiles = t.groups * t.nsuper, cap = resident_wgs(kern, 64 * t.K, cache);
  return (unsigned)(tiles < cap ? tiles : cap);
}


// Whole-sequence tiling (diag_whole_fwd / diag_whole_bwd): TC steps per chunk; lane groups of 64
// (256-byte row segments of fp32) when they already give every CU a workgroup, else of 16 (four
// times the workgroups; 64-byte segments, paired in L2) or, in the forward, of 8 while that stays
// within one workgroup per CU. A workgroup holds up to 1024 threads: 16 chunks of 64 lanes, or up
// to 64 chunks of 16 or 8 lanes (the backward 16 chunks of 16 lanes, so that 256 threads may keep
// a chunk's values in registers). Longer sequences take the look-back.
constexpr int whole_tc(bool cplx, bool bwd) { return cplx ? (bwd ? 16 : 32) : 64; }
struct WholeTile {
  int lg = 0, kmax = 0;  // kmax == 0: the sequence is too long for one workgroup
};
inline WholeTile whole_tile(int64_t lanes, int64_t L, int tc, bool bwd) {
  const int64_t chunks = (L + tc - 1) / tc;
  if ((lanes + 63) / 64 >= 256) return chunks <= 16 ? WholeTile{64, 16} : WholeTile{};
  // the forward narrows its groups to 8 lanes while that keeps within one workgroup per CU (8-lane
  // groups measured 4-9% faster on configs 5 and 1, 4-lane groups no faster than 8); the
  // backward stays at 16 lanes (narrower groups measured 12% slower on config 1)
  const int lg = (!bwd && (lanes + 7) / 8 <= 256) ? 8 : 16;
  if (chunks <= 16) return {lg, 16};
  // 64 chunks of 16 or 8 lanes: forward only, and only while one round of workgroups covers the
  // lanes (the backward of so long a chunk run reloads its values, slower than the look-back; a
  // 4-lane backward that keeps them measured 29% slower on config 5 at one wave per SIMD)
  if (!bwd && chunks <= 64 && (lanes + lg - 1) / lg <= 256) return {lg, 64};
  return {};
}
inline bool whole_both(int64_t lanes, int64_t L, bool cplx) {
  return whole_tile(lanes, L, whole_tc(cplx, false), false).kmax > 0 &&
         whole_tile(lanes, L, whole_tc(cplx, true), true).kmax > 0;
}

template <typename T, int TC>
void whole_fwd_launch(const WholeTile& w, int64_t lanes, int64_t L, int64_t N, const T* lam, const T* v, const T* x0,
                      T* out, unsigned* ws, hipStream_t s) {
  const dim3 grid((unsigned)((lanes + w.lg - 1) / w.lg)), block((unsigned)(w.lg * ((L + TC - 1) / TC)));
#define TSF_WHOLE_FWD(LG, KMAX) \
  if (w.lg == LG && w.kmax == KMAX) { \
    hipLaunchKernelGGL((diag_whole_fwd<T, TC, LG, KMAX>), grid, block, 0, s, lam, v, x0, out, ws, lanes, L, N); \
    return; \
  }
  TSF_WHOLE_FWD(64, 16) TSF_WHOLE_FWD(16, 16) TSF_WHOLE_FWD(8, 16) TSF_WHOLE_FWD(16, 64) TSF_WHOLE_FWD(8, 64)
#undef TSF_WHOLE_FWD
}

template <typename T, int TC>
void whole_bwd_launch(const WholeTile& w, int64_t lanes, int64_t L, int64_t N, const T* lam, const T* g, const T* out,
                      const T* x0, T* gv, T* glam, T* gx0, unsigned* ws, hipStream_t s) {
  const dim3 grid((unsigned)((lanes + w.lg - 1) / w.lg)), block((unsigned)(w.lg * ((L + TC - 1) / TC)));
#define TSF_WHOLE_BWD(LG, KMAX) \
  if (w.lg == LG && w.kmax == KMAX) { \
    hipLaunchKernelGGL((diag_whole_bwd<T, TC, LG, KMAX>), grid, block, 0, s, lam, g, out, x0, gv, glam, gx0, ws, \
                       lanes, L, N); \
    return; \
  }
  TSF_WHOLE_BWD(64, 16) TSF_WHOLE_BWD(16, 16)
#undef TSF_WHOLE_BWD
}

template <typename T, int TC>
void diag_fwd_launch(const DiagTile& t, const T* lam, const T* v, const T* x0, T* out, char* ws, int64_t L, int64_t N,
                     hipStream_t s) {
  using W = typename Wide<T>::type;
  static int occ[kMaxWaves + 1];
  auto* agg = reinterpret_cast<Map<W>*>(ws + kCounterBytes);
  auto* inc = reinterpret_cast<W*>(agg + t.nsuper * t.lanes);
  lookback_reset_launch(ws, lookback_bytes(t, sizeof(W)) / 8, s);
  hipLaunchKernelGGL((diag_fwd<T, TC>), dim3(persistent_grid(t, diag_fwd<T, TC>, occ)), dim3(64 * t.K), 0, s, lam, v,
                     x0, out, agg, inc, reinterpret_cast<unsigned*>(ws), t.lanes, L, N, t.groups, t.K, t.nsuper, lb_spacing_for(anchor_spacing_for_groups(t.groups)));
}

template <typename T, int TC>
void diag_bwd_launch(const DiagTile& t, const T* g, const T* lam, const T* out, const T* x0, T* gv, T* glam, T* gx0,
                     char* ws, int64_t L, int64_t N, hipStream_t s) {
  using W = typename Wide<T>::type;
  static int occ[kMaxWaves + 1];
  auto* agg = reinterpret_cast<Map<W>*>(ws + kCounterBytes);
  auto* inc = reinterpret_cast<W*>(agg + t.nsuper * t.lanes);
  W* part = inc + t.nsuper * t.lanes;
  lookback_reset_launch(ws, lookback_bytes(t, sizeof(W)) / 8, s);
  hipLaunchKernelGGL((diag_bwd<T, TC>), dim3(persistent_grid(t, diag_bwd<T, TC>, occ)), dim3(64 * t.K), 0, s, lam, g,
                     out, x0, agg, inc, reinterpret_cast<unsigned*>(ws), gv, part, glam, gx0, t.lanes, L, N, t.groups,
                     t.K, t.nsuper, lb_spacing_for(anchor_spacing_for_groups(t.groups)));
  if (t.nsuper > 1)
    hipLaunchKernelGGL(diag_sum_parts<T>, dim3((unsigned)t.groups), dim3(64 * kMaxWaves), 0, s, (const W*)part, glam,
                       t.lanes, t.nsuper);
}

template <int TC>
void sel_fwd_launch(const DiagTile& t, const float* a, const float* v, const float* x0, float* out, char* ws,
                    int64_t L, int64_t N, hipStream_t s) {
  static int occ[kMaxWaves + 1];
  auto* agg = reinterpret_cast<Map<double>*>(ws + kCounterBytes);
  auto* inc = reinterpret_cast<double*>(agg + t.nsuper * t.lanes);
  lookback_reset_launch(ws, lookback_bytes(t, 8) / 8, s);
  hipLaunchKernelGGL((sel_fwd<TC>), dim3(persistent_grid(t, sel_fwd<TC>, occ)), dim3(64 * t.K), 0, s, a, v, x0, out,
                     agg, inc, reinterpret_cast<unsigned*>(ws), t.lanes, L, N, t.groups, t.K, t.nsuper, lb_spacing_for(anchor_spacing_for_groups(t.groups)));
}

void sel_bwd_launch(const DiagTile& t, const float* g, const float* a, const float* out, const float* x0, float* glam,
                    float* gv, float* gx0, char* ws, int64_t L, int64_t N, hipStream_t s) {
  static int occ[kMaxWaves + 1];
  auto* agg = reinterpret_cast<Map<double>*>(ws + kCounterBytes);
  auto* inc = reinterpret_cast<double*>(agg + t.nsuper * t.lanes);
  lookback_reset_launch(ws, lookback_bytes(t, 8) / 8, s);
  hipLaunchKernelGGL((sel_bwd<16>), dim3(persistent_grid(t, sel_bwd<16>, occ)), dim3(64 * t.K), 0, s, a, g, out, x0,
                     agg, inc, reinterpret_cast<unsigned*>(ws), glam, gv, gx0, t.lanes, L, N, t.groups, t.K,
                     t.nsuper, lb_spacing_for(anchor_spacing_for_groups(t.groups)));
}

}  // namespace

// ---------------------------------------------------------------- no-allocation entry point
// The look-back workspace of tsfast_hip_diag_fwd_noalloc: a fixed array in device memory, one
// copy per GPU, held until the process ends. Host code never uses this name as an address: the
// device address of each GPU's copy comes from hipGetSymbolAddress (below).
constexpr int64_t kNoAllocScratchBytes = (int64_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<char*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this GPU's `scratch`, looked up once per device with that device current;
// the call's stream must belong to the current device.
int noalloc_scratch(hipStream_t s, char** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return tsf_record_hip_error(e);
  if (s != nullptr) {
    hipDevice_t sdev = cur;
    e = hipStreamGetDevice(s, &sdev);
    if (e != hipSuccess) return tsf_record_hip_error(e);
    if (sdev != cur) return TSF_ERR_ARG;
  }
  if (cur < 0 || cur >= kMaxDevices) return TSF_ERR_UNSUPPORTED;
  char* p = g_scratch_addr[cur].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[cur].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return tsf_record_hip_error(e);
      p = static_cast<char*>(addr);
      g_scratch_addr[cur].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return TSF_OK;
}

// Workspace bytes the forward alone touches: the header (the give-up word) on whole-sequence
// tiles, else the header and its look-back words (maps and states, 3 fp64 words per lane and
// super-chunk, complex128 when complex).
int64_t diag_fwd_workspace_bytes(int64_t M, int64_t L, int64_t N, bool cplx) {
  if (whole_tile(M * N, L, whole_tc(cplx, false), false).kmax > 0) return kCounterBytes;
  return kCounterBytes + lookback_bytes(const_tile(M * N, L, cplx, false), cplx ? 16 : 8);
}

}  // namespace

extern "C" {

int64_t tsfast_hip_diag_workspace_bytes(int64_t M, int64_t L, int64_t N, int is_complex) {
  // whole-sequence tiles in both directions: only the header (its look-back flag word) is used
  if (whole_both(M * N, L, is_complex != 0)) return kCounterBytes;
  const DiagTile f = const_tile(M * N, L, is_complex != 0, false), b = const_tile(M * N, L, is_complex != 0, true);
  // counter, then fp64 look-back maps and states and glam partials, 4 words per lane and
  // super-chunk (complex128 when complex), for the larger of the forward / backward tilings
  return kCounterBytes + 4 * (f.nsuper > b.nsuper ? f.nsuper : b.nsuper) * M * N * (is_complex ? 16 : 8);
}

int tsfast_hip_diag_fwd(int64_t M, int64_t L, int64_t N, int is_complex, const void* lam, const void* v,
                        const void* x0, void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  if (M == 0 || L == 0 || N == 0) return TSF_OK;
  if (!lam || !v || !out) return TSF_ERR_ARG;
  if (workspace_bytes < diag_fwd_workspace_bytes(M, L, N, is_complex != 0) || !workspace) return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const WholeTile wf = whole_tile(M * N, L, whole_tc(is_complex != 0, false), false);
  if (wf.kmax > 0) {
    if ((M * N + 15) / 16 > INT32_MAX) return TSF_ERR_UNSUPPORTED;
    if (is_complex)
      whole_fwd_launch<float2, whole_tc(true, false)>(wf, M * N, L, N, (const float2*)lam, (const float2*)v,
                                                      (const float2*)x0, (float2*)out, (unsigned*)workspace, s);
    else
      whole_fwd_launch<float, whole_tc(false, false)>(wf, M * N, L, N, (const float*)lam, (const float*)v,
                                                      (const float*)x0, (float*)out, (unsigned*)workspace, s);
    return tsf_launch_status();
  }
  const DiagTile t = const_tile(M * N, L, is_complex != 0, false);
  if (!grid_fits(t)) return TSF_ERR_UNSUPPORTED;
  char* ws = static_cast<char*>(workspace);
  if (is_complex)
    diag_fwd_launch<float2, 16>(t, (const float2*)lam, (const float2*)v, (const float2*)x0, (float2*)out, ws, L, N, s);
  else if (t.TC == 32)
    diag_fwd_launch<float, 32>(t, (const float*)lam, (const float*)v, (const float*)x0, (float*)out, ws, L, N, s);
  else
    diag_fwd_launch<float, 16>(t, (const float*)lam, (const float*)v, (const float*)x0, (float*)out, ws, L, N, s);
  return tsf_launch_status();
}

int tsfast_hip_diag_bwd(int64_t M, int64_t L, int64_t N, int is_complex, const void* g, const void* lam,
                        const void* out, const void* x0, void* gv, void* glam, void* gx0, void* workspace,
                        int64_t workspace_bytes, void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t lanes = M * N;
  if (lanes == 0) return TSF_OK;
  if (!lam || !glam || (x0 && !gx0)) return TSF_ERR_ARG;
  if (L == 0) {
    // empty sequence: every gradient is zero
    const int64_t nf = lanes * (is_complex ? 2 : 1);
    hipLaunchKernelGGL(zero_fill, grid_for(nf), dim3(256), 0, s, (float*)glam, nf);
    if (gx0) hipLaunchKernelGGL(zero_fill, grid_for(nf), dim3(256), 0, s, (float*)gx0, nf);
    return tsf_launch_status();
  }
  if (!g || !out || !gv) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_diag_workspace_bytes(M, L, N, is_complex) || !workspace) return TSF_ERR_WORKSPACE;
  const WholeTile wb = whole_tile(lanes, L, whole_tc(is_complex != 0, true), true);
  if (wb.kmax > 0) {
    if ((lanes + 15) / 16 > INT32_MAX) return TSF_ERR_UNSUPPORTED;
    if (is_complex)
      whole_bwd_launch<float2, whole_tc(true, true)>(wb, lanes, L, N, (const float2*)lam, (const float2*)g,
                                                     (const float2*)out, (const float2*)x0, (float2*)gv,
                                                     (float2*)glam, (float2*)gx0, (unsigned*)workspace, s);
    else
      whole_bwd_launch<float, whole_tc(false, true)>(wb, lanes, L, N, (const float*)lam, (const float*)g,
                                                     (const float*)out, (const float*)x0, (float*)gv, (float*)glam,
                                                     (float*)gx0, (unsigned*)workspace, s);
    return tsf_launch_status();
  }
  const DiagTile t = const_tile(lanes, L, is_complex != 0, true);
  if (!grid_fits(t)) return TSF_ERR_UNSUPPORTED;
  char* ws = static_cast<char*>(workspace);
  if (is_complex)
    diag_bwd_launch<float2, 16>(t, (const float2*)g, (const float2*)lam, (const float2*)out, (const float2*)x0,
                                (float2*)gv, (float2*)glam, (float2*)gx0, ws, L, N, s);
  else if (t.TC == 32)
    diag_bwd_launch<float, 32>(t, (const float*)g, (const float*)lam, (const float*)out, (const float*)x0, (float*)gv,
                               (float*)glam, (float*)gx0, ws, L, N, s);
  else
    diag_bwd_launch<float, 16>(t, (const float*)g, (const float*)lam, (const float*)out, (const float*)x0, (float*)gv,
                               (float*)glam, (float*)gx0, ws, L, N, s);
  return tsf_launch_status();
}

int64_t tsfast_hip_diag_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

int tsfast_hip_diag_fwd_noalloc(int64_t M, int64_t L, int64_t N, int is_complex, const void* lam, const void* v,
                                const void* x0, void* out, void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  if (M == 0 || L == 0 || N == 0) return TSF_OK;
  if (!lam || !v || !out) return TSF_ERR_ARG;
  const int64_t need = diag_fwd_workspace_bytes(M, L, N, is_complex != 0);
  if (need > kNoAllocScratchBytes) return TSF_ERR_SCRATCH;
  char* ws = nullptr;
  const int st = noalloc_scratch(static_cast<hipStream_t>(stream), &ws);
  if (st != TSF_OK) return st;
  // the kernels of tsfast_hip_diag_fwd; its reset kernel marks the look-back words in `scratch`
  // unset and zeroes the tile counter on the stream before the scan runs
  return tsfast_hip_diag_fwd(M, L, N, is_complex, lam, v, x0, out, ws, need, stream);
}

int64_t tsfast_hip_sel_workspace_bytes(int64_t M, int64_t L, int64_t N) {
  // counter, then fp64 look-back maps (P, e) and states, 3 words per lane and super-chunk, for
  // the larger of the forward / backward tilings
  const DiagTile f = sel_tile(M * N, L, false), b = sel_tile(M * N, L, true);
  return kCounterBytes + (f.nsuper > b.nsuper ? f.nsuper : b.nsuper) * M * N * 24;
}

int tsfast_hip_sel_fwd(int64_t M, int64_t L, int64_t N, const float* a, const float* v, const float* x0, float* out,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  if (M == 0 || L == 0 || N == 0) return TSF_OK;
  if (!a || !v || !out) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_sel_workspace_bytes(M, L, N) || !workspace) return TSF_ERR_WORKSPACE;
  const DiagTile t = sel_tile(M * N, L, false);
  if (!grid_fits(t)) return TSF_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (t.TC == 32)
    sel_fwd_launch<32>(t, a, v, x0, out, ws, L, N, s);
  else
    sel_fwd_launch<16>(t, a, v, x0, out, ws, L, N, s);
  return tsf_launch_status();
}

int tsfast_hip_sel_bwd(int64_t M, int64_t L, int64_t N, const float* g, const float* a, const float* out,
                       const float* x0, float* glam, float* gv, float* gx0, void* workspace, int64_t workspace_bytes,
                       void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t lanes = M * N;
  if (lanes == 0) return TSF_OK;
  if (x0 && !gx0) return TSF_ERR_ARG;
  if (L == 0) {
    if (gx0) hipLaunchKernelGGL(zero_fill, grid_for(lanes), dim3(256), 0, s, gx0, lanes);
    return tsf_launch_status();
  }
  if (!g || !a || !out || !gv || !glam) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_sel_workspace_bytes(M, L, N) || !workspace) return TSF_ERR_WORKSPACE;
  const DiagTile t = sel_tile(lanes, L, true);
  if (!grid_fits(t)) return TSF_ERR_UNSUPPORTED;
  sel_bwd_launch(t, g, a, out, x0, glam, gv, gx0, static_cast<char*>(workspace), L, N, s);
  return tsf_launch_status();
}

}  // extern "C"
