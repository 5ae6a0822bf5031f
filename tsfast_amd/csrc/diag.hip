// Diagonal linear-recurrence scans on the lane layout [M, L, N] (N contiguous):
//   constant coefficient  x_t = lam * x_{t-1} + v_t            (lam [M, N], real or complex)
//   time-varying          x_t = a_t * x_{t-1} + v_t            (a   [M, L, N], real)
// and their adjoints G_t = g_t + conj(c_{t+1}) G_{t+1}.
//
// Reference semantics: tsfast/models/_core/scan.py:100-215 (ops), :52-80 (doubling scans),
// scan_backends/diagonal_triton.py:82-228 and selective_triton.py:48-109 (kernels).
//
// Both are chunked two-pass scans with no inter-workgroup waiting: chunk summaries from a zero
// state first, then a re-scan of every chunk from its true start state, the carries composed in
// fp64 (complex128). Consecutive threads own consecutive lanes, so every per-step load/store is a
// coalesced row segment along N; the re-read of the input in pass 2 is the price of needing no
// global barrier. Both keep a chunk in registers and combine chunk summaries inside a workgroup
// through LDS (tiling described at the constant-coefficient kernels); the time-varying kernels
// carry (product of coefficients, state) affine maps where the constant ones carry states.
#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

// All kernels load fp32 (or complex64) and carry the recurrence in fp64 (complex128): W below.

// ---------------------------------------------------------------- constant coefficient
// Tiling. A workgroup of K waves (K <= 16) owns 64 consecutive lanes (thread lid of every wave
// owns lane group * 64 + lid) and one super-chunk of K * TC consecutive steps; wave k owns the
// k-th chunk of TC steps. A thread keeps its chunk's TC inputs in registers, scans them from a
// zero state, the K chunk summaries meet in LDS, and the thread re-runs its chunk from its true
// start state. Super-chunk summaries (one per lane and super-chunk) go through HBM:
//   summary  end state of every super-chunk but the last from a zero start, E [nsuper, lanes]
//   carry    (long sequences only) in-place scan of E into true super-chunk start states
//   apply    fold of E before the super-chunk (or the carried start), then the chunk scan.
// The backward mirrors this from the right end with conj(lam), and reduces the glam partials of
// the K chunks in LDS and of the super-chunks in a fixed-order sum (deterministic).
constexpr int kMaxWaves = 16;

template <typename T, int TC>
__global__ void __launch_bounds__(1024) diag_fwd_summary(const T* __restrict__ lam, const T* __restrict__ v,
                                                         typename Wide<T>::type* __restrict__ E, int64_t lanes,
                                                         int64_t L, int64_t N, int64_t groups, int K) {
  using W = typename Wide<T>::type;
  __shared__ W s_e[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t g = blockIdx.x % groups, sc = blockIdx.x / groups;  // super-chunks 0 .. nsuper-2
  const int64_t lane = g * 64 + lid;
  const bool live = lane < lanes;
  W a = Num<W>::zero(), e = Num<W>::zero();
  if (live) {
    a = Wide<T>::up(lam[lane]);
    const int64_t m = lane / N, n = lane - m * N;
    // every chunk of a super-chunk before the last is full
    const T* vp = v + (m * L + sc * K * TC + (int64_t)k * TC) * N + n;
    T vb[TC];
#pragma unroll
    for (int i = 0; i < TC; ++i) vb[i] = vp[i * N];
#pragma unroll
    for (int i = 0; i < TC; ++i) e = Num<W>::fma(a, e, Wide<T>::up(vb[i]));
  }
  s_e[k][lid] = e;
  __syncthreads();
  if (k == 0 && live) {
    const W P = ipow(a, TC);
    W s = s_e[0][lid];
    for (int j = 1; j < K; ++j) s = Num<W>::fma(P, s, s_e[j][lid]);
    E[sc * lanes + lane] = s;
  }
}

// In-place inclusive scan s_r = c * s_{r-1} + S[r] over n summaries per lane, with s_{-1} = init
// (NULL: zero). Summary r of lane `lane` sits at S[(first + dir * r) * lanes + lane]; c is the
// per-super-chunk multiplier lam^SL (conj(lam)^SL when `conjugate`). One workgroup per 64-lane
// group; wave k scans the k-th of 16 contiguous segments, and the segment results meet in LDS.
template <typename T>
__global__ void __launch_bounds__(1024) diag_carry(const T* __restrict__ lam, const T* __restrict__ init,
                                                   typename Wide<T>::type* __restrict__ S, int64_t lanes, int64_t n,
                                                   int64_t first, int64_t dir, int64_t SL, int conjugate) {
  using W = typename Wide<T>::type;
  __shared__ W s_p[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t lane = blockIdx.x * 64 + lid;
  const bool live = lane < lanes;
  const int64_t seg = (n + kMaxWaves - 1) / kMaxWaves;
  const int64_t r0 = k * seg, r1 = (r0 + seg < n) ? r0 + seg : n;
  W c = Num<W>::zero(), p = Num<W>::zero();
  if (live) {
    W a = Wide<T>::up(lam[lane]);
    if (conjugate) a = Num<W>::conj(a);
    c = ipow(a, SL);
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) p = Num<W>::fma(c, p, S[(first + dir * r) * lanes + lane]);
  }
  s_p[k][lid] = p;
  __syncthreads();
  if (live && r0 < r1) {
    W s = init ? Wide<T>::up(init[lane]) : Num<W>::zero();
    const W cs = ipow(c, seg);  // every segment before a non-empty one is full
    for (int j = 0; j < k; ++j) s = Num<W>::fma(cs, s, s_p[j][lid]);
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) {
      W* q = S + (first + dir * r) * lanes + lane;
      s = Num<W>::fma(c, s, *q);
      *q = s;
    }
  }
}

template <typename T, int TC>
__global__ void __launch_bounds__(1024) diag_fwd_apply(const T* __restrict__ lam, const T* __restrict__ v,
                                                       const T* __restrict__ x0,
                                                       const typename Wide<T>::type* __restrict__ E,
                                                       T* __restrict__ out, int64_t lanes, int64_t L, int64_t N,
                                                       int64_t groups, int K, int starts_ready) {
  using W = typename Wide<T>::type;
  __shared__ W s_e[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t g = blockIdx.x % groups, sc = blockIdx.x / groups;
  const int64_t lane = g * 64 + lid;
  const bool live = lane < lanes;
  const int64_t SL = (int64_t)K * TC;
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
  __syncthreads();
  if (!live || len == 0) return;  // no barrier follows
  // state entering the super-chunk
  W s = x0 ? Wide<T>::up(x0[lane]) : Num<W>::zero();
  if (sc > 0) {
    if (starts_ready) {
      s = E[(sc - 1) * lanes + lane];
    } else {
      const W Q = ipow(a, SL);
#pragma unroll 8
      for (int64_t j = 0; j < sc; ++j) s = Num<W>::fma(Q, s, E[j * lanes + lane]);
    }
  }
  // state entering chunk k
  if (k > 0) {
    const W P = ipow(a, TC);
    for (int j = 0; j < k; ++j) s = Num<W>::fma(P, s, s_e[j][lid]);
  }
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

// Reverse summary of super-chunk sc >= 1: G at its first step with no gradient entering from the
// right, F [nsuper, lanes] (slot 0 unused). Chunks past the end of the sequence are empty and
// contribute zero, so the full-chunk multiplier conj(lam)^TC is right for every fold.
template <typename T, int TC>
__global__ void __launch_bounds__(1024) diag_bwd_summary(const T* __restrict__ lam, const T* __restrict__ g,
                                                         typename Wide<T>::type* __restrict__ F, int64_t lanes,
                                                         int64_t L, int64_t N, int64_t groups, int K) {
  using W = typename Wide<T>::type;
  __shared__ W s_f[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t gr = blockIdx.x % groups, sc = blockIdx.x / groups + 1;  // super-chunks 1 .. nsuper-1
  const int64_t lane = gr * 64 + lid;
  const bool live = lane < lanes;
  const int64_t t0 = sc * K * TC + (int64_t)k * TC;
  const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
  W ac = Num<W>::zero(), f = Num<W>::zero();
  if (live) {
    ac = Num<W>::conj(Wide<T>::up(lam[lane]));
    const int64_t m = lane / N, n = lane - m * N;
    const T* gp = g + (m * L + t0) * N + n;
    T gb[TC];
    if (len == TC) {
#pragma unroll
      for (int i = 0; i < TC; ++i) gb[i] = gp[i * N];
#pragma unroll
      for (int i = TC - 1; i >= 0; --i) f = Num<W>::fma(ac, f, Wide<T>::up(gb[i]));
    } else {
#pragma unroll
      for (int i = 0; i < TC; ++i)
        if (i < len) gb[i] = gp[i * N];
#pragma unroll
      for (int i = TC - 1; i >= 0; --i)
        if (i < len) f = Num<W>::fma(ac, f, Wide<T>::up(gb[i]));
    }
  }
  s_f[k][lid] = f;
  __syncthreads();
  if (k == 0 && live) {
    const W P = ipow(ac, TC);
    W s = s_f[K - 1][lid];
    for (int j = K - 2; j >= 0; --j) s = Num<W>::fma(P, s, s_f[j][lid]);
    F[sc * lanes + lane] = s;
  }
}

template <typename T, int TC>
__global__ void __launch_bounds__(1024) diag_bwd_apply(const T* __restrict__ lam, const T* __restrict__ g,
                                                       const T* __restrict__ out, const T* __restrict__ x0,
                                                       const typename Wide<T>::type* __restrict__ F,
                                                       T* __restrict__ gv, typename Wide<T>::type* __restrict__ part,
                                                       T* __restrict__ glam, T* __restrict__ gx0, int64_t lanes,
                                                       int64_t L, int64_t N, int64_t groups, int K, int64_t nsuper,
                                                       int starts_ready) {
  using W = typename Wide<T>::type;
  __shared__ W s_f[kMaxWaves][64];
  __shared__ W s_acc[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t gr = blockIdx.x % groups, sc = blockIdx.x / groups;
  const int64_t lane = gr * 64 + lid;
  const bool live = lane < lanes;
  const int64_t SL = (int64_t)K * TC;
  const int64_t t0 = sc * SL + (int64_t)k * TC;
  const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
  W ac = Num<W>::zero(), f = Num<W>::zero();
  T gb[TC], xb[TC];  // g_t and x_{t-1} of the chunk's steps
  int64_t base = 0;
  if (live) {
    ac = Num<W>::conj(Wide<T>::up(lam[lane]));
    const int64_t m = lane / N, n = lane - m * N;
    base = (m * L + t0) * N + n;
    const T* gp = g + base;
    const T* xp = out + base;
    if (len == TC && t0 > 0) {
#pragma unroll
      for (int i = 0; i < TC; ++i) {
        gb[i] = gp[i * N];
        xb[i] = xp[(i - 1) * N];
      }
#pragma unroll
      for (int i = TC - 1; i >= 0; --i) f = Num<W>::fma(ac, f, Wide<T>::up(gb[i]));
    } else if (len > 0) {
      const T xinit = x0 ? x0[lane] : T{};  // x_{-1}: the initial state (zero without x0)
#pragma unroll
      for (int i = 0; i < TC; ++i)
        if (i < len) {
          gb[i] = gp[i * N];
          xb[i] = (t0 + i > 0) ? xp[(i - 1) * N] : xinit;
        }
#pragma unroll
      for (int i = TC - 1; i >= 0; --i)
        if (i < len) f = Num<W>::fma(ac, f, Wide<T>::up(gb[i]));
    }
  }
  s_f[k][lid] = f;
  __syncthreads();
  W acc = Num<W>::zero();
  if (live && len > 0) {
    // G entering the super-chunk from the right: G at the first step of super-chunk sc + 1
    W R = Num<W>::zero();
    if (sc + 1 < nsuper) {
      if (starts_ready) {
        R = F[(sc + 1) * lanes + lane];
      } else {
        const W Q = ipow(ac, SL);
        R = F[(nsuper - 1) * lanes + lane];
#pragma unroll 8
        for (int64_t j = nsuper - 2; j > sc; --j) R = Num<W>::fma(Q, R, F[j * lanes + lane]);
      }
    }
    // G entering chunk k from the right
    if (k + 1 < K) {
      const W P = ipow(ac, TC);
      for (int j = K - 1; j > k; --j) R = Num<W>::fma(P, R, s_f[j][lid]);
    }
    W G = R;
    T* gvp = gv + base;
    if (len == TC) {
#pragma unroll
      for (int i = TC - 1; i >= 0; --i) {
        G = Num<W>::fma(ac, G, Wide<T>::up(gb[i]));
        gvp[i * N] = Wide<T>::down(G);
        acc = Num<W>::add(acc, Num<W>::mul_conj(G, Wide<T>::up(xb[i])));
      }
    } else {
#pragma unroll
      for (int i = TC - 1; i >= 0; --i)
        if (i < len) {
          G = Num<W>::fma(ac, G, Wide<T>::up(gb[i]));
          gvp[i * N] = Wide<T>::down(G);
          acc = Num<W>::add(acc, Num<W>::mul_conj(G, Wide<T>::up(xb[i])));
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
// Same tiling as the constant-coefficient kernels; a chunk's summary is the affine map
// s -> P s + e with P the product of its coefficients, stored as double2 (P, e), composed in
// LDS across the K chunks of a super-chunk and through HBM across super-chunks.
TSF_DEV double2 compose(double2 first, double2 then) {  // apply `first`, then `then`
  return make_double2(then.x * first.x, fma(then.x, first.y, then.y));
}

template <int TC>
__global__ void __launch_bounds__(1024) sel_fwd_summary(const float* __restrict__ a, const float* __restrict__ v,
                                                        double2* __restrict__ E, int64_t lanes, int64_t L, int64_t N,
                                                        int64_t groups, int K) {
  __shared__ double2 s_e[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t g = blockIdx.x % groups, sc = blockIdx.x / groups;  // super-chunks 0 .. nsuper-2
  const int64_t lane = g * 64 + lid;
  const bool live = lane < lanes;
  double P = 1.0, e = 0.0;
  if (live) {
    const int64_t m = lane / N, n = lane - m * N;
    const int64_t base = (m * L + sc * K * TC + (int64_t)k * TC) * N + n;  // full chunks only
    float ab[TC], vb[TC];
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
  }
  s_e[k][lid] = make_double2(P, e);
  __syncthreads();
  if (k == 0 && live) {
    double2 s = s_e[0][lid];
    for (int j = 1; j < K; ++j) s = compose(s, s_e[j][lid]);
    E[sc * lanes + lane] = s;
  }
}

// In-place inclusive scan of n affine maps per lane: state_r = P_r state_{r-1} + e_r from
// init (NULL: zero); the state replaces e_r. Map r of a lane sits at S[(first + dir*r) * lanes
// + lane]. One workgroup per 64-lane group; wave k composes the k-th of 16 contiguous segments.
__global__ void __launch_bounds__(1024) sel_carry(const float* __restrict__ init, double2* __restrict__ S,
                                                  int64_t lanes, int64_t n, int64_t first, int64_t dir) {
  __shared__ double2 s_p[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t lane = blockIdx.x * 64 + lid;
  const bool live = lane < lanes;
  const int64_t seg = (n + kMaxWaves - 1) / kMaxWaves;
  const int64_t r0 = k * seg, r1 = (r0 + seg < n) ? r0 + seg : n;
  double2 p = make_double2(1.0, 0.0);
  if (live) {
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) p = compose(p, S[(first + dir * r) * lanes + lane]);
  }
  s_p[k][lid] = p;
  __syncthreads();
  if (live && r0 < r1) {
    double s = init ? (double)init[lane] : 0.0;
    for (int j = 0; j < k; ++j) s = fma(s_p[j][lid].x, s, s_p[j][lid].y);
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) {
      double2* q = S + (first + dir * r) * lanes + lane;
      const double2 m = *q;
      s = fma(m.x, s, m.y);
      q->y = s;
    }
  }
}

template <int TC>
__global__ void __launch_bounds__(1024) sel_fwd_apply(const float* __restrict__ a, const float* __restrict__ v,
                                                      const float* __restrict__ x0, const double2* __restrict__ E,
                                                      float* __restrict__ out, int64_t lanes, int64_t L, int64_t N,
                                                      int64_t groups, int K, int starts_ready) {
  __shared__ double2 s_e[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t g = blockIdx.x % groups, sc = blockIdx.x / groups;
  const int64_t lane = g * 64 + lid;
  const bool live = lane < lanes;
  const int64_t t0 = sc * K * TC + (int64_t)k * TC;
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
  s_e[k][lid] = make_double2(P, e);
  __syncthreads();
  if (!live || len == 0) return;  // no barrier follows
  double s = x0 ? (double)x0[lane] : 0.0;
  if (sc > 0) {
    if (starts_ready) {
      s = E[(sc - 1) * lanes + lane].y;
    } else {
#pragma unroll 8
      for (int64_t j = 0; j < sc; ++j) {
        const double2 mp = E[j * lanes + lane];
        s = fma(mp.x, s, mp.y);
      }
    }
  }
  for (int j = 0; j < k; ++j) s = fma(s_e[j][lid].x, s, s_e[j][lid].y);
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

// Reverse summary of super-chunk sc >= 1: the map G_enter -> G at its first step,
// G_t = g_t + a_{t+1} G_{t+1}, as (multiplier, value) with the multiplier the product of
// a_{t0+1} .. a_{t1} (a_{t1} is the next super-chunk's first coefficient). F [nsuper, lanes].
template <int TC>
__global__ void __launch_bounds__(1024) sel_bwd_summary(const float* __restrict__ a, const float* __restrict__ g,
                                                        double2* __restrict__ F, int64_t lanes, int64_t L, int64_t N,
                                                        int64_t groups, int K) {
  __shared__ double2 s_f[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t gr = blockIdx.x % groups, sc = blockIdx.x / groups + 1;  // super-chunks 1 .. nsuper-1
  const int64_t lane = gr * 64 + lid;
  const bool live = lane < lanes;
  const int64_t t0 = sc * K * TC + (int64_t)k * TC;
  const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
  double M = 1.0, f = 0.0;
  if (live && len > 0) {
    const int64_t m = lane / N, n = lane - m * N;
    const int64_t base = (m * L + t0) * N + n;
    float gb[TC], an[TC];  // g_t and a_{t+1} of the chunk's steps (a_L taken as 0: nothing enters)
    if (len == TC && t0 + TC < L) {  // full chunk with a following step: no per-step guard
#pragma unroll
      for (int i = 0; i < TC; ++i) {
        gb[i] = g[base + i * N];
        an[i] = a[base + (i + 1) * N];
      }
    } else {
#pragma unroll
      for (int i = 0; i < TC; ++i) {
        gb[i] = i < len ? g[base + i * N] : 0.0f;
        an[i] = (i < len && t0 + i + 1 < L) ? a[base + (i + 1) * N] : 0.0f;
      }
    }
#pragma unroll
    for (int i = TC - 1; i >= 0; --i)
      if (i < len) {
        f = fma((double)an[i], f, (double)gb[i]);
        M *= (double)an[i];
      }
  }
  s_f[k][lid] = make_double2(M, f);
  __syncthreads();
  if (k == 0 && live) {
    double2 s = s_f[K - 1][lid];
    for (int j = K - 2; j >= 0; --j) s = compose(s, s_f[j][lid]);
    F[sc * lanes + lane] = s;
  }
}

template <int TC>
__global__ void __launch_bounds__(1024) sel_bwd_apply(const float* __restrict__ a, const float* __restrict__ g,
                                                      const float* __restrict__ out, const float* __restrict__ x0,
                                                      const double2* __restrict__ F, float* __restrict__ glam,
                                                      float* __restrict__ gv, float* __restrict__ gx0, int64_t lanes,
                                                      int64_t L, int64_t N, int64_t groups, int K, int64_t nsuper,
                                                      int starts_ready) {
  __shared__ double2 s_f[kMaxWaves][64];
  const int lid = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int64_t gr = blockIdx.x % groups, sc = blockIdx.x / groups;
  const int64_t lane = gr * 64 + lid;
  const bool live = lane < lanes;
  const int64_t t0 = sc * K * TC + (int64_t)k * TC;
  const int len = (L - t0) >= TC ? TC : (L - t0) > 0 ? (int)(L - t0) : 0;
  double M = 1.0, f = 0.0;
  float gb[TC], an[TC], xb[TC];  // g_t, a_{t+1}, x_{t-1}
  int64_t base = 0;
  if (live && len > 0) {
    const int64_t m = lane / N, n = lane - m * N;
    base = (m * L + t0) * N + n;
    const float xinit = x0 ? x0[lane] : 0.0f;  // x_{-1}
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
  s_f[k][lid] = make_double2(M, f);
  __syncthreads();
  if (!live || len == 0) return;  // no barrier follows
  // G entering the super-chunk from the right: G at the first step of super-chunk sc + 1
  double R = 0.0;
  if (sc + 1 < nsuper) {
    if (starts_ready) {
      R = F[(sc + 1) * lanes + lane].y;
    } else {
      R = F[(nsuper - 1) * lanes + lane].y;
#pragma unroll 8
      for (int64_t j = nsuper - 2; j > sc; --j) {
        const double2 mp = F[j * lanes + lane];
        R = fma(mp.x, R, mp.y);
      }
    }
  }
  for (int j = K - 1; j > k; --j) R = fma(s_f[j][lid].x, R, s_f[j][lid].y);
  double G = R;
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

inline dim3 grid_for(int64_t threads) { return dim3((unsigned)((threads + 255) / 256)); }

// Tile shape of the constant-coefficient kernels for one call. TC (steps per chunk) is a
// template parameter: 16 or 32 for real lanes, 16 for complex ones (their backward keeps 2 x TC
// complex values per thread in registers, within the 128 VGPRs a 1024-thread workgroup allows).
// Every thread issues all TC loads of its chunk at once, so the bytes in flight do not depend on
// TC; the wave count (lanes / 64 x L / TC) does, and real lanes drop to TC = 16 when 32 would
// leave fewer than kDiagWaveTarget waves. K (chunks per workgroup) starts at 16, which keeps
// the super-chunk count and the summary folds small, and halves down to 4 only while the grid
// holds fewer than kDiagWgTarget workgroups. The carry kernel replaces the per-thread fold of
// super-chunk summaries once there are more than kDiagFoldMax of them.
#ifndef TSF_DIAG_WG_TARGET
#define TSF_DIAG_WG_TARGET 256
#endif
#ifndef TSF_DIAG_WAVE_TARGET
#define TSF_DIAG_WAVE_TARGET 4096
#endif
#ifndef TSF_DIAG_FOLD_MAX
#define TSF_DIAG_FOLD_MAX 16
#endif
constexpr int64_t kDiagWgTarget = TSF_DIAG_WG_TARGET;
constexpr int64_t kDiagWaveTarget = TSF_DIAG_WAVE_TARGET;
constexpr int64_t kDiagFoldMax = TSF_DIAG_FOLD_MAX;

struct DiagTile {
  int64_t lanes = 0, groups = 0, nsuper = 0, SL = 0;
  int TC = 0, K = 0;
  bool carry_kernel = false;
};

DiagTile diag_tile(int64_t lanes, int64_t L, bool cplx, int kmax = kMaxWaves) {
  DiagTile t;
  t.lanes = lanes;
  if (lanes < 1 || L < 1) return t;
  t.groups = (lanes + 63) / 64;
  t.TC = (cplx || t.groups * ((L + 31) / 32) < kDiagWaveTarget) ? 16 : 32;
  t.K = kmax;
  auto wgs = [&](int K) { return t.groups * ((L + (int64_t)t.TC * K - 1) / ((int64_t)t.TC * K)); };
  while (t.K > 4 && wgs(t.K) < kDiagWgTarget) t.K /= 2;
  const int64_t chunks = (L + t.TC - 1) / t.TC;
  if (t.K > chunks) t.K = (int)chunks;  // no waves past the end of a short sequence
  t.SL = (int64_t)t.TC * t.K;
  t.nsuper = (L + t.SL - 1) / t.SL;
  t.carry_kernel = t.nsuper - 1 > kDiagFoldMax;
  return t;
}

inline bool grid_fits(const DiagTile& t) { return t.groups * t.nsuper <= INT32_MAX; }

template <typename T, int TC>
void diag_fwd_launch(const DiagTile& t, const T* lam, const T* v, const T* x0, T* out, typename Wide<T>::type* E,
                     int64_t L, int64_t N, hipStream_t s) {
  const dim3 blk(64 * t.K);
  if (t.nsuper > 1) {
    hipLaunchKernelGGL((diag_fwd_summary<T, TC>), dim3((unsigned)(t.groups * (t.nsuper - 1))), blk, 0, s, lam, v, E,
                       t.lanes, L, N, t.groups, t.K);
    if (t.carry_kernel)
      hipLaunchKernelGGL(diag_carry<T>, dim3((unsigned)t.groups), dim3(64 * kMaxWaves), 0, s, lam, x0, E, t.lanes,
                         t.nsuper - 1, (int64_t)0, (int64_t)1, t.SL, 0);
  }
  hipLaunchKernelGGL((diag_fwd_apply<T, TC>), dim3((unsigned)(t.groups * t.nsuper)), blk, 0, s, lam, v, x0,
                     (const typename Wide<T>::type*)E, out, t.lanes, L, N, t.groups, t.K, (int)t.carry_kernel);
}

template <typename T, int TC>
void diag_bwd_launch(const DiagTile& t, const T* g, const T* lam, const T* out, const T* x0, T* gv, T* glam, T* gx0,
                     typename Wide<T>::type* F, typename Wide<T>::type* part, int64_t L, int64_t N, hipStream_t s) {
  const dim3 blk(64 * t.K);
  if (t.nsuper > 1) {
    hipLaunchKernelGGL((diag_bwd_summary<T, TC>), dim3((unsigned)(t.groups * (t.nsuper - 1))), blk, 0, s, lam, g, F,
                       t.lanes, L, N, t.groups, t.K);
    if (t.carry_kernel)
      hipLaunchKernelGGL(diag_carry<T>, dim3((unsigned)t.groups), dim3(64 * kMaxWaves), 0, s, lam, (const T*)nullptr,
                         F, t.lanes, t.nsuper - 1, t.nsuper - 1, (int64_t)-1, t.SL, 1);
  }
  hipLaunchKernelGGL((diag_bwd_apply<T, TC>), dim3((unsigned)(t.groups * t.nsuper)), blk, 0, s, lam, g, out, x0,
                     (const typename Wide<T>::type*)F, gv, part, glam, gx0, t.lanes, L, N, t.groups, t.K, t.nsuper,
                     (int)t.carry_kernel);
  if (t.nsuper > 1)
    hipLaunchKernelGGL(diag_sum_parts<T>, dim3((unsigned)t.groups), dim3(64 * kMaxWaves), 0, s,
                       (const typename Wide<T>::type*)part, glam, t.lanes, t.nsuper);
}

// The time-varying kernels use the same tiles; the backward keeps three TC-step arrays per
// thread (g_t, a_{t+1}, x_{t-1}), so it always runs TC = 16.
DiagTile sel_tile(int64_t lanes, int64_t L, bool bwd) { return diag_tile(lanes, L, bwd); }

template <int TC>
void sel_fwd_launch(const DiagTile& t, const float* a, const float* v, const float* x0, float* out, double2* E,
                    int64_t L, int64_t N, hipStream_t s) {
  const dim3 blk(64 * t.K);
  if (t.nsuper > 1) {
    hipLaunchKernelGGL((sel_fwd_summary<TC>), dim3((unsigned)(t.groups * (t.nsuper - 1))), blk, 0, s, a, v, E,
                       t.lanes, L, N, t.groups, t.K);
    if (t.carry_kernel)
      hipLaunchKernelGGL(sel_carry, dim3((unsigned)t.groups), dim3(64 * kMaxWaves), 0, s, x0, E, t.lanes,
                         t.nsuper - 1, (int64_t)0, (int64_t)1);
  }
  hipLaunchKernelGGL((sel_fwd_apply<TC>), dim3((unsigned)(t.groups * t.nsuper)), blk, 0, s, a, v, x0,
                     (const double2*)E, out, t.lanes, L, N, t.groups, t.K, (int)t.carry_kernel);
}

void sel_bwd_launch(const DiagTile& t, const float* g, const float* a, const float* out, const float* x0, float* glam,
                    float* gv, float* gx0, double2* F, int64_t L, int64_t N, hipStream_t s) {
  const dim3 blk(64 * t.K);
  if (t.nsuper > 1) {
    hipLaunchKernelGGL((sel_bwd_summary<16>), dim3((unsigned)(t.groups * (t.nsuper - 1))), blk, 0, s, a, g, F,
                       t.lanes, L, N, t.groups, t.K);
    if (t.carry_kernel)
      hipLaunchKernelGGL(sel_carry, dim3((unsigned)t.groups), dim3(64 * kMaxWaves), 0, s, (const float*)nullptr, F,
                         t.lanes, t.nsuper - 1, t.nsuper - 1, (int64_t)-1);
  }
  hipLaunchKernelGGL((sel_bwd_apply<16>), dim3((unsigned)(t.groups * t.nsuper)), blk, 0, s, a, g, out, x0,
                     (const double2*)F, glam, gv, gx0, t.lanes, L, N, t.groups, t.K, t.nsuper, (int)t.carry_kernel);
}

}  // namespace

extern "C" {

int64_t tsfast_hip_diag_workspace_bytes(int64_t M, int64_t L, int64_t N, int is_complex) {
  const DiagTile t = diag_tile(M * N, L, is_complex != 0);
  // fp64 super-chunk summaries [nsuper, lanes] plus fp64 glam partials [nsuper, lanes]
  // (complex128 when complex)
  return 2 * t.nsuper * t.lanes * (is_complex ? 16 : 8);
}

int tsfast_hip_diag_fwd(int64_t M, int64_t L, int64_t N, int is_complex, const void* lam, const void* v,
                        const void* x0, void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  if (M == 0 || L == 0 || N == 0) return TSF_OK;
  if (!lam || !v || !out) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_diag_workspace_bytes(M, L, N, is_complex) || !workspace) return TSF_ERR_WORKSPACE;
  const DiagTile t = diag_tile(M * N, L, is_complex != 0);
  if (!grid_fits(t)) return TSF_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (is_complex)
    diag_fwd_launch<float2, 16>(t, (const float2*)lam, (const float2*)v, (const float2*)x0, (float2*)out,
                                static_cast<double2*>(workspace), L, N, s);
  else if (t.TC == 32)
    diag_fwd_launch<float, 32>(t, (const float*)lam, (const float*)v, (const float*)x0, (float*)out,
                               static_cast<double*>(workspace), L, N, s);
  else
    diag_fwd_launch<float, 16>(t, (const float*)lam, (const float*)v, (const float*)x0, (float*)out,
                               static_cast<double*>(workspace), L, N, s);
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
  const DiagTile t = diag_tile(lanes, L, is_complex != 0);
  if (!grid_fits(t)) return TSF_ERR_UNSUPPORTED;
  if (is_complex) {
    auto* F = static_cast<double2*>(workspace);
    diag_bwd_launch<float2, 16>(t, (const float2*)g, (const float2*)lam, (const float2*)out, (const float2*)x0,
                                (float2*)gv, (float2*)glam, (float2*)gx0, F, F + t.nsuper * lanes, L, N, s);
  } else {
    auto* F = static_cast<double*>(workspace);
    if (t.TC == 32)
      diag_bwd_launch<float, 32>(t, (const float*)g, (const float*)lam, (const float*)out, (const float*)x0,
                                 (float*)gv, (float*)glam, (float*)gx0, F, F + t.nsuper * lanes, L, N, s);
    else
      diag_bwd_launch<float, 16>(t, (const float*)g, (const float*)lam, (const float*)out, (const float*)x0,
                                 (float*)gv, (float*)glam, (float*)gx0, F, F + t.nsuper * lanes, L, N, s);
  }
  return tsf_launch_status();
}

int64_t tsfast_hip_sel_workspace_bytes(int64_t M, int64_t L, int64_t N) {
  // fp64 (product, state) maps [nsuper, lanes] for the larger of the forward / backward tilings
  const DiagTile f = sel_tile(M * N, L, false), b = sel_tile(M * N, L, true);
  return (f.nsuper > b.nsuper ? f.nsuper : b.nsuper) * M * N * 16;
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
  auto* E = static_cast<double2*>(workspace);
  if (t.TC == 32)
    sel_fwd_launch<32>(t, a, v, x0, out, E, L, N, s);
  else
    sel_fwd_launch<16>(t, a, v, x0, out, E, L, N, s);
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
  sel_bwd_launch(t, g, a, out, x0, glam, gv, gx0, static_cast<double2*>(workspace), L, N, s);
  return tsf_launch_status();
}

}  // extern "C"
