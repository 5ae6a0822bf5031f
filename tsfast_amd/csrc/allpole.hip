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
// Parallel structure: time is cut into chunks of T_c steps and every (lane, chunk) pair is a
// thread. The state entering a chunk is the last NA outputs before it. A chunk maps its
// entering state s to  M s + e,  with M = C^{T_c} the companion matrix raised to the chunk
// length and e the chunk's zero-state end, so:
//   1. transfer   per lane: M by binary powering of C (NA x NA), stored in the workspace;
//   2. chunk_end  per (lane, chunk): e_c from a zero entering state;
//   3. carry      per lane: entering states S_c = M S_{c-1} + e_{c-1}, sequential over chunks;
//   4. apply      per (lane, chunk): run the chunk from S_c and write y.
// The adjoint G_t = g_t - sum_i a_i G_{t+i} is the same filter run backwards, so the backward
// reuses M with the chunk order reversed, accumulates grad_a partials per chunk, and a final
// per-lane kernel adds the y0 head taps and grad_y0.
#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

constexpr int kMaxNA = 16;

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
TSF_DEV void tile_fetch(TileRegs& rg, const float* __restrict__ src, int64_t lanes, int64_t L, int64_t l0, int64_t c0,
                        int ncol) {
  const int col = threadIdx.x & (kTileT - 1), half = threadIdx.x >> 5;
#pragma unroll
  for (int r2 = 0; r2 < kTile / 2; ++r2) {
    const int64_t lane = l0 + 2 * r2 + half;
    rg.v[r2] = (lane < lanes && col < ncol) ? src[lane * L + c0 + col] : 0.0f;
  }
}
TSF_DEV void tile_put(const TileRegs& rg, float (*tile)[kTileT + 1]) {
  const int col = threadIdx.x & (kTileT - 1), half = threadIdx.x >> 5;
#pragma unroll
  for (int r2 = 0; r2 < kTile / 2; ++r2) tile[2 * r2 + half][col] = rg.v[r2];
}
TSF_DEV void tile_store(float (*tile)[kTileT + 1], float* __restrict__ dst, int64_t lanes, int64_t L, int64_t l0,
                        int64_t c0, int ncol) {
  const int col = threadIdx.x & (kTileT - 1), half = threadIdx.x >> 5;
#pragma unroll 8
  for (int r2 = 0; r2 < kTile / 2; ++r2) {
    const int r = 2 * r2 + half;
    const int64_t lane = l0 + r;
    if (lane < lanes && col < ncol) dst[lane * L + c0 + col] = tile[r][col];
  }
}

// 1. M = C^{T_c} for the companion matrix C of lane `lane`: row 0 is (-a_1 .. -a_NA), row k is
//    the unit shift e_{k-1}. Stored row-major per lane.
template <int NA>
__global__ void __launch_bounds__(256) allpole_transfer(const float* __restrict__ a, double* __restrict__ Mout,
                                                        int64_t lanes, int64_t T_c) {
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  double P[NA][NA], R[NA][NA], T[NA][NA];
#pragma unroll
  for (int r = 0; r < NA; ++r)
#pragma unroll
    for (int c = 0; c < NA; ++c) {
      P[r][c] = (r == 0) ? -(double)a[lane * NA + c] : (c == r - 1 ? 1.0 : 0.0);
      R[r][c] = (r == c) ? 1.0 : 0.0;
    }
  int64_t k = T_c;
  while (k > 0) {
    if (k & 1) {
#pragma unroll
      for (int r = 0; r < NA; ++r)
#pragma unroll
        for (int c = 0; c < NA; ++c) {
          double s = 0.0;
#pragma unroll
          for (int j = 0; j < NA; ++j) s = fma(R[r][j], P[j][c], s);
          T[r][c] = s;
        }
#pragma unroll
      for (int r = 0; r < NA; ++r)
#pragma unroll
        for (int c = 0; c < NA; ++c) R[r][c] = T[r][c];
    }
    k >>= 1;
    if (k > 0) {
#pragma unroll
      for (int r = 0; r < NA; ++r)
#pragma unroll
        for (int c = 0; c < NA; ++c) {
          double s = 0.0;
#pragma unroll
          for (int j = 0; j < NA; ++j) s = fma(P[r][j], P[j][c], s);
          T[r][c] = s;
        }
#pragma unroll
      for (int r = 0; r < NA; ++r)
#pragma unroll
        for (int c = 0; c < NA; ++c) P[r][c] = T[r][c];
    }
  }
#pragma unroll
  for (int r = 0; r < NA; ++r)
#pragma unroll
    for (int c = 0; c < NA; ++c) Mout[(lane * NA + r) * NA + c] = R[r][c];
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
  tile_fetch(rg, w, lanes, L, l0, t0, (int)(T_c < kTileT ? T_c : kTileT));
  for (int64_t tt = 0; tt < T_c; tt += kTileT) {
    const int n = (int)((T_c - tt) < kTileT ? (T_c - tt) : kTileT);
    tile_put(rg, tile);
    __syncthreads();
    if (tt + kTileT < T_c)
      tile_fetch(rg, w, lanes, L, l0, t0 + tt + kTileT, (int)((T_c - tt - kTileT) < kTileT ? (T_c - tt - kTileT) : kTileT));
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

// 3. forward carries: entering state of every chunk, sequential over chunks per lane.
template <int NA>
__global__ void __launch_bounds__(256) allpole_fwd_carry(const double* __restrict__ M, const double* __restrict__ e,
                                                         const float* __restrict__ y0, double* __restrict__ S,
                                                         int64_t lanes, int64_t nchunk) {
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  double m[NA][NA], s[NA], t[NA];
#pragma unroll
  for (int r = 0; r < NA; ++r)
#pragma unroll
    for (int c = 0; c < NA; ++c) m[r][c] = M[(lane * NA + r) * NA + c];
#pragma unroll
  for (int k = 0; k < NA; ++k) s[k] = y0 ? (double)y0[lane * NA + k] : 0.0;
  for (int64_t c = 0; c < nchunk; ++c) {
#pragma unroll
    for (int k = 0; k < NA; ++k) S[(c * lanes + lane) * NA + k] = s[k];
    if (c + 1 < nchunk) {
#pragma unroll
      for (int r = 0; r < NA; ++r) {
        double acc = e[(c * lanes + lane) * NA + r];
#pragma unroll
        for (int j = 0; j < NA; ++j) acc = fma(m[r][j], s[j], acc);
        t[r] = acc;
      }
#pragma unroll
      for (int k = 0; k < NA; ++k) s[k] = t[k];
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
  tile_fetch(rg, w, lanes, L, l0, t0, (int)(len < kTileT ? len : kTileT));
  for (int64_t tt = 0; tt < len; tt += kTileT) {
    const int n = (int)((len - tt) < kTileT ? (len - tt) : kTileT);
    tile_put(rg, tile);
    __syncthreads();
    if (tt + kTileT < len)
      tile_fetch(rg, w, lanes, L, l0, t0 + tt + kTileT, (int)((len - tt - kTileT) < kTileT ? (len - tt - kTileT) : kTileT));
    if (n == kTileT) {
#pragma unroll
      for (int k = 0; k < kTileT; ++k) tile[tid][k] = (float)step<NA>(av, s, (double)tile[tid][k]);
    } else {
      for (int k = 0; k < n; ++k) tile[tid][k] = (float)step<NA>(av, s, (double)tile[tid][k]);
    }
    __syncthreads();
    tile_store(tile, y, lanes, L, l0, t0 + tt, n);
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
  tile_fetch(rg, g, lanes, L, l0, t0 + last, (int)((len - last) < kTileT ? (len - last) : kTileT));
  for (int64_t tt = last; tt >= 0; tt -= kTileT) {
    const int n = (int)((len - tt) < kTileT ? (len - tt) : kTileT);
    tile_put(rg, tile);
    __syncthreads();
    if (tt > 0) tile_fetch(rg, g, lanes, L, l0, t0 + tt - kTileT, kTileT);
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
// R_c = M R_{c+1} + f_{c+1}.
template <int NA>
__global__ void __launch_bounds__(256) allpole_bwd_carry(const double* __restrict__ M, const double* __restrict__ f,
                                                         double* __restrict__ R, int64_t lanes, int64_t nchunk) {
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  double m[NA][NA], s[NA], t[NA];
#pragma unroll
  for (int r = 0; r < NA; ++r)
#pragma unroll
    for (int c = 0; c < NA; ++c) m[r][c] = M[(lane * NA + r) * NA + c];
#pragma unroll
  for (int k = 0; k < NA; ++k) s[k] = 0.0;
  for (int64_t c = nchunk - 1; c >= 0; --c) {
#pragma unroll
    for (int k = 0; k < NA; ++k) R[(c * lanes + lane) * NA + k] = s[k];
    if (c > 0) {
      // exit of chunk c toward the left = entering state of chunk c-1
      const bool last = (c == nchunk - 1);  // its entering state is zero, M is irrelevant
#pragma unroll
      for (int r = 0; r < NA; ++r) {
        double acc = f[(c * lanes + lane) * NA + r];
        if (!last) {
#pragma unroll
          for (int j = 0; j < NA; ++j) acc = fma(m[r][j], s[j], acc);
        }
        t[r] = acc;
      }
#pragma unroll
      for (int k = 0; k < NA; ++k) s[k] = t[k];
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
  TileRegs rgg, rgy;
  {
    const int n0 = (int)((len - last) < kTileT ? (len - last) : kTileT);
    tile_fetch(rgg, g, lanes, L, l0, t0 + last, n0);
    tile_fetch(rgy, y, lanes, L, l0, t0 + last, n0);
  }
  for (int64_t tt = last; tt >= 0; tt -= kTileT) {
    const int n = (int)((len - tt) < kTileT ? (len - tt) : kTileT);
    tile_put(rgg, tg);
    tile_put(rgy, ty);
    __syncthreads();
    if (tt > 0) {
      tile_fetch(rgg, g, lanes, L, l0, t0 + tt - kTileT, kTileT);
      tile_fetch(rgy, y, lanes, L, l0, t0 + tt - kTileT, kTileT);
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
    tile_store(tg, gw, lanes, L, l0, t0 + tt, n);
    __syncthreads();
  }
  if (act) {
#pragma unroll
    for (int k = 0; k < NA; ++k) ga_part[(c * lanes + lane) * NA + k] = ga[k];
  }
}

// Backward 5. per lane: grad_a = -(sum of chunk partials + y0 head taps), grad_y0.
template <int NA>
__global__ void __launch_bounds__(256) allpole_bwd_finish(const float* __restrict__ a, const float* __restrict__ gw,
                                                          const float* __restrict__ y0,
                                                          const double* __restrict__ ga_part, float* __restrict__ ga,
                                                          float* __restrict__ gy0, int64_t lanes, int64_t L,
                                                          int64_t nchunk) {
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  double Gh[NA];  // G_0 .. G_{NA-1}, zero past the end of the sequence
#pragma unroll
  for (int k = 0; k < NA; ++k) Gh[k] = (k < L) ? (double)gw[lane * L + k] : 0.0;
#pragma unroll
  for (int k = 0; k < NA; ++k) {
    double acc = 0.0;
    for (int64_t c = 0; c < nchunk; ++c) acc += ga_part[(c * lanes + lane) * NA + k];
    if (y0) {
      // a_i (i = k + 1) also multiplied y_{t-i} = y0[i-t-1] for t < i
#pragma unroll
      for (int j = 1; j <= k + 1; ++j) acc = fma(Gh[k + 1 - j], (double)y0[lane * NA + j - 1], acc);
    }
    ga[lane * NA + k] = (float)(-acc);
  }
  if (y0 && gy0) {
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      double acc = 0.0;
#pragma unroll
      for (int i = j + 1; i <= NA; ++i) acc = fma((double)a[lane * NA + i - 1], Gh[i - 1 - j], acc);
      gy0[lane * NA + j] = (float)(-acc);
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
int fwd_impl(int64_t lanes, int64_t L, const float* a, const float* w, const float* y0, float* y, char* ws,
             hipStream_t s) {
  const Plan p = plan(lanes, L, NA);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  double* e = reinterpret_cast<double*>(ws + p.off_e);
  double* S = reinterpret_cast<double*>(ws + p.off_S);
  hipLaunchKernelGGL((allpole_transfer<NA>), grid_for(lanes), dim3(256), 0, s, a, M, lanes, p.T_c);
  const unsigned groups = (unsigned)((lanes + kTile - 1) / kTile);
  if (p.nchunk > 1)
    hipLaunchKernelGGL((allpole_fwd_chunk_end<NA>), dim3(groups, (unsigned)(p.nchunk - 1)), dim3(kTile), 0, s, a, w, e,
                       lanes, L, p.T_c, p.nchunk);
  hipLaunchKernelGGL((allpole_fwd_carry<NA>), grid_for(lanes), dim3(256), 0, s, M, e, y0, S, lanes, p.nchunk);
  hipLaunchKernelGGL((allpole_fwd_apply<NA>), dim3(groups, (unsigned)p.nchunk), dim3(kTile), 0, s, a, w, S, y, lanes,
                     L, p.T_c, p.nchunk);
  return tsf_launch_status();
}

template <int NA>
int bwd_impl(int64_t lanes, int64_t L, const float* g, const float* a, const float* y, const float* y0, float* gw,
             float* ga, float* gy0, char* ws, hipStream_t s) {
  const Plan p = plan(lanes, L, NA);
  double* M = reinterpret_cast<double*>(ws + p.off_M);
  double* f = reinterpret_cast<double*>(ws + p.off_e);
  double* R = reinterpret_cast<double*>(ws + p.off_S);
  double* part = reinterpret_cast<double*>(ws + p.off_part);
  if (L > 0) {
    hipLaunchKernelGGL((allpole_transfer<NA>), grid_for(lanes), dim3(256), 0, s, a, M, lanes, p.T_c);
    const unsigned groups = (unsigned)((lanes + kTile - 1) / kTile);
    if (p.nchunk > 1)
      hipLaunchKernelGGL((allpole_bwd_chunk_start<NA>), dim3(groups, (unsigned)(p.nchunk - 1)), dim3(kTile), 0, s, a,
                         g, f, lanes, L, p.T_c, p.nchunk);
    hipLaunchKernelGGL((allpole_bwd_carry<NA>), grid_for(lanes), dim3(256), 0, s, M, f, R, lanes, p.nchunk);
    hipLaunchKernelGGL((allpole_bwd_apply<NA>), dim3(groups, (unsigned)p.nchunk), dim3(kTile), 0, s, a, g, y, R, gw,
                       part, lanes, L, p.T_c, p.nchunk);
  }
  hipLaunchKernelGGL((allpole_bwd_finish<NA>), grid_for(lanes), dim3(256), 0, s, a, gw, y0, part, ga, gy0, lanes, L,
                     p.nchunk);
  return tsf_launch_status();
}

#define TSF_NA_CASES(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15) X(16)

}  // namespace

extern "C" {

int64_t tsfast_hip_allpole_workspace_bytes(int64_t lanes, int64_t L, int64_t na) {
  if (lanes < 0 || L < 0 || na < 1 || na > kMaxNA) return -1;
  return (int64_t)plan(lanes, L, na).bytes;
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
