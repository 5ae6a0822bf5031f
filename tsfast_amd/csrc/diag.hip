// Diagonal linear-recurrence scans on the lane layout [M, L, N] (N contiguous):
//   constant coefficient  x_t = lam * x_{t-1} + v_t            (lam [M, N], real or complex)
//   time-varying          x_t = a_t * x_{t-1} + v_t            (a   [M, L, N], real)
// and their adjoints G_t = g_t + conj(c_{t+1}) G_{t+1}.
//
// Reference semantics: tsfast/models/_core/scan.py:100-215 (ops), :52-80 (doubling scans),
// scan_backends/diagonal_triton.py:82-228 and selective_triton.py:48-109 (kernels).
//
// Parallel structure (chunked two-pass scan, no inter-workgroup waiting):
//   pass 1  one thread per (lane, time chunk) runs the chunk from a zero state and records the
//           chunk's end state (and, for time-varying coefficients, the product of its
//           coefficients) in a small carry buffer [nchunk, lanes].
//   pass 2  one thread per (lane, time chunk) composes the carries of the chunks before it
//           (Horner over at most nchunk small affine maps), then re-runs its chunk from the
//           true start state and streams the result out.
// Consecutive threads own consecutive lanes, so every per-step load/store is a coalesced row
// segment along N. The chunk count is picked on the host so that lanes x chunks fills the
// 256 CUs; the re-read of the input in pass 2 is the price of needing no global barrier.
#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

// All kernels load fp32 (or complex64) and carry the recurrence in fp64 (complex128): W below.
// ---------------------------------------------------------------- constant coefficient, forward
template <typename T>
__global__ void __launch_bounds__(256) diag_fwd_chunk_end(const T* __restrict__ lam, const T* __restrict__ v,
                                                          typename Wide<T>::type* __restrict__ carry, int64_t M,
                                                          int64_t L, int64_t N, int64_t T_c, int64_t nchunk) {
  using W = typename Wide<T>::type;
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes;  // chunks 0 .. nchunk-2 (the last chunk's end is never needed)
  if (c >= nchunk - 1) return;
  const int64_t m = lane / N, n = lane % N;
  const W a = Wide<T>::up(lam[lane]);
  const T* vp = v + (m * L + c * T_c) * N + n;
  W x = Num<W>::zero();
#pragma unroll 8
  for (int64_t i = 0; i < T_c; ++i) x = Num<W>::fma(a, x, Wide<T>::up(vp[i * N]));
  carry[c * lanes + lane] = x;
}

template <typename T>
__global__ void __launch_bounds__(256) diag_fwd_apply(const T* __restrict__ lam, const T* __restrict__ v,
                                                      const T* __restrict__ x0,
                                                      const typename Wide<T>::type* __restrict__ carry,
                                                      T* __restrict__ out, int64_t M, int64_t L, int64_t N,
                                                      int64_t T_c, int64_t nchunk) {
  using W = typename Wide<T>::type;
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes;
  if (c >= nchunk) return;
  const int64_t m = lane / N, n = lane % N;
  const W a = Wide<T>::up(lam[lane]);
  // state entering chunk c: x0 carried through the full-length chunks before it
  W x = x0 ? Wide<T>::up(x0[lane]) : Num<W>::zero();
  if (c > 0) {
    const W P = ipow(a, T_c);
    for (int64_t j = 0; j < c; ++j) x = Num<W>::fma(P, x, carry[j * lanes + lane]);
  }
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const T* vp = v + (m * L + t0) * N + n;
  T* op = out + (m * L + t0) * N + n;
#pragma unroll 8
  for (int64_t i = 0; i < len; ++i) {
    x = Num<W>::fma(a, x, Wide<T>::up(vp[i * N]));
    op[i * N] = Wide<T>::down(x);
  }
}

// ---------------------------------------------------------------- constant coefficient, backward
// Reverse chunk summaries: G at the chunk's first step with no gradient entering from the right.
template <typename T>
__global__ void __launch_bounds__(256) diag_bwd_chunk_start(const T* __restrict__ lam, const T* __restrict__ g,
                                                            typename Wide<T>::type* __restrict__ carry, int64_t M,
                                                            int64_t L, int64_t N, int64_t T_c, int64_t nchunk) {
  using W = typename Wide<T>::type;
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes + 1;  // chunks 1 .. nchunk-1 (chunk 0's start feeds nobody)
  if (c >= nchunk) return;
  const int64_t m = lane / N, n = lane % N;
  const W ac = Num<W>::conj(Wide<T>::up(lam[lane]));
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const T* gp = g + (m * L + t0) * N + n;
  W G = Num<W>::zero();
#pragma unroll 8
  for (int64_t i = len - 1; i >= 0; --i) G = Num<W>::fma(ac, G, Wide<T>::up(gp[i * N]));
  carry[c * lanes + lane] = G;
}

template <typename T>
__global__ void __launch_bounds__(256) diag_bwd_apply(const T* __restrict__ lam, const T* __restrict__ g,
                                                      const T* __restrict__ out, const T* __restrict__ x0,
                                                      const typename Wide<T>::type* __restrict__ carry,
                                                      T* __restrict__ gv, typename Wide<T>::type* __restrict__ glam_part,
                                                      T* __restrict__ gx0, int64_t M, int64_t L, int64_t N,
                                                      int64_t T_c, int64_t nchunk) {
  using W = typename Wide<T>::type;
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes;
  if (c >= nchunk) return;
  const int64_t m = lane / N, n = lane % N;
  const W ac = Num<W>::conj(Wide<T>::up(lam[lane]));
  // G at the first step of chunk c+1: fold the chunk summaries from the right end inwards.
  // Every chunk but the last has full length, and the last one receives no gradient.
  W R = Num<W>::zero();
  if (c + 1 < nchunk) {
    const W P = ipow(ac, T_c);
    R = carry[(nchunk - 1) * lanes + lane];
    for (int64_t j = nchunk - 2; j > c; --j) R = Num<W>::fma(P, R, carry[j * lanes + lane]);
  }
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const T* gp = g + (m * L + t0) * N + n;
  const T* xp = out + (m * L + t0) * N + n;
  T* gvp = gv + (m * L + t0) * N + n;
  W G = R;
  W acc = Num<W>::zero();
#pragma unroll 8
  for (int64_t i = len - 1; i >= 0; --i) {
    G = Num<W>::fma(ac, G, Wide<T>::up(gp[i * N]));
    gvp[i * N] = Wide<T>::down(G);
    W xprev;
    if (t0 + i > 0)
      xprev = Wide<T>::up(xp[(i - 1) * N]);
    else
      xprev = x0 ? Wide<T>::up(x0[lane]) : Num<W>::zero();
    acc = Num<W>::add(acc, Num<W>::mul_conj(G, xprev));
  }
  glam_part[c * lanes + lane] = acc;
  if (c == 0 && gx0) gx0[lane] = Wide<T>::down(Num<W>::mul(ac, G));
}

// Sum of per-chunk partials in a fixed order (deterministic run to run).
template <typename T>
__global__ void __launch_bounds__(256) sum_chunks(const typename Wide<T>::type* __restrict__ part,
                                                  T* __restrict__ dst, int64_t lanes, int64_t nchunk) {
  using W = typename Wide<T>::type;
  const int64_t lane = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (lane >= lanes) return;
  W s = Num<W>::zero();
  for (int64_t c = 0; c < nchunk; ++c) s = Num<W>::add(s, part[c * lanes + lane]);
  dst[lane] = Wide<T>::down(s);
}

// ---------------------------------------------------------------- time-varying coefficient (real)
// Pass-1 summary of a forward chunk: (product of its coefficients, end state from zero).
__global__ void __launch_bounds__(256) sel_fwd_chunk_end(const float* __restrict__ a, const float* __restrict__ v,
                                                         double2* __restrict__ carry, int64_t M, int64_t L, int64_t N,
                                                         int64_t T_c, int64_t nchunk) {
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes;
  if (c >= nchunk - 1) return;
  const int64_t m = lane / N, n = lane % N;
  const int64_t off = (m * L + c * T_c) * N + n;
  double P = 1.0, x = 0.0;
#pragma unroll 8
  for (int64_t i = 0; i < T_c; ++i) {
    const double at = a[off + i * N];
    x = fma(at, x, (double)v[off + i * N]);
    P *= at;
  }
  carry[c * lanes + lane] = make_double2(P, x);
}

__global__ void __launch_bounds__(256) sel_fwd_apply(const float* __restrict__ a, const float* __restrict__ v,
                                                     const float* __restrict__ x0, const double2* __restrict__ carry,
                                                     float* __restrict__ out, int64_t M, int64_t L, int64_t N,
                                                     int64_t T_c, int64_t nchunk) {
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes;
  if (c >= nchunk) return;
  const int64_t m = lane / N, n = lane % N;
  double x = x0 ? (double)x0[lane] : 0.0;
  for (int64_t j = 0; j < c; ++j) {
    const double2 pe = carry[j * lanes + lane];
    x = fma(pe.x, x, pe.y);
  }
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const int64_t off = (m * L + t0) * N + n;
#pragma unroll 8
  for (int64_t i = 0; i < len; ++i) {
    x = fma((double)a[off + i * N], x, (double)v[off + i * N]);
    out[off + i * N] = (float)x;
  }
}

// Reverse summary of chunk c >= 1: G at its first step with zero entering gradient, and the
// multiplier of the entering gradient, prod_{s=t0+1..t1} a_s (a_{t1} is the next chunk's first
// coefficient; the last chunk has no entering gradient, so its multiplier is never used).
__global__ void __launch_bounds__(256) sel_bwd_chunk_start(const float* __restrict__ a, const float* __restrict__ g,
                                                           double2* __restrict__ carry, int64_t M, int64_t L,
                                                           int64_t N, int64_t T_c, int64_t nchunk) {
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes + 1;
  if (c >= nchunk) return;
  const int64_t m = lane / N, n = lane % N;
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const int64_t off = (m * L + t0) * N + n;
  double G = 0.0, P = 1.0;
  for (int64_t i = len - 1; i >= 0; --i) {
    // G_t = g_t + a_{t+1} G_{t+1}; inside the chunk a_{t+1} is at i+1
    const double an = (i + 1 < len) ? (double)a[off + (i + 1) * N] : 1.0;
    G = fma(an, G, (double)g[off + i * N]);
    P *= an;
  }
  // the entering gradient passes through a_{t1}, the next chunk's first coefficient
  if (t0 + len < L) P *= a[off + len * N];
  carry[c * lanes + lane] = make_double2(P, G);
}

__global__ void __launch_bounds__(256) sel_bwd_apply(const float* __restrict__ a, const float* __restrict__ g,
                                                     const float* __restrict__ out, const float* __restrict__ x0,
                                                     const double2* __restrict__ carry, float* __restrict__ glam,
                                                     float* __restrict__ gv, float* __restrict__ gx0, int64_t M,
                                                     int64_t L, int64_t N, int64_t T_c, int64_t nchunk) {
  const int64_t lanes = M * N;
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t lane = gid % lanes;
  const int64_t c = gid / lanes;
  if (c >= nchunk) return;
  const int64_t m = lane / N, n = lane % N;
  // G_{t1} (first step of chunk c+1), folded from the right end
  double R = 0.0;
  if (c + 1 < nchunk) {
    R = carry[(nchunk - 1) * lanes + lane].y;
    for (int64_t j = nchunk - 2; j > c; --j) {
      const double2 pe = carry[j * lanes + lane];
      // pe.x multiplies G at the first step of chunk j+1
      R = fma(pe.x, R, pe.y);
    }
  }
  const int64_t t0 = c * T_c;
  const int64_t len = (L - t0) < T_c ? (L - t0) : T_c;
  const int64_t off = (m * L + t0) * N + n;
  double G = R;
  for (int64_t i = len - 1; i >= 0; --i) {
    const int64_t t = t0 + i;
    const double an = (t + 1 < L) ? (double)a[off + (i + 1) * N] : 1.0;
    G = fma(an, G, (double)g[off + i * N]);
    gv[off + i * N] = (float)G;
    const double xprev = (t > 0) ? (double)out[off + (i - 1) * N] : (x0 ? (double)x0[lane] : 0.0);
    glam[off + i * N] = (float)(G * xprev);
  }
  if (c == 0 && gx0) gx0[lane] = (float)((double)a[off] * G);
}

// Chunk length: enough (lane, chunk) threads to cover the device several times over, but
// chunks long enough that the carry fold (O(nchunk) per thread) stays negligible.
int64_t pick_chunk(int64_t lanes, int64_t L) {
  if (L < 1) return 1;
  const int64_t target_threads = 256 * 1024 * 2;  // ~8 waves of 64 per SIMD on 256 CUs
  int64_t T_c = L;
  while (T_c > 64 && lanes * ((L + T_c - 1) / T_c) < target_threads) T_c = (T_c + 1) / 2;
  if (T_c < 1) T_c = 1;
  return T_c;
}

inline dim3 grid_for(int64_t threads) { return dim3((unsigned)((threads + 255) / 256)); }

}  // namespace

extern "C" {

int64_t tsfast_hip_diag_workspace_bytes(int64_t M, int64_t L, int64_t N, int is_complex) {
  const int64_t lanes = M * N;
  const int64_t T_c = pick_chunk(lanes, L);
  const int64_t nchunk = (L + T_c - 1) / T_c;
  // fp64 carries [nchunk, lanes] plus fp64 glam partials [nchunk, lanes] (complex128 when complex)
  return 2 * nchunk * lanes * (is_complex ? 16 : 8);
}

int tsfast_hip_diag_fwd(int64_t M, int64_t L, int64_t N, int is_complex, const void* lam, const void* v,
                        const void* x0, void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  if (M == 0 || L == 0 || N == 0) return TSF_OK;
  if (!lam || !v || !out) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_diag_workspace_bytes(M, L, N, is_complex) || !workspace) return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t lanes = M * N;
  const int64_t T_c = pick_chunk(lanes, L);
  const int64_t nchunk = (L + T_c - 1) / T_c;
  if (is_complex) {
    auto* c = static_cast<double2*>(workspace);
    if (nchunk > 1)
      hipLaunchKernelGGL(diag_fwd_chunk_end<float2>, grid_for(lanes * (nchunk - 1)), dim3(256), 0, s,
                         (const float2*)lam, (const float2*)v, c, M, L, N, T_c, nchunk);
    hipLaunchKernelGGL(diag_fwd_apply<float2>, grid_for(lanes * nchunk), dim3(256), 0, s, (const float2*)lam,
                       (const float2*)v, (const float2*)x0, c, (float2*)out, M, L, N, T_c, nchunk);
  } else {
    auto* c = static_cast<double*>(workspace);
    if (nchunk > 1)
      hipLaunchKernelGGL(diag_fwd_chunk_end<float>, grid_for(lanes * (nchunk - 1)), dim3(256), 0, s,
                         (const float*)lam, (const float*)v, c, M, L, N, T_c, nchunk);
    hipLaunchKernelGGL(diag_fwd_apply<float>, grid_for(lanes * nchunk), dim3(256), 0, s, (const float*)lam,
                       (const float*)v, (const float*)x0, c, (float*)out, M, L, N, T_c, nchunk);
  }
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
    const size_t esz = is_complex ? 8 : 4;
    if (hipMemsetAsync(glam, 0, lanes * esz, s) != hipSuccess) return TSF_ERR_HIP;
    if (gx0 && hipMemsetAsync(gx0, 0, lanes * esz, s) != hipSuccess) return TSF_ERR_HIP;
    return TSF_OK;
  }
  if (!g || !out || !gv) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_diag_workspace_bytes(M, L, N, is_complex) || !workspace) return TSF_ERR_WORKSPACE;
  const int64_t T_c = pick_chunk(lanes, L);
  const int64_t nchunk = (L + T_c - 1) / T_c;
  if (is_complex) {
    auto* c = static_cast<double2*>(workspace);
    auto* part = c + nchunk * lanes;
    if (nchunk > 1)
      hipLaunchKernelGGL(diag_bwd_chunk_start<float2>, grid_for(lanes * (nchunk - 1)), dim3(256), 0, s,
                         (const float2*)lam, (const float2*)g, c, M, L, N, T_c, nchunk);
    hipLaunchKernelGGL(diag_bwd_apply<float2>, grid_for(lanes * nchunk), dim3(256), 0, s, (const float2*)lam,
                       (const float2*)g, (const float2*)out, (const float2*)x0, c, (float2*)gv, part, (float2*)gx0, M,
                       L, N, T_c, nchunk);
    hipLaunchKernelGGL(sum_chunks<float2>, grid_for(lanes), dim3(256), 0, s, part, (float2*)glam, lanes, nchunk);
  } else {
    auto* c = static_cast<double*>(workspace);
    auto* part = c + nchunk * lanes;
    if (nchunk > 1)
      hipLaunchKernelGGL(diag_bwd_chunk_start<float>, grid_for(lanes * (nchunk - 1)), dim3(256), 0, s,
                         (const float*)lam, (const float*)g, c, M, L, N, T_c, nchunk);
    hipLaunchKernelGGL(diag_bwd_apply<float>, grid_for(lanes * nchunk), dim3(256), 0, s, (const float*)lam,
                       (const float*)g, (const float*)out, (const float*)x0, c, (float*)gv, part, (float*)gx0, M, L,
                       N, T_c, nchunk);
    hipLaunchKernelGGL(sum_chunks<float>, grid_for(lanes), dim3(256), 0, s, part, (float*)glam, lanes, nchunk);
  }
  return tsf_launch_status();
}

int64_t tsfast_hip_sel_workspace_bytes(int64_t M, int64_t L, int64_t N) {
  const int64_t lanes = M * N;
  const int64_t T_c = pick_chunk(lanes, L);
  const int64_t nchunk = (L + T_c - 1) / T_c;
  return nchunk * lanes * 16;  // fp64 (product, state) pairs
}

int tsfast_hip_sel_fwd(int64_t M, int64_t L, int64_t N, const float* a, const float* v, const float* x0, float* out,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  if (M < 0 || L < 0 || N < 0) return TSF_ERR_ARG;
  if (M == 0 || L == 0 || N == 0) return TSF_OK;
  if (!a || !v || !out) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_sel_workspace_bytes(M, L, N) || !workspace) return TSF_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t lanes = M * N;
  const int64_t T_c = pick_chunk(lanes, L);
  const int64_t nchunk = (L + T_c - 1) / T_c;
  auto* c = static_cast<double2*>(workspace);
  if (nchunk > 1)
    hipLaunchKernelGGL(sel_fwd_chunk_end, grid_for(lanes * (nchunk - 1)), dim3(256), 0, s, a, v, c, M, L, N, T_c,
                       nchunk);
  hipLaunchKernelGGL(sel_fwd_apply, grid_for(lanes * nchunk), dim3(256), 0, s, a, v, x0, c, out, M, L, N, T_c, nchunk);
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
    if (gx0 && hipMemsetAsync(gx0, 0, lanes * 4, s) != hipSuccess) return TSF_ERR_HIP;
    return TSF_OK;
  }
  if (!g || !a || !out || !gv || !glam) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_sel_workspace_bytes(M, L, N) || !workspace) return TSF_ERR_WORKSPACE;
  const int64_t T_c = pick_chunk(lanes, L);
  const int64_t nchunk = (L + T_c - 1) / T_c;
  auto* c = static_cast<double2*>(workspace);
  if (nchunk > 1)
    hipLaunchKernelGGL(sel_bwd_chunk_start, grid_for(lanes * (nchunk - 1)), dim3(256), 0, s, a, g, c, M, L, N, T_c,
                       nchunk);
  hipLaunchKernelGGL(sel_bwd_apply, grid_for(lanes * nchunk), dim3(256), 0, s, a, g, out, x0, c, glam, gv, gx0, M, L,
                     N, T_c, nchunk);
  return tsf_launch_status();
}

}  // extern "C"
