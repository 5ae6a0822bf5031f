// CPU baseline: C++/OpenMP port of the reference CPU kernels for the scan family — TEST
// INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and tests; never part of the product).
//
// mamba_fwd / mamba_bwd restate tsfast/models/architectures/mamba/backend_c.py:105-245:
//   tasks (batch, block of BD=8 channels), state h[BD][N] in registers, N a compile-time
//   constant, one checkpoint every CHK=16 steps (slot k = state after step (k+1)*CHK-1); the
//   backward walks the checkpoints in reverse, recomputes each chunk into a small L1 buffer and
//   sweeps it backwards with G_t = gy_t C_t + lam_{t+1} G_{t+1}; grad B_t / grad C_t go to
//   per-block partial buffers [nblk, B, L, N] and grad A / grad Dp to per-batch partials, which
//   the caller sums (the reference sums them in torch, backend_c.py:432-441).
// diag_fwd / diag_bwd restate scan_backends/diagonal_c.py:53-443 for the single-pass case the
//   reference takes at configs 1, 2 and 5 (tasks = (row, 64-lane block), time walked once).
//
// Build (compile and link split, as tsfast/models/_core/kernel_c.py:136-150, 248-270 does, so
// the fast-math objects do not turn on flush-to-zero for the whole process):
//   g++ -O3 -march=native -ffast-math -fopenmp -fPIC -c cpu_baseline.cpp
//   g++ -shared -fopenmp cpu_baseline.o -o libtsfast_cpu_baseline.so
#include <omp.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstring>

namespace {

constexpr int BD = 8;
constexpr int CHK = 16;

// The reference CPU kernel's own exp (mamba/backend_c.py:55-74), so that this column times the
// reference's CPU arithmetic: clamp to [-88, 88]; x = k ln2 + r with k = round(x / ln2), ln2
// taken as the float 0.693359375 minus 2.12194440e-4 (a Cody-Waite split: k * 0.693359375 is
// exact in float for |k| <= 128); e^r by its Taylor series through r^6 / 6!; 2^k from the
// exponent bits. Plain arithmetic keeps the state loop vectorisable, as in the reference.
inline float ref_expf(float x) {
  x = std::min(88.0f, std::max(-88.0f, x));
  const float t = x * 1.44269504088896341f;
  const int32_t k = (int32_t)(t >= 0.0f ? t + 0.5f : t - 0.5f);
  const float kf = (float)k;
  const float r = (x - kf * 0.693359375f) + kf * 2.12194440e-4f;
  // sum_{n<=6} r^n / n!, Horner form from the highest power
  float p = 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  int32_t bits = (k + 127) << 23;
  float scale;
  std::memcpy(&scale, &bits, sizeof(scale));
  return p * scale;
}
inline float softplusf(float x) { return x > 20.0f ? x : std::log1p(ref_expf(x)); }
inline float sigmoidf(float x) { return 1.0f / (1.0f + ref_expf(-x)); }

template <int N>
void mamba_fwd_t(int64_t B, int64_t L, int64_t D, const float* draw, const float* A, const float* Bt,
                 const float* Ct, const float* u, const float* z, const float* Dp, const float* h0, float* out,
                 float* chk, float* hlast) {
  const int64_t nblk = (D + BD - 1) / BD, nc = (L + CHK - 1) / CHK;
#pragma omp parallel for schedule(dynamic)
  for (int64_t task = 0; task < B * nblk; ++task) {
    const int64_t b = task / nblk, d0 = (task % nblk) * BD;
    const int nd = (int)std::min<int64_t>(BD, D - d0);
    float h[BD][N];
    for (int j = 0; j < nd; ++j)
      for (int n = 0; n < N; ++n) h[j][n] = h0 ? h0[(b * D + d0 + j) * N + n] : 0.0f;
    for (int64_t t = 0; t < L; ++t) {
      const float* bt = Bt + (b * L + t) * N;
      const float* ct = Ct + (b * L + t) * N;
      const int64_t row = (b * L + t) * D + d0;
      for (int j = 0; j < nd; ++j) {
        const float* a = A + (d0 + j) * N;
        const float dl = softplusf(draw[row + j]);
        const float uu = u[row + j], du = dl * uu;
        float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
        for (int n = 0; n < N; ++n) {
          const float hv = ref_expf(dl * a[n]) * h[j][n] + du * bt[n];
          h[j][n] = hv;
          acc += hv * ct[n];
        }
        const float zz = z[row + j];
        out[row + j] = (acc + Dp[d0 + j] * uu) * zz * sigmoidf(zz);
      }
      if (chk && (t + 1) % CHK == 0) {
        const int64_t slot = (t + 1) / CHK - 1;
        for (int j = 0; j < nd; ++j) std::memcpy(chk + ((b * nc + slot) * D + d0 + j) * N, h[j], sizeof(float) * N);
      }
    }
    for (int j = 0; j < nd; ++j) std::memcpy(hlast + (b * D + d0 + j) * N, h[j], sizeof(float) * N);
  }
}

template <int N>
void mamba_bwd_t(int64_t B, int64_t L, int64_t D, const float* draw, const float* A, const float* Bt,
                 const float* Ct, const float* u, const float* z, const float* Dp, const float* h0, const float* chk,
                 const float* gout, const float* ghlast, float* gdraw, float* gA_part, float* gBt_part,
                 float* gCt_part, float* gu, float* gz, float* gDp_part, float* gh0) {
  const int64_t nblk = (D + BD - 1) / BD, nc = (L + CHK - 1) / CHK;
#pragma omp parallel for schedule(dynamic)
  for (int64_t task = 0; task < B * nblk; ++task) {
    const int64_t b = task / nblk, blk = task % nblk, d0 = blk * BD;
    const int nd = (int)std::min<int64_t>(BD, D - d0);
    float G[BD][N], gA[BD][N], hs[BD][N], hbuf[CHK][BD][N], dbuf[CHK][BD], gdp[BD];
    for (int j = 0; j < nd; ++j) {
      gdp[j] = 0.0f;
      for (int n = 0; n < N; ++n) {
        G[j][n] = ghlast ? ghlast[(b * D + d0 + j) * N + n] : 0.0f;
        gA[j][n] = 0.0f;
      }
    }
    float* gBp = gBt_part + (blk * B + b) * L * N;
    float* gCp = gCt_part + (blk * B + b) * L * N;
    std::memset(gBp, 0, sizeof(float) * L * N);
    std::memset(gCp, 0, sizeof(float) * L * N);
    for (int64_t c = nc - 1; c >= 0; --c) {
      const int64_t t0 = c * CHK;
      const int len = (int)(std::min<int64_t>(L, t0 + CHK) - t0);
      for (int j = 0; j < nd; ++j)
        for (int n = 0; n < N; ++n)
          hs[j][n] = c > 0 ? chk[((b * nc + c - 1) * D + d0 + j) * N + n] : (h0 ? h0[(b * D + d0 + j) * N + n] : 0.0f);
      for (int i = 0; i < len; ++i) {
        const float* bt = Bt + (b * L + t0 + i) * N;
        const int64_t row = (b * L + t0 + i) * D + d0;
        for (int j = 0; j < nd; ++j) {
          const float* a = A + (d0 + j) * N;
          const float dl = softplusf(draw[row + j]);
          const float du = dl * u[row + j];
          dbuf[i][j] = dl;
#pragma omp simd
          for (int n = 0; n < N; ++n) {
            hs[j][n] = ref_expf(dl * a[n]) * hs[j][n] + du * bt[n];
            hbuf[i][j][n] = hs[j][n];
          }
        }
      }
      for (int i = len - 1; i >= 0; --i) {
        const int64_t t = t0 + i;
        const float* bt = Bt + (b * L + t) * N;
        const float* ct = Ct + (b * L + t) * N;
        const int64_t row = (b * L + t) * D + d0;
        float* gBr = gBp + t * N;
        float* gCr = gCp + t * N;
        for (int j = 0; j < nd; ++j) {
          const float* a = A + (d0 + j) * N;
          const float* hv = hbuf[i][j];
          const float dl = dbuf[i][j];
          const float uu = u[row + j], zz = z[row + j], du = dl * uu;
          float y = Dp[d0 + j] * uu;
          for (int n = 0; n < N; ++n) y += hv[n] * ct[n];
          const float sg = sigmoidf(zz), go = gout[row + j];
          const float gy = go * zz * sg;
          gz[row + j] = go * y * sg * (1.0f + zz * (1.0f - sg));
          gdp[j] += gy * uu;
          if (t + 1 < L) {
            const float dn = softplusf(draw[row + j + D]);
#pragma omp simd
            for (int n = 0; n < N; ++n) G[j][n] = gy * ct[n] + ref_expf(dn * a[n]) * G[j][n];
          } else {
            for (int n = 0; n < N; ++n) G[j][n] = gy * ct[n] + G[j][n];
          }
          float gdelta = 0.0f, gus = 0.0f;
#pragma omp simd reduction(+ : gdelta, gus)
          for (int n = 0; n < N; ++n) {
            const float lh = hv[n] - du * bt[n], g = G[j][n];
            gCr[n] += gy * hv[n];
            gBr[n] += g * du;
            gA[j][n] += g * lh * dl;
            gdelta += g * (a[n] * lh + uu * bt[n]);
            gus += g * bt[n];
          }
          gdraw[row + j] = gdelta * sigmoidf(draw[row + j]);
          gu[row + j] = dl * gus + gy * Dp[d0 + j];
        }
      }
    }
    for (int j = 0; j < nd; ++j) {
      gDp_part[b * D + d0 + j] = gdp[j];
      std::memcpy(gA_part + (b * D + d0 + j) * N, gA[j], sizeof(float) * N);
    }
    if (gh0) {
      for (int j = 0; j < nd; ++j) {
        const float* a = A + (d0 + j) * N;
        const float d_0 = L > 0 ? softplusf(draw[b * L * D + d0 + j]) : 0.0f;
        for (int n = 0; n < N; ++n) gh0[(b * D + d0 + j) * N + n] = ref_expf(d_0 * a[n]) * G[j][n];
      }
    }
  }
}

// Constant-coefficient diagonal scan, real (re only) or complex (interleaved re/im), single pass.
constexpr int KMAX = 64;

void diag_fwd_impl(int64_t M, int64_t L, int64_t N, int cplx, const float* lam, const float* v, const float* x0,
                   float* out) {
  const int64_t nblk = (N + KMAX - 1) / KMAX;
  const int w = cplx ? 2 : 1;
#pragma omp parallel for schedule(dynamic)
  for (int64_t task = 0; task < M * nblk; ++task) {
    const int64_t m = task / nblk, k0 = (task % nblk) * KMAX;
    const int nk = (int)std::min<int64_t>(KMAX, N - k0);
    float xr[KMAX], xi[KMAX], lr[KMAX], li[KMAX];
    for (int k = 0; k < nk; ++k) {
      const int64_t o = (m * N + k0 + k) * w;
      lr[k] = lam[o];
      li[k] = cplx ? lam[o + 1] : 0.0f;
      xr[k] = x0 ? x0[o] : 0.0f;
      xi[k] = (x0 && cplx) ? x0[o + 1] : 0.0f;
    }
    for (int64_t t = 0; t < L; ++t) {
      const float* vp = v + ((m * L + t) * N + k0) * w;
      float* op = out + ((m * L + t) * N + k0) * w;
      if (cplx) {
#pragma omp simd
        for (int k = 0; k < nk; ++k) {
          const float r = lr[k] * xr[k] - li[k] * xi[k] + vp[2 * k];
          const float i = lr[k] * xi[k] + li[k] * xr[k] + vp[2 * k + 1];
          xr[k] = r;
          xi[k] = i;
          op[2 * k] = r;
          op[2 * k + 1] = i;
        }
      } else {
#pragma omp simd
        for (int k = 0; k < nk; ++k) {
          xr[k] = lr[k] * xr[k] + vp[k];
          op[k] = xr[k];
        }
      }
    }
  }
}

void diag_bwd_impl(int64_t M, int64_t L, int64_t N, int cplx, const float* g, const float* lam, const float* out,
                   const float* x0, float* gv, float* glam, float* gx0) {
  const int64_t nblk = (N + KMAX - 1) / KMAX;
  const int w = cplx ? 2 : 1;
#pragma omp parallel for schedule(dynamic)
  for (int64_t task = 0; task < M * nblk; ++task) {
    const int64_t m = task / nblk, k0 = (task % nblk) * KMAX;
    const int nk = (int)std::min<int64_t>(KMAX, N - k0);
    float Gr[KMAX], Gi[KMAX], lr[KMAX], li[KMAX], ar[KMAX], ai[KMAX];
    for (int k = 0; k < nk; ++k) {
      const int64_t o = (m * N + k0 + k) * w;
      lr[k] = lam[o];
      li[k] = cplx ? -lam[o + 1] : 0.0f;  // conj(lam)
      Gr[k] = Gi[k] = ar[k] = ai[k] = 0.0f;
    }
    for (int64_t t = L - 1; t >= 0; --t) {
      const float* gp = g + ((m * L + t) * N + k0) * w;
      float* gvp = gv + ((m * L + t) * N + k0) * w;
      const float* xp = t > 0 ? out + ((m * L + t - 1) * N + k0) * w : (x0 ? x0 + (m * N + k0) * w : nullptr);
      if (cplx) {
        for (int k = 0; k < nk; ++k) {
          const float r = lr[k] * Gr[k] - li[k] * Gi[k] + gp[2 * k];
          const float i = lr[k] * Gi[k] + li[k] * Gr[k] + gp[2 * k + 1];
          Gr[k] = r;
          Gi[k] = i;
          gvp[2 * k] = r;
          gvp[2 * k + 1] = i;
          if (xp) {  // G * conj(x)
            ar[k] += r * xp[2 * k] + i * xp[2 * k + 1];
            ai[k] += i * xp[2 * k] - r * xp[2 * k + 1];
          }
        }
      } else {
        for (int k = 0; k < nk; ++k) {
          Gr[k] = lr[k] * Gr[k] + gp[k];
          gvp[k] = Gr[k];
          if (xp) ar[k] += Gr[k] * xp[k];
        }
      }
    }
    for (int k = 0; k < nk; ++k) {
      const int64_t o = (m * N + k0 + k) * w;
      glam[o] = ar[k];
      if (cplx) glam[o + 1] = ai[k];
      if (gx0) {
        gx0[o] = lr[k] * Gr[k] - li[k] * Gi[k];
        if (cplx) gx0[o + 1] = lr[k] * Gi[k] + li[k] * Gr[k];
      }
    }
  }
}

// Time-varying diagonal scan (scan_backends/selective_c.py:45-121): one task per (row, 64-lane
// tile) keeps the tile's state resident and streams over L; the inner lane loop vectorises.
void sel_fwd_impl(int64_t M, int64_t L, int64_t N, const float* a, const float* v, const float* x0, float* out) {
  const int64_t nt = (N + 63) / 64;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * nt; ++i) {
    const int64_t m = i / nt, n0 = (i % nt) * 64;
    const int nw = (int)std::min<int64_t>(64, N - n0);
    float x[64];
    for (int j = 0; j < nw; ++j) x[j] = x0 ? x0[m * N + n0 + j] : 0.0f;
    for (int64_t t = 0; t < L; ++t) {
      const int64_t p = (m * L + t) * N + n0;
      for (int j = 0; j < nw; ++j) {
        x[j] = a[p + j] * x[j] + v[p + j];
        out[p + j] = x[j];
      }
    }
  }
}

void sel_bwd_impl(int64_t M, int64_t L, int64_t N, const float* g, const float* a, const float* out,
                  const float* x0, float* glam, float* gv, float* gx0) {
  const int64_t nt = (N + 63) / 64;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * nt; ++i) {
    const int64_t m = i / nt, n0 = (i % nt) * 64;
    const int nw = (int)std::min<int64_t>(64, N - n0);
    float G[64];
    for (int j = 0; j < nw; ++j) G[j] = 0.0f;
    for (int64_t t = L - 1; t >= 0; --t) {
      const int64_t p = (m * L + t) * N + n0;
      for (int j = 0; j < nw; ++j) {
        G[j] = g[p + j] + (t + 1 < L ? a[p + N + j] * G[j] : 0.0f);
        gv[p + j] = G[j];
        const float xp = t > 0 ? out[p - N + j] : (x0 ? x0[m * N + n0 + j] : 0.0f);
        glam[p + j] = G[j] * xp;
      }
      if (t == 0 && gx0)
        for (int j = 0; j < nw; ++j) gx0[m * N + n0 + j] = a[p + j] * G[j];
    }
  }
}

}  // namespace

#define TSF_CPU_NS(X) X(1) X(2) X(3) X(4) X(8) X(12) X(16) X(32) X(64)

extern "C" {

int cpu_num_threads(void) { return omp_get_max_threads(); }
void cpu_set_threads(int n) { omp_set_num_threads(n); }

// ref_expf elementwise (for its accuracy pin in the tests)
void cpu_ref_expf(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = ref_expf(x[i]);
}

int cpu_mamba_chk(void) { return CHK; }
int cpu_mamba_bd(void) { return BD; }

int cpu_mamba_fwd(int64_t B, int64_t L, int64_t D, int64_t N, const float* draw, const float* A, const float* Bt,
                  const float* Ct, const float* u, const float* z, const float* Dp, const float* h0, float* out,
                  float* chk, float* hlast) {
  switch (N) {
#define X(K)                                                                      \
  case K:                                                                         \
    mamba_fwd_t<K>(B, L, D, draw, A, Bt, Ct, u, z, Dp, h0, out, chk, hlast);      \
    return 0;
    TSF_CPU_NS(X)
#undef X
  }
  return -3;
}

int cpu_mamba_bwd(int64_t B, int64_t L, int64_t D, int64_t N, const float* draw, const float* A, const float* Bt,
                  const float* Ct, const float* u, const float* z, const float* Dp, const float* h0, const float* chk,
                  const float* gout, const float* ghlast, float* gdraw, float* gA_part, float* gBt_part,
                  float* gCt_part, float* gu, float* gz, float* gDp_part, float* gh0) {
  switch (N) {
#define X(K)                                                                                                   \
  case K:                                                                                                      \
    mamba_bwd_t<K>(B, L, D, draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gA_part, gBt_part, gCt_part, \
                   gu, gz, gDp_part, gh0);                                                                     \
    return 0;
    TSF_CPU_NS(X)
#undef X
  }
  return -3;
}

int cpu_diag_fwd(int64_t M, int64_t L, int64_t N, int cplx, const float* lam, const float* v, const float* x0,
                 float* out) {
  diag_fwd_impl(M, L, N, cplx, lam, v, x0, out);
  return 0;
}

int cpu_diag_bwd(int64_t M, int64_t L, int64_t N, int cplx, const float* g, const float* lam, const float* out,
                 const float* x0, float* gv, float* glam, float* gx0) {
  diag_bwd_impl(M, L, N, cplx, g, lam, out, x0, gv, glam, gx0);
  return 0;
}

int cpu_sel_fwd(int64_t M, int64_t L, int64_t N, const float* a, const float* v, const float* x0, float* out) {
  sel_fwd_impl(M, L, N, a, v, x0, out);
  return 0;
}

int cpu_sel_bwd(int64_t M, int64_t L, int64_t N, const float* g, const float* a, const float* out, const float* x0,
                float* glam, float* gv, float* gx0) {
  sel_bwd_impl(M, L, N, g, a, out, x0, glam, gv, gx0);
  return 0;
}

}  // extern "C"
