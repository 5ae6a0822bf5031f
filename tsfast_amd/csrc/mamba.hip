// Fused Mamba selective SSM, forward and backward, bf16 or fp32 I/O with fp32 state.
//
//   delta_t = softplus(draw_t)                        (threshold 20, as F.softplus)
//   h_t     = exp(delta_t A) * h_{t-1} + delta_t u_t B_t
//   out_t   = (sum_n h_t C_t + Dp u_t) * z_t * sigmoid(z_t)
//
// Reference semantics: tsfast/models/architectures/mamba/mamba_triton.py:85-286 (kernels) and
// :286-489 (ops), mamba/backend_c.py:105-245 (CPU kernels, same algebra).
//
// Thread layout: one lane per (batch b, channel d), holding all N states of that channel in
// VGPRs; a wave covers 64 consecutive channels of one batch row, so every per-step load of
// draw/u/z (and store of out) is one coalesced 64-element row segment, and the per-step B_t/C_t
// rows are wave-uniform. The [B, L, D, N] state never touches HBM: the training forward writes
// one fp32 checkpoint per channel every CHK steps, and the backward walks the checkpoints in
// reverse, recomputes the chunk's states into registers, and runs the adjoint
//   G_t = gy_t C_t + lam_{t+1} G_{t+1}
// in the same pass. lam_t h_{t-1} is recovered as h_t - delta_t u_t B_t, so states before the
// chunk are never needed. grad B_t / grad C_t are reduced over the wave's 64 channels with a
// register reduce-scatter and written as per-wave partials that a second kernel sums in a fixed
// order (no atomics: deterministic).
#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

template <int NS>
constexpr int chk_for() {
  return NS <= 16 ? 16 : (NS == 32 ? 8 : 4);
}

int ns_for(int64_t N) {
  if (N <= 4) return 4;
  if (N <= 8) return 8;
  if (N <= 16) return 16;
  if (N <= 32) return 32;
  if (N <= 64) return 64;
  return 0;
}

// ------------------------------------------------------------------------------------ forward
template <typename TIO, int NS>
__global__ void __launch_bounds__(64) mamba_fwd_kernel(const TIO* __restrict__ draw, const float* __restrict__ A,
                                                       const TIO* __restrict__ Bt, const TIO* __restrict__ Ct,
                                                       const TIO* __restrict__ u, const TIO* __restrict__ z,
                                                       const float* __restrict__ Dp, const float* __restrict__ h0,
                                                       TIO* __restrict__ out, float* __restrict__ h_last,
                                                       float* __restrict__ chk, int64_t L, int64_t D, int N,
                                                       int64_t NC) {
  constexpr int CHK = chk_for<NS>();
  const int lane = threadIdx.x;
  const int64_t d = (int64_t)blockIdx.x * 64 + lane;
  const int64_t b = blockIdx.y;
  const bool act = d < D;

  float Av[NS], h[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    Av[n] = (act && n < N) ? A[d * N + n] : 0.0f;
    h[n] = (act && h0 && n < N) ? h0[(b * D + d) * N + n] : 0.0f;
  }
  const float dp = act ? Dp[d] : 0.0f;
  const TIO* Bb = Bt + b * L * N;
  const TIO* Cb = Ct + b * L * N;

  for (int64_t t = 0; t < L; ++t) {
    const int64_t idx = (b * L + t) * D + d;
    const float dr = act ? to_f32(draw[idx]) : 0.0f;
    const float uu = act ? to_f32(u[idx]) : 0.0f;
    const float zz = act ? to_f32(z[idx]) : 0.0f;
    const float delta = act ? softplus(dr) : 0.0f;
    const float dl2 = delta * kLog2e;
    const float du = delta * uu;
    float acc = 0.0f;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const float bt = n < N ? to_f32(Bb[t * N + n]) : 0.0f;
      const float ct = n < N ? to_f32(Cb[t * N + n]) : 0.0f;
      const float lam = fast_exp2(dl2 * Av[n]);
      h[n] = fmaf(lam, h[n], du * bt);
      acc = fmaf(h[n], ct, acc);
    }
    if (act) out[idx] = from_f32<TIO>((acc + dp * uu) * zz * sigmoid(zz));
    if (chk && ((t + 1) % CHK) == 0 && act) {
      const int64_t slot = (t + 1) / CHK - 1;
      float* cp = chk + ((b * NC + slot) * D + d) * N;
#pragma unroll
      for (int n = 0; n < NS; ++n)
        if (n < N) cp[n] = h[n];
    }
  }
  if (act) {
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) h_last[(b * D + d) * N + n] = h[n];
  }
}

// ------------------------------------------------------------------------------------ backward
template <typename TIO, int NS>
__global__ void __launch_bounds__(64) mamba_bwd_kernel(
    const TIO* __restrict__ draw, const float* __restrict__ A, const TIO* __restrict__ Bt,
    const TIO* __restrict__ Ct, const TIO* __restrict__ u, const TIO* __restrict__ z, const float* __restrict__ Dp,
    const float* __restrict__ h0, const float* __restrict__ chk, const TIO* __restrict__ gout,
    const float* __restrict__ ghlast, TIO* __restrict__ gdraw, TIO* __restrict__ gu, TIO* __restrict__ gz,
    float* __restrict__ gA_part, float* __restrict__ gDp_part, float* __restrict__ gBC_part, float* __restrict__ gh0,
    int64_t B, int64_t L, int64_t D, int N, int64_t NC) {
  constexpr int CHK = chk_for<NS>();
  constexpr int KR = (2 * NS) < 64 ? 2 * NS : 64;  // values per reduce-scatter call
  constexpr int NRED = (2 * NS) / KR;               // calls per step
  constexpr int GROUP = 64 / KR;                    // lanes holding each reduced value
  const int lane = threadIdx.x;
  const int64_t d = (int64_t)blockIdx.x * 64 + lane;
  const int64_t b = blockIdx.y;
  const bool act = d < D;

  float Av[NS], G[NS], gA[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    Av[n] = (act && n < N) ? A[d * N + n] : 0.0f;
    G[n] = (act && ghlast && n < N) ? ghlast[(b * D + d) * N + n] : 0.0f;
    gA[n] = 0.0f;
  }
  const float dp = act ? Dp[d] : 0.0f;
  float gdp = 0.0f;
  const TIO* Bb = Bt + b * L * N;
  const TIO* Cb = Ct + b * L * N;
  float* part = gBC_part + ((int64_t)blockIdx.x * B + b) * L * (2 * NS);

  float hb[CHK][NS];
  float db[CHK];
  for (int64_t c = NC - 1; c >= 0; --c) {
    const int64_t t0 = c * CHK;
    const int len = (int)((L - t0) < CHK ? (L - t0) : CHK);
    float hs[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      float v0 = 0.0f;
      if (act && n < N) {
        if (c > 0)
          v0 = chk[((b * NC + c - 1) * D + d) * N + n];
        else if (h0)
          v0 = h0[(b * D + d) * N + n];
      }
      hs[n] = v0;
    }
    // recompute the chunk's states from its checkpoint
#pragma unroll
    for (int i = 0; i < CHK; ++i) {
      if (i < len) {
        const int64_t t = t0 + i;
        const int64_t idx = (b * L + t) * D + d;
        const float delta = act ? softplus(to_f32(draw[idx])) : 0.0f;
        const float uu = act ? to_f32(u[idx]) : 0.0f;
        const float dl2 = delta * kLog2e;
        const float du = delta * uu;
        db[i] = delta;
#pragma unroll
        for (int n = 0; n < NS; ++n) {
          const float bt = n < N ? to_f32(Bb[t * N + n]) : 0.0f;
          hs[n] = fmaf(fast_exp2(dl2 * Av[n]), hs[n], du * bt);
          hb[i][n] = hs[n];
        }
      }
    }
    // adjoint sweep, backwards through the chunk
#pragma unroll
    for (int ii = 0; ii < CHK; ++ii) {
      const int i = CHK - 1 - ii;
      if (i < len) {
        const int64_t t = t0 + i;
        const int64_t idx = (b * L + t) * D + d;
        const float delta = db[i];
        const float dr = act ? to_f32(draw[idx]) : 0.0f;
        const float uu = act ? to_f32(u[idx]) : 0.0f;
        const float zz = act ? to_f32(z[idx]) : 0.0f;
        const float go = act ? to_f32(gout[idx]) : 0.0f;
        const bool has_next = (t + 1) < L;
        float dn = 0.0f;  // delta_{t+1}
        if (i + 1 < len)
          dn = db[i + 1];
        else if (has_next && act)
          dn = softplus(to_f32(draw[idx + D]));
        const float dn2 = dn * kLog2e;

        float y = dp * uu;
#pragma unroll
        for (int n = 0; n < NS; ++n) {
          const float ct = n < N ? to_f32(Cb[t * N + n]) : 0.0f;
          y = fmaf(hb[i][n], ct, y);
        }
        const float sig = sigmoid(zz);
        const float gy = go * zz * sig;
        const float gzv = go * y * sig * (1.0f + zz * (1.0f - sig));
        gdp = fmaf(gy, uu, gdp);
        const float du = delta * uu;

        float gdelta = 0.0f, gus = 0.0f;
        float red[2 * NS];
#pragma unroll
        for (int n = 0; n < NS; ++n) {
          const float bt = n < N ? to_f32(Bb[t * N + n]) : 0.0f;
          const float ct = n < N ? to_f32(Cb[t * N + n]) : 0.0f;
          const float an = has_next ? fast_exp2(dn2 * Av[n]) : 1.0f;
          G[n] = fmaf(an, G[n], gy * ct);
          const float lamh = hb[i][n] - du * bt;  // lam_t h_{t-1}
          const float Q = G[n] * lamh;
          gA[n] = fmaf(delta, Q, gA[n]);
          gdelta = fmaf(Av[n], Q, gdelta);
          gus = fmaf(G[n], bt, gus);
          red[n] = G[n] * du;
          red[NS + n] = gy * hb[i][n];
        }
        gdelta = fmaf(uu, gus, gdelta);
        if (act) {
          gdraw[idx] = from_f32<TIO>(gdelta * sigmoid(dr));
          gu[idx] = from_f32<TIO>(fmaf(delta, gus, gy * dp));
          gz[idx] = from_f32<TIO>(gzv);
        }
#pragma unroll
        for (int r = 0; r < NRED; ++r) {
          wave_reduce_scatter<KR>(red + r * KR, lane);
          if ((lane % GROUP) == 0) part[t * (2 * NS) + r * KR + lane / GROUP] = red[r * KR];
        }
      }
    }
  }
  if (act) {
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) gA_part[(b * D + d) * N + n] = gA[n];
    gDp_part[b * D + d] = gdp;
    if (gh0) {
      // an empty sequence passes the state through unchanged (gh0 = ghlast)
      const float d0 = L > 0 ? softplus(to_f32(draw[b * L * D + d])) * kLog2e : 0.0f;
#pragma unroll
      for (int n = 0; n < NS; ++n)
        if (n < N) gh0[(b * D + d) * N + n] = fast_exp2(d0 * Av[n]) * G[n];
    }
  }
}

// gBt/gCt: sum the per-wave partials [nDB, B, L, 2*NS] over the channel blocks.
template <typename TIO>
__global__ void __launch_bounds__(256) mamba_reduce_bc(const float* __restrict__ part, TIO* __restrict__ gBt,
                                                       TIO* __restrict__ gCt, int64_t nDB, int64_t BL, int N,
                                                       int NS) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;  // over BL * N
  if (i >= BL * N) return;
  const int64_t row = i / N;
  const int n = (int)(i % N);
  float sb = 0.0f, sc = 0.0f;
  for (int64_t k = 0; k < nDB; ++k) {
    const float* p = part + (k * BL + row) * (2 * NS);
    sb += p[n];
    sc += p[NS + n];
  }
  gBt[i] = from_f32<TIO>(sb);
  gCt[i] = from_f32<TIO>(sc);
}

// Sum [B, X] partials over the batch into [X] (gA with X = D*N, gDp with X = D).
__global__ void __launch_bounds__(256) mamba_reduce_batch(const float* __restrict__ part, float* __restrict__ dst,
                                                          int64_t B, int64_t X) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= X) return;
  float s = 0.0f;
  for (int64_t b = 0; b < B; ++b) s += part[b * X + i];
  dst[i] = s;
}

template <typename TIO, int NS>
int launch_fwd(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
               const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, void* out,
               float* h_last, float* chk, hipStream_t s) {
  constexpr int CHK = chk_for<NS>();
  const int64_t NC = (L + CHK - 1) / CHK;
  dim3 grid((unsigned)((D + 63) / 64), (unsigned)B);
  hipLaunchKernelGGL((mamba_fwd_kernel<TIO, NS>), grid, dim3(64), 0, s, (const TIO*)draw, A, (const TIO*)Bt,
                     (const TIO*)Ct, (const TIO*)u, (const TIO*)z, Dp, h0, (TIO*)out, h_last, chk, L, D, (int)N, NC);
  return tsf_launch_status();
}

template <typename TIO, int NS>
int launch_bwd(int64_t B, int64_t L, int64_t D, int64_t N, const void* draw, const float* A, const void* Bt,
               const void* Ct, const void* u, const void* z, const float* Dp, const float* h0, const float* chk,
               const void* gout, const float* ghlast, void* gdraw, float* gA, void* gBt, void* gCt, void* gu, void* gz,
               float* gDp, float* gh0, void* workspace, hipStream_t s) {
  constexpr int CHK = chk_for<NS>();
  const int64_t NC = (L + CHK - 1) / CHK;
  const int64_t nDB = (D + 63) / 64;
  float* gBC_part = static_cast<float*>(workspace);
  float* gA_part = gBC_part + nDB * B * L * 2 * NS;
  float* gDp_part = gA_part + B * D * N;
  dim3 grid((unsigned)nDB, (unsigned)B);
  if (B > 0 && D > 0)
    hipLaunchKernelGGL((mamba_bwd_kernel<TIO, NS>), grid, dim3(64), 0, s, (const TIO*)draw, A, (const TIO*)Bt,
                       (const TIO*)Ct, (const TIO*)u, (const TIO*)z, Dp, h0, chk, (const TIO*)gout, ghlast,
                       (TIO*)gdraw, (TIO*)gu, (TIO*)gz, gA_part, gDp_part, gBC_part, gh0, B, L, D, (int)N, NC);
  const int64_t BLN = B * L * N;
  if (BLN > 0)
    hipLaunchKernelGGL((mamba_reduce_bc<TIO>), dim3((unsigned)((BLN + 255) / 256)), dim3(256), 0, s, gBC_part,
                       (TIO*)gBt, (TIO*)gCt, nDB, B * L, (int)N, NS);
  if (D > 0) {
    hipLaunchKernelGGL(mamba_reduce_batch, dim3((unsigned)((D * N + 255) / 256)), dim3(256), 0, s, gA_part, gA, B,
                       D * N);
    hipLaunchKernelGGL(mamba_reduce_batch, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, s, gDp_part, gDp, B, D);
  }
  return tsf_launch_status();
}

#define TSF_DISPATCH_NS(NSV, FN, ...)            \
  switch (NSV) {                                 \
    case 4:                                      \
      return FN<4>(__VA_ARGS__);                 \
    case 8:                                      \
      return FN<8>(__VA_ARGS__);                 \
    case 16:                                     \
      return FN<16>(__VA_ARGS__);                \
    case 32:                                     \
      return FN<32>(__VA_ARGS__);                \
    case 64:                                     \
      return FN<64>(__VA_ARGS__);                \
    default:                                     \
      return TSF_ERR_UNSUPPORTED;                \
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

int chk_interval_for(int ns) {
  switch (ns) {
    case 4:
      return chk_for<4>();
    case 8:
      return chk_for<8>();
    case 16:
      return chk_for<16>();
    case 32:
      return chk_for<32>();
    case 64:
      return chk_for<64>();
    default:
      return 0;
  }
}

}  // namespace

extern "C" {

int64_t tsfast_hip_mamba_chk_interval(int64_t N) { return chk_interval_for(ns_for(N)); }

int64_t tsfast_hip_mamba_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t N) {
  const int ns = ns_for(N);
  if (ns == 0) return -1;
  const int64_t nDB = (D + 63) / 64;
  return 4 * (nDB * B * L * 2 * ns + B * D * N + B * D);
}

int tsfast_hip_mamba_fwd(int64_t B, int64_t L, int64_t D, int64_t N, int io_dtype, const void* draw, const float* A,
                         const void* Bt, const void* Ct, const void* u, const void* z, const float* Dp,
                         const float* h0, void* out, float* h_last, float* chk, void* stream) {
  if (B < 0 || L < 0 || D < 0 || N < 1) return TSF_ERR_ARG;
  if (B > 65535) return TSF_ERR_UNSUPPORTED;
  const int ns = ns_for(N);
  if (ns == 0) return TSF_ERR_UNSUPPORTED;
  if (B == 0 || D == 0) return TSF_OK;
  if (!A || !Dp || !h_last) return TSF_ERR_ARG;
  if (L > 0 && (!draw || !Bt || !Ct || !u || !z || !out)) return TSF_ERR_ARG;
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
  if (B > 65535) return TSF_ERR_UNSUPPORTED;
  const int ns = ns_for(N);
  if (ns == 0) return TSF_ERR_UNSUPPORTED;
  if (!A || !Dp || !gA || !gDp) return TSF_ERR_ARG;
  if (L > 0 && (!draw || !Bt || !Ct || !u || !z || !gout || !gdraw || !gBt || !gCt || !gu || !gz)) return TSF_ERR_ARG;
  if (h0 && !gh0) return TSF_ERR_ARG;
  if (L > 0 && !chk && L > chk_interval_for(ns)) return TSF_ERR_ARG;
  if (workspace_bytes < tsfast_hip_mamba_workspace_bytes(B, L, D, N) || !workspace) return TSF_ERR_WORKSPACE;
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
