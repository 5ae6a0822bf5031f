// Chunked adjoint scan of a time-varying matrix recurrence: the sequence-parallel part of a
// NeuralStateSpace backward. With the per-step matrices A_t = jt[b, t] (n x n, row-major; the
// transposed state Jacobians of the rollout) and the upstream gradients gout [B, L, n],
//   gy_t = gout_t + A_{t+1} gy_{t+1},   gy_{L-1} = gout_{L-1}.
// Chunk c covers steps [c CL, min((c + 1) CL, L)). Its summary is the affine map that carries the
// adjoint entering the chunk from the right to its first step, gy_{t0} = P_c gy_{t1} + s_c, and a
// sequential pass over the chunks from the right composes the summaries into the adjoint at every
// chunk start, bnd [B, C + 1, n] (bnd[C] = 0), from which the rollout's own backward re-runs each
// chunk. Reference: tsfast/models/architectures/ssm/backend_metal.py:285-357 (ssm_bwd_summary,
// ssm_bwd_scan) and their call in `backward` (:466-476).
//
// Summary kernel: one workgroup per (row b, chunk c) holds the augmented map [P | s] (n x (n + 1),
// fp64) in LDS and steps it right to left, [P | s] <- A_{t+1} [P | s] + [0 | gout_t], on the fp64
// matrix cores (v_mfma_f64_16x16x4f64): one wave per 16-column block (over the state plus the s
// column) computing every row block of it, so the waves only meet once per batch. The step matrices
// stream through LDS four steps at a time with coalesced loads, the next batch in flight while the
// current one is used.
// fp64 keeps a chunk's product of up to a few hundred matrices at fp64 rounding (fp32 inputs).
// Carry kernel: one workgroup per row b, four lanes per state row, the next eight chunks' summaries
// in flight.
#include <algorithm>

#include "common.h"
#include "tsfast_hip.h"

using namespace tsf;

namespace {

using d4 = __attribute__((__vector_size__(4 * sizeof(double)))) double;

constexpr int kMasMaxN = 32;
constexpr int kMasBatch = 4;  // step matrices per LDS batch

TSF_DEV d4 mfma64(double a, double b, d4 c) { return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0); }

// NBR 16-row blocks cover the state (n <= 16 NBR); NBC 16-column blocks cover the state and the s
// column (n + 1 <= 16 NBC). A column block of A [P | s] depends only on the same column block of
// [P | s], so wave w owns column block w for every row block: it reads and rewrites only its own
// columns, and the waves meet at a barrier once per batch of step matrices, not once per step.
template <int NBR, int NBC>
__global__ void __launch_bounds__(64 * NBC) mas_summary(const float* __restrict__ jt, const float* __restrict__ gout,
                                                        double* __restrict__ pc, double* __restrict__ sc, int64_t L,
                                                        int n, int64_t CL, int64_t C) {
  constexpr int R = 16 * NBR, Q = 16 * NBC, RS = R + 1;
  __shared__ double s_p[R][Q + 1];             // [P | s]; each wave rewrites only its own columns
  __shared__ float s_a[2][kMasBatch][R][RS];   // step matrices, zero outside n x n
  __shared__ float s_g[2][kMasBatch][R];       // gout of the batch's steps
  const int lane = threadIdx.x & 63, bj = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.x / C, c = blockIdx.x - b * C;
  const int64_t t0 = c * CL, t1 = std::min(t0 + CL, L);
  const int nn = n * n;

  for (int e = threadIdx.x; e < R * (Q + 1); e += blockDim.x) {
    const int r = e / (Q + 1), q = e - r * (Q + 1);
    s_p[r][q] = (r == q && r < n) ? 1.0 : 0.0;
  }
  for (int e = threadIdx.x; e < 2 * kMasBatch * R * RS; e += blockDim.x) (&s_a[0][0][0][0])[e] = 0.0f;
  __syncthreads();

  // Batch k holds the matrices of steps t = t1 - 1 - kMasBatch k - i (i < kMasBatch), i.e. A_{t+1}
  // = jt[b, t1 - kMasBatch k - i]. Thread (i, r) = (threadIdx / n, threadIdx % n) moves row r of
  // step i's matrix (n contiguous floats) and gout_t[r]; kMasBatch n <= blockDim for every
  // instantiation the host picks.
  const int fi = threadIdx.x / n, fr = threadIdx.x - fi * n;
  const bool mover = fi < kMasBatch;
  const bool vec4 = (n & 3) == 0 && (reinterpret_cast<uintptr_t>(jt) & 15) == 0;
  float reg[R], greg = 0.0f;
  auto fetch = [&](int64_t k) __attribute__((always_inline)) {
    const int64_t t = t1 - 1 - kMasBatch * k - fi;
    const bool ok = mover && t >= t0;
    const float* row = jt + ((b * L + t + 1) * n + fr) * n;
    const bool have = ok && t + 1 < L;
    if (vec4) {  // n % 4 == 0 and 16-byte aligned rows: whole float4s
#pragma unroll
      for (int q = 0; q < R; q += 4) {
        const float4 v = (have && q < n) ? *reinterpret_cast<const float4*>(row + q) : make_float4(0.f, 0.f, 0.f, 0.f);
        reg[q] = v.x;
        reg[q + 1] = v.y;
        reg[q + 2] = v.z;
        reg[q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < R; ++q) reg[q] = (have && q < n) ? row[q] : 0.0f;
    }
    greg = ok ? gout[(b * L + t) * n + fr] : 0.0f;
  };
  auto stash = [&](int buf) __attribute__((always_inline)) {
    if (mover) {
#pragma unroll
      for (int q = 0; q < R; ++q)
        if (q < n) s_a[buf][fi][fr][q] = reg[q];
      s_g[buf][fi][fr] = greg;
    }
  };
  const int64_t steps = t1 - t0, batches = (steps + kMasBatch - 1) / kMasBatch;
  if (batches > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  const int col = 16 * bj + j;
  for (int64_t k = 0; k < batches; ++k) {
    const int buf = (int)(k & 1);
    if (k + 1 < batches) fetch(k + 1);  // in flight while this batch's steps run
    for (int i = 0; i < kMasBatch; ++i) {
      const int64_t t = t1 - 1 - kMasBatch * k - i;
      if (t < t0) break;  // uniform over the workgroup
      d4 acc[NBR];
#pragma unroll
      for (int bi = 0; bi < NBR; ++bi) acc[bi] = d4{0.0, 0.0, 0.0, 0.0};
      if (t + 1 < L) {
#pragma unroll
        for (int kk = 0; kk < 4 * NBR; ++kk) {
          const double bv = s_p[4 * kk + g][col];
#pragma unroll
          for (int bi = 0; bi < NBR; ++bi) acc[bi] = mfma64((double)s_a[buf][i][16 * bi + j][4 * kk + g], bv, acc[bi]);
        }
      }
      // the f64 16x16x4 result holds rows g, g + 4, g + 8, g + 12 of column j in lane (g, j)
      // (unlike the f32 16x16x4 layout, rows 4g .. 4g + 3). The wave's reads of its columns are
      // complete (their values fed the MFMAs) before these writes, so one buffer suffices.
#pragma unroll
      for (int bi = 0; bi < NBR; ++bi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * bi + g + 4 * r;
          double v = acc[bi][r];
          if (col == n && row < n) v += (double)s_g[buf][i][row];
          s_p[row][col] = v;
        }
    }
    if (k + 1 < batches) stash(buf ^ 1);
    __syncthreads();
  }
  double* pcb = pc + (b * C + c) * nn;
  double* scb = sc + (b * C + c) * n;
  for (int e = threadIdx.x; e < n * (n + 1); e += blockDim.x) {
    const int r = e / (n + 1), q = e - r * (n + 1);
    const double v = s_p[r][q];
    if (q < n)
      pcb[r * n + q] = v;
    else
      scb[r] = v;
  }
}

// bnd[b, c] = s_c + P_c bnd[b, c + 1] from the right, bnd[b, C] = 0. One workgroup per row b of
// 4 NP threads: four lanes per state row i, each summing NP / 4 columns of P_c's row (the four
// partials meet through two lane swaps). A lane keeps the row parts of the next kRing chunks in a
// register ring, so each chunk's loads are issued kRing chunks before they are needed.
constexpr int kRing = 8;
template <int NP>
__global__ void __launch_bounds__(4 * NP) mas_carry(const double* __restrict__ pc, const double* __restrict__ sc,
                                                    float* __restrict__ bnd, int n, int64_t C) {
  constexpr int CP = NP / 4;
  __shared__ double s_v[2][NP];
  const int tid = threadIdx.x, i = tid >> 2, h = tid & 3;
  const int64_t b = blockIdx.x;
  const bool live = i < n;
  // both buffers start at zero: columns n..NP-1 of either one are read (times a zero P entry) in
  // every chunk, so no earlier kernel's LDS contents (possibly NaN or Inf bits) may remain there
  if (tid < 2 * NP) s_v[tid / NP][tid % NP] = 0.0;
  if (h == 0 && live) bnd[(b * (C + 1) + C) * n + i] = 0.0f;
  double ring[kRing][CP], sring[kRing];
  auto load = [&](int64_t c, int slot) __attribute__((always_inline)) {
    const double* p = pc + ((b * C + c) * n + (live ? i : 0)) * n + h * CP;
#pragma unroll
    for (int m = 0; m < CP; ++m) ring[slot][m] = (live && c >= 0 && h * CP + m < n) ? p[m] : 0.0;
    sring[slot] = (live && h == 0 && c >= 0) ? sc[(b * C + c) * n + i] : 0.0;
  };
#pragma unroll
  for (int d = 0; d < kRing; ++d) load(C - 1 - d, d);
  __syncthreads();
  int cur = 0;
  for (int64_t c0 = C - 1; c0 >= 0; c0 -= kRing) {
#pragma unroll
    for (int d = 0; d < kRing; ++d) {
      const int64_t c = c0 - d;
      if (c < 0) break;  // uniform over the workgroup
      double part = sring[d];
#pragma unroll
      for (int m = 0; m < CP; ++m) part = fma(ring[d][m], s_v[cur][h * CP + m], part);
      part += __shfl_xor(part, 1);
      part += __shfl_xor(part, 2);
      load(c - kRing, d);  // the ring slot now holds the chunk kRing further left
      if (h == 0 && live) {
        s_v[cur ^ 1][i] = part;
        bnd[(b * (C + 1) + c) * n + i] = (float)part;
      }
      __syncthreads();
      cur ^= 1;
    }
  }
}

__global__ void __launch_bounds__(256) mas_zero(float* __restrict__ p, int64_t count) {
  const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (e < count) p[e] = 0.0f;
}

int mas_args_status(int64_t B, int64_t L, int64_t n, int64_t CL) {
  if (B < 0 || L < 0 || n < 1 || CL < 1) return TSF_ERR_ARG;
  if (n > kMasMaxN) return TSF_ERR_UNSUPPORTED;
  const int64_t C = (L + CL - 1) / CL;
  if (B * C > INT32_MAX || B > INT32_MAX) return TSF_ERR_UNSUPPORTED;
  return TSF_OK;
}

template <int NBR, int NBC>
void summary_launch(int64_t B, int64_t L, int n, int64_t CL, int64_t C, const float* jt, const float* gout, double* pc,
                    double* sc, hipStream_t s) {
  hipLaunchKernelGGL((mas_summary<NBR, NBC>), dim3((unsigned)(B * C)), dim3(64 * NBC), 0, s, jt, gout, pc, sc, L,
                     n, CL, C);
}

}  // namespace

extern "C" {

int64_t tsfast_hip_mat_adjoint_workspace_bytes(int64_t B, int64_t L, int64_t n, int64_t CL) {
  if (mas_args_status(B, L, n, CL) != TSF_OK) return -1;
  const int64_t C = (L + CL - 1) / CL;
  return (int64_t)sizeof(double) * B * C * (n * n + n);
}

int tsfast_hip_mat_adjoint_bounds(int64_t B, int64_t L, int64_t n, int64_t CL, const float* jt, const float* gout,
                                  float* bnd, void* workspace, int64_t workspace_bytes, void* stream) {
  const int st = mas_args_status(B, L, n, CL);
  if (st != TSF_OK) return st;
  if (B == 0) return TSF_OK;
  if (!bnd) return TSF_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t C = (L + CL - 1) / CL;
  if (C == 0) {  // empty sequence: the single boundary is zero
    hipLaunchKernelGGL(mas_zero, dim3((unsigned)((B * n + 255) / 256)), dim3(256), 0, s, bnd, B * n);
    return tsf_launch_status();
  }
  if (!jt || !gout) return TSF_ERR_ARG;
  if (!workspace || workspace_bytes < tsfast_hip_mat_adjoint_workspace_bytes(B, L, n, CL)) return TSF_ERR_WORKSPACE;
  double* pc = static_cast<double*>(workspace);
  double* sc = pc + B * C * n * n;
  const int nn = (int)n;
  if (n <= 15)
    summary_launch<1, 1>(B, L, nn, CL, C, jt, gout, pc, sc, s);
  else if (n <= 16)
    summary_launch<1, 2>(B, L, nn, CL, C, jt, gout, pc, sc, s);
  else if (n <= 31)
    summary_launch<2, 2>(B, L, nn, CL, C, jt, gout, pc, sc, s);
  else
    summary_launch<2, 3>(B, L, nn, CL, C, jt, gout, pc, sc, s);
  if (n <= 16)
    hipLaunchKernelGGL(mas_carry<16>, dim3((unsigned)B), dim3(64), 0, s, (const double*)pc, (const double*)sc, bnd, nn,
                       C);
  else
    hipLaunchKernelGGL(mas_carry<32>, dim3((unsigned)B), dim3(128), 0, s, (const double*)pc, (const double*)sc, bnd, nn,
                       C);
  return tsf_launch_status();
}

}  // extern "C"
