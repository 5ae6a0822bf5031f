/*
 * tsfast_hip.h - C ABI of libtsfast_hip.so, the MI355X (gfx950) scan-family kernels behind
 * tsfast's scan dispatch layer.
 *
 * Conventions (shared by every entry point):
 *   - sizes are int64_t; tensors are raw device pointers to contiguous row-major buffers in the
 *     layouts named below; optional tensors are NULL when absent;
 *   - outputs and workspaces are allocated by the caller (the Python shim allocates them with
 *     torch.empty on the caller's device); the library never allocates device memory;
 *   - `stream` is a hipStream_t passed as void* (torch.cuda.current_stream().cuda_stream); every
 *     launch is asynchronous on that stream, with no host synchronisation, so calls can be
 *     captured in a HIP graph;
 *   - the return value is a status: TSF_OK (0) on success, a negative TSF_ERR_* code otherwise;
 *     tsfast_hip_status_string() names it (for TSF_ERR_HIP, with the HIP runtime's message).
 *
 * The single-pass look-back scans (diag, selective, all-pole with na <= 4, linear recurrence with
 * n <= 4, G-block, projected) start their workspace with a 256-byte header: the tile counter in
 * bytes 0..3 and, in bytes 64..67, a give-up flag (int32) that a look-back sets to 1 when it waited
 * about a second without progress and gave up, its lanes then holding NaN (a GPU kept busy by
 * other work). Each call clears the header on its stream before the scan, so after the call the
 * flag tells a give-up apart from NaN that came with the inputs.
 *
 * Complex tensors are interleaved (re, im) float pairs, i.e. torch.view_as_real layout.
 * bf16 tensors are raw 16-bit bfloat16 words (torch.bfloat16 storage).
 */
#ifndef TSFAST_HIP_H
#define TSFAST_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSF_OK 0
#define TSF_ERR_ARG (-1)         /* a size or pointer argument is invalid */
#define TSF_ERR_WORKSPACE (-2)   /* workspace missing or smaller than the *_workspace_bytes query */
#define TSF_ERR_UNSUPPORTED (-3) /* shape outside what the kernels are built for (e.g. H > 32 in the projected scan) */
#define TSF_ERR_HIP (-4)         /* a HIP runtime call or kernel launch failed */
#define TSF_ERR_SCRATCH (-5)     /* more scratch than a no-allocation entry point holds */

#define TSF_DTYPE_F32 0
#define TSF_DTYPE_BF16 1

const char* tsfast_hip_status_string(int status);

/* Deterministic mode of the single-pass look-back scans (diag, selective, all-pole, linear
 * recurrence, G-block, projected), process-wide, read when a scan is launched. On (1, the
 * default): anchor tiles in scan order publish their leaving state and the others their aggregates,
 * so every launch composes the same maps in the same order and the outputs are bitwise reproducible
 * (the parameter-gradient sums of the projected scan's fused backward excepted); 0-4% slower than
 * off. Off (0): a tile composes the published maps back to the nearest tile that has published
 * its leaving state, so which maps are composed depends on timing and results agree run to run to
 * fp64 rounding. No counterpart in the reference, whose kernels are deterministic by construction
 * (tsfast/models/architectures/mamba/mamba_triton.py:19-22); the Python backends keep it on unless
 * reproducibility is switched off (tsfast_amd.set_reproducible(False) or
 * TSFAST_HIP_REPRODUCIBLE=0) and torch.are_deterministic_algorithms_enabled() is false. */
void tsfast_hip_set_deterministic(int on);
int tsfast_hip_get_deterministic(void);
/* Look-back failure reporting. Every look-back wait is bounded: a scan whose wait makes no
 * progress for the spin limit gives up, writes NaN into the lanes concerned, sets the
 * workspace's give-up word (byte 64) and writes the scan's call number into the library's alarm
 * word, a word in mapped host memory. tsfast_hip_lookback_gave_up reads that word without
 * synchronising with the device: 1 if it names a scan call not yet reported (a give-up shows
 * there once its kernel has ended), 0 if not, -1 if the word could not be allocated; with
 * `clear` nonzero the call it names counts as reported from then on, so each failing call is
 * reported once. tsfast_hip_set_lookback_spin_limit sets the polls without progress allowed before a
 * give-up (default 2^20, passed to each scan's kernels when they are enqueued) and returns the
 * previous limit; a small limit lets a test force a give-up while every kernel still exits.
 * No counterpart in the reference, whose scans never wait on other workgroups. */
int tsfast_hip_lookback_gave_up(int clear);
int64_t tsfast_hip_set_lookback_spin_limit(int64_t polls);
/* Library version, for the Python loader's sanity check. */
int tsfast_hip_version(void);

/* ------------------------------------------------------------------------------------------
 * Constant-coefficient diagonal scan  x_t = lam * x_{t-1} + v_t  and its adjoint.
 * Replaces the backend contract of tsfast/models/_core/scan_backends/diagonal_triton.py:255-305
 * (forward(lam, v, x0) / backward(g, lam, out, x0)), reached from the tsfast::scan_diagonal ops
 * (tsfast/models/_core/scan.py:100-154).
 * Layout: lam [M, N], v/out/g/gv [M, L, N], x0/gx0/glam [M, N]; float32 or complex64.
 * Single-pass kernels with an inter-workgroup look-back: the workspace holds the tile counter and
 * the published super-chunk states; each call re-initialises it on its stream (no caller set-up),
 * so two calls in flight at once must not share one workspace. A sequence short enough for one
 * workgroup per lane group in a direction (whole-sequence tiles: up to 16 chunks of 64 real
 * steps, or 32 / 16 complex steps forward / backward; a forward on 16-lane groups up to 64
 * chunks) runs without a look-back; when both directions do, the workspace is just the header.
 */
int64_t tsfast_hip_diag_workspace_bytes(int64_t M, int64_t L, int64_t N, int is_complex);
int tsfast_hip_diag_fwd(int64_t M, int64_t L, int64_t N, int is_complex, const void* lam, const void* v,
                        const void* x0, void* out, void* workspace, int64_t workspace_bytes, void* stream);
/* glam = sum_t G_t conj(x_{t-1}), gv = G, gx0 = conj(lam) G_0 (gx0 required iff x0 given). */
int tsfast_hip_diag_bwd(int64_t M, int64_t L, int64_t N, int is_complex, const void* g, const void* lam,
                        const void* out, const void* x0, void* gv, void* glam, void* gx0, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* No-allocation variant of tsfast_hip_diag_fwd. It has no counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The look-back workspace is a fixed per-GPU device array of
 * tsfast_hip_diag_noalloc_max_bytes() bytes (32 MiB), held until the process ends; a shape whose
 * tsfast_hip_diag_workspace_bytes exceeds it returns TSF_ERR_SCRATCH before any launch. Each call
 * re-initialises the array on its stream before the scan, but calls that overlap on one GPU (two
 * streams or two host threads) share the array and race: serialise them. The stream must belong
 * to the current device. Same results as tsfast_hip_diag_fwd; allocates nothing. */
int64_t tsfast_hip_diag_noalloc_max_bytes(void);
int tsfast_hip_diag_fwd_noalloc(int64_t M, int64_t L, int64_t N, int is_complex, const void* lam, const void* v,
                                const void* x0, void* out, void* stream);

/* ------------------------------------------------------------------------------------------
 * Time-varying (selective) diagonal scan  x_t = a_t * x_{t-1} + v_t  and its adjoint, float32.
 * Replaces tsfast/models/_core/scan_backends/selective_triton.py:112-160 (forward / backward),
 * reached from the tsfast::scan_selective ops (tsfast/models/_core/scan.py:157-215).
 * Layout: a/v/out/g/gv/glam [M, L, N], x0/gx0 [M, N]. Workspace as for the diagonal scan.
 */
int64_t tsfast_hip_sel_workspace_bytes(int64_t M, int64_t L, int64_t N);
int tsfast_hip_sel_fwd(int64_t M, int64_t L, int64_t N, const float* a, const float* v, const float* x0, float* out,
                       void* workspace, int64_t workspace_bytes, void* stream);
/* glam_t = G_t x_{t-1}, gv = G, gx0 = a_0 G_0 (gx0 required iff x0 given). */
int tsfast_hip_sel_bwd(int64_t M, int64_t L, int64_t N, const float* g, const float* a, const float* out,
                       const float* x0, float* glam, float* gv, float* gx0, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* ------------------------------------------------------------------------------------------
 * Fused Mamba selective SSM (softplus discretisation, exp(delta A), input injection, recurrence,
 * C contraction, D skip, SiLU gate):
 *   h_t = exp(softplus(draw_t) A) h_{t-1} + softplus(draw_t) u_t B_t
 *   out_t = (h_t . C_t + Dp u_t) * z_t * sigmoid(z_t)
 * Replaces the kernels behind tsfast/models/architectures/mamba/mamba_triton.py:286-489
 * (tsfast::mamba_scan / mamba_scan_train / mamba_scan_bwd) and the C ABI of
 * tsfast/models/architectures/mamba/backend_c.py:105-245 (mamba_fwd / mamba_bwd).
 * Layout: draw/u/z/out/gout/gdraw/gu/gz [B, L, D] and Bt/Ct/gBt/gCt [B, L, N] in io_dtype
 * (TSF_DTYPE_F32 or TSF_DTYPE_BF16); A/gA [D, N], Dp/gDp [D], h0/h_last/ghlast/gh0 [B, D, N]
 * always float32 (the state is float32 in both regimes). 1 <= N <= 64.
 * chk is the training forward's saved state, [B, S] float32 words with
 * S = tsfast_hip_mamba_saved_floats(L, D, N, io_dtype) per batch row: the float32 checkpoints
 * [NC, N, D] with NC = ceil(L / tsfast_hip_mamba_chk_interval(N)) (slot k = the state after step
 * (k + 1) * interval - 1, channel-contiguous so that checkpoint traffic is coalesced), then
 * y [L, D] = sum_n h_t C_t + Dp u_t in io_dtype, the output before the gate (the backward's gate
 * gradient reads it instead of recomputing sum_n h_t C_t). chk == NULL selects the inference
 * kernel, which saves nothing.
 * The kernels address one batch row with 32-bit byte offsets: (L + 64) * D, (L + 64) * 2 * N'
 * (N' = N rounded up to 4, 8, 16, 32 or 64) and NC * N * D + L * D must stay below 2^29, else
 * TSF_ERR_UNSUPPORTED (tsfast_hip_mamba_saved_floats then returns -1, so it doubles as the size
 * check).
 */
int64_t tsfast_hip_mamba_chk_interval(int64_t N);
int64_t tsfast_hip_mamba_saved_floats(int64_t L, int64_t D, int64_t N, int io_dtype);
int tsfast_hip_mamba_fwd(int64_t B, int64_t L, int64_t D, int64_t N, int io_dtype, const void* draw, const float* A,
                         const void* Bt, const void* Ct, const void* u, const void* z, const float* Dp,
                         const float* h0, void* out, float* h_last, float* chk, void* stream);
/* Backward from the forward's saved state chk (required when L > 0). ghlast may be NULL (zero
 * upstream state gradient); gh0 is written iff h0 is given. gA/gDp are the full parameter
 * gradients (summed over the batch). */
int64_t tsfast_hip_mamba_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t N);
int tsfast_hip_mamba_bwd(int64_t B, int64_t L, int64_t D, int64_t N, int io_dtype, const void* draw, const float* A,
                         const void* Bt, const void* Ct, const void* u, const void* z, const float* Dp,
                         const float* h0, const float* chk, const void* gout, const float* ghlast, void* gdraw,
                         float* gA, void* gBt, void* gCt, void* gu, void* gz, float* gDp, float* gh0, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * dynoNet all-pole IIR scan  y_t = w_t - sum_{i=1..na} a_i y_{t-i},  float32, 1 <= na <= 16.
 * Replaces the generated kernels of tsfast/models/architectures/dynonet/allpole_triton.py:59-233
 * (tsfast::dynonet_allpole / dynonet_allpole_bwd, including the host-side y0 head taps at :202-213).
 * Layout: a [lanes, na], w/y/g/gw [lanes, L] (time contiguous), y0/gy0 [lanes, na] newest first
 * (y0[j] = y_{-1-j}). For na <= 4 the workspace also carries the look-back state of a single-pass
 * scan, re-initialised by each call on its stream: two calls in flight must not share one.
 */
int64_t tsfast_hip_allpole_workspace_bytes(int64_t lanes, int64_t L, int64_t na);
int tsfast_hip_allpole_fwd(int64_t lanes, int64_t L, int64_t na, const float* a, const float* w, const float* y0,
                           float* y, void* workspace, int64_t workspace_bytes, void* stream);
/* ga = d loss / d a (full gradient, y0 taps included), gw = G, gy0 written iff y0 given. */
int tsfast_hip_allpole_bwd(int64_t lanes, int64_t L, int64_t na, const float* g, const float* a, const float* y,
                           const float* y0, float* gw, float* ga, float* gy0, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Fused causal depthwise convolution + SiLU (the Mamba conv section):
 *   out_t = silu(bias + sum_{k<K} w_k xbuf_{t-(K-1)+k}),  xbuf = cat(tail, x) along time,
 * per channel, 2 <= K <= 8. Replaces tsfast/models/architectures/mamba/conv_triton.py:59-263
 * (tsfast::mamba_conv_silu / mamba_conv_silu_bwd, the tail gradient of :241-250 included).
 * Layout: x [B, L, D] in io_dtype read through element strides (sxb, sxl, sxd) (the in_proj
 * chunk view needs no copy); tail/gtail [B, D, K-1] in io_dtype (NULL tail = zero left
 * context; gtail may be NULL); weight/gw [D, K] and bias/gb [D] float32 (bias NULL = none);
 * out, gy, gx [B, L, D] contiguous in io_dtype. B <= 65535; strides >= 0. One batch row of x
 * ((L + 8) * sxl + (D + 8) * sxd elements) and of the outputs ((L + 8) * D) must stay below
 * 4 GiB, else TSF_ERR_UNSUPPORTED.
 */
int tsfast_hip_conv_silu_fwd(int64_t B, int64_t L, int64_t D, int64_t K, int io_dtype, const void* x, int64_t sxb,
                             int64_t sxl, int64_t sxd, const void* tail, const float* weight, const float* bias,
                             void* out, void* stream);
/* Backward; gw/gb are the full parameter gradients (summed over batch and time). */
int64_t tsfast_hip_conv_silu_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t K);
int tsfast_hip_conv_silu_bwd(int64_t B, int64_t L, int64_t D, int64_t K, int io_dtype, const void* x, int64_t sxb,
                             int64_t sxl, int64_t sxd, const void* tail, const float* weight, const float* bias,
                             const void* gy, void* gx, void* gtail, float* gw, float* gb, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Fused dynoNet G-block: the FIR + all-pole + input-sum body of LinearDynamicalOperator.forward
 * (tsfast/models/architectures/dynonet/core.py:196-258; the reference runs it as F.conv1d at
 * :219-222, the tsfast::dynonet_allpole op at :225-235 and a sum at :250), per pair p = j*O + o:
 *   w_p[t] = sum_k b[o,j,k] u[t-k, j],  y_p[t] = w_p[t] - sum_i a[o,j,i] y_p[t-i],
 *   y[t, o] = sum_j y_p[t],  x_last[p, q] = y_p[L-1-q] (x0 beyond the start).
 * float32 in and out, fp64 state; 1 <= na <= 4, 1 <= nb <= 16, I*O <= 64 (a caller splits a
 * larger block into groups of whole inputs or outputs and adds their outputs), else
 * TSF_ERR_UNSUPPORTED. Layout: u/gu [B, L, I], y/gy [B, L, O] (channel-last, contiguous),
 * b/gb [O, I, nb], a/ga [O, I, na], u_tail/gu_tail [B, nb-1, I] (the carried FIR input; NULL =
 * zeros), x0/gx0/x_last/g_xlast [B, I*O, na] newest first (NULL x0 = zeros; x_last, g_xlast may
 * be NULL). `saved` [saved_doubles] (fp64) receives the per-super-chunk entering states for the
 * backward (may be NULL for inference). The workspace holds the look-back state of a single-pass
 * scan, re-initialised by each call on its stream: two calls in flight must not share one.
 */
int64_t tsfast_hip_gblock_workspace_bytes(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na);
int64_t tsfast_hip_gblock_saved_doubles(int64_t B, int64_t L, int64_t I, int64_t O, int64_t na);
int tsfast_hip_gblock_fwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na, const float* u,
                          const float* b, const float* a, const float* u_tail, const float* x0, float* y,
                          float* x_last, double* saved, void* workspace, int64_t workspace_bytes, void* stream);
/* gb, ga: full parameter gradients (summed over batch and time); gu_tail and gx0 may be NULL. */
int tsfast_hip_gblock_bwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, int64_t na, const float* gy,
                          const float* g_xlast, const float* u, const float* b, const float* a, const float* u_tail,
                          const float* x0, const double* saved, float* gu, float* gu_tail, float* gb, float* ga,
                          float* gx0, void* workspace, int64_t workspace_bytes, void* stream);
/* The G-block's FIR stage alone, for blocks the fused kernels decline (denominator orders above 4):
 * the grouped causal convolution F.conv1d(cat(u_tail, u), flipped taps, groups=I) of
 * dynonet/core.py:219-222, w[b, j*O + o, t] = sum_{k < nb} b[o, j, k] u[b, t - k, j] (u before the
 * sequence from u_tail, zero when NULL), written in the all-pole lane layout w [B, I*O, L]; the
 * pairs then run tsfast_hip_allpole_fwd/bwd and are summed over inputs by the caller. The
 * backward gives gu [B, L, I], gu_tail [B, nb-1, I] (may be NULL) and gb [O, I, nb] (summed over
 * batch and time in a fixed order; the workspace holds fp64 per-tile partials). 1 <= nb <= 64. */
int64_t tsfast_hip_gblock_fir_workspace_bytes(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb);
int tsfast_hip_gblock_fir_fwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, const float* u, const float* b,
                              const float* u_tail, float* w, void* stream);
int tsfast_hip_gblock_fir_bwd(int64_t B, int64_t L, int64_t I, int64_t O, int64_t nb, const float* gw,
                              const float* u, const float* b, const float* u_tail, float* gu, float* gu_tail,
                              float* gb, void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Constant-matrix linear recurrence  x_t = A x_{t-1} + v_t  (x_0 = x0, zero when NULL), the
 * tsfast::linear_recurrence op and its adjoint tsfast::linear_recurrence_bwd
 * (tsfast/models/architectures/dynonet/core.py:45-52 forward, :60-73 adjoint
 * G_t = A^T G_{t+1} + g_t, grad_A = sum_t G_t x_{t-1}^T, grad_x0 = A^T G_1; the reference runs
 * both as log-doubling scans, :23-37). Lanes are the flattened leading dims:
 * A/gA [lanes, n, n] row-major, v/x/g/gv [lanes, L, n] contiguous, x0/gx0 [lanes, n].
 * float32 in and out, fp64 state; 1 <= n <= 16, else TSF_ERR_UNSUPPORTED (n <= 4: a single-pass
 * look-back scan; n = 5..16: chunk summaries, a per-lane carry and a re-run, with L at most
 * 65535 * 256; n = 9..16 run each lane and chunk on a group of 16 threads, one state component
 * each). The workspace holds the scan's intermediate state, re-initialised by each call
 * on its stream: two calls in flight must not share one.
 */
int64_t tsfast_hip_linrec_workspace_bytes(int64_t lanes, int64_t L, int64_t n);
int tsfast_hip_linrec_fwd(int64_t lanes, int64_t L, int64_t n, const float* A, const float* v, const float* x0,
                          float* x, void* workspace, int64_t workspace_bytes, void* stream);
/* out = the forward's x; gA is the full per-lane gradient; gx0 written iff x0 given. */
int tsfast_hip_linrec_bwd(int64_t lanes, int64_t L, int64_t n, const float* g, const float* A, const float* out,
                          const float* x0, float* gA, float* gv, float* gx0, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* ------------------------------------------------------------------------------------------
 * Projected complex diagonal scan, the LRU / S5 layer core in one pass:
 *   v_t = W u_t,  x_t = lam * x_{t-1} + v_t (x_{-1} = x0, zero when NULL),  y_t = Re(C x_t).
 * Replaces the composition complex_in_proj -> diagonal_recurrence -> real_out_proj
 * (tsfast/models/_core/scan.py:221-243, 272-313) as LRU.forward (architectures/lru.py:100-110)
 * and S5.forward (architectures/s5.py:180-198) call it, plus the returned state x[..., -1, :].
 * Layout: u [B, L, H] float32; w_re/w_im [N, H]; lam [N] complex64 (interleaved re, im);
 * c_re/c_im [O, N]; x0 and x_last [B, N] complex64; y [B, L, O] float32; all contiguous.
 * Limits: H <= 32, N <= 256, O <= 32 and B * L * H * 4 < 2^31, else TSF_ERR_UNSUPPORTED. Wider
 * layers run as two GEMMs around tsfast_hip_diag_fwd / tsfast_hip_diag_bwd (the Python backend's
 * wide route), which have no width limits.
 * saved (may be NULL) receives the state entering each 32-step sub-chunk, [B, ceil(L/32), N]
 * complex64 (tsfast_hip_projscan_saved_floats floats), for the backward pass. The workspace holds
 * the look-back words, re-initialised by each call on its stream: two calls in flight must not
 * share one.
 */
int64_t tsfast_hip_projscan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O);
int64_t tsfast_hip_projscan_saved_floats(int64_t B, int64_t L, int64_t N);
int tsfast_hip_projscan_fwd(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O, const float* u, const float* w_re,
                            const float* w_im, const void* lam, const float* c_re, const float* c_im, const void* x0,
                            float* y, void* x_last, float* saved, void* workspace, int64_t workspace_bytes,
                            void* stream);
/* Adjoint of tsfast_hip_projscan_fwd (the autograd of the same reference composition):
 * gy [B, L, O] float32, g_xlast [B, N] complex64 (gradient of the returned state; NULL = zero),
 * saved = the forward's saved states. Writes g_u [B, L, H], g_w_re/g_w_im [N, H], g_lam [N]
 * complex64 (summed over rows), g_c_re/g_c_im [O, N], and g_x0 [B, N] complex64 when non-NULL.
 * Parameter gradients are per-workgroup partial sums added in a fixed workgroup order. */
int64_t tsfast_hip_projscan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O);
int tsfast_hip_projscan_bwd(int64_t B, int64_t L, int64_t H, int64_t N, int64_t O, const float* gy,
                            const void* g_xlast, const float* saved, const float* u, const float* w_re,
                            const float* w_im, const void* lam, const float* c_re, const float* c_im, float* g_u,
                            float* g_w_re, float* g_w_im, void* g_lam, float* g_c_re, float* g_c_im, void* g_x0,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Chunked adjoint of a time-varying matrix recurrence (the sequence-parallel part of a
 * NeuralStateSpace backward). Replaces the pair ssm_bwd_summary + ssm_bwd_scan
 * (tsfast/models/architectures/ssm/backend_metal.py:285-357) as `backward` calls it (:466-476):
 *   jt [B, L, n, n] float32 (per-step matrices A_t, row-major), gout [B, L, n] float32;
 *   gy_t = gout_t + A_{t+1} gy_{t+1}, gy_{L-1} = gout_{L-1};
 *   chunks of CL steps, C = ceil(L / CL); writes bnd [B, C + 1, n] float32, bnd[b, c] = gy at the
 *   first step of chunk c, bnd[b, C] = 0.
 * 1 <= n <= 32 (TSF_ERR_UNSUPPORTED above). Summaries in fp64 on the matrix cores; the workspace
 * holds them ([B, C, n, n + 1] doubles). */
int64_t tsfast_hip_mat_adjoint_workspace_bytes(int64_t B, int64_t L, int64_t n, int64_t CL);
int tsfast_hip_mat_adjoint_bounds(int64_t B, int64_t L, int64_t n, int64_t CL, const float* jt, const float* gout,
                                  float* bnd, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TSFAST_HIP_H */
