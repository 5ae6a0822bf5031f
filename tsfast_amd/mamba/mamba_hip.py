"""Fused HIP backend for the Mamba selective SSM section (softplus discretisation, exp(delta A),
input injection, recurrence, C contraction, D skip and SiLU gate in one kernel).

Drop-in for the ``mamba.ssm`` registry of ``tsfast/models/architectures/mamba/core.py:22-23``
(the role of ``mamba_triton.py:286-534``): ``supports(draw, A, Bt, Ct, u, z, Dp, h0)`` and
``run(...) -> (out [B, L, D], h_last [B, D, N])``, differentiable in all eight inputs through
the ``tsfast_hip::mamba_scan`` / ``mamba_scan_train`` / ``mamba_scan_bwd`` custom ops.

Two I/O regimes: float32 everywhere (tsfast's regime), or bfloat16 sequence tensors
(draw, u, z, Bt, Ct and their gradients) with float32 parameters (A, Dp) and float32 state
(h0, h_last, the checkpoints). The state never leaves registers in fp32 arithmetic; only the
training forward saves state for the backward: one fp32 checkpoint per channel every
``chk_interval(N)`` steps (``tsfast_hip_mamba_chk_interval``), from which the backward
recomputes, and the output before the gate (in the I/O dtype). The saved tensor is
[B, saved_floats(L, D, N, dtype)] float32 words (per batch row: checkpoints [NC, N, D], then
y [L, D]).
"""

from __future__ import annotations

__all__ = ["supports", "run", "chk_interval", "saved_floats"]

import torch

from .. import _lib

_IO_DTYPES = {torch.float32: _lib.TSF_DTYPE_F32, torch.bfloat16: _lib.TSF_DTYPE_BF16}
_MAX_N = 64


def _state_tile(N: int) -> int:
    """N rounded up to the kernels' state tile (4, 8, 16, 32 or 64)."""
    return next(k for k in (4, 8, 16, 32, 64) if N <= k)


def _chk_steps(N: int) -> int:
    """Checkpoint interval for state size N (the kernels' MCfg<NS>::CHK; tests pin it against
    tsfast_hip_mamba_chk_interval). Kept in Python so that supports() makes no library call."""
    return 4 if _state_tile(N) == 64 else 8


def _rows_fit(L: int, D: int, N: int) -> bool:
    """The kernels' per-batch-row addressing limit (mamba.hip offsets_fit): one row of every
    [B, L, *] tensor, of the saved state and of the grad-B/C partials below 2 GiB of fp32."""
    lim = (1 << 31) // 4
    nc = -(-L // _chk_steps(N))
    return (L + 64) * D < lim and (L + 64) * 2 * _state_tile(N) < lim and nc * N * D + L * D < lim


def chk_interval(N: int) -> int:
    """Checkpoint interval (steps) the kernels use for state size N."""
    return int(_lib.load().tsfast_hip_mamba_chk_interval(N))


def saved_floats(L: int, D: int, N: int, dtype: torch.dtype = torch.float32) -> int:
    """float32 words of training-forward saved state per batch row for I/O dtype ``dtype``:
    fp32 checkpoints [NC, N, D], then the pre-gate output y [L, D] in ``dtype`` (padded to whole
    words). Computed here rather than through the library, so that the training op's fake
    implementation makes no library call while torch.compile traces it (tests pin this formula
    against tsfast_hip_mamba_saved_floats)."""
    nc = -(-L // _chk_steps(N))
    esz = 2 if dtype == torch.bfloat16 else 4
    return nc * N * D + (L * D * esz + 3) // 4


def supports(draw, A, Bt, Ct, u, z, Dp, h0) -> str | None:
    """Reason the fused HIP kernel cannot handle these tensors, or None if it can."""
    seq = {"draw": draw, "Bt": Bt, "Ct": Ct, "u": u, "z": z}
    params = {"A": A, "Dp": Dp}
    if h0 is not None:
        params["h0"] = h0
    for name, t in {**seq, **params}.items():
        if t.device.type != "cuda":
            return f"{name} on {t.device.type}, hip backend is GPU-only"
        if t.device != draw.device:
            return f"{name} on {t.device}, expected {draw.device}"
    if draw.dtype not in _IO_DTYPES:
        return f"sequence dtype {draw.dtype} unsupported (need float32 or bfloat16)"
    for name, t in seq.items():
        if t.dtype != draw.dtype:
            return f"{name} dtype {t.dtype} != draw dtype {draw.dtype}"
    for name, t in params.items():
        if t.dtype != torch.float32:
            return f"needs float32 {name}, got {t.dtype}"
    if draw.dim() != 3:
        return f"draw must be [B, L, D], got {draw.dim()} dims"
    B, L, D = draw.shape
    if A.dim() != 2:
        return f"A must be [D, N], got {tuple(A.shape)}"
    N = A.shape[-1]
    if tuple(A.shape) != (D, N):
        return f"A.shape {tuple(A.shape)} incompatible with draw {tuple(draw.shape)}"
    if N < 1:
        return f"state size N={N} below 1"
    dt = 16 if min(N, _MAX_N) > 16 else 32  # the backward's channel tile (the forward's is 32)
    if -(-D // dt) * B > 2**31 - 1:
        return f"{B} batch rows x {-(-D // dt)} channel tiles exceed the kernels' one-dimensional grid"
    if not _rows_fit(L, D, min(N, _MAX_N)):
        return f"one batch row (L={L}, D={D}, N={N}) exceeds the kernels' 2 GiB per-row addressing"
    if tuple(u.shape) != (B, L, D) or tuple(z.shape) != (B, L, D):
        return f"u/z shapes {tuple(u.shape)}/{tuple(z.shape)} != {(B, L, D)}"
    if tuple(Bt.shape) != (B, L, N) or tuple(Ct.shape) != (B, L, N):
        return f"Bt/Ct shapes {tuple(Bt.shape)}/{tuple(Ct.shape)} != {(B, L, N)}"
    if tuple(Dp.shape) != (D,):
        return f"Dp.shape {tuple(Dp.shape)} != {(D,)}"
    if h0 is not None and tuple(h0.shape) != (B, D, N):
        return f"h0.shape {tuple(h0.shape)} != {(B, D, N)}"
    return None


def _contig(*ts):
    return [t.contiguous() if t is not None else None for t in ts]


def _check_inputs(draw, A, Bt, Ct, u, z, Dp, h0):
    io = (draw.dtype,)
    dev = draw.device
    for name, t in (("draw", draw), ("Bt", Bt), ("Ct", Ct), ("u", u), ("z", z)):
        _lib.require(t, name, io, dev)
    for name, t in (("A", A), ("Dp", Dp), ("h0", h0)):
        _lib.require(t, name, (torch.float32,), dev)


def _forward(draw, A, Bt, Ct, u, z, Dp, h0, store_chk: bool):
    lib = _lib.load()
    _check_inputs(draw, A, Bt, Ct, u, z, Dp, h0)
    B, L, D = draw.shape
    N = A.shape[-1]
    out = torch.empty_like(draw)
    h_last = torch.empty(B, D, N, device=draw.device, dtype=torch.float32)
    chk = None
    if store_chk:
        chk = torch.empty(B, saved_floats(L, D, N, draw.dtype), device=draw.device, dtype=torch.float32)
    _lib.check(
        lib.tsfast_hip_mamba_fwd(
            B, L, D, N, _IO_DTYPES[draw.dtype], *map(_lib.ptr, (draw, A, Bt, Ct, u, z, Dp, h0, out, h_last, chk)),
            _lib.stream_of(draw),
        ),
        "tsfast_hip_mamba_fwd",
    )
    return out, h_last, chk


@torch.library.custom_op("tsfast_hip::mamba_scan", mutates_args=())
def _scan_op(
    draw: torch.Tensor,
    A: torch.Tensor,
    Bt: torch.Tensor,
    Ct: torch.Tensor,
    u: torch.Tensor,
    z: torch.Tensor,
    Dp: torch.Tensor,
    h0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor]:
    draw, A, Bt, Ct, u, z, Dp, h0 = _contig(draw, A, Bt, Ct, u, z, Dp, h0)
    out, h_last, _ = _forward(draw, A, Bt, Ct, u, z, Dp, h0, store_chk=False)
    return out, h_last


@torch.library.custom_op("tsfast_hip::mamba_scan_train", mutates_args=())
def _scan_train_op(
    draw: torch.Tensor,
    A: torch.Tensor,
    Bt: torch.Tensor,
    Ct: torch.Tensor,
    u: torch.Tensor,
    z: torch.Tensor,
    Dp: torch.Tensor,
    h0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    draw, A, Bt, Ct, u, z, Dp, h0 = _contig(draw, A, Bt, Ct, u, z, Dp, h0)
    out, h_last, chk = _forward(draw, A, Bt, Ct, u, z, Dp, h0, store_chk=True)
    return out, h_last, chk


def _fake_outs(draw, A, with_chk: bool):
    B, L, D = draw.shape
    N = A.shape[-1]
    out = torch.empty_like(draw)
    h_last = draw.new_empty(B, D, N, dtype=torch.float32)
    if not with_chk:
        return out, h_last
    return out, h_last, draw.new_empty(B, saved_floats(L, D, N, draw.dtype), dtype=torch.float32)


@_scan_op.register_fake
def _(draw, A, Bt, Ct, u, z, Dp, h0):
    return _fake_outs(draw, A, with_chk=False)


@_scan_train_op.register_fake
def _(draw, A, Bt, Ct, u, z, Dp, h0):
    return _fake_outs(draw, A, with_chk=True)


@torch.library.custom_op("tsfast_hip::mamba_scan_bwd", mutates_args=())
def _scan_bwd_op(
    gout: torch.Tensor,
    ghlast: torch.Tensor | None,
    chk: torch.Tensor,
    draw: torch.Tensor,
    A: torch.Tensor,
    Bt: torch.Tensor,
    Ct: torch.Tensor,
    u: torch.Tensor,
    z: torch.Tensor,
    Dp: torch.Tensor,
    h0: torch.Tensor | None,
) -> tuple[
    torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor
]:
    lib = _lib.load()
    gout, ghlast, chk, draw, A, Bt, Ct, u, z, Dp, h0 = _contig(gout, ghlast, chk, draw, A, Bt, Ct, u, z, Dp, h0)
    _check_inputs(draw, A, Bt, Ct, u, z, Dp, h0)
    _lib.require(gout, "gout", (draw.dtype,), draw.device)
    _lib.require(ghlast, "ghlast", (torch.float32,), draw.device)
    _lib.require(chk, "chk", (torch.float32,), draw.device)
    B, L, D = draw.shape
    N = A.shape[-1]
    gdraw = torch.empty_like(draw)
    gu = torch.empty_like(draw)
    gz = torch.empty_like(draw)
    gBt = torch.empty_like(Bt)
    gCt = torch.empty_like(Ct)
    gA = torch.empty(D, N, device=draw.device, dtype=torch.float32)
    gDp = torch.empty(D, device=draw.device, dtype=torch.float32)
    gh0 = torch.empty(B, D, N, device=draw.device, dtype=torch.float32) if h0 is not None else None
    nbytes = lib.tsfast_hip_mamba_workspace_bytes(B, L, D, N)
    ws = _lib.workspace(nbytes, draw.device)
    _lib.check(
        lib.tsfast_hip_mamba_bwd(
            B, L, D, N, _IO_DTYPES[draw.dtype],
            *map(_lib.ptr, (draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gA, gBt, gCt, gu, gz, gDp, gh0, ws)),
            nbytes, _lib.stream_of(draw),
        ),
        "tsfast_hip_mamba_bwd",
    )
    return gdraw, gA, gBt, gCt, gu, gz, gDp, (gh0 if gh0 is not None else draw.new_empty(0, dtype=torch.float32))


@_scan_bwd_op.register_fake
def _(gout, ghlast, chk, draw, A, Bt, Ct, u, z, Dp, h0):
    B, L, D = draw.shape
    N = A.shape[-1]
    f32 = torch.float32
    return (
        torch.empty_like(draw),
        draw.new_empty(D, N, dtype=f32),
        torch.empty_like(Bt),
        torch.empty_like(Ct),
        torch.empty_like(draw),
        torch.empty_like(draw),
        draw.new_empty(D, dtype=f32),
        (draw.new_empty(B, D, N, dtype=f32) if h0 is not None else draw.new_empty(0, dtype=f32)),
    )


def _scan_setup(ctx, inputs, output):
    draw, A, Bt, Ct, u, z, Dp, h0 = inputs
    ctx.save_for_backward(draw, A, Bt, Ct, u, z, Dp, h0, output[2])


def _scan_backward(ctx, gout, ghlast, gchk):
    draw, A, Bt, Ct, u, z, Dp, h0, chk = ctx.saved_tensors
    if gout is None:
        gout = torch.zeros_like(draw)
    gdraw, gA, gBt, gCt, gu, gz, gDp, gh0 = _scan_bwd_op(gout, ghlast, chk, draw, A, Bt, Ct, u, z, Dp, h0)
    return gdraw, gA, gBt, gCt, gu, gz, gDp, (gh0 if h0 is not None else None)


_scan_train_op.register_autograd(_scan_backward, setup_context=_scan_setup)


def _run_group(draw, A, Bt, Ct, u, z, Dp, h0):
    inputs = (draw, A, Bt, Ct, u, z, Dp) + ((h0,) if h0 is not None else ())
    if not torch.is_grad_enabled() or not any(t.requires_grad for t in inputs):
        return _scan_op(draw, A, Bt, Ct, u, z, Dp, h0)
    out, h_last, _chk = _scan_train_op(draw, A, Bt, Ct, u, z, Dp, h0)
    return out, h_last


def run(draw, A, Bt, Ct, u, z, Dp, h0):
    """Fused Mamba SSM: ``h_t = exp(softplus(draw_t) A) h_{t-1} + softplus(draw_t) u_t B_t``,
    ``out_t = (h_t . C_t + Dp u_t) * silu(z_t)``.

    Returns ``(out [B, L, D], h_last [B, D, N] float32)``; differentiable in all inputs. Without
    grad the inference op (no checkpoints) runs. (Contract of ``mamba_triton.py:523-534``.)

    A launch serves at most 64 states. Larger N runs the states in groups of up to 64: the states
    evolve independently, and the output is linear in the per-state sum ``h . C`` for fixed
    draw, u, z (``out = (sum over groups of h_g . C_g + Dp u) * silu(z)``), so the groups' outputs
    add up to the output (the D skip goes with the first group only), and their gradients add up
    the same way through autograd. Each group's launch rounds its output (and its gradients of
    the I/O tensors) to the I/O dtype; the outputs are then added in float32 and rounded again,
    and autograd adds the groups' gradients in the I/O dtype. With float32 I/O that is ordinary
    float32 rounding; with bfloat16 I/O it is up to one bfloat16 rounding per group on top of the
    final one, inside the 2e-2 bar of bf16 I/O (the GPU tests at N 96 and 130 check it).
    """
    N = A.shape[-1]
    if N <= _MAX_N:
        return _run_group(draw, A, Bt, Ct, u, z, Dp, h0)
    outs, lasts = [], []
    for n0 in range(0, N, _MAX_N):
        n1 = min(n0 + _MAX_N, N)
        dp = Dp if n0 == 0 else torch.zeros_like(Dp)
        hg = h0[..., n0:n1] if h0 is not None else None
        o, hl = _run_group(draw, A[:, n0:n1], Bt[..., n0:n1], Ct[..., n0:n1], u, z, dp, hg)
        outs.append(o.float())
        lasts.append(hl)
    out = outs[0]
    for o in outs[1:]:
        out = out + o
    return out.to(draw.dtype), torch.cat(lasts, dim=-1)
