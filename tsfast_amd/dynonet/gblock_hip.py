"""Fused dynoNet G-block, HIP backend: FIR + all-pole + sum over inputs in one pass.

The body of ``LinearDynamicalOperator.forward`` (``tsfast/models/architectures/dynonet/core.py:196-258``)
for a non-zero denominator: the reference forms ``w = F.conv1d(cat(u_tail, u), flipped taps,
groups=I)`` (``:219-222``), runs the all-pole op per pair (``:225-235``, ``_fused_allpole``) and sums
the pairs over inputs (``:250``). Here one kernel per direction does all three, so neither ``w``
nor the per-pair outputs (each ``[B, I*O, L]``) reach HBM; the backward recomputes the pair
outputs from per-super-chunk states the forward saves (a few MB).

``supports(u, b_coeff, a_coeff, u_tail, x0)`` and ``run(u, b_coeff, a_coeff, u_tail, x0) ->
(y, x_last)``, differentiable in all inputs through the ``tsfast_hip::dynonet_gblock`` /
``dynonet_gblock_bwd`` custom ops. Shapes follow the reference: ``u [B, L, I]``, ``b_coeff
[O, I, nb]``, ``a_coeff [O, I, na]``, ``u_tail [B, nb-1, I]``, ``x0 [B, I*O, na]`` (pairs input-major,
newest first); ``y [B, L, O]``, ``x_last [B, I*O, na]``. float32, any number of channel pairs.
Orders ``na <= 4`` with ``nb <= 8`` run the fused kernels: one launch per direction serves up to
64 pairs (a batch row's pairs padded to a power of two inside the kernels); a larger block runs as
groups of whole inputs (and, past 64 outputs, of outputs) of at most 64 pairs each, whose outputs
and gradients add up. Orders ``5 <= na <= 16`` (or ``9 <= nb <= 64``) run the three stages on this
library's kernels: the FIR stage (``tsfast_hip::dynonet_fir``, writing ``w`` in the all-pole lane
layout), the all-pole op on the pair lanes (``allpole_hip``), and a sum over inputs.
"""

from __future__ import annotations

__all__ = ["supports", "run"]

import torch

from .. import _lib

_MAX_NA = 4  # orders of the fused kernels
_MAX_NB = 8  # taps the operator fuses (the kernels take up to 16; 9..16 ran 1.5x slower than staged)
_MAX_PAIRS = 64  # pairs one launch serves (a tile of 64 lanes holds whole batch rows)
_MAX_NA_STAGED = 16  # orders of the staged path (the all-pole kernels' range)
_MAX_NB_STAGED = 64  # taps of the FIR kernel


def supports(u, b_coeff, a_coeff, u_tail, x0) -> str | None:
    """Reason the fused G-block kernel cannot handle these tensors, or None if it can."""
    if u.device.type != "cuda":
        return f"u on {u.device.type}, hip backend is GPU-only"
    tensors = {"u": u, "b_coeff": b_coeff, "a_coeff": a_coeff, "u_tail": u_tail, "x0": x0}
    for name, t in tensors.items():
        if t is None:
            continue
        if t.dtype != torch.float32:
            return f"{name} dtype {t.dtype} not float32"
        if t.device != u.device:
            return f"{name} on {t.device}, u on {u.device}"
    if u.dim() != 3 or b_coeff.dim() != 3 or a_coeff.dim() != 3:
        return "expected u [B, L, I], b_coeff [O, I, nb], a_coeff [O, I, na]"
    B, L, I = u.shape
    O, I_b, nb = b_coeff.shape
    na = a_coeff.shape[-1]
    if I_b != I or tuple(a_coeff.shape[:2]) != (O, I):
        return f"coefficient shapes {tuple(b_coeff.shape)}, {tuple(a_coeff.shape)} do not match {I} inputs"
    if not 1 <= na <= _MAX_NA_STAGED:
        return f"denominator order {na} outside [1, {_MAX_NA_STAGED}]"
    if not 1 <= nb <= _MAX_NB_STAGED:
        return f"numerator taps {nb} outside [1, {_MAX_NB_STAGED}]"
    if u_tail is not None and tuple(u_tail.shape) != (B, nb - 1, I):
        return f"u_tail.shape {tuple(u_tail.shape)} != {(B, nb - 1, I)}"
    if x0 is not None and tuple(x0.shape) != (B, I * O, na):
        return f"x0.shape {tuple(x0.shape)} != {(B, I * O, na)}"
    return None


def _dims(u, b, a):
    B, L, I = u.shape
    O, _, nb = b.shape
    return B, L, I, O, nb, a.shape[-1]


def _workspace(lib, u, b, a):
    n = lib.tsfast_hip_gblock_workspace_bytes(*_dims(u, b, a))
    if n < 0:
        raise RuntimeError("tsfast_hip_gblock_workspace_bytes: unsupported shape")
    return _lib.workspace(n, u.device), n


def _screen(u, b, a, u_tail, x0):
    dev = u.device
    for name, t in (("u", u), ("b_coeff", b), ("a_coeff", a), ("u_tail", u_tail), ("x0", x0)):
        _lib.require(t, name, (torch.float32,), dev)


@torch.library.custom_op("tsfast_hip::dynonet_gblock", mutates_args=())
def _gblock_op(
    u: torch.Tensor, b: torch.Tensor, a: torch.Tensor, u_tail: torch.Tensor | None, x0: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    _lib.sync_deterministic()
    u, b, a = u.contiguous(), b.contiguous(), a.contiguous()
    u_tail = u_tail.contiguous() if u_tail is not None else None
    x0 = x0.contiguous() if x0 is not None else None
    _screen(u, b, a, u_tail, x0)
    B, L, I, O, nb, na = _dims(u, b, a)
    y = torch.empty(B, L, O, device=u.device, dtype=torch.float32)
    x_last = torch.empty(B, I * O, na, device=u.device, dtype=torch.float32)
    saved = torch.empty(max(lib.tsfast_hip_gblock_saved_doubles(B, L, I, O, na), 1), device=u.device,
                        dtype=torch.float64)
    ws, nbytes = _workspace(lib, u, b, a)
    _lib.check(
        lib.tsfast_hip_gblock_fwd(
            B, L, I, O, nb, na, _lib.ptr(u), _lib.ptr(b), _lib.ptr(a), _lib.ptr(u_tail), _lib.ptr(x0), _lib.ptr(y),
            _lib.ptr(x_last), _lib.ptr(saved), _lib.ptr(ws), nbytes, _lib.stream_of(u),
        ),
        "tsfast_hip_gblock_fwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_gblock_fwd")
    return y, x_last, saved


@_gblock_op.register_fake
def _(u, b, a, u_tail, x0):
    B, L, I = u.shape
    O = b.shape[0]
    na = a.shape[-1]
    # the saved boundary states must have the size the real op allocates, or a compiled graph's
    # metadata disagrees with what the kernel writes
    n_saved = _lib.load().tsfast_hip_gblock_saved_doubles(int(B), int(L), int(I), int(O), int(na))
    return u.new_empty(B, L, O), u.new_empty(B, I * O, na), u.new_empty(max(n_saved, 1), dtype=torch.float64)


@torch.library.custom_op("tsfast_hip::dynonet_gblock_bwd", mutates_args=())
def _gblock_bwd_op(
    gy: torch.Tensor, g_xlast: torch.Tensor | None, u: torch.Tensor, b: torch.Tensor, a: torch.Tensor,
    u_tail: torch.Tensor | None, x0: torch.Tensor | None, saved: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    _lib.sync_deterministic()
    gy = gy.contiguous()
    g_xlast = g_xlast.contiguous() if g_xlast is not None else None
    _lib.require(gy, "gy", (torch.float32,), u.device)
    _lib.require(g_xlast, "g_xlast", (torch.float32,), u.device)
    B, L, I, O, nb, na = _dims(u, b, a)
    gu = torch.empty_like(u)
    gu_tail = torch.zeros(B, nb - 1, I, device=u.device, dtype=torch.float32)
    gb = torch.empty_like(b)
    ga = torch.empty_like(a)
    gx0 = torch.empty(B, I * O, na, device=u.device, dtype=torch.float32)
    ws, nbytes = _workspace(lib, u, b, a)
    _lib.check(
        lib.tsfast_hip_gblock_bwd(
            B, L, I, O, nb, na, _lib.ptr(gy), _lib.ptr(g_xlast), _lib.ptr(u), _lib.ptr(b), _lib.ptr(a),
            _lib.ptr(u_tail), _lib.ptr(x0), _lib.ptr(saved), _lib.ptr(gu), _lib.ptr(gu_tail), _lib.ptr(gb),
            _lib.ptr(ga), _lib.ptr(gx0), _lib.ptr(ws), nbytes, _lib.stream_of(u),
        ),
        "tsfast_hip_gblock_bwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_gblock_bwd")
    return gu, gu_tail, gb, ga, gx0


@_gblock_bwd_op.register_fake
def _(gy, g_xlast, u, b, a, u_tail, x0, saved):
    B, _, I = u.shape
    O, _, nb = b.shape
    na = a.shape[-1]
    return (torch.empty_like(u), u.new_empty(B, nb - 1, I), torch.empty_like(b), torch.empty_like(a),
            u.new_empty(B, I * O, na))


def _gblock_setup(ctx, inputs, output):
    u, b, a, u_tail, x0 = inputs
    _, _, saved = output
    ctx.has_tail, ctx.has_x0 = u_tail is not None, x0 is not None
    ctx.save_for_backward(u, b, a, u_tail, x0, saved)


def _gblock_backward(ctx, gy, g_xlast, g_saved):
    u, b, a, u_tail, x0, saved = ctx.saved_tensors
    if gy is None:
        gy = torch.zeros(u.shape[0], u.shape[1], b.shape[0], device=u.device, dtype=torch.float32)
    gu, gu_tail, gb, ga, gx0 = _gblock_bwd_op(gy, g_xlast, u.contiguous(), b.contiguous(), a.contiguous(),
                                              u_tail.contiguous() if u_tail is not None else None,
                                              x0.contiguous() if x0 is not None else None, saved)
    return gu, gb, ga, (gu_tail if ctx.has_tail else None), (gx0 if ctx.has_x0 else None)


_gblock_op.register_autograd(_gblock_backward, setup_context=_gblock_setup)


def _groups(I: int, O: int) -> tuple[list[range], list[range]]:
    """Input and output ranges whose pair counts fit one launch (``_MAX_PAIRS``)."""
    go = min(O, _MAX_PAIRS)
    gi = max(1, _MAX_PAIRS // go)
    return ([range(i, min(i + gi, I)) for i in range(0, I, gi)], [range(o, min(o + go, O)) for o in range(0, O, go)])


def _fused(na: int, nb: int) -> bool:
    return na <= _MAX_NA and nb <= _MAX_NB


# ------------------------------------------------------------------------------ staged path
@torch.library.custom_op("tsfast_hip::dynonet_fir", mutates_args=())
def _fir_op(u: torch.Tensor, b: torch.Tensor, u_tail: torch.Tensor | None) -> torch.Tensor:
    lib = _lib.load()
    u, b = u.contiguous(), b.contiguous()
    u_tail = u_tail.contiguous() if u_tail is not None else None
    for name, t in (("u", u), ("b_coeff", b), ("u_tail", u_tail)):
        _lib.require(t, name, (torch.float32,), u.device)
    B, L, I = u.shape
    O, _, nb = b.shape
    w = torch.empty(B, I * O, L, device=u.device, dtype=torch.float32)
    _lib.check(
        lib.tsfast_hip_gblock_fir_fwd(B, L, I, O, nb, _lib.ptr(u), _lib.ptr(b), _lib.ptr(u_tail), _lib.ptr(w),
                                      _lib.stream_of(u)),
        "tsfast_hip_gblock_fir_fwd",
    )
    return w


@_fir_op.register_fake
def _(u, b, u_tail):
    B, L, I = u.shape
    return u.new_empty(B, I * b.shape[0], L)


@torch.library.custom_op("tsfast_hip::dynonet_fir_bwd", mutates_args=())
def _fir_bwd_op(
    gw: torch.Tensor, u: torch.Tensor, b: torch.Tensor, u_tail: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    gw = gw.contiguous()
    _lib.require(gw, "gw", (torch.float32,), u.device)
    B, L, I = u.shape
    O, _, nb = b.shape
    gu = torch.empty_like(u)
    gu_tail = torch.zeros(B, nb - 1, I, device=u.device, dtype=torch.float32)
    gb = torch.empty_like(b)
    n = lib.tsfast_hip_gblock_fir_workspace_bytes(B, L, I, O, nb)
    if n < 0:
        raise RuntimeError("tsfast_hip_gblock_fir_workspace_bytes: unsupported shape")
    ws = _lib.workspace(n, u.device)
    _lib.check(
        lib.tsfast_hip_gblock_fir_bwd(
            B, L, I, O, nb, _lib.ptr(gw), _lib.ptr(u), _lib.ptr(b), _lib.ptr(u_tail), _lib.ptr(gu),
            _lib.ptr(gu_tail), _lib.ptr(gb), _lib.ptr(ws), n, _lib.stream_of(u),
        ),
        "tsfast_hip_gblock_fir_bwd",
    )
    return gu, gu_tail, gb


@_fir_bwd_op.register_fake
def _(gw, u, b, u_tail):
    B, _, I = u.shape
    return torch.empty_like(u), u.new_empty(B, b.shape[-1] - 1, I), torch.empty_like(b)


def _fir_setup(ctx, inputs, output):
    u, b, u_tail = inputs
    ctx.has_tail = u_tail is not None
    ctx.save_for_backward(u, b, u_tail)


def _fir_backward(ctx, gw):
    u, b, u_tail = ctx.saved_tensors
    gu, gu_tail, gb = _fir_bwd_op(gw, u.contiguous(), b.contiguous(),
                                  u_tail.contiguous() if u_tail is not None else None)
    return gu, gb, (gu_tail if ctx.has_tail else None)


_fir_op.register_autograd(_fir_backward, setup_context=_fir_setup)


def _run_staged(u, b_coeff, a_coeff, u_tail, x0):
    """FIR stage, all-pole op on the pair lanes and the sum over inputs, as the reference's three
    stages (dynonet/core.py:219-250) but on this library's kernels; every step is differentiable."""
    from . import allpole_hip

    B, L, I = u.shape
    O, _, nb = b_coeff.shape
    na = a_coeff.shape[-1]
    P = I * O
    w = _fir_op(u, b_coeff, u_tail)  # [B, P, L], pair p = j * O + o
    a_pairs = a_coeff.permute(1, 0, 2).reshape(P, na)
    y_pairs = allpole_hip.run(a_pairs, w, x0)
    if L >= na:
        x_last = y_pairs[..., L - na :].flip(-1)
    else:
        head = x0[..., : na - L] if x0 is not None else y_pairs.new_zeros(B, P, na - L)
        x_last = torch.cat((y_pairs.flip(-1), head), dim=-1)
    y = y_pairs.view(B, I, O, L).sum(1).transpose(1, 2)
    return y, x_last


def run(u, b_coeff, a_coeff, u_tail, x0):
    """Fused G-block: ``y [B, L, O]`` and the all-pole state ``x_last [B, I*O, na]`` (newest first).

    ``u_tail`` (the last ``nb - 1`` inputs before ``u``) and ``x0`` may be None (zero initial
    conditions). Differentiable in all inputs (``tsfast_hip::dynonet_gblock``). More than 64
    pairs run as groups (``_groups``): the pair outputs of a group of inputs sum into y like any
    other pairs, so y adds the groups' outputs and each pair's state comes from its own group.
    """
    I, O = u.shape[-1], b_coeff.shape[0]
    if not _fused(a_coeff.shape[-1], b_coeff.shape[-1]):
        return _run_staged(u, b_coeff, a_coeff, u_tail, x0)
    if I * O <= _MAX_PAIRS:
        y, x_last, _ = _gblock_op(u, b_coeff, a_coeff, u_tail, x0)
        return y, x_last
    B, na = u.shape[0], a_coeff.shape[-1]
    in_groups, out_groups = _groups(I, O)
    x0v = None if x0 is None else x0.view(B, I, O, na)
    y_cols, x_rows = [], [[None] * len(out_groups) for _ in in_groups]
    for oi, og in enumerate(out_groups):
        o0, o1 = og.start, og.stop
        y_part = None
        for ii, ig in enumerate(in_groups):
            i0, i1 = ig.start, ig.stop
            x0g = None if x0v is None else x0v[:, i0:i1, o0:o1].reshape(B, (i1 - i0) * (o1 - o0), na)
            yg, xg, _ = _gblock_op(
                u[..., i0:i1], b_coeff[o0:o1, i0:i1], a_coeff[o0:o1, i0:i1],
                None if u_tail is None else u_tail[..., i0:i1], x0g,
            )
            y_part = yg if y_part is None else y_part + yg
            x_rows[ii][oi] = xg.view(B, i1 - i0, o1 - o0, na)
        y_cols.append(y_part)
    y = torch.cat(y_cols, dim=-1) if len(y_cols) > 1 else y_cols[0]
    x_last = torch.cat([torch.cat(row, dim=2) for row in x_rows], dim=1).reshape(B, I * O, na)
    return y, x_last
