"""HIP backend for the projected complex diagonal scan (the LRU / S5 layer core), float32.

One pass computes ``y = real_out_proj(diagonal_recurrence(lam, complex_in_proj(u, W), x0), C)``
and the last state, the composition ``LRU.forward`` (``tsfast/models/architectures/lru.py:100-110``)
and ``S5.forward`` (``s5.py:180-198``) run through ``tsfast/models/_core/scan.py:221-243, 272-313``;
the complex ``v`` and ``x`` (``[B, L, N]`` each) never reach HBM. Kernels: ``csrc/projscan.hip``
(both projections on the fp32 matrix cores, the recurrence chained across chunks by a decoupled
look-back). Shapes: ``u [B, L, H]`` float32, ``W_re/W_im [N, H]``, ``lam [N]`` complex64,
``C_re/C_im [O, N]``, ``x0 [B, N]`` complex64 or None; H <= 32, N <= 256, O <= 32.
"""

from __future__ import annotations

__all__ = ["supports", "run"]

import torch

from .. import _lib

_MAX_H, _MAX_N, _MAX_O = 32, 256, 32
_SUB = 32  # steps per backward tile; the saved states entering each are [B, ceil(L / 32), N]


def supports(u, W_re, W_im, lam, C_re, C_im, x0) -> str | None:
    """Reason the fused kernel cannot handle these tensors, or None if it can."""
    if u.device.type != "cuda":
        return f"u on {u.device.type}, hip backend is GPU-only"
    for name, t in (("u", u), ("W_re", W_re), ("W_im", W_im), ("C_re", C_re), ("C_im", C_im)):
        if t.dtype != torch.float32:
            return f"{name} dtype {t.dtype} is not float32"
    for name, t in (("lam", lam), ("x0", x0)):
        if t is not None and t.dtype != torch.complex64:
            return f"{name} dtype {t.dtype} is not complex64"
    if any(t is not None and t.device != u.device for t in (W_re, W_im, lam, C_re, C_im, x0)):
        return "inputs on different devices"
    if u.dim() != 3 or W_re.dim() != 2 or C_re.dim() != 2 or lam.dim() != 1:
        return "expects u [B, L, H], W [N, H], lam [N], C [O, N]"
    B, L, H = u.shape
    N, O = lam.shape[0], C_re.shape[0]
    if tuple(W_re.shape) != (N, H) or tuple(W_im.shape) != (N, H):
        return f"W shapes {tuple(W_re.shape)}/{tuple(W_im.shape)} != {(N, H)}"
    if tuple(C_re.shape) != (O, N) or tuple(C_im.shape) != (O, N):
        return f"C shapes {tuple(C_re.shape)}/{tuple(C_im.shape)} != {(O, N)}"
    if x0 is not None and tuple(x0.shape) != (B, N):
        return f"x0 shape {tuple(x0.shape)} != {(B, N)}"
    return shape_reason(B, L, H, N, O)


def shape_reason(B: int, L: int, H: int, N: int, O: int) -> str | None:
    """The kernel's size limits (``ps_args_status`` in ``csrc/projscan.hip``): widths, and u / y /
    gy read through buffer resources with 32-bit byte offsets, chunk and row indices in int."""
    if H > _MAX_H or N > _MAX_N or O > _MAX_O:
        return f"H={H}, N={N}, O={O} beyond the kernel's H <= {_MAX_H}, N <= {_MAX_N}, O <= {_MAX_O}"
    if B * L * H * 4 >= 2**31:
        return f"u of {B * L * H * 4} bytes beyond the kernel's 2 GiB buffer addressing"
    if B * L * O * 4 >= 2**31:
        return f"y of {B * L * O * 4} bytes beyond the kernel's 2 GiB buffer addressing"
    if B > (2**31 - 1) // 2 or L > (2**31 - 1) // 2:
        return f"B={B} or L={L} beyond the kernel's int chunk and row indices"
    return None


def saved_floats(B: int, L: int, N: int) -> int:
    """Floats of the saved chunk-entering states (``tsfast_hip_projscan_saved_floats``)."""
    return 2 * B * (-(-L // _SUB)) * N


def _forward(u, W_re, W_im, lam, C_re, C_im, x0, train: bool):
    lib = _lib.load()
    _lib.sync_deterministic()
    dev = u.device
    for name, t in (("u", u), ("W_re", W_re), ("W_im", W_im), ("C_re", C_re), ("C_im", C_im)):
        _lib.require(t, name, (torch.float32,), dev)
    _lib.require(lam, "lam", (torch.complex64,), dev)
    _lib.require(x0, "x0", (torch.complex64,), dev)
    B, L, H = u.shape
    N, O = lam.shape[0], C_re.shape[0]
    y = torch.empty(B, L, O, device=dev, dtype=torch.float32)
    x_last = torch.empty(B, N, device=dev, dtype=torch.complex64)
    saved = torch.empty(saved_floats(B, L, N) if train else 0, device=dev, dtype=torch.float32)
    nbytes = lib.tsfast_hip_projscan_workspace_bytes(B, L, H, N, O)
    if nbytes < 0:
        raise RuntimeError(f"tsfast_hip_projscan_workspace_bytes: unsupported shape B={B} L={L} H={H} N={N} O={O}")
    ws = _lib.workspace(nbytes, dev)
    _lib.check(
        lib.tsfast_hip_projscan_fwd(
            B, L, H, N, O, *map(_lib.ptr, (u, W_re, W_im, lam, C_re, C_im, x0, y, x_last)),
            _lib.ptr(saved) if train else None, _lib.ptr(ws), nbytes, _lib.stream_of(u),
        ),
        "tsfast_hip_projscan_fwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_projscan_fwd")
    return y, x_last, saved


def _dense(*ts):
    return [t.contiguous() if t is not None else None for t in ts]


@torch.library.custom_op("tsfast_hip::projected_scan", mutates_args=())
def _scan_op(
    u: torch.Tensor, W_re: torch.Tensor, W_im: torch.Tensor, lam: torch.Tensor, C_re: torch.Tensor,
    C_im: torch.Tensor, x0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor]:
    y, x_last, _ = _forward(*_dense(u, W_re, W_im, lam, C_re, C_im, x0), train=False)
    return y, x_last


@torch.library.custom_op("tsfast_hip::projected_scan_train", mutates_args=())
def _scan_train_op(
    u: torch.Tensor, W_re: torch.Tensor, W_im: torch.Tensor, lam: torch.Tensor, C_re: torch.Tensor,
    C_im: torch.Tensor, x0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _forward(*_dense(u, W_re, W_im, lam, C_re, C_im, x0), train=True)


def _fake_outs(u, lam, C_re, train: bool):
    B, L, _ = u.shape
    N, O = lam.shape[0], C_re.shape[0]
    y = u.new_empty(B, L, O)
    x_last = u.new_empty(B, N, dtype=torch.complex64)
    if not train:
        return y, x_last
    return y, x_last, u.new_empty(saved_floats(B, L, N))


@_scan_op.register_fake
def _(u, W_re, W_im, lam, C_re, C_im, x0):
    return _fake_outs(u, lam, C_re, train=False)


@_scan_train_op.register_fake
def _(u, W_re, W_im, lam, C_re, C_im, x0):
    return _fake_outs(u, lam, C_re, train=True)


def _composition_bwd(gy, g_xlast, u, W_re, W_im, lam, C_re, C_im, x0):
    """Every gradient of the projected scan through the three-step composition
    ``complex_in_proj -> diagonal_recurrence -> real_out_proj`` (the reference's own formulation,
    ``models/_core/scan.py:221-243, 272-313``), differentiated by autograd. Used under
    ``torch.use_deterministic_algorithms(True)``: the fused backward adds its parameter gradients
    (grad W, grad lam, grad C) per workgroup over the tiles the workgroup takes from a counter,
    and which tiles those are depends on timing, while the composition's GEMMs and the diagonal
    scan's anchored look-back give the same bits on every run."""
    from ..scan import complex_in_proj, diagonal_recurrence, real_out_proj

    B, L, _ = u.shape
    if L == 0:
        zeros = [torch.zeros_like(t) for t in (u, W_re, W_im, lam, C_re, C_im)]
        g_x0 = lam.new_empty(0)
        if x0 is not None:
            g_x0 = g_xlast.clone() if g_xlast is not None else torch.zeros_like(x0)
        return (*zeros, g_x0)
    with torch.enable_grad():
        leaves = [t.detach().requires_grad_() for t in (u, W_re, W_im, lam, C_re, C_im)]
        if x0 is not None:
            leaves.append(x0.detach().requires_grad_())
        x = diagonal_recurrence(leaves[3], complex_in_proj(leaves[0], leaves[1], leaves[2]),
                                leaves[6] if x0 is not None else None)
        outs, ups = [real_out_proj(x, leaves[4], leaves[5])], [gy]
        if g_xlast is not None:
            outs.append(x[:, -1, :])
            ups.append(g_xlast)
        grads = torch.autograd.grad(outs, leaves, ups, allow_unused=True)
    grads = [torch.zeros_like(t) if g is None else g for g, t in zip(grads, leaves)]
    return (*grads[:6], grads[6] if x0 is not None else lam.new_empty(0))


@torch.library.custom_op("tsfast_hip::projected_scan_bwd", mutates_args=())
def _scan_bwd_op(
    gy: torch.Tensor, g_xlast: torch.Tensor | None, saved: torch.Tensor, u: torch.Tensor, W_re: torch.Tensor,
    W_im: torch.Tensor, lam: torch.Tensor, C_re: torch.Tensor, C_im: torch.Tensor, x0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    _lib.sync_deterministic()
    gy, g_xlast, saved, u, W_re, W_im, lam, C_re, C_im = _dense(gy, g_xlast, saved, u, W_re, W_im, lam, C_re, C_im)
    dev = u.device
    for name, t in (("gy", gy), ("saved", saved), ("u", u), ("W_re", W_re), ("W_im", W_im), ("C_re", C_re),
                    ("C_im", C_im)):
        _lib.require(t, name, (torch.float32,), dev)
    _lib.require(lam, "lam", (torch.complex64,), dev)
    _lib.require(g_xlast, "g_xlast", (torch.complex64,), dev)
    B, L, H = u.shape
    N, O = lam.shape[0], C_re.shape[0]
    g_u = torch.empty_like(u)
    g_W_re, g_W_im = torch.empty_like(W_re), torch.empty_like(W_im)
    g_C_re, g_C_im = torch.empty_like(C_re), torch.empty_like(C_im)
    g_lam = torch.empty_like(lam)
    g_x0 = torch.empty(B, N, device=dev, dtype=torch.complex64) if x0 is not None else None
    nbytes = lib.tsfast_hip_projscan_bwd_workspace_bytes(B, L, H, N, O)
    if nbytes < 0:
        raise RuntimeError(f"tsfast_hip_projscan_bwd_workspace_bytes: unsupported shape B={B} L={L} H={H} N={N} O={O}")
    ws = _lib.workspace(nbytes, dev)
    _lib.check(
        lib.tsfast_hip_projscan_bwd(
            B, L, H, N, O,
            *map(_lib.ptr, (gy, g_xlast, saved, u, W_re, W_im, lam, C_re, C_im, g_u, g_W_re, g_W_im, g_lam, g_C_re,
                            g_C_im, g_x0, ws)),
            nbytes, _lib.stream_of(u),
        ),
        "tsfast_hip_projscan_bwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_projscan_bwd")
    return g_u, g_W_re, g_W_im, g_lam, g_C_re, g_C_im, (g_x0 if g_x0 is not None else lam.new_empty(0))


@_scan_bwd_op.register_fake
def _(gy, g_xlast, saved, u, W_re, W_im, lam, C_re, C_im, x0):
    g_x0 = lam.new_empty(u.shape[0], lam.shape[0]) if x0 is not None else lam.new_empty(0)
    return (torch.empty_like(u), torch.empty_like(W_re), torch.empty_like(W_im), torch.empty_like(lam),
            torch.empty_like(C_re), torch.empty_like(C_im), g_x0)


def backward(gy, g_xlast, saved, u, W_re, W_im, lam, C_re, C_im, x0):
    """Every gradient of the projected scan: ``(g_u, g_W_re, g_W_im, g_lam, g_C_re, g_C_im,
    g_x0)`` (``g_x0`` empty when ``x0`` is None). The fused backward kernel, or under
    ``torch.use_deterministic_algorithms(True)`` the composition's autograd
    (``_composition_bwd``), whose bits do not depend on timing."""
    if torch.are_deterministic_algorithms_enabled():
        return _composition_bwd(*_dense(gy, g_xlast, u, W_re, W_im, lam, C_re, C_im, x0))
    return _scan_bwd_op(gy, g_xlast, saved, u, W_re, W_im, lam, C_re, C_im, x0)


def _scan_setup(ctx, inputs, output):
    u, W_re, W_im, lam, C_re, C_im, x0 = inputs
    ctx.save_for_backward(u, W_re, W_im, lam, C_re, C_im, x0, output[2])


def _scan_backward(ctx, gy, g_xlast, g_saved):
    u, W_re, W_im, lam, C_re, C_im, x0, saved = ctx.saved_tensors
    if gy is None:
        gy = u.new_zeros(u.shape[0], u.shape[1], C_re.shape[0])
    g_u, g_W_re, g_W_im, g_lam, g_C_re, g_C_im, g_x0 = backward(
        gy, g_xlast, saved, u, W_re, W_im, lam, C_re, C_im, x0
    )
    return g_u, g_W_re, g_W_im, g_lam, g_C_re, g_C_im, (g_x0 if x0 is not None else None)


_scan_train_op.register_autograd(_scan_backward, setup_context=_scan_setup)


def run(u, W_re, W_im, lam, C_re, C_im, x0):
    """``(y [B, L, O], x_last [B, N])`` of the projected scan; differentiable in every input.
    Without grad the inference op runs (no saved states)."""
    inputs = (u, W_re, W_im, lam, C_re, C_im) + ((x0,) if x0 is not None else ())
    if not torch.is_grad_enabled() or not any(t.requires_grad for t in inputs):
        return _scan_op(u, W_re, W_im, lam, C_re, C_im, x0)
    y, x_last, _saved = _scan_train_op(u, W_re, W_im, lam, C_re, C_im, x0)
    return y, x_last
