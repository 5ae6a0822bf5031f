"""HIP backend for the projected complex diagonal scan (the LRU / S5 layer core), float32.

It computes ``y = real_out_proj(diagonal_recurrence(lam, complex_in_proj(u, W), x0), C)`` and the
last state, the composition ``LRU.forward`` (``tsfast/models/architectures/lru.py:100-110``) and
``S5.forward`` (``s5.py:180-198``) run through ``tsfast/models/_core/scan.py:221-243, 272-313``.
Shapes: ``u [B, L, H]`` float32, ``W_re/W_im [N, H]``, ``lam [N]`` complex64, ``C_re/C_im [O, N]``,
``x0 [B, N]`` complex64 or None. Two routes:

* fused (H <= 32, N <= 256, O <= 32): one kernel per direction (``csrc/projscan.hip``: both
  projections on the fp32 matrix cores, the recurrence chained across chunks by a decoupled
  look-back); the complex ``v`` and ``x`` (``[B, L, N]`` each) never reach HBM.
* wide (any other widths): each projection is one packed real GEMM (hipBLASLt) around this
  library's diagonal scan kernels, and the backward is written out by hand so that the two weight
  gradients, products over all B L rows, run as split-K batched GEMMs (``_gram``). At these widths
  the matrix work dominates and the library GEMMs run it at a higher share of the matrix-core peak
  than the fused kernel's scan-bound pipeline.
"""

from __future__ import annotations

__all__ = ["supports", "run"]

import torch
import torch.nn.functional as F

from .. import _lib
from . import diagonal_hip

_MAX_H, _MAX_N, _MAX_O = 32, 256, 32
_SUB = 32  # steps per backward tile; the saved states entering each are [B, ceil(L / 32), N]


def supports(u, W_re, W_im, lam, C_re, C_im, x0) -> str | None:
    """Reason this backend cannot handle these tensors, or None if it can (any widths: the fused
    kernel within its limits, ``shape_reason``, the wide route beyond)."""
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
    return None


def shape_reason(B: int, L: int, H: int, N: int, O: int) -> str | None:
    """Why the fused kernel declines a shape, or None when it runs it (``ps_args_status`` in
    ``csrc/projscan.hip``): widths, and u / y / gy read through buffer resources with 32-bit byte
    offsets, chunk and row indices in int. Declined shapes take the wide route."""
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


def _deterministic_bwd(gy, g_xlast, u, W_re, W_im, lam, C_re, C_im, x0):
    """Every gradient of the projected scan through the wide route: the states recomputed by one
    GEMM and the diagonal scan kernels, then ``_wide_backward`` (GEMMs, the adjoint scan kernels and
    the fixed-order split-K weight sums). Used under ``torch.use_deterministic_algorithms(True)``:
    the fused backward adds its parameter gradients (grad W, grad lam, grad C) per workgroup over
    the tiles the workgroup takes from a counter, and which tiles those are depends on timing,
    while every step here gives the same bits on every run (the diagonal scan's look-back is
    anchored in this mode)."""
    return _wide_backward(gy, g_xlast, _wide_states(u, W_re, W_im, lam, x0), u, W_re, W_im, lam, C_re, C_im, x0)


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
    ``torch.use_deterministic_algorithms(True)`` the wide route's recompute and backward
    (``_deterministic_bwd``), whose bits do not depend on timing."""
    if torch.are_deterministic_algorithms_enabled():
        return _deterministic_bwd(*_dense(gy, g_xlast, u, W_re, W_im, lam, C_re, C_im, x0))
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


# ------------------------------------------------------------------------------ the wide route

_SPLITK_PARTS = 16  # products per split-K weight gradient ...
_SPLITK_ROWS = 4096  # ... each over at least this many rows


def _gram(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a^T b`` for ``a [K, M]``, ``b [K, N]`` with K = B L rows and small M, N: the weight
    gradients of the projections. One GEMM with K in the hundreds of thousands keeps few output
    tiles busy (24-73 TFLOP/s measured at M, N = 512..1024, 32..128); cut into 16 batched products
    over consecutive row blocks and summed in a fixed order, the same product runs at 110-134."""
    K, M = a.shape
    parts = min(_SPLITK_PARTS, K // _SPLITK_ROWS)
    if parts < 2:
        return a.t() @ b
    rows = K // parts
    main = parts * rows
    out = torch.bmm(a[:main].view(parts, rows, M).transpose(1, 2), b[:main].view(parts, rows, b.shape[1])).sum(0)
    if main < K:
        out += a[main:].t() @ b[main:]
    return out


def _w_cat(W_re, W_im):
    """The in-projection as one real weight ``[2N, H]``: rows 2s, 2s + 1 are W_re[s], W_im[s], so
    ``u @ w^T`` is the interleaved (re, im) layout of ``u W^T``."""
    N, H = W_re.shape
    return torch.stack((W_re, W_im), 1).view(2 * N, H)


def _c_cat(C_re, C_im):
    """The read-out as one real weight ``[O, 2N]``: columns 2s, 2s + 1 are C_re[:, s], -C_im[:, s],
    so ``view_as_real(x) @ c^T = Re(x C^T)``."""
    O, N = C_re.shape
    return torch.stack((C_re, -C_im), -1).view(O, 2 * N)


def _fresh(t):
    """A contiguous copy: a custom op's outputs may not alias each other (a slice that is already
    contiguous, as at B = 1 or N = 1, would come back from ``contiguous()`` as a view)."""
    return t.clone(memory_format=torch.contiguous_format)


def _wide_states(u, W_re, W_im, lam, x0):
    """The states x [B, L, N] (B L > 0): v by one GEMM, then the diagonal scan kernels."""
    B, L, _ = u.shape
    N = lam.shape[0]
    v = torch.view_as_complex(F.linear(u, _w_cat(W_re, W_im)).view(B, L, N, 2))
    return diagonal_hip.forward(lam.expand(B, N).contiguous(), v, x0)


def _wide_forward(u, W_re, W_im, lam, C_re, C_im, x0):
    """``(y, x_last, x)``: v by one GEMM, the states by the diagonal scan kernels, y by one GEMM."""
    B, L, H = u.shape
    N, O = lam.shape[0], C_re.shape[0]
    if B * L == 0:
        x_last = x0.clone() if x0 is not None else lam.new_zeros(B, N)
        return u.new_zeros(B, L, O), x_last, lam.new_empty(B, L, N)
    x = _wide_states(u, W_re, W_im, lam, x0)
    y = F.linear(torch.view_as_real(x).view(B, L, 2 * N), _c_cat(C_re, C_im))
    return y, _fresh(x[:, -1]), x


def _wide_backward(gy, g_xlast, x, u, W_re, W_im, lam, C_re, C_im, x0):
    """Every gradient of the wide route, written out: g_x = gy C (one GEMM, plus the returned
    state's gradient at the last step), the adjoint scan kernels (grad v, grad lam per row, grad
    x0), g_u = grad v W (one GEMM), and the weight gradients by ``_gram``."""
    B, L, H = u.shape
    N, O = lam.shape[0], C_re.shape[0]
    g_x0 = lam.new_empty(0)
    if B * L == 0:
        if x0 is not None:
            g_x0 = g_xlast.clone() if g_xlast is not None else torch.zeros_like(x0)
        zeros = [torch.zeros_like(t) for t in (u, W_re, W_im, lam, C_re, C_im)]
        return (*zeros, g_x0)
    w, c = _w_cat(W_re, W_im), _c_cat(C_re, C_im)
    g_x = torch.view_as_complex((gy.view(B * L, O) @ c).view(B, L, N, 2))
    if g_xlast is not None:
        g_x[:, -1] += g_xlast
    g_lam_rows, g_v, g_x0 = diagonal_hip.backward(g_x, lam.expand(B, N).contiguous(), x, x0)
    del g_x
    g_vr = torch.view_as_real(g_v).view(B * L, 2 * N)
    g_u = (g_vr @ w).view(B, L, H)
    g_w = _gram(g_vr, u.view(B * L, H))
    g_c = _gram(gy.view(B * L, O), torch.view_as_real(x).view(B * L, 2 * N))
    return (g_u, _fresh(g_w[0::2]), _fresh(g_w[1::2]), g_lam_rows.sum(0), _fresh(g_c[:, 0::2]), -g_c[:, 1::2],
            g_x0 if x0 is not None else lam.new_empty(0))


@torch.library.custom_op("tsfast_hip::projected_scan_wide", mutates_args=())
def _wide_op(
    u: torch.Tensor, W_re: torch.Tensor, W_im: torch.Tensor, lam: torch.Tensor, C_re: torch.Tensor,
    C_im: torch.Tensor, x0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor]:
    y, x_last, _ = _wide_forward(*_dense(u, W_re, W_im, lam, C_re, C_im, x0))
    return y, x_last


@torch.library.custom_op("tsfast_hip::projected_scan_wide_train", mutates_args=())
def _wide_train_op(
    u: torch.Tensor, W_re: torch.Tensor, W_im: torch.Tensor, lam: torch.Tensor, C_re: torch.Tensor,
    C_im: torch.Tensor, x0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _wide_forward(*_dense(u, W_re, W_im, lam, C_re, C_im, x0))


@torch.library.custom_op("tsfast_hip::projected_scan_wide_bwd", mutates_args=())
def _wide_bwd_op(
    gy: torch.Tensor, g_xlast: torch.Tensor | None, x: torch.Tensor, u: torch.Tensor, W_re: torch.Tensor,
    W_im: torch.Tensor, lam: torch.Tensor, C_re: torch.Tensor, C_im: torch.Tensor, x0: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    return _wide_backward(*_dense(gy, g_xlast, x, u, W_re, W_im, lam, C_re, C_im, x0))


@_wide_op.register_fake
def _(u, W_re, W_im, lam, C_re, C_im, x0):
    return _fake_outs(u, lam, C_re, train=False)


@_wide_train_op.register_fake
def _(u, W_re, W_im, lam, C_re, C_im, x0):
    B, L, _ = u.shape
    y, x_last = _fake_outs(u, lam, C_re, train=False)
    return y, x_last, lam.new_empty(B, L, lam.shape[0])


@_wide_bwd_op.register_fake
def _(gy, g_xlast, x, u, W_re, W_im, lam, C_re, C_im, x0):
    g_x0 = lam.new_empty(u.shape[0], lam.shape[0]) if x0 is not None else lam.new_empty(0)
    return (torch.empty_like(u), torch.empty_like(W_re), torch.empty_like(W_im), torch.empty_like(lam),
            torch.empty_like(C_re), torch.empty_like(C_im), g_x0)


def _wide_setup(ctx, inputs, output):
    u, W_re, W_im, lam, C_re, C_im, x0 = inputs
    ctx.save_for_backward(u, W_re, W_im, lam, C_re, C_im, x0, output[2])


def _wide_backward_rule(ctx, gy, g_xlast, g_x):
    # g_x is autograd's zero fill for the states output, which run() keeps for the backward only
    u, W_re, W_im, lam, C_re, C_im, x0, x = ctx.saved_tensors
    if gy is None:
        gy = u.new_zeros(u.shape[0], u.shape[1], C_re.shape[0])
    g_u, g_W_re, g_W_im, g_lam, g_C_re, g_C_im, g_x0 = _wide_bwd_op(gy, g_xlast, x, u, W_re, W_im, lam, C_re, C_im, x0)
    return g_u, g_W_re, g_W_im, g_lam, g_C_re, g_C_im, (g_x0 if x0 is not None else None)


_wide_train_op.register_autograd(_wide_backward_rule, setup_context=_wide_setup)


def is_fused(u, lam, C_re) -> bool:
    """Whether these widths run on the fused kernel (else the wide route)."""
    B, L, H = u.shape
    return shape_reason(B, L, H, lam.shape[0], C_re.shape[0]) is None


def run(u, W_re, W_im, lam, C_re, C_im, x0):
    """``(y [B, L, O], x_last [B, N])`` of the projected scan; differentiable in every input.
    The fused kernel where its widths allow, else the wide route. Without grad the inference ops
    run (no saved states)."""
    inputs = (u, W_re, W_im, lam, C_re, C_im) + ((x0,) if x0 is not None else ())
    fused = is_fused(u, lam, C_re)
    if not torch.is_grad_enabled() or not any(t.requires_grad for t in inputs):
        return (_scan_op if fused else _wide_op)(u, W_re, W_im, lam, C_re, C_im, x0)
    y, x_last, _saved = (_scan_train_op if fused else _wide_train_op)(u, W_re, W_im, lam, C_re, C_im, x0)
    return y, x_last
