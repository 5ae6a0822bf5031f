"""HIP backend for the constant-coefficient diagonal scan (LRU/S5 core), float32 and complex64.

Drop-in for the ``diagonal`` family of ``tsfast/models/_core/scan.py:32-42`` (the role of
``scan_backends/diagonal_triton.py:236-305``). Lane layout: lam ``[M, N]``, v ``[M, L, N]``,
x0 ``[M, N]``, contiguous, on the GPU. The kernels (``csrc/diag.hip``) are single-pass scans with
a decoupled look-back between workgroups: each tile of lanes x steps publishes its summary, takes
its start state from the tiles before it and re-scans its chunk from registers.
"""

from __future__ import annotations

__all__ = ["supports", "forward", "backward"]

import torch

from .. import _lib

_DTYPES = (torch.float32, torch.complex64)


def supports(lam: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> str | None:
    """Reason this backend cannot handle the inputs, or None when it can."""
    if v.device.type != "cuda":
        return f"input on {v.device.type}, hip backend is GPU-only"
    if v.dtype not in _DTYPES:
        return f"dtype {v.dtype} unsupported (need float32 or complex64)"
    if lam.dtype != v.dtype:
        return f"lam dtype {lam.dtype} != v dtype {v.dtype}"
    if x0 is not None and x0.dtype != v.dtype:
        return f"x0 dtype {x0.dtype} != v dtype {v.dtype}"
    if v.dim() != 3 or lam.dim() != 2:
        return "expects the lane layout lam [M, N], v [M, L, N]"
    if tuple(lam.shape) != (v.shape[0], v.shape[2]):
        return f"lam {tuple(lam.shape)} does not match v {tuple(v.shape)}"
    if x0 is not None and tuple(x0.shape) != tuple(lam.shape):
        return f"x0 {tuple(x0.shape)} does not match lam {tuple(lam.shape)}"
    if any(t.device != v.device for t in (lam, x0) if t is not None):
        return "inputs on different devices"
    if not all(t.is_contiguous() for t in (lam, v, x0) if t is not None):
        return "inputs must be contiguous"
    return None


def forward(lam: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> torch.Tensor:
    """Forward recurrence on the lane layout; returns the states ``[M, L, N]``."""
    lib = _lib.load()
    _lib.sync_deterministic()
    M, L, N = v.shape
    for name, t in (("lam", lam), ("v", v), ("x0", x0)):
        _lib.require(t, name, (v.dtype,), v.device)
    cplx = int(v.is_complex())
    out = torch.empty_like(v)
    nbytes = lib.tsfast_hip_diag_workspace_bytes(M, L, N, cplx)
    ws = _lib.workspace(nbytes, v.device)
    _lib.check(
        lib.tsfast_hip_diag_fwd(
            M, L, N, cplx, _lib.ptr(lam), _lib.ptr(v), _lib.ptr(x0), _lib.ptr(out), _lib.ptr(ws), nbytes,
            _lib.stream_of(v),
        ),
        "tsfast_hip_diag_fwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_diag_fwd")
    return out


def backward(
    g: torch.Tensor, lam: torch.Tensor, out: torch.Tensor, x0: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Adjoint sweep, returning ``(glam, gv, gx0)`` (gx0 empty when x0 is None)."""
    lib = _lib.load()
    _lib.sync_deterministic()
    M, L, N = out.shape
    for name, t in (("g", g), ("lam", lam), ("out", out), ("x0", x0)):
        _lib.require(t, name, (out.dtype,), out.device)
    cplx = int(out.is_complex())
    gv = torch.empty_like(out)
    glam = torch.empty_like(lam)
    gx0 = torch.empty_like(lam) if x0 is not None else None
    nbytes = lib.tsfast_hip_diag_workspace_bytes(M, L, N, cplx)
    ws = _lib.workspace(nbytes, out.device)
    _lib.check(
        lib.tsfast_hip_diag_bwd(
            M, L, N, cplx, _lib.ptr(g), _lib.ptr(lam), _lib.ptr(out), _lib.ptr(x0), _lib.ptr(gv), _lib.ptr(glam),
            _lib.ptr(gx0), _lib.ptr(ws), nbytes, _lib.stream_of(out),
        ),
        "tsfast_hip_diag_bwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_diag_bwd")
    return glam, gv, (gx0 if gx0 is not None else lam.new_empty(0))
