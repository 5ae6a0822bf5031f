"""HIP backend for the time-varying (selective) diagonal scan, float32.

Drop-in for the ``selective`` family of ``tsfast/models/_core/scan.py:32-42`` (the role of
``scan_backends/selective_triton.py:112-160``). Lane layout: lam and v ``[M, L, N]``, x0
``[M, N]``. Kernels in ``csrc/diag.hip``: single-pass look-back scans whose chunk summaries are
(coefficient product, state) affine maps.
"""

from __future__ import annotations

__all__ = ["supports", "forward", "backward"]

import torch

from .. import _lib


def supports(lam: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> str | None:
    """Reason this backend cannot handle the inputs, or None when it can."""
    if v.device.type != "cuda":
        return f"input on {v.device.type}, hip backend is GPU-only"
    if any(t is not None and t.dtype != torch.float32 for t in (lam, v, x0)):
        return "needs float32 tensors"
    if v.dim() != 3 or lam.shape != v.shape:
        return f"expects lam and v of one lane layout [M, L, N], got {tuple(lam.shape)} / {tuple(v.shape)}"
    if x0 is not None and tuple(x0.shape) != (v.shape[0], v.shape[2]):
        return f"x0 {tuple(x0.shape)} does not match v {tuple(v.shape)}"
    if any(t.device != v.device for t in (lam, x0) if t is not None):
        return "inputs on different devices"
    if not all(t.is_contiguous() for t in (lam, v, x0) if t is not None):
        return "inputs must be contiguous"
    return None


def forward(lam: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None) -> torch.Tensor:
    lib = _lib.load()
    _lib.sync_deterministic()
    M, L, N = v.shape
    for name, t in (("lam", lam), ("v", v), ("x0", x0)):
        _lib.require(t, name, (torch.float32,), v.device)
    out = torch.empty_like(v)
    nbytes = lib.tsfast_hip_sel_workspace_bytes(M, L, N)
    ws = _lib.workspace(nbytes, v.device)
    _lib.check(
        lib.tsfast_hip_sel_fwd(
            M, L, N, _lib.ptr(lam), _lib.ptr(v), _lib.ptr(x0), _lib.ptr(out), _lib.ptr(ws), nbytes, _lib.stream_of(v)
        ),
        "tsfast_hip_sel_fwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_sel_fwd")
    return out


def backward(
    g: torch.Tensor, lam: torch.Tensor, out: torch.Tensor, x0: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    _lib.sync_deterministic()
    M, L, N = out.shape
    for name, t in (("g", g), ("lam", lam), ("out", out), ("x0", x0)):
        _lib.require(t, name, (torch.float32,), out.device)
    gv = torch.empty_like(out)
    glam = torch.empty_like(out)
    gx0 = torch.empty_like(x0) if x0 is not None else None
    nbytes = lib.tsfast_hip_sel_workspace_bytes(M, L, N)
    ws = _lib.workspace(nbytes, out.device)
    _lib.check(
        lib.tsfast_hip_sel_bwd(
            M, L, N, _lib.ptr(g), _lib.ptr(lam), _lib.ptr(out), _lib.ptr(x0), _lib.ptr(glam), _lib.ptr(gv),
            _lib.ptr(gx0), _lib.ptr(ws), nbytes, _lib.stream_of(out),
        ),
        "tsfast_hip_sel_bwd",
    )
    _lib.check_lookback(ws, "tsfast_hip_sel_bwd")
    return glam, gv, (gx0 if gx0 is not None else lam.new_empty(0))
