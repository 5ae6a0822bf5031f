"""HIP backend for the chunked adjoint scan of a NeuralStateSpace backward, float32.

The sequence-parallel part of ``tsfast/models/architectures/ssm/backend_metal.py:446-479``
(``backward``): with the per-step transposed state Jacobians ``jt [B, L, n, n]`` (``_build_jt``,
``:377-394``) and the upstream gradients ``gout [B, L, n]``, the adjoint
``gy_t = gout_t + jt[t+1] gy_{t+1}`` (``gy_{L-1} = gout_{L-1}``) is summarised per chunk of ``cl``
steps and composed from the right into ``bnd [B, C + 1, n]``: ``bnd[:, c]`` is ``gy`` at the first
step of chunk ``c`` and ``bnd[:, C]`` is zero. ``run(jt, gout, cl)`` replaces the reference's two
kernels ``ssm_bwd_summary`` + ``ssm_bwd_scan`` (``:285-357``), with the same chunking (``C =
ceil(L / cl)``) and output, and ``supports`` its shape contract (``n <= 32``, the reference's
``_SCAN_MAX_STATE``). Kernels: ``csrc/masscan.hip``.
"""

from __future__ import annotations

__all__ = ["supports", "run"]

import torch

from .. import _lib

_MAX_N = 32


def supports(jt: torch.Tensor, gout: torch.Tensor, cl: int) -> str | None:
    """Reason this backend cannot handle the inputs, or None when it can."""
    if gout.device.type != "cuda":
        return f"input on {gout.device.type}, hip backend is GPU-only"
    if jt.dtype != torch.float32 or gout.dtype != torch.float32:
        return "needs float32 jt and gout"
    if jt.device != gout.device:
        return "inputs on different devices"
    if gout.dim() != 3 or jt.dim() != 4:
        return "expected jt [B, L, n, n] and gout [B, L, n]"
    B, L, n = gout.shape
    if tuple(jt.shape) != (B, L, n, n):
        return f"jt.shape {tuple(jt.shape)} != {(B, L, n, n)}"
    if not 1 <= n <= _MAX_N:
        return f"state size n={n} outside the supported range [1, {_MAX_N}]"
    if int(cl) < 1:
        return f"chunk length {cl} < 1"
    return None


def run(jt: torch.Tensor, gout: torch.Tensor, cl: int) -> torch.Tensor:
    """``bnd [B, C + 1, n]``: the adjoint entering each chunk of ``cl`` steps (zero past the end)."""
    lib = _lib.load()
    B, L, n = gout.shape
    cl = int(cl)
    C = -(-L // cl)
    jt, gout = jt.contiguous(), gout.contiguous()
    bnd = torch.empty(B, C + 1, n, device=gout.device, dtype=torch.float32)
    nbytes = lib.tsfast_hip_mat_adjoint_workspace_bytes(B, L, n, cl)
    if nbytes < 0:
        raise RuntimeError("tsfast_hip_mat_adjoint_workspace_bytes: unsupported shape")
    ws = _lib.workspace(nbytes, gout.device)
    _lib.check(
        lib.tsfast_hip_mat_adjoint_bounds(B, L, n, cl, _lib.ptr(jt), _lib.ptr(gout), _lib.ptr(bnd), _lib.ptr(ws), nbytes,
                                          _lib.stream_of(gout)),
        "tsfast_hip_mat_adjoint_bounds",
    )
    return bnd
