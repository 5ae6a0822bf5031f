"""Torch fallback for the linear recurrences: a blocked two-level scan.

The HIP kernels serve every GPU call these modules dispatch; this module is what runs when no
backend serves the inputs (CPU tensors, an explicit ``"reference"`` preference, or shapes a
kernel declines). It is this package's own formulation, not the reference's doubling scan
(``tsfast/models/_core/scan.py:52-80``, ``dynonet/core.py:23-37``): the sequence is cut into
``nb`` blocks of ``T`` steps (``T`` about ``sqrt(L)``, so the two Python loops below run
``T + nb`` iterations), and

1. every block is swept from a zero state, vectorised over all blocks at once, keeping the
   running product of the coefficients (the map ``x -> P_i x`` that the block applies to the
   state entering it, up to step ``i``);
2. the block carries are chained in a short sequential sweep over the blocks;
3. each block adds ``P_i`` applied to the state entering it.

Work is ``O(L)`` elementwise (``O(L n^3 / T + L n^2)`` for matrix coefficients) instead of the
doubling scan's ``O(L log L)``, and at most three ``[..., L, n]`` temporaries are alive.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = ["block_len", "scan_diagonal", "scan_matrix", "sequential"]


def block_len(L: int) -> int:
    """Block length: the power of two nearest ``sqrt(L)`` (at least 8)."""
    return max(8, 1 << max(0, round(math.log2(max(L, 1)) / 2)))


def _blocks(x: torch.Tensor, T: int, fill: float) -> torch.Tensor:
    """``[..., L, n] -> [..., nb, T, n]``, padding the time axis with ``fill``."""
    L = x.shape[-2]
    nb = -(-L // T)
    if nb * T != L:
        x = F.pad(x, (0, 0, 0, nb * T - L), value=fill)
    return x.reshape(*x.shape[:-2], nb, T, x.shape[-1])


def scan_diagonal(coef: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None = None) -> torch.Tensor:
    """``x_t = coef_t * x_{t-1} + v_t`` elementwise along ``[..., L, n]``.

    ``coef`` is ``[..., L, n]`` (time-varying) or ``[..., n]`` (constant); ``x0`` is
    ``[..., n]`` or None (zero). Returns the states ``x_1 .. x_L`` shaped like ``v``.
    """
    L = v.shape[-2]
    if L == 0:
        return v.clone()
    T = block_len(L)
    const = coef.dim() == v.dim() - 1
    vb = _blocks(v, T, 0.0)
    lead = vb.shape[:-2]  # [..., nb]
    n = v.shape[-1]
    dtype = torch.promote_types(v.dtype, coef.dtype)
    # a constant coefficient broadcasts over blocks and steps; a time-varying one is padded with
    # identity steps (coefficient 1, input 0)
    cb = coef.unsqueeze(-2).to(dtype) if const else _blocks(coef, T, 1.0).to(dtype)
    xs = torch.empty(lead + (T, n), dtype=dtype, device=v.device)
    prods = torch.empty_like(xs)
    acc = torch.zeros(lead + (n,), dtype=dtype, device=v.device)
    run = torch.ones(lead + (n,), dtype=dtype, device=v.device)
    for i in range(T):  # 1. every block from a zero state
        c = cb if const else cb[..., i, :]
        acc = c * acc + vb[..., i, :]
        xs[..., i, :] = acc
        run = run * c
        prods[..., i, :] = run
    nb = lead[-1]
    state = torch.zeros(lead[:-1] + (n,), dtype=dtype, device=v.device) if x0 is None else x0.to(dtype)
    entering = torch.empty(lead + (n,), dtype=dtype, device=v.device)
    for k in range(nb):  # 2. chain the carries
        entering[..., k, :] = state
        state = prods[..., k, T - 1, :] * state + xs[..., k, T - 1, :]
    xs += prods * entering.unsqueeze(-2)  # 3. fix-up
    return xs.reshape(*lead[:-1], nb * T, n)[..., :L, :]


def scan_matrix(A: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None = None) -> torch.Tensor:
    """``x_t = A x_{t-1} + v_t`` with a constant matrix ``A [..., n, n]`` along ``v [..., L, n]``.

    Same three phases as :func:`scan_diagonal` with ``A``'s powers ``A^(i+1)`` (``i < T``) as
    the block maps. Returns the states shaped like ``v``.
    """
    L, n = v.shape[-2], v.shape[-1]
    if L == 0:
        return v.clone()
    T = block_len(L)
    vb = _blocks(v, T, 0.0)  # [..., nb, T, n]
    lead = vb.shape[:-2]
    At = A.transpose(-1, -2).unsqueeze(-3)  # row-vector form: x @ A^T, broadcast over blocks
    xs = torch.empty(lead + (T, n), dtype=v.dtype, device=v.device)
    acc = torch.zeros(lead + (n,), dtype=v.dtype, device=v.device)
    for i in range(T):  # 1. every block from a zero state
        acc = (acc.unsqueeze(-2) @ At).squeeze(-2) + vb[..., i, :]
        xs[..., i, :] = acc
    # powers (A^T)^(i+1), i < T, as [..., T, n, n]
    pows = [A.transpose(-1, -2)]
    for _ in range(T - 1):
        pows.append(pows[-1] @ A.transpose(-1, -2))
    Pt = torch.stack(pows, dim=-3)
    nb = lead[-1]
    state = torch.zeros(lead[:-1] + (n,), dtype=v.dtype, device=v.device) if x0 is None else x0.to(v.dtype)
    entering = torch.empty(lead + (n,), dtype=v.dtype, device=v.device)
    Pend = Pt[..., T - 1, :, :]
    for k in range(nb):  # 2. chain the carries
        entering[..., k, :] = state
        state = (state.unsqueeze(-2) @ Pend).squeeze(-2) + xs[..., k, T - 1, :]
    # 3. fix-up: x[k, i] += entering_k @ (A^T)^(i+1)
    xs += (entering.unsqueeze(-2).unsqueeze(-2) @ Pt.unsqueeze(-4)).squeeze(-2)
    return xs.reshape(*lead[:-1], nb * T, n)[..., :L, :]


def sequential(coef: torch.Tensor, v: torch.Tensor, x0: torch.Tensor | None = None) -> torch.Tensor:
    """The same diagonal recurrence as :func:`scan_diagonal`, one step at a time (the eager path)."""
    const = coef.dim() == v.dim() - 1
    out = torch.empty_like(v, dtype=torch.promote_types(v.dtype, coef.dtype))
    x = torch.zeros_like(out[..., 0, :]) if x0 is None else x0.to(out.dtype)
    for t in range(v.shape[-2]):
        x = (coef if const else coef[..., t, :]) * x + v[..., t, :]
        out[..., t, :] = x
    return out
