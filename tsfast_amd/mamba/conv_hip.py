"""Fused causal depthwise convolution + SiLU, HIP backend for the Mamba conv section.

Computes ``silu(conv1d(cat(tail, x), weight, bias))`` along time per channel, channel-last:
``x [B, L, D]`` (any strides: the kernel reads the strided ``in_proj`` chunk view directly),
``tail [B, D, K-1]`` the carried causal left context, ``weight [D, 1, K]``, ``bias [D]`` or None.
Drop-in for the ``mamba.conv`` registry of ``tsfast/models/architectures/mamba/core.py:22``
(the role of ``conv_triton.py``): ``supports(x, tail, weight, bias)`` and
``run(x, tail, weight, bias) -> out [B, L, D]`` (contiguous), differentiable in all inputs
through the ``tsfast_hip::mamba_conv_silu`` / ``mamba_conv_silu_bwd`` custom ops.

Sequence tensors (x, tail, out and their gradients) are float32 or bfloat16; the kernels run
the taps and the SiLU in float32, with float32 weights and bias (a bfloat16 weight or bias is
upcast before the op, so autograd casts its gradient back). ``2 <= K <= 8``.
"""

from __future__ import annotations

__all__ = ["supports", "run"]

import torch

from .. import _lib

_IO_DTYPES = {torch.float32: _lib.TSF_DTYPE_F32, torch.bfloat16: _lib.TSF_DTYPE_BF16}
_PARAM_DTYPES = (torch.float32, torch.bfloat16)
_SEG = 128  # steps per workgroup segment (conv.hip kSeg); tests pin it against the library's size query


def supports(x, tail, weight, bias) -> str | None:
    """Reason the fused conv kernel cannot handle these tensors, or None if it can."""
    if x.device.type != "cuda":
        return f"x on {x.device.type}, hip backend is GPU-only"
    if x.dtype not in _IO_DTYPES:
        return f"x dtype {x.dtype} not float32/bfloat16"
    tensors = {"tail": tail, "weight": weight}
    if bias is not None:
        tensors["bias"] = bias
    for name, t in tensors.items():
        if t.device != x.device:
            return f"{name} on {t.device}, x on {x.device}"
    if tail.dtype != x.dtype:
        return f"tail dtype {tail.dtype} != x dtype {x.dtype}"
    if weight.dtype not in _PARAM_DTYPES or (bias is not None and bias.dtype not in _PARAM_DTYPES):
        return "weight/bias must be float32 or bfloat16"
    if x.dim() != 3:
        return f"x must be [B, L, D], got {x.dim()} dims"
    B, L, D = x.shape
    if weight.dim() != 3 or weight.shape[0] != D or weight.shape[1] != 1:
        return f"weight.shape {tuple(weight.shape)} is not depthwise [D, 1, K] for D={D}"
    K = weight.shape[-1]
    if not 2 <= K <= 8:
        return f"kernel width {K} outside the supported range [2, 8]"
    if tuple(tail.shape) != (B, D, K - 1):
        return f"tail.shape {tuple(tail.shape)} != {(B, D, K - 1)}"
    if bias is not None and tuple(bias.shape) != (D,):
        return f"bias.shape {tuple(bias.shape)} != {(D,)}"
    return _size_reason(B, L, D, x.stride(1), x.stride(2), x.element_size())


def _size_reason(B: int, L: int, D: int, sxl: int, sxd: int, esz: int) -> str | None:
    """The kernels' grid limit (conv.hip conv_args_status: a one-dimensional grid of at most
    2^24 - 1 workgroups, the most of which the one-channel register-tile forward launches) and
    32-bit per-row addressing (conv_layout_status), repeated here so that supports() makes no
    library call."""
    per_row = -(-D // 64) * -(-(-(-L // 16)) // 4)
    if per_row > 0 and B > ((1 << 24) - 1) // per_row:
        return f"B={B}, L={L}, D={D} needs more than 2^24 - 1 workgroups"
    if ((L + 8) * sxl + (D + 8) * sxd) * esz >= 1 << 32 or (L + 8) * D * esz >= 1 << 32:
        return f"one batch row (L={L}, D={D}, strides {sxl}, {sxd}) exceeds the kernels' 32-bit row addressing"
    return None


def _screen(x, tail, weight, bias):
    dev = x.device
    if x.dtype not in _IO_DTYPES:
        raise TypeError(f"x: dtype {x.dtype} not float32/bfloat16")
    if x.device.type != "cuda":
        raise TypeError(f"x: on {x.device}, expected a GPU tensor")
    _lib.require(tail, "tail", (x.dtype,), dev)
    _lib.require(weight, "weight", (torch.float32,), dev)
    _lib.require(bias, "bias", (torch.float32,), dev)


@torch.library.custom_op("tsfast_hip::mamba_conv_silu", mutates_args=())
def _conv_silu_op(x: torch.Tensor, tail: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    lib = _lib.load()
    tail, weight = tail.contiguous(), weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    _screen(x, tail, weight, bias)
    B, L, D = x.shape
    K = weight.shape[-1]
    out = torch.empty(B, L, D, device=x.device, dtype=x.dtype)
    _lib.check(
        lib.tsfast_hip_conv_silu_fwd(
            B, L, D, K, _IO_DTYPES[x.dtype], _lib.ptr(x), *x.stride(), _lib.ptr(tail), _lib.ptr(weight),
            _lib.ptr(bias), _lib.ptr(out), _lib.stream_of(x),
        ),
        "tsfast_hip_conv_silu_fwd",
    )
    return out


@_conv_silu_op.register_fake
def _(x, tail, weight, bias):
    return torch.empty(x.shape, device=x.device, dtype=x.dtype)


@torch.library.custom_op("tsfast_hip::mamba_conv_silu_bwd", mutates_args=())
def _conv_silu_bwd_op(
    gy: torch.Tensor, x: torch.Tensor, tail: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    gy, tail, weight = gy.contiguous(), tail.contiguous(), weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    _screen(x, tail, weight, bias)
    _lib.require(gy, "gy", (x.dtype,), x.device)
    B, L, D = x.shape
    K = weight.shape[-1]
    gx = torch.empty(B, L, D, device=x.device, dtype=x.dtype)
    g_tail = torch.empty_like(tail)
    gw = torch.empty(D, K, device=x.device, dtype=torch.float32)
    gb = torch.empty(D, device=x.device, dtype=torch.float32) if bias is not None else None
    nbytes = lib.tsfast_hip_conv_silu_workspace_bytes(B, L, D, K)
    ws = _lib.workspace(nbytes, x.device)
    if L == 0:
        g_tail.zero_()  # an empty sequence passes no gradient to the carried context
    _lib.check(
        lib.tsfast_hip_conv_silu_bwd(
            B, L, D, K, _IO_DTYPES[x.dtype], _lib.ptr(x), *x.stride(), _lib.ptr(tail), _lib.ptr(weight),
            _lib.ptr(bias), _lib.ptr(gy), _lib.ptr(gx), _lib.ptr(g_tail), _lib.ptr(gw), _lib.ptr(gb),
            _lib.ptr(ws), nbytes, _lib.stream_of(x),
        ),
        "tsfast_hip_conv_silu_bwd",
    )
    return gx, g_tail, gw, (gb if gb is not None else gx.new_empty(0))


@_conv_silu_bwd_op.register_fake
def _(gy, x, tail, weight, bias):
    gb = torch.empty_like(bias) if bias is not None else gy.new_empty(0)
    return torch.empty(x.shape, device=x.device, dtype=x.dtype), torch.empty_like(tail), torch.empty_like(weight), gb


def _conv_setup(ctx, inputs, output):
    x, tail, weight, bias = inputs
    ctx.save_for_backward(x, tail, weight, bias)


def _conv_backward(ctx, gy):
    x, tail, weight, bias = ctx.saved_tensors
    gx, g_tail, gw, gb = _conv_silu_bwd_op(gy, x, tail, weight, bias)
    return gx, g_tail, gw, (gb if bias is not None else None)


_conv_silu_op.register_autograd(_conv_backward, setup_context=_conv_setup)


def run(x, tail, weight, bias):
    """Fused causal depthwise conv + SiLU: ``silu(conv1d(cat(tail, x), weight, bias))``.

    ``x`` is channel-last ``[B, L, D]`` (any strides); ``tail`` is the carried causal left
    context ``[B, D, K-1]``. Returns the activated signal ``[B, L, D]``, contiguous;
    differentiable in all inputs (via the ``tsfast_hip::mamba_conv_silu`` op).
    """
    w = weight.squeeze(1).float()
    b = bias.float() if bias is not None else None
    return _conv_silu_op(x, tail.contiguous(), w.contiguous(), b)
