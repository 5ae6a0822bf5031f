"""GPU parity: fused causal depthwise conv + SiLU (HIP) vs the fp64 oracle.

Shapes follow the reference's Mamba suites (tests/test_mamba.py: d_inner 8..32, L = 1, L shorter
than the conv tail, lengths not multiples of anything, d_conv 4) plus kernel widths 2..8,
channel counts off the 4-channel vector width, the strided in_proj chunk view the reference
passes in, and a reduced config-3 shape. Inputs are seeded; the oracle runs in fp64 on exactly
the values the kernel sees. Bar: max relative error <= 1e-5 (fp32 I/O) and <= 2e-2 (bf16 I/O).
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import dispatch
from tsfast_amd.mamba import conv_hip
from tsfast_amd.mamba import core as mcore

pytestmark = pytest.mark.gpu


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def _make(Bsz, L, D, K, seed, dtype, with_bias=True, strided=True):
    g = torch.Generator().manual_seed(seed)
    # x as the in_proj chunk view: the first D of 2D features, row stride 2D
    xz = torch.randn(Bsz, L, 2 * D, generator=g)
    x = xz[..., :D] if strided else xz[..., :D].contiguous()
    tail = torch.randn(Bsz, D, K - 1, generator=g)
    weight = torch.randn(D, 1, K, generator=g) * 0.5
    bias = torch.randn(D, generator=g) if with_bias else None
    gy = torch.randn(Bsz, L, D, generator=g)
    return xz, x, tail, weight, bias, gy


# (B, L, D, K, bias, strided)
_SHAPES = [
    (4, 50, 32, 4, True, True),
    (3, 40, 8, 4, True, True),
    (2, 33, 20, 4, True, True),  # D = 20: vector path (20 % 4 == 0)
    (2, 33, 10, 4, True, True),  # D = 10: scalar path
    (1, 2, 8, 4, True, True),  # L shorter than the tail
    (1, 1, 8, 2, False, True),
    (2, 64, 64, 8, True, False),
    (3, 17, 12, 3, False, False),
    (2, 100, 24, 5, True, True),
    (2, 150, 40, 6, True, True),  # K = 6: 18-row tiles
    (1, 300, 16, 7, False, True),  # K = 7: 21-row tiles, several segments
    (3, 700, 264, 4, True, True),  # two channel blocks, the second nearly empty
    (2, 1024, 1536, 4, True, True),  # config-3 channel count, reduced batch and length
    (70000, 3, 8, 4, True, True),  # more batch rows than a grid dimension's 65535 (1-D grid)
    (70000, 3, 12, 3, True, False),  # the same on the scalar (one channel per thread) path
]


def _run(xz, x, tail, weight, bias, gy, dev, dtype):
    xz_d = xz.to(dev, dtype).requires_grad_()
    x_d = xz_d[..., : x.shape[-1]]
    if x.is_contiguous():
        x_d = x_d.contiguous()
    tail_d = tail.to(dev, dtype).requires_grad_()
    w_d = weight.to(dev).requires_grad_()
    b_d = bias.to(dev).requires_grad_() if bias is not None else None
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("mamba.conv", mcore._CONV_BACKENDS, ("hip",), (x_d, tail_d, w_d, b_d)) is conv_hip
        out = mcore.mamba_conv(x_d, tail_d, w_d, b_d)
    out.backward(gy.to(dev, dtype))
    gx = xz_d.grad[..., : x.shape[-1]]
    return out, gx, tail_d.grad, w_d.grad, (b_d.grad if b_d is not None else None), x_d, tail_d


@pytest.mark.parametrize("io", ["fp32", "bf16"])
@pytest.mark.parametrize("shape", _SHAPES)
def test_conv_silu_matches_oracle(gpu, shape, io):
    Bsz, L, D, K, with_bias, strided = shape
    dtype = torch.float32 if io == "fp32" else torch.bfloat16
    tol = 1e-5 if io == "fp32" else 2e-2
    xz, x, tail, weight, bias, gy = _make(Bsz, L, D, K, seed=sum(shape[:4]), dtype=dtype, with_bias=with_bias,
                                          strided=strided)
    out, gx, gtail, gw, gb, x_d, tail_d = _run(xz, x, tail, weight, bias, gy, gpu, dtype)
    # the oracle sees exactly the (rounded) values the kernel saw
    xs, ts, gys = _np(x_d), _np(tail_d), _np(gy.to(dtype))
    ws = _np(weight[:, 0])
    bs = _np(bias)
    assert out.is_contiguous() and out.dtype == dtype and out.shape == (Bsz, L, D)
    assert O.rel_err(_np(out), O.conv_silu_forward(xs, ts, ws, bs)) < tol
    w_gx, w_gt, w_gw, w_gb = O.conv_silu_backward(gys, xs, ts, ws, bs)
    assert O.rel_err(_np(gx), w_gx) < tol, "gx"
    assert O.rel_err(_np(gtail), w_gt) < tol, "gtail"
    assert O.rel_err(_np(gw[:, 0]), w_gw) < tol, "gw"
    if bias is not None:
        assert O.rel_err(_np(gb), w_gb) < tol, "gb"


def test_conv_chunked_equals_full(gpu):
    """TBPTT: the last K-1 steps of each chunk carried as the next chunk's tail give the full pass."""
    g = torch.Generator().manual_seed(3)
    Bsz, L, D, K = 3, 70, 16, 4
    x = torch.randn(Bsz, L, D, generator=g).to(gpu)
    w = (torch.randn(D, 1, K, generator=g) * 0.5).to(gpu)
    b = torch.randn(D, generator=g).to(gpu)
    tail = torch.zeros(Bsz, D, K - 1, device=gpu)
    with torch.no_grad():
        full = conv_hip.run(x, tail, w, b)
        outs, t = [], tail
        for lo, hi in ((0, 17), (17, 19), (19, 70)):
            xc = x[:, lo:hi]
            outs.append(conv_hip.run(xc, t, w, b))
            t = torch.cat((t, xc.mT), dim=-1)[..., -(K - 1):].contiguous()
    assert O.rel_err(_np(torch.cat(outs, 1)), _np(full)) < 1e-6


def test_conv_empty_sequence(gpu):
    x = torch.zeros(2, 0, 8, device=gpu, requires_grad=True)
    tail = torch.randn(2, 8, 3, device=gpu, requires_grad=True)
    w = torch.randn(8, 1, 4, device=gpu, requires_grad=True)
    b = torch.randn(8, device=gpu, requires_grad=True)
    out = conv_hip.run(x, tail, w, b)
    assert out.shape == (2, 0, 8)
    out.sum().backward()
    assert torch.count_nonzero(w.grad) == 0 and torch.count_nonzero(b.grad) == 0
    assert torch.count_nonzero(tail.grad) == 0


def test_conv_supports_reasons(gpu):
    x = torch.randn(2, 5, 8, device=gpu)
    tail = torch.randn(2, 8, 3, device=gpu)
    w = torch.randn(8, 1, 4, device=gpu)
    assert conv_hip.supports(x, tail, w, None) is None
    assert "kernel width" in conv_hip.supports(x, torch.randn(2, 8, 8, device=gpu), torch.randn(8, 1, 9, device=gpu), None)
    assert "tail.shape" in conv_hip.supports(x, torch.randn(2, 8, 2, device=gpu), w, None)
    assert "GPU-only" in conv_hip.supports(x.cpu(), tail.cpu(), w.cpu(), None)
