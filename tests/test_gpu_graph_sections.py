"""The fused Mamba and dynoNet sections under HIP graph capture: the Mamba SSM training forward +
backward, the causal conv + SiLU forward + backward, and the G-block forward + backward.

Each op sizes its own scratch from torch's allocator (inside a capture that is the graph's private
pool) and clears what must start at zero with kernels, never memset nodes, so one captured
forward + backward must reproduce eager results on every replay, with new inputs copied in and
eager work between replays. Mirrors the reference's graph tests for these sections
(tests/test_mamba.py:329-344 runs the model through the captured path,
models/_core/cudagraph.py:53-185 is the capture/replay wrapper it exercises).
"""

import numpy as np
import pytest
import torch

from tsfast_amd.dynonet import gblock_hip
from tsfast_amd.mamba import conv_hip, mamba_hip

pytestmark = pytest.mark.gpu

TOL = 1e-6


def _close(a, b):
    if a.numel() == 0:
        return True
    return (a.float() - b.float()).abs().max().item() <= TOL * max(b.float().abs().max().item(), 1e-30)


def _mamba_inputs(seed, dev, B=2, L=1000, D=64, N=16):
    g = torch.Generator().manual_seed(seed)
    draw = torch.randn(B, L, D, generator=g) - 2.0
    A = -torch.exp(torch.randn(D, N, generator=g) * 0.5)
    Bt, Ct = torch.randn(B, L, N, generator=g), torch.randn(B, L, N, generator=g)
    u, z = torch.randn(B, L, D, generator=g), torch.randn(B, L, D, generator=g)
    Dp = torch.randn(D, generator=g)
    h0 = torch.randn(B, D, N, generator=g) * 0.5
    gout, ghlast = torch.randn(B, L, D, generator=g), torch.randn(B, D, N, generator=g)
    return [t.to(dev) for t in (draw, A, Bt, Ct, u, z, Dp, h0, gout, ghlast)]


def _run_mamba(draw, A, Bt, Ct, u, z, Dp, h0, gout, ghlast):
    out, h_last, chk = mamba_hip._scan_train_op(draw, A, Bt, Ct, u, z, Dp, h0)
    grads = mamba_hip._scan_bwd_op(gout, ghlast, chk, draw, A, Bt, Ct, u, z, Dp, h0)
    return (out, h_last, *grads)


def _conv_inputs(seed, dev, B=3, L=3000, D=96, K=4):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, L, D, generator=g)
    tail = torch.randn(B, D, K - 1, generator=g)
    w = torch.randn(D, K, generator=g) * 0.5
    bias = torch.randn(D, generator=g)
    gy = torch.randn(B, L, D, generator=g)
    return [t.to(dev) for t in (x, tail, w, bias, gy)]


def _run_conv(x, tail, w, bias, gy):
    y = conv_hip._conv_silu_op(x, tail, w, bias)
    return (y, *conv_hip._conv_silu_bwd_op(gy, x, tail, w, bias))


def _gblock_inputs(seed, dev, B=16, L=6000, I=2, O=4, nb=3, na=2):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, L, I, generator=g)
    b = torch.randn(O, I, nb, generator=g) * 0.3
    r = torch.rand(O * I, na, generator=g, dtype=torch.float64) * 0.9
    a = torch.stack([torch.tensor(np.poly(ri.numpy())[1:]) for ri in r]).float().view(O, I, na)
    u_tail = torch.randn(B, nb - 1, I, generator=g)
    x0 = torch.randn(B, I * O, na, generator=g)
    gy = torch.randn(B, L, O, generator=g)
    g_xlast = torch.randn(B, I * O, na, generator=g)
    return [t.to(dev) for t in (u, b, a, u_tail, x0, gy, g_xlast)]


def _run_gblock(u, b, a, u_tail, x0, gy, g_xlast):
    y, x_last, saved = gblock_hip._gblock_op(u, b, a, u_tail, x0)
    return (y, x_last, *gblock_hip._gblock_bwd_op(gy, g_xlast, u, b, a, u_tail, x0, saved))


_SECTIONS = {
    "mamba": (_mamba_inputs, _run_mamba),
    "conv": (_conv_inputs, _run_conv),
    "gblock": (_gblock_inputs, _run_gblock),
}


@pytest.mark.parametrize("section", list(_SECTIONS))
def test_graph_replay_matches_eager(gpu, section):
    make, run = _SECTIONS[section]
    ins = make(0, gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(*ins)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run(*ins)
    for rep in range(1, 4):
        for dst, src in zip(ins, make(rep, gpu)):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        eager = run(*ins)  # eager work between replays
        torch.cuda.synchronize()
        for i, (c, e) in enumerate(zip(captured, eager)):
            assert _close(c, e), f"replay {rep}: output {i}"
