"""Dynamo traces every public section without a graph break (CPU, fallback ops).

``torch.compile(fullgraph=True, backend="eager")`` runs Dynamo's tracing and the custom ops'
fake implementations but no code generation, so this checks on the CPU that the wrappers hold
nothing Dynamo refuses (mapping ``match`` patterns, ``importlib`` in a registry, data-dependent
Python control flow); the compiled result must equal eager execution. The GPU suite repeats the
sections through the HIP ops with Inductor.
"""

import numpy as np
import torch

from tsfast_amd import scan
from tsfast_amd.dynonet import core as dcore
from tsfast_amd.mamba import core as mcore


def _check(fn, *args):
    torch._dynamo.reset()
    leaves_e = [a.detach().clone().requires_grad_() for a in args]
    leaves_c = [a.detach().clone().requires_grad_() for a in args]
    want = fn(*leaves_e)
    got = torch.compile(fn, fullgraph=True, backend="eager")(*leaves_c)
    torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-6)
    gout = torch.randn_like(want)
    want.backward(gout)
    got.backward(gout)
    for e, c in zip(leaves_e, leaves_c):
        assert c.grad is not None
        torch.testing.assert_close(c.grad, e.grad, rtol=1e-5, atol=1e-6)


def _denominators(g, rows, na):
    r = torch.rand(rows, na, generator=g, dtype=torch.float64) * 0.8
    return torch.stack([torch.tensor(np.poly(ri.numpy())[1:]) for ri in r]).float()


def test_trace_scans():
    g = torch.Generator().manual_seed(0)
    lam = torch.rand(5, generator=g) * 0.1 + 0.85
    v = torch.randn(2, 40, 5, generator=g)
    x0 = torch.randn(2, 5, generator=g)
    _check(lambda lam, v, x0: scan.diagonal_recurrence(lam, v, x0), lam, v, x0)
    a = torch.rand(2, 40, 5, generator=g) * 0.5 + 0.5
    _check(lambda a, v, x0: scan.selective_recurrence(a, v, x0), a, v, x0)


def test_trace_mamba_sections():
    g = torch.Generator().manual_seed(1)
    B, L, D, N, K = 2, 24, 6, 4, 4
    x = torch.randn(B, L, D, generator=g)
    tail = torch.randn(B, D, K - 1, generator=g)
    w = torch.randn(D, 1, K, generator=g) * 0.5
    bias = torch.randn(D, generator=g)
    draw = torch.randn(B, L, D, generator=g) - 1.0
    A = -torch.exp(torch.randn(D, N, generator=g) * 0.5)
    Bt, Ct = torch.randn(B, L, N, generator=g), torch.randn(B, L, N, generator=g)
    z, Dp = torch.randn(B, L, D, generator=g), torch.randn(D, generator=g)

    def section(x, tail, w, bias, draw, A, Bt, Ct, z, Dp):
        u = mcore.mamba_conv(x, tail, w, bias)
        out, h_last = mcore.mamba_ssm(draw, A, Bt, Ct, u, z, Dp)
        return out + h_last.sum() * 1e-2

    _check(section, x, tail, w, bias, draw, A, Bt, Ct, z, Dp)


def test_trace_dynonet_sections():
    g = torch.Generator().manual_seed(2)
    A = torch.randn(3, 3, 3, generator=g) * 0.3
    v = torch.randn(3, 50, 3, generator=g)
    _check(lambda A, v: dcore.linear_recurrence(A, v), A, v)
    a = _denominators(g, 4, 2)
    w = torch.randn(4, 50, generator=g)
    _check(lambda a, w: dcore.allpole(a, w), a, w)
    u = torch.randn(2, 30, 2, generator=g)
    b = torch.randn(3, 2, 3, generator=g) * 0.3
    ad = _denominators(g, 6, 2).view(3, 2, 2)
    tail, x0 = torch.randn(2, 2, 2, generator=g), torch.randn(2, 6, 2, generator=g)

    def gblock(u, b, ad, tail, x0):
        y, state = dcore.linear_dynamical_operator(u, b, ad, {"u": tail, "x": x0}, return_state=True)
        return y + 1e-2 * state["x"].sum()

    _check(gblock, u, b, ad, tail, x0)
    _check(lambda u, b, ad: dcore.linear_dynamical_operator(u, b, ad), u, b, ad)
