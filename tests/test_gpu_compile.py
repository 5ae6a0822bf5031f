"""torch.compile(fullgraph=True) through the HIP ops on the GPU, forward and backward.

The custom ops (tsfast_hip::*) carry fake implementations and registered autograd, so a compiled
graph must hold them without a graph break; the compiled result must match eager execution to
1e-4 and every gradient must be present and match too. Mirrors the reference's GPU compile tests
(tests/test_mamba.py:329-344, tests/test_dynonet.py:246-265, tests/test_scan_dispatch.py:102-112)
at the level of the sections these ops implement: the Mamba conv + SSM, the diagonal scan (real
and complex), the all-pole scan, the constant-matrix recurrence and the dynoNet G-block.
"""

import warnings

import numpy as np
import pytest
import torch

from tsfast_amd import dispatch, scan
from tsfast_amd.dynonet import core as dcore
from tsfast_amd.mamba import core as mcore

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _rel(a, b):
    a, b = torch.view_as_real(a) if a.is_complex() else a, torch.view_as_real(b) if b.is_complex() else b
    return ((a.detach() - b.detach()).abs().max() / b.detach().abs().max().clamp_min(1e-30)).item()


def _compare(fn, leaves, gout_seed=0):
    """Run fn eagerly and compiled (fullgraph) on copies of the leaves; compare output and grads.

    A fallback to a torch path raises (the dispatcher warns once per op and backend; the warning
    list is cleared and warnings are errors here), so both runs go through the HIP kernels.
    """
    torch._dynamo.reset()
    eager_leaves = [t.detach().clone().requires_grad_(t.requires_grad) for t in leaves]
    comp_leaves = [t.detach().clone().requires_grad_(t.requires_grad) for t in leaves]
    dispatch._warned.clear()
    with dispatch.use_backend("hip"), warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        eager = fn(*eager_leaves)
        g = torch.Generator(device=eager.device).manual_seed(gout_seed)
        gout = torch.randn(eager.shape, dtype=eager.dtype, device=eager.device, generator=g)
        eager.backward(gout)
        compiled = torch.compile(fn, fullgraph=True)(*comp_leaves)
        compiled.backward(gout)
    assert _rel(compiled, eager) < TOL
    for i, (e, c) in enumerate(zip(eager_leaves, comp_leaves)):
        if e.requires_grad:
            assert c.grad is not None, f"leaf {i} has no gradient"
            assert _rel(c.grad, e.grad) < TOL, f"leaf {i}: {_rel(c.grad, e.grad):.2e}"


def test_compile_mamba_conv_and_ssm(gpu):
    g = torch.Generator().manual_seed(0)
    B, L, D, N, K = 2, 64, 48, 16, 4
    xz = torch.randn(B, L, 2 * D, generator=g)
    tail = torch.randn(B, D, K - 1, generator=g)
    w = torch.randn(D, 1, K, generator=g) * 0.5
    bias = torch.randn(D, generator=g)
    draw = torch.randn(B, L, D, generator=g) - 2.0
    A = -torch.exp(torch.randn(D, N, generator=g) * 0.5)
    Bt, Ct = torch.randn(B, L, N, generator=g), torch.randn(B, L, N, generator=g)
    Dp = torch.randn(D, generator=g)
    h0 = torch.randn(B, D, N, generator=g) * 0.5
    leaves = [t.to(gpu).requires_grad_() for t in (xz, tail, w, bias, draw, A, Bt, Ct, Dp, h0)]

    def section(xz, tail, w, bias, draw, A, Bt, Ct, Dp, h0):
        x, z = xz[..., :D], xz[..., D:]  # strided in_proj halves, as a Mamba layer hands them over
        u = mcore.mamba_conv(x, tail, w, bias)
        out, h_last = mcore.mamba_ssm(draw, A, Bt, Ct, u, z, Dp, h0)
        return out + h_last.sum() * 1e-3

    _compare(section, leaves)


@pytest.mark.parametrize("cplx", [False, True])
def test_compile_diagonal_recurrence(gpu, cplx):
    g = torch.Generator().manual_seed(1)
    if cplx:
        lam = torch.polar(torch.rand(6, generator=g) * 0.09 + 0.9, torch.rand(6, generator=g))
        v = torch.randn(3, 2, 500, 6, dtype=torch.complex64, generator=g)
        x0 = torch.randn(3, 2, 6, dtype=torch.complex64, generator=g)
    else:
        lam = torch.rand(6, generator=g) * 0.09 + 0.9
        v = torch.randn(3, 2, 500, 6, generator=g)
        x0 = torch.randn(3, 2, 6, generator=g)
    leaves = [t.to(gpu).requires_grad_() for t in (lam, v, x0)]
    _compare(lambda lam, v, x0: scan.diagonal_recurrence(lam, v, x0), leaves)


def test_compile_selective_recurrence(gpu):
    g = torch.Generator().manual_seed(2)
    a = torch.rand(4, 300, 10, generator=g) * 0.5 + 0.5
    v = torch.randn(4, 300, 10, generator=g)
    x0 = torch.randn(4, 10, generator=g)
    leaves = [t.to(gpu).requires_grad_() for t in (a, v, x0)]
    _compare(lambda a, v, x0: scan.selective_recurrence(a, v, x0), leaves)


def _stable_denominators(g, rows, na):
    r = torch.rand(rows, na, generator=g, dtype=torch.float64) * 0.8
    return torch.stack([torch.tensor(np.poly(ri.numpy())[1:]) for ri in r]).float()


def test_compile_allpole(gpu):
    g = torch.Generator().manual_seed(3)
    a = _stable_denominators(g, 12, 3)
    w = torch.randn(12, 700, generator=g)
    y0 = torch.randn(12, 3, generator=g)
    leaves = [t.to(gpu).requires_grad_() for t in (a, w, y0)]
    _compare(lambda a, w, y0: dcore.allpole(a, w, y0), leaves)


@pytest.mark.parametrize("n", [3, 6])
def test_compile_linear_recurrence(gpu, n):
    g = torch.Generator().manual_seed(4 + n)
    A = torch.randn(5, n, n, generator=g)
    A = A * (0.9 / torch.linalg.eigvals(A.double()).abs().amax(-1).float())[:, None, None]
    v = torch.randn(5, 400, n, generator=g)
    x0 = torch.randn(5, n, generator=g)
    leaves = [t.to(gpu).requires_grad_() for t in (A, v, x0)]
    _compare(lambda A, v, x0: dcore.linear_recurrence(A, v, x0), leaves)


def test_compile_linear_dynamical_operator(gpu):
    g = torch.Generator().manual_seed(5)
    B, L, I, O, nb, na = 2, 300, 2, 4, 4, 2  # 8 channel pairs: the fused G-block serves it
    u = torch.randn(B, L, I, generator=g)
    b = torch.randn(O, I, nb, generator=g) * 0.3
    a = _stable_denominators(g, O * I, na).view(O, I, na)
    leaves = [t.to(gpu).requires_grad_() for t in (u, b, a)]
    _compare(lambda u, b, a: dcore.linear_dynamical_operator(u, b, a), leaves)


def test_compile_linear_dynamical_operator_with_state(gpu):
    """The TBPTT form: a carried state in, the new state out, through the compiled G-block."""
    g = torch.Generator().manual_seed(6)
    B, L, I, O, nb, na = 3, 257, 1, 8, 3, 3
    u = torch.randn(B, L, I, generator=g)
    b = torch.randn(O, I, nb, generator=g) * 0.3
    a = _stable_denominators(g, O * I, na).view(O, I, na)
    u_tail = torch.randn(B, nb - 1, I, generator=g)
    x0 = torch.randn(B, I * O, na, generator=g)
    leaves = [t.to(gpu).requires_grad_() for t in (u, b, a, u_tail, x0)]

    def section(u, b, a, u_tail, x0):
        y, state = dcore.linear_dynamical_operator(u, b, a, {"u": u_tail, "x": x0}, return_state=True)
        return y + 1e-2 * (state["x"].sum() + state["u"].sum())

    _compare(section, leaves)


@pytest.mark.parametrize("widths", [(6, 40, 5), (40, 300, 36)], ids=["fused", "wide"])
def test_compile_projected_diagonal_recurrence(gpu, widths):
    """The LRU/S5 layer core under fullgraph: the fused ops (tsfast_hip::projected_scan_train /
    _bwd) and, beyond their widths, the wide route's (projected_scan_wide_train / _bwd)."""
    g = torch.Generator().manual_seed(9)
    (B, L), (H, N, O) = (2, 400), widths
    leaves = [t.to(gpu).requires_grad_() for t in (
        torch.randn(B, L, H, generator=g), torch.randn(N, H, generator=g) / H**0.5, torch.randn(N, H, generator=g) / H**0.5,
        torch.polar(torch.rand(N, generator=g) * 0.099 + 0.9, torch.rand(N, generator=g) * 0.3),
        torch.randn(O, N, generator=g) / N**0.5, torch.randn(O, N, generator=g) / N**0.5,
        torch.randn(B, N, dtype=torch.complex64, generator=g))]

    def fn(u, W_re, W_im, lam, C_re, C_im, x0):
        y, x_last = scan.projected_diagonal_recurrence(u, W_re, W_im, lam, C_re, C_im, x0)
        return y + torch.view_as_real(x_last).sum()

    _compare(fn, leaves)
