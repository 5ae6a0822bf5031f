"""The torch fallback paths of the op layer, on the CPU, against the fp64 oracle.

These run whenever no HIP backend serves the inputs (CPU tensors, an explicit "reference"
preference, shapes a kernel declines): the blocked two-level scans of tsfast_amd.blocked_scan
behind the scan ops and linear_recurrence, the sliced unfused Mamba SSM, the grouped-conv
Mamba conv, and the complex projections around the LRU/S5 scan. Inputs are float64 (and
complex128) so the comparison tests the algorithms, at 1e-10 max relative error.
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import blocked_scan, scan
from tsfast_amd.mamba import core as mcore

TOL = 1e-10


def _t(x, grad=True):
    t = torch.tensor(x)
    return t.requires_grad_() if grad else t


@pytest.mark.parametrize("L", [1, 7, 64, 65, 300])
@pytest.mark.parametrize("cplx", [False, True])
def test_diagonal_recurrence_fallback(L, cplx):
    rng = np.random.default_rng(L + 7 * cplx)
    M, n = 3, 5
    if cplx:
        lam = rng.uniform(0.8, 0.99, (M, n)) * np.exp(1j * rng.uniform(0, 1, (M, n)))
        v = rng.standard_normal((M, L, n)) + 1j * rng.standard_normal((M, L, n))
        x0 = rng.standard_normal((M, n)) + 1j * rng.standard_normal((M, n))
        g = rng.standard_normal((M, L, n)) + 1j * rng.standard_normal((M, L, n))
    else:
        lam, v, x0 = rng.uniform(0.8, 0.99, (M, n)), rng.standard_normal((M, L, n)), rng.standard_normal((M, n))
        g = rng.standard_normal((M, L, n))
    lt, vt, xt = _t(lam), _t(v), _t(x0)
    out = scan.diagonal_recurrence(lt, vt, xt)
    out.backward(torch.tensor(g))
    want = O.diag_forward(lam, v, x0)
    glam, gv, gx0 = O.diag_backward(g, lam, want, x0)
    assert O.rel_err(out.detach().numpy(), want) < TOL
    assert O.rel_err(lt.grad.numpy(), glam) < TOL
    assert O.rel_err(vt.grad.numpy(), gv) < TOL
    assert O.rel_err(xt.grad.numpy(), gx0) < TOL


def test_diagonal_recurrence_broadcast_lam():
    """lam [n] against v [B, P, L, n]: the lane grads are summed back to lam's shape."""
    rng = np.random.default_rng(3)
    lam, v, g = rng.uniform(0.5, 0.95, 4), rng.standard_normal((2, 3, 20, 4)), rng.standard_normal((2, 3, 20, 4))
    lt, vt = _t(lam), _t(v)
    scan.diagonal_recurrence(lt, vt).backward(torch.tensor(g))
    lanes = np.broadcast_to(lam, (6, 4))
    want = O.diag_forward(lanes, v.reshape(6, 20, 4))
    glam, _, _ = O.diag_backward(g.reshape(6, 20, 4), lanes, want)
    assert O.rel_err(lt.grad.numpy(), glam.sum(0)) < TOL


@pytest.mark.parametrize("L", [1, 33, 129])
def test_selective_recurrence_fallback(L):
    rng = np.random.default_rng(L)
    M, n = 2, 6
    a, v = rng.uniform(0.3, 1.0, (M, L, n)), rng.standard_normal((M, L, n))
    x0, g = rng.standard_normal((M, n)), rng.standard_normal((M, L, n))
    at, vt, xt = _t(a), _t(v), _t(x0)
    out = scan.selective_recurrence(at, vt, xt)
    out.backward(torch.tensor(g))
    want = O.selective_forward(a, v, x0)
    ga, gv, gx0 = O.selective_backward(g, a, want, x0)
    assert O.rel_err(out.detach().numpy(), want) < TOL
    for got, w in ((at.grad, ga), (vt.grad, gv), (xt.grad, gx0)):
        assert O.rel_err(got.numpy(), w) < TOL


def test_blocked_scan_matches_sequential_loop():
    rng = np.random.default_rng(5)
    a, v, x0 = (torch.tensor(rng.uniform(0.5, 1.0, (2, 1000, 3))), torch.tensor(rng.standard_normal((2, 1000, 3))),
                torch.tensor(rng.standard_normal((2, 3))))
    assert torch.allclose(blocked_scan.scan_diagonal(a, v, x0), blocked_scan.sequential(a, v, x0), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("backend", ["scan", "eager"])
@pytest.mark.parametrize("with_h0", [False, True])
def test_mamba_ssm_unfused_path(backend, with_h0, monkeypatch):
    rng = np.random.default_rng(11 + with_h0)
    B, L, D, N = 2, 37, 5, 4
    A = -np.exp(rng.standard_normal((D, N)) * 0.5)
    args = dict(
        draw=rng.standard_normal((B, L, D)) - 1.0, A=A, Bt=rng.standard_normal((B, L, N)),
        Ct=rng.standard_normal((B, L, N)), u=rng.standard_normal((B, L, D)), z=rng.standard_normal((B, L, D)),
        Dp=rng.standard_normal(D), h0=rng.standard_normal((B, D, N)) if with_h0 else None,
    )
    # slices of 3 steps, so the carried state crosses many slice boundaries
    monkeypatch.setattr(mcore, "_SLICE_ELEMS", 3 * B * D * N)
    ts = {k: (None if v is None else _t(v)) for k, v in args.items()}
    out, h_last = mcore.mamba_ssm(*ts.values(), backend=backend)
    gout = rng.standard_normal((B, L, D))
    out.backward(torch.tensor(gout))
    want_out, want_h = O.mamba_forward(*args.values())
    assert O.rel_err(out.detach().numpy(), want_out) < TOL
    assert O.rel_err(h_last.detach().numpy().reshape(B, D, N), want_h) < TOL
    grads = O.mamba_backward(gout, None, *args.values())
    for name, w in zip(("draw", "A", "Bt", "Ct", "u", "z", "Dp", "h0"), grads):
        if w is not None:
            assert O.rel_err(ts[name].grad.numpy(), w) < TOL, name


def test_mamba_conv_unfused_path():
    rng = np.random.default_rng(2)
    B, L, D, K = 2, 19, 6, 4
    x, tail = rng.standard_normal((B, L, D)), rng.standard_normal((B, D, K - 1))
    w, bias = rng.standard_normal((D, 1, K)), rng.standard_normal(D)
    xt, tt, wt, bt = _t(x), _t(tail), _t(w), _t(bias)
    y = mcore.mamba_conv(xt, tt, wt, bt, backend="eager")
    gy = rng.standard_normal((B, L, D))
    y.backward(torch.tensor(gy))
    assert O.rel_err(y.detach().numpy(), O.conv_silu_forward(x, tail, w[:, 0], bias)) < TOL
    got = (xt.grad, tt.grad, wt.grad[:, 0], bt.grad)
    for g_, want in zip(got, O.conv_silu_backward(gy, x, tail, w[:, 0], bias)):
        assert O.rel_err(g_.numpy(), want) < TOL


def test_complex_projections_match_complex_matmul():
    """complex_in_proj / real_out_proj (one real GEMM each, interleaved weights) against the
    complex products written out with numpy, forward and every gradient (autograd of a
    complex128 matmul as the independent route)."""
    rng = np.random.default_rng(4)
    d, n, o = 6, 5, 3
    u = rng.standard_normal((2, 7, d))
    W_re, W_im = rng.standard_normal((n, d)), rng.standard_normal((n, d))
    x = rng.standard_normal((2, 7, n)) + 1j * rng.standard_normal((2, 7, n))
    C_re, C_im = rng.standard_normal((o, n)), rng.standard_normal((o, n))
    v = scan.complex_in_proj(torch.tensor(u), torch.tensor(W_re), torch.tensor(W_im))
    assert O.rel_err(v.numpy(), u @ (W_re + 1j * W_im).T) < TOL
    y = scan.real_out_proj(torch.tensor(x), torch.tensor(C_re), torch.tensor(C_im))
    assert O.rel_err(y.numpy(), (x @ (C_re + 1j * C_im).T).real) < TOL

    def through(in_fn, out_fn):
        leaves = [_t(a) for a in (u, W_re, W_im, C_re, C_im)]
        h = in_fn(*leaves[:3])
        out_fn(h * 0.7, *leaves[3:]).square().sum().backward()
        return [t.grad.numpy() for t in leaves]

    got = through(scan.complex_in_proj, scan.real_out_proj)
    want = through(
        lambda u_, a, b: u_.to(torch.complex128) @ torch.complex(a, b).T,
        lambda h, a, b: (h @ torch.complex(a, b).T).real,
    )
    for g_, w_ in zip(got, want):
        assert O.rel_err(g_, w_) < TOL
