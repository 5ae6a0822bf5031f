"""GPU parity: the fused projected complex diagonal scan (LRU / S5 layer core) vs the fp64 oracle.

``scan.projected_diagonal_recurrence`` runs ``complex_in_proj -> diagonal_recurrence ->
real_out_proj`` (tsfast/models/_core/scan.py:221-243, 272-313) as LRU.forward and S5.forward call
it (architectures/lru.py:100-110, s5.py:180-198). Its ``hip`` backend keeps v and x out of HBM.
The oracle composes the same three steps in fp64 (``oracle/scan_oracle.py::projscan_*``). Bar:
max relative error <= 1e-5 on y, the returned state and all seven gradients.

Shapes cover every (H, O) kernel instantiation, N that is not a multiple of 64, L that is not a
multiple of the 64-step forward tile or the 32-step backward tile, L = 1, several look-back
chunks per row, and config 2 (N 256, H = O = 32) at full length with the batch reduced. Widths
beyond the fused kernel's (H or O > 32, N > 256) take the wide route (packed GEMMs around the
diagonal scan kernels, split-K weight gradients) and are held to the same bar, with B L large
enough for the split-K products, a remainder row block included.
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import dispatch, scan
from tsfast_amd.scan_backends import projected_hip

pytestmark = pytest.mark.gpu

TOL = 1e-5

# (B, L, H, N, O)
_SHAPES = [
    (2, 7, 3, 4, 2),
    (3, 1, 2, 5, 3),
    (2, 64, 4, 64, 16),
    (3, 100, 5, 70, 3),
    (2, 96, 8, 128, 17),
    (2, 257, 16, 200, 32),
    (2, 300, 32, 256, 32),
    (1, 1000, 1, 1, 1),
    (5, 513, 12, 192, 8),
    (4, 4096, 32, 256, 32),  # config 2, batch reduced
]
# wider than the fused kernel: the wide route
_WIDE_SHAPES = [
    (2, 7, 33, 4, 2),
    (2, 300, 48, 64, 40),
    (2, 257, 16, 300, 8),
    (3, 130, 33, 256, 33),
    (1, 9001, 64, 96, 48),  # split-K over 2 row blocks and a one-row remainder
    (2, 8192, 128, 512, 128),  # the widths of a large LRU / S5 layer, 16 row blocks
]


def _make(B, L, H, N, O_, seed):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, L, H, generator=g)
    W_re = torch.randn(N, H, generator=g) / np.sqrt(H)
    W_im = torch.randn(N, H, generator=g) / np.sqrt(H)
    r = torch.rand(N, generator=g) * 0.099 + 0.9
    th = torch.rand(N, generator=g) * (np.pi / 10)
    lam = torch.polar(r, th)
    C_re = torch.randn(O_, N, generator=g) / np.sqrt(N)
    C_im = torch.randn(O_, N, generator=g) / np.sqrt(N)
    x0 = torch.randn(B, N, dtype=torch.complex64, generator=g)
    gy = torch.randn(B, L, O_, generator=g)
    g_xl = torch.randn(B, N, dtype=torch.complex64, generator=g)
    return u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl


def _np(t):
    return None if t is None else t.detach().cpu().numpy()


def _run(gpu, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl):
    ins = [t.to(gpu).requires_grad_() for t in (u, W_re, W_im, lam, C_re, C_im)]
    x0_d = x0.to(gpu).requires_grad_() if x0 is not None else None
    args = (*ins, x0_d)
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("scan.projected", scan._BACKENDS["projected"], ("hip",), args) is projected_hip
        y, xl = scan.projected_diagonal_recurrence(*args)
    outs, grads = [y], [gy.to(gpu)]
    if g_xl is not None:
        outs.append(xl)
        grads.append(g_xl.to(gpu))
    torch.autograd.backward(outs, grads)
    got_g = [t.grad for t in ins] + [x0_d.grad if x0_d is not None else None]
    return y, xl, got_g


def _check(got_y, got_xl, got_g, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl):
    want_y, want_x = O.projscan_forward(*map(_np, (u, W_re, W_im, lam, C_re, C_im, x0)))
    assert O.rel_err(_np(got_y), want_y) < TOL
    L = want_x.shape[1]
    want_xl = want_x[:, -1] if L > 0 else (_np(x0) if x0 is not None else np.zeros_like(want_x[:, 0]))
    assert O.rel_err(_np(got_xl), want_xl) < TOL
    want_g = O.projscan_backward(
        _np(gy), _np(g_xl), *map(_np, (u, W_re, W_im, lam, C_re, C_im)), want_x, _np(x0)
    )
    names = ("g_u", "g_W_re", "g_W_im", "g_lam", "g_C_re", "g_C_im", "g_x0")
    for name, gg, gw in zip(names, got_g, want_g):
        if gw is None:
            assert gg is None, name
            continue
        assert O.rel_err(_np(gg), gw) < TOL, name


@pytest.mark.parametrize("shape", _SHAPES)
@pytest.mark.parametrize("with_x0", [True, False])
def test_projscan_matches_oracle(gpu, shape, with_x0):
    u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl = _make(*shape, seed=sum(shape))
    x0 = x0 if with_x0 else None
    print(f"projscan shape={shape} x0={with_x0}", flush=True)
    y, xl, grads = _run(gpu, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl)
    torch.cuda.synchronize()
    _check(y, xl, grads, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl)


@pytest.mark.parametrize("shape", _WIDE_SHAPES)
@pytest.mark.parametrize("with_x0", [True, False])
def test_projscan_wide_route_matches_oracle(gpu, shape, with_x0):
    B, L, H, N, O_ = shape
    assert projected_hip.shape_reason(B, L, H, N, O_) is not None
    u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl = _make(*shape, seed=sum(shape))
    x0 = x0 if with_x0 else None
    print(f"projscan wide shape={shape} x0={with_x0}", flush=True)
    y, xl, grads = _run(gpu, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl)
    torch.cuda.synchronize()
    _check(y, xl, grads, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl)


def test_projscan_wide_route_inference_and_chunks(gpu):
    """Wide route: the no-grad op gives the training forward's outputs bit for bit, and carrying
    the returned state through four chunks equals one call."""
    u, W_re, W_im, lam, C_re, C_im, *_ = _make(2, 1024, 40, 300, 36, seed=12)
    d = [t.to(gpu) for t in (u, W_re, W_im, lam, C_re, C_im)]
    with torch.no_grad():
        y0, xl0 = projected_hip.run(*d, None)
        state, ys = None, []
        for k in range(4):
            yk, state = projected_hip.run(d[0][:, 256 * k : 256 * (k + 1)].contiguous(), *d[1:], state)
            ys.append(yk)
    y1, xl1, x = projected_hip._wide_train_op(*d, None)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(xl0, xl1) and x.shape == (2, 1024, 300)
    assert O.rel_err(_np(torch.cat(ys, 1)), _np(y0)) < TOL
    assert O.rel_err(_np(state), _np(xl0)) < TOL


def test_projscan_wide_route_empty_sequence(gpu):
    u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl = _make(2, 0, 40, 8, 3, seed=9)
    y, xl, grads = _run(gpu, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl)
    torch.cuda.synchronize()
    assert y.shape == (2, 0, 3)
    assert torch.equal(xl.cpu(), x0)
    assert torch.equal(grads[6].cpu(), g_xl)
    for gw in grads[1:6]:
        assert not gw.cpu().any()


def test_projscan_without_state_gradient(gpu):
    """Only y is used downstream: the returned state's gradient is zero."""
    u, W_re, W_im, lam, C_re, C_im, x0, gy, _ = _make(2, 130, 6, 90, 5, seed=3)
    y, xl, grads = _run(gpu, u, W_re, W_im, lam, C_re, C_im, x0, gy, None)
    torch.cuda.synchronize()
    _check(y, xl, grads, u, W_re, W_im, lam, C_re, C_im, x0, gy, None)


def test_projscan_inference_matches_training_forward(gpu):
    """The no-grad op (no saved states) gives the training forward's outputs bit for bit."""
    u, W_re, W_im, lam, C_re, C_im, x0, *_ = _make(3, 777, 32, 256, 32, seed=5)
    d = [t.to(gpu) for t in (u, W_re, W_im, lam, C_re, C_im, x0)]
    with torch.no_grad():
        y0, xl0 = projected_hip.run(*d)
    y1, xl1, saved = projected_hip._scan_train_op(*d)
    torch.cuda.synchronize()
    assert saved.numel() == projected_hip.saved_floats(3, 777, 256)
    want_y, want_x = O.projscan_forward(*map(_np, (u, W_re, W_im, lam, C_re, C_im, x0)))
    assert O.rel_err(_np(y0), want_y) < TOL and O.rel_err(_np(y1), want_y) < TOL
    assert O.rel_err(_np(xl0), want_x[:, -1]) < TOL and O.rel_err(_np(xl1), want_x[:, -1]) < TOL


def test_projscan_empty_sequence(gpu):
    """L = 0: y is empty, the returned state is x0, and x0's gradient is the state's gradient."""
    u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl = _make(2, 0, 4, 8, 3, seed=9)
    y, xl, grads = _run(gpu, u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl)
    torch.cuda.synchronize()
    assert y.shape == (2, 0, 3)
    assert torch.equal(xl.cpu(), x0)
    assert torch.equal(grads[6].cpu(), g_xl)
    for gw in grads[1:6]:
        assert not gw.cpu().any()


def test_projscan_tbptt_chunks_equal_one_call(gpu):
    """Carrying the returned state as x0 of the next chunk equals one call over the whole sequence."""
    u, W_re, W_im, lam, C_re, C_im, _, _, _ = _make(2, 1024, 16, 128, 16, seed=11)
    d = [t.to(gpu) for t in (u, W_re, W_im, lam, C_re, C_im)]
    with torch.no_grad():
        y_full, xl_full = projected_hip.run(*d, None)
        state, ys = None, []
        for k in range(4):
            yk, state = projected_hip.run(d[0][:, 256 * k : 256 * (k + 1)].contiguous(), *d[1:], state)
            ys.append(yk)
    torch.cuda.synchronize()
    assert O.rel_err(_np(torch.cat(ys, 1)), _np(y_full)) < TOL
    assert O.rel_err(_np(state), _np(xl_full)) < TOL
