"""Bitwise run-to-run reproducibility of every HIP scan (the reference's kernels are deterministic
by construction, tsfast/models/architectures/mamba/mamba_triton.py:19-22).

In deterministic mode (tsfast_hip_set_deterministic: on by default, kept on by the backends unless
tsfast_amd.set_reproducible(False) and torch.are_deterministic_algorithms_enabled() is false) the
look-back scans (diagonal, selective, all-pole, linear recurrence, G-block, projected) chain their
tiles with anchored publication (csrc/lookback.h): a tile composes exactly the aggregates back to
its anchor's published state, so which tiles happen to be finished when it looks back does not
change a single bit. Sums over tiles run in fixed orders. Each test calls an op three times on the
same inputs (a different amount of other GPU work queued before each call) under
torch.use_deterministic_algorithms and requires every output to be equal bit for bit, and the
results to agree with the fast mode's (reproducibility off: the nearest published maps) to fp32
rounding. Shapes span many super-chunks, so the walks cross several anchor spans. One test repeats
the diagonal scan in the library's default mode, with torch's flag off.
"""

import math

import numpy as np
import pytest
import torch

from tsfast_amd import _lib
from tsfast_amd.dynonet import allpole_hip, gblock_hip, linrec_hip
from tsfast_amd.mamba import conv_hip, mamba_hip
from tsfast_amd.scan_backends import diagonal_hip, projected_hip, selective_hip

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def deterministic_mode():
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(False)


def _repeat(fn, *args, reps=3):
    fast = _default_mode(fn, *args)
    outs = []
    noise = torch.randn(1 << 22, device=args[0].device)
    for r in range(reps):
        for _ in range(r * 3):  # vary what the GPU is doing when the call starts
            noise.mul_(1.0001)
        res = fn(*args)
        res = res if isinstance(res, (tuple, list)) else (res,)
        outs.append([t.clone() if isinstance(t, torch.Tensor) else t for t in res])
    torch.cuda.synchronize()
    for i, (d, f) in enumerate(zip(outs[0], fast)):
        if isinstance(d, torch.Tensor) and d.numel():
            scale = f.abs().max().clamp_min(1e-30)
            assert ((d - f).abs().max() / scale).item() < 1e-6, f"output {i}: deterministic vs default mode"
    return outs


def _default_mode(fn, *args):
    """The op in the fast mode (reproducibility off, torch's flag off)."""
    torch.use_deterministic_algorithms(False)
    prev = _lib.set_reproducible(False)
    try:
        res = fn(*args)
        res = res if isinstance(res, (tuple, list)) else (res,)
        res = [t.clone() if isinstance(t, torch.Tensor) else t for t in res]
        torch.cuda.synchronize()
        return res
    finally:
        _lib.set_reproducible(prev)
        torch.use_deterministic_algorithms(True, warn_only=True)


def _assert_same(outs):
    for rep in outs[1:]:
        for i, (a, b) in enumerate(zip(outs[0], rep)):
            if isinstance(a, torch.Tensor):
                assert torch.equal(a, b), f"output {i} differs between runs"


@pytest.mark.parametrize("cplx", [False, True])
def test_diagonal_scan_bitwise_repeatable(gpu, cplx):
    g = torch.Generator().manual_seed(1)
    M, L, N = 16, 16384, 64
    if cplx:
        lam = torch.polar(torch.rand(M, N, generator=g) * 0.099 + 0.9, torch.rand(M, N, generator=g) * 0.3)
        v = torch.randn(M, L, N, dtype=torch.complex64, generator=g)
        gy = torch.randn(M, L, N, dtype=torch.complex64, generator=g)
        x0 = torch.randn(M, N, dtype=torch.complex64, generator=g)
    else:
        lam = torch.rand(M, N, generator=g) * 0.0099 + 0.99
        v, gy, x0 = torch.randn(M, L, N, generator=g), torch.randn(M, L, N, generator=g), torch.randn(M, N, generator=g)
    lam, v, gy, x0 = (t.to(gpu) for t in (lam, v, gy, x0))

    def call(lam, v, gy, x0):
        x = diagonal_hip.forward(lam, v, x0)
        return (x, *diagonal_hip.backward(gy, lam, x, x0))

    _assert_same(_repeat(call, lam, v, gy, x0))


def test_selective_scan_bitwise_repeatable(gpu):
    g = torch.Generator().manual_seed(2)
    M, L, N = 8, 12000, 128
    lam = (torch.rand(M, L, N, generator=g) * 0.1 + 0.9).to(gpu)
    v, gy = torch.randn(M, L, N, generator=g).to(gpu), torch.randn(M, L, N, generator=g).to(gpu)
    x0 = torch.randn(M, N, generator=g).to(gpu)

    def call(lam, v, gy, x0):
        x = selective_hip.forward(lam, v, x0)
        return (x, *selective_hip.backward(gy, lam, x, x0))

    _assert_same(_repeat(call, lam, v, gy, x0))


def test_allpole_bitwise_repeatable(gpu):
    g = torch.Generator().manual_seed(3)
    lanes, L, na = 512, 16384, 3
    r = torch.rand(lanes, na, generator=g, dtype=torch.float64) * 0.48 + 0.5
    a = torch.stack([torch.tensor(np.poly(ri.numpy())[1:]) for ri in r]).float().to(gpu)
    w, gy = torch.randn(lanes, L, generator=g).to(gpu), torch.randn(lanes, L, generator=g).to(gpu)
    y0 = torch.randn(lanes, na, generator=g).to(gpu)

    def call(a, w, y0, gy):
        y = allpole_hip._allpole_op(a, w, y0)
        return (y, *allpole_hip._allpole_bwd_op(gy, a, y, y0))

    _assert_same(_repeat(call, a, w, y0, gy))


@pytest.mark.parametrize("n", [3, 6])
def test_linrec_bitwise_repeatable(gpu, n):
    g = torch.Generator().manual_seed(4)
    M, L = 600, 8000
    A = torch.randn(M, n, n, generator=g, dtype=torch.float64)
    rho = torch.linalg.eigvals(A).abs().amax(-1).clamp_min(1e-6)
    A = (A * (0.97 / rho)[:, None, None]).float().to(gpu)
    v, gx = torch.randn(M, L, n, generator=g).to(gpu), torch.randn(M, L, n, generator=g).to(gpu)
    x0 = torch.randn(M, n, generator=g).to(gpu)

    def call(A, v, x0, gx):
        x = linrec_hip._linrec_op(A, v, x0)
        return (x, *linrec_hip._linrec_bwd_op(gx, A, x, x0))

    _assert_same(_repeat(call, A, v, x0, gx))


def test_gblock_bitwise_repeatable(gpu):
    g = torch.Generator().manual_seed(5)
    B, L, I, O, nb, na = 8, 16384, 4, 4, 6, 2
    u = torch.randn(B, L, I, generator=g).to(gpu)
    b = (torch.randn(O, I, nb, generator=g) * 0.1).to(gpu)
    a = torch.tensor([-1.1, 0.3]).expand(O, I, na).contiguous().to(gpu)
    gy = torch.randn(B, L, O, generator=g).to(gpu)
    tail, x0 = u.new_zeros(B, nb - 1, I), u.new_zeros(B, I * O, na)

    def call(u, b, a, gy):
        y, x_last, saved = gblock_hip._gblock_op(u, b, a, tail, x0)
        return (y, x_last, *gblock_hip._gblock_bwd_op(gy, None, u, b, a, tail, x0, saved))

    _assert_same(_repeat(call, u, b, a, gy))


def test_projected_scan_repeatable(gpu):
    """Every output and gradient is bitwise repeatable: y and the returned state from the fused
    forward's anchored look-back, and all seven gradients from the backward, which in this mode
    recomputes the states and runs the wide route's backward (the fused backward's parameter
    gradients are sums a workgroup accumulates over the tiles it takes from a counter, whose order
    depends on timing). The deterministic gradients also agree with the fused backward's to 1e-5."""
    g = torch.Generator().manual_seed(6)
    B, L, H, N, O = 4, 8192, 32, 256, 32
    u = torch.randn(B, L, H, generator=g)
    W_re, W_im = torch.randn(N, H, generator=g) / math.sqrt(H), torch.randn(N, H, generator=g) / math.sqrt(H)
    lam = torch.polar(torch.rand(N, generator=g) * 0.099 + 0.9, torch.rand(N, generator=g) * 0.3)
    C_re, C_im = torch.randn(O, N, generator=g) / 16, torch.randn(O, N, generator=g) / 16
    gy = torch.randn(B, L, O, generator=g)
    x0 = torch.randn(B, N, dtype=torch.complex64, generator=g)
    gxl = torch.randn(B, N, dtype=torch.complex64, generator=g)
    ins = [t.to(gpu) for t in (u, W_re, W_im, lam, C_re, C_im, x0, gy, gxl)]

    def call(u, W_re, W_im, lam, C_re, C_im, x0, gy, gxl):
        y, x_last, saved = projected_hip._scan_train_op(u, W_re, W_im, lam, C_re, C_im, x0)
        return (y, x_last, *projected_hip.backward(gy, gxl, saved, u, W_re, W_im, lam, C_re, C_im, x0))

    fused = _default_mode(call, *ins)  # the fused backward kernel
    noise = torch.randn(1 << 22, device=gpu)
    outs = []
    for r in range(3):
        for _ in range(r * 3):
            noise.mul_(1.0001)
        outs.append([t.clone() for t in call(*ins)])
    torch.cuda.synchronize()
    _assert_same(outs)
    for i, (a, b) in enumerate(zip(outs[0], fused)):
        if b.numel():
            assert ((a - b).abs().max() / b.abs().max()).item() < 1e-5, f"output {i}: deterministic vs fused"


def test_projected_wide_route_bitwise_repeatable(gpu):
    """Beyond the fused widths the projected scan runs GEMMs around the diagonal scan kernels and
    takes its weight gradients as split-K products summed in a fixed order: every output and
    gradient repeats bit for bit, and matches the fast mode's to 1e-6."""
    g = torch.Generator().manual_seed(12)
    B, L, H, N, O = 2, 9000, 48, 300, 40
    assert projected_hip.shape_reason(B, L, H, N, O) is not None
    u = torch.randn(B, L, H, generator=g)
    W_re, W_im = torch.randn(N, H, generator=g) / math.sqrt(H), torch.randn(N, H, generator=g) / math.sqrt(H)
    lam = torch.polar(torch.rand(N, generator=g) * 0.099 + 0.9, torch.rand(N, generator=g) * 0.3)
    C_re, C_im = torch.randn(O, N, generator=g) / 16, torch.randn(O, N, generator=g) / 16
    gy = torch.randn(B, L, O, generator=g)
    x0 = torch.randn(B, N, dtype=torch.complex64, generator=g)
    g_xl = torch.randn(B, N, dtype=torch.complex64, generator=g)
    ins = [t.to(gpu) for t in (u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl)]

    def call(u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl):
        y, x_last, x = projected_hip._wide_train_op(u, W_re, W_im, lam, C_re, C_im, x0)
        return (y, x_last, *projected_hip._wide_bwd_op(gy, g_xl, x, u, W_re, W_im, lam, C_re, C_im, x0))

    _assert_same(_repeat(call, *ins))


def test_mamba_and_conv_bitwise_repeatable(gpu):
    """No look-back here (one workgroup walks a whole sequence); the channel and batch sums run in
    fixed orders."""
    g = torch.Generator().manual_seed(7)
    B, L, D, N = 4, 2048, 512, 16
    bf = torch.bfloat16
    args = [
        (torch.randn(B, L, D, generator=g) - 4).to(bf), -torch.arange(1, N + 1.0).expand(D, N).contiguous(),
        torch.randn(B, L, N, generator=g).to(bf), torch.randn(B, L, N, generator=g).to(bf),
        torch.randn(B, L, D, generator=g).to(bf), torch.randn(B, L, D, generator=g).to(bf), torch.randn(D, generator=g),
    ]
    args = [t.to(gpu) for t in args] + [None]
    gout = torch.randn(B, L, D, generator=g).to(bf).to(gpu)

    def mamba(*a):
        out, h_last, chk = mamba_hip._scan_train_op(*a)
        return (out, h_last, *mamba_hip._scan_bwd_op(gout, None, chk, *a)[:7])

    _assert_same(_repeat(mamba, *args))
    x = torch.randn(B, L, 2 * D, generator=g).to(gpu)
    tail, w, bias = (torch.randn(B, D, 3, generator=g).to(gpu), torch.randn(D, 1, 4, generator=g).to(gpu),
                     torch.randn(D, generator=g).to(gpu))
    gyc = torch.randn(B, L, D, generator=g).to(gpu)

    def conv(x, tail, w, bias, gyc):
        xv = x[..., :D]
        y = conv_hip._conv_silu_op(xv, tail, w, bias)
        return (y, *conv_hip._conv_silu_bwd_op(gyc, xv, tail, w, bias))

    _assert_same(_repeat(conv, x, tail, w, bias, gyc))


def test_backends_follow_the_reproducibility_settings(gpu):
    """A look-back scan runs in the library's deterministic mode by default and under
    torch.use_deterministic_algorithms(True) whatever set_reproducible says; only with both off
    does it take the fast mode."""
    lam = torch.full((4, 8), 0.9, device=gpu)
    v = torch.randn(4, 100, 8, device=gpu)
    diagonal_hip.forward(lam, v, None)
    assert _lib.load().tsfast_hip_get_deterministic() == 1
    prev = _lib.set_reproducible(False)
    try:
        diagonal_hip.forward(lam, v, None)  # torch's flag is on (fixture)
        assert _lib.load().tsfast_hip_get_deterministic() == 1
        torch.use_deterministic_algorithms(False)
        diagonal_hip.forward(lam, v, None)
        assert _lib.load().tsfast_hip_get_deterministic() == 0
        _lib.set_reproducible(True)
        diagonal_hip.forward(lam, v, None)
        assert _lib.load().tsfast_hip_get_deterministic() == 1
    finally:
        _lib.set_reproducible(prev)


def test_default_mode_is_bitwise_repeatable(gpu):
    """Without torch's flag, the library's default mode alone makes the look-back scans repeat bit
    for bit (diagonal scan over many super-chunks, forward and backward)."""
    torch.use_deterministic_algorithms(False)
    g = torch.Generator().manual_seed(11)
    lam = (torch.rand(8, 256, generator=g) * 0.099 + 0.9).to(gpu)
    v = torch.randn(8, 20000, 256, generator=g).to(gpu)
    gv = torch.randn(8, 20000, 256, generator=g).to(gpu)
    x0 = torch.randn(8, 256, generator=g).to(gpu)

    def call(lam, v, gv, x0):
        out = diagonal_hip.forward(lam, v, x0)
        return (out, *diagonal_hip.backward(gv, lam, out, x0))

    noise = torch.randn(1 << 22, device=gpu)
    outs = []
    for r in range(3):
        for _ in range(r * 3):
            noise.mul_(1.0001)
        outs.append([t.clone() for t in call(lam, v, gv, x0)])
    torch.cuda.synchronize()
    _assert_same(outs)


def test_nss_adjoint_scan_bitwise_repeatable(gpu):
    """No look-back and no atomics: every chunk summary and the carry run in a fixed order."""
    from tsfast_amd.ssm import adjoint_hip

    g = torch.Generator().manual_seed(8)
    jt = (torch.randn(4, 2000, 24, 24, generator=g) * (0.9 / 24**0.5)).to(gpu)
    gout = torch.randn(4, 2000, 24, generator=g).to(gpu)
    _assert_same(_repeat(lambda jt, gout: adjoint_hip.run(jt, gout, 100), jt, gout))
