"""The CPU-baseline port (oracle/cpu_baseline.cpp) computes the same thing as the fp64 oracle,
so the bench's CPU column times the right work."""

import math

import numpy as np
import pytest

from oracle import cpu_baseline as CB
from oracle import scan_oracle as O


@pytest.fixture(scope="module")
def lib():
    try:
        return CB.load(prefer_native=False)
    except Exception as e:  # pragma: no cover - no compiler
        pytest.skip(f"cpu baseline unavailable: {e}")


@pytest.mark.parametrize("B,L,D,N,with_h0", [(2, 50, 20, 16, True), (1, 33, 9, 4, False), (2, 17, 8, 12, True)])
def test_mamba_port_matches_oracle(lib, B, L, D, N, with_h0):
    rng = np.random.default_rng(B + L + D + N)
    args = dict(
        draw=rng.normal(-1, 1, (B, L, D)), A=-np.exp(rng.normal(0, 0.5, (D, N))), Bt=rng.standard_normal((B, L, N)),
        Ct=rng.standard_normal((B, L, N)), u=rng.standard_normal((B, L, D)), z=rng.standard_normal((B, L, D)),
        Dp=rng.standard_normal(D),
    )
    args = {k: v.astype(np.float32).astype(np.float64) for k, v in args.items()}
    h0 = rng.standard_normal((B, D, N)).astype(np.float32).astype(np.float64) if with_h0 else None
    gout = rng.standard_normal((B, L, D)).astype(np.float32).astype(np.float64)
    ghl = rng.standard_normal((B, D, N)).astype(np.float32).astype(np.float64) if with_h0 else None
    order = ("draw", "A", "Bt", "Ct", "u", "z", "Dp")
    got = CB.mamba_fwd_bwd(*(args[k] for k in order), gout, h0=h0, ghlast=ghl)
    out, hl = O.mamba_forward(*(args[k] for k in order), h0)
    want = O.mamba_backward(gout, ghl, *(args[k] for k in order), h0)
    assert O.rel_err(got[0], out) < 1e-4 and O.rel_err(got[1], hl) < 1e-4
    for a, b in zip(got[2:], want):
        if b is not None:
            assert O.rel_err(a, b) < 1e-4


@pytest.mark.parametrize("cplx", [False, True])
def test_diag_port_matches_oracle(lib, cplx):
    rng = np.random.default_rng(3)
    M, L, N = 3, 70, 100
    lam = rng.uniform(0.9, 0.999, (M, N))
    v, g, x0 = rng.standard_normal((M, L, N)), rng.standard_normal((M, L, N)), rng.standard_normal((M, N))
    if cplx:
        lam = lam * np.exp(1j * rng.uniform(0, np.pi / 10, (M, N)))
        v, g, x0 = v + 1j * rng.standard_normal(v.shape), g + 1j * rng.standard_normal(g.shape), x0 + 1j
    dt = np.complex64 if cplx else np.float32
    lam, v, g, x0 = (a.astype(dt) for a in (lam, v, g, x0))
    out, glam, gv, gx0 = CB.diag_fwd_bwd(lam, v, g, x0)
    want = O.diag_forward(lam, v, x0)
    wl, wv, wx = O.diag_backward(g, lam, want, x0)
    assert O.rel_err(out, want) < 1e-5
    assert O.rel_err(glam, wl) < 1e-4 and O.rel_err(gv, wv) < 1e-5 and O.rel_err(gx0, wx) < 1e-5


def test_selective_port_matches_oracle(lib):
    rng = np.random.default_rng(4)
    M, L, N = 3, 70, 100
    a = rng.uniform(0.05, 0.95, (M, L, N)).astype(np.float32)
    v, g = rng.standard_normal((M, L, N)).astype(np.float32), rng.standard_normal((M, L, N)).astype(np.float32)
    x0 = rng.standard_normal((M, N)).astype(np.float32)
    out, glam, gv, gx0 = CB.sel_fwd_bwd(a, v, g, x0)
    want = O.selective_forward(a, v, x0)
    wl, wv, wx = O.selective_backward(g, a, want, x0)
    assert O.rel_err(out, want) < 1e-5
    assert O.rel_err(glam, wl) < 1e-5 and O.rel_err(gv, wv) < 1e-5 and O.rel_err(gx0, wx) < 1e-5


def test_torch_reference_doubling_scan_matches_oracle():
    """Config 4's CPU column (oracle/torch_reference.py, the reference's doubling scan and its
    adjoint restated) against the fp64 oracle, x0 included."""
    import torch

    from oracle import torch_reference as TR

    rng = np.random.default_rng(21)
    A = rng.standard_normal((3, 4, 4)) * 0.3
    v, g, x0 = rng.standard_normal((3, 50, 4)), rng.standard_normal((3, 50, 4)), rng.standard_normal((3, 4))
    x = TR.linrec_forward(torch.tensor(A), torch.tensor(v), torch.tensor(x0))
    want = O.linrec_forward(A, v, x0)
    assert O.rel_err(x.numpy(), want) < 1e-12
    got = TR.linrec_backward(torch.tensor(g), torch.tensor(A), x, torch.tensor(x0))
    for a, b in zip(got, O.linrec_backward(g, A, want, x0)):
        assert O.rel_err(a.numpy(), b) < 1e-12


def test_torch_reference_conv_matches_oracle():
    import torch

    from oracle import torch_reference as TR

    rng = np.random.default_rng(22)
    B, L, D, K = 2, 13, 5, 4
    x, tail, w, b = (rng.standard_normal(s) for s in ((B, L, D), (B, D, K - 1), (D, 1, K), (D,)))
    y = TR.causal_depthwise_silu(*(torch.tensor(t) for t in (x, tail, w, b)))
    assert O.rel_err(y.numpy(), O.conv_silu_forward(x, tail, w[:, 0], b)) < 1e-12


def test_ref_expf_is_the_reference_cpu_exp(lib):
    """The port's exp restates the reference CPU kernel's (range reduction to 2^k, Taylor series
    through r^6 / 6!, clamp to [-88, 88]; backend_c.py:55-74): within 2e-7 relative of the true
    exponential on [-1, 1] (k = 0 or +-1), within 5e-6 wherever 2^k is a normal float (built with
    the reference's -ffast-math, the compiler may fold the two-part ln 2 of the reduction into one
    rounded product, so r carries up to half an ulp of x), exact at 0, clamped above 88, and zero
    where k reaches -127 (the exponent-bits scale is then 0). A series cut one term short
    (r^5 / 5!) misses the [-1, 1] bound."""
    x = np.linspace(-1, 1, 20_001).astype(np.float32)
    got = CB.ref_expf(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    assert np.max(np.abs(got / want - 1)) < 2e-7
    xw = np.linspace(-87.0, 87.9, 200_001).astype(np.float32)
    assert np.max(np.abs(CB.ref_expf(xw).astype(np.float64) / np.exp(xw.astype(np.float64)) - 1)) < 5e-6
    assert CB.ref_expf(np.zeros(1))[0] == 1.0
    assert CB.ref_expf(np.array([100.0]))[0] == CB.ref_expf(np.array([88.0]))[0]
    assert CB.ref_expf(np.array([-88.0]))[0] == 0.0 and CB.ref_expf(np.array([-1000.0]))[0] == 0.0
    # the mutant: drop the r^6 term of the same reduction
    r = x.astype(np.float64) - np.round(x.astype(np.float64) / np.log(2)) * np.log(2)
    short = np.exp(x.astype(np.float64) - r) * sum(r**n / math.factorial(n) for n in range(6))
    assert np.max(np.abs(short / want - 1)) > 2e-7
