"""GPU parity: HIP all-pole IIR scan vs the fp64 oracle (through the dynoNet dispatch point).

Shapes follow tests/test_scan_allpole_backend.py:21-28 of the reference (L = 1, L < na, na = 8,
a single odd-length lane) plus the order limits (na = 1, 16) and a reduced config 4. Outputs and
all gradients (a, w, y0) must match within 1e-5 relative (fp32 vs fp64).
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import dispatch
from tsfast_amd.dynonet import allpole_hip
from tsfast_amd.dynonet import core as dcore

pytestmark = pytest.mark.gpu

TOL = 1e-5

_SHAPES = [
    (32, 8, 200, 2),
    (4, 32, 100, 8),
    (3, 5, 7, 3),
    (2, 4, 1, 2),
    (2, 4, 2, 4),
    (1, 1, 513, 1),
    (2, 3, 300, 16),
    (8, 64, 16384, 3),  # config 4 with the batch reduced from 64 to 8
    # single-pass look-back path (na <= 4): many super-chunks, lanes off multiples of 64,
    # sequence lengths off multiples of the 32-step chunk
    (3, 50, 5000, 3),
    (2, 100, 3333, 4),
    (1, 70, 20000, 1),
    (5, 13, 4100, 2),
    (4, 20, 2000, 6),  # two-pass path (na > 4) with several chunks
]


def _np(t):
    return t.detach().cpu().numpy().astype(np.float64)


def _stable_poles(P, na, g):
    """Denominators with poles |p| in [0.5, 0.98] (conjugate pairs plus a real pole when odd)."""
    rows = []
    for _ in range(P):
        poles = []
        while len(poles) < na:
            r = 0.5 + 0.48 * torch.rand(1, generator=g).item()
            if na - len(poles) >= 2:
                th = np.pi * torch.rand(1, generator=g).item()
                poles += [r * np.exp(1j * th), r * np.exp(-1j * th)]
            else:
                poles.append(r * (1 if torch.rand(1, generator=g).item() < 0.5 else -1))
        rows.append(np.real(np.poly(poles))[1:])
    return torch.tensor(np.array(rows), dtype=torch.float32)


@pytest.mark.parametrize("B,P,L,na", _SHAPES)
@pytest.mark.parametrize("with_y0", [True, False])
def test_allpole_matches_oracle(gpu, B, P, L, na, with_y0):
    g = torch.Generator().manual_seed(B * L + na)
    a = _stable_poles(P, na, g)  # per pair, broadcast over the batch
    w = torch.randn(B, P, L, generator=g)
    y0 = torch.randn(B, P, na, generator=g) if with_y0 else None
    gout = torch.randn(B, P, L, generator=g)
    a_d, w_d = a.to(gpu).requires_grad_(), w.to(gpu).requires_grad_()
    y0_d = y0.to(gpu).requires_grad_() if y0 is not None else None
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("dynonet.allpole", dcore._ALLPOLE_BACKENDS, ("hip",), (a_d, w_d, y0_d)) is allpole_hip
        y = dcore.allpole(a_d, w_d, y0_d)
        y.backward(gout.to(gpu))
    lanes = B * P
    a_l = _np(a.expand(B, P, na).reshape(lanes, na))
    y0_l = None if y0 is None else _np(y0.reshape(lanes, na))
    want = O.allpole_forward(a_l, _np(w.reshape(lanes, L)), y0_l)
    ga, gw, gy0 = O.allpole_backward(_np(gout.reshape(lanes, L)), a_l, want, y0_l)
    assert O.rel_err(_np(y).reshape(lanes, L), want) < TOL
    assert O.rel_err(_np(w_d.grad).reshape(lanes, L), gw) < TOL
    assert O.rel_err(_np(a_d.grad), ga.reshape(B, P, na).sum(0)) < TOL
    if y0 is not None:
        assert O.rel_err(_np(y0_d.grad).reshape(lanes, na), gy0) < TOL


def test_allpole_chunked_state_shorter_than_na(gpu):
    """Chunked filtering with chunks shorter than na equals one pass (newest-first y0 carry)."""
    g = torch.Generator().manual_seed(0)
    lanes, L, na = 6, 23, 5
    a = (_stable_poles(lanes, na, g)).to(gpu)
    w = torch.randn(lanes, L, generator=g).to(gpu)
    with torch.no_grad():
        full = allpole_hip.run(a, w, None)
        y0 = None
        parts = []
        for lo, hi in ((0, 2), (2, 3), (3, 11), (11, 23)):
            y = allpole_hip.run(a, w[:, lo:hi].contiguous(), y0)
            parts.append(y)
            n = hi - lo
            prev = y0 if y0 is not None else torch.zeros(lanes, na, device=gpu)
            y0 = y.flip(-1)[:, :na] if n >= na else torch.cat((y.flip(-1), prev[:, : na - n]), -1)
    assert O.rel_err(_np(torch.cat(parts, -1)), _np(full)) < TOL


def _ref_draw(P, na, g, L):
    """The reference suite's coefficients, a = 0.25 N(0, 1) per pair
    (tests/test_scan_allpole_backend.py:61). On sequences longer than 600 steps a pair whose
    filter has a pole at radius >= 0.999 is drawn again, so the outputs stay finite in fp32."""
    rows = []
    for _ in range(P):
        while True:
            a = torch.randn(na, generator=g) * 0.25
            if L <= 600 or np.max(np.abs(np.roots(np.r_[1.0, a.double().numpy()]))) < 0.999:
                break
        rows.append(a)
    return torch.stack(rows)


@pytest.mark.parametrize(
    "B,P,L,na",
    [
        (32, 8, 200, 2), (4, 32, 100, 8), (3, 5, 7, 3), (2, 4, 1, 2), (2, 4, 2, 4), (1, 1, 513, 1),
        (2, 3, 60, 16),
        (3, 50, 5000, 3), (2, 100, 3333, 4), (1, 70, 20000, 1), (5, 13, 4100, 2), (4, 20, 2000, 6),
    ],
)
@pytest.mark.parametrize("with_y0", [True, False])
def test_allpole_reference_coefficient_draws(gpu, B, P, L, na, with_y0):
    """The reference's coefficient draws (not constructed stable poles) on its own shapes and on
    the look-back and two-pass paths."""
    g = torch.Generator().manual_seed(7 * B * L + na)
    a = _ref_draw(P, na, g, L)
    w = torch.randn(B, P, L, generator=g)
    y0 = torch.randn(B, P, na, generator=g) if with_y0 else None
    gout = torch.randn(B, P, L, generator=g)
    a_d, w_d = a.to(gpu).requires_grad_(), w.to(gpu).requires_grad_()
    y0_d = y0.to(gpu).requires_grad_() if y0 is not None else None
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("dynonet.allpole", dcore._ALLPOLE_BACKENDS, ("hip",), (a_d, w_d, y0_d)) is allpole_hip
        y = dcore.allpole(a_d, w_d, y0_d)
        y.backward(gout.to(gpu))
    lanes = B * P
    a_l = _np(a.expand(B, P, na).reshape(lanes, na))
    y0_l = None if y0 is None else _np(y0.reshape(lanes, na))
    want = O.allpole_forward(a_l, _np(w.reshape(lanes, L)), y0_l)
    ga, gw, gy0 = O.allpole_backward(_np(gout.reshape(lanes, L)), a_l, want, y0_l)
    assert np.isfinite(want).all()
    assert O.rel_err(_np(y).reshape(lanes, L), want) < TOL, "y"
    assert O.rel_err(_np(w_d.grad).reshape(lanes, L), gw) < TOL, "gw"
    assert O.rel_err(_np(a_d.grad), ga.reshape(B, P, na).sum(0)) < TOL, "ga"
    if y0 is not None:
        assert O.rel_err(_np(y0_d.grad).reshape(lanes, na), gy0) < TOL, "gy0"


def test_allpole_long_chunks_square_the_transfer(gpu):
    """A sequence of more than 65535 x 256 steps takes all-pole chunks longer than 256 steps (one
    grid row per chunk), whose transfer matrix is C^256 squared up (allpole_transfer) rather than
    stepped column by column: one lane, na 5, against scipy's lfilter (the textbook form the
    oracle is pinned to) for y and the adjoint G = the same filter run backwards, with
    grad a_i = -sum_t G_t y_{t-i} and grad w = G."""
    from scipy.signal import lfilter

    g = torch.Generator().manual_seed(17)
    L, na = 65535 * 256 + 4097, 5
    a = _stable_poles(1, na, g)
    w = torch.randn(1, L, generator=g)
    gy = torch.randn(1, L, generator=g)
    ag, wg = a.to(gpu).requires_grad_(), w.to(gpu).requires_grad_()
    y = allpole_hip.run(ag, wg, None)
    y.backward(gy.to(gpu))
    den = np.concatenate(([1.0], a[0].double().numpy()))
    y_ref = lfilter([1.0], den, w[0].double().numpy())
    G = lfilter([1.0], den, gy[0].double().numpy()[::-1])[::-1]
    ga_ref = np.array([-(G[i:] * y_ref[: L - i]).sum() for i in range(1, na + 1)])
    assert O.rel_err(_np(y)[0], y_ref) < TOL
    assert O.rel_err(_np(wg.grad)[0], G) < TOL
    assert O.rel_err(_np(ag.grad)[0], ga_ref) < TOL
