"""GPU parity: the constant-matrix linear recurrence x_t = A x_{t-1} + v_t vs the fp64 oracle.

The oracle (oracle/scan_oracle.py::linrec_forward/backward) is pinned against matrix-power
closed forms, torch float64 autograd through a sequential loop, and the diagonal-scan and
all-pole special cases (tests/test_oracle.py). Shapes cover every state size n = 1..4 (chunks of
32, 16, 10 and 8 steps), lane counts below, at and above one 64-lane tile row, sequences shorter
than one chunk and than one super-chunk, ragged tails, many super-chunks (the look-back), and
absent initial state; n = 5..8 (the two-pass path, blocks of 256 lanes) with one and many
256-step chunks, ragged last chunks, and several lane blocks combined with several chunks; n =
9..16 (the spread two-pass path: a 16-thread group per lane and chunk, state components beyond n
padded) with lane counts below, at and above one 16-group workgroup, one and many chunks and
ragged tails. Bar: max relative error <= 1e-5 for x and every gradient (fp32 I/O, fp64 state). Matrices are scaled to spectral radius 0.97 so the states neither vanish nor blow up.
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import dispatch
from tsfast_amd.dynonet import core as dcore
from tsfast_amd.dynonet import linrec_hip

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _np(t):
    return None if t is None else t.detach().cpu().numpy().astype(np.float64)


def _make(M, L, n, seed, with_x0=True, radius=0.97):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(M, n, n, generator=g, dtype=torch.float64)
    rho = torch.linalg.eigvals(A).abs().amax(-1).clamp_min(1e-6)
    A = (A * (radius / rho)[:, None, None]).float()
    v = torch.randn(M, L, n, generator=g)
    x0 = torch.randn(M, n, generator=g) if with_x0 else None
    gx = torch.randn(M, L, n, generator=g)
    return A, v, x0, gx


# (M lanes, L, n)
_SHAPES = [
    (5, 40, 1),
    (64, 1000, 2),
    (70, 333, 3),  # two tile rows, the second almost empty
    (3, 7, 4),  # shorter than one 8-step chunk
    (130, 4099, 4),  # ragged last chunk, many super-chunks
    (200, 2000, 3),
    (1, 20000, 1),  # one lane, a long look-back chain
    (33, 1, 2),  # L = 1
    (96, 5000, 2),
    # n = 5..8: the two-pass path (chunks of 256 steps)
    (5, 40, 5),
    (70, 1000, 6),  # ragged last chunk, one lane block (256 lanes per block)
    (130, 777, 7),
    (64, 600, 8),
    (3, 1, 8),
    (1, 5000, 5),  # one lane, 20 chunks of carry
    (300, 256, 6),  # exactly one chunk, two lane blocks
    (600, 3000, 8),  # three lane blocks (the last partial) x twelve chunks (the last ragged)
    (520, 1500, 5),  # three lane blocks x six chunks
    # chunks that end off a prefetch block (4 steps) and off an output sub-block: the remainder
    # after the whole blocks, and chunk 0's guarded re-run with x0 at step 0
    (9, 263, 8),  # a 7-step second chunk
    (4, 5, 6),  # one 5-step chunk, shorter than a sub-block
    (2, 514, 7),  # odd n, a 2-step third chunk
    # n = 9..16: spread path (16 lanes of a workgroup, one 16-thread group each)
    (5, 40, 9),
    (33, 1000, 12),  # three lane groups (the last with one lane), ragged last chunk
    (17, 777, 16),
    (3, 1, 16),  # L = 1
    (1, 5000, 11),  # one lane, 20 chunks of carry
    (40, 600, 13),
    (20, 256, 10),  # exactly one chunk
    (16, 2000, 15),  # exactly one workgroup of lanes
    (6, 262, 12),  # a 6-step second chunk, shorter than one 8-step prefetch block
    (5, 1283, 16),  # a 3-step last chunk after five whole ones
]


@pytest.mark.parametrize("with_x0", [True, False])
@pytest.mark.parametrize("shape", _SHAPES)
def test_linrec_matches_oracle(gpu, shape, with_x0):
    M, L, n = shape
    A, v, x0, gx = _make(M, L, n, seed=sum(shape), with_x0=with_x0)
    ts = [t.to(gpu).requires_grad_() if t is not None else None for t in (A, v, x0)]
    assert linrec_hip.supports(*ts) is None
    x = linrec_hip.run(*ts)
    want = O.linrec_forward(_np(A), _np(v), _np(x0))
    assert O.rel_err(_np(x), want) < TOL, "x"
    x.backward(gx.to(gpu))
    gA, gv, gx0 = O.linrec_backward(_np(gx), _np(A), want, _np(x0))
    assert O.rel_err(_np(ts[0].grad), gA) < TOL, "gA"
    assert O.rel_err(_np(ts[1].grad), gv) < TOL, "gv"
    if with_x0:
        assert O.rel_err(_np(ts[2].grad), gx0) < TOL, "gx0"


@pytest.mark.parametrize("n", [3, 6, 12])
def test_linrec_empty_sequence(gpu, n):
    A, _, x0, _ = _make(4, 1, n, seed=3)
    A, x0 = A.to(gpu).requires_grad_(), x0.to(gpu).requires_grad_()
    v = torch.zeros(4, 0, n, device=gpu, requires_grad=True)
    x = linrec_hip.run(A, v, x0)
    assert x.shape == (4, 0, n)
    x.sum().backward()
    assert torch.count_nonzero(A.grad) == 0 and torch.count_nonzero(x0.grad) == 0


def test_linrec_dispatch_broadcast_and_doubling_scan(gpu):
    """linear_recurrence picks the hip backend; a shared A broadcast over the batch gets its
    gradient summed over lanes; the result equals the reference's log-doubling scan op."""
    B, P, L, n = 3, 4, 777, 3
    A, v, x0, gx = _make(P, L, n, seed=5)
    A = A.to(gpu).requires_grad_()
    v = v.to(gpu)[None].expand(B, P, L, n).contiguous().requires_grad_()
    x0 = x0.to(gpu)
    gx = gx.to(gpu)[None].expand(B, P, L, n)
    with dispatch.use_backend("hip"):
        A_b = A.broadcast_to(B, P, n, n)
        assert dispatch.resolve("dynonet.linear_recurrence", dcore._LINREC_BACKENDS, ("hip",),
                                (A_b, v, x0.broadcast_to(B, P, n))) is linrec_hip
        x = dcore.linear_recurrence(A, v, x0)
    (gA_hip,) = torch.autograd.grad(x, A, gx)
    with dispatch.use_backend("reference"):
        A64 = A.detach().double().requires_grad_()
        x_ref = dcore.linear_recurrence(A64, v.detach().double(), x0.double())
        (gA_ref,) = torch.autograd.grad(x_ref, A64, gx.double())
    assert O.rel_err(_np(x), _np(x_ref)) < TOL
    assert O.rel_err(_np(gA_hip), _np(gA_ref)) < TOL


@pytest.mark.parametrize("na", [3, 6, 12, 16])
def test_linrec_companion_is_allpole(gpu, na):
    """Companion matrices with input (w_t, 0, ..) give the all-pole filter (the reference's CPU
    route for dynoNet, allpole via linear_recurrence), matching the fused all-pole kernel."""
    lanes, L = 100, 3000
    g = torch.Generator().manual_seed(8)
    r = torch.rand(lanes, na, generator=g).double().numpy() * 0.9
    rows = []
    for ri in r:
        # high orders: real poles this clustered move under the fp32 rounding of the coefficients;
        # pull them inwards until the rounded filter has spectral radius below 0.95
        for _ in range(60):
            ai = np.poly(ri)[1:].astype(np.float32)
            cm = np.eye(na, k=-1)
            cm[0] = -ai.astype(np.float64)
            if np.abs(np.linalg.eigvals(cm)).max() < 0.95:
                break
            ri = ri * 0.95
        rows.append(ai)
    a = torch.tensor(np.array(rows), dtype=torch.float32).to(gpu)
    w = torch.randn(lanes, L, generator=g).to(gpu)
    y0 = torch.randn(lanes, na, generator=g).to(gpu)
    v = torch.nn.functional.pad(w.unsqueeze(-1), (0, na - 1))
    x = linrec_hip.run(dcore.companion(a).contiguous(), v, y0)
    y = dcore.allpole(a, w, y0)
    assert O.rel_err(_np(x[..., 0]), _np(y)) < TOL


def test_linrec_supports_reasons(gpu):
    A = torch.randn(2, 17, 17, device=gpu)
    v = torch.randn(2, 10, 17, device=gpu)
    assert "state size" in linrec_hip.supports(A, v, None)
    assert linrec_hip.supports(A[:, :16, :16], v[..., :16], None) is None
    assert "GPU-only" in linrec_hip.supports(A[:, :2, :2].cpu(), v[..., :2].cpu(), None)
    assert "float32" in linrec_hip.supports(A[:, :2, :2].double(), v[..., :2].double(), None)


@pytest.mark.parametrize("n", [6, 8])
def test_linrec_wide_misaligned_rows(gpu, n):
    """n = 5..8 read and write whole steps as float4 / float2 when every row pointer allows it;
    inputs that start 4 bytes into a buffer take the per-float path and give the same result."""
    M, L = 40, 700
    A, v, x0, gx = _make(M, L, n, seed=11 + n)
    buf = torch.empty(1 + M * L * n, device=gpu)
    v_mis = buf[1:].view(M, L, n)
    v_mis.copy_(v.to(gpu))
    assert v_mis.data_ptr() % 8 != 0
    ts = [A.to(gpu).requires_grad_(), v_mis.requires_grad_(), x0.to(gpu).requires_grad_()]
    x = linrec_hip.run(*ts)
    want = O.linrec_forward(_np(A), _np(v), _np(x0))
    assert O.rel_err(_np(x), want) < TOL
    gbuf = torch.empty(1 + M * L * n, device=gpu)
    g_mis = gbuf[1:].view(M, L, n)
    g_mis.copy_(gx.to(gpu))
    x.backward(g_mis)
    gA, gv, gx0 = O.linrec_backward(_np(gx), _np(A), want, _np(x0))
    assert O.rel_err(_np(ts[0].grad), gA) < TOL and O.rel_err(_np(ts[1].grad), gv) < TOL
    assert O.rel_err(_np(ts[2].grad), gx0) < TOL
