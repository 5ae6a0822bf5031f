"""GPU parity: the fused dynoNet G-block (FIR + all-pole + input sum) vs the fp64 oracle.

The oracle (oracle/scan_oracle.py::gblock_forward/backward) is pinned against float64 autograd
through the reference's own formulation (grouped conv1d, a sequential all-pole loop, the sum
over inputs; tests/test_oracle.py). Shapes cover every tap padding of the fused kernels (nb 1..16 -> 2, 4, 8, 16; 9..16 taps through
the op itself, since the operator stages them),
every order na 1..4, pair counts that divide 64 (64 / (I*O) batch rows per tile) and that do
not (a batch row padded to the next power of two: 3, 15, 24 and 40 pairs), more than 64 pairs
(run as groups of inputs, and of outputs past 64), sequences shorter than na and than one chunk,
many super-chunks, and absent initial state; orders 5..16 (and 17..64 taps) through the staged
path (this library's FIR op, the all-pole op on the pair lanes, the sum over inputs). Bar: max relative
error <= 1e-5 for outputs, the returned state and every gradient (fp32 I/O, fp64 state).
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import dispatch
from tsfast_amd.dynonet import core as dcore
from tsfast_amd.dynonet import gblock_hip

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _np(t):
    return None if t is None else t.detach().cpu().numpy().astype(np.float64)


def _make(B, L, I, O_, nb, na, seed, with_state=True):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, L, I, generator=g)
    b = torch.randn(O_, I, nb, generator=g) * (0.5 / nb)
    # stable denominators: poles inside 0.9 of the unit circle, scaled per pair
    a = torch.empty(O_, I, na)
    for o in range(O_):
        for j in range(I):
            r = torch.rand(na, generator=g).double().numpy() * 0.9
            sgn = np.sign(torch.rand(na, generator=g).numpy() - 0.5)
            # high orders: real poles this clustered move under the fp32 rounding of the
            # coefficients; pull them inwards until the rounded filter has spectral radius < 0.95
            for _ in range(60):
                ai = np.poly(r * sgn)[1:].astype(np.float32)
                cm = np.eye(na, k=-1)
                cm[0] = -ai.astype(np.float64)
                if na == 1 or np.abs(np.linalg.eigvals(cm)).max() < 0.95:
                    break
                r = r * 0.95
            a[o, j] = torch.tensor(ai, dtype=torch.float32)
    ut = torch.randn(B, nb - 1, I, generator=g) if with_state else None
    x0 = torch.randn(B, I * O_, na, generator=g) if with_state else None
    gy = torch.randn(B, L, O_, generator=g)
    gxl = torch.randn(B, I * O_, na, generator=g)
    return u, b, a, ut, x0, gy, gxl


# (B, L, I, O, nb, na)
_SHAPES = [
    (2, 100, 8, 8, 8, 3),  # 64 pairs: one batch row per tile
    (4, 300, 2, 4, 4, 2),
    (3, 77, 1, 1, 1, 1),  # 1 pair: 64 batch rows per tile, mostly idle lanes
    (2, 5000, 4, 4, 16, 4),  # 16 taps, many super-chunks
    (1, 2, 2, 2, 3, 4),  # L < na
    (2, 1, 8, 8, 8, 2),  # L = 1
    (5, 1000, 2, 2, 5, 1),
    (6, 2049, 1, 8, 2, 3),
    (4, 4096, 8, 8, 8, 3),  # config-4 channel structure, reduced batch and length
    # lanes beyond one tile, not a multiple of 64: the second tile holds a partial lane group
    # whose pairs (lane % P) repeat the first tile's (coefficients and transfer matrices staged once)
    (5, 700, 4, 4, 8, 3),  # 80 lanes, matrices in LDS
    (9, 500, 2, 4, 4, 4),  # 72 lanes, na 4: matrices read from global memory
    # pair counts that do not divide 64: each batch row padded to the next power of two
    (3, 900, 3, 8, 8, 2),  # 24 pairs (DynoNet(input_size=3)'s first block): 32 lanes per row
    (4, 600, 8, 3, 8, 2),  # 24 pairs, input-major with 3 outputs
    (5, 700, 5, 3, 6, 3),  # 15 pairs: 80 lanes, a partial second tile
    (7, 333, 3, 1, 4, 4),  # 3 pairs, na 4
    (3, 500, 5, 8, 8, 3),  # 40 pairs: 24 idle lanes per row
    (2, 5000, 3, 5, 16, 4),  # 15 pairs, 16 taps, many super-chunks
    # more than 64 pairs: groups of inputs (and of outputs past 64 outputs)
    (2, 400, 9, 8, 8, 2),  # 72 pairs: inputs 0..7 and 8
    (2, 300, 2, 70, 4, 1),  # 140 pairs: 64 + 6 outputs, one input per group
    # staged path: orders above the fused kernels', taps above 16
    (3, 700, 3, 8, 8, 6),  # 24 pairs, na 6
    (2, 1500, 2, 4, 8, 8),  # na 8
    (4, 600, 1, 1, 1, 16),  # na 16, a single tap
    (2, 300, 4, 4, 20, 5),  # 20 taps (above the fused kernels' 16)
    (2, 3, 2, 2, 3, 8),  # L < na
    (2, 5000, 8, 8, 8, 7),  # 64 pairs, many FIR tiles and all-pole chunks
    (2, 400, 9, 8, 8, 6),  # 72 pairs in one call (no grouping on this path)
    (3, 257, 2, 3, 64, 5),  # 64 taps, a ragged second FIR tile
    (2, 2051, 2, 12, 12, 6),  # 12 outputs: two FIR channel blocks (8 + 4); 12 taps padded to 16; 3 FIR tiles
    (1, 1030, 3, 9, 32, 5),  # 9 outputs (8 + 1), 32 taps, a 6-step last FIR tile, L % 4 = 2
]


@pytest.mark.parametrize("with_state", [True, False])
@pytest.mark.parametrize("shape", _SHAPES)
def test_gblock_matches_oracle(gpu, shape, with_state):
    _check_against_oracle(gpu, shape, with_state, gblock_hip.run)


# 9..16 taps take the staged path in gblock_hip.run (faster there than the fused kernels' 16-tap
# instances); C callers reach the fused kernels with them, so they are checked through the op
@pytest.mark.parametrize("with_state", [True, False])
@pytest.mark.parametrize("shape", [(2, 5000, 4, 4, 16, 4), (2, 5000, 3, 5, 16, 4), (3, 700, 2, 4, 12, 3)])
def test_gblock_fused_kernel_wide_taps_matches_oracle(gpu, shape, with_state):
    assert not gblock_hip._fused(shape[5], shape[4])
    _check_against_oracle(gpu, shape, with_state, lambda *ts: gblock_hip._gblock_op(*ts)[:2])


def _check_against_oracle(gpu, shape, with_state, call):
    B, L, I, O_, nb, na = shape
    u, b, a, ut, x0, gy, gxl = _make(*shape, seed=sum(shape), with_state=with_state)
    ts = [t.to(gpu).requires_grad_() if t is not None else None for t in (u, b, a, ut, x0)]
    assert gblock_hip.supports(*ts) is None
    y, x_last = call(*ts)
    torch.autograd.backward([y, x_last], [gy.to(gpu), gxl.to(gpu)])
    z = lambda t, shp: np.zeros(shp) if t is None else _np(t)  # noqa: E731
    args = (_np(u), _np(b), _np(a), z(ut, (B, nb - 1, I)), z(x0, (B, I * O_, na)))
    want_y, want_xl, _ = O.gblock_forward(*args)
    assert O.rel_err(_np(y), want_y) < TOL, "y"
    assert O.rel_err(_np(x_last), want_xl) < TOL, "x_last"
    gu, gut, gb, ga, gx0 = O.gblock_backward(_np(gy), _np(gxl), *args)
    assert O.rel_err(_np(ts[0].grad), gu) < TOL, "gu"
    assert O.rel_err(_np(ts[1].grad), gb) < TOL, "gb"
    assert O.rel_err(_np(ts[2].grad), ga) < TOL, "ga"
    if with_state:
        if nb > 1:
            assert O.rel_err(_np(ts[3].grad), gut) < TOL, "gu_tail"
        assert O.rel_err(_np(ts[4].grad), gx0) < TOL, "gx0"


@pytest.mark.parametrize("na", [2, 6])
def test_gblock_operator_dispatch_and_chunked_state(gpu, na):
    """linear_dynamical_operator picks the hip G-block (fused kernels at na 2, the staged path at
    na 6), and two chunks with the carried state ({"u": FIR tail, "x": IIR state}) equal one pass
    over the whole sequence."""
    B, L, I, O_, nb = 3, 700, 4, 2, 6
    u, b, a, _, _, _, _ = _make(B, L, I, O_, nb, na, seed=9)
    u, b, a = u.to(gpu), b.to(gpu), a.to(gpu)
    with dispatch.use_backend("hip"):
        zeros = (u.new_zeros(B, nb - 1, I), u.new_zeros(B, I * O_, na))
        assert dispatch.resolve("dynonet.gblock", dcore._GBLOCK_BACKENDS, ("hip",), (u, b, a, *zeros)) is gblock_hip
        full, st_full = dcore.linear_dynamical_operator(u, b, a, return_state=True)
        y1, st = dcore.linear_dynamical_operator(u[:, :333], b, a, return_state=True)
        y2, st2 = dcore.linear_dynamical_operator(u[:, 333:], b, a, state=st, return_state=True)
    chunked = torch.cat((y1, y2), 1)
    want, want_xl, _ = O.gblock_forward(_np(u), _np(b), _np(a), np.zeros((B, nb - 1, I)), np.zeros((B, I * O_, na)))
    assert O.rel_err(_np(full), want) < TOL
    assert O.rel_err(_np(chunked), want) < TOL
    assert O.rel_err(_np(st2["x"]), want_xl) < TOL
    assert torch.equal(st2["u"], st_full["u"])


def test_dynonet_default_blocks_take_the_fused_kernel(gpu):
    """DynoNet(input_size=3, output_size=2) builds G-blocks of 3 x 8, 8 x 2 and 3 x 2 pairs
    (dynonet/core.py:304-306): every one resolves to the fused kernel and matches the oracle."""
    for I, O_ in ((3, 8), (8, 2), (3, 2)):
        B, L, nb, na = 2, 500, 8, 2
        u, b, a, _, _, _, _ = _make(B, L, I, O_, nb, na, seed=I * 10 + O_)
        u, b, a = u.to(gpu), b.to(gpu), a.to(gpu)
        zeros = (u.new_zeros(B, nb - 1, I), u.new_zeros(B, I * O_, na))
        assert dispatch.resolve("dynonet.gblock", dcore._GBLOCK_BACKENDS, ("hip",), (u, b, a, *zeros)) is gblock_hip
        y = dcore.linear_dynamical_operator(u, b, a)
        want, _, _ = O.gblock_forward(_np(u), _np(b), _np(a), np.zeros((B, nb - 1, I)), np.zeros((B, I * O_, na)))
        assert O.rel_err(_np(y), want) < TOL


def test_gblock_matches_unfused_path(gpu):
    """The fused kernel and the reference's three-stage path (conv1d, all-pole op, sum) agree."""
    B, L, I, O_, nb, na = 4, 1500, 8, 8, 8, 3
    u, b, a, ut, x0, gy, _ = _make(B, L, I, O_, nb, na, seed=21)
    state = {"u": ut.to(gpu), "x": x0.to(gpu)}
    u, b, a = u.to(gpu), b.to(gpu), a.to(gpu)
    fused = dcore.linear_dynamical_operator(u, b, a, state=state)
    P = I * O_
    u_buf = torch.cat((state["u"], u), dim=1)
    w = torch.nn.functional.conv1d(u_buf.transpose(1, 2), b.permute(1, 0, 2).reshape(P, 1, nb).flip(-1), groups=I)
    y_pairs = dcore.allpole(a.permute(1, 0, 2).reshape(P, na).expand(B, P, na), w, state["x"])
    unfused = y_pairs.view(B, I, O_, L).sum(1).transpose(1, 2)
    assert O.rel_err(_np(fused), _np(unfused)) < TOL


def test_gblock_supports_reasons(gpu):
    u = torch.randn(2, 10, 3, device=gpu)
    b = torch.randn(5, 3, 4, device=gpu)
    a = torch.randn(5, 3, 2, device=gpu)
    assert gblock_hip.supports(u, b, a, None, None) is None  # 15 pairs
    assert "taps" in gblock_hip.supports(u, torch.randn(5, 3, 65, device=gpu), a, None, None)
    b2, a2 = torch.randn(2, 3, 4, device=gpu), torch.randn(2, 3, 17, device=gpu)
    assert "order" in gblock_hip.supports(u[..., :2], b2[:, :2], a2[:, :2], None, None)
    assert "GPU-only" in gblock_hip.supports(u.cpu(), b.cpu(), a.cpu(), None, None)
