"""The projected scan's wide route on the CPU: its GEMM packing and hand-written backward.

Beyond the fused kernel's widths, ``projected_hip`` runs ``complex_in_proj -> diagonal_recurrence
-> real_out_proj`` (tsfast/models/_core/scan.py:221-243, 272-313) as one real GEMM per projection
around the diagonal scan kernels, with the weight gradients as split-K batched products. Here the
diagonal scan kernels are replaced by the fp64 oracle's scan (cast to complex64), so the test
pins everything the route adds around them against the oracle's composition: the interleaved
weight layouts, torch's complex gradient convention through the real views, the returned state's
gradient, the per-row grad lam sum and the split-K sums. The kernels themselves are pinned by the
GPU tests.
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd.scan_backends import projected_hip


class _OracleScan:
    """Stand-in for ``diagonal_hip`` with the oracle's scans, in complex64 like the kernels."""

    @staticmethod
    def forward(lam, v, x0):
        out = O.diag_forward(lam.numpy(), v.numpy(), None if x0 is None else x0.numpy())
        return torch.from_numpy(out.astype(np.complex64))

    @staticmethod
    def backward(g, lam, out, x0):
        glam, gv, gx0 = O.diag_backward(g.numpy(), lam.numpy(), out.numpy(), None if x0 is None else x0.numpy())
        c64 = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.complex64))
        return c64(glam), c64(gv), (c64(gx0) if gx0 is not None else lam.new_empty(0))


@pytest.fixture
def oracle_scan(monkeypatch):
    monkeypatch.setattr(projected_hip, "diagonal_hip", _OracleScan)


def _make(B, L, H, N, O_, seed):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, L, H, generator=g)
    W_re, W_im = torch.randn(N, H, generator=g) / np.sqrt(H), torch.randn(N, H, generator=g) / np.sqrt(H)
    lam = torch.polar(torch.rand(N, generator=g) * 0.099 + 0.9, torch.rand(N, generator=g) * (np.pi / 10))
    C_re, C_im = torch.randn(O_, N, generator=g) / np.sqrt(N), torch.randn(O_, N, generator=g) / np.sqrt(N)
    x0 = torch.randn(B, N, dtype=torch.complex64, generator=g)
    gy = torch.randn(B, L, O_, generator=g)
    g_xl = torch.randn(B, N, dtype=torch.complex64, generator=g)
    return u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl


@pytest.mark.parametrize("K", [1, 100, 4096 * 2 - 1, 4096 * 2, 4096 * 3 + 7, 4096 * 20 + 5])
def test_gram_is_the_plain_product(K):
    """Split-K sums (up to 16 row blocks and a remainder) equal a^T b."""
    g = torch.Generator().manual_seed(K)
    a = torch.randn(K, 24, generator=g, dtype=torch.float64)
    b = torch.randn(K, 10, generator=g, dtype=torch.float64)
    got = projected_hip._gram(a, b)
    want = a.numpy().T @ b.numpy()
    assert got.shape == (24, 10)
    assert np.abs(got.numpy() - want).max() <= 1e-12 * max(1.0, np.abs(want).max()) * np.sqrt(K)


def test_weight_layouts():
    """u @ w^T is the interleaved (re, im) layout of u W^T; view_as_real(x) @ c^T = Re(x C^T)."""
    u, W_re, W_im, _, C_re, C_im, *_ = _make(2, 5, 3, 4, 6, seed=1)
    v = torch.view_as_complex((u @ projected_hip._w_cat(W_re, W_im).T).view(2, 5, 4, 2))
    assert O.rel_err(v.numpy(), O.complex_in_proj(u.numpy(), W_re.numpy(), W_im.numpy())) < 1e-6
    x = torch.randn(2, 5, 4, dtype=torch.complex64)
    y = torch.view_as_real(x).reshape(2, 5, 8) @ projected_hip._c_cat(C_re, C_im).T
    assert O.rel_err(y.numpy(), O.real_out_proj(x.numpy(), C_re.numpy(), C_im.numpy())) < 1e-6


@pytest.mark.parametrize(
    "shape", [(2, 7, 3, 4, 2), (3, 50, 40, 33, 36), (1, 4096 * 2 + 3, 5, 6, 4), (1, 9, 1, 1, 1), (2, 5, 3, 1, 2)]
)
@pytest.mark.parametrize("with_x0", [True, False])
@pytest.mark.parametrize("with_gxl", [True, False])
def test_wide_route_matches_oracle(oracle_scan, shape, with_x0, with_gxl):
    u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl = _make(*shape, seed=sum(shape))
    x0 = x0 if with_x0 else None
    g_xl = g_xl if with_gxl else None
    y, x_last, x = projected_hip._wide_forward(u, W_re, W_im, lam, C_re, C_im, x0)
    want_y, want_x = O.projscan_forward(*(t.numpy() if t is not None else None for t in (u, W_re, W_im, lam, C_re, C_im, x0)))
    assert O.rel_err(y.numpy(), want_y) < 1e-5
    assert O.rel_err(x_last.numpy(), want_x[:, -1]) < 1e-5
    got = projected_hip._wide_backward(gy, g_xl, x, u, W_re, W_im, lam, C_re, C_im, x0)
    want = O.projscan_backward(
        gy.numpy(), None if g_xl is None else g_xl.numpy(), u.numpy(), W_re.numpy(), W_im.numpy(), lam.numpy(),
        C_re.numpy(), C_im.numpy(), want_x, None if x0 is None else x0.numpy(),
    )
    names = ("g_u", "g_W_re", "g_W_im", "g_lam", "g_C_re", "g_C_im", "g_x0")
    storages = [gg.untyped_storage().data_ptr() for gg in (y, x_last, x) + tuple(got) if gg.numel() > 0]
    assert len(set(storages)) == len(storages), "outputs share memory"
    for name, gg, gw in zip(names, got, want):
        if gw is None:
            assert gg.numel() == 0, name
            continue
        assert tuple(gg.shape) == gw.shape, name
        assert O.rel_err(gg.numpy(), gw) < 1e-5, name


def test_wide_route_empty_sequence(oracle_scan):
    """L = 0: y is empty, the returned state is x0, x0's gradient is the state's gradient."""
    u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl = _make(2, 0, 4, 8, 3, seed=9)
    y, x_last, x = projected_hip._wide_forward(u, W_re, W_im, lam, C_re, C_im, x0)
    assert y.shape == (2, 0, 3) and torch.equal(x_last, x0)
    grads = projected_hip._wide_backward(gy, g_xl, x, u, W_re, W_im, lam, C_re, C_im, x0)
    assert torch.equal(grads[6], g_xl)
    assert all(not t.any() for t in grads[1:6])


@pytest.mark.parametrize("with_x0", [True, False])
def test_deterministic_backward_matches_oracle(oracle_scan, with_x0):
    """The backward used under torch.use_deterministic_algorithms recomputes the states with the
    wide route and runs its backward: the same seven gradients as the oracle's."""
    u, W_re, W_im, lam, C_re, C_im, x0, gy, g_xl = _make(2, 37, 6, 10, 5, seed=4)
    x0 = x0 if with_x0 else None
    got = projected_hip._deterministic_bwd(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x0)
    _, want_x = O.projscan_forward(*(t.numpy() if t is not None else None for t in (u, W_re, W_im, lam, C_re, C_im, x0)))
    want = O.projscan_backward(
        gy.numpy(), g_xl.numpy(), u.numpy(), W_re.numpy(), W_im.numpy(), lam.numpy(), C_re.numpy(), C_im.numpy(),
        want_x, None if x0 is None else x0.numpy(),
    )
    for name, gg, gw in zip(("g_u", "g_W_re", "g_W_im", "g_lam", "g_C_re", "g_C_im", "g_x0"), got, want):
        if gw is None:
            assert gg.numel() == 0, name
        else:
            assert O.rel_err(gg.numpy(), gw) < 1e-5, name
