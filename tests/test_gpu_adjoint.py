"""GPU parity: the chunked NSS adjoint scan (``tsfast_amd.ssm.adjoint_hip``, the HIP replacement
of backend_metal.py's ``ssm_bwd_summary`` + ``ssm_bwd_scan``) against the fp64 oracle.

Shapes cover every kernel instantiation (n <= 15, 16, 17..31, 32), ragged last chunks, one-step
chunks, a chunk longer than the sequence, the reference's largest scan batch (16) and its
largest state (32), the empty sequence, and the reference's own chunking for an NSS-sized
backward (B 16, L 4096, n 32: C = min(ceil(512 / B), L // 64) chunks). Step matrices are random
with spectral radius near 0.9, and near 1.05 for one long-chunk case (growth through the chunk
products). Bar: max relative error <= 1e-5.
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd.ssm import adjoint_hip

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _inputs(B, L, n, seed, radius=0.9):
    g = torch.Generator().manual_seed(seed)
    jt = torch.randn(B, L, n, n, generator=g) * (radius / n**0.5)
    gout = torch.randn(B, L, n, generator=g)
    return jt, gout


@pytest.mark.parametrize(
    "B,L,n,cl",
    [
        (1, 1, 1, 1),
        (2, 37, 3, 8),
        (3, 100, 15, 16),
        (2, 64, 16, 64),
        (4, 257, 17, 32),
        (2, 300, 31, 100),
        (16, 512, 32, 64),
        (5, 1000, 32, 128),
        (2, 50, 8, 1),
        (3, 40, 12, 200),
        (1, 4096, 32, 256),
        (2, 200, 7, 16),
        (2, 200, 20, 24),
    ],
)
def test_mat_adjoint_matches_oracle(gpu, B, L, n, cl):
    jt, gout = _inputs(B, L, n, seed=1000 * B + L + n)
    jd, gd = jt.to(gpu), gout.to(gpu)
    assert adjoint_hip.supports(jd, gd, cl) is None
    bnd = adjoint_hip.run(jd, gd, cl)
    want = O.mat_adjoint_bounds(jt.numpy(), gout.numpy(), cl)
    assert tuple(bnd.shape) == want.shape
    assert O.rel_err(bnd.cpu().numpy(), want) < TOL


def test_mat_adjoint_growing_products(gpu):
    """Spectral radius above one: the chunk products grow by orders of magnitude (fp64 inside)."""
    jt, gout = _inputs(2, 600, 10, seed=7, radius=1.05)
    bnd = adjoint_hip.run(jt.to(gpu), gout.to(gpu), 300)
    want = O.mat_adjoint_bounds(jt.numpy(), gout.numpy(), 300)
    assert O.rel_err(bnd.cpu().numpy(), want) < TOL


def test_mat_adjoint_reference_chunking_full_size(gpu):
    """An NSS-sized backward with the reference's own chunk count: B 16, L 4096, n 32."""
    B, L, n = 16, 4096, 32
    C = max(1, min(-(-512 // B), L // 64))
    cl = -(-L // C)
    jt, gout = _inputs(B, L, n, seed=11)
    bnd = adjoint_hip.run(jt.to(gpu), gout.to(gpu), cl)
    rows = [0, 15]  # the oracle on two rows (rows are independent)
    want = O.mat_adjoint_bounds(jt[rows].numpy(), gout[rows].numpy(), cl)
    assert O.rel_err(bnd[rows].cpu().numpy(), want) < TOL


def test_mat_adjoint_empty_and_unsupported(gpu):
    jt, gout = torch.zeros(3, 0, 4, 4, device=gpu), torch.zeros(3, 0, 4, device=gpu)
    bnd = adjoint_hip.run(jt, gout, 8)
    assert tuple(bnd.shape) == (3, 1, 4) and not bnd.any()
    big = torch.zeros(1, 4, 33, 33, device=gpu), torch.zeros(1, 4, 33, device=gpu)
    assert "n=33" in adjoint_hip.supports(*big, 2)
    assert "float32" in adjoint_hip.supports(jt.double(), gout.double(), 2)


def test_mat_adjoint_matches_step_by_step_adjoint(gpu):
    """The boundaries equal the adjoint computed step by step (torch float64 loop, independent of
    the oracle's chunk summaries)."""
    B, L, n, cl = 3, 90, 7, 16
    jt, gout = _inputs(B, L, n, seed=5)
    j64, g64 = jt.double(), gout.double()
    gy = torch.zeros(B, L, n, dtype=torch.float64)
    nxt = torch.zeros(B, n, dtype=torch.float64)
    for t in range(L - 1, -1, -1):
        gy[:, t] = g64[:, t] + (torch.einsum("bij,bj->bi", j64[:, t + 1], nxt) if t + 1 < L else 0.0)
        nxt = gy[:, t]
    bnd = adjoint_hip.run(jt.to(gpu), gout.to(gpu), cl).cpu().double()
    C = -(-L // cl)
    assert O.rel_err(bnd[:, :C].numpy(), gy[:, ::cl].numpy()) < TOL
    assert not bnd[:, C].any()
