"""GPU parity of the look-back scans in the fast mode (reproducibility off: a tile composes the
published maps back to the nearest finished tile).

The library's default is the reproducible mode (anchored publication), in which the other parity
modules run. This module re-runs their oracle comparisons for the diagonal, selective, all-pole,
linear-recurrence, G-block and projected scans with ``tsfast_amd.set_reproducible(False)``, so
both publication schemes meet the same bars (the comparison functions, shapes and tolerances are
the other modules' own).
"""

import pytest
from test_gpu_allpole import test_allpole_matches_oracle, test_allpole_reference_coefficient_draws  # noqa: F401
from test_gpu_gblock import test_gblock_matches_oracle  # noqa: F401
from test_gpu_linrec import test_linrec_matches_oracle  # noqa: F401
from test_gpu_projscan import test_projscan_matches_oracle  # noqa: F401
from test_gpu_scan import (  # noqa: F401
    test_diag_matches_oracle,
    test_diag_reference_coefficient_draws,
    test_selective_matches_oracle,
    test_tbptt_chunked_equals_unchunked,
)

from tsfast_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fast_mode():
    prev = _lib.set_reproducible(False)
    try:
        yield
    finally:
        _lib.set_reproducible(prev)


def test_fast_mode_is_selected(gpu):
    import torch

    from tsfast_amd.scan_backends import diagonal_hip

    lam = torch.full((4, 8), 0.9, device=gpu)
    diagonal_hip.forward(lam, torch.randn(4, 100, 8, device=gpu), None)
    assert _lib.load().tsfast_hip_get_deterministic() == 0
