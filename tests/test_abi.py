"""The C ABI: libtsfast_hip.so loads on the CPU host and exports every symbol include/tsfast_hip.h
declares, and the size/status queries behave (no kernel is launched here)."""

import ctypes
import re
from pathlib import Path

import pytest

from tsfast_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "tsfast_hip.h").read_text()
    return sorted(set(re.findall(r"\b(tsfast_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.available():
        pytest.skip("libtsfast_hip.so not built (run __graft_entry__.build())")
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_loader_signatures_cover_the_header():
    assert sorted(_lib._SIGNATURES) == _declared()


def test_status_strings(lib):
    assert lib.tsfast_hip_status_string(0) == b"ok"
    assert b"workspace" in lib.tsfast_hip_status_string(-2)
    assert lib.tsfast_hip_version() >= 1


def test_whole_sequence_tiling_needs_only_the_header(lib):
    """Diagonal scans whose both directions fit one workgroup per lane group (whole-sequence
    tiles: no look-back words) need only the 256-byte header; any longer sequence needs the
    look-back words. Chunks are 64 real steps (complex: 32 forward, 16 backward); groups are
    64 lanes from 16384 lanes up (16 chunks), else 16 lanes (16 chunks; the forward alone may
    take 64 when 256 groups cover the lanes)."""
    ws = lib.tsfast_hip_diag_workspace_bytes
    assert ws(32, 1000, 64, 0) == 256  # config 1: 2048 lanes, 16 chunks
    assert ws(64, 1024, 256, 0) == 256  # 16384 lanes in 64-lane groups, 16 chunks
    assert ws(64, 1025, 256, 0) > 256  # 17 chunks
    assert ws(2, 1024, 64, 0) == 256 and ws(2, 1025, 64, 0) > 256
    assert ws(8, 4096, 128, 0) > 256  # config 5: the forward alone is whole-sequence
    assert ws(2, 256, 32, 1) == 256 and ws(2, 257, 32, 1) > 256  # complex backward: 16 x 16 steps


def test_size_queries(lib):
    assert lib.tsfast_hip_diag_workspace_bytes(32, 1000, 64, 0) > 0
    # a 256-byte tile counter, then 4 words per lane and super-chunk (complex: 16-byte words)
    real, cplx = (lib.tsfast_hip_diag_workspace_bytes(32, 1000, 64, c) for c in (0, 1))
    assert (real - 256) % (32 * 64 * 4 * 8) == 0 and (cplx - 256) % (32 * 64 * 4 * 16) == 0
    assert (lib.tsfast_hip_sel_workspace_bytes(4, 300, 40) - 256) % (4 * 40 * 24) == 0
    assert lib.tsfast_hip_mamba_chk_interval(16) >= 1
    k = lib.tsfast_hip_mamba_chk_interval(16)
    # per batch row: fp32 checkpoints [ceil(L/k), N, D], then y [L, D] in the I/O type
    assert lib.tsfast_hip_mamba_saved_floats(45, 40, 16, 0) == -(-45 // k) * 16 * 40 + 45 * 40
    assert lib.tsfast_hip_mamba_saved_floats(45, 40, 16, 1) == -(-45 // k) * 16 * 40 + (45 * 40 * 2 + 3) // 4
    assert lib.tsfast_hip_mamba_saved_floats(45, 40, 65, 0) == -1
    assert lib.tsfast_hip_mamba_workspace_bytes(16, 4096, 1536, 16) > 0
    assert lib.tsfast_hip_mamba_workspace_bytes(1, 1, 1, 65) == -1  # N above 64
    assert lib.tsfast_hip_allpole_workspace_bytes(4096, 16384, 3) > 0
    assert lib.tsfast_hip_allpole_workspace_bytes(4, 16, 17) == -1  # na above 16
    assert lib.tsfast_hip_conv_silu_workspace_bytes(16, 4096, 1536, 4) > 0
    assert lib.tsfast_hip_conv_silu_workspace_bytes(1, 8, 4, 9) == -1  # kernel width above 8
    # counter, agg and inc [nsuper][lanes][n], grad_A partials [nsuper][lanes][n][n], Mc and Ms
    # [lanes][n][n]: n = 2 has 16-step chunks, K = 2 here (few tiles), so nsuper = ceil(100 / 32)
    assert lib.tsfast_hip_linrec_workspace_bytes(64, 100, 2) == 256 + 8 * (4 * 64 * (2 + 2 + 4) + 2 * 64 * 4)
    # n = 5..8: e/f and carries [chunks][lanes][n], the lane matrices and the grad_A partials
    assert lib.tsfast_hip_linrec_workspace_bytes(4, 300, 5) == 8 * (2 * 2 * 4 * 5 + 4 * 25 + 2 * 4 * 25)
    # n = 9..16 (spread path): the same areas with the same 256-step chunks
    assert lib.tsfast_hip_linrec_workspace_bytes(4, 300, 12) == 8 * (2 * 2 * 4 * 12 + 4 * 144 + 2 * 4 * 144)
    assert lib.tsfast_hip_linrec_workspace_bytes(4, 16, 17) == -1  # n above 16


def test_argument_errors_before_any_launch(lib):
    # negative sizes and unsupported orders are rejected on the host, before touching a device
    assert lib.tsfast_hip_diag_fwd(-1, 1, 1, 0, None, None, None, None, None, 0, None) == -1
    assert lib.tsfast_hip_allpole_fwd(4, 16, 17, None, None, None, None, None, 0, None) == -3
    assert lib.tsfast_hip_linrec_fwd(4, 16, 17, None, None, None, None, None, 0, None) == -3
    assert lib.tsfast_hip_linrec_fwd(4, 16, 9, None, None, None, None, None, 0, None) == -1  # NULL inputs
    assert lib.tsfast_hip_linrec_bwd(-1, 16, 2, *([None] * 8), 0, None) == -1
    assert lib.tsfast_hip_mamba_fwd(1, 1, 1, 65, 0, *([None] * 12)) == -3
    assert lib.tsfast_hip_conv_silu_fwd(1, 8, 4, 1, 0, *([None, 0, 0, 0] + [None] * 5)) == -1  # K < 2
    assert lib.tsfast_hip_conv_silu_fwd(1, 8, 4, 9, 0, *([None, 0, 0, 0] + [None] * 5)) == -3  # K > 8
    # empty problems are a no-op
    assert lib.tsfast_hip_diag_fwd(0, 5, 3, 0, None, None, None, None, None, 0, None) == 0


def _declared_arity():
    text = (ROOT / "include" / "tsfast_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(tsfast_hip_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_loader_arity_matches_header():
    """ctypes argtypes must have exactly the header's parameter count (a short list shifts the
    stream handle into the wrong slot)."""
    arity = _declared_arity()
    assert sorted(arity) == _declared()
    for name, (argtypes, _) in _lib._SIGNATURES.items():
        assert len(argtypes) == arity[name], name


def test_mamba_supports_mirrors_the_kernel_size_limits(lib):
    """mamba_hip keeps the checkpoint interval and the per-row addressing limit in Python (so
    supports() makes no library call inside a compiled graph); both must agree with the C side,
    so a shape the kernels would reject falls back through dispatch instead of raising."""
    from tsfast_amd.mamba import mamba_hip

    for N in range(1, 65):
        assert mamba_hip._chk_steps(N) == lib.tsfast_hip_mamba_chk_interval(N), N
    # around the 2 GiB row boundary at D = 1536 (L near 2^29 / 1536 = 349525 minus padding)
    for N in (1, 16, 64):
        for L in (1, 4096, 349_000, 349_400, 349_460, 349_500, 349_600, 400_000):
            c_ok = lib.tsfast_hip_mamba_saved_floats(L, 1536, N, 0) >= 0
            assert mamba_hip._rows_fit(L, 1536, N) == c_ok, (L, N)


def test_mamba_saved_floats_formula_matches_the_library(lib):
    import torch

    from tsfast_amd.mamba import mamba_hip

    for L, D, N in ((1, 1, 1), (45, 40, 16), (4096, 1536, 16), (33, 16, 8), (1000, 70, 64), (7, 8, 33)):
        for dt, code in ((torch.float32, 0), (torch.bfloat16, 1)):
            assert mamba_hip.saved_floats(L, D, N, dt) == lib.tsfast_hip_mamba_saved_floats(L, D, N, code)


def test_conv_supports_mirrors_the_kernel_grid_limit(lib):
    """conv_hip's size screen repeats the kernels' limit (a one-dimensional grid of at most
    2^24 - 1 workgroups; batch and sequence length have no cap of their own), so a shape the
    library rejects falls back through dispatch instead of raising in the op."""
    from tsfast_amd.mamba import conv_hip

    D, K = 64, 4
    cases = ((1, 1), (1, 128), (1, 65536 * 128), (65536, 8), (70000, 3), (2**24 - 1, 8), (2**24, 8),
             (2**23 - 1, 65), (2**23, 65), (2**20, 1024), (2**18, 1024))
    for B, L in cases:
        c_ok = lib.tsfast_hip_conv_silu_workspace_bytes(B, L, D, K) >= 0
        py_ok = conv_hip._size_reason(B, L, D, D, 1, 2) is None
        assert py_ok == c_ok, (B, L)
    assert conv_hip._size_reason(70000, 3, D, D, 1, 2) is None
    assert conv_hip._size_reason(2**24, 8, D, D, 1, 2) is not None


@pytest.mark.parametrize(
    "B,L,H,N,O",
    [
        (64, 4096, 32, 256, 32),
        (1, 2**24, 32, 16, 31),  # u just under 2 GiB, y under
        (1, 2**24, 31, 16, 32),  # y at 2 GiB: O > H on a long sequence
        (1, 2**24, 32, 16, 32),  # both at 2 GiB
        (2, 3, 33, 8, 8),
        (2, 3, 8, 257, 8),
        (2, 3, 8, 8, 33),
        (2**30, 1, 1, 1, 1),
    ],
)
def test_projected_supports_mirrors_the_library_size_check(lib, B, L, H, N, O):
    """projected_hip's shape screen accepts exactly what tsfast_hip_projscan_workspace_bytes
    accepts, so a call that passes supports() never meets a -1 workspace query."""
    from tsfast_amd.scan_backends import projected_hip

    ok_lib = lib.tsfast_hip_projscan_workspace_bytes(B, L, H, N, O) >= 0
    assert (projected_hip.shape_reason(B, L, H, N, O) is None) == ok_lib


def test_reproducible_by_default_and_switch(lib):
    """The library starts in deterministic mode; the backends keep it there unless reproducibility
    is switched off and torch's deterministic flag is off (no kernel is launched here)."""
    import torch

    _lib._det_mode = None
    assert lib.tsfast_hip_get_deterministic() in (0, 1)
    prev = _lib.set_reproducible(True)
    try:
        _lib.sync_deterministic()
        assert lib.tsfast_hip_get_deterministic() == 1
        _lib.set_reproducible(False)
        _lib.sync_deterministic()
        assert lib.tsfast_hip_get_deterministic() == 0
        torch.use_deterministic_algorithms(True, warn_only=True)
        try:
            _lib.sync_deterministic()
            assert lib.tsfast_hip_get_deterministic() == 1
        finally:
            torch.use_deterministic_algorithms(False)
    finally:
        _lib.set_reproducible(prev)
        _lib.sync_deterministic()


def test_library_default_is_deterministic(lib):
    """A fresh process's library (C callers included) starts in deterministic mode."""
    import subprocess
    import sys

    code = ("from tsfast_amd import _lib; import sys; "
            "sys.exit(0 if _lib.load().tsfast_hip_get_deterministic() == 1 else 1)")
    assert subprocess.run([sys.executable, "-c", code], cwd=ROOT).returncode == 0
