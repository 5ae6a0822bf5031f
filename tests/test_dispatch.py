"""Dispatch semantics (mirrors the reference's tests/test_scan_dispatch.py:17-112) on the CPU."""

import sys
import types
import warnings

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O

from tsfast_amd import dispatch, scan


@pytest.fixture(autouse=True)
def _fresh(monkeypatch):
    monkeypatch.setattr(dispatch, "_default_backend", "auto")
    monkeypatch.setattr(dispatch, "_warned", set())


def test_unknown_backend_rejected():
    with pytest.raises(ValueError):
        dispatch.set_backend("cuda")
    with pytest.raises(ValueError):
        with dispatch.use_backend("nope"):
            pass


def test_scopes_nest_and_restore():
    dispatch.set_backend("reference")
    assert dispatch.get_backend() == "reference"
    with dispatch.use_backend("hip"):
        assert dispatch.get_backend() == "hip"
        with dispatch.use_backend("auto"):
            assert dispatch.get_backend() == "auto"
        assert dispatch.get_backend() == "hip"
    assert dispatch.get_backend() == "reference"


def test_hip_is_auto_choice_for_gpu_tensors():
    assert scan._AUTO_ORDER["cuda"][0] == "hip"
    from tsfast_amd.dynonet import core as dcore
    from tsfast_amd.mamba import core as mcore

    assert mcore._SSM_AUTO_ORDER["cuda"][0] == "hip"
    assert "hip" in dcore._ALLPOLE_BACKENDS


def test_cpu_tensors_take_reference_path_silently():
    lam, v = torch.rand(2, 3), torch.randn(2, 5, 3)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        out = scan.diagonal_recurrence(lam, v)
    assert np.allclose(out.numpy(), O.diag_forward(lam.numpy(), v.numpy()), atol=1e-6)


def test_import_failure_warns_once_then_falls_back(monkeypatch):
    monkeypatch.setitem(sys.modules, "tsfast_amd.fake_backend", None)
    reg = {"hip": "tsfast_amd.fake_backend"}
    with dispatch.use_backend("hip"):
        with pytest.warns(RuntimeWarning, match="import failed"):
            assert dispatch.resolve("scan.test", reg, ("hip",), ()) is None
        with warnings.catch_warnings():
            warnings.simplefilter("error")
            assert dispatch.resolve("scan.test", reg, ("hip",), ()) is None


def test_decline_reason_is_warned():
    fake = types.ModuleType("fake")
    fake.supports = lambda *a: "no thanks"
    with pytest.warns(RuntimeWarning, match="no thanks"):
        assert dispatch.resolve("scan.test", {"hip": fake}, ("hip",), ()) is None


def test_reference_preference_never_probes():
    fake = types.ModuleType("fake")

    def boom(*a):
        raise AssertionError("probed")

    fake.supports = boom
    with dispatch.use_backend("reference"):
        assert dispatch.resolve("scan.test", {"hip": fake}, ("hip",), ()) is None


def test_missing_family_is_silent():
    with dispatch.use_backend("c"), warnings.catch_warnings():
        warnings.simplefilter("error")
        assert dispatch.resolve("scan.test", {"hip": object()}, ("hip",), ()) is None


def test_backends_decline_cpu_tensors():
    from tsfast_amd.dynonet import allpole_hip
    from tsfast_amd.mamba import mamba_hip
    from tsfast_amd.scan_backends import diagonal_hip, selective_hip

    lam, v = torch.rand(2, 3), torch.randn(2, 5, 3)
    assert "GPU-only" in diagonal_hip.supports(lam, v, None)
    assert "GPU-only" in selective_hip.supports(torch.rand(2, 5, 3), v, None)
    assert "GPU-only" in allpole_hip.supports(torch.rand(2, 2), torch.randn(2, 9), None)
    B, L, D, N = 1, 4, 3, 2
    args = (torch.randn(B, L, D), -torch.rand(D, N), torch.randn(B, L, N), torch.randn(B, L, N),
            torch.randn(B, L, D), torch.randn(B, L, D), torch.randn(D), None)
    assert "GPU-only" in mamba_hip.supports(*args)


def test_compile_fullgraph_reference_path():
    """The custom ops do not graph-break under torch.compile (reference path on CPU)."""
    lam = torch.rand(3, 4)
    v = torch.randn(3, 9, 4, requires_grad=True)

    @torch.compile(fullgraph=True, backend="eager")
    def f(lam, v):
        return scan.diagonal_recurrence(lam, v).square().sum()

    f(lam, v).backward()
    assert v.grad is not None


def test_lookback_give_up_check(monkeypatch):
    """TSFAST_HIP_CHECK_LOOKBACK's check reads the workspace's give-up flag (byte offset 64, set by
    a look-back that gave up waiting) and raises instead of letting its NaN pass as a result."""
    from tsfast_amd import _lib

    ws = torch.zeros(256, dtype=torch.uint8)
    monkeypatch.setattr(_lib, "_CHECK_LOOKBACK", True)
    _lib.check_lookback(ws, "scan")  # flag clear: no error
    ws[_lib.LOOKBACK_ERR_OFFSET] = 1
    assert _lib.lookback_gave_up(ws)
    with pytest.raises(RuntimeError, match="gave up"):
        _lib.check_lookback(ws, "scan")
    monkeypatch.setattr(_lib, "_CHECK_LOOKBACK", False)
    _lib.check_lookback(ws, "scan")  # debug mode off: never reads the flag
