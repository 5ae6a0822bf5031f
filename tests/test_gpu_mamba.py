"""GPU parity: fused HIP Mamba selective scan vs the fp64 oracle, fp32 and bf16 I/O.

Shapes follow the reference's fused-backend suite (tests/test_mamba.py:276-285: L not a multiple
of the checkpoint interval, L shorter than one chunk, a partial channel block, N = 12) plus a
reduced config 3. Every output and gradient is compared: out, h_last, gdraw, gA, gBt, gCt, gu, gz,
gDp and gh0. Bars: max relative error <= 1e-5 for fp32 I/O; <= 2e-2 for
bf16 I/O with fp32 state, measured against the fp64 oracle on the bf16-rounded inputs.
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import dispatch
from tsfast_amd.mamba import core as mcore
from tsfast_amd.mamba import mamba_hip

pytestmark = pytest.mark.gpu

_NAMES = ("draw", "A", "Bt", "Ct", "u", "z", "Dp", "h0")


def _make(B, L, D, N, seed, io_dtype, with_h0=True, a_structured=False):
    g = torch.Generator().manual_seed(seed)
    if a_structured:
        A = -torch.exp(torch.log(torch.arange(1, N + 1, dtype=torch.float32))).expand(D, N).contiguous()
    else:
        A = -torch.exp(torch.randn(D, N, generator=g) * 0.5)
    t = dict(
        draw=torch.randn(B, L, D, generator=g) - 4.0 if a_structured else torch.randn(B, L, D, generator=g) - 1.0,
        A=A,
        Bt=torch.randn(B, L, N, generator=g),
        Ct=torch.randn(B, L, N, generator=g),
        u=torch.randn(B, L, D, generator=g),
        z=torch.randn(B, L, D, generator=g),
        Dp=torch.randn(D, generator=g),
        h0=torch.randn(B, D, N, generator=g) * 0.5 if with_h0 else None,
    )
    for k in ("draw", "Bt", "Ct", "u", "z"):
        t[k] = t[k].to(io_dtype)
    gout = torch.randn(B, L, D, generator=g).to(io_dtype)
    ghlast = torch.randn(B, D, N, generator=g)
    return t, gout, ghlast


def _np64(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def _run_hip(t, gout, ghlast, dev, use_ghlast):
    leaves = {k: (v.to(dev).requires_grad_() if v is not None else None) for k, v in t.items()}
    args = [leaves[k] for k in _NAMES]
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("mamba.ssm", mcore._SSM_BACKENDS, ("hip",), tuple(args)) is mamba_hip
        out, h_last = mcore.mamba_ssm(*args)
    h_last = h_last.view(args[0].shape[0], args[0].shape[2], -1)
    grads = [gout.to(dev)] + ([ghlast.to(dev)] if use_ghlast else [])
    torch.autograd.backward([out, h_last] if use_ghlast else [out], grads)
    return out, h_last, {k: (v.grad if v is not None else None) for k, v in leaves.items()}


@pytest.mark.parametrize(
    "B,L,D,N",
    [(4, 50, 32, 16), (2, 33, 16, 8), (1, 7, 8, 32), (2, 64, 20, 16), (2, 40, 24, 12), (3, 100, 130, 4),
     (2, 37, 70, 64), (2, 16, 64, 1),
     # from 32 states the backward takes 16-channel tiles: several whole tiles, and a partial one
     (2, 75, 48, 32), (1, 130, 40, 20)],
)
@pytest.mark.parametrize("io", ["fp32", "bf16"])
@pytest.mark.parametrize("with_h0,use_ghlast", [(True, True), (False, False)])
def test_mamba_matches_oracle(gpu, B, L, D, N, io, with_h0, use_ghlast):
    io_dtype = torch.float32 if io == "fp32" else torch.bfloat16
    tol = 1e-5 if io == "fp32" else 2e-2
    t, gout, ghlast = _make(B, L, D, N, seed=B * L + D + N, io_dtype=io_dtype, with_h0=with_h0)
    out, h_last, grads = _run_hip(t, gout, ghlast, gpu, use_ghlast)
    assert out.dtype == io_dtype and h_last.dtype == torch.float32
    args = [_np64(t[k]) for k in _NAMES]
    want_out, want_h = O.mamba_forward(*args)
    got = O.mamba_backward(_np64(gout), _np64(ghlast) if use_ghlast else None, *args)
    assert O.rel_err(_np64(out), want_out) < tol, "out"
    assert O.rel_err(_np64(h_last), want_h) < tol, "h_last"
    for name, want in zip(("draw", "A", "Bt", "Ct", "u", "z", "Dp", "h0"), got):
        if want is None:
            continue
        gk = grads[name]
        assert gk.dtype == t[name].dtype
        assert O.rel_err(_np64(gk), want) < tol, f"grad {name}: {O.rel_err(_np64(gk), want):.2e}"


@pytest.mark.parametrize("io", ["fp32", "bf16"])
def test_mamba_config3_reduced(gpu, io):
    """Config 3's distributions (A = -(n+1), draw ~ N(-4, 1), h0 = None, ghlast = None) at
    B=2, L=1024, D=256, N=16."""
    io_dtype = torch.float32 if io == "fp32" else torch.bfloat16
    tol = 1e-5 if io == "fp32" else 2e-2
    t, gout, _ = _make(2, 1024, 256, 16, seed=3, io_dtype=io_dtype, with_h0=False, a_structured=True)
    out, h_last, grads = _run_hip(t, gout, None, gpu, use_ghlast=False)
    args = [_np64(t[k]) for k in _NAMES]
    want_out, want_h = O.mamba_forward(*args)
    got = O.mamba_backward(_np64(gout), None, *args)
    assert O.rel_err(_np64(out), want_out) < tol
    assert O.rel_err(_np64(h_last), want_h) < tol
    for name, want in zip(_NAMES, got):
        if want is not None:
            assert O.rel_err(_np64(grads[name]), want) < tol, name


def test_mamba_inference_equals_train_forward(gpu):
    t, _, _ = _make(2, 45, 40, 16, seed=11, io_dtype=torch.float32)
    args = [t[k].to(gpu) if t[k] is not None else None for k in _NAMES]
    with torch.no_grad():
        a_out, a_h = mamba_hip.run(*args)
    b_out, b_h, chk = mamba_hip._scan_train_op(*args)
    assert torch.equal(a_out, b_out) and torch.equal(a_h, b_h)
    assert chk.shape == (2, mamba_hip.saved_floats(45, 40, 16, torch.float32))


def test_mamba_saved_state_layout(gpu):
    """The training forward's saved state, per batch row: checkpoint slot k = the state after
    step (k + 1) * interval - 1 as [N, D], then y = sum_n h C + Dp u as [L, D] (fp64 oracle)."""
    B, L, D, N = 2, 45, 40, 16
    t, _, _ = _make(B, L, D, N, seed=13, io_dtype=torch.float32)
    args = [t[k].to(gpu) if t[k] is not None else None for k in _NAMES]
    _, _, saved = mamba_hip._scan_train_op(*args)
    k = mamba_hip.chk_interval(N)
    nc = -(-L // k)
    saved = saved.cpu().numpy().astype(np.float64)
    chk = saved[:, : nc * N * D].reshape(B, nc, N, D)
    y = saved[:, nc * N * D :].reshape(B, L, D)
    np_t = {n: _np64(v) for n, v in t.items()}
    _, _, states = O.mamba_forward(*[np_t[n] for n in _NAMES], return_states=True)  # [B, L, D, N]
    full = L // k  # slots whose step exists
    want_chk = states[:, k - 1 :: k][:, :full].transpose(0, 1, 3, 2)  # [B, full, N, D]
    assert O.rel_err(chk[:, :full], want_chk) < 1e-5
    want_y = np.einsum("bldn,bln->bld", states, np_t["Ct"]) + np_t["Dp"] * np_t["u"]
    assert O.rel_err(y, want_y) < 1e-5


def test_mamba_chunked_state_equivalence(gpu):
    """TBPTT through h0/h_last: three chunks (17, 2, rest) equal the full pass."""
    t, _, _ = _make(3, 70, 48, 16, seed=12, io_dtype=torch.float32, with_h0=False)
    args = {k: (v.to(gpu) if v is not None else None) for k, v in t.items()}
    with torch.no_grad():
        full, _ = mamba_hip.run(*[args[k] for k in _NAMES])
        outs, h = [], None
        for lo, hi in ((0, 17), (17, 19), (19, 70)):
            sl = {k: (args[k][:, lo:hi].contiguous() if k in ("draw", "Bt", "Ct", "u", "z") else args[k]) for k in _NAMES}
            sl["h0"] = h
            o, h = mamba_hip.run(*[sl[k] for k in _NAMES])
            outs.append(o)
    assert O.rel_err(_np64(torch.cat(outs, 1)), _np64(full)) < 1e-5


@pytest.mark.parametrize("N", [96, 130])
@pytest.mark.parametrize("io", ["fp32", "bf16"])
def test_mamba_state_groups_above_64(gpu, N, io):
    """N above the 64 states of one launch runs in state groups of up to 64 (96 = 64 + 32,
    130 = 64 + 64 + 2), every output and gradient against the oracle (the reference's fused
    backend has no state cap, mamba_triton.py:490-520)."""
    io_dtype = torch.float32 if io == "fp32" else torch.bfloat16
    tol = 1e-5 if io == "fp32" else 2e-2
    t, gout, ghlast = _make(2, 45, 40, N, seed=N, io_dtype=io_dtype, with_h0=True)
    out, h_last, grads = _run_hip(t, gout, ghlast, gpu, use_ghlast=True)
    assert out.dtype == io_dtype and h_last.shape == (2, 40, N)
    args = [_np64(t[k]) for k in _NAMES]
    want_out, want_h = O.mamba_forward(*args)
    got = O.mamba_backward(_np64(gout), _np64(ghlast), *args)
    assert O.rel_err(_np64(out), want_out) < tol, "out"
    assert O.rel_err(_np64(h_last), want_h) < tol, "h_last"
    for name, want in zip(_NAMES, got):
        if want is not None:
            assert grads[name].dtype == t[name].dtype
            assert O.rel_err(_np64(grads[name]), want) < tol, name


def test_mamba_batch_above_65535(gpu):
    """More batch rows than a grid's y dimension holds: the grid is one-dimensional."""
    t, gout, ghlast = _make(70_000, 3, 32, 4, seed=21, io_dtype=torch.float32, with_h0=True)
    out, h_last, grads = _run_hip(t, gout, ghlast, gpu, use_ghlast=True)
    args = [_np64(t[k]) for k in _NAMES]
    want_out, want_h = O.mamba_forward(*args)
    got = O.mamba_backward(_np64(gout), _np64(ghlast), *args)
    assert O.rel_err(_np64(out), want_out) < 1e-5
    assert O.rel_err(_np64(h_last), want_h) < 1e-5
    for name, want in zip(_NAMES, got):
        if want is not None:
            assert O.rel_err(_np64(grads[name]), want) < 1e-5, name
