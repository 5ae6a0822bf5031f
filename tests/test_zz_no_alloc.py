"""The no-allocation diagonal forward scan (tsfast_hip_diag_fwd_noalloc) against the workspace
entry point (tsfast_hip_diag_fwd), both called through the C ABI.

The no-allocation entry point keeps its look-back workspace in a fixed per-GPU device array, so
two calls in a row share it: the second (smaller) call must not see the first call's published
words or tile counter. Bar: 1e-5 max relative error against the fp64 oracle (fp32 / complex64
I/O), and the two entry points agree to 1e-6 (the look-back may compose the same affine maps in
a different order from run to run, so the last bit of an output can differ).
"""

import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import _lib

pytestmark = pytest.mark.gpu

TSF_ERR_SCRATCH = -5


def _fns():
    lib = _lib.load()
    return lib, lib.tsfast_hip_diag_fwd_noalloc, lib.tsfast_hip_diag_noalloc_max_bytes


def _inputs(M, L, N, cplx, seed, dev):
    g = torch.Generator().manual_seed(seed)
    if cplx:
        lam = torch.polar(torch.rand(M, N, generator=g) * 0.099 + 0.9, torch.rand(M, N, generator=g) * 0.3)
        v = torch.randn(M, L, N, dtype=torch.complex64, generator=g)
        x0 = torch.randn(M, N, dtype=torch.complex64, generator=g)
    else:
        lam = torch.rand(M, N, generator=g) * 0.099 + 0.9
        v = torch.randn(M, L, N, generator=g)
        x0 = torch.randn(M, N, generator=g)
    return lam.to(dev), v.to(dev), x0.to(dev)


def _with_workspace(lib, lam, v, x0, cplx):
    M, L, N = v.shape
    out = torch.empty_like(v)
    nbytes = lib.tsfast_hip_diag_workspace_bytes(M, L, N, int(cplx))
    ws = _lib.workspace(nbytes, v.device)
    st = lib.tsfast_hip_diag_fwd(M, L, N, int(cplx), lam.data_ptr(), v.data_ptr(), _lib.ptr(x0), out.data_ptr(),
                                 ws.data_ptr(), nbytes, _lib.stream_of(v))
    _lib.check(st, "tsfast_hip_diag_fwd")
    return out


def _no_alloc(na, lam, v, x0, cplx):
    M, L, N = v.shape
    out = torch.empty_like(v)
    st = na(M, L, N, int(cplx), lam.data_ptr(), v.data_ptr(), _lib.ptr(x0), out.data_ptr(), _lib.stream_of(v))
    _lib.check(st, "tsfast_hip_diag_fwd_noalloc")
    return out


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("cplx", [False, True])
def test_no_alloc_matches_workspace_entry_point(gpu, cplx):
    lib, na, mx = _fns()
    # complex: a shape whose forward look-back words (25 MiB) fit the 32 MiB array although a
    # forward-and-backward workspace would not (the entry point sizes for the forward alone),
    # config 2's shape (the largest BASELINE diagonal call), then a smaller ragged one
    shapes = [(64, 4096, 512), (64, 4096, 256), (3, 1000, 70)] if cplx else [(8, 8192, 128), (5, 777, 33)]
    if cplx:
        assert lib.tsfast_hip_diag_workspace_bytes(64, 4096, 512, 1) > mx()
    for i, (M, L, N) in enumerate(shapes):
        lam, v, x0 = _inputs(M, L, N, cplx, seed=10 + i, dev=gpu)
        x0 = x0 if i == len(shapes) - 1 else None
        want = _with_workspace(lib, lam, v, x0, cplx)
        got = _no_alloc(na, lam, v, x0, cplx)
        torch.cuda.synchronize()
        assert torch.isfinite(torch.view_as_real(got) if cplx else got).all(), f"call {i}"
        assert _rel(got, want) < 1e-6, f"call {i}: {_rel(got, want):.2e}"
        rows = slice(0, 2)
        ref = O.diag_forward(
            lam[rows].cpu().numpy(), v[rows].cpu().numpy(), None if x0 is None else x0[rows].cpu().numpy()
        )
        assert O.rel_err(got[rows].cpu().numpy(), ref) < 1e-5, f"call {i} vs oracle"


def test_no_alloc_rejects_shapes_beyond_its_scratch(gpu):
    lib, na, mx = _fns()
    # complex, 65536 lanes x 32 super-chunks of 256 steps: 96 MiB of forward look-back words
    M, L, N = 64, 8192, 1024
    assert lib.tsfast_hip_diag_workspace_bytes(M, L, N, 1) > 2 * mx()
    # the size check returns before anything is launched, so small stand-in buffers do
    lam = torch.ones(4, dtype=torch.complex64, device=gpu)
    v = torch.zeros(4, dtype=torch.complex64, device=gpu)
    out = torch.empty_like(v)
    st = na(M, L, N, 1, lam.data_ptr(), v.data_ptr(), None, out.data_ptr(), _lib.stream_of(lam))
    assert st == TSF_ERR_SCRATCH
    assert b"scratch" in lib.tsfast_hip_status_string(st)
