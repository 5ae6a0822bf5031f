"""GPU parity: HIP diagonal / selective scans vs the fp64 oracle (through the scan custom ops).

Shapes follow the reference's backend-equivalence suite (tests/test_scan_diagonal_backends.py:18-26,
test_scan_selective_backends.py) plus reduced versions of BASELINE configs 1, 2 and 5. Inputs are
seeded fp32/complex64; the oracle runs in fp64 on exactly those values. Bar: max relative error
<= 1e-5 (fp32) for outputs and every gradient.
"""

import numpy as np
import pytest
import torch

from oracle import scan_oracle as O
from tsfast_amd import dispatch, scan
from tsfast_amd.scan_backends import diagonal_hip, selective_hip

pytestmark = pytest.mark.gpu

TOL = 1e-5

# (v_shape, lam_shape) — tests/test_scan_diagonal_backends.py:18-26 plus config-sized cases
_DIAG_SHAPES = [
    ((32, 200, 64), (64,)),
    ((16, 200, 32), (32,)),
    ((4, 257, 8), (4, 8)),
    ((2, 7, 3), (3,)),
    ((3, 1, 6), (6,)),
    ((1, 8192, 24), (24,)),
    ((2, 300, 100), (100,)),
    ((32, 1000, 64), (32, 64)),  # config 1
    ((4, 4096, 256), (256,)),  # config 2, batch reduced
    ((16, 2048, 256), (256,)),  # enough lanes for the 32-step real chunk tiles
    # bounds of the whole-sequence tiles (one workgroup per lane group covers L <= 16 chunks:
    # 1024 real steps, 512 complex forward, 256 complex backward) and ragged lane groups
    ((2, 1024, 64), (64,)),
    ((2, 1025, 64), (64,)),
    ((2, 512, 32), (32,)),
    ((3, 256, 70), (70,)),
    # whole-sequence lane groups: 64 lanes once they fill 256 workgroups (16384 lanes), 16 below;
    # 500 lanes = 32 groups of 16 (XCD-contiguous group order) with a ragged last group
    ((64, 200, 256), (256,)),
    ((5, 200, 100), (100,)),
    ((48, 500, 256), (256,)),  # 12288 lanes: 768 16-lane workgroups, several rounds per CU
    # forward on whole-sequence tiles of up to 64 chunks (16-lane groups, L <= 4096), backward on
    # the look-back: ragged lanes and last chunk; and a long look-back with 128 super-chunks
    ((3, 3000, 70), (70,)),
    ((6, 8192, 100), (100,)),
]


def _np(t):
    return t.detach().cpu().numpy()


def _make_diag(v_shape, lam_shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype.is_complex:
        r = torch.rand(*lam_shape, generator=g) * 0.099 + 0.9
        th = torch.rand(*lam_shape, generator=g) * (np.pi / 10)
        lam = torch.polar(r, th)
        v = torch.randn(*v_shape, dtype=torch.complex64, generator=g)
        x0 = torch.randn(v_shape[0], v_shape[-1], dtype=torch.complex64, generator=g)
        gout = torch.randn(*v_shape, dtype=torch.complex64, generator=g)
    else:
        lam = torch.rand(*lam_shape, generator=g) * 0.099 + 0.9
        v = torch.randn(*v_shape, generator=g)
        x0 = torch.randn(v_shape[0], v_shape[-1], generator=g)
        gout = torch.randn(*v_shape, generator=g)
    return lam, v, x0, gout


def _lanes(lam, v, x0):
    """The lane layout the ops see (scan.py wrappers): lam [M, N], v [M, L, N]."""
    M, L, N = v.shape
    return lam.broadcast_to(M, N).contiguous(), v, x0


@pytest.mark.parametrize("dtype", [torch.float32, torch.complex64])
@pytest.mark.parametrize("v_shape,lam_shape", _DIAG_SHAPES)
@pytest.mark.parametrize("with_x0", [True, False])
def test_diag_matches_oracle(gpu, dtype, v_shape, lam_shape, with_x0):
    lam, v, x0, gout = _make_diag(v_shape, lam_shape, dtype, seed=sum(v_shape))
    x0 = x0 if with_x0 else None
    lam_d = lam.to(gpu).requires_grad_()
    v_d = v.to(gpu).requires_grad_()
    x0_d = x0.to(gpu).requires_grad_() if x0 is not None else None
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("scan.diagonal", scan._BACKENDS["diagonal"], ("hip",), _lanes(lam_d, v_d, x0_d)) is diagonal_hip
        out = scan.diagonal_recurrence(lam_d, v_d, x0_d)
        out.backward(gout.to(gpu))
    lam_l, _, _ = _lanes(lam, v, x0)
    want = O.diag_forward(_np(lam_l), _np(v), None if x0 is None else _np(x0))
    glam_w, gv_w, gx0_w = O.diag_backward(_np(gout), _np(lam_l), want, None if x0 is None else _np(x0))
    if lam.dim() == 1:
        glam_w = glam_w.sum(0)  # broadcast lam: autograd reduces the lane gradients
    assert O.rel_err(_np(out), want) < TOL
    assert O.rel_err(_np(v_d.grad), gv_w) < TOL
    assert O.rel_err(_np(lam_d.grad), glam_w) < TOL
    if x0 is not None:
        assert O.rel_err(_np(x0_d.grad), gx0_w) < TOL


def test_diag_inference_equals_grad_path(gpu):
    lam, v, x0, _ = _make_diag((8, 64, 16), (16,), torch.complex64, 0)
    lam, v, x0 = lam.to(gpu), v.to(gpu), x0.to(gpu)
    with dispatch.use_backend("hip"):
        with torch.no_grad():
            a = scan.diagonal_recurrence(lam, v, x0)
        b = scan.diagonal_recurrence(lam.requires_grad_(), v.requires_grad_(), x0.requires_grad_())
    assert torch.equal(a, b.detach())


# (1, 3000, 24): more than 16 super-chunks (cooperative carry kernel); (16, 2048, 512): 32-step
# forward chunks
@pytest.mark.parametrize(
    "shape", [(2, 7, 3), (4, 257, 8), (2, 1, 3), (3, 5000, 40), (8, 1024, 128), (1, 3000, 24), (16, 2048, 512)]
)
@pytest.mark.parametrize("with_x0", [True, False])
def test_selective_matches_oracle(gpu, shape, with_x0):
    g = torch.Generator().manual_seed(sum(shape))
    lam = torch.rand(*shape, generator=g) * 0.9 + 0.05
    v = torch.randn(*shape, generator=g)
    x0 = torch.randn(shape[0], shape[2], generator=g) if with_x0 else None
    gout = torch.randn(*shape, generator=g)
    lam_d, v_d = lam.to(gpu).requires_grad_(), v.to(gpu).requires_grad_()
    x0_d = x0.to(gpu).requires_grad_() if x0 is not None else None
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("scan.selective", scan._BACKENDS["selective"], ("hip",), (lam_d, v_d, x0_d)) is selective_hip
        out = scan.selective_recurrence(lam_d, v_d, x0_d)
        out.backward(gout.to(gpu))
    x0n = None if x0 is None else _np(x0)
    want = O.selective_forward(_np(lam), _np(v), x0n)
    glam_w, gv_w, gx0_w = O.selective_backward(_np(gout), _np(lam), want, x0n)
    assert O.rel_err(_np(out), want) < TOL
    assert O.rel_err(_np(lam_d.grad), glam_w) < TOL
    assert O.rel_err(_np(v_d.grad), gv_w) < TOL
    if x0 is not None:
        assert O.rel_err(_np(x0_d.grad), gx0_w) < TOL


def test_empty_sequence(gpu):
    lam = torch.rand(3, 4, device=gpu)
    v = torch.zeros(3, 0, 4, device=gpu)
    x0 = torch.randn(3, 4, device=gpu)
    out = diagonal_hip.forward(lam, v, x0)
    assert out.shape == (3, 0, 4)
    glam, gv, gx0 = diagonal_hip.backward(torch.zeros_like(v), lam, out, x0)
    assert torch.count_nonzero(glam) == 0 and torch.count_nonzero(gx0) == 0 and gv.shape == v.shape


def test_tbptt_chunked_equals_unchunked(gpu):
    """Config 5 shape (reduced L): 16 consecutive chunks of 4096 with the final state carried as
    x0 equal one unchunked scan; chunk slicing is exact and the forward stays within 1e-5."""
    g = torch.Generator().manual_seed(5)
    B, N, C, T = 8, 128, 16, 4096
    lam = (torch.rand(B, N, generator=g) * 0.0099 + 0.99).to(gpu)
    v = torch.randn(B, C * T, N, generator=g).to(gpu)
    with torch.no_grad():
        full = diagonal_hip.forward(lam, v, None)
        x0 = None
        parts = []
        for k in range(C):
            o = diagonal_hip.forward(lam, v[:, k * T : (k + 1) * T].contiguous(), x0)
            parts.append(o)
            x0 = o[:, -1].contiguous()
    chunked = torch.cat(parts, 1)
    assert chunked.shape == full.shape
    want = O.diag_forward(_np(lam), _np(v), None)
    assert O.rel_err(_np(full), want) < TOL
    assert O.rel_err(_np(chunked), want) < TOL


@pytest.mark.parametrize("cplx", [0, 1])
def test_whole_sequence_tiles_clear_the_flag(gpu, cplx):
    """A call served by whole-sequence tiles (no look-back, no reset kernel) leaves the workspace's
    give-up flag clear even when the buffer held a stale one, in both directions."""
    from tsfast_amd import _lib

    lib = _lib.load()
    dtype = torch.complex64 if cplx else torch.float32
    lam, v, x0, gout = _make_diag((4, 200, 64), (64,), dtype, seed=33)
    lam_l, _, _ = _lanes(lam, v, x0)
    M, L, N = v.shape
    nbytes = lib.tsfast_hip_diag_workspace_bytes(M, L, N, cplx)
    lam_d, v_d, x0_d, g_d = (t.to(gpu) for t in (lam_l, v, x0, gout))
    out = torch.empty_like(v_d)
    gv, glam, gx0 = torch.empty_like(v_d), torch.empty_like(lam_d), torch.empty_like(x0_d)
    for call in ("fwd", "bwd"):
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
        ws[_lib.LOOKBACK_ERR_OFFSET] = 1
        if call == "fwd":
            st = lib.tsfast_hip_diag_fwd(M, L, N, cplx, _lib.ptr(lam_d), _lib.ptr(v_d), _lib.ptr(x0_d), _lib.ptr(out),
                                         _lib.ptr(ws), nbytes, _lib.stream_of(v_d))
        else:
            st = lib.tsfast_hip_diag_bwd(M, L, N, cplx, _lib.ptr(g_d), _lib.ptr(lam_d), _lib.ptr(out), _lib.ptr(x0_d),
                                         _lib.ptr(gv), _lib.ptr(glam), _lib.ptr(gx0), _lib.ptr(ws), nbytes,
                                         _lib.stream_of(v_d))
        _lib.check(st, f"tsfast_hip_diag_{call}")
        torch.cuda.synchronize()
        assert not _lib.lookback_gave_up(ws), call
    want = O.diag_forward(_np(lam_l), _np(v), _np(x0))
    glam_w, gv_w, gx0_w = O.diag_backward(_np(gout), _np(lam_l), want, _np(x0))
    assert O.rel_err(_np(out), want) < TOL
    assert O.rel_err(_np(gv), gv_w) < TOL and O.rel_err(_np(glam), glam_w) < TOL and O.rel_err(_np(gx0), gx0_w) < TOL


def test_lookback_give_up_flag_cleared_and_unset(gpu):
    """Every scan's reset clears the workspace's give-up flag, and a scan whose look-backs all
    complete leaves it clear (outputs checked against the oracle)."""
    from tsfast_amd import _lib

    lib = _lib.load()
    lam, v, x0, _ = _make_diag((8, 5000, 64), (64,), torch.float32, seed=31)
    lam_l, v_l, _ = _lanes(lam, v, None)
    M, L, N = v.shape
    nbytes = lib.tsfast_hip_diag_workspace_bytes(M, L, N, 0)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    ws[_lib.LOOKBACK_ERR_OFFSET] = 1  # stale flag from an earlier (imagined) give-up
    out = torch.empty_like(v_l, device=gpu)
    lam_d, v_d = lam_l.to(gpu), v_l.to(gpu)
    _lib.check(lib.tsfast_hip_diag_fwd(M, L, N, 0, _lib.ptr(lam_d), _lib.ptr(v_d), None, _lib.ptr(out), _lib.ptr(ws),
                                       nbytes, _lib.stream_of(v_d)), "tsfast_hip_diag_fwd")
    torch.cuda.synchronize()
    assert not _lib.lookback_gave_up(ws)
    assert O.rel_err(_np(out), O.diag_forward(_np(lam_l), _np(v_l))) < TOL


# The reference suite's coefficient draws (tests/test_scan_diagonal_backends.py:33-40: real
# lam ~ U(0, 0.85); complex |lam| ~ U(0, 0.85) with phase ~ U(0, 3)), plus negative real
# coefficients and complex ones near the unit circle with large phases, on shapes that take the
# look-back (real L > 1024, complex L > 512: fp64 powers of lam composed across super-chunks,
# underflowing fast for small |lam|) and on whole-sequence tiles. Lane 0 of every draw has
# lam = 0 exactly (x_t = v_t).
_DRAW_SHAPES = [
    ((2, 1025, 64), (64,)),
    ((1, 8192, 24), (24,)),
    ((6, 8192, 100), (100,)),
    ((3, 3000, 70), (70,)),
    ((16, 2048, 256), (256,)),
    ((4, 4096, 256), (256,)),
    ((32, 1000, 64), (32, 64)),
    ((2, 512, 32), (32,)),
    ((48, 500, 256), (256,)),
]


def _draw_lam(kind, shape, g):
    u = torch.rand(*shape, generator=g)
    if kind == "ref_real":
        lam = u * 0.85
    elif kind == "neg_real":
        lam = -(u * 0.9 + 0.05)
    elif kind == "neg_real_near_one":
        lam = -(u * 0.099 + 0.9)
    elif kind == "ref_complex":
        lam = torch.polar(u * 0.85, torch.rand(*shape, generator=g) * 3.0)
    else:  # "wide_complex": near the unit circle, phases up to 3 rad
        lam = torch.polar(u * 0.099 + 0.9, torch.rand(*shape, generator=g) * 3.0)
    lam[..., 0] = 0
    return lam


@pytest.mark.parametrize("kind", ["ref_real", "neg_real", "neg_real_near_one", "ref_complex", "wide_complex"])
@pytest.mark.parametrize("v_shape,lam_shape", _DRAW_SHAPES)
def test_diag_reference_coefficient_draws(gpu, kind, v_shape, lam_shape):
    g = torch.Generator().manual_seed(sum(v_shape) + len(kind))
    cplx = kind.endswith("complex")
    dt = torch.complex64 if cplx else torch.float32
    lam = _draw_lam(kind, lam_shape, g)
    v = torch.randn(*v_shape, dtype=dt, generator=g)
    x0 = torch.randn(v_shape[0], v_shape[-1], dtype=dt, generator=g)
    gout = torch.randn(*v_shape, dtype=dt, generator=g)
    lam_d = lam.to(gpu).requires_grad_()
    v_d, x0_d = v.to(gpu).requires_grad_(), x0.to(gpu).requires_grad_()
    with dispatch.use_backend("hip"):
        assert dispatch.resolve("scan.diagonal", scan._BACKENDS["diagonal"], ("hip",), _lanes(lam_d, v_d, x0_d)) is diagonal_hip
        out = scan.diagonal_recurrence(lam_d, v_d, x0_d)
        out.backward(gout.to(gpu))
    lam_l, _, _ = _lanes(lam, v, x0)
    want = O.diag_forward(_np(lam_l), _np(v), _np(x0))
    glam_w, gv_w, gx0_w = O.diag_backward(_np(gout), _np(lam_l), want, _np(x0))
    if lam.dim() == 1:
        glam_w = glam_w.sum(0)
    assert O.rel_err(_np(out), want) < TOL, "out"
    assert O.rel_err(_np(v_d.grad), gv_w) < TOL, "gv"
    assert O.rel_err(_np(lam_d.grad), glam_w) < TOL, "glam"
    assert O.rel_err(_np(x0_d.grad), gx0_w) < TOL, "gx0"


def test_forced_give_up_raises_without_debug_mode(gpu):
    """A look-back that gives up is reported by default (no TSFAST_HIP_CHECK_LOOKBACK): the host
    forces it with a zero spin limit (a wait ends at its first round without progress, so every
    kernel still exits), and the give-up reaches the Python layer through the library's alarm
    word, as a RuntimeError from the call that launched it or from the next check, and only once
    per failing call. Scans then run normally again."""
    from tsfast_amd import _lib

    _lib.raise_if_lookback_gave_up("before")  # no earlier give-up pending
    assert _lib.load().tsfast_hip_lookback_gave_up(0) == 0
    g = torch.Generator().manual_seed(41)
    lam = (torch.rand(8, 64, generator=g) * 0.099 + 0.9).to(gpu)
    v = torch.randn(8, 100_000, 64, generator=g).to(gpu)  # 12800 look-back tiles
    lib = _lib.load()
    prev = lib.tsfast_hip_set_lookback_spin_limit(0)
    raised = False
    out = None
    try:
        out = diagonal_hip.forward(lam, v, None)
    except RuntimeError as e:
        raised = "gave up" in str(e)
    finally:
        lib.tsfast_hip_set_lookback_spin_limit(prev)
    torch.cuda.synchronize()
    if not raised:
        assert torch.isnan(out).any()  # the lanes whose wait gave up
        with pytest.raises(RuntimeError, match="gave up"):
            _lib.raise_if_lookback_gave_up("after")
    # reported once: the same call's later give-ups do not raise again
    assert lib.tsfast_hip_lookback_gave_up(0) == 0
    _lib.raise_if_lookback_gave_up("again")
    # normal limit again: a clean scan that matches the oracle and raises nothing
    small_v = v[:2, :5000].contiguous()
    out2 = diagonal_hip.forward(lam[:2], small_v, None)
    torch.cuda.synchronize()
    _lib.raise_if_lookback_gave_up("clean")
    assert O.rel_err(_np(out2), O.diag_forward(_np(lam[:2]), _np(small_v))) < TOL
