"""Pin the fp64 oracle (oracle/scan_oracle.py) against independent routes, on the CPU.

Every oracle function is checked against something that does not share its arithmetic:
brute-force closed-form sums, scipy.signal.lfilter, a textbook selective scan written as
einsums (the state-spaces/mamba ``selective_scan_ref`` form the reference transcribes in
tests/test_mamba.py:26-50), the companion-matrix blocked scan, and torch float64 autograd
through plain sequential loops. Each check is also run against deliberately broken variants
of the oracle (a dropped conjugate, a sign flip, a missing factor, an off-by-one in time) and
must reject every one of them, so the checks have the power to catch those mistakes.
"""

import numpy as np
import pytest
import scipy.signal
import torch

from oracle import scan_oracle as O

TOL = 1e-10


def _rng(seed):
    return np.random.default_rng(seed)


def _cplx(rng, *shape):
    return rng.standard_normal(shape) + 1j * rng.standard_normal(shape)


# ------------------------------------------------------------------------ torch loop references
def _torch_diag_loop(lam, v, x0):
    x = torch.zeros_like(v[:, 0]) if x0 is None else x0
    outs = []
    for t in range(v.shape[1]):
        x = lam * x + v[:, t]
        outs.append(x)
    return torch.stack(outs, 1)


def _torch_sel_loop(a, v, x0):
    x = torch.zeros_like(v[:, 0]) if x0 is None else x0
    outs = []
    for t in range(v.shape[1]):
        x = a[:, t] * x + v[:, t]
        outs.append(x)
    return torch.stack(outs, 1)


def _torch_mamba_textbook(draw, A, Bt, Ct, u, z, Dp, h0):
    """Textbook selective scan in the (B, D, L) einsum form of state-spaces/mamba's
    selective_scan_ref, extended by an initial state; float64 torch."""
    delta = torch.nn.functional.softplus(draw).transpose(1, 2)  # (B, D, L)
    uu = u.transpose(1, 2)
    BB = Bt.transpose(1, 2)  # (B, N, L)
    CC = Ct.transpose(1, 2)
    dA = torch.exp(torch.einsum("bdl,dn->bdln", delta, A))
    dBu = torch.einsum("bdl,bnl,bdl->bdln", delta, BB, uu)
    x = h0 if h0 is not None else A.new_zeros(draw.shape[0], A.shape[0], A.shape[1])
    ys = []
    for i in range(draw.shape[1]):
        x = dA[:, :, i] * x + dBu[:, :, i]
        ys.append(torch.einsum("bdn,bn->bd", x, CC[:, :, i]))
    y = torch.stack(ys, 2) + uu * Dp[:, None]
    out = y * torch.nn.functional.silu(z.transpose(1, 2))
    return out.transpose(1, 2), x


def _torch_allpole_loop(a, w, y0):
    na = a.shape[-1]
    s = [y0[:, k] for k in range(na)] if y0 is not None else [torch.zeros_like(w[:, 0])] * na
    ys = []
    for t in range(w.shape[1]):
        yt = w[:, t] - sum(a[:, k] * s[k] for k in range(na))
        ys.append(yt)
        s = [yt] + s[:-1]
    return torch.stack(ys, 1)


def _vjp(f, inputs, g):
    ts = [torch.tensor(x, requires_grad=True) if x is not None else None for x in inputs]
    out = f(*ts)
    outs = out if isinstance(out, tuple) else (out,)
    gs = g if isinstance(g, tuple) else (g,)
    pairs = [(o, torch.tensor(gg)) for o, gg in zip(outs, gs) if gg is not None]
    leaves = [t for t in ts if t is not None]
    grads = torch.autograd.grad([p[0] for p in pairs], leaves, [p[1] for p in pairs], allow_unused=True)
    it = iter(grads)
    return [None if t is None else (np.zeros_like(t.detach().numpy()) if (gr := next(it)) is None else gr.numpy())
            for t in ts]


# ------------------------------------------------------------------------ checks (implementation-parametrised)
def check_diag_forward(fwd):
    rng = _rng(1)
    for cplx in (False, True):
        for L in (1, 2, 5, 8):
            M, N = 3, 4
            if cplx:
                lam = 0.9 * np.exp(1j * rng.uniform(0, 3, (M, N))) * rng.uniform(0.2, 1, (M, N))
                v, x0 = _cplx(rng, M, L, N), _cplx(rng, M, N)
            else:
                lam, v, x0 = rng.uniform(-0.95, 0.95, (M, N)), rng.standard_normal((M, L, N)), rng.standard_normal((M, N))
            # closed form: x_t = lam^(t+1) x0 + sum_{s<=t} lam^(t-s) v_s
            want = np.stack(
                [lam ** (t + 1) * x0 + sum(lam ** (t - s) * v[:, s] for s in range(t + 1)) for t in range(L)], 1
            )
            got = fwd(lam, v, x0)
            if O.rel_err(got, want) > TOL:
                return False
            want0 = want - np.stack([lam ** (t + 1) * x0 for t in range(L)], 1)
            if O.rel_err(fwd(lam, v, None), want0) > TOL:
                return False
    return True


def check_diag_backward(bwd):
    rng = _rng(2)
    for cplx in (False, True):
        for L, with_x0 in ((1, True), (7, True), (7, False), (33, True)):
            M, N = 2, 5
            if cplx:
                lam = rng.uniform(0.3, 0.95, (M, N)) * np.exp(1j * rng.uniform(0, 3, (M, N)))
                v, x0, g = _cplx(rng, M, L, N), _cplx(rng, M, N), _cplx(rng, M, L, N)
            else:
                lam = rng.uniform(-0.95, 0.95, (M, N))
                v, x0, g = rng.standard_normal((M, L, N)), rng.standard_normal((M, N)), rng.standard_normal((M, L, N))
            x0 = x0 if with_x0 else None
            out = O.diag_forward(lam, v, x0)
            want_lam, want_v, want_x0 = _vjp(_torch_diag_loop, [lam, v, x0], g)
            glam, gv, gx0 = bwd(g, lam, out, x0)
            if O.rel_err(glam, want_lam) > TOL or O.rel_err(gv, want_v) > TOL:
                return False
            if with_x0 and O.rel_err(gx0, want_x0) > TOL:
                return False
    return True


def check_selective(fwd, bwd):
    rng = _rng(3)
    for cplx in (False, True):
        for L, with_x0 in ((1, True), (6, False), (19, True)):
            M, N = 2, 3
            if cplx:
                a = rng.uniform(0.2, 0.95, (M, L, N)) * np.exp(1j * rng.uniform(0, 3, (M, L, N)))
                v, x0, g = _cplx(rng, M, L, N), _cplx(rng, M, N), _cplx(rng, M, L, N)
            else:
                a = rng.uniform(-0.95, 0.95, (M, L, N))
                v, x0, g = rng.standard_normal((M, L, N)), rng.standard_normal((M, N)), rng.standard_normal((M, L, N))
            x0 = x0 if with_x0 else None
            want_out = _torch_sel_loop(*(torch.tensor(t) if t is not None else None for t in (a, v, x0))).numpy()
            out = fwd(a, v, x0)
            if O.rel_err(out, want_out) > TOL:
                return False
            want_a, want_v, want_x0 = _vjp(_torch_sel_loop, [a, v, x0], g)
            glam, gv, gx0 = bwd(g, a, out, x0)
            if O.rel_err(glam, want_a) > TOL or O.rel_err(gv, want_v) > TOL:
                return False
            if with_x0 and O.rel_err(gx0, want_x0) > TOL:
                return False
    return True


def _mamba_inputs(rng, B, L, D, N, with_h0):
    return dict(
        draw=rng.normal(-1.0, 1.0, (B, L, D)),
        A=-np.exp(rng.normal(0.0, 0.5, (D, N))),
        Bt=rng.standard_normal((B, L, N)),
        Ct=rng.standard_normal((B, L, N)),
        u=rng.standard_normal((B, L, D)),
        z=rng.standard_normal((B, L, D)),
        Dp=rng.standard_normal(D),
        h0=rng.standard_normal((B, D, N)) * 0.5 if with_h0 else None,
    )


def check_mamba(fwd, bwd):
    rng = _rng(4)
    for (B, L, D, N), with_h0 in (((2, 9, 3, 4), True), ((1, 1, 2, 3), True), ((2, 17, 5, 2), False)):
        x = _mamba_inputs(rng, B, L, D, N, with_h0)
        args = [x[k] for k in ("draw", "A", "Bt", "Ct", "u", "z", "Dp", "h0")]
        want_out, want_h = (t.detach().numpy() for t in _torch_mamba_textbook(*(torch.tensor(a) if a is not None else None for a in args)))
        out, h_last = fwd(*args)
        if O.rel_err(out, want_out) > TOL or O.rel_err(h_last, want_h) > TOL:
            return False
        gout = rng.standard_normal((B, L, D))
        ghl = rng.standard_normal((B, D, N))
        for gh in (ghl, None):
            want = _vjp(_torch_mamba_textbook, args, (gout, gh))
            got = bwd(gout, gh, *args)
            # got: gdraw, gA, gBt, gCt, gu, gz, gDp, gh0 ; want in input order
            order = [0, 1, 2, 3, 4, 5, 6]
            pairs = [(got[0], want[0]), (got[1], want[1]), (got[2], want[2]), (got[3], want[3]), (got[4], want[4]),
                     (got[5], want[5]), (got[6], want[6])]
            del order
            if with_h0:
                pairs.append((got[7], want[7]))
            for a_, b_ in pairs:
                if O.rel_err(a_, b_) > 1e-9:
                    return False
    return True


def check_allpole(fwd, bwd):
    rng = _rng(5)
    for lanes, L, na, with_y0 in ((3, 40, 3, True), (2, 1, 2, True), (2, 2, 4, True), (4, 25, 1, False), (2, 30, 8, True)):
        a = rng.standard_normal((lanes, na)) * 0.25
        w = rng.standard_normal((lanes, L))
        y0 = rng.standard_normal((lanes, na)) if with_y0 else None
        want = np.stack(
            [
                scipy.signal.lfilter(
                    [1.0], np.r_[1.0, a[i]], w[i],
                    zi=scipy.signal.lfiltic([1.0], np.r_[1.0, a[i]], y0[i]) if y0 is not None else np.zeros(na),
                )[0]
                for i in range(lanes)
            ]
        )
        y = fwd(a, w, y0)
        if O.rel_err(y, want) > TOL:
            return False
        g = rng.standard_normal((lanes, L))
        want_a, want_w, want_y0 = _vjp(_torch_allpole_loop, [a, w, y0], g)
        ga, gw, gy0 = bwd(g, a, y, y0)
        if O.rel_err(ga, want_a) > TOL or O.rel_err(gw, want_w) > TOL:
            return False
        if with_y0 and O.rel_err(gy0, want_y0) > TOL:
            return False
    return True


# ------------------------------------------------------------------------ the oracle passes
def test_diag_forward_closed_form():
    assert check_diag_forward(O.diag_forward)


def test_diag_backward_autograd():
    assert check_diag_backward(O.diag_backward)


def test_selective_autograd():
    assert check_selective(O.selective_forward, O.selective_backward)


def test_selective_constant_coefficient_is_diag():
    rng = _rng(6)
    M, L, N = 3, 12, 4
    lam = rng.uniform(-0.9, 0.9, (M, N))
    v, x0, g = rng.standard_normal((M, L, N)), rng.standard_normal((M, N)), rng.standard_normal((M, L, N))
    a = np.broadcast_to(lam[:, None], (M, L, N))
    assert O.rel_err(O.selective_forward(a, v, x0), O.diag_forward(lam, v, x0)) < TOL
    out = O.diag_forward(lam, v, x0)
    gs = O.selective_backward(g, a, out, x0)
    gd = O.diag_backward(g, lam, out, x0)
    assert O.rel_err(gs[0].sum(1), gd[0]) < TOL
    assert O.rel_err(gs[1], gd[1]) < TOL and O.rel_err(gs[2], gd[2]) < TOL


def test_mamba_textbook_and_autograd():
    assert check_mamba(O.mamba_forward, O.mamba_backward)


def test_mamba_special_cases():
    rng = _rng(7)
    B, L, D, N = 2, 6, 3, 4
    x = _mamba_inputs(rng, B, L, D, N, True)
    # delta -> 0: lam = 1, no injection; the state stays h0
    x0 = dict(x, draw=np.full((B, L, D), -60.0))
    out, h = O.mamba_forward(**x0)
    assert np.allclose(h, x["h0"], atol=1e-20)
    want = (np.einsum("bdn,bln->bld", x["h0"], x["Ct"]) + x["Dp"] * x["u"]) * x["z"] / (1 + np.exp(-x["z"]))
    assert O.rel_err(out, want) < TOL
    # N = 1: each channel is a scalar selective recurrence a_t = exp(delta A), v_t = delta u B
    x1 = _mamba_inputs(rng, B, L, D, 1, True)
    d = O.softplus(x1["draw"])
    a = np.exp(d * x1["A"][:, 0])  # [B, L, D]
    v = d * x1["u"] * x1["Bt"]  # Bt [B, L, 1] broadcasts over D
    h = O.selective_forward(a, v, x1["h0"][:, :, 0])
    _, _, hs = O.mamba_forward(**x1, return_states=True)
    assert O.rel_err(hs[..., 0], h) < TOL


def test_allpole_lfilter_and_autograd():
    assert check_allpole(O.allpole_forward, O.allpole_backward)


def test_allpole_matches_companion_scan():
    from tsfast_amd.dynonet.core import companion, linear_recurrence

    rng = _rng(8)
    lanes, L, na = 4, 37, 3
    a = rng.standard_normal((lanes, na)) * 0.3
    w = rng.standard_normal((lanes, L))
    y0 = rng.standard_normal((lanes, na))
    x = linear_recurrence(
        companion(torch.tensor(a)), torch.nn.functional.pad(torch.tensor(w).unsqueeze(-1), (0, na - 1)), torch.tensor(y0)
    )
    assert O.rel_err(O.allpole_forward(a, w, y0), x[..., 0].numpy()) < TOL


# ------------------------------------------------------------------------ the checks reject broken oracles
def _conj_glam(g, lam, out, x0=None):
    glam, gv, gx0 = O.diag_backward(g, lam, out, x0)
    return np.conj(glam), gv, gx0


def _no_conj_gx0(g, lam, out, x0=None):
    glam, gv, gx0 = O.diag_backward(g, lam, out, x0)
    return glam, gv, (None if gx0 is None else lam * gv[:, 0])


def _gv_shifted(g, lam, out, x0=None):
    glam, gv, gx0 = O.diag_backward(g, lam, out, x0)
    return glam, np.roll(gv, 1, axis=1), gx0


def _fwd_off_by_one(lam, v, x0=None):
    out = O.diag_forward(lam, v, x0)
    return np.concatenate([out[:, :1], out[:, :-1]], axis=1) if out.shape[1] > 1 else out * lam


@pytest.mark.parametrize("mutant", [_conj_glam, _no_conj_gx0, _gv_shifted])
def test_diag_backward_check_rejects(mutant):
    assert not check_diag_backward(mutant)


def test_diag_forward_check_rejects():
    assert not check_diag_forward(_fwd_off_by_one)


def _sel_glam_next(g, a, out, x0=None):
    glam, gv, gx0 = O.selective_backward(g, a, out, x0)
    return np.roll(glam, -1, axis=1), gv, gx0


def test_selective_check_rejects():
    assert not check_selective(O.selective_forward, _sel_glam_next)


def _mamba_no_sigmoid(gout, ghlast, draw, *rest):
    res = list(O.mamba_backward(gout, ghlast, draw, *rest))
    res[0] = res[0] / (1.0 / (1.0 + np.exp(-np.asarray(draw))))  # drop softplus' derivative
    return tuple(res)


def _mamba_half_gA(*args):
    res = list(O.mamba_backward(*args))
    res[1] = res[1] * 0.5
    return tuple(res)


def _mamba_gh0_no_lam(gout, ghlast, draw, A, Bt, Ct, u, z, Dp, h0=None):
    res = list(O.mamba_backward(gout, ghlast, draw, A, Bt, Ct, u, z, Dp, h0))
    if h0 is not None:
        res[7] = res[7] / np.exp(O.softplus(np.asarray(draw))[:, 0, :, None] * np.asarray(A)[None])
    return tuple(res)


def _mamba_fwd_no_gate(draw, A, Bt, Ct, u, z, Dp, h0=None):
    out, h = O.mamba_forward(draw, A, Bt, Ct, u, z, Dp, h0)
    return out / (1.0 / (1.0 + np.exp(-np.asarray(z)))), h


@pytest.mark.parametrize("mutant", [_mamba_no_sigmoid, _mamba_half_gA, _mamba_gh0_no_lam])
def test_mamba_check_rejects_backward(mutant):
    assert not check_mamba(O.mamba_forward, mutant)


def test_mamba_check_rejects_forward():
    assert not check_mamba(_mamba_fwd_no_gate, O.mamba_backward)


def _allpole_sign(a, w, y0=None):
    return O.allpole_forward(-np.asarray(a), w, y0)


def _allpole_y0_oldest_first(a, w, y0=None):
    return O.allpole_forward(a, w, None if y0 is None else np.asarray(y0)[:, ::-1])


def _allpole_no_head_taps(g, a, y, y0=None):
    ga, gw, gy0 = O.allpole_backward(g, a, y, None)
    return ga, gw, (None if y0 is None else O.allpole_backward(g, a, y, y0)[2])


@pytest.mark.parametrize("mutant", [_allpole_sign, _allpole_y0_oldest_first])
def test_allpole_check_rejects_forward(mutant):
    assert not check_allpole(mutant, O.allpole_backward)


def test_allpole_check_rejects_backward():
    assert not check_allpole(O.allpole_forward, _allpole_no_head_taps)


# ------------------------------------------------------------------------ causal depthwise conv + SiLU
def _torch_conv_silu(x, tail, w, bias):
    """F.conv1d (cross-correlation, groups = D) over cat(tail, x) along time, then SiLU."""
    xb = torch.cat((tail, x.transpose(1, 2)), dim=-1)  # [B, D, K-1+L]
    p = torch.nn.functional.conv1d(xb, w[:, None, :], bias, groups=w.shape[0])
    return torch.nn.functional.silu(p).transpose(1, 2)


def check_conv(fwd, bwd):
    rng = _rng(7)
    for Bsz, L, D, K, with_bias in ((2, 9, 5, 4, True), (1, 2, 3, 4, True), (3, 1, 2, 2, False), (2, 13, 4, 8, True)):
        x = rng.standard_normal((Bsz, L, D))
        tail = rng.standard_normal((Bsz, D, K - 1))
        w = rng.standard_normal((D, K)) * 0.5
        bias = rng.standard_normal(D) if with_bias else None
        gy = rng.standard_normal((Bsz, L, D))
        args = (x, tail, w, bias)
        want = _torch_conv_silu(*[None if a is None else torch.tensor(a) for a in args]).numpy()
        if O.rel_err(fwd(*args), want) > TOL:
            return False
        gw_ = _vjp(_torch_conv_silu, args, gy)
        got = bwd(gy, *args)
        for g_got, g_want in zip(got, gw_):
            if (g_got is None) != (g_want is None):
                return False
            if g_got is not None and O.rel_err(g_got, g_want) > TOL:
                return False
        # zero tail: the reference test's form, conv1d with K-1 zero padding cut to L steps
        # (tests/test_mamba.py:60)
        z = np.zeros_like(tail)
        pad = torch.nn.functional.conv1d(
            torch.tensor(x).transpose(1, 2), torch.tensor(w)[:, None, :], None if bias is None else torch.tensor(bias),
            padding=K - 1, groups=D,
        )[..., :L]
        if O.rel_err(fwd(x, z, w, bias), torch.nn.functional.silu(pad).transpose(1, 2).numpy()) > TOL:
            return False
    return True


def test_conv_silu_conv1d_and_autograd():
    assert check_conv(O.conv_silu_forward, O.conv_silu_backward)


def _conv_flipped_taps(x, tail, w, bias=None):
    return O.conv_silu_forward(x, tail, np.asarray(w)[:, ::-1], bias)


def _conv_tail_reversed(x, tail, w, bias=None):
    return O.conv_silu_forward(x, np.asarray(tail)[..., ::-1], w, bias)


def _conv_no_silu_prime(gy, x, tail, w, bias=None):
    # gradient of p instead of silu(p): drops the silu' factor
    p, _ = O._conv_pre(x, tail, w, bias)
    s = 1.0 / (1.0 + np.exp(-p))
    return O.conv_silu_backward(np.asarray(gy) / (1.0 + p * (1.0 - s)), x, tail, w, bias)


def _conv_tail_grad_zero(gy, x, tail, w, bias=None):
    gx, gtail, gw, gb = O.conv_silu_backward(gy, x, tail, w, bias)
    return gx, np.zeros_like(gtail), gw, gb


@pytest.mark.parametrize("mutant", [_conv_flipped_taps, _conv_tail_reversed])
def test_conv_check_rejects_forward(mutant):
    assert not check_conv(mutant, O.conv_silu_backward)


@pytest.mark.parametrize("mutant", [_conv_no_silu_prime, _conv_tail_grad_zero])
def test_conv_check_rejects_backward(mutant):
    assert not check_conv(O.conv_silu_forward, mutant)


# ------------------------------------------------------------------------ dynoNet G-block (FIR + all-pole + input sum)
def _torch_gblock(u, b, a, u_tail, x0):
    """LinearDynamicalOperator.forward written as the reference does it (dynonet/core.py:212-258):
    grouped conv1d with flipped taps over cat(u_tail, u), the all-pole recurrence as a plain
    sequential loop per pair (input-major pairs), then the sum over inputs; returns (y, x_last)."""
    Bsz, L, I = u.shape
    O_, _, nb = b.shape
    na = a.shape[-1]
    P = I * O_
    ubuf = torch.cat((u_tail, u), dim=1)
    weight = b.permute(1, 0, 2).reshape(P, 1, nb).flip(-1)
    w = torch.nn.functional.conv1d(ubuf.transpose(1, 2), weight, groups=I)
    ap = a.permute(1, 0, 2).reshape(P, na)
    s = [x0[:, :, k] for k in range(na)]
    ys = []
    for t in range(L):
        yt = w[:, :, t] - sum(ap[:, i] * s[i] for i in range(na))
        ys.append(yt)
        s = [yt] + s[:-1]
    yp = torch.stack(ys, -1) if L > 0 else w
    y = yp.view(Bsz, I, O_, L).sum(1).transpose(1, 2)
    return y, torch.stack(s, -1)


def check_gblock(fwd, bwd):
    rng = _rng(11)
    for Bsz, L, I, O_, nb, na in ((2, 23, 3, 2, 4, 2), (1, 9, 2, 4, 8, 3), (3, 2, 2, 2, 3, 4), (2, 30, 1, 1, 1, 1),
                                  (1, 17, 4, 2, 6, 2)):
        P = I * O_
        u = rng.standard_normal((Bsz, L, I))
        b = rng.standard_normal((O_, I, nb)) * 0.5
        a = rng.uniform(-0.3, 0.3, (O_, I, na))
        ut = rng.standard_normal((Bsz, nb - 1, I))
        x0 = rng.standard_normal((Bsz, P, na))
        args = (u, b, a, ut, x0)
        want_y, want_xl = (t.numpy() for t in _torch_gblock(*[torch.tensor(x) for x in args]))
        y, xl, _ = fwd(*args)
        if O.rel_err(y, want_y) > TOL or O.rel_err(xl, want_xl) > TOL:
            return False
        gy = rng.standard_normal((Bsz, L, O_))
        gxl = rng.standard_normal((Bsz, P, na))
        want = _vjp(_torch_gblock, list(args), (gy, gxl))
        gu, gut, gb, ga, gx0 = bwd(gy, gxl, *args)
        for g_got, g_want in zip((gu, gb, ga, gut, gx0), want):  # the order of args
            if O.rel_err(g_got, g_want) > TOL:
                return False
    return True


def test_gblock_conv1d_loop_and_autograd():
    assert check_gblock(O.gblock_forward, O.gblock_backward)


def _gblock_output_major(u, b, a, u_tail, x0):
    # pairs flattened output-major (o * I + j) instead of input-major
    Bsz, L, I = np.shape(u)
    O_ = np.shape(b)[0]
    y, xl, yp = O.gblock_forward(u, b, a, u_tail, x0)
    yp2 = yp.reshape(Bsz, O_, I, L)
    return yp2.sum(2).transpose(0, 2, 1), xl, yp


def _gblock_no_tail(u, b, a, u_tail, x0):
    return O.gblock_forward(u, b, a, np.zeros_like(u_tail), x0)


def _gblock_taps_unflipped(u, b, a, u_tail, x0):
    return O.gblock_forward(u, np.asarray(b)[:, :, ::-1], a, u_tail, x0)


def _gblock_drop_gxlast(gy, g_xlast, *args):
    return O.gblock_backward(gy, None, *args)


def _gblock_gb_unsummed_batch(gy, g_xlast, u, b, a, u_tail, x0):
    gu, gut, gb, ga, gx0 = O.gblock_backward(gy, g_xlast, u, b, a, u_tail, x0)
    return gu, gut, gb / np.shape(u)[0], ga, gx0


@pytest.mark.parametrize("mutant", [_gblock_output_major, _gblock_no_tail, _gblock_taps_unflipped])
def test_gblock_check_rejects_forward(mutant):
    assert not check_gblock(mutant, O.gblock_backward)


@pytest.mark.parametrize("mutant", [_gblock_drop_gxlast, _gblock_gb_unsummed_batch])
def test_gblock_check_rejects_backward(mutant):
    assert not check_gblock(O.gblock_forward, mutant)


# ------------------------------------------------------------------------ constant-matrix recurrence
def _torch_linrec_loop(A, v, x0):
    x = torch.zeros_like(v[:, 0]) if x0 is None else x0
    outs = []
    for t in range(v.shape[1]):
        x = torch.einsum("mij,mj->mi", A, x) + v[:, t]
        outs.append(x)
    return torch.stack(outs, 1)


def check_linrec(fwd, bwd):
    """Forward: the matrix-power closed form ``x_t = A^(t+1) x0 + sum_{s<=t} A^(t-s) v_s``.
    Backward: torch float64 autograd through a sequential loop (all of gA, gv, gx0)."""
    rng = _rng(11)
    for M, L, n, with_x0 in ((3, 9, 3, True), (2, 1, 2, True), (2, 6, 4, False), (4, 7, 1, True), (2, 5, 5, True)):
        A = rng.standard_normal((M, n, n)) * (0.8 / np.sqrt(n))
        v = rng.standard_normal((M, L, n))
        x0 = rng.standard_normal((M, n)) if with_x0 else None
        P = [np.stack([np.linalg.matrix_power(A[m], p) for m in range(M)]) for p in range(L + 1)]
        want = np.stack(
            [
                sum(np.einsum("mij,mj->mi", P[t - s], v[:, s]) for s in range(t + 1))
                + (np.einsum("mij,mj->mi", P[t + 1], x0) if with_x0 else 0.0)
                for t in range(L)
            ],
            1,
        )
        out = fwd(A, v, x0)
        if O.rel_err(out, want) > TOL:
            return False
        g = rng.standard_normal((M, L, n))
        want_A, want_v, want_x0 = _vjp(_torch_linrec_loop, [A, v, x0], g)
        gA, gv, gx0 = bwd(g, A, out, x0)
        if O.rel_err(gA, want_A) > TOL or O.rel_err(gv, want_v) > TOL:
            return False
        if with_x0 and O.rel_err(gx0, want_x0) > TOL:
            return False
    return True


def test_linrec_closed_form_and_autograd():
    assert check_linrec(O.linrec_forward, O.linrec_backward)


def test_linrec_special_cases():
    """A diagonal matrix is n independent diagonal scans; a companion matrix with input
    (w_t, 0, ..., 0) is the all-pole filter, its first state component the output."""
    rng = _rng(12)
    M, L, n = 3, 17, 3
    lam = rng.uniform(-0.9, 0.9, (M, n))
    v, x0, g = rng.standard_normal((M, L, n)), rng.standard_normal((M, n)), rng.standard_normal((M, L, n))
    A = np.stack([np.diag(lam[m]) for m in range(M)])
    out = O.linrec_forward(A, v, x0)
    assert O.rel_err(out, O.diag_forward(lam, v, x0)) < TOL
    gA, gv, gx0 = O.linrec_backward(g, A, out, x0)
    glam, gvd, gx0d = O.diag_backward(g, lam, out, x0)
    assert O.rel_err(np.diagonal(gA, axis1=1, axis2=2), glam) < TOL
    assert O.rel_err(gv, gvd) < TOL and O.rel_err(gx0, gx0d) < TOL
    a = rng.standard_normal((M, n)) * 0.3
    w = rng.standard_normal((M, L))
    y0 = rng.standard_normal((M, n))
    C = np.zeros((M, n, n))
    C[:, 0, :] = -a
    C[:, 1:, :-1] = np.eye(n - 1)
    vc = np.zeros((M, L, n))
    vc[:, :, 0] = w
    assert O.rel_err(O.linrec_forward(C, vc, y0)[:, :, 0], O.allpole_forward(a, w, y0)) < TOL


def _linrec_transposed(A, v, x0=None):
    return O.linrec_forward(np.swapaxes(np.asarray(A), 1, 2), v, x0)


def _linrec_bwd_adjoint_untransposed(g, A, out, x0=None):
    return O.linrec_backward(g, np.swapaxes(np.asarray(A), 1, 2), out, x0)


def _linrec_bwd_gA_transposed(g, A, out, x0=None):
    gA, gv, gx0 = O.linrec_backward(g, A, out, x0)
    return np.swapaxes(gA, 1, 2), gv, gx0


def _linrec_bwd_prev_off_by_one(g, A, out, x0=None):
    gA, gv, gx0 = O.linrec_backward(g, A, out, x0)
    return np.einsum("mti,mtj->mij", gv, np.asarray(out, dtype=np.float64)), gv, gx0


def test_linrec_check_rejects_forward():
    assert not check_linrec(_linrec_transposed, O.linrec_backward)


@pytest.mark.parametrize(
    "mutant", [_linrec_bwd_adjoint_untransposed, _linrec_bwd_gA_transposed, _linrec_bwd_prev_off_by_one]
)
def test_linrec_check_rejects_backward(mutant):
    assert not check_linrec(O.linrec_forward, mutant)


def test_linrec_blocked_scan_matches_oracle():
    """The CPU route of linear_recurrence (the blocked two-level matrix scan and its adjoint, which
    every non-GPU call and every unsupported shape takes) against the oracle, with A broadcast
    over a batch dim so the adjoint's grad_A is summed back."""
    from tsfast_amd.dynonet.core import linear_recurrence

    rng = _rng(13)
    Bb, P, L, n = 2, 3, 37, 5  # n = 5: beyond the GPU kernel's range
    A = rng.standard_normal((P, n, n)) * (0.8 / np.sqrt(n))
    v = rng.standard_normal((Bb, P, L, n))
    x0 = rng.standard_normal((Bb, P, n))
    g = rng.standard_normal((Bb, P, L, n))
    At, vt, x0t = (torch.tensor(t, requires_grad=True) for t in (A, v, x0))
    x = linear_recurrence(At, vt, x0t)
    x.backward(torch.tensor(g))
    Ab = np.broadcast_to(A, (Bb, P, n, n)).reshape(Bb * P, n, n)
    want = O.linrec_forward(Ab, v.reshape(Bb * P, L, n), x0.reshape(Bb * P, n))
    assert O.rel_err(x.detach().numpy().reshape(Bb * P, L, n), want) < TOL
    gA, gv, gx0 = O.linrec_backward(g.reshape(Bb * P, L, n), Ab, want, x0.reshape(Bb * P, n))
    assert O.rel_err(At.grad.numpy(), gA.reshape(Bb, P, n, n).sum(0)) < TOL
    assert O.rel_err(vt.grad.numpy().reshape(Bb * P, L, n), gv) < TOL
    assert O.rel_err(x0t.grad.numpy().reshape(Bb * P, n), gx0) < TOL


# ------------------------------------------------------------------------ projected diagonal scan
def _torch_projscan_loop(u, W_re, W_im, lam, C_re, C_im, x0):
    W = torch.complex(W_re, W_im)
    C = torch.complex(C_re, C_im)
    x = torch.zeros(u.shape[0], W.shape[0], dtype=torch.complex128) if x0 is None else x0
    ys = []
    for t in range(u.shape[1]):
        x = lam * x + u[:, t].to(torch.complex128) @ W.T
        ys.append((x @ C.T).real)
    return torch.stack(ys, 1), x


def check_projscan(fwd, bwd):
    """Forward: the closed form ``y_t = Re C (lam^(t+1) x0 + sum_{s<=t} lam^(t-s) W u_s)`` with
    explicit powers. Backward: torch float64/complex128 autograd through a per-step loop, for
    the upstream gradient of y and of the returned last state (all seven gradients)."""
    rng = _rng(14)
    for Bsz, L, d, n, o, with_x0 in ((2, 7, 3, 4, 2, True), (1, 1, 2, 3, 3, True), (3, 5, 4, 2, 5, False)):
        u = rng.standard_normal((Bsz, L, d))
        W_re, W_im = rng.standard_normal((n, d)), rng.standard_normal((n, d))
        lam = rng.uniform(0.5, 0.95, n) * np.exp(1j * rng.uniform(0, np.pi, n))
        C_re, C_im = rng.standard_normal((o, n)), rng.standard_normal((o, n))
        x0 = _cplx(rng, Bsz, n) if with_x0 else None
        W, C = W_re + 1j * W_im, C_re + 1j * C_im
        want = np.zeros((Bsz, L, o))
        for b in range(Bsz):
            for t in range(L):
                state = sum(lam ** (t - s) * (W @ u[b, s]) for s in range(t + 1))
                if with_x0:
                    state = state + lam ** (t + 1) * x0[b]
                want[b, t] = (C @ state).real
        y, x = fwd(u, W_re, W_im, lam, C_re, C_im, x0)
        if O.rel_err(y, want) > TOL:
            return False
        gy, g_xl = rng.standard_normal((Bsz, L, o)), _cplx(rng, Bsz, n)
        want_g = _vjp(_torch_projscan_loop, [u, W_re, W_im, lam, C_re, C_im, x0], (gy, g_xl))
        got = bwd(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0)
        for gw, gg in zip(want_g, got):
            if gw is not None and O.rel_err(gg, gw) > TOL:
                return False
    return True


def test_projscan_closed_form_and_autograd():
    assert check_projscan(O.projscan_forward, O.projscan_backward)


def test_projections_match_interleaved_real_gemm():
    """complex_in_proj / real_out_proj as the reference computes them: one real GEMM against
    the interleaved weight ``[d, 2n]`` (re, im per state) read as complex pairs, and one real
    GEMM of the interleaved state against ``[o, 2n]`` with ``-W_im`` in the odd columns."""
    rng = _rng(15)
    u = rng.standard_normal((2, 5, 3))
    W_re, W_im = rng.standard_normal((4, 3)), rng.standard_normal((4, 3))
    inter = np.stack((W_re, W_im), -1).transpose(1, 0, 2).reshape(3, 8)
    v = (u @ inter).reshape(2, 5, 4, 2)
    assert O.rel_err(O.complex_in_proj(u, W_re, W_im), v[..., 0] + 1j * v[..., 1]) < TOL
    x = _cplx(rng, 2, 5, 4)
    C_re, C_im = rng.standard_normal((6, 4)), rng.standard_normal((6, 4))
    Wo = np.stack((C_re, -C_im), -1).reshape(6, 8)
    xr = np.stack((x.real, x.imag), -1).reshape(2, 5, 8)
    assert O.rel_err(O.real_out_proj(x, C_re, C_im), xr @ Wo.T) < TOL


def _projscan_fwd_readout_conj(u, W_re, W_im, lam, C_re, C_im, x0=None):
    y, x = O.projscan_forward(u, W_re, W_im, lam, C_re, C_im, x0)
    return O.real_out_proj(x, C_re, -np.asarray(C_im)), x


def _projscan_bwd_gu_no_conj(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0=None):
    r = list(O.projscan_backward(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0))
    r[0] = O.projscan_backward(gy, g_xl, u, W_re, -np.asarray(W_im), lam, C_re, C_im, x, x0)[0]
    return tuple(r)


def _projscan_bwd_gc_im_sign(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0=None):
    r = list(O.projscan_backward(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0))
    r[5] = -r[5]
    return tuple(r)


def _projscan_bwd_glam_current_state(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0=None):
    r = list(O.projscan_backward(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0))
    G = O.diag_backward(np.asarray(gy) @ np.conj(np.asarray(C_re) + 1j * np.asarray(C_im)), np.broadcast_to(lam, x.shape[::2]), x, x0)[1]
    r[3] = (G * np.conj(x)).sum((0, 1))
    return tuple(r)


def _projscan_bwd_no_state_grad(gy, g_xl, u, W_re, W_im, lam, C_re, C_im, x, x0=None):
    return O.projscan_backward(gy, None, u, W_re, W_im, lam, C_re, C_im, x, x0)


def test_projscan_check_rejects_forward():
    assert not check_projscan(_projscan_fwd_readout_conj, O.projscan_backward)


@pytest.mark.parametrize(
    "mutant",
    [_projscan_bwd_gu_no_conj, _projscan_bwd_gc_im_sign, _projscan_bwd_glam_current_state, _projscan_bwd_no_state_grad],
)
def test_projscan_check_rejects_backward(mutant):
    assert not check_projscan(O.projscan_forward, mutant)


# ------------------------------------------------------------------------ NSS chunked adjoint
def _adjoint_steps(jt, gout):
    """The adjoint at every step by its definition, gy_t = gout_t + jt[t+1] gy_{t+1}."""
    B, L, n = gout.shape
    gy = np.zeros((B, L, n))
    nxt = np.zeros((B, n))
    for t in range(L - 1, -1, -1):
        gy[:, t] = gout[:, t] + (np.einsum("bij,bj->bi", jt[:, t + 1], nxt) if t + 1 < L else 0.0)
        nxt = gy[:, t]
    return gy


def check_mat_adjoint(fn):
    """Boundaries against the step-by-step adjoint (gy at every chunk's first step, zero past the
    end) on ragged chunkings, and the diagonal special case against the selective scan's adjoint
    (G_t = g_t + a_{t+1} G_{t+1} with a_t the diagonal of jt[t])."""
    rng = _rng(16)
    for B, L, n, cl in ((2, 37, 3, 8), (1, 5, 4, 5), (3, 64, 2, 64), (2, 33, 5, 1), (1, 20, 1, 7), (2, 50, 6, 100)):
        jt = rng.standard_normal((B, L, n, n)) * (0.9 / np.sqrt(n))
        gout = rng.standard_normal((B, L, n))
        C = -(-L // cl)
        want = np.zeros((B, C + 1, n))
        want[:, :C] = _adjoint_steps(jt, gout)[:, ::cl][:, :C]
        got = np.asarray(fn(jt, gout, cl))
        if got.shape != want.shape or O.rel_err(got, want) > TOL:
            return False
    B, L, n, cl = 2, 40, 4, 6
    a = rng.uniform(0.2, 0.95, (B, L, n))
    jt = np.zeros((B, L, n, n))
    for i in range(n):
        jt[:, :, i, i] = a[:, :, i]
    gout = rng.standard_normal((B, L, n))
    _, gv, _ = O.selective_backward(gout, a, np.zeros((B, L, n)))
    got = np.asarray(fn(jt, gout, cl))
    return O.rel_err(got[:, :-1], gv[:, ::cl]) <= TOL and not np.any(got[:, -1])


def test_mat_adjoint_step_recurrence_and_diagonal_case():
    assert check_mat_adjoint(O.mat_adjoint_bounds)


def _mat_adjoint_transposed(jt, gout, cl):
    return O.mat_adjoint_bounds(np.swapaxes(jt, -1, -2), gout, cl)


def _mat_adjoint_current_step(jt, gout, cl):  # A_t instead of A_{t+1}
    return O.mat_adjoint_bounds(np.roll(jt, 1, axis=1), gout, cl)


def _mat_adjoint_chunk_end_dropped(jt, gout, cl):  # each chunk's last gout left out
    g = np.array(gout, copy=True)
    g[:, cl - 1 :: cl] = 0.0
    return O.mat_adjoint_bounds(jt, g, cl)


def _mat_adjoint_shifted(jt, gout, cl):  # the boundary of the next chunk
    return np.roll(O.mat_adjoint_bounds(jt, gout, cl), -1, axis=1)


@pytest.mark.parametrize(
    "mutant", [_mat_adjoint_transposed, _mat_adjoint_current_step, _mat_adjoint_chunk_end_dropped, _mat_adjoint_shifted]
)
def test_mat_adjoint_check_rejects(mutant):
    assert not check_mat_adjoint(mutant)
