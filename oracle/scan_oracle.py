"""fp64 sequential oracle for tsfast's scan family — TEST INFRASTRUCTURE ONLY.

This module is the checker, never the thing measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it. The product path
(``tsfast_amd``) never calls into ``oracle/``.

Each function restates the reference algorithm as a per-time-step loop in float64 (complex128
for complex lanes), vectorised over lanes with numpy, following the cited reference lines.
Backward functions are the closed-form adjoints the reference derives; they take the upstream
gradient in torch's convention (conjugate Wirtinger for complex tensors), so they equal
``torch.autograd.grad`` through the forward loop.

Pinning (see tests/test_oracle.py): every function here is checked against an independent
route — brute-force closed-form sums, ``scipy.signal.lfilter``, a textbook selective-scan
written as einsums, the companion-matrix doubling scan, and torch float64 autograd through
sequential loops — plus special cases (constant coefficients reduce the selective scan to the
diagonal one, delta -> 0 makes Mamba the identity map on the state, N = 1 reduces it to a
scalar recurrence); the G-block functions compose the FIR and all-pole restatements and are
checked against autograd through the reference's grouped-conv1d formulation; the constant-matrix
recurrence is checked against matrix-power closed forms, torch float64 autograd through a loop,
and its diagonal and companion special cases (the diagonal scan and the all-pole filter); the
chunked matrix adjoint is checked against the step-by-step adjoint recurrence and its diagonal
special case (the selective scan's adjoint).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "rel_err",
    "diag_forward",
    "diag_backward",
    "selective_forward",
    "selective_backward",
    "softplus",
    "mamba_forward",
    "mamba_backward",
    "allpole_forward",
    "allpole_backward",
    "conv_silu_forward",
    "conv_silu_backward",
    "gblock_forward",
    "gblock_backward",
    "linrec_forward",
    "linrec_backward",
    "complex_in_proj",
    "real_out_proj",
    "projscan_forward",
    "projscan_backward",
    "mat_adjoint_bounds",
]


def rel_err(a, b) -> float:
    """``max|a - b| / max|b|`` — the reference tests' metric (tests/test_scan.py:13-14)."""
    a = np.asarray(a)
    b = np.asarray(b)
    if b.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)) / (np.max(np.abs(b)) + 1e-30))


def _hi(x):
    x = np.asarray(x)
    return x.astype(np.complex128) if np.iscomplexobj(x) else x.astype(np.float64)


# --------------------------------------------------------------------------- diagonal scans
def diag_forward(lam, v, x0=None):
    """``x_t = lam * x_{t-1} + v_t`` on lanes: lam [M, N], v [M, L, N], x0 [M, N] or None.

    Follows tsfast/models/_core/scan.py:316-328 (the sequential loop), semantics of the
    ``tsfast::scan_diagonal`` op (:100-115).
    """
    lam, v = _hi(lam), _hi(v)
    M, L, N = v.shape
    dt = np.result_type(lam, v)
    x = np.zeros((M, N), dt) if x0 is None else _hi(x0).astype(dt)
    out = np.empty((M, L, N), dt)
    for t in range(L):
        x = lam * x + v[:, t]
        out[:, t] = x
    return out


def diag_backward(g, lam, out, x0=None):
    """Adjoint of :func:`diag_forward`: ``G_t = g_t + conj(lam) G_{t+1}``;
    ``glam = sum_t G_t conj(x_{t-1})``, ``gv = G``, ``gx0 = conj(lam) G_0``
    (tsfast/models/_core/scan.py:10-15, 118-140)."""
    g, lam, out = _hi(g), _hi(lam), _hi(out)
    M, L, N = out.shape
    dt = np.result_type(g, lam, out)
    lc = np.conj(lam)
    G = np.zeros((M, N), dt)
    gv = np.empty((M, L, N), dt)
    glam = np.zeros((M, N), dt)
    for t in range(L - 1, -1, -1):
        G = g[:, t] + lc * G
        gv[:, t] = G
        xprev = out[:, t - 1] if t > 0 else (np.zeros((M, N), dt) if x0 is None else _hi(x0))
        glam = glam + G * np.conj(xprev)
    gx0 = None if x0 is None else lc * (gv[:, 0] if L > 0 else np.zeros((M, N), dt))
    return glam, gv, gx0


def selective_forward(a, v, x0=None):
    """``x_t = a_t * x_{t-1} + v_t``: a, v [M, L, N] (tsfast/models/_core/scan.py:157-168, 316-328)."""
    a, v = _hi(a), _hi(v)
    M, L, N = v.shape
    dt = np.result_type(a, v)
    x = np.zeros((M, N), dt) if x0 is None else _hi(x0).astype(dt)
    out = np.empty((M, L, N), dt)
    for t in range(L):
        x = a[:, t] * x + v[:, t]
        out[:, t] = x
    return out


def selective_backward(g, a, out, x0=None):
    """Adjoint: ``G_t = g_t + conj(a_{t+1}) G_{t+1}``; ``glam_t = G_t conj(x_{t-1})``, ``gv = G``,
    ``gx0 = conj(a_0) G_0`` (tsfast/models/_core/scan.py:176-195)."""
    g, a, out = _hi(g), _hi(a), _hi(out)
    M, L, N = out.shape
    dt = np.result_type(g, a, out)
    G = np.zeros((M, N), dt)
    gv = np.empty((M, L, N), dt)
    glam = np.empty((M, L, N), dt)
    for t in range(L - 1, -1, -1):
        an = np.conj(a[:, t + 1]) if t + 1 < L else np.zeros((M, N), dt)
        G = g[:, t] + an * G
        gv[:, t] = G
        xprev = out[:, t - 1] if t > 0 else (np.zeros((M, N), dt) if x0 is None else _hi(x0))
        glam[:, t] = G * np.conj(xprev)
    gx0 = None if x0 is None else np.conj(a[:, 0]) * gv[:, 0]
    return glam, gv, gx0


# --------------------------------------------------------------------------- Mamba
def softplus(x):
    """torch.nn.functional.softplus with threshold 20 (mamba_triton.py:75-78)."""
    x = np.asarray(x, np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def mamba_forward(draw, A, Bt, Ct, u, z, Dp, h0=None, return_states=False):
    """Fused Mamba SSM forward (mamba_triton.py:85-157; backend_c.py:105-144):

    ``delta = softplus(draw)``, ``h_t = exp(delta_t A) h_{t-1} + delta_t u_t B_t``,
    ``out_t = (sum_n h_t C_t + Dp u_t) * z_t * sigmoid(z_t)``.
    Shapes: draw/u/z [B, L, D], A [D, N], Bt/Ct [B, L, N], Dp [D], h0 [B, D, N].
    Returns ``(out [B, L, D], h_last [B, D, N])`` (and all states ``[B, L, D, N]`` if asked).
    """
    draw, A, Bt, Ct, u, z, Dp = map(_hi, (draw, A, Bt, Ct, u, z, Dp))
    Bsz, L, D = draw.shape
    N = A.shape[-1]
    h = np.zeros((Bsz, D, N)) if h0 is None else _hi(h0).copy()
    delta = softplus(draw)
    out = np.empty((Bsz, L, D))
    hs = np.empty((Bsz, L, D, N)) if return_states else None
    for t in range(L):
        lam = np.exp(delta[:, t, :, None] * A[None])
        h = lam * h + (delta[:, t] * u[:, t])[:, :, None] * Bt[:, t, None, :]
        y = np.einsum("bdn,bn->bd", h, Ct[:, t]) + Dp * u[:, t]
        out[:, t] = y * z[:, t] * _sigmoid(z[:, t])
        if hs is not None:
            hs[:, t] = h
    if return_states:
        return out, h, hs
    return out, h


def mamba_backward(gout, ghlast, draw, A, Bt, Ct, u, z, Dp, h0=None):
    """Closed-form adjoint of :func:`mamba_forward` (mamba_triton.py:163-286; backend_c.py:149-245).

    With ``gy = gout z sigmoid(z)`` and ``G_t = gy_t C_t + lam_{t+1} G_{t+1}`` (``lam_L = 1``, so
    ``ghlast`` enters ``G_{L-1}``) and ``P_t = lam_t h_{t-1}``:
    ``gz = gout y sigmoid(z) (1 + z (1 - sigmoid(z)))``, ``gA = sum G P delta``,
    ``gdelta = sum_n G (A P + u B)``, ``gdraw = gdelta sigmoid(draw)``,
    ``gu = delta sum_n G B + gy Dp``, ``gBt = sum_d G delta u``, ``gCt = sum_d gy h``,
    ``gDp = sum gy u``, ``gh0 = lam_0 G_0``.
    Returns ``(gdraw, gA, gBt, gCt, gu, gz, gDp, gh0)`` (gh0 None when h0 is None).
    """
    draw, A, Bt, Ct, u, z, Dp, gout = map(_hi, (draw, A, Bt, Ct, u, z, Dp, gout))
    Bsz, L, D = draw.shape
    N = A.shape[-1]
    _, _, hs = mamba_forward(draw, A, Bt, Ct, u, z, Dp, h0, return_states=True)
    delta = softplus(draw)
    sig = _sigmoid(z)
    y = np.einsum("bldn,bln->bld", hs, Ct) + Dp * u
    gy = gout * z * sig
    gz = gout * y * sig * (1.0 + z * (1.0 - sig))
    G = np.zeros((Bsz, D, N)) if ghlast is None else _hi(ghlast).copy()
    gdraw = np.empty((Bsz, L, D))
    gu = np.empty((Bsz, L, D))
    gBt = np.empty((Bsz, L, N))
    gCt = np.empty((Bsz, L, N))
    gA = np.zeros((D, N))
    h_init = np.zeros((Bsz, D, N)) if h0 is None else _hi(h0)
    for t in range(L - 1, -1, -1):
        if t + 1 < L:
            G = np.exp(delta[:, t + 1, :, None] * A[None]) * G
        G = G + gy[:, t, :, None] * Ct[:, t, None, :]
        hprev = hs[:, t - 1] if t > 0 else h_init
        P = np.exp(delta[:, t, :, None] * A[None]) * hprev
        gA += np.sum(G * P * delta[:, t, :, None], axis=0)
        gdelta = np.sum(G * (A[None] * P + u[:, t, :, None] * Bt[:, t, None, :]), axis=2)
        gdraw[:, t] = gdelta * _sigmoid(draw[:, t])
        gu[:, t] = delta[:, t] * np.sum(G * Bt[:, t, None, :], axis=2) + gy[:, t] * Dp
        gBt[:, t] = np.sum(G * (delta[:, t] * u[:, t])[:, :, None], axis=1)
        gCt[:, t] = np.sum(gy[:, t, :, None] * hs[:, t], axis=1)
    gDp = np.sum(gy * u, axis=(0, 1))
    gh0 = None
    if h0 is not None:
        gh0 = (np.exp(delta[:, 0, :, None] * A[None]) * G) if L > 0 else G
    return gdraw, gA, gBt, gCt, gu, gz, gDp, gh0


# --------------------------------------------------------------------------- all-pole
def allpole_forward(a, w, y0=None):
    """``y_t = w_t - sum_{i=1..na} a_i y_{t-i}`` per lane: a [lanes, na], w [lanes, L],
    y0 [lanes, na] newest first (``y0[j] = y_{-1-j}``) (allpole_triton.py:1-31, 80-96)."""
    a, w = _hi(a), _hi(w)
    lanes, L = w.shape
    na = a.shape[-1]
    s = np.zeros((lanes, na)) if y0 is None else _hi(y0).copy()  # s[:, k] = y_{t-1-k}
    y = np.empty((lanes, L))
    for t in range(L):
        yt = w[:, t] - np.sum(a * s, axis=1)
        y[:, t] = yt
        s = np.concatenate([yt[:, None], s[:, :-1]], axis=1)
    return y


def allpole_backward(g, a, y, y0=None):
    """Adjoint (allpole_triton.py:19-27, 101-122, 191-213): ``G_t = g_t - sum_i a_i G_{t+i}``,
    ``gw = G``, ``ga_i = -sum_{t>=0} G_t y_{t-i}`` with ``y_{-k} = y0[k-1]``,
    ``gy0_j = -sum_{i=j+1..na} a_i G_{i-1-j}``. Returns ``(ga, gw, gy0)``."""
    g, a, y = _hi(g), _hi(a), _hi(y)
    lanes, L = y.shape
    na = a.shape[-1]
    Gpad = np.zeros((lanes, L + na))
    for t in range(L - 1, -1, -1):
        Gpad[:, t] = g[:, t] - np.sum(a * Gpad[:, t + 1 : t + 1 + na], axis=1)
    gw = Gpad[:, :L].copy()
    # y extended to the left by y0: yext[:, na + t] = y_t, yext[:, na - 1 - j] = y0[j]
    yext = np.zeros((lanes, na + L))
    yext[:, na:] = y
    if y0 is not None:
        yext[:, :na] = _hi(y0)[:, ::-1]
    ga = np.zeros((lanes, na))
    for i in range(1, na + 1):
        # sum_t G_t y_{t-i}, t = 0..L-1, y_{t-i} = yext[:, na + t - i]
        ga[:, i - 1] = -np.sum(gw * yext[:, na - i : na - i + L], axis=1)
    gy0 = None
    if y0 is not None:
        gy0 = np.zeros((lanes, na))
        for j in range(na):
            for i in range(j + 1, na + 1):
                gy0[:, j] -= a[:, i - 1] * Gpad[:, i - 1 - j]
    return ga, gw, gy0


# --------------------------------------------------------------------------- causal depthwise conv + SiLU
def _conv_pre(x, tail, w, bias):
    """Pre-activation ``p_t = bias + sum_k w_k xbuf_{t-(K-1)+k}`` with ``xbuf = cat(tail, x)``
    along time, as the shifted multiply-adds of mamba/core.py:38-58 (the reference's ``_causal_depthwise_silu``).
    x [B, L, D], tail [B, D, K-1], w [D, K], bias [D] or None. Returns (p [B, L, D], xbuf)."""
    x, tail, w = _hi(x), _hi(tail), _hi(w)
    Bsz, L, D = x.shape
    K = w.shape[-1]
    buf = np.concatenate([np.transpose(tail, (0, 2, 1)), x], axis=1)  # [B, K-1+L, D]
    p = np.zeros((Bsz, L, D)) if bias is None else np.broadcast_to(_hi(bias), (Bsz, L, D)).copy()
    for k in range(K):
        p += w[:, k] * buf[:, k : k + L]
    return p, buf


def conv_silu_forward(x, tail, w, bias=None):
    """``silu(p)`` (mamba/core.py:38-58; conv_triton.py:59-118)."""
    p, _ = _conv_pre(x, tail, w, bias)
    return p * _sigmoid(p)


def conv_silu_backward(gy, x, tail, w, bias=None):
    """Adjoint (conv_triton.py:120-263): ``gpre = gy silu'(p)``, ``gx_t = sum_k w_k
    gpre_{t+K-1-k}``, ``gw_k = sum_{b,t} gpre_t xbuf_{t-(K-1)+k}``, ``gb = sum gpre``,
    ``gtail_j = sum_{t<=j} gpre_t w_{j-t}`` (the loop at :244-248).
    Returns ``(gx, gtail, gw, gb)`` (gb None when bias is None)."""
    gy, w = _hi(gy), _hi(w)
    p, buf = _conv_pre(x, tail, w, bias)
    Bsz, L, D = p.shape
    K = w.shape[-1]
    sg = _sigmoid(p)
    gpre = gy * sg * (1.0 + p * (1.0 - sg))
    gbuf = np.zeros((Bsz, K - 1 + L, D))  # gradient of every xbuf position
    for k in range(K):
        gbuf[:, k : k + L] += w[:, k] * gpre
    gx = gbuf[:, K - 1 :]
    gtail = np.transpose(gbuf[:, : K - 1], (0, 2, 1))
    gw = np.stack([np.sum(gpre * buf[:, k : k + L], axis=(0, 1)) for k in range(K)], axis=1)
    gb = None if bias is None else np.sum(gpre, axis=(0, 1))
    return gx, gtail, gw, gb


# --------------------------------------------------------------------------- dynoNet G-block
def _gblock_fir(u, b, u_tail):
    """FIR stage of LinearDynamicalOperator.forward (dynonet/core.py:219-222): ``ubuf =
    cat(u_tail, u)`` along time and, per pair p = j * O + o (input-major, :158-159),
    ``w[b, p, t] = sum_k bcoef[o, j, k] ubuf[b, t + nb - 1 - k, j]``. u [B, L, I], bcoef
    [O, I, nb], u_tail [B, nb-1, I]. Returns (w [B, P, L], ubuf [B, nb-1+L, I])."""
    u, b, u_tail = _hi(u), _hi(b), _hi(u_tail)
    Bsz, L, I = u.shape
    O, _, nb = b.shape
    ubuf = np.concatenate([u_tail, u], axis=1)
    w = np.zeros((Bsz, I, O, L))
    for k in range(nb):
        # [B, I, 1, L] * [1, I, O, 1]
        w += ubuf[:, nb - 1 - k : nb - 1 - k + L, :].transpose(0, 2, 1)[:, :, None, :] * b[:, :, k].T[None, :, :, None]
    return w.reshape(Bsz, I * O, L), ubuf


def gblock_forward(u, b, a, u_tail, x0):
    """LinearDynamicalOperator.forward (dynonet/core.py:196-258) with the all-pole stage:
    FIR per pair, ``y_pairs = allpole(a, w, x0)`` per pair (:228-235), then the sum over inputs
    ``y[b, t, o] = sum_j y_pairs[b, j * O + o, t]`` (:250). a [O, I, na] (pair coefficients
    a.permute(1, 0, 2), :229), x0 [B, P, na] newest first. Returns (y [B, L, O], x_last
    [B, P, na], y_pairs [B, P, L]); x_last[j] = y_{L-1-j}, from x0 when L < na (:239-244)."""
    Bsz, L, I = np.shape(u)
    O, _, na = np.shape(a)
    P = I * O
    w, _ = _gblock_fir(u, b, u_tail)
    ap = np.broadcast_to(_hi(a).transpose(1, 0, 2).reshape(1, P, na), (Bsz, P, na)).reshape(-1, na)
    yp = allpole_forward(ap, w.reshape(-1, L), _hi(x0).reshape(-1, na)).reshape(Bsz, P, L)
    y = yp.reshape(Bsz, I, O, L).sum(1).transpose(0, 2, 1)
    ext = np.concatenate([_hi(x0)[:, :, ::-1], yp], axis=2)  # oldest .. newest
    x_last = ext[:, :, ::-1][:, :, :na]
    return y, x_last, yp


def gblock_backward(gy, g_xlast, u, b, a, u_tail, x0):
    """Adjoint of gblock_forward: the upstream gradient of every pair's output is gy of its
    output channel, plus g_xlast on the last na outputs (or on x0 when the sequence is shorter);
    the all-pole adjoint gives (ga, gw, gx0) per pair; the FIR adjoint gives
    ``gb[o, j, k] = sum_{b,t} gw[b, p, t] ubuf[b, t + nb - 1 - k, j]`` and the input gradient
    ``gubuf[b, s, j] = sum_o sum_k bcoef[o, j, k] gw[b, p, s - (nb - 1) + k]``.
    Returns (gu [B, L, I], gu_tail [B, nb-1, I], gb [O, I, nb], ga [O, I, na], gx0 [B, P, na])."""
    gy, b = _hi(gy), _hi(b)
    Bsz, L, O = gy.shape
    _, I, nb = b.shape
    na = np.shape(a)[2]
    P = I * O
    _, _, yp = gblock_forward(u, b, a, u_tail, x0)
    w, ubuf = _gblock_fir(u, b, u_tail)
    gpair = np.broadcast_to(gy.transpose(0, 2, 1)[:, None, :, :], (Bsz, I, O, L)).reshape(Bsz, P, L).copy()
    gx0_direct = np.zeros((Bsz, P, na))
    if g_xlast is not None:
        gxl = _hi(g_xlast)
        for j in range(na):  # x_last[j] = y_{L-1-j}, or x0[j - L] for j >= L
            if L - 1 - j >= 0:
                gpair[:, :, L - 1 - j] += gxl[:, :, j]
            else:
                gx0_direct[:, :, j - L] += gxl[:, :, j]
    ap = np.broadcast_to(_hi(a).transpose(1, 0, 2).reshape(1, P, na), (Bsz, P, na)).reshape(-1, na)
    ga_l, gw, gx0_l = allpole_backward(gpair.reshape(-1, L), ap, yp.reshape(-1, L), _hi(x0).reshape(-1, na))
    gw = gw.reshape(Bsz, I, O, L)
    ga = ga_l.reshape(Bsz, I, O, na).sum(0).transpose(1, 0, 2)
    gx0 = gx0_l.reshape(Bsz, P, na) + gx0_direct
    gb = np.zeros((O, I, nb))
    gubuf = np.zeros((Bsz, nb - 1 + L, I))
    for k in range(nb):
        seg = ubuf[:, nb - 1 - k : nb - 1 - k + L, :].transpose(0, 2, 1)  # [B, I, L]
        gb[:, :, k] = np.einsum("bjol,bjl->oj", gw, seg)
        gubuf[:, nb - 1 - k : nb - 1 - k + L, :] += np.einsum("bjol,oj->blj", gw, b[:, :, k])
    return gubuf[:, nb - 1 :], gubuf[:, : nb - 1], gb, ga, gx0


# --------------------------------------------------------------------------- constant-matrix recurrence
def linrec_forward(A, v, x0=None):
    """``x_t = A x_{t-1} + v_t`` per lane with a constant matrix (dynonet/core.py:23-52, 103-127):
    A [M, n, n], v [M, L, n], x0 [M, n] or None (zero start). Returns x_1 .. x_L as [M, L, n]."""
    A, v = _hi(A), _hi(v)
    M, L, n = v.shape
    x = np.zeros((M, n)) if x0 is None else _hi(x0).copy()
    out = np.empty((M, L, n))
    for t in range(L):
        x = np.einsum("mij,mj->mi", A, x) + v[:, t]
        out[:, t] = x
    return out


def linrec_backward(g, A, out, x0=None):
    """Adjoint (dynonet/core.py:60-73): ``G_t = A^T G_{t+1} + g_t`` from the right end,
    ``gv = G``, ``gA = sum_t G_t x_{t-1}^T`` with ``x_0 = x0`` (zero if None), ``gx0 = A^T G_1``
    (None without x0; zero for an empty sequence). Returns ``(gA, gv, gx0)``."""
    g, A, out = _hi(g), _hi(A), _hi(out)
    M, L, n = g.shape
    G = np.zeros((M, L, n))
    acc = np.zeros((M, n))
    for t in range(L - 1, -1, -1):
        acc = np.einsum("mji,mj->mi", A, acc) + g[:, t]
        G[:, t] = acc
    head = np.zeros((M, 1, n)) if x0 is None else _hi(x0)[:, None, :]
    prev = np.concatenate([head, out[:, :-1]], axis=1)[:, :L]
    gA = np.einsum("mti,mtj->mij", G, prev)
    gx0 = None
    if x0 is not None:
        gx0 = np.einsum("mji,mj->mi", A, G[:, 0]) if L > 0 else np.zeros((M, n))
    return gA, G, gx0


# --------------------------------------------------------------------------- projected diagonal scan (LRU / S5 core)
def complex_in_proj(u, W_re, W_im):
    """``u @ (W_re + i W_im)^T``: real ``u [..., d]``, weights ``[n, d]`` -> complex ``[..., n]``
    (tsfast/models/_core/scan.py:272-291)."""
    return _hi(u) @ (_hi(W_re) + 1j * _hi(W_im)).T


def real_out_proj(x, W_re, W_im):
    """``Re(x @ (W_re + i W_im)^T)``: complex ``x [..., n]``, weights ``[o, n]`` -> real ``[..., o]``
    (tsfast/models/_core/scan.py:294-313)."""
    return (_hi(x) @ (_hi(W_re) + 1j * _hi(W_im)).T).real


def projscan_forward(u, W_re, W_im, lam, C_re, C_im, x0=None):
    """The LRU / S5 layer core as the reference composes it (lru.py:100-110, s5.py:180-198):
    ``v = complex_in_proj(u, W)``, ``x = diagonal_recurrence(lam, v, x0)`` with ``lam [n]`` shared
    by every row, ``y = real_out_proj(x, C)``. u [B, L, d]; returns ``(y [B, L, o], x [B, L, n])``
    (the states, whose last step is the layer's returned state)."""
    v = complex_in_proj(u, W_re, W_im)
    Bsz, L, n = v.shape
    lanes = np.broadcast_to(_hi(lam), (Bsz, n))
    x = diag_forward(lanes, v, x0)
    return real_out_proj(x, C_re, C_im), x


def projscan_backward(gy, g_xlast, u, W_re, W_im, lam, C_re, C_im, x, x0=None):
    """Adjoint of :func:`projscan_forward` given the upstream ``gy [B, L, o]`` and the gradient
    ``g_xlast [B, n]`` of the returned last state (None for zero), in torch's convention.

    ``g_x = gy @ conj(C)`` (+ ``g_xlast`` at the last step); ``G`` = the diagonal adjoint scan of
    ``g_x``; ``g_u = Re(G @ conj(W))``; ``g_W_re = sum G_re u^T``, ``g_W_im = sum G_im u^T``;
    ``g_C_re = sum gy Re(x)^T``, ``g_C_im = -sum gy Im(x)^T``; ``g_lam = sum_{b,t} G_t conj(x_{t-1})``;
    ``g_x0 = conj(lam) G_0``. Returns ``(g_u, g_W_re, g_W_im, g_lam, g_C_re, g_C_im, g_x0)``."""
    gy, u, x = _hi(gy), _hi(u), _hi(x)
    W = _hi(W_re) + 1j * _hi(W_im)
    C = _hi(C_re) + 1j * _hi(C_im)
    gx = gy @ np.conj(C)
    if g_xlast is not None and gx.shape[1] > 0:
        gx[:, -1] += _hi(g_xlast)
    Bsz, L, n = x.shape
    lanes = np.broadcast_to(_hi(lam), (Bsz, n))
    glam_rows, G, gx0 = diag_backward(gx, lanes, x, x0)
    g_u = (G @ np.conj(W)).real
    g_W_re = np.einsum("bln,bld->nd", G.real, u)
    g_W_im = np.einsum("bln,bld->nd", G.imag, u)
    g_C_re = np.einsum("blo,bln->on", gy, x.real)
    g_C_im = -np.einsum("blo,bln->on", gy, x.imag)
    return g_u, g_W_re, g_W_im, glam_rows.sum(0), g_C_re, g_C_im, gx0


# --------------------------------------------------------------------------- NSS chunked adjoint
def mat_adjoint_bounds(jt, gout, cl):
    """Chunk boundaries of ``gy_t = gout_t + jt[t+1] gy_{t+1}`` (``gy_{L-1} = gout_{L-1}``).

    Restates ``ssm_bwd_summary`` and ``ssm_bwd_scan``
    (tsfast/models/architectures/ssm/backend_metal.py:285-357) with the chunking of ``backward``
    (:466-476): chunk ``c`` covers steps ``[c cl, min((c + 1) cl, L))``; its summary ``(P, s)``
    starts from ``(I, 0)`` and, right to left over its steps, becomes ``(A P, gout_t + A s)`` with
    ``A = jt[t + 1]``, or ``(0, gout_t)`` at ``t = L - 1``; then ``v`` runs over the chunks from
    the right from zero, ``v <- s_c + P_c v``, and ``bnd[:, c] = v``, ``bnd[:, C] = 0``.
    Returns ``bnd [B, C + 1, n]`` in float64."""
    jt, gout = _hi(jt), _hi(gout)
    B, L, n = gout.shape
    C = -(-L // int(cl)) if L > 0 else 0
    pc = np.zeros((B, C, n, n))
    sc = np.zeros((B, C, n))
    for c in range(C):
        t0, t1 = c * cl, min((c + 1) * cl, L)
        P = np.broadcast_to(np.eye(n), (B, n, n)).copy()
        sv = np.zeros((B, n))
        for t in range(t1 - 1, t0 - 1, -1):
            if t + 1 < L:
                A = jt[:, t + 1]
                P = A @ P
                sv = gout[:, t] + np.einsum("bim,bm->bi", A, sv)
            else:
                P = np.zeros((B, n, n))
                sv = gout[:, t].copy()
        pc[:, c], sc[:, c] = P, sv
    bnd = np.zeros((B, C + 1, n))
    v = np.zeros((B, n))
    for c in range(C - 1, -1, -1):
        v = sc[:, c] + np.einsum("bim,bm->bi", pc[:, c], v)
        bnd[:, c] = v
    return bnd
