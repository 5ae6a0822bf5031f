"""Benchmark of the scan family on one MI355X; default = the headline metric.

Default workload: fused Mamba selective scan, B=16, L=4096, D=1536,
N=16, bf16 I/O (draw, u, z, Bt, Ct, out and their gradients) with fp32 state and fp32 A/Dp.
A = -exp(log(arange(1, 17))) broadcast over D; delta = softplus(draw), draw ~ N(-4, 1);
Bt, Ct, u, z, Dp ~ N(0, 1); h0 = None; upstream gradient gout ~ N(0, 1), ghlast = None.
Synthetic data, inputs resident in HBM before timing.

One step = the training forward (tsfast_hip::mamba_scan_train: output, h_last and the state
checkpoints) followed by the backward (tsfast_hip::mamba_scan_bwd: all eight gradients). W warmup
steps, then K timed steps between two device synchronisations. ``value`` is the achieved
algorithmic HBM bandwidth of the whole step (compulsory bytes of the op's inputs, outputs and
gradients, once each) in GB/s; ``ms_per_step`` is fwd+bwd milliseconds.

``--config 1|2|4|5`` runs the other BASELINE configs the same way (diagonal scan real / complex,
dynoNet all-pole, TBPTT diagonal scan as 64 chunks with the state carried); these are for the
design notes, the driver's line is config 3.

The CPU column times the reference CPU path on a bounded sample of the same workload, on the
host's cores: the C++/OpenMP port of the reference CPU kernels (oracle/cpu_baseline.cpp, after
mamba/backend_c.py and scan_backends/diagonal_c.py) for configs 1, 2, 3, 5, and the
companion-matrix doubling scan and its adjoint (oracle/torch_reference.py, a restatement of the
reference CPU path of dynonet/core.py:23-88) for config 4.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config 3] [--io bf16|fp32] [--no-cpu]
       (or one of --selective, --conv, --gblock, --linrec, --projected, --adjoint for the other
       rows' workloads)
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fwd+bwd ms + achieved HBM GB/s (% peak), selective scan B16 L4096 D1536 N16"
HBM_PEAK_GBS = 8000.0
CFG3 = dict(B=16, L=4096, D=1536, N=16)

# HBM bytes per call measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on the default bench
# workload, each scaled by the same counter on a 512 MiB elementwise copy (FETCH x 2.0, WRITE
# x 1.0): (config number or "selective", I/O dtype) -> {phase: (bytes, source)}. Counters cannot be read from inside
# this process, so the figures come from the committed summary and must be re-measured when the
# kernels change.
MEASURED_TRAFFIC = {
    (3, "bf16"): {
        "fwd": (2_088_500_000, "profiles/mamba_scan_config3_traffic.md"),
        "bwd": (3_103_900_000, "profiles/mamba_scan_config3_traffic.md"),
    },
    (2, "f32"): {
        "fwd": (1_109_100_000, "profiles/diag_scan_config2_traffic.md"),
        "bwd": (1_656_200_000, "profiles/diag_scan_config2_traffic.md"),
    },
    ("selective", "f32"): {
        "fwd": (1_624_700_000, "profiles/selective_scan_traffic.md"),
        "bwd": (2_713_100_000, "profiles/selective_scan_traffic.md"),
    },
    (4, "f32"): {
        "fwd": (668_600_000, "profiles/allpole_scan_config4_traffic.md"),
        "bwd": (959_800_000, "profiles/allpole_scan_config4_traffic.md"),
    },
    ("linrec", "f32"): {
        "fwd": (2_120_800_000, "profiles/linrec_config4route_traffic.md"),
        "bwd": (3_283_900_000, "profiles/linrec_config4route_traffic.md"),
    },
}

# VALU issue per call, for the VALU-bound fused Mamba scan: rocprofv3 SQ_ACTIVE_INST_VALU (quad-cycles
# a SIMD spends issuing vector instructions, transcendentals counting two) summed over the
# kernels of one ABI call; same provenance rules as MEASURED_TRAFFIC.
MEASURED_VALU = {
    (3, "bf16"): {
        "fwd": (230_092_800, "profiles/mamba_scan_config3_valu.md"),
        "bwd": (501_884_608, "profiles/mamba_scan_config3_valu.md"),
    },
}
VALU_PEAK_CLOCK_HZ = 2.4e9  # MI355X peak engine clock
SIMDS_PER_CU = 4


# --------------------------------------------------------------------------- algorithmic bytes
def mamba_bytes(B, L, D, N, io_bytes):
    """Compulsory bytes, once each: (fwd, bwd)."""
    bld, bln = B * L * D, B * L * N
    params = D * N * 4 + D * 4
    fwd = 3 * bld * io_bytes + 2 * bln * io_bytes + params + bld * io_bytes + B * D * N * 4
    bwd = 4 * bld * io_bytes + 2 * bln * io_bytes + params + 3 * bld * io_bytes + 2 * bln * io_bytes + params
    return fwd, bwd


def scan_bytes(elems, esz, lanes, lane_esz):
    """Diagonal / all-pole scan: fwd reads v, writes out; bwd reads g and out, writes gv (+ per-lane terms)."""
    return 2 * elems * esz + lanes * lane_esz, 3 * elems * esz + 2 * lanes * lane_esz


# --------------------------------------------------------------------------- inputs
def mamba_inputs(B, L, D, N, io_dtype, device, seed=2):
    import torch

    g = torch.Generator().manual_seed(seed)
    A = -torch.exp(torch.log(torch.arange(1, N + 1, dtype=torch.float32))).expand(D, N).contiguous()
    t = dict(
        draw=torch.randn(B, L, D, generator=g) - 4.0,
        A=A,
        Bt=torch.randn(B, L, N, generator=g),
        Ct=torch.randn(B, L, N, generator=g),
        u=torch.randn(B, L, D, generator=g),
        z=torch.randn(B, L, D, generator=g),
        Dp=torch.randn(D, generator=g),
        gout=torch.randn(B, L, D, generator=g),
    )
    for k in ("draw", "Bt", "Ct", "u", "z", "gout"):
        t[k] = t[k].to(io_dtype)
    return {k: v.to(device) for k, v in t.items()}


def diag_inputs(cfg, device):
    """Configs 1, 2, 5 in the lane layout (lam [M, N], v/g [M, L, N])."""
    import torch

    g = torch.Generator().manual_seed(cfg - 1)
    if cfg == 1:
        lam = torch.rand(32, 64, generator=g) * 0.099 + 0.9
        v = torch.randn(32, 1000, 64, generator=g)
        gv = torch.randn(32, 1000, 64, generator=g)
    elif cfg == 2:
        from tsfast_amd.scan import complex_in_proj, real_out_proj

        H, n = 32, 256
        lam1 = torch.polar(torch.rand(n, generator=g) * 0.099 + 0.9, torch.rand(n, generator=g) * (math.pi / 10))
        lam = lam1.expand(64, n).contiguous()
        u = torch.randn(64, 4096, H, generator=g)
        B_re = torch.randn(n, H, generator=g) / math.sqrt(2 * H)
        B_im = torch.randn(n, H, generator=g) / math.sqrt(2 * H)
        v = complex_in_proj(u, B_re, B_im).contiguous()
        C_re = torch.randn(H, n, generator=g) / math.sqrt(n)
        C_im = torch.randn(H, n, generator=g) / math.sqrt(n)
        # g_h = d(sum(gy * Re(h C^T)))/dh for gy ~ N(0,1): the readout's adjoint, computed once
        h = torch.zeros_like(v, requires_grad=True)
        gy = torch.randn(64, 4096, H, generator=g)
        (real_out_proj(h, C_re, C_im) * gy).sum().backward()
        gv = h.grad.contiguous()
    else:  # 5: one 4096-step chunk shape; the runner loops 64 chunks
        lam = torch.rand(8, 128, generator=g) * 0.0099 + 0.99
        v = torch.randn(8, 64 * 4096, 128, generator=g)
        gv = torch.randn(8, 64 * 4096, 128, generator=g)
    return lam.to(device), v.to(device), gv.to(device)


def allpole_inputs(device, P=64, B=64, L=16384, na=3):
    """Config 4: per pair, poles p, conj(p), r with |p|, |r| ~ U(0.5, 0.98); a = poly(poles)[1:].
    Other orders (the --linrec --order option) draw na // 2 conjugate pairs, plus a real pole
    when na is odd, from the same distributions (na = 3 gives config 4's draws)."""
    import numpy as np
    import torch

    rng = np.random.default_rng(3)
    rows = []
    for _ in range(P):
        poles = []
        while len(poles) < na:
            if na - len(poles) >= 2:
                rp = rng.uniform(0.5, 0.98)
                th = rng.uniform(0, math.pi)
                poles += [rp * np.exp(1j * th), rp * np.exp(-1j * th)]
            else:
                poles.append(rng.uniform(0.5, 0.98) * (1 if rng.random() < 0.5 else -1))
        rows.append(np.real(np.poly(poles))[1:])
    # keep every filter stable after the coefficients' fp32 rounding (high orders with poles near
    # the unit circle can cross it): pull a row's poles inwards until its companion matrix has
    # spectral radius below 0.99 (no row of config 4's order-3 draws needs it)
    rows = np.array(rows)
    for i in range(P):
        for _ in range(40):
            cm = np.eye(na, k=-1)
            cm[0] = -rows[i].astype(np.float32).astype(np.float64)
            if np.abs(np.linalg.eigvals(cm)).max() < 0.99:
                break
            rows[i] = rows[i] * 0.97 ** np.arange(1, na + 1)  # poles scaled by 0.97
    a = torch.tensor(rows, dtype=torch.float32)
    g = torch.Generator().manual_seed(3)
    w = torch.randn(B, P, L, generator=g)
    gout = torch.randn(B, P, L, generator=g)
    a_lane = a.expand(B, P, na).reshape(B * P, na).contiguous()
    return a_lane.to(device), w.reshape(B * P, L).to(device), gout.reshape(B * P, L).to(device)


# --------------------------------------------------------------------------- timing
def time_steps(step, steps, warmup):
    """W untimed steps, then K timed steps between device synchronisations, with nothing else in
    them; then K more steps in which step(ev) records events at the phase boundaries, for the
    per-phase times (an event record costs microseconds of host and device time, a measurable
    share of the smallest configs' steps, so it stays out of the timed steps). Returns (ms per
    timed step, [mean ms per phase]). Python's cyclic collector is run before and held off during
    the steps (as timeit does): a full collection stalls the host for tens of milliseconds,
    starving the GPU of launches, and where it falls depends on allocation counts that differ
    between a first and a later process."""
    import torch

    gc.collect()
    gc.disable()
    try:
        for _ in range(warmup):
            step(None)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step(None)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        events = []
        for _ in range(steps):
            ev = []
            step(ev)
            events.append(ev)
        torch.cuda.synchronize()
    finally:
        gc.enable()
    phases = []
    if events and events[0]:
        for p in range(len(events[0]) - 1):
            phases.append(statistics.mean(e[p].elapsed_time(e[p + 1]) for e in events))
    return (t1 - t0) * 1e3 / steps, phases


def mark(ev):
    """Record an event on the current stream (the one every kernel here is launched on)."""
    import torch

    if ev is not None:
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        ev.append(e)


def cpu_time(fn, budget_s=20.0, reps=5, warmup=3):
    """The CPU protocol of the baseline notes: `warmup` untimed runs, then the median of up to
    `reps` timed runs (fewer if they exceed `budget_s`); returns (median seconds, runs)."""
    for _ in range(warmup):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < reps and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


# --------------------------------------------------------------------------- workloads
def run_mamba(args, line):
    import torch

    from tsfast_amd.mamba import mamba_hip

    io_dtype = torch.bfloat16 if args.io == "bf16" else torch.float32
    B, L, D, N = CFG3["B"], CFG3["L"], CFG3["D"], CFG3["N"]
    x = mamba_inputs(B, L, D, N, io_dtype, "cuda")
    fargs = [x[k] for k in ("draw", "A", "Bt", "Ct", "u", "z", "Dp")] + [None]

    def step(ev):
        mark(ev)
        out, h_last, chk = mamba_hip._scan_train_op(*fargs)
        mark(ev)
        mamba_hip._scan_bwd_op(x["gout"], None, chk, *fargs)
        mark(ev)

    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)
    fwd_b, bwd_b = mamba_bytes(B, L, D, N, 2 if io_dtype == torch.bfloat16 else 4)
    line.update(
        config={
            "workload": "fused Mamba selective scan, train forward (checkpoints) + backward, BASELINE config 3",
            "B": B, "L": L, "D": D, "N": N, "io_dtype": args.io, "state_dtype": "f32",
        },
        fwd_ms=round(fwd_ms, 4),
        bwd_ms=round(bwd_ms, 4),
    )
    kernels = {"fwd": ("mamba_fwd_kernel", fwd_ms, fwd_b),
               "bwd": ("mamba_bwd_kernel + its partial reductions (one ABI call)", bwd_ms, bwd_b)}
    cpu = None
    if not args.no_cpu:
        def cpu_leg():
            from oracle import cpu_baseline as CB

            lib = CB.load(prefer_native=True)
            threads = os.cpu_count() or 1
            lib.cpu_set_threads(threads)
            xs = mamba_inputs(B, L, D, N, io_dtype, "cpu")
            a = {k: v.float().numpy() for k, v in xs.items()}
            del xs
            margs = [a[k] for k in ("draw", "A", "Bt", "Ct", "u", "z", "Dp")]
            med, n = cpu_time(lambda: CB.mamba_fwd_bwd(*margs, a["gout"]), budget_s=60.0)
            sf, sb = mamba_bytes(B, L, D, N, 2 if io_dtype == torch.bfloat16 else 4)
            return {
                "value": round((sf + sb) / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": (f"the whole config 3 workload (B={B}, L={L}, D={D}, N={N}) in fp32 (the reference CPU "
                           f"kernel's regime: the bf16 inputs upcast; oracle/cpu_baseline.cpp after "
                           f"mamba/backend_c.py, its exp included), fwd+bwd with the partial sums, 3 warmup runs, "
                           f"median of {n} = {med * 1e3:.1f} ms; build {CB.lib_path().name}"),
                "ms_per_step_sample": round(med * 1e3, 3),
            }
        cpu = cpu_leg
    return ms, fwd_b + bwd_b, kernels, cpu


def run_diag(args, line):
    from tsfast_amd.scan_backends import diagonal_hip

    cfg = args.config
    lam, v, gv = diag_inputs(cfg, "cuda")
    cplx = v.is_complex()
    esz = 8 if cplx else 4
    if cfg == 5:
        T, C = 4096, 64
        chunks_v = [v[:, k * T : (k + 1) * T].contiguous() for k in range(C)]
        chunks_g = [gv[:, k * T : (k + 1) * T].contiguous() for k in range(C)]

        def step(ev):
            mark(ev)
            x0 = None
            outs = []
            for k in range(C):
                o = diagonal_hip.forward(lam, chunks_v[k], x0)
                outs.append((o, x0))
                x0 = o[:, -1].contiguous()
            mark(ev)
            for k in range(C - 1, -1, -1):
                o, xin = outs[k]
                diagonal_hip.backward(chunks_g[k], lam, o, xin)
            mark(ev)

        fwd_b, bwd_b = scan_bytes(v.numel(), esz, lam.numel() * C, esz)
        workload = "TBPTT real diagonal scan, 64 chunks x 4096 with x0 carry, fwd+bwd, BASELINE config 5"
    else:
        def step(ev):
            mark(ev)
            o = diagonal_hip.forward(lam, v, None)
            mark(ev)
            diagonal_hip.backward(gv, lam, o, None)
            mark(ev)

        fwd_b, bwd_b = scan_bytes(v.numel(), esz, lam.numel(), esz)
        workload = ("real diagonal scan fwd+bwd, BASELINE config 1" if cfg == 1
                    else "complex64 diagonal scan fwd+bwd (scan only; projections outside), BASELINE config 2")
    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)
    M, L, N = v.shape
    line.update(config={"workload": workload, "M": M, "L": L, "N": N, "io_dtype": "complex64" if cplx else "f32"},
                fwd_ms=round(fwd_ms, 4), bwd_ms=round(bwd_ms, 4))
    line["dtype"] = "c128" if cplx else "f64"  # fp32/complex64 I/O, fp64 state inside
    # the kernels csrc/diag.hip picks for these shapes (whole_tile): config 1 runs whole-sequence
    # tiles both ways, config 5's 64-chunk forward too, and the rest the look-back
    whole_fwd = "diag_whole_fwd (whole-sequence tiles, one launch)"
    look_fwd = "diag_fwd look-back scan + workspace reset"
    kernels = {"fwd": (whole_fwd if cfg in (1, 5) else look_fwd, fwd_ms, fwd_b),
               "bwd": ("diag_whole_bwd (whole-sequence tiles, one launch)" if cfg == 1
                       else "diag_bwd look-back scan + reset + glam lane sums", bwd_ms, bwd_b)}
    cpu = None
    if not args.no_cpu:
        def cpu_leg():
            from oracle import cpu_baseline as CB

            lib = CB.load(prefer_native=True)
            threads = os.cpu_count() or 1
            lib.cpu_set_threads(threads)
            rows = {1: M, 2: 4, 5: M}[cfg]
            Ls = {1: L, 2: L, 5: 4 * 4096}[cfg]
            lam_c, v_c, g_c = (t.cpu().numpy() for t in (lam[:rows], v[:rows, :Ls], gv[:rows, :Ls]))
            med, n = cpu_time(lambda: CB.diag_fwd_bwd(lam_c, v_c, g_c, None))
            sf, sb = scan_bytes(rows * Ls * N, esz, rows * N, esz)
            return {
                "value": round((sf + sb) / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": (f"rows={rows}, L={Ls}, N={N} of config {cfg} (oracle/cpu_baseline.cpp after "
                           f"scan_backends/diagonal_c.py, single pass per (row, 64-lane block)), fwd+bwd median "
                           f"of {n} runs = {med * 1e3:.2f} ms"),
            }
        cpu = cpu_leg
    return ms, fwd_b + bwd_b, kernels, cpu


def run_conv(args, line):
    """The fused Mamba causal depthwise conv + SiLU (the scope table's next row, not a BASELINE
    config) at config 3's shape: x is the in_proj chunk view of a [B, L, 2D] tensor, K = 4."""
    import torch

    from tsfast_amd.mamba import conv_hip

    io_dtype = torch.bfloat16 if args.io == "bf16" else torch.float32
    esz = 2 if io_dtype == torch.bfloat16 else 4
    B, L, D, K = CFG3["B"], CFG3["L"], CFG3["D"], 4
    g = torch.Generator().manual_seed(5)
    xz = torch.randn(B, L, 2 * D, generator=g).to("cuda", io_dtype)
    x = xz[..., :D]
    tail = torch.randn(B, D, K - 1, generator=g).to("cuda", io_dtype)
    w = (torch.randn(D, K, generator=g) * 0.5).cuda()
    b = torch.randn(D, generator=g).cuda()
    gy = torch.randn(B, L, D, generator=g).to("cuda", io_dtype)

    def step(ev):
        mark(ev)
        conv_hip._conv_silu_op(x, tail, w, b)
        mark(ev)
        conv_hip._conv_silu_bwd_op(gy, x, tail, w, b)
        mark(ev)

    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)
    bld = B * L * D
    params = D * K * 4 + D * 4
    fwd_b = 2 * bld * esz + B * D * (K - 1) * esz + params
    bwd_b = 3 * bld * esz + 2 * B * D * (K - 1) * esz + 2 * params
    line.update(
        config={"workload": "fused Mamba causal depthwise conv + SiLU fwd+bwd at config 3's shape (next row)",
                "B": B, "L": L, "D": D, "K": K, "io_dtype": args.io, "x": "strided in_proj chunk view"},
        fwd_ms=round(fwd_ms, 4),
        bwd_ms=round(bwd_ms, 4),
    )
    line["metric"] = "fwd+bwd ms + achieved HBM GB/s, fused Mamba conv+SiLU at B16 L4096 D1536 K4"
    kernels = {"fwd": ("conv_silu_fwd_kernel", fwd_ms, fwd_b),
               "bwd": ("conv_silu_bwd_kernel + conv_reduce_params (one ABI call)", bwd_ms, bwd_b)}
    cpu = None
    if not args.no_cpu:
        def cpu_leg():
            from oracle import torch_reference as TR

            threads = os.cpu_count() or 1
            torch.set_num_threads(threads)
            rows = 2
            xc = xz[:rows].float().cpu()[..., :D].requires_grad_()
            tc = tail[:rows].float().cpu().requires_grad_()
            wc = w.cpu()[:, None, :].requires_grad_()
            bc = b.cpu().requires_grad_()
            gc = gy[:rows].float().cpu()

            def fb():
                TR.causal_depthwise_silu(xc, tc, wc, bc).backward(gc)

            med, n = cpu_time(fb)
            sf = 2 * rows * L * D * 4 + 3 * rows * L * D * 4
            return {
                "value": round(sf / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": (f"{rows} of {B} batch rows, fp32: the reference's eager CPU conv path "
                           f"(shifted multiply-adds + SiLU, mamba/core.py:38-58) in torch with autograd, fwd+bwd "
                           f"median of {n} runs = {med * 1e3:.2f} ms"),
            }
        cpu = cpu_leg
    return ms, fwd_b + bwd_b, kernels, cpu


def run_selective(args, line):
    """The time-varying (selective) diagonal scan, fp32, in the Mamba generic-fallback layout
    [B, L, D*N] (scope-table rows a6/a7; not a BASELINE config): B16 L4096, 2048 lanes per row."""
    import torch

    from tsfast_amd.scan_backends import selective_hip

    g = torch.Generator().manual_seed(6)
    M, L, N = 16, 4096, 2048
    a = (torch.rand(M, L, N, generator=g) * 0.5 + 0.49).cuda()
    v = torch.randn(M, L, N, generator=g).cuda()
    gv_up = torch.randn(M, L, N, generator=g).cuda()

    def step(ev):
        mark(ev)
        o = selective_hip.forward(a, v, None)
        mark(ev)
        selective_hip.backward(gv_up, a, o, None)
        mark(ev)

    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)
    e = M * L * N
    fwd_b, bwd_b = 3 * e * 4, 5 * e * 4  # fwd: a, v -> out; bwd: g, a, out -> glam, gv
    line.update(
        config={"workload": "selective diagonal scan fwd+bwd, fp32, [B, L, lanes] = [16, 4096, 2048] (rows a6/a7)",
                "M": M, "L": L, "N": N, "io_dtype": "f32"},
        fwd_ms=round(fwd_ms, 4),
        bwd_ms=round(bwd_ms, 4),
    )
    line["metric"] = "fwd+bwd ms + achieved HBM GB/s, selective scan [16, 4096, 2048] fp32"
    line["dtype"] = "f64"  # fp32 I/O, fp64 state inside
    kernels = {"fwd": ("sel_fwd look-back scan + workspace reset", fwd_ms, fwd_b),
               "bwd": ("sel_bwd look-back scan + workspace reset", bwd_ms, bwd_b)}
    cpu = None
    if not args.no_cpu:
        def cpu_leg():
            from oracle import cpu_baseline as CB

            lib = CB.load(prefer_native=True)
            threads = os.cpu_count() or 1
            lib.cpu_set_threads(threads)
            rows = 2
            a_c, v_c, g_c = (t[:rows].cpu().numpy() for t in (a, v, gv_up))
            med, n = cpu_time(lambda: CB.sel_fwd_bwd(a_c, v_c, g_c, None))
            eb = rows * L * N * 4
            return {
                "value": round(8 * eb / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": (f"rows={rows} of {M}, L={L}, N={N} (oracle/cpu_baseline.cpp after "
                           f"scan_backends/selective_c.py, sequential per (row, 64-lane block)), fwd+bwd median "
                           f"of {n} runs = {med * 1e3:.2f} ms"),
            }
        cpu = cpu_leg
    return ms, fwd_b + bwd_b, kernels, cpu


def run_allpole(args, line):
    from tsfast_amd.dynonet import allpole_hip

    a, w, gout = allpole_inputs("cuda")
    lanes, L = w.shape

    def step(ev):
        mark(ev)
        y = allpole_hip._allpole_op(a, w, None)
        mark(ev)
        allpole_hip._allpole_bwd_op(gout, a, y, None)
        mark(ev)

    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)
    fwd_b, bwd_b = scan_bytes(w.numel(), 4, lanes, 12)
    line.update(config={"workload": "dynoNet all-pole IIR scan fwd+bwd, na=3, BASELINE config 4",
                        "lanes": lanes, "L": L, "na": 3}, fwd_ms=round(fwd_ms, 4), bwd_ms=round(bwd_ms, 4))
    line["dtype"] = "f64"  # fp32 I/O, fp64 recurrence inside
    kernels = {"fwd": ("allpole_fwd_lb look-back scan + transfer + reset", fwd_ms, fwd_b),
               "bwd": ("allpole_bwd_lb look-back scan + transfer + reset + finish", bwd_ms, bwd_b)}
    cpu = None
    if not args.no_cpu:
        def cpu_leg():
            import torch
            import torch.nn.functional as F

            from oracle import torch_reference as TR
            from tsfast_amd.dynonet.core import companion

            threads = os.cpu_count() or 1
            torch.set_num_threads(threads)
            rows = 64
            a_c = a[:rows].cpu()
            w_c = w[:rows].cpu()
            g_c = F.pad(gout[:rows].cpu().unsqueeze(-1), (0, 2))
            Cm = companion(a_c)

            def fb():
                x = TR.linrec_forward(Cm, F.pad(w_c.unsqueeze(-1), (0, 2)))
                TR.linrec_backward(g_c, Cm, x)

            med, n = cpu_time(fb)
            sf, sb = scan_bytes(rows * L, 4, rows, 12)
            return {
                "value": round((sf + sb) / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": (f"{rows} of {lanes} lanes, L={L}: companion-matrix doubling scan on CPU (the reference "
                           f"CPU path, dynonet/core.py:23-88), fwd+bwd median of {n} runs = {med * 1e3:.1f} ms"),
            }
        cpu = cpu_leg
    return ms, fwd_b + bwd_b, kernels, cpu


def gblock_inputs(dev, B=64, L=16384, I=8, O=8, nb=8, na=3):
    """Config 4's channel structure (batch 64, 8 in x 8 out, L 16384, na 3) through a whole G-block
    with nb = 8 FIR taps (the reference's default, dynonet/core.py:172), stable poles."""
    import numpy as np
    import torch

    g = torch.Generator().manual_seed(4)
    u = torch.randn(B, L, I, generator=g)
    b = torch.randn(O, I, nb, generator=g) * 0.05
    a = torch.empty(O, I, na)
    for o in range(O):
        for j in range(I):
            r = (torch.rand(na, generator=g) * 0.48 + 0.5).double().numpy()
            # higher orders (--order): keep the fp32-rounded filter stable (spectral radius < 0.99)
            for _ in range(60):
                ai = np.poly(r)[1:].astype(np.float32)
                cm = np.eye(na, k=-1)
                cm[0] = -ai.astype(np.float64)
                if na == 1 or np.abs(np.linalg.eigvals(cm)).max() < 0.99:
                    break
                r = r * 0.97
            a[o, j] = torch.tensor(ai, dtype=torch.float32)
    gy = torch.randn(B, L, O, generator=g)
    return u.to(dev), b.to(dev), a.to(dev), gy.to(dev)


def run_gblock(args, line):
    """The fused dynoNet G-block (FIR + all-pole + input sum) at config 4's channel structure, with
    the reference's unfused three-stage path (conv1d, all-pole op, sum) timed in the same run.
    ``--order`` above 4 times the staged path (this library's FIR op, all-pole op and sum)."""
    import torch

    from tsfast_amd.dynonet import core as dcore
    from tsfast_amd.dynonet import gblock_hip

    u, b, a, gy = gblock_inputs("cuda", na=args.order)
    B, L, I = u.shape
    O, _, nb = b.shape
    na = a.shape[-1]
    P = I * O
    tail = u.new_zeros(B, nb - 1, I)
    x0 = u.new_zeros(B, P, na)

    fused = na <= 4

    def step(ev):
        if fused:
            mark(ev)
            y, x_last, saved = gblock_hip._gblock_op(u, b, a, tail, x0)
            mark(ev)
            gblock_hip._gblock_bwd_op(gy, None, u, b, a, tail, x0, saved)
            mark(ev)
        else:
            uu, bb, aa = (t.detach().requires_grad_() for t in (u, b, a))
            mark(ev)
            y, x_last = gblock_hip.run(uu, bb, aa, tail, x0)
            mark(ev)
            torch.autograd.backward(y, gy)
            mark(ev)

    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)

    def unfused(ev):
        uu = u.detach().requires_grad_()
        bb = b.detach().requires_grad_()
        aa = a.detach().requires_grad_()
        mark(ev)
        u_buf = torch.cat((tail, uu), dim=1)
        w = torch.nn.functional.conv1d(u_buf.transpose(1, 2), bb.permute(1, 0, 2).reshape(P, 1, nb).flip(-1), groups=I)
        y_pairs = dcore.allpole(aa.permute(1, 0, 2).reshape(P, na).expand(B, P, na), w, x0)
        y = y_pairs.view(B, I, O, L).sum(1).transpose(1, 2)
        mark(ev)
        torch.autograd.backward(y, gy)
        mark(ev)

    ums, (ufwd, ubwd) = time_steps(unfused, max(args.steps // 2, 2), 2)
    f4 = 4
    fwd_b = B * L * I * f4 + B * L * O * f4  # read u, write y
    bwd_b = B * L * O * f4 + B * L * I * f4 + B * L * I * f4  # read gy and u, write gu
    line.update(
        metric="fwd+bwd ms + achieved HBM GB/s, fused dynoNet G-block (FIR + all-pole + input sum)",
        config={"workload": f"fused dynoNet G-block fwd+bwd: batch {B}, {I} in x {O} out, L {L}, nb {nb}, na {na} "
                            "(BASELINE config 4 channel structure)", "B": B, "L": L, "I": I, "O": O, "nb": nb,
                "na": na},
        fwd_ms=round(fwd_ms, 4),
        bwd_ms=round(bwd_ms, 4),
        unfused_ms={"fwd": round(ufwd, 4), "bwd": round(ubwd, 4), "total": round(ums, 4),
                    "path": "F.conv1d + tsfast_hip::dynonet_allpole + sum over inputs (the reference's stages)"},
    )
    line["dtype"] = "f64"  # fp32 I/O, fp64 recurrence inside
    if fused:
        kernels = {"fwd": ("gblock_fwd_lb look-back scan + transfer + reset", fwd_ms, fwd_b),
                   "bwd": ("gblock_bwd_lb look-back scan + transfer + reset + finish", bwd_ms, bwd_b)}
    else:
        kernels = {"fwd": ("gb_fir_fwd + all-pole two-pass scan + input sum (staged)", fwd_ms, fwd_b),
                   "bwd": ("all-pole two-pass adjoint + gb_fir_bwd + gb_fir_reduce (staged)", bwd_ms, bwd_b)}
    cpu = None
    if not args.no_cpu:
        def cpu_leg():
            import torch.nn.functional as F

            from oracle import torch_reference as TR
            from tsfast_amd.dynonet.core import companion

            threads = os.cpu_count() or 1
            torch.set_num_threads(threads)
            rows = 2
            u_c = u[:rows].cpu().requires_grad_()
            b_c, a_c, gy_c = b.cpu(), a.cpu(), gy[:rows].cpu()
            Cm = companion(a_c.permute(1, 0, 2).reshape(P, na))

            def fb():
                u_buf = torch.cat((u_c.new_zeros(rows, nb - 1, I), u_c), dim=1)
                w = F.conv1d(u_buf.transpose(1, 2), b_c.permute(1, 0, 2).reshape(P, 1, nb).flip(-1), groups=I)
                x = TR.LinRec.apply(Cm.expand(rows, P, na, na), F.pad(w.unsqueeze(-1), (0, na - 1)))
                y = x[..., 0].view(rows, I, O, L).sum(1).transpose(1, 2)
                y.backward(gy_c)

            med, n = cpu_time(fb)
            sf = rows * L * (I + O) * 4
            sb = rows * L * (O + 2 * I) * 4
            return {
                "value": round((sf + sb) / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": (f"{rows} of {B} batch rows, L={L}: conv1d + companion-matrix doubling scan + sum on CPU "
                           f"(the reference CPU path, dynonet/core.py:23-88, 212-250), fwd+bwd median of {n} runs "
                           f"= {med * 1e3:.1f} ms"),
            }
        cpu = cpu_leg
    return ms, fwd_b + bwd_b, kernels, cpu


def projected_inputs(device, B=64, L=4096, H=32, N=256, O=32, seed=4):
    """BASELINE config 2's layer: u ~ N(0,1) [B, L, H], lam = r e^(i theta) with r ~ U(0.9, 0.999)
    and theta ~ U(0, pi/10), C ~ N(0, 1/N) (the readout of config 2), W ~ N(0, 1/H)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    u = torch.randn(B, L, H, generator=g)
    W_re, W_im = torch.randn(N, H, generator=g) / math.sqrt(H), torch.randn(N, H, generator=g) / math.sqrt(H)
    lam = torch.polar(torch.rand(N, generator=g) * 0.099 + 0.9, torch.rand(N, generator=g) * (math.pi / 10))
    C_re, C_im = torch.randn(O, N, generator=g) / math.sqrt(N), torch.randn(O, N, generator=g) / math.sqrt(N)
    gy = torch.randn(B, L, O, generator=g)
    return [t.to(device) for t in (u, W_re, W_im, lam, C_re, C_im, gy)]


def run_projected(args, line):
    """The projected complex diagonal scan (LRU / S5 layer core) at config 2's shape (or the widths
    --widths names) as projected_diagonal_recurrence runs it: the fused kernels within their widths
    (H, O <= 32, N <= 256), the wide route beyond (one GEMM per projection around the diagonal scan
    kernels, split-K weight gradients). The reference's unfused stack (complex_in_proj ->
    diagonal_recurrence -> real_out_proj, HIP scan backend, autograd) is timed in the same run. The
    projections run on the fp32 matrix cores, so the roofline is fp32 MFMA."""
    import torch

    from tsfast_amd import scan
    from tsfast_amd.scan_backends import projected_hip

    H, N, O = (int(v) for v in args.widths.split(","))
    u, W_re, W_im, lam, C_re, C_im, gy = projected_inputs("cuda", H=H, N=N, O=O)
    B, L = u.shape[:2]
    bl = B * L
    fused = projected_hip.shape_reason(B, L, H, N, O) is None
    fwd_f = 2 * bl * 2 * N * (H + O)  # in-projection and read-out
    # g_x, grad C, grad W, g_u; the fused backward also recomputes v (the wide route saves x)
    bwd_f = 2 * bl * 2 * N * (2 * O + (3 if fused else 2) * H)
    train_op = projected_hip._scan_train_op if fused else projected_hip._wide_train_op
    bwd_op = projected_hip._scan_bwd_op if fused else projected_hip._wide_bwd_op

    def step(ev):
        mark(ev)
        y, x_last, saved = train_op(u, W_re, W_im, lam, C_re, C_im, None)
        mark(ev)
        bwd_op(gy, None, saved, u, W_re, W_im, lam, C_re, C_im, None)
        mark(ev)

    def unfused(ev):
        ins = [t.detach().requires_grad_() for t in (u, W_re, W_im, lam, C_re, C_im)]
        mark(ev)
        x = scan.diagonal_recurrence(ins[3], scan.complex_in_proj(ins[0], ins[1], ins[2]))
        y = scan.real_out_proj(x, ins[4], ins[5])
        mark(ev)
        torch.autograd.backward(y, gy)
        mark(ev)

    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)
    ums, (ufwd, ubwd) = time_steps(unfused, max(args.steps // 2, 2), 2)
    route = "fused" if fused else "wide route (GEMMs around the diagonal scan kernels, split-K weight gradients)"
    line.update(
        metric=f"fwd+bwd ms + achieved fp32 TFLOP/s, projected complex diagonal scan (LRU/S5 layer core), {route}",
        unit="TFLOP/s",
        config={"workload": f"{route} complex_in_proj -> diagonal_recurrence -> real_out_proj fwd+bwd: batch {B}, "
                            f"L {L}, N {N} complex states, H {H} inputs, O {O} outputs"
                            + (" (BASELINE config 2 scan)" if (H, N, O) == (32, 256, 32) else ""),
                "B": B, "L": L, "N": N, "H": H, "O": O},
        fwd_ms=round(fwd_ms, 4),
        bwd_ms=round(bwd_ms, 4),
        unfused_ms={"fwd": round(ufwd, 4), "bwd": round(ubwd, 4), "total": round(ums, 4),
                    "path": "complex_in_proj (GEMM) + tsfast_hip::scan_diagonal + real_out_proj (GEMM), autograd"},
        algorithmic_flops={"fwd": fwd_f, "bwd": bwd_f},
        _mfma_peak_tflops=157.3,
    )
    if fused:
        kernels = {"fwd": ("projscan_fwd (in-projection, scan, read-out on fp32 MFMA)", fwd_ms, fwd_f),
                   "bwd": ("projscan_bwd + projscan_bwd_reduce", bwd_ms, bwd_f)}
    else:
        kernels = {"fwd": ("wide forward: 2 GEMMs + diag_fwd", fwd_ms, fwd_f),
                   "bwd": ("wide backward: 2 GEMMs + diag_bwd + 2 split-K weight-gradient GEMMs", bwd_ms, bwd_f)}
    return ms, fwd_f + bwd_f, kernels, None


def run_linrec(args, line):
    """The constant-matrix linear_recurrence (dynonet/core.py:103-127) on config 4's route: the
    companion matrices of the config-4 denominators (n = 3) driven by (w_t, 0, 0), the way the
    reference runs dynoNet's all-pole section without a fused kernel."""
    import torch
    import torch.nn.functional as F

    from tsfast_amd.dynonet import core as dcore
    from tsfast_amd.dynonet import linrec_hip

    a, w, gout = allpole_inputs("cuda", na=args.order)
    lanes, L = w.shape
    n = a.shape[-1]
    A = dcore.companion(a).contiguous()
    v = F.pad(w.unsqueeze(-1), (0, n - 1)).contiguous()
    g = F.pad(gout.unsqueeze(-1), (0, n - 1)).contiguous()
    del w, gout

    def step(ev):
        mark(ev)
        x = linrec_hip._linrec_op(A, v, None)
        mark(ev)
        linrec_hip._linrec_bwd_op(g, A, x, None)
        mark(ev)

    ms, (fwd_ms, bwd_ms) = time_steps(step, args.steps, args.warmup)

    nbytes = v.numel() * 4
    fwd_b, bwd_b = 2 * nbytes, 3 * nbytes  # read v, write x | read g and x, write grad_v
    line.update(
        metric="fwd+bwd ms + achieved HBM GB/s, constant-matrix linear_recurrence (BASELINE config 4 route)",
        config={"workload": f"linear_recurrence fwd+bwd: {lanes} lanes x L {L}, n {n} companion matrices of "
                            + ("the config-4 denominators" if n == 3 else f"order-{n} denominators drawn like config 4's")
                            + ", input (w_t, 0, ..) (BASELINE config 4 via the reference's companion-matrix route)",
                "lanes": lanes, "L": L, "n": n},
        fwd_ms=round(fwd_ms, 4),
        bwd_ms=round(bwd_ms, 4),
    )
    line["dtype"] = "f64"  # fp32 I/O, fp64 recurrence inside
    if n <= 4:
        kernels = {"fwd": ("linrec_fwd_lb look-back scan + transfer + reset", fwd_ms, fwd_b),
                   "bwd": ("linrec_bwd_lb look-back scan + transfer + reset + finish", bwd_ms, bwd_b)}
    elif n <= 8:
        kernels = {"fwd": ("lw_sum_fwd + lw_carry_fwd + lw_apply_fwd two-pass scan + lw_power", fwd_ms, fwd_b),
                   "bwd": ("lw_sum_bwd + lw_carry_bwd + lw_apply_bwd two-pass scan + lw_power + finish", bwd_ms,
                           bwd_b)}
    else:
        kernels = {"fwd": ("lsp_sum_fwd + lsp_carry_fwd + lsp_apply_fwd spread two-pass scan + lsp_power", fwd_ms,
                           fwd_b),
                   "bwd": ("lsp_sum_bwd + lsp_carry_bwd + lsp_apply_bwd spread two-pass scan + lsp_power + finish",
                           bwd_ms, bwd_b)}
    cpu = None
    if not args.no_cpu:
        def cpu_leg():
            threads = os.cpu_count() or 1
            torch.set_num_threads(threads)
            rows = 64
            A_c, v_c, g_c = A[:rows].cpu(), v[:rows].cpu(), g[:rows].cpu()

            from oracle import torch_reference as TR

            def fb():
                x = TR.linrec_forward(A_c, v_c)
                TR.linrec_backward(g_c, A_c, x)

            med, nrun = cpu_time(fb)
            sb = rows * L * n * 4 * 5
            return {
                "value": round(sb / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": (f"{rows} of {lanes} lanes, L={L}, n={n}: the log-doubling scan and its adjoint on CPU "
                           f"(the reference CPU path, dynonet/core.py:23-73), fwd+bwd median of {nrun} runs "
                           f"= {med * 1e3:.1f} ms"),
            }
        cpu = cpu_leg
    return ms, fwd_b + bwd_b, kernels, cpu


def run_adjoint(args, line):
    """The chunked NeuralStateSpace adjoint scan (ssm/backend_metal.py:446-479, kernels :285-357)
    at an NSS-sized backward with the reference's own chunking: B 16 (its largest scan batch),
    L 4096, n 32 (its largest scan state), C = min(ceil(512 / B), L // 64) chunks. The chunk
    summaries run on the fp64 matrix cores, so the roofline is fp64 MFMA (78.6 TFLOP/s)."""
    import torch

    from tsfast_amd.ssm import adjoint_hip

    B, L, n = 16, 4096, 32
    C = max(1, min(-(-512 // B), L // 64))
    cl = -(-L // C)
    g = torch.Generator(device="cuda").manual_seed(0)
    jt = torch.randn(B, L, n, n, device="cuda", generator=g) * (0.9 / n**0.5)
    gout = torch.randn(B, L, n, device="cuda", generator=g)

    def step(ev):
        mark(ev)
        adjoint_hip.run(jt, gout, cl)
        mark(ev)

    ms, (call_ms,) = time_steps(step, args.steps, args.warmup)
    flops = 2 * B * (L - 1) * n * n * (n + 1)  # [P | s] <- A [P | s] per step
    line.update(
        metric="ms per call + achieved fp64 TFLOP/s, chunked NSS adjoint scan (ssm_bwd_summary + ssm_bwd_scan)",
        unit="TFLOP/s",
        config={"workload": f"chunked adjoint of gy_t = gout_t + jt[t+1] gy_t+1: batch {B}, L {L}, n {n}, "
                            f"{C} chunks of {cl} steps (the reference's chunking), jt {B * L * n * n * 4 / 2**20:.0f} MiB",
                "B": B, "L": L, "n": n, "chunks": C, "chunk_len": cl},
        call_ms=round(call_ms, 4),
        algorithmic_flops={"call": flops},
        _mfma_peak_tflops=78.6,
    )
    line["dtype"] = "f64"  # fp32 inputs, fp64 summaries on the matrix cores
    kernels = {"call": ("mas_summary + mas_carry (fp64 MFMA chunk summaries, sequential carry)", call_ms, flops)}
    return ms, flops, kernels, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=(1, 2, 3, 4, 5))
    ap.add_argument("--io", choices=("bf16", "fp32"), default="bf16", help="config 3 / --conv I/O dtype")
    ap.add_argument("--selective", action="store_true",
                    help="measure the selective (time-varying) diagonal scan instead of a BASELINE config")
    ap.add_argument("--conv", action="store_true",
                    help="measure the fused Mamba conv+SiLU at config 3's shape instead of a BASELINE config")
    ap.add_argument("--gblock", action="store_true",
                    help="measure the fused dynoNet G-block (FIR + all-pole + input sum) at config 4's channels")
    ap.add_argument("--linrec", action="store_true",
                    help="measure the constant-matrix linear_recurrence on config 4's companion-matrix route")
    ap.add_argument("--projected", action="store_true",
                    help="measure the fused projected complex diagonal scan (LRU/S5 core) at config 2's shape")
    ap.add_argument("--widths", default="32,256,32",
                    help="with --projected: the layer's H,N,O (config 2's scan is 32,256,32); widths beyond the "
                         "fused kernel's (H, O <= 32, N <= 256) run the wide route")
    ap.add_argument("--adjoint", action="store_true",
                    help="measure the chunked NSS adjoint scan (n 32, the reference's chunking)")
    ap.add_argument("--order", type=int, default=3,
                    help="with --linrec: the denominator order n (state size 1..16; config 4 is 3); with "
                         "--gblock: the G-block's denominator order (1..16; above 4 the staged path)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    ap.add_argument(
        "--copy-calibration",
        action="store_true",
        help="only run a plain 512 MiB elementwise copy (to scale rocprofv3 FETCH_SIZE/WRITE_SIZE)",
    )
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures one GPU only: this build has no multi-GPU path (every config would "
            "shard over independent lanes: batch rows, channels or filter pairs, with no "
            "communication in the scan). Run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        # an elementwise kernel (plain vector loads/stores), not the runtime's blit copy
        src = torch.ones(128 << 20, dtype=torch.float32, device="cuda")  # 512 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "copies": 5}), flush=True)
        return

    from tsfast_amd import _lib

    _lib.load()
    line = {
        "metric": METRIC if args.config == 3 else f"fwd+bwd ms + achieved HBM GB/s, BASELINE config {args.config}",
        "value": None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
    }
    runner = (run_conv if args.conv else run_selective if args.selective else run_gblock if args.gblock
              else run_linrec if args.linrec else run_projected if args.projected else run_adjoint if args.adjoint
              else {1: run_diag, 2: run_diag, 3: run_mamba, 4: run_allpole, 5: run_diag}[args.config])
    ms, total_bytes, kernels, cpu = runner(args, line)
    # the look-back scans' mode: bitwise reproducible (the library's default) or fast
    # (TSFAST_HIP_REPRODUCIBLE=0: composition back to the nearest finished tile)
    line["lookback_mode"] = "reproducible" if _lib._reproducible else "fast"
    mfma_peak = line.pop("_mfma_peak_tflops", None)
    if mfma_peak is not None:
        # a matrix-core workload: throughput in algorithmic TFLOP/s against the dense fp32 MFMA peak
        line["value"] = round(total_bytes / (ms * 1e-3) / 1e12, 3)
        line["ms_per_step"] = round(ms, 4)
        phase = max(kernels, key=lambda k: kernels[k][1])
        name, dom_ms, dom_f = kernels[phase]
        got = dom_f / (dom_ms * 1e-3) / 1e12
        line["roofline"] = {"bound": "mfma", "kernel": name, "achieved": round(got, 3), "peak": mfma_peak,
                            "unit": "TFLOP/s", "frac": round(got / mfma_peak, 4), "traffic": None}
        print(json.dumps(line), flush=True)
        return
    gbs = total_bytes / (ms * 1e-3) / 1e9
    line["value"] = round(gbs, 2)
    line["ms_per_step"] = round(ms, 4)
    line["pct_hbm_peak"] = round(100 * gbs / HBM_PEAK_GBS, 2)
    line["algorithmic_bytes"] = {k: v[2] for k, v in kernels.items()}
    phase = max(kernels, key=lambda k: kernels[k][1])
    name, dom_ms, dom_b = kernels[phase]
    achieved = dom_b / (dom_ms * 1e-3) / 1e9
    key = (("selective", "f32") if args.selective else ("linrec", "f32") if args.linrec and args.order == 3
           else None if args.linrec else (args.config, args.io if args.config == 3 else "f32"))
    measured = None if (args.conv or args.gblock) else MEASURED_TRAFFIC.get(key, {}).get(phase)
    line["roofline"] = {
        "bound": "hbm",
        "kernel": name,
        "achieved": round(achieved, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": measured[0] if measured else None,
    }
    if measured:
        line["roofline"]["traffic_unit"] = "bytes per call"
        line["roofline"]["traffic_source"] = measured[1]
        line["roofline"]["algorithmic_bytes"] = dom_b
    valu = None if (args.conv or args.selective or args.gblock or args.linrec) else MEASURED_VALU.get(key, {}).get(phase)
    if valu:
        # VALU issue capacity: every SIMD issues one wave64 instruction per quad-cycle
        import torch

        cus = torch.cuda.get_device_properties(0).multi_processor_count
        peak = cus * SIMDS_PER_CU * VALU_PEAK_CLOCK_HZ / 4
        got = valu[0] / (dom_ms * 1e-3)
        line["valu"] = {
            "kernel": name,
            "achieved": round(got / 1e9, 2),
            "peak": round(peak / 1e9, 2),
            "unit": "G VALU issue quad-cycles/s",
            "frac": round(got / peak, 4),
            "issue_per_call": valu[0],
            "source": valu[1],
        }
    if cpu is not None:
        try:
            line["cpu_baseline"] = cpu()
        except Exception as e:  # noqa: BLE001 - reported, not fatal to the GPU number
            line["cpu_baseline"] = {"value": None, "error": repr(e)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
