"""Build, load and time the C++/OpenMP port of the reference CPU kernels — TEST INFRASTRUCTURE.

Used only by bench.py's ``cpu_baseline`` leg and by tests. ``build()`` compiles
``cpu_baseline.cpp`` with the reference's flags (tsfast/models/_core/kernel_c.py:136-150:
``-O3 -march=native -ffast-math -fopenmp``; compile and link split, :248-270) into
``oracle/build/``. A portable ``-march=x86-64-v3`` copy is built as well so that a library built
in one container still loads on a GPU box whose host CPU differs; ``load()`` prefers a native
build made on the current host.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "cpu_baseline.cpp"
OUT = HERE / "build"
PORTABLE = OUT / "libtsfast_cpu_baseline_v3.so"

_lib = None
_lib_path = None


def _compile(dst: Path, march: str) -> None:
    dst.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory() as td:
        obj = Path(td) / "cpu_baseline.o"
        subprocess.run(
            ["g++", "-O3", f"-march={march}", "-ffast-math", "-fopenmp", "-fPIC", "-std=c++17", "-c", str(SRC), "-o", str(obj)],
            check=True,
            capture_output=True,
        )
        tmp = dst.with_suffix(".so.tmp")
        subprocess.run(["g++", "-shared", "-fopenmp", str(obj), "-o", str(tmp)], check=True, capture_output=True)
        os.replace(tmp, dst)


def build() -> Path:
    """Build the portable (x86-64-v3) library in-tree."""
    _compile(PORTABLE, "x86-64-v3")
    return PORTABLE


def load(prefer_native: bool = True) -> ctypes.CDLL:
    """Load the baseline library: a -march=native build for this host if g++ can make one
    (a few seconds, into a temp dir), else the portable in-tree build."""
    global _lib, _lib_path
    if _lib is not None:
        return _lib
    path = None
    if prefer_native:
        try:
            native = Path(tempfile.gettempdir()) / f"tsfast_cpu_baseline_native_{os.getpid()}.so"
            _compile(native, "native")
            path = native
        except (OSError, subprocess.CalledProcessError):
            path = None
    if path is None:
        if not PORTABLE.exists():
            build()
        path = PORTABLE
    lib = ctypes.CDLL(str(path))
    i64, ptr, i32 = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    lib.cpu_mamba_fwd.argtypes = [i64] * 4 + [ptr] * 11
    lib.cpu_mamba_bwd.argtypes = [i64] * 4 + [ptr] * 19
    lib.cpu_diag_fwd.argtypes = [i64, i64, i64, i32] + [ptr] * 4
    lib.cpu_diag_bwd.argtypes = [i64, i64, i64, i32] + [ptr] * 7
    lib.cpu_sel_fwd.argtypes = [i64, i64, i64] + [ptr] * 4
    lib.cpu_sel_bwd.argtypes = [i64, i64, i64] + [ptr] * 7
    for name in ("cpu_mamba_fwd", "cpu_mamba_bwd", "cpu_diag_fwd", "cpu_diag_bwd", "cpu_sel_fwd", "cpu_sel_bwd",
                 "cpu_num_threads",
                 "cpu_mamba_chk", "cpu_mamba_bd"):
        getattr(lib, name).restype = i32
    lib.cpu_set_threads.argtypes = [i32]
    lib.cpu_set_threads.restype = None
    lib.cpu_ref_expf.argtypes = [ptr, ptr, i64]
    lib.cpu_ref_expf.restype = None
    _lib, _lib_path = lib, path
    return lib


def lib_path() -> Path | None:
    return _lib_path


def ref_expf(x: np.ndarray) -> np.ndarray:
    """The port's restatement of the reference CPU kernel's exp (backend_c.py:55-74), elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    load().cpu_ref_expf(_p(x), _p(y), x.size)
    return y


def _p(a: np.ndarray | None):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def mamba_fwd_bwd(draw, A, Bt, Ct, u, z, Dp, gout, h0=None, ghlast=None):
    """fp32 fused Mamba forward (with checkpoints) + backward on numpy arrays; returns
    ``(out, h_last, gdraw, gA, gBt, gCt, gu, gz, gDp, gh0)`` with the partial buffers summed."""
    lib = load()
    f = lambda a: None if a is None else np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
    draw, A, Bt, Ct, u, z, Dp, gout, h0, ghlast = map(f, (draw, A, Bt, Ct, u, z, Dp, gout, h0, ghlast))
    B, L, D = draw.shape
    N = A.shape[1]
    chk_n = lib.cpu_mamba_chk()
    nblk = -(-D // lib.cpu_mamba_bd())
    out = np.empty_like(draw)
    hlast = np.empty((B, D, N), np.float32)
    chk = np.empty((B, -(-L // chk_n), D, N), np.float32)
    if lib.cpu_mamba_fwd(B, L, D, N, *map(_p, (draw, A, Bt, Ct, u, z, Dp, h0, out, chk, hlast))) != 0:
        raise ValueError(f"N={N} not built into the CPU baseline")
    gdraw, gu, gz = (np.empty_like(draw) for _ in range(3))
    gA_p = np.empty((B, D, N), np.float32)
    gB_p = np.empty((nblk, B, L, N), np.float32)
    gC_p = np.empty((nblk, B, L, N), np.float32)
    gDp_p = np.empty((B, D), np.float32)
    gh0 = np.empty((B, D, N), np.float32) if h0 is not None else None
    lib.cpu_mamba_bwd(
        B, L, D, N,
        *map(_p, (draw, A, Bt, Ct, u, z, Dp, h0, chk, gout, ghlast, gdraw, gA_p, gB_p, gC_p, gu, gz, gDp_p, gh0)),
    )
    return out, hlast, gdraw, gA_p.sum(0), gB_p.sum(0), gC_p.sum(0), gu, gz, gDp_p.sum(0), gh0


def diag_fwd_bwd(lam, v, g, x0=None):
    """Constant-coefficient diagonal scan forward + backward (float32 or complex64 numpy arrays)."""
    lib = load()
    cplx = int(np.iscomplexobj(v))
    dt = np.complex64 if cplx else np.float32
    lam, v, g = (np.ascontiguousarray(a, dtype=dt) for a in (lam, v, g))
    x0 = None if x0 is None else np.ascontiguousarray(x0, dtype=dt)
    M, L, N = v.shape
    out = np.empty_like(v)
    lib.cpu_diag_fwd(M, L, N, cplx, _p(lam), _p(v), _p(x0), _p(out))
    gv = np.empty_like(v)
    glam = np.empty_like(lam)
    gx0 = np.empty_like(lam) if x0 is not None else None
    lib.cpu_diag_bwd(M, L, N, cplx, _p(g), _p(lam), _p(out), _p(x0), _p(gv), _p(glam), _p(gx0))
    return out, glam, gv, gx0


def sel_fwd_bwd(a, v, g, x0=None):
    """Time-varying diagonal scan forward + backward (float32 numpy arrays [M, L, N])."""
    lib = load()
    a, v, g = (np.ascontiguousarray(t, dtype=np.float32) for t in (a, v, g))
    x0 = None if x0 is None else np.ascontiguousarray(x0, dtype=np.float32)
    M, L, N = v.shape
    out = np.empty_like(v)
    lib.cpu_sel_fwd(M, L, N, _p(a), _p(v), _p(x0), _p(out))
    glam, gv = np.empty_like(v), np.empty_like(v)
    gx0 = np.empty_like(x0) if x0 is not None else None
    lib.cpu_sel_bwd(M, L, N, _p(g), _p(a), _p(out), _p(x0), _p(glam), _p(gv), _p(gx0))
    return out, glam, gv, gx0
