"""ctypes loader for libtsfast_hip.so and the marshalling shared by the backend shims.

The library is built in-tree by ``tsfast_amd.build`` (``python -m tsfast_amd.build``). Loading
is lazy (first kernel call) and failures raise: there is no silent fallback from a backend
module once it has been selected — a missing or unloadable library is a ``RuntimeError``
naming the path and the loader's reason.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("TSFAST_HIP_LIB", Path(__file__).resolve().parent / "libtsfast_hip.so"))

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p

# Entry points and their argument types (mirrors include/tsfast_hip.h).
_SIGNATURES: dict[str, tuple[list, object]] = {
    "tsfast_hip_version": ([], _int),
    "tsfast_hip_status_string": ([_int], ctypes.c_char_p),
    "tsfast_hip_set_deterministic": ([_int], None),
    "tsfast_hip_get_deterministic": ([], _int),
    "tsfast_hip_lookback_gave_up": ([_int], _int),
    "tsfast_hip_set_lookback_spin_limit": ([_i64], _i64),
    "tsfast_hip_diag_workspace_bytes": ([_i64, _i64, _i64, _int], _i64),
    "tsfast_hip_diag_fwd": ([_i64, _i64, _i64, _int] + [_ptr] * 5 + [_i64, _ptr], _int),
    "tsfast_hip_diag_bwd": ([_i64, _i64, _i64, _int] + [_ptr] * 8 + [_i64, _ptr], _int),
    "tsfast_hip_diag_noalloc_max_bytes": ([], _i64),
    "tsfast_hip_diag_fwd_noalloc": ([_i64, _i64, _i64, _int] + [_ptr] * 5, _int),
    "tsfast_hip_sel_workspace_bytes": ([_i64, _i64, _i64], _i64),
    "tsfast_hip_sel_fwd": ([_i64, _i64, _i64] + [_ptr] * 5 + [_i64, _ptr], _int),
    "tsfast_hip_sel_bwd": ([_i64, _i64, _i64] + [_ptr] * 8 + [_i64, _ptr], _int),
    "tsfast_hip_mamba_chk_interval": ([_i64], _i64),
    "tsfast_hip_mamba_saved_floats": ([_i64, _i64, _i64, _int], _i64),
    "tsfast_hip_mamba_workspace_bytes": ([_i64, _i64, _i64, _i64], _i64),
    "tsfast_hip_mamba_fwd": ([_i64, _i64, _i64, _i64, _int] + [_ptr] * 11 + [_ptr], _int),
    "tsfast_hip_mamba_bwd": ([_i64, _i64, _i64, _i64, _int] + [_ptr] * 20 + [_i64, _ptr], _int),
    "tsfast_hip_allpole_workspace_bytes": ([_i64, _i64, _i64], _i64),
    "tsfast_hip_allpole_fwd": ([_i64, _i64, _i64] + [_ptr] * 5 + [_i64, _ptr], _int),
    "tsfast_hip_allpole_bwd": ([_i64, _i64, _i64] + [_ptr] * 8 + [_i64, _ptr], _int),
    "tsfast_hip_conv_silu_workspace_bytes": ([_i64, _i64, _i64, _i64], _i64),
    "tsfast_hip_conv_silu_fwd": ([_i64, _i64, _i64, _i64, _int, _ptr, _i64, _i64, _i64] + [_ptr] * 5, _int),
    "tsfast_hip_conv_silu_bwd": (
        [_i64, _i64, _i64, _i64, _int, _ptr, _i64, _i64, _i64] + [_ptr] * 9 + [_i64, _ptr],
        _int,
    ),
    "tsfast_hip_gblock_workspace_bytes": ([_i64] * 6, _i64),
    "tsfast_hip_gblock_saved_doubles": ([_i64] * 5, _i64),
    "tsfast_hip_gblock_fwd": ([_i64] * 6 + [_ptr] * 9 + [_i64, _ptr], _int),
    "tsfast_hip_gblock_bwd": ([_i64] * 6 + [_ptr] * 14 + [_i64, _ptr], _int),
    "tsfast_hip_gblock_fir_workspace_bytes": ([_i64] * 5, _i64),
    "tsfast_hip_gblock_fir_fwd": ([_i64] * 5 + [_ptr] * 5, _int),
    "tsfast_hip_gblock_fir_bwd": ([_i64] * 5 + [_ptr] * 8 + [_i64, _ptr], _int),
    "tsfast_hip_linrec_workspace_bytes": ([_i64] * 3, _i64),
    "tsfast_hip_linrec_fwd": ([_i64] * 3 + [_ptr] * 5 + [_i64, _ptr], _int),
    "tsfast_hip_linrec_bwd": ([_i64] * 3 + [_ptr] * 8 + [_i64, _ptr], _int),
    "tsfast_hip_projscan_workspace_bytes": ([_i64] * 5, _i64),
    "tsfast_hip_projscan_saved_floats": ([_i64] * 3, _i64),
    "tsfast_hip_projscan_fwd": ([_i64] * 5 + [_ptr] * 11 + [_i64, _ptr], _int),
    "tsfast_hip_projscan_bwd_workspace_bytes": ([_i64] * 5, _i64),
    "tsfast_hip_projscan_bwd": ([_i64] * 5 + [_ptr] * 17 + [_i64, _ptr], _int),
    "tsfast_hip_mat_adjoint_workspace_bytes": ([_i64] * 4, _i64),
    "tsfast_hip_mat_adjoint_bounds": ([_i64] * 4 + [_ptr] * 4 + [_i64, _ptr], _int),
}

TSF_DTYPE_F32 = 0
TSF_DTYPE_BF16 = 1


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if it is missing or broken."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"libtsfast_hip.so not found at {LIB_PATH}; build it with `python -m tsfast_amd.build`"
                )
            try:
                lib = ctypes.CDLL(str(LIB_PATH))
            except OSError as e:
                raise RuntimeError(f"failed to load {LIB_PATH}: {e}") from e
            for name, (argtypes, restype) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            if torch.cuda.is_available():
                # allocate the look-back alarm word now, not inside a later graph capture
                lib.tsfast_hip_lookback_gave_up(0)
            _lib = lib
    return _lib


_det_mode: int | None = None
_reproducible = os.environ.get("TSFAST_HIP_REPRODUCIBLE", "1") not in ("", "0")


def set_reproducible(on: bool) -> bool:
    """Whether the look-back scans compose their tiles in a fixed order (bitwise reproducible
    outputs, the default; 0-4% slower) or back to the nearest finished tile (results agree run to
    run to fp64 rounding). Under ``torch.use_deterministic_algorithms(True)`` they are reproducible
    either way. Also set by the environment variable ``TSFAST_HIP_REPRODUCIBLE`` (``0`` = off).
    Returns the previous setting."""
    global _reproducible
    prev, _reproducible = _reproducible, bool(on)
    return prev


def sync_deterministic() -> None:
    """Put the library's look-back scans in deterministic mode unless reproducibility is switched
    off (``set_reproducible``) and ``torch.are_deterministic_algorithms_enabled()`` is false;
    called before every look-back scan is launched."""
    global _det_mode
    want = 1 if (_reproducible or torch.are_deterministic_algorithms_enabled()) else 0
    if want != _det_mode:
        load().tsfast_hip_set_deterministic(want)
        _det_mode = want


_CHECK_LOOKBACK = os.environ.get("TSFAST_HIP_CHECK_LOOKBACK", "0") not in ("", "0")
LOOKBACK_ERR_OFFSET = 64  # byte offset of the give-up flag in a look-back workspace (lookback.h kErrWord)


def lookback_gave_up(ws: torch.Tensor) -> bool:
    """Whether a look-back in the scan that used workspace ``ws`` gave up waiting (its lanes then
    hold NaN). Synchronises with the device."""
    return bool(ws[LOOKBACK_ERR_OFFSET : LOOKBACK_ERR_OFFSET + 4].view(torch.int32).item())


_gpu_seen = False


def _alarm(clear: bool) -> int:
    """1 if the library's look-back alarm word names a scan call that gave up and has not been
    reported, else 0 (-1 if the word is unavailable; 0 without a GPU, where no scan can have
    run); ``clear`` marks that call reported."""
    global _gpu_seen
    if not _gpu_seen:  # a GPU, once found, stays (the query costs more than the word's read)
        if not torch.cuda.is_available():
            return 0
        _gpu_seen = True
    return load().tsfast_hip_lookback_gave_up(1 if clear else 0)


def raise_if_lookback_gave_up(what: str) -> None:
    """Raise if a look-back scan of this process gave up and has not been reported yet, reading
    the library's alarm word in mapped host memory (no device synchronisation). A give-up shows
    there once its kernel has ended, so it is reported, once, by the first check after that:
    the call that launched it, or a later one."""
    if _alarm(clear=True) > 0:
        raise RuntimeError(
            f"{what}: a look-back wait in this or an earlier scan call gave up without progress (the "
            "GPU was probably shared with work that kept the scan's workgroups from running); the "
            "outputs of that call hold NaN"
        )


def check_lookback(ws: torch.Tensor, what: str) -> None:
    """Called after every look-back scan is enqueued: raises if a look-back gave up (this call's,
    if its kernels have ended, or an earlier call's) rather than let its NaN pass as a numerical
    result. With TSFAST_HIP_CHECK_LOOKBACK=1 in the environment (a debug mode) it first
    synchronises, so that this call's own give-up is always the one reported."""
    if _CHECK_LOOKBACK and lookback_gave_up(ws):
        _alarm(clear=True)
        raise RuntimeError(
            f"{what}: a look-back wait gave up without progress (the GPU was probably shared with "
            "work that kept the scan's workgroups from running); its outputs hold NaN"
        )
    raise_if_lookback_gave_up(what)


def available() -> bool:
    """True when the library file exists (does not load it)."""
    return LIB_PATH.exists()


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().tsfast_hip_status_string(status).decode()
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    """Raw device pointer of a tensor (None passes NULL)."""
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of the tensor's device, as an integer handle (torch's raw-stream
    query: a fraction of the cost of building a ``torch.cuda.Stream`` object on every call)."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


def require(t: torch.Tensor | None, name: str, dtypes: tuple, device: torch.device) -> None:
    """Screen a tensor handed to a raw-pointer kernel: dtype, device and density."""
    if t is None:
        return
    if t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if t.device != device:
        raise TypeError(f"{name}: on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise TypeError(f"{name}: must be contiguous")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch buffer for partial results (uninitialised; the kernels write before reading)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
