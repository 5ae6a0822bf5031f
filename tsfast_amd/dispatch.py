"""Backend preference and fused-kernel resolution, mirroring tsfast's dispatcher.

Same protocol and policy as ``tsfast/models/_core/dispatch.py:1-153``: a process-wide default
(``set_backend``), a ContextVar scope (``use_backend``), and ``resolve`` which tries candidate
backend modules in order, asking each ``supports(*args)`` for a decline reason and warning once
per ``"{op}.{family}"`` key before falling back. The only change is the family list: ``"hip"``
(this package's kernels) is added, and it is the first ``"auto"`` choice for ``"cuda"`` devices,
which is what ROCm tensors report.
"""

from __future__ import annotations

__all__ = [
    "BACKENDS",
    "get_backend",
    "set_backend",
    "use_backend",
    "resolve",
    "warn_fallback",
]

import contextvars
import importlib
import warnings
from contextlib import contextmanager
from types import ModuleType

import torch

#: Recognised preferences (tsfast's list plus "hip"); "reference" disables fused kernels.
BACKENDS = ("auto", "hip", "triton", "c", "metal", "reference")

_default_backend: str = "auto"
_override: contextvars.ContextVar[str | None] = contextvars.ContextVar("tsfast_amd_backend_override", default=None)


def _checked(name: str) -> str:
    if name not in BACKENDS:
        raise ValueError(f"unknown backend {name!r}, expected one of {BACKENDS}")
    return name


def get_backend() -> str:
    """Innermost ``use_backend`` scope, else the process default (only the default inside a trace)."""
    if torch.compiler.is_compiling():
        return _default_backend
    return _override.get() or _default_backend


def set_backend(name: str) -> None:
    """Set the process-wide default backend preference (one of ``BACKENDS``)."""
    global _default_backend
    _default_backend = _checked(name)


@contextmanager
def use_backend(name: str):
    """Scope a backend preference to a ``with`` block (thread- and async-safe)."""
    token = _override.set(_checked(name))
    try:
        yield
    finally:
        _override.reset(token)


def resolve(
    op: str,
    registry: dict[str, str | ModuleType],
    auto_order: tuple[str, ...],
    args: tuple,
    requested: str | None = None,
):
    """Pick the backend module for ``op``, or None for the reference path.

    ``"reference"`` -> None; ``"auto"`` -> try ``auto_order``; an explicit family -> only that
    family; a family missing from ``registry`` -> reference path silently; an import failure
    or a ``supports()`` reason -> warn once per ``"{op}.{family}"`` and try the next candidate.
    (Semantics of ``tsfast/models/_core/dispatch.py:80-135``.)
    """
    requested = get_backend() if requested is None else requested
    if requested == "reference":
        return None
    names = auto_order if requested == "auto" else (requested,)
    for name in names:
        target = registry.get(name)
        if target is None:
            continue
        if isinstance(target, str):
            try:
                mod = importlib.import_module(target)
            except Exception as e:
                warn_fallback(
                    f"{op}.{name}",
                    f"backend {name!r} unusable for {op}: backend import failed ({e!r}); "
                    "using the reference implementation",
                )
                continue
        else:
            mod = target
        reason = mod.supports(*args)
        if reason is None:
            return mod
        warn_fallback(
            f"{op}.{name}",
            f"backend {name!r} unusable for {op}: {reason}; using the reference implementation",
        )
    return None


_warned: set[str] = set()


def warn_fallback(key: str, message: str) -> None:
    """Emit ``message`` as a RuntimeWarning once per process per ``key`` (silent inside a trace)."""
    if torch.compiler.is_compiling():
        return
    if key not in _warned:
        _warned.add(key)
        warnings.warn(message, RuntimeWarning, stacklevel=3)
