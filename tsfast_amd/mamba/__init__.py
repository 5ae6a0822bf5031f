"""Fused Mamba selective-SSM dispatch point and its HIP backend (``mamba_hip``)."""

from .core import mamba_ssm  # noqa: F401
