"""dynoNet all-pole dispatch point, its HIP backend (``allpole_hip``) and the companion-matrix scan."""

from .core import allpole, linear_recurrence  # noqa: F401
