"""tsfast_amd: MI355X-native (gfx950) HIP backend for tsfast's linear-recurrence scan family.

The package mirrors the part of tsfast that the scans sit behind — the backend-preference
dispatcher (``dispatch``), the scan custom ops and public wrappers (``scan``), and the fused
Mamba / dynoNet all-pole dispatch points (``mamba``, ``dynonet``) — and adds one backend family,
``"hip"``, whose modules speak tsfast's backend protocol:

- ``scan_backends.diagonal_hip`` / ``scan_backends.selective_hip``:
  ``supports(lam, v, x0)``, ``forward(lam, v, x0)``, ``backward(g, lam, out, x0)``;
- ``mamba.mamba_hip``: ``supports(draw, A, Bt, Ct, u, z, Dp, h0)``, ``run(...)``;
- ``dynonet.allpole_hip``: ``supports(a, w, y0)``, ``run(a, w, y0)``.

Every kernel is hand-written HIP in ``csrc/`` compiled into ``libtsfast_hip.so`` (C ABI in
``include/tsfast_hip.h``) and loaded with ctypes by ``_lib``. The look-back scans are bitwise
reproducible by default, like the reference's kernels; ``set_reproducible(False)`` trades that for
0-4% of speed.
"""

from ._lib import set_reproducible  # noqa: F401
from .dispatch import BACKENDS, get_backend, set_backend, use_backend  # noqa: F401

__version__ = "0.1.0"
