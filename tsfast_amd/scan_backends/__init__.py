"""HIP kernel backends for the scan ops, one module per (op, backend) pair.

Same contract as ``tsfast/models/_core/scan_backends/__init__.py:1-22``: each module exposes
``supports(lam, v, x0) -> str | None`` and the raw lane-layout entry points
``forward(lam, v, x0) -> out`` and ``backward(g, lam, out, x0) -> (glam, gv, gx0)``, called from
inside the scan custom ops, which own dispatch and autograd.
"""
