"""CPU oracle and CPU-baseline ports for the scan family — test infrastructure only.

``scan_oracle`` is the fp64 sequential checker; ``cpu_baseline`` builds and loads the C/OpenMP
port of the reference CPU kernels used as bench.py's ``cpu_baseline``. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import this package.
"""
