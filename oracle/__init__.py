"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the five units.

``oracle.cm`` wraps ``cm_oracle.c`` (a C restatement of the reference simulator's integer
arithmetic) through ctypes; ``oracle.sim_numpy`` restates the reference simulator's own
float64 algorithm for the CPU-baseline timing.  Only ``tests/``, the smoke check and the
CPU-baseline leg of ``bench.py`` import this package; the product library never does.
"""
