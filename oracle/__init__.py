"""CPU oracle (the checker) for the canonical W4G64 linear path.

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, never by the HIP product package.
"""
