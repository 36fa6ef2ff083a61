"""CPU oracle for the EXL3 / Marlin int4 quantized-weight path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  Never part of the product path.
"""
