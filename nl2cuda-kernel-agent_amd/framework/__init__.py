"""Algorithm-agnostic harness: the Case protocol, tolerances and timing
constants, parity checking, timing, and the HIP library loader.

Mirrors the reference's framework/ package (framework/case.py,
protocol.py, verify.py, bench.py, loader.py) for MI355X.
"""
