"""Parity oracle for the mHC forward path -- TEST INFRASTRUCTURE ONLY.

mhc_ref: torch CPU restatement of the reference's PyTorch path (rounding points
included); brute: float64 scalar loops for tiny cases.  Imported only by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
"""
