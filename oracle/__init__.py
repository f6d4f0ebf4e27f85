"""CPU oracle of the reference MHSEA attention path — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this package,
as the checker or the timed CPU baseline; the hamiltonzero_amd product never imports it.
"""
