"""CPU oracle for the token-selection path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker or the timed CPU baseline.  The
product path (whallm_amd) never imports it.
"""
