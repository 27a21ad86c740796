"""CPU oracle for the flarellm decode path (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker.  The product (flarellm_amd/) never
imports it.
"""
